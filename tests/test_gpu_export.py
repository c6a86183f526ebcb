"""Export and inference policies of a plugin trained on the GPU, as upstream's runner takes them
(rsl_rl/runners/on_policy_runner.py:171-201): ``get_inference_policy(device)`` on the GPU is the live model (its
parameters still views of the update's flat buffers, so later updates reach it), on the CPU a plain-torch copy; the
TorchScript / ONNX exports compute what the GPU model computes (1e-5: fp32 CPU GEMMs against the MFMA kernels)."""

from __future__ import annotations

import pytest
import torch

from oracle import rollout as R
from tests.parity import make_pair, rel_err

pytestmark = pytest.mark.gpu


def _flat(w, obs, groups):
    return torch.cat([obs[g] for g in groups], dim=-1)


@pytest.mark.parametrize("recurrent", [False, "lstm", "gru"])
def test_inference_policies_and_exports_after_an_update(recurrent):
    if recurrent:
        w = R.scaled(R.WORKLOADS["lstm256"], num_envs=64, steps=8, hidden_dims=[64, 32])
        w["rnn"] = dict(w["rnn"], rnn_hidden_dim=32, rnn_type=recurrent, rnn_num_layers=2 if recurrent == "gru" else 1)
        w["obs_normalization"] = True
    else:
        w = R.scaled(R.WORKLOADS["humanoid"], num_envs=64, steps=8, hidden_dims=[64, 32])
    _, hip, _ = make_pair(w, seed=0)
    torch.manual_seed(1)
    hip.update()
    hip.eval_mode()
    actor = hip.get_policy()
    dev = hip.device
    # the runner's get_inference_policy(device) on the GPU: the live model, parameters still in the flat buffers
    live = actor.to(dev)
    assert live is actor
    lo = hip.flat.param.data_ptr()
    hi = lo + hip.flat.param.numel() * 4
    assert all(lo <= p.data_ptr() < hi for p in live.parameters())
    # on the CPU: a plain-torch copy; the live model is untouched
    cpu = actor.to("cpu")
    assert cpu is not actor and all(lo <= p.data_ptr() < hi for p in actor.parameters())
    groups = actor.obs_groups
    g = torch.Generator().manual_seed(3)
    n = w["num_envs"]
    seq = [R.sample_obs(w, n) for _ in range(4)]
    dones = [(torch.rand(n, generator=g) < 0.3).float() for _ in range(4)]
    jit = torch.jit.script(actor.as_jit())
    onnx_model = actor.as_onnx()
    actor.reset(hidden_state=None)
    cpu.reset(hidden_state=None)
    h = c = None
    with torch.inference_mode():
        for t, (obs, d) in enumerate(zip(seq, dones)):
            ref = actor({k: v.to(dev) for k, v in obs.items()}).cpu()
            assert rel_err(cpu(obs), ref) < 1e-5, t
            x = _flat(w, obs, groups)
            if recurrent:
                # the exports are batch-1 steppers: follow env 0 (reset after its dones)
                out_j = jit(x[:1])
                if h is None:
                    state = list(onnx_model.get_dummy_inputs()[1:])  # (h, c) for the LSTM, (h,) for the GRU
                out_o, h, c = onnx_model(x[:1], *state)
                state = [h, c] if c is not None else [h]
                assert rel_err(out_j, ref[:1]) < 1e-5 and rel_err(out_o, ref[:1]) < 1e-5, t
                if d[0] == 1.0:
                    jit.reset()
                    state = [torch.zeros_like(v) for v in state]
            else:
                assert rel_err(jit(x), ref) < 1e-5 and rel_err(onnx_model(x), ref) < 1e-5, t
            actor.reset(d.to(dev))
            cpu.reset(d)
