"""Export and inference copies of the plugin's models against upstream's structure (rsl_rl/models/mlp_model.py:163-255,
rsl_rl/models/rnn_model.py:98-247) and the oracle's forward, on the CPU (no GPU): TorchScript (as_jit), the ONNX
wrappers (as_onnx: inputs / outputs, dummy inputs, traceable; the file itself is written where the onnx package is
installed), and the plain-torch inference copy that ``model.to("cpu")`` -- hence upstream's
``runner.get_inference_policy("cpu")`` -- returns."""

from __future__ import annotations

import io

import pytest
import torch

from oracle import ppo_ref as O
from tt_rsl_rl_amd import models as M

OBS = {"policy": torch.zeros(4, 10), "extra": torch.zeros(4, 6)}
GROUPS = {"actor": ["policy", "extra"], "critic": ["policy"]}
DIST = {"class_name": "GaussianDistribution", "init_std": 1.0, "std_type": "log"}


def _pair(recurrent: bool, normalization: bool, layers: int = 1, rnn_type: str = "lstm"):
    kw = dict(hidden_dims=[32, 16], activation="elu", obs_normalization=normalization, distribution_cfg=DIST)
    if recurrent:
        kw.update(rnn_type=rnn_type, rnn_hidden_dim=24, rnn_num_layers=layers)
    torch.manual_seed(0)
    ora = (O.RNNModel if recurrent else O.MLPModel)(OBS, GROUPS, "actor", 5, **kw)
    torch.manual_seed(0)
    hip = (M.RNNModel if recurrent else M.MLPModel)(OBS, GROUPS, "actor", 5, **kw)
    for p_h, p_o in zip(hip.parameters(), ora.parameters()):
        assert torch.equal(p_h, p_o), "the plugin's initial weights are upstream's (same generator order)"
    if normalization:
        g = torch.Generator().manual_seed(1)
        for m in (ora, hip):
            n = m.obs_normalizer
            n._mean.copy_(torch.randn(n._mean.shape, generator=torch.Generator().manual_seed(2)))
            n._std.copy_(torch.rand(n._std.shape, generator=torch.Generator().manual_seed(3)) + 0.5)
            n._var.copy_(n._std ** 2)
            n.count.fill_(7)
        del g
    ora.eval()
    return ora, hip


def _obs(n: int, seed: int) -> dict:
    g = torch.Generator().manual_seed(seed)
    return {"policy": torch.randn(n, 10, generator=g), "extra": torch.randn(n, 6, generator=g)}


def _flat(obs: dict) -> torch.Tensor:
    return torch.cat([obs["policy"], obs["extra"]], dim=-1)


@pytest.mark.parametrize("normalization", [False, True])
def test_mlp_jit_export_matches_upstreams_structure_and_forward(normalization):
    ora, hip = _pair(False, normalization)
    jit = hip.as_jit()
    # upstream's copy holds exactly the normaliser and the MLP of the model (deepcopy), plus a parameterless output
    expected = [k for k in ora.state_dict() if not k.startswith("distribution.")]
    assert list(jit.state_dict().keys()) == expected
    scripted = torch.jit.script(jit)
    obs = _obs(9, 4)
    with torch.no_grad():
        ref = ora(obs)  # the deterministic output: the mean
        assert torch.equal(scripted(_flat(obs)), ref)
        assert torch.equal(jit(_flat(obs)), ref)
    scripted.reset()
    buf = io.BytesIO()
    torch.jit.save(scripted, buf)
    buf.seek(0)
    with torch.no_grad():
        assert torch.equal(torch.jit.load(buf)(_flat(obs)), ref)


def test_mlp_onnx_wrapper():
    ora, hip = _pair(False, True)
    onnx_model = hip.as_onnx()
    assert onnx_model.is_recurrent is False
    assert onnx_model.input_names == ["obs"] and onnx_model.output_names == ["actions"]
    (dummy,) = onnx_model.get_dummy_inputs()
    assert dummy.shape == (1, 16)
    obs = _obs(3, 5)
    with torch.no_grad():
        assert torch.equal(onnx_model(_flat(obs)), ora(obs))
        traced = torch.jit.trace(onnx_model, (dummy,))
        assert torch.equal(traced(_flat(obs)), ora(obs))
    _maybe_onnx_export(onnx_model)


def _maybe_onnx_export(m):
    """The runner's export call (rsl_rl/runners/on_policy_runner.py:189-201), where the onnx package is present."""
    try:
        import onnx  # noqa: F401
    except ImportError:
        return  # not installed in this image: the wrapper's forward and tracing are checked above
    buf = io.BytesIO()
    m.eval()
    torch.onnx.export(m, m.get_dummy_inputs(), buf, export_params=True, opset_version=18,
                      input_names=m.input_names, output_names=m.output_names, dynamo=False)
    assert len(buf.getvalue()) > 0


def _oracle_steps(ora, seq: list[dict], dones: list[torch.Tensor]) -> list[torch.Tensor]:
    outs = []
    ora.reset(hidden_state=None)
    with torch.no_grad():
        for obs, d in zip(seq, dones):
            outs.append(ora(obs))
            ora.reset(d)
    return outs


class _TensorOutputs(torch.nn.Module):
    def __init__(self, m: torch.nn.Module) -> None:
        super().__init__()
        self.m = m

    def forward(self, obs: torch.Tensor, h: torch.Tensor):
        return self.m(obs, h)[:2]


@pytest.mark.parametrize("rnn_type,layers", [("lstm", 1), ("lstm", 2), ("gru", 1), ("gru", 2)])
def test_recurrent_jit_and_onnx_exports_step_like_upstream(rnn_type, layers):
    ora, hip = _pair(True, True, layers, rnn_type)
    lstm = rnn_type == "lstm"
    jit = hip.as_jit()
    # upstream's copy: its state buffers (the GRU has no cell state), then the normaliser, the torch RNN (the
    # wrapper's inner nn.LSTM / nn.GRU) and the MLP, in that order
    sd = ora.state_dict()
    states = ["hidden_state", "cell_state"] if lstm else ["hidden_state"]
    expected = (states + [k for k in sd if k.startswith("obs_normalizer.")] +
                [k.replace("rnn.rnn.", "rnn.") for k in sd if k.startswith("rnn.")] +
                [k for k in sd if k.startswith("mlp.")])
    assert list(jit.state_dict().keys()) == expected
    assert list(hip.as_onnx().state_dict().keys()) == expected[len(states):]
    assert isinstance(jit.rnn, torch.nn.LSTM if lstm else torch.nn.GRU)
    for name in states:
        assert getattr(jit, name).shape == (layers, 1, 24)
    scripted = torch.jit.script(jit)
    seq = [_obs(1, 10 + t) for t in range(6)]
    dones = [torch.tensor([1.0 if t == 2 else 0.0]) for t in range(6)]
    ref = _oracle_steps(ora, seq, dones)
    onnx_model = hip.as_onnx()
    assert onnx_model.input_names == (["obs", "h_in", "c_in"] if lstm else ["obs", "h_in"])
    assert onnx_model.output_names == (["actions", "h_out", "c_out"] if lstm else ["actions", "h_out"])
    dummy = onnx_model.get_dummy_inputs()
    assert len(dummy) == (3 if lstm else 2)
    state = list(dummy[1:])
    with torch.no_grad():
        for t, (obs, d) in enumerate(zip(seq, dones)):
            assert torch.allclose(scripted(_flat(obs)), ref[t], rtol=1e-6, atol=1e-7), t
            out, h, c = onnx_model(_flat(obs), *state)
            assert (c is None) == (not lstm)
            state = [h, c] if lstm else [h]
            assert torch.allclose(out, ref[t], rtol=1e-6, atol=1e-7), t
            if d.item() == 1.0:  # a done: the exported models start the next step from the zero state
                scripted.reset()
                state = [torch.zeros_like(x) for x in state]
        # the GRU's (out, h, None) as upstream's: torch.jit.trace takes tensor outputs only, so trace the two tensors
        fn = onnx_model if lstm else _TensorOutputs(onnx_model)
        traced = torch.jit.trace(fn, onnx_model.get_dummy_inputs())
        out = traced(*onnx_model.get_dummy_inputs())[0]
        assert out.shape == (1, 5)
    _maybe_onnx_export(onnx_model)


@pytest.mark.parametrize("recurrent", [False, "lstm", "gru"])
def test_to_cpu_gives_an_inference_copy(recurrent):
    """model.to("cpu") returns a plain-torch copy with upstream's forward on observation dicts (the deterministic
    mean; recurrent models carry a per-env state that reset(dones) zeroes) and leaves the model itself alone."""
    ora, hip = _pair(bool(recurrent), True, rnn_type=recurrent or "lstm")
    before = [p.data_ptr() for p in hip.parameters()]
    pol = hip.to("cpu")
    assert isinstance(pol, M.TorchPolicy) and pol is not hip
    assert [p.data_ptr() for p in hip.parameters()] == before
    n = 5
    seq = [_obs(n, 20 + t) for t in range(4)]
    dones = [(torch.rand(n, generator=torch.Generator().manual_seed(30 + t)) < 0.4).float() for t in range(4)]
    ref = _oracle_steps(ora, seq, dones) if recurrent else [ora(o).detach() for o in seq]
    pol.reset(hidden_state=None)
    with torch.no_grad():
        for t, (obs, d) in enumerate(zip(seq, dones)):
            out = pol(obs)
            assert torch.allclose(out, ref[t], rtol=1e-6, atol=1e-7), t
            pol.reset(d)
