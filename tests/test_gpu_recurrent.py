"""The recurrent rollout side on the GPU against the CPU oracle: ``act`` / ``process_env_step`` / ``compute_returns``
with LSTM actor and critic (upstream rsl_rl/algorithms/ppo.py:124-191, rsl_rl/modules/rnn.py:35-71,
rsl_rl/storage/rollout_storage.py:333-359).

Same initial weights; each step both sides see the same observations, rewards and dones.  Actions are sampled
from different generators, so the comparison is on what does not depend on them: the policy mean, the values, the
LSTM states the models carry (zeroed for done envs) and the states the storage saves before each step.  Bar: 1e-5
relative (fp32 GEMMs of a different summation order over a few recurrent steps)."""

from __future__ import annotations

import torch

import pytest

from oracle import rollout as R
from tests.parity import make_hip, rel_err

pytestmark = pytest.mark.gpu


def _workload():
    w = R.scaled(R.WORKLOADS["lstm256"], num_envs=96, steps=6, hidden_dims=[64, 32])
    w["rnn"] = dict(w["rnn"], rnn_hidden_dim=64)
    w["obs_normalization"] = True
    return w


def test_recurrent_rollout_matches_oracle():
    w = _workload()
    ora = R.make_oracle(w, seed=0)
    ora.train_mode()
    hip = make_hip(w, seed=0)
    with torch.no_grad():
        hip.actor.load_state_dict(ora.actor.state_dict())
        hip.critic.load_state_dict(ora.critic.state_dict())
    dev = hip.device
    g = torch.Generator().manual_seed(11)
    n = w["num_envs"]
    with torch.inference_mode():
        obs = R.sample_obs(w)
        for step in range(w["steps"]):
            hip.act({k: v.to(dev) for k, v in obs.items()})
            ora.act(obs)
            th, to = hip.transition, ora.transition
            assert rel_err(th.distribution_params[0], to.distribution_params[0]) < 1e-5, step
            assert rel_err(th.values, to.values) < 1e-5, step
            for side in (0, 1):
                sh, so = th.hidden_states[side], to.hidden_states[side]
                if step == 0:
                    assert sh is None and so is None
                    continue
                for a, b in zip(sh, so):
                    assert a.shape == b.shape == (1, n, w["rnn"]["rnn_hidden_dim"])
                    assert rel_err(a, b) < 1e-5, (step, side)
            rewards = 0.1 * torch.randn(n, generator=g)
            dones = (torch.rand(n, generator=g) < 0.2).float()
            obs = R.sample_obs(w)
            hip.process_env_step({k: v.to(dev) for k, v in obs.items()}, rewards.to(dev), dones.to(dev), {})
            ora.process_env_step(obs, rewards, dones, {})
            for model_h, model_o in ((hip.actor, ora.actor), (hip.critic, ora.critic)):
                for a, b in zip(model_h.get_hidden_state(), model_o.get_hidden_state()):
                    assert torch.equal(a[0].cpu()[dones == 1], torch.zeros_like(b[0, dones == 1]))
                    assert rel_err(a, b) < 1e-5, step
        # the stored states: step 0 stays zero (no state yet), later steps the state before that step
        for side in ("a", "c"):
            for a, b in zip(getattr(hip.storage, f"saved_hidden_state_{side}"),
                            getattr(ora.storage, f"saved_hidden_state_{side}")):
                assert a.shape == b.shape
                assert rel_err(a, b) < 1e-5
        # the bootstrap forward leaves the critic's rollout state as it was
        before = [t.clone() for t in hip.critic.get_hidden_state()]
        hip.compute_returns({k: v.to(dev) for k, v in obs.items()})
        ora.compute_returns(obs)
        for a, b in zip(hip.critic.get_hidden_state(), before):
            assert torch.equal(a, b)
        assert rel_err(hip.storage.returns, ora.storage.returns) < 1e-5

