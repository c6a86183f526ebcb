"""The rollout side on the GPU against the CPU oracle: ``act`` / ``process_env_step`` / ``compute_returns``
(upstream rsl_rl/algorithms/ppo.py:124-191) with feed-forward and with LSTM actor and critic (rsl_rl/modules/rnn.py:35-71,
rsl_rl/storage/rollout_storage.py:333-359).

Same initial weights; each step both sides see the same observations, rewards, dones and time-outs.  Actions are
sampled from different generators, so the comparison is on what does not depend on them: the policy mean and std, the
values, the log-probability of the GPU's own actions under the oracle's policy, the LSTM states the models carry
(zeroed for done envs) and the states the storage saves before each step, the stored rewards and GAE.  Bar: 1e-5
relative (fp32 GEMMs of a different summation order over a few steps)."""

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



def test_mlp_rollout_matches_oracle():
    """The feed-forward rollout side: humanoid-shaped actor / critic (separate observation groups, observation
    normalisation) over several steps with dones and time-outs.  Per step: the policy mean and std, the values, and
    the log-probability the GPU stores for its own sampled actions against the oracle's log-probability of those
    actions; then the stored rewards (time-out bootstrap r + gamma V(s_t) on time-outs, ppo.py:150-156) and the
    returns / advantages of compute_returns.  Bar: 1e-5 relative."""
    w = R.scaled(R.WORKLOADS["humanoid"], num_envs=96, steps=5, hidden_dims=[64, 32])
    ora = R.make_oracle(w, seed=0)
    ora.train_mode()
    hip = make_hip(w, seed=0)
    with torch.no_grad():
        hip.actor.load_state_dict(ora.actor.state_dict())
        hip.critic.load_state_dict(ora.critic.state_dict())
    dev = hip.device
    g = torch.Generator().manual_seed(5)
    n = w["num_envs"]
    with torch.inference_mode():
        obs = R.sample_obs(w)
        for step in range(w["steps"]):
            actions = hip.act({k: v.to(dev) for k, v in obs.items()})
            ora.act(obs)
            th, to = hip.transition, ora.transition
            for a, b in zip(th.distribution_params, to.distribution_params):
                assert rel_err(a, b) < 1e-5, step
            assert rel_err(th.values, to.values) < 1e-5, step
            ora.actor(obs, stochastic_output=True)  # the oracle's distribution at this step, then its log-prob
            logp_ref = ora.actor.get_output_log_prob(actions.cpu())
            assert rel_err(th.actions_log_prob, logp_ref) < 1e-5, step
            rewards = 0.1 * torch.randn(n, generator=g)
            dones = (torch.rand(n, generator=g) < 0.2).float()
            time_outs = dones * (torch.rand(n, generator=g) < 0.5).float()
            obs = R.sample_obs(w)
            hip.process_env_step({k: v.to(dev) for k, v in obs.items()}, rewards.to(dev), dones.to(dev),
                                 {"time_outs": time_outs.to(dev)})
            ora.process_env_step(obs, rewards, dones, {"time_outs": time_outs})
        assert rel_err(hip.storage.rewards, ora.storage.rewards) < 1e-5
        assert torch.equal(hip.storage.dones.cpu().float(), ora.storage.dones.float())
        hip.compute_returns({k: v.to(dev) for k, v in obs.items()})
        ora.compute_returns(obs)
        assert rel_err(hip.storage.returns, ora.storage.returns) < 1e-5
        assert rel_err(hip.storage.advantages, ora.storage.advantages) < 1e-5
