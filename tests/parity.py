"""Parity harness shared by the GPU tests, smoke() and bench.py: the oracle and the HIP plugin on one rollout."""

from __future__ import annotations

import contextlib
from types import SimpleNamespace

import torch

from oracle import ppo_ref as O
from oracle import rollout as R


def rel_err(a: torch.Tensor, b: torch.Tensor, floor: float = 0.0) -> float:
    """||a - b|| / max(||b||, floor), in float64."""
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    den = max(float(b.norm()), floor)
    if den == 0.0:
        return float((a - b).norm())
    return float((a - b).norm()) / den


def make_hip(workload: dict, seed: int = 0, device: str = "cuda", **alg_overrides):
    from tt_rsl_rl_amd.ppo import PPO

    torch.manual_seed(seed)
    cfg = R.train_cfg(workload, algorithm_class="tt_rsl_rl_amd.ppo:PPO", **alg_overrides)
    env = SimpleNamespace(num_envs=workload["num_envs"], num_actions=workload["num_actions"])
    alg = PPO.construct_algorithm(R.zero_obs(workload), env, cfg, device)
    alg.train_mode()
    return alg


def make_pair(workload: dict, seed: int = 0, carry_state: bool = False, **alg_overrides):
    """Oracle with a generated rollout + the HIP plugin with identical weights and the same stored rollout.
    Both have their returns / advantages computed from the same bootstrap values."""
    ora, roll = R.generate(workload, seed, carry_state=carry_state, **alg_overrides)
    hip = make_hip(workload, seed, **alg_overrides)
    with torch.no_grad():
        hip.actor.load_state_dict(roll.init_state["actor"])
        hip.critic.load_state_dict(roll.init_state["critic"])
    R.feed(hip.storage, roll)
    with torch.inference_mode():
        last_values = ora.critic(roll.last_obs).detach()
    ora.compute_returns(roll.last_obs, last_values=last_values)
    hip.compute_returns_from(last_values.to(hip.device).contiguous())
    return ora, hip, roll


@contextlib.contextmanager
def oracle_logp_fp64():
    """Run the oracle with the per-action log-prob sum accumulated in fp64 and rounded once, instead of torch's
    fp32 reduction order.  Same formula, a different (more accurate) fp32 evaluation: the difference between the
    two oracles is the oracle's own rounding floor for quantities that depend on the sum of A log-prob terms."""
    orig = O.GaussianDistribution.log_prob
    O.GaussianDistribution.log_prob = lambda self, x: self._distribution.log_prob(x).double().sum(dim=-1).float()
    try:
        yield
    finally:
        O.GaussianDistribution.log_prob = orig
