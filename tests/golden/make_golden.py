"""Writes tests/golden/ppo_update_small.npz: a small seeded PPO update computed by the CPU oracle.

Inputs: the initial actor / critic weights, the rollout (per step: observations, actions, values, log-probs,
distribution params, rewards, dones) and the bootstrap values.  Outputs: returns, advantages, the loss dict,
the learning-rate / KL trace, and every parameter after one update (torch.manual_seed(1) before it).

Run from the repository root: ``python tests/golden/make_golden.py``.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import rollout as R  # noqa: E402

OUT = Path(__file__).resolve().parent / "ppo_update_small.npz"

WORKLOAD = dict(num_envs=32, steps=8, obs={"policy": ("normal", 16), "critic": ("normal", 19)},
                obs_groups={"actor": ["policy"], "critic": ["critic"]}, num_actions=5, hidden_dims=[32, 16],
                reward_std=0.2, p_done=0.05, obs_normalization=True)
ALG = dict(num_mini_batches=3)


def compute() -> dict[str, np.ndarray]:
    torch.set_num_threads(1)
    ora, roll = R.generate(WORKLOAD, seed=11, **ALG)
    with torch.inference_mode():
        last_values = ora.critic(roll.last_obs).detach()
    ora.compute_returns(roll.last_obs, last_values=last_values)
    out: dict[str, np.ndarray] = {}
    for m in ("actor", "critic"):
        for k, v in roll.init_state[m].items():
            out[f"init.{m}.{k}"] = v.numpy()
    for t, rec in enumerate(roll.transitions):
        for k, v in rec.observations.items():
            out[f"roll.{t}.obs.{k}"] = v.numpy()
        out[f"roll.{t}.actions"] = rec.actions.numpy()
        out[f"roll.{t}.values"] = rec.values.numpy()
        out[f"roll.{t}.logp"] = rec.actions_log_prob.numpy()
        out[f"roll.{t}.mean"] = rec.distribution_params[0].numpy()
        out[f"roll.{t}.std"] = rec.distribution_params[1].numpy()
        out[f"roll.{t}.rewards"] = rec.rewards.numpy()
        out[f"roll.{t}.dones"] = rec.dones.numpy()
    out["last_values"] = last_values.numpy()
    out["returns"] = ora.storage.returns.numpy()
    out["advantages"] = ora.storage.advantages.numpy()
    torch.manual_seed(1)
    losses = ora.update()
    out["losses"] = np.array([losses["value"], losses["surrogate"], losses["entropy"]], dtype=np.float64)
    out["trace.lr"] = np.array([t["lr"] for t in ora.trace], dtype=np.float64)
    out["trace.kl"] = np.array([t["kl_mean"] for t in ora.trace], dtype=np.float64)
    out["perm"] = torch.cat([t["indices"] for t in ora.trace[:ora.num_mini_batches]]).numpy()
    for m, model in (("actor", ora.actor), ("critic", ora.critic)):
        for k, v in model.state_dict().items():
            out[f"final.{m}.{k}"] = v.numpy()
    return out


if __name__ == "__main__":
    np.savez_compressed(OUT, **compute())
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")
