"""The HIP PPO update against the committed golden fixture (no oracle at run time): the fixture's rollout and
initial weights go in through upstream's add_transition / load_state_dict, torch.manual_seed(1) precedes the update,
and the outputs are held to the parity bars (returns bit-exact, advantages 1e-6, losses 1e-4, learning-rate trace
identical, every parameter 1e-4 relative)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from tests.golden.make_golden import ALG, WORKLOAD

pytestmark = pytest.mark.gpu
FIXTURE = Path(__file__).resolve().parent / "golden" / "ppo_update_small.npz"


def test_hip_update_matches_golden_fixture(cuda):
    from tests.parity import make_hip, rel_err
    from tt_rsl_rl_amd.storage import RolloutStorage

    g = np.load(FIXTURE)
    hip = make_hip(WORKLOAD, seed=0, **ALG)
    for m, model in (("actor", hip.actor), ("critic", hip.critic)):
        sd = {k[len(f"init.{m}."):]: torch.from_numpy(g[k]) for k in g.files if k.startswith(f"init.{m}.")}
        model.load_state_dict(sd)
    for t in range(WORKLOAD["steps"]):
        tr = RolloutStorage.Transition()
        tr.observations = {k: torch.from_numpy(g[f"roll.{t}.obs.{k}"]) for k in WORKLOAD["obs"]}
        tr.actions = torch.from_numpy(g[f"roll.{t}.actions"])
        tr.values = torch.from_numpy(g[f"roll.{t}.values"])
        tr.actions_log_prob = torch.from_numpy(g[f"roll.{t}.logp"])
        tr.distribution_params = (torch.from_numpy(g[f"roll.{t}.mean"]), torch.from_numpy(g[f"roll.{t}.std"]))
        tr.rewards = torch.from_numpy(g[f"roll.{t}.rewards"])
        tr.dones = torch.from_numpy(g[f"roll.{t}.dones"])
        hip.storage.add_transition(tr)
    hip.compute_returns_from(torch.from_numpy(g["last_values"]).to(cuda).contiguous())
    assert np.array_equal(hip.storage.returns.cpu().numpy(), g["returns"])
    np.testing.assert_allclose(hip.storage.advantages.cpu().numpy(), g["advantages"], rtol=0, atol=1e-6)
    torch.manual_seed(1)
    out = hip.update()
    ref = g["losses"]
    for i, k in enumerate(("value", "surrogate", "entropy")):
        den = max(abs(ref[i]), 0.1 if k == "surrogate" else 0.0)
        assert abs(out[k] - ref[i]) <= 1e-4 * den, (k, out[k], ref[i])
    assert [t["lr"] for t in hip.last_trace] == list(g["trace.lr"])
    for m, model in (("actor", hip.actor), ("critic", hip.critic)):
        for k, v in model.state_dict().items():
            r = torch.from_numpy(g[f"final.{m}.{k}"])
            if k.endswith("count"):
                assert int(v) == int(r)
            else:
                assert rel_err(v, r, 1e-12) < 1e-4, (m, k, rel_err(v, r, 1e-12))
