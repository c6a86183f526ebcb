"""The plugin storage's recurrent_mini_batch_generator (API compatibility; upstream rollout_storage.py:262-331 with
rsl_rl/utils/utils.py:395-449) against the oracle's, on the CPU: every field of every mini-batch bit for bit --
padded trajectory observations, masks, the states the trajectories start from, the unpadded fields -- for LSTM
(h, c) states and for a rollout whose last step and first step have dones."""

from __future__ import annotations

import pytest
import torch

from oracle import ppo_ref as O
from tt_rsl_rl_amd.storage import RolloutStorage


def _fill(T=9, N=7, A=3, H=5, p_done=0.3, seed=0):
    g = torch.Generator().manual_seed(seed)
    obs0 = {"policy": torch.zeros(N, 4), "extra": torch.zeros(N, 2)}
    mine = RolloutStorage("rl", N, T, obs0, [A], device="cpu")
    ora = O.RolloutStorage(N, T, obs0, [A])
    for t in range(T):
        tr = O.Transition()
        tr.observations = {k: torch.randn(N, v.shape[1], generator=g) for k, v in obs0.items()}
        tr.actions = torch.randn(N, A, generator=g)
        tr.values = torch.randn(N, 1, generator=g)
        tr.actions_log_prob = torch.randn(N, generator=g)
        tr.distribution_params = (torch.randn(N, A, generator=g), torch.rand(N, A, generator=g))
        tr.rewards = torch.randn(N, generator=g)
        d = (torch.rand(N, generator=g) < p_done).float()
        if t == 0:
            d[0] = 1.0
        if t == T - 1:
            d[1] = 1.0
        tr.dones = d
        tr.hidden_states = tuple((torch.randn(1, N, H, generator=g), torch.randn(1, N, H, generator=g))
                                 for _ in range(2))
        for st in (mine, ora):
            st.add_transition(tr)
    g2 = torch.Generator().manual_seed(seed + 1)
    adv, ret = torch.randn(T, N, 1, generator=g2), torch.randn(T, N, 1, generator=g2)
    for st in (mine, ora):
        st.advantages, st.returns = adv.clone(), ret.clone()
    return mine, ora


@pytest.mark.parametrize("M", [1, 2, 3, 7])
def test_recurrent_generator_matches_upstreams(M):
    mine, ora = _fill()
    got = list(mine.recurrent_mini_batch_generator(M, num_epochs=2))
    ref = list(ora.recurrent_mini_batch_generator(M, num_epochs=2))
    assert len(got) == len(ref) == 2 * M
    for a, b in zip(got, ref):
        for k in b.observations:
            assert torch.equal(a.observations[k], b.observations[k]), k
        assert torch.equal(a.masks, b.masks)
        for f in ("actions", "values", "advantages", "returns", "old_actions_log_prob"):
            assert torch.equal(getattr(a, f), getattr(b, f)), f
        for x, y in zip(a.old_distribution_params, b.old_distribution_params):
            assert torch.equal(x, y)
        for side in (0, 1):
            for x, y in zip(a.hidden_states[side], b.hidden_states[side]):
                assert torch.equal(x, y)


def test_recurrent_generator_partition_errors():
    mine, _ = _fill()
    with pytest.raises(ValueError):
        next(mine.recurrent_mini_batch_generator(8))
