"""Pins the oracle's rollout storage and mini-batch generator (restating rsl_rl/storage/rollout_storage.py).

Known behaviours restated from upstream's tests/storage/test_rollout_storage.py:69-126, 275-316, 371-406, 486-491.
"""

from __future__ import annotations

import pytest
import torch

from oracle import ppo_ref as O

N, T, D, A = 6, 8, 4, 3


def _filled():
    obs = {"policy": torch.randn(N, D)}
    st = O.RolloutStorage(N, T, obs, [A])
    for step in range(T):
        t = O.Transition()
        t.observations = {"policy": torch.full((N, D), float(step))}
        t.actions = torch.full((N, A), float(step))
        t.values = torch.full((N, 1), float(step) * 10)
        t.actions_log_prob = torch.full((N,), float(step) * 0.1)
        t.distribution_params = (torch.full((N, A), float(step)), torch.ones(N, A))
        t.rewards = torch.full((N,), float(step) * 100)
        t.dones = torch.zeros(N)
        st.add_transition(t)
    st.returns = torch.randn_like(st.returns)
    st.advantages = torch.randn_like(st.advantages)
    return st


def test_every_transition_once_per_epoch():
    st = _filled()
    seen = torch.cat([b.indices for b in st.mini_batch_generator(4, num_epochs=1)])
    assert sorted(seen.tolist()) == list(range(N * T))


def test_epoch_count_and_single_permutation_reused():
    st = _filled()
    batches = list(st.mini_batch_generator(3, num_epochs=5))
    assert len(batches) == 15
    first = torch.cat([b.indices for b in batches[:3]])
    for e in range(1, 5):
        assert torch.equal(torch.cat([b.indices for b in batches[3 * e:3 * e + 3]]), first)


def test_permutation_is_torch_randperm_of_the_seeded_cpu_generator():
    st = _filled()
    torch.manual_seed(123)
    got = torch.cat([b.indices for b in st.mini_batch_generator(4, num_epochs=1)])
    torch.manual_seed(123)
    assert torch.equal(got, torch.randperm(N * T))


def test_fields_aligned_and_time_major_rows():
    st = _filled()
    for b in st.mini_batch_generator(2, num_epochs=1):
        step = b.indices // N  # row = t * N + n
        assert torch.equal(b.actions[:, 0], step.float())
        assert torch.allclose(b.values[:, 0], step.float() * 10)
        assert torch.allclose(b.old_actions_log_prob[:, 0], step.float() * 0.1)
        assert torch.equal(b.observations["policy"][:, 0], step.float())


@pytest.mark.parametrize("m", [5, 7])
def test_remainder_batches_cover_everything(m):
    st = _filled()
    sizes = [b.actions.shape[0] for b in st.mini_batch_generator(m, num_epochs=1)]
    B = N * T
    assert sizes == [(i + 1) * B // m - i * B // m for i in range(m)]


@pytest.mark.parametrize("m", [0, N * T + 1])
def test_invalid_partition_counts_rejected(m):
    st = _filled()
    with pytest.raises(ValueError):
        next(st.mini_batch_generator(m, num_epochs=1))


def test_overflow_raises_and_clear_allows_refill():
    st = _filled()
    t = O.Transition()
    with pytest.raises(OverflowError):
        st.add_transition(t)
    st.clear()
    assert st.step == 0
