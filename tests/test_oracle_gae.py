"""Pins the oracle's GAE / advantage normalisation (restating rsl_rl/algorithms/ppo.py:166-191).

Known answers restated from upstream's tests/algorithms/test_ppo.py:112-259, plus an fp64 textbook recursion
(independent of upstream's operation order) on random inputs with terminations.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ppo_ref as O


def _col(vals):
    return torch.tensor(vals, dtype=torch.float32).view(-1, 1, 1)


def test_hand_computed_returns():
    """tests/algorithms/test_ppo.py:139-195: rewards 1,2,3; values .5,1,1.5; no dones; bootstrap 2."""
    rewards, values, dones = _col([1.0, 2.0, 3.0]), _col([0.5, 1.0, 1.5]), torch.zeros(3, 1, 1, dtype=torch.uint8)
    ret, _ = O.gae_returns(rewards, values, dones, torch.full((1, 1), 2.0), 0.99, 0.95, normalize=False)
    adv = [1.49 + 0.99 * 0.95 * (2.485 + 0.99 * 0.95 * 3.48), 2.485 + 0.99 * 0.95 * 3.48, 3.48]
    expected = [a + v for a, v in zip(adv, [0.5, 1.0, 1.5])]
    for i in range(3):
        assert ret[i, 0, 0].item() == pytest.approx(expected[i], abs=1e-4)


def test_terminal_state_cuts_bootstrap():
    """tests/algorithms/test_ppo.py:197-237: done at step 0 -> no bootstrap from step 1."""
    rewards, values = _col([1.0, 2.0]), _col([0.5, 1.0])
    dones = torch.tensor([1, 0], dtype=torch.uint8).view(2, 1, 1)
    ret, _ = O.gae_returns(rewards, values, dones, torch.full((1, 1), 3.0), 0.99, 0.95, normalize=False)
    assert ret[0, 0, 0].item() == pytest.approx(0.5 + 0.5, abs=1e-4)
    assert ret[1, 0, 0].item() == pytest.approx(3.97 + 1.0, abs=1e-4)


def test_singleton_advantage_is_not_normalised():
    """tests/algorithms/test_ppo.py:112-137: one transition keeps its advantage (numel() == 1 skips the norm)."""
    rewards, values = _col([2.3]), _col([0.3])
    ret, adv = O.gae_returns(rewards, values, torch.zeros(1, 1, 1, dtype=torch.uint8), torch.zeros(1, 1), 0.0, 0.95)
    assert adv.item() == pytest.approx(2.0, abs=1e-6)


def test_global_normalisation_mean_zero_std_one():
    """tests/algorithms/test_ppo.py:239-259."""
    g = torch.Generator().manual_seed(0)
    T, N = 8, 4
    ret, adv = O.gae_returns(torch.randn(T, N, 1, generator=g), torch.randn(T, N, 1, generator=g),
                             torch.zeros(T, N, 1, dtype=torch.uint8), torch.randn(N, 1, generator=g), 0.99, 0.95)
    assert abs(adv.mean().item()) < 1e-5
    assert abs(adv.std().item() - 1.0) < 1e-3  # unbiased std, eps 1e-8 outside the sqrt


@pytest.mark.parametrize("p_done", [0.0, 0.05, 0.5, 1.0])
def test_matches_fp64_textbook_recursion(p_done):
    g = torch.Generator().manual_seed(int(p_done * 100))
    T, N = 24, 257
    r = torch.randn(T, N, 1, generator=g) * 0.3
    v = torch.randn(T, N, 1, generator=g)
    d = (torch.rand(T, N, 1, generator=g) < p_done).to(torch.uint8)
    last = torch.randn(N, 1, generator=g)
    ret, adv_raw = O.gae_returns(r, v, d, last, 0.99, 0.95, normalize=False)
    ret64, adv64 = O.gae_fp64(r[..., 0].numpy(), v[..., 0].numpy(), d[..., 0].numpy(), last.numpy(), 0.99, 0.95)
    assert np.allclose(ret[..., 0].numpy(), ret64, rtol=0, atol=2e-5)
    assert np.allclose(adv_raw[..., 0].numpy(), adv64, rtol=0, atol=2e-5)
    # a planted mistake in the oracle's recursion (dropped lambda) is caught by the same check
    ret_bad, _ = O.gae_returns(r, v, d, last, 0.99, 1.0, normalize=False)
    if p_done < 1.0:
        assert not np.allclose(ret_bad[..., 0].numpy(), ret64, rtol=0, atol=2e-5)


def test_normalised_advantages_match_closed_form():
    g = torch.Generator().manual_seed(3)
    T, N = 24, 100
    r, v = torch.randn(T, N, 1, generator=g), torch.randn(T, N, 1, generator=g)
    d = (torch.rand(T, N, 1, generator=g) < 0.1).to(torch.uint8)
    last = torch.randn(N, 1, generator=g)
    _, adv = O.gae_returns(r, v, d, last, 0.99, 0.95, normalize=True)
    _, a64 = O.gae_fp64(r[..., 0].numpy(), v[..., 0].numpy(), d[..., 0].numpy(), last.numpy(), 0.99, 0.95)
    ref = (a64 - a64.mean()) / (a64.std(ddof=1) + 1e-8)
    assert np.allclose(adv[..., 0].numpy(), ref, atol=1e-5)
