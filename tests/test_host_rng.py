"""The update's CPU-generator draws, computed natively, against torch itself (no GPU): the discarded Normal samples of
every mini-batch (upstream's stochastic forward, rsl_rl/models/mlp_model.py:103-106 via
rsl_rl/algorithms/ppo.py:228-233) skipped with ppo_host_rng_skip, after the permutation, leave the generator exactly
where upstream's CPU update leaves it, so the next rollout's noise and the next update's permutation are upstream's."""

from __future__ import annotations

import time

import pytest
import torch
from torch.distributions import Normal

from tt_rsl_rl_amd import ops


def _state_after(fn, seed=7):
    torch.manual_seed(seed)
    fn()
    return torch.get_rng_state()


@pytest.mark.parametrize("n", [16, 17, 31, 32, 100, 1000, 24576 * 29, 393216 * 12 + 5])
def test_skip_matches_torch_normal(n):
    """torch's float normal_ of n >= 16 elements takes n draws plus 16 when n % 16 != 0: skipping that many leaves the
    same generator record, and the next draws agree."""
    ref = _state_after(lambda: torch.randn(n))
    got = _state_after(lambda: ops.SplitRandperm(0, None, 0, [n]).join())
    assert torch.equal(ref, got)
    torch.set_rng_state(ref)
    a = torch.randn(37)
    torch.set_rng_state(got)
    assert torch.equal(a, torch.randn(37))
    # negative control: one draw fewer is another state
    if n > 16:
        short = _state_after(lambda: ops.SplitRandperm(0, None, 0, [n - 1 if n % 16 != 1 else n - 2]).join())
        assert not torch.equal(ref, short)


def test_sample_is_a_standard_normal_scaled():
    """Normal(mean, std).sample() on the CPU = randn(shape) * std + mean in fp32, with the same draws: so a rollout
    that takes its standard-normal noise from the CPU generator and scales it on the GPU reproduces upstream's."""
    torch.manual_seed(3)
    mean, std = torch.randn(4096, 29), torch.rand(29) + 0.3
    torch.manual_seed(11)
    a = Normal(mean, std).sample()
    st_a = torch.get_rng_state()
    torch.manual_seed(11)
    z = torch.randn(4096, 29)
    b = z * std + mean
    assert torch.equal(a, b) and torch.equal(st_a, torch.get_rng_state())


@pytest.mark.parametrize("first_on_worker", [False, True], ids=["first_here", "first_on_worker"])
@pytest.mark.parametrize("n,split,normals", [(98304, 24576, [24576 * 29] * 20),
                                             (1000, 250, [250 * 12, 3, 250 * 12, 7, 250 * 12]),
                                             (0, 0, [1024 * 24 * 12] * 20)])
def test_update_draws_match_upstream_order(n, split, normals, first_on_worker):
    """randperm(n) then one discarded sample per mini-batch (sizes in order; tiny ones included), as upstream's update
    draws them, against torch doing exactly that."""
    def upstream():
        perm = torch.randperm(n) if n else None
        for k in normals:
            Normal(torch.zeros(k), torch.ones(k)).sample()
        return perm

    torch.manual_seed(5)
    p_ref = upstream()
    st_ref = torch.get_rng_state()
    torch.manual_seed(5)
    out = torch.empty(n, dtype=torch.int64) if n else None
    job = ops.SplitRandperm(n, out, split, normals, first_on_worker=first_on_worker)
    p = job.join()
    assert torch.equal(st_ref, torch.get_rng_state())
    if n:
        assert torch.equal(p, p_ref)


def test_skip_is_fast():
    """The discarded samples of one 4096 x 24 humanoid update (20 x 24,576 x 29 draws) are skipped in well under the
    update's GPU time (the skip runs on a worker thread beside it)."""
    torch.manual_seed(1)
    t0 = time.perf_counter()
    ops.SplitRandperm(0, None, 0, [24576 * 29] * 20).join()
    dt = time.perf_counter() - t0
    assert dt < 0.05, dt
