"""Pins the oracle's Gaussian head and observation normaliser.

Restates upstream's tests/modules/test_distribution.py:14-120 (closed-form log-prob, entropy, KL) and
tests/modules/test_normalization.py:15-80, and adds the parallel-moment closed form for the running statistics.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import ppo_ref as O


def test_log_prob_at_mean_of_standard_normal():
    d = O.GaussianDistribution(4, init_std=1.0, std_type="scalar")
    d.update(torch.zeros(1, 4))
    assert d.log_prob(torch.zeros(1, 4)).item() == pytest.approx(-0.5 * math.log(2 * math.pi) * 4, abs=1e-5)


def test_entropy_closed_form():
    d = O.GaussianDistribution(3, init_std=2.0, std_type="scalar")
    d.update(torch.zeros(1, 3))
    assert d.entropy.item() == pytest.approx(0.5 * 3 * math.log(2 * math.pi * math.e * 4.0), abs=1e-4)


def test_kl_closed_form_and_self_kl():
    d = O.GaussianDistribution(1)
    kl = d.kl_divergence((torch.tensor([[0.0]]), torch.tensor([[1.0]])), (torch.tensor([[1.0]]), torch.tensor([[2.0]])))
    assert kl.item() == pytest.approx(math.log(2.0) + (1.0 + 1.0) / (2 * 4.0) - 0.5, abs=1e-6)
    p = (torch.zeros(1, 4), torch.full((1, 4), 1.5))
    assert d.kl_divergence(p, p).abs().item() < 1e-6


def test_scalar_and_log_std_agree_and_clamp():
    m = torch.randn(2, 3)
    a, b = O.GaussianDistribution(3, 1.5, std_type="scalar"), O.GaussianDistribution(3, 1.5, std_type="log")
    a.update(m)
    b.update(m)
    x = torch.randn(2, 3)
    assert torch.allclose(a.log_prob(x), b.log_prob(x), atol=1e-5)
    assert torch.allclose(a.entropy, b.entropy, atol=1e-5)
    hi = O.GaussianDistribution(2, 10.0, std_range=(0.1, 2.0), std_type="log")
    hi.update(torch.zeros(1, 2))
    assert torch.allclose(hi.std, torch.full((1, 2), 2.0), atol=1e-6)


def test_log_prob_gradient_matches_fp64_formula():
    """d logp / d mu = (a - mu) / std^2 and d logp / d log std = (a - mu)^2 / std^2 - 1 (closed forms)."""
    g = torch.Generator().manual_seed(0)
    d = O.GaussianDistribution(5, std_type="log")
    with torch.no_grad():
        d.log_std_param.copy_(torch.randn(5, generator=g) * 0.3)
    mu = torch.randn(7, 5, generator=g).requires_grad_(True)
    a = torch.randn(7, 5, generator=g)
    d.update(mu)
    d.log_prob(a).sum().backward()
    sd = torch.exp(d.log_std_param.detach()).double()
    diff = a.double() - mu.detach().double()
    assert torch.allclose(mu.grad.double(), diff / sd ** 2, rtol=1e-5)
    assert torch.allclose(d.log_std_param.grad.double(), (diff ** 2 / sd ** 2 - 1).sum(0), rtol=1e-5, atol=1e-6)


# ----------------------------------------------------------------------------------------------------------------------
# EmpiricalNormalization (rsl_rl/modules/normalization.py)
# ----------------------------------------------------------------------------------------------------------------------


def test_initial_transform_is_x_over_1_01():
    n = O.EmpiricalNormalization(3)
    x = torch.randn(5, 3)
    assert torch.equal(n(x), (x - 0.0) / (1.0 + 0.01))


def test_convergence_forward_until_and_eval():
    torch.manual_seed(0)
    n = O.EmpiricalNormalization(4)
    n.train()
    for _ in range(200):
        n.update(5.0 + 2.0 * torch.randn(64, 4))
    assert torch.allclose(n.mean, torch.full((4,), 5.0), atol=0.15)
    assert torch.allclose(n.std, torch.full((4,), 2.0), atol=0.15)
    u = O.EmpiricalNormalization(2, until=100)
    u.train()
    for _ in range(10):
        u.update(torch.randn(20, 2))
    snap = u._mean.clone()
    u.update(torch.randn(20, 2) + 100)
    assert torch.equal(u._mean, snap)
    e = O.EmpiricalNormalization(3)
    e.eval()
    e.update(torch.randn(10, 3) + 7)
    assert int(e.count) == 0


def test_running_moments_equal_pooled_moments():
    """Parallel-moment closed form: after updates with X1 then X2 the statistics are those of cat(X1, X2), given
    the initial state (mean 0, var 1, count 0) is replaced on the first update (rate = 1)."""
    g = torch.Generator().manual_seed(1)
    x1 = torch.randn(3000, 6, generator=g) * 3 + 1
    x2 = torch.randn(500, 6, generator=g) * 0.5 - 2
    n = O.EmpiricalNormalization(6)
    n.train()
    n.update(x1)
    n.update(x2)
    pooled = torch.cat([x1, x2]).double()
    assert torch.allclose(n._mean.double().view(-1), pooled.mean(0), rtol=1e-5, atol=1e-6)
    assert torch.allclose(n._var.double().view(-1), pooled.var(0, unbiased=False), rtol=1e-5)
    assert int(n.count) == 3500


def test_activation_modules_are_the_closed_forms():
    """rsl_rl/utils/utils.py:34-68: every name resolves to the module whose output is the textbook function (torch's
    default arguments: SELU's alpha / scale, LeakyReLU slope 0.01, CELU alpha 1, Softplus beta 1 with threshold 20,
    exact-erf GELU), checked in fp64 on values across every branch; unknown names raise ValueError."""
    import math

    from oracle import ppo_ref as O

    x = torch.linspace(-30.0, 30.0, 2001, dtype=torch.float64)
    e = lambda v: torch.tensor([math.exp(t) for t in v.tolist()], dtype=torch.float64)  # noqa: E731
    sig = 1.0 / (1.0 + e(-x))
    sp = torch.where(x > 20, x, torch.log(1.0 + e(x)))
    want = {
        "elu": torch.where(x > 0, x, e(x) - 1), "crelu": torch.where(x > 0, x, e(x) - 1),
        "selu": 1.0507009873554805 * torch.where(x > 0, x, 1.6732632423543772 * (e(x) - 1)),
        "relu": torch.where(x > 0, x, torch.zeros_like(x)), "lrelu": torch.where(x > 0, x, 0.01 * x),
        "tanh": torch.tensor([math.tanh(t) for t in x.tolist()], dtype=torch.float64), "sigmoid": sig,
        "softplus": sp, "gelu": torch.tensor([0.5 * t * (1 + math.erf(t / math.sqrt(2))) for t in x.tolist()],
                                             dtype=torch.float64),
        "swish": x * sig, "mish": x * torch.tensor([math.tanh(t) for t in torch.log(1.0 + e(x)).tolist()],
                                                     dtype=torch.float64),
        "identity": x,
    }
    for name, ref in want.items():
        got = O.activation_module(name)(x)
        assert torch.allclose(got, ref, rtol=1e-12, atol=1e-12), name
    with pytest.raises(ValueError):
        O.activation_module("swishy")
