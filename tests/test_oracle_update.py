"""Pins the oracle's PPO.update (restating rsl_rl/algorithms/ppo.py:193-358).

* Known-answer tables restated from upstream's tests/algorithms/test_ppo.py: surrogate clipping :385-395, value
  clipping :397-409, adaptive learning rate :415-437, normaliser timing :293-326, Adam first step :492-505.
* The gradient of one full-batch step against an independent float64 functional evaluation of the PPO objective
  (plain matrices, no nn.Module / torch.distributions), with negative controls that plant a mistake.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import ppo_ref as O

NUM_ENVS, NUM_STEPS, OBS_DIM, NUM_ACTIONS = 4, 8, 8, 4


def _build(**over):
    obs = {"policy": torch.randn(NUM_ENVS, OBS_DIM)}
    groups = {"actor": ["policy"], "critic": ["policy"]}
    a_kw = dict(hidden_dims=[32, 32], activation="elu",
                distribution_cfg={"class_name": "GaussianDistribution", "init_std": 1.0, "std_type": "scalar"})
    c_kw = dict(hidden_dims=[32, 32], activation="elu")
    for k in ("obs_normalization",):
        if k in over:
            a_kw[k] = c_kw[k] = over.pop(k)
    actor = O.MLPModel(obs, groups, "actor", NUM_ACTIONS, **a_kw)
    critic = O.MLPModel(obs, groups, "critic", 1, **c_kw)
    storage = O.RolloutStorage(NUM_ENVS, NUM_STEPS, obs, [NUM_ACTIONS])
    kw = dict(num_learning_epochs=2, num_mini_batches=2, clip_param=0.2, gamma=0.99, lam=0.95, value_loss_coef=1.0,
              entropy_coef=0.01, learning_rate=1e-3, max_grad_norm=1.0, schedule="fixed", desired_kl=0.01)
    kw.update(over)
    return O.PPO(actor, critic, storage, **kw), obs


def _fill(ppo, obs):
    with torch.no_grad():
        for _ in range(NUM_STEPS):
            ppo.act(obs)
            ppo.process_env_step(obs, torch.zeros(NUM_ENVS), torch.zeros(NUM_ENVS), {})


@pytest.mark.parametrize("advantage, ratio, expected", [(1.0, 1.5, -1.2), (-1.0, 0.5, 0.8), (1.0, 0.5, -0.5)])
def test_surrogate_clipping_table(advantage, ratio, expected):
    torch.manual_seed(0)
    ppo, obs = _build(num_learning_epochs=1, num_mini_batches=1)
    _fill(ppo, obs)
    ppo.storage.actions_log_prob.sub_(math.log(ratio))
    ppo.storage.advantages.fill_(advantage)
    assert ppo.update()["surrogate"] == pytest.approx(expected)


@pytest.mark.parametrize("clipped, offset, expected", [(True, 0.0, 0.64), (False, 0.0, 0.0), (True, -1.0, 1.0)])
def test_value_clipping_table(clipped, offset, expected):
    torch.manual_seed(0)
    ppo, obs = _build(num_learning_epochs=1, num_mini_batches=1, use_clipped_value_loss=clipped)
    _fill(ppo, obs)
    ppo.storage.returns.copy_(ppo.storage.values + offset)
    ppo.storage.values.sub_(1.0)
    assert ppo.update()["value"] == pytest.approx(expected, abs=1e-6)


@pytest.mark.parametrize("kl, lr0, lr1", [(0.03, 1e-3, 1e-3 / 1.5), (0.002, 1e-3, 1.5e-3), (0.01, 1e-3, 1e-3),
                                          (0.0, 1e-3, 1e-3), (0.03, 1.2e-5, 1e-5), (0.002, 8e-3, 1e-2)])
def test_adaptive_lr_table(monkeypatch, kl, lr0, lr1):
    torch.manual_seed(0)
    ppo, obs = _build(num_learning_epochs=1, num_mini_batches=1, schedule="adaptive", learning_rate=lr0)
    _fill(ppo, obs)
    monkeypatch.setattr(ppo.actor, "get_kl_divergence", lambda *_: torch.tensor(kl))
    ppo.update()
    assert ppo.learning_rate == pytest.approx(lr1)
    assert all(g["lr"] == pytest.approx(lr1) for g in ppo.optimizer.param_groups)


def test_lr_rule_compares_in_fp32():
    """torch compares the fp32 kl_mean with the Python float rounded to fp32: fp32(0.02) is not > 0.02."""
    assert O.adaptive_lr(torch.tensor(0.02, dtype=torch.float32), 1e-3, 0.01) == 1e-3
    up = torch.nextafter(torch.tensor(0.02, dtype=torch.float32), torch.tensor(1.0))
    assert O.adaptive_lr(up, 1e-3, 0.01) == 1e-3 / 1.5


def test_normaliser_frozen_during_rollout_and_updated_after():
    torch.manual_seed(0)
    ppo, _ = _build(num_learning_epochs=1, num_mini_batches=1, obs_normalization=True)
    for step in range(NUM_STEPS):
        ppo.act({"policy": torch.full((NUM_ENVS, OBS_DIM), float(step + 1))})
        ppo.process_env_step({"policy": torch.full((NUM_ENVS, OBS_DIM), float(step + 2))}, torch.ones(NUM_ENVS),
                             torch.zeros(NUM_ENVS), {})
    assert int(ppo.actor.obs_normalizer.count) == 0
    expected = ppo.storage.observations["policy"].flatten(0, 1).mean(0)
    ppo.compute_returns({"policy": torch.full((NUM_ENVS, OBS_DIM), 9.0)})
    ppo.update()
    assert int(ppo.actor.obs_normalizer.count) == NUM_ENVS * NUM_STEPS
    assert torch.allclose(ppo.actor.obs_normalizer.mean, expected)


def test_adam_first_step_moves_each_parameter_by_lr():
    torch.manual_seed(0)
    ppo, _ = _build()
    params = ppo.optimizer.param_groups[0]["params"]
    before = [p.detach().clone() for p in params]
    for p in params:
        p.grad = torch.ones_like(p)
    ppo.optimizer.step()
    for b, p in zip(before, params):
        assert torch.allclose((b - p.detach()).abs(), torch.full_like(b, 1e-3), atol=1e-6)


# ----------------------------------------------------------------------------------------------------------------------
# one full-batch step against an independent fp64 evaluation of the objective
# ----------------------------------------------------------------------------------------------------------------------


def _mlp64(x, layers):
    h = x
    for i, (w, b) in enumerate(layers):
        z = h @ w.t() + b
        h = torch.where(z > 0, z, torch.expm1(z)) if i < len(layers) - 1 else z
    return h


def _objective64(p, batch, clip=0.2, cv=1.0, ce=0.01, clipped=True):
    x = batch["obs"] / (1.0 + 0.01)  # fresh normaliser: (x - 0) / (1 + eps)
    mu = _mlp64(x, p["actor"])
    v = _mlp64(x, p["critic"])[:, 0]
    log_sd = p["log_std"]
    sd = torch.exp(log_sd)
    logp = (-(batch["actions"] - mu) ** 2 / (2 * sd ** 2) - log_sd - 0.5 * math.log(2 * math.pi)).sum(-1)
    ratio = torch.exp(logp - batch["old_logp"])
    adv = batch["adv"]
    surr = torch.maximum(-adv * ratio, -adv * ratio.clamp(1 - clip, 1 + clip)).mean()
    if clipped:
        vc = batch["old_v"] + (v - batch["old_v"]).clamp(-clip, clip)
        vloss = torch.maximum((v - batch["ret"]) ** 2, (vc - batch["ret"]) ** 2).mean()
    else:
        vloss = ((batch["ret"] - v) ** 2).mean()
    entropy = (0.5 + 0.5 * math.log(2 * math.pi) + log_sd).sum()
    return surr + cv * vloss - ce * entropy


@pytest.mark.parametrize("clipped", [True, False])
def test_full_batch_gradient_matches_fp64_objective(clipped):
    torch.manual_seed(4)
    n, T, d, A = 16, 4, 5, 3
    obs = {"policy": torch.randn(n, d)}
    groups = {"actor": ["policy"], "critic": ["policy"]}
    actor = O.MLPModel(obs, groups, "actor", A, hidden_dims=[8, 6], obs_normalization=True,
                       distribution_cfg={"class_name": "GaussianDistribution", "init_std": 0.8, "std_type": "log"})
    critic = O.MLPModel(obs, groups, "critic", 1, hidden_dims=[8, 6], obs_normalization=True)
    ppo = O.PPO(actor, critic, O.RolloutStorage(n, T, obs, [A]), num_learning_epochs=1, num_mini_batches=1,
                learning_rate=0.0, max_grad_norm=1e9, schedule="fixed", use_clipped_value_loss=clipped)
    ppo.train_mode()
    with torch.no_grad():
        for _ in range(T):
            o = {"policy": torch.randn(n, d)}
            ppo.act(o)
            ppo.process_env_step(o, torch.randn(n), (torch.rand(n) < 0.2).float(), {})
    ppo.compute_returns({"policy": torch.randn(n, d)})
    st = ppo.storage
    # perturb old log-probs so that both clip branches are exercised
    st.actions_log_prob.add_(0.3 * torch.randn_like(st.actions_log_prob))
    lin = lambda m: [(l.weight.detach().double().clone().requires_grad_(True),
                      l.bias.detach().double().clone().requires_grad_(True))
                     for l in m.mlp if isinstance(l, torch.nn.Linear)]
    p = {"actor": lin(actor), "critic": lin(critic),
         "log_std": actor.distribution.log_std_param.detach().double().clone().requires_grad_(True)}
    f = lambda t: t.flatten(0, 1).double()
    batch = {"obs": f(st.observations["policy"]), "actions": f(st.actions), "old_logp": f(st.actions_log_prob)[:, 0],
             "adv": f(st.advantages)[:, 0], "old_v": f(st.values)[:, 0], "ret": f(st.returns)[:, 0]}
    _objective64(p, batch, clipped=clipped).backward()
    torch.manual_seed(1)
    ppo.update()
    got = [actor.distribution.log_std_param.grad] + [t.grad for m in (actor, critic) for l in m.mlp
                                                       if isinstance(l, torch.nn.Linear) for t in (l.weight, l.bias)]
    ref = [p["log_std"].grad] + [t.grad for k in ("actor", "critic") for wb in p[k] for t in wb]
    for g, r in zip(got, ref):
        assert torch.allclose(g.double(), r, rtol=2e-4, atol=1e-7), (g, r)
    # negative control: a sign error in the entropy bonus is visible in the std gradient
    for t in [p["log_std"]] + [t for k in ("actor", "critic") for wb in p[k] for t in wb]:
        t.grad = None
    _objective64(p, batch, ce=-0.01, clipped=clipped).backward()
    assert not torch.allclose(got[0].double(), p["log_std"].grad, rtol=2e-4, atol=1e-7)


def test_full_batch_gradient_clipped_per_model():
    """clip_grad_norm_ per model (ppo.py:309-310) with clipping active: each model's gradient is the fp64 objective's
    gradient scaled by min(1, max_norm / (||g_model|| + 1e-6)), the actor's norm including its std parameter.  Negative
    control: one norm over both models (a plausible mistake) gives other gradients."""
    torch.manual_seed(5)
    n, T, d, A = 16, 4, 5, 3
    obs = {"policy": torch.randn(n, d)}
    groups = {"actor": ["policy"], "critic": ["policy"]}
    actor = O.MLPModel(obs, groups, "actor", A, hidden_dims=[8, 6],
                       distribution_cfg={"class_name": "GaussianDistribution", "init_std": 0.8, "std_type": "log"})
    critic = O.MLPModel(obs, groups, "critic", 1, hidden_dims=[8, 6])
    max_norm = 0.05
    ppo = O.PPO(actor, critic, O.RolloutStorage(n, T, obs, [A]), num_learning_epochs=1, num_mini_batches=1,
                learning_rate=0.0, max_grad_norm=max_norm, schedule="fixed")
    ppo.train_mode()
    with torch.no_grad():
        for _ in range(T):
            o = {"policy": torch.randn(n, d)}
            ppo.act(o)
            ppo.process_env_step(o, torch.randn(n), (torch.rand(n) < 0.2).float(), {})
    ppo.compute_returns({"policy": torch.randn(n, d)})
    st = ppo.storage
    lin = lambda m: [(l.weight.detach().double().clone().requires_grad_(True),
                      l.bias.detach().double().clone().requires_grad_(True))
                     for l in m.mlp if isinstance(l, torch.nn.Linear)]
    p = {"actor": lin(actor), "critic": lin(critic),
         "log_std": actor.distribution.log_std_param.detach().double().clone().requires_grad_(True)}
    f = lambda t: t.flatten(0, 1).double()
    batch = {"obs": f(st.observations["policy"]) * 1.01, "actions": f(st.actions),
             "old_logp": f(st.actions_log_prob)[:, 0], "adv": f(st.advantages)[:, 0], "old_v": f(st.values)[:, 0],
             "ret": f(st.returns)[:, 0]}
    _objective64(p, batch).backward()  # no normaliser here: undo the fresh normaliser's 1/(1 + eps) of _objective64
    torch.manual_seed(1)
    ppo.update()
    ref_a = [p["log_std"].grad] + [t.grad for wb in p["actor"] for t in wb]
    ref_c = [t.grad for wb in p["critic"] for t in wb]
    norm = lambda gs: math.sqrt(sum(float((g * g).sum()) for g in gs))
    coef = lambda gs: min(1.0, max_norm / (norm(gs) + 1e-6))
    ca, cc = coef(ref_a), coef(ref_c)
    assert ca < 0.5 and cc < 0.5  # clipping is active for both models
    got_a = [actor.distribution.log_std_param.grad] + [t.grad for l in actor.mlp if isinstance(l, torch.nn.Linear)
                                                        for t in (l.weight, l.bias)]
    got_c = [t.grad for l in critic.mlp if isinstance(l, torch.nn.Linear) for t in (l.weight, l.bias)]
    for g, r in zip(got_a, ref_a):
        assert torch.allclose(g.double(), r * ca, rtol=2e-4, atol=1e-9)
    for g, r in zip(got_c, ref_c):
        assert torch.allclose(g.double(), r * cc, rtol=2e-4, atol=1e-9)
    # negative control: a single norm over both models
    cg = coef(ref_a + ref_c)
    assert not all(torch.allclose(g.double(), r * cg, rtol=2e-4, atol=1e-9) for g, r in zip(got_a, ref_a))


# ----------------------------------------------------------------------------------------------------------------------
# clip-branch forcing (test infrastructure of the GPU parity tests: not upstream)
# ----------------------------------------------------------------------------------------------------------------------


def _loss_case(n=4000, seed=3):
    g = torch.Generator().manual_seed(seed)
    logp = (torch.randn(n, generator=g) * 0.15).requires_grad_(True)
    old = torch.zeros(n, 1)
    adv = torch.randn(n, 1, generator=g)
    adv[:7] = 0.0
    values = (torch.randn(n, 1, generator=g) * 0.3).requires_grad_(True)
    old_v = torch.zeros(n, 1)
    ret = torch.randn(n, 1, generator=g) * 0.3
    ent = torch.full((n,), 1.3)
    return logp, old, adv, values, old_v, ret, ent


def _loss_grads(branch):
    logp, old, adv, values, old_v, ret, ent = _loss_case()
    s, v, loss = O.ppo_loss_terms(logp, old, adv, values, old_v, ret, ent, 0.2, True, 1.0, 0.01, branch)
    loss.backward()
    return logp.grad.clone(), values.grad.reshape(-1).clone(), (logp, old, adv, values, old_v, ret)


def test_branch_record_own_decisions_are_autograds():
    """The recorded decisions are exactly the rows where torch's autograd passes a non-zero gradient (max ties split,
    clamp closed interval), on rows spread over both sides of both boundaries, and forcing them changes nothing."""
    plain_lp, plain_v, _ = _loss_grads(None)
    rec = O.BranchRecord()
    lp, v, _ = _loss_grads(rec)
    assert torch.equal(lp, plain_lp) and torch.equal(v, plain_v)
    assert torch.equal(rec.own["surrogate"], plain_lp != 0)
    assert torch.equal(rec.own["value"], plain_v != 0)
    s = rec.own["surrogate"]
    assert 0 < int(s.sum()) < s.numel() and 0 < int(rec.own["value"].sum()) < s.numel()
    forced = O.BranchRecord({"surrogate": rec.own["surrogate"].clone(), "value": rec.own["value"].clone()})
    lp2, v2, _ = _loss_grads(forced)
    assert torch.equal(lp2, plain_lp) and torch.equal(v2, plain_v)
    assert all(idx.numel() == 0 for idx, _ in forced.flips.values())


def test_branch_record_forces_single_rows_and_reports_their_distance():
    """Forcing one row's surrogate off and another's on, and one value row on: only those rows' gradients change,
    to 0 and to the unclipped branch's -adv * ratio / R and 2 (V - R) / R; every other row is bit-identical, and the
    flips are reported with |ratio - (1 +- clip)| and the value rows' distance."""
    plain_lp, plain_v, (logp, old, adv, values, old_v, ret) = _loss_grads(None)
    n = plain_lp.numel()
    ratio = torch.exp(logp.detach() - old.squeeze(-1))
    on_rows = torch.nonzero(plain_lp != 0).reshape(-1)
    off_rows = torch.nonzero((plain_lp == 0) & (adv.squeeze(-1) != 0)).reshape(-1)
    voff = torch.nonzero(plain_v == 0).reshape(-1)
    i, j, kv = int(on_rows[0]), int(off_rows[0]), int(voff[0])
    s_mask = plain_lp != 0
    s_mask[i] = False
    s_mask[j] = True
    v_mask = plain_v != 0
    v_mask[kv] = True
    rec = O.BranchRecord({"surrogate": s_mask, "value": v_mask})
    lp, v, _ = _loss_grads(rec)
    keep = torch.ones(n, dtype=torch.bool)
    keep[[i, j]] = False
    assert torch.equal(lp[keep], plain_lp[keep])
    assert lp[i] == 0
    expect_j = -adv[j, 0] * ratio[j] / n
    assert torch.allclose(lp[j], expect_j, rtol=1e-6)
    keep_v = torch.ones(n, dtype=torch.bool)
    keep_v[kv] = False
    assert torch.equal(v[keep_v], plain_v[keep_v])
    assert torch.allclose(v[kv], 2 * (values[kv, 0] - ret[kv, 0]).detach() / n, rtol=1e-6)
    idx, dist = rec.flips["surrogate"]
    assert sorted(idx.tolist()) == sorted([i, j])
    r64 = ratio.double()
    for row, d in zip(idx.tolist(), dist.tolist()):
        assert d == pytest.approx(min(abs(float(r64[row]) - 1.2), abs(float(r64[row]) - 0.8)), rel=1e-12)
    assert rec.flips["value"][0].tolist() == [kv]
