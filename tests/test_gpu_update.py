"""Parity of the PPO update (all epochs x mini-batches) on the GPU against the CPU oracle.

Same seeded rollout, same initial weights, same bootstrap values, torch.manual_seed(1) before both updates.
Bars (the contract of this path): permutation / mini-batch rows bit-exact; GAE returns bit-exact and advantages
1e-6 relative; losses 1e-4 relative (surrogate against the mean |term| ~ O(1), its natural scale); identical
learning-rate decisions; every parameter tensor 1e-4 relative Frobenius.

Two complementary tests:

* test_update_steps_teacher_forced -- every optimiser step of the update is replayed on the GPU from the oracle's
  exact state before that step (parameters, Adam moments and step, learning rate; the packed mini-batch table of
  the whole update) and must land on the oracle's state after it: KL, learning-rate decision, losses, parameters
  and moments of every step.  This checks the numerics of all E x M steps, clipped samples included, without
  compounding.

* test_update_matches_oracle -- the drop-in update() end to end (state threading between steps, schedule,
  normaliser update).  The clipped surrogate max(-A r, -A clip(r)) is discontinuous in its gradient at
  r = 1 +- clip: a sample whose ratio lies within fp32 rounding of a boundary takes either branch depending on the
  last bits, and one changed branch moves the next Adam steps by O(lr) in some elements.  So the 1e-4 parameter
  bar over a whole multi-step trajectory is well posed only when the oracle's trajectory keeps every ratio at least
  CLIP_MARGIN away from the boundaries (oracle trace "clip_margin"); for trajectories that pass closer (the large
  cases: down to 5e-8) the end-to-end parameters get a 1e-2 sanity bar and the teacher-forced test carries the
  1e-4 bar.

The parameter bar is checked against two oracles: upstream's fp32 arithmetic (ref) and the same formulas with the
A-term log-prob sum accumulated in fp64 (ref_lp64, which is what the kernels evaluate).  Against ref_lp64 every
tensor must be within 1e-4.  Against ref it must be within max(1e-4, 1.5 x floor), floor = |ref_lp64 - ref|: for
29 actions the log-prob is ~-30 and its fp32 sum carries ~ulp(30) = 2e-6 of order-dependent rounding, which moves
the ratio by 2e-6 per row and the std parameter by ~1.1e-4 over 20 Adam steps -- in the oracle itself.
"""

from __future__ import annotations

import copy
from itertools import chain

import pytest
import torch

from oracle import rollout as R
from tests.parity import make_pair, oracle_logp_fp64, rel_err
from tt_rsl_rl_amd import ops

pytestmark = pytest.mark.gpu

CLIP_MARGIN = 1e-4
# a ratio this close to 1 +- clip can take either surrogate branch under fp32 rounding of a ~30-magnitude log-prob
AMBIGUOUS = 1e-5

def _lstm(num_envs: int, steps: int, hidden: int, hidden_dims: list[int], **kw) -> dict:
    w = R.scaled(R.WORKLOADS["lstm256"], num_envs=num_envs, steps=steps, hidden_dims=hidden_dims)
    w["rnn"] = dict(w["rnn"], rnn_hidden_dim=hidden)
    w.update(kw)
    return w


CASES = {
    # the headline workload at its full size: 4096 envs x 24 steps, 5 epochs x 4 mini-batches of 24,576 rows
    "humanoid_full": (R.WORKLOADS["humanoid"], {}),
    "humanoid_1k": (R.scaled(R.WORKLOADS["humanoid"], num_envs=1024), {}),
    "flat48_1k": (R.scaled(R.WORKLOADS["flat48"], num_envs=1024), {}),
    "rough235_512": (R.scaled(R.WORKLOADS["rough235"], num_envs=512), {}),
    "humanoid_small_permb_adv": (R.scaled(R.WORKLOADS["humanoid"], num_envs=128, steps=8, hidden_dims=[64, 32]),
                                 {"normalize_advantage_per_mini_batch": True, "num_mini_batches": 3}),
    "flat48_unclipped_fixed": (R.scaled(R.WORKLOADS["flat48"], num_envs=200, steps=5, hidden_dims=[128, 64, 32]),
                               {"use_clipped_value_loss": False, "schedule": "fixed", "num_learning_epochs": 2}),
    # 40 actions on a 48-wide last hidden layer: outside the fused head's shapes, the separate output-layer path
    "flat48_a40_unfused": (dict(R.scaled(R.WORKLOADS["flat48"], num_envs=256, steps=8, hidden_dims=[64, 48]),
                                num_actions=40), {}),
    # recurrent (LSTM before the MLP head): env-slice mini-batches, sequences started from the saved states
    "lstm256_512": (_lstm(512, 24, 256, [256, 128]), {}),
    "lstm64_norm_carry": (_lstm(128, 16, 64, [64, 32], obs_normalization=True), {"carry_state": True}),
    "lstm32_ragged_permb_fixed": (_lstm(200, 10, 32, [32, 32, 16]),
                                  {"num_mini_batches": 3, "normalize_advantage_per_mini_batch": True,
                                   "schedule": "fixed", "use_clipped_value_loss": False, "carry_state": True}),
}


# cases whose output layers fall outside the fused head (more than 32 actions, or a last hidden width that is not a
# multiple of 16)
UNFUSED = {"flat48_a40_unfused"}


def _table_order(ora, hip) -> torch.Tensor:
    """Storage row of every packed-table row: the oracle's permutation (feed-forward) or, for the recurrent update,
    each env slice's rows t-major (what upstream's recurrent generator yields as [T, E] blocks)."""
    engine = hip._get_engine()
    if engine.recurrent:
        return engine.order.cpu()
    return torch.cat([t["indices"] for t in ora.trace[:ora.num_mini_batches]])


def _update_both(name):
    w, over = CASES[name]
    ora, hip, roll = make_pair(w, seed=0, **over)
    st_o, st_h = ora.storage, hip.storage
    assert torch.equal(st_h.returns.cpu(), st_o.returns), "GAE returns must be bit-exact"
    assert rel_err(st_h.advantages, st_o.advantages) < 1e-6
    ora_lp64 = copy.deepcopy(ora)
    torch.manual_seed(1)
    ref = ora.update()
    with oracle_logp_fp64():
        torch.manual_seed(1)
        ora_lp64.update()
    torch.manual_seed(1)
    out = hip.update()
    torch.cuda.synchronize()
    hip.ora_lp64 = ora_lp64
    return w, over, ora, hip, ref, out


@pytest.mark.parametrize("name", list(CASES))
def test_update_matches_oracle(name):
    w, over, ora, hip, ref, out = _update_both(name)
    # permutation / mini-batch rows: the packed table holds storage rows in oracle permutation order
    B = w["num_envs"] * w["steps"]
    perm = _table_order(ora, hip)
    lay = hip._engine.layout
    A = w["num_actions"]
    acts = hip._engine.table[:, lay.actions:lay.actions + A].cpu()
    assert torch.equal(acts, ora.storage.actions.flatten(0, 1)[perm]), "mini-batch rows must be bit-exact"
    assert perm.numel() == B
    # the fused output-layer + loss launch runs wherever it takes the shapes
    assert hip._engine.fused_head == (name not in UNFUSED), name
    # learning-rate decisions
    assert [t["lr"] for t in hip.last_trace] == [t["lr"] for t in ora.trace]
    assert hip.learning_rate == ora.learning_rate
    # losses
    for k, scale in (("value", 0.0), ("surrogate", 0.1), ("entropy", 0.0)):
        den = max(abs(ref[k]), scale)
        assert abs(out[k] - ref[k]) <= 1e-4 * den, (k, out[k], ref[k])
    # parameters and optimiser moments
    margin = min(t["clip_margin"] for t in ora.trace)
    bar = 1e-4 if margin >= CLIP_MARGIN else 1e-2
    print(f"oracle trajectory clip margin {margin:.2e} -> end-to-end parameter bar {bar:g}")
    ora64 = hip.ora_lp64
    for model_h, model_o, model_64 in ((hip.actor, ora.actor, ora64.actor), (hip.critic, ora.critic, ora64.critic)):
        for (name_p, p_o), p_h, p_64 in zip(model_o.named_parameters(), model_h.parameters(), model_64.parameters()):
            floor = rel_err(p_64, p_o)
            err, err64 = rel_err(p_h, p_o), rel_err(p_h, p_64)
            print(f"{name_p:28s} vs oracle {err:.2e} (floor {floor:.2e})  vs lp64 oracle {err64:.2e}")
            assert err64 < bar, name_p
            assert err < max(bar, 1.5 * floor), name_p
            s_o = ora.optimizer.state[p_o]
            s_h = hip.optimizer.state[p_h]
            s_64 = ora64.optimizer.state[p_64]
            assert rel_err(s_h["exp_avg"], s_64["exp_avg"], 1e-12) < 10 * bar, name_p
            assert rel_err(s_h["exp_avg_sq"], s_64["exp_avg_sq"], 1e-20) < 10 * bar, name_p
            assert float(s_h["step"]) == float(s_o["step"])
    # normaliser statistics (updated after the epochs from all stored observations)
    if w["obs_normalization"]:
        for m_h, m_o in ((hip.actor, ora.actor), (hip.critic, ora.critic)):
            n_h, n_o = m_h.obs_normalizer, m_o.obs_normalizer
            assert int(n_h.count) == int(n_o.count)
            assert rel_err(n_h._mean, n_o._mean) < 1e-6
            assert rel_err(n_h._var, n_o._var) < 1e-6


def test_recorded_launches_match_rebuilt_launches():
    """From the third update on, the engine issues each mini-batch from its recorded launch sequence (only Adam's bias
    corrections recomputed); those updates must equal, bit for bit, updates whose every launch is rebuilt in Python:
    parameters, Adam moments, losses and learning rate, over several consecutive updates (obs normalisation on, so the
    frozen normaliser statistics and the normaliser update are exercised too)."""
    w = R.scaled(R.WORKLOADS["humanoid"], num_envs=256, steps=8, hidden_dims=[64, 32])
    _, a, _ = make_pair(w, seed=0)
    _, b, _ = make_pair(w, seed=0)
    for alg, replay in ((a, True), (b, False)):
        alg._get_engine().replay = replay
    for rep in range(4):
        outs = []
        for alg in (a, b):
            alg.storage.step = alg.storage.num_transitions_per_env
            torch.manual_seed(1 + rep)
            outs.append(alg.update())
        torch.cuda.synchronize()
        assert outs[0] == outs[1], rep
        assert a.learning_rate == b.learning_rate
        for pa, pb in zip(chain(a.actor.parameters(), a.critic.parameters()),
                          chain(b.actor.parameters(), b.critic.parameters())):
            assert torch.equal(pa, pb), rep
        assert torch.equal(a.flat.exp_avg, b.flat.exp_avg) and torch.equal(a.flat.exp_avg_sq, b.flat.exp_avg_sq)
        for ma, mb in ((a.actor, b.actor), (a.critic, b.critic)):
            assert torch.equal(ma.obs_normalizer._mean, mb.obs_normalizer._mean)
    assert a._engine.replays > 0 and b._engine.replays == 0


def _adam_state(opt, p):
    st = opt.state.get(p, {})
    if "exp_avg" not in st:
        return torch.zeros_like(p), torch.zeros_like(p), 0
    return st["exp_avg"].clone(), st["exp_avg_sq"].clone(), int(st["step"])


@pytest.mark.parametrize("name", list(CASES))
def test_update_steps_teacher_forced(name):
    w, over = CASES[name]
    ora, hip, _ = make_pair(w, seed=0, **over)
    snaps = []

    def record(phase, alg):
        params = list(chain(alg.actor.parameters(), alg.critic.parameters()))
        moments = [_adam_state(alg.optimizer, p) for p in params]
        snaps.append((phase, {"params": [p.detach().clone() for p in params], "lr": alg.learning_rate,
                              "exp_avg": [m[0] for m in moments], "exp_avg_sq": [m[1] for m in moments],
                              "step": moments[0][2]}))

    ora.recorder = record
    torch.manual_seed(1)
    ora.update()
    pre = [s for ph, s in snaps if ph == "pre"]
    post = [s for ph, s in snaps if ph == "post"]
    M, B = ora.num_mini_batches, w["num_envs"] * w["steps"]
    assert len(pre) == len(post) == len(ora.trace) == ora.num_learning_epochs * M

    # the GPU side: the update's packed table (same permutation), then one step at a time from the oracle's state
    engine = hip._get_engine()
    engine.gather(None if engine.recurrent else _table_order(ora, hip).to(hip.device))
    params = list(chain(hip.actor.parameters(), hip.critic.parameters()))
    names = [n for n, _ in chain(ora.actor.named_parameters(), ora.critic.named_parameters())]
    worst, n_amb = 0.0, 0
    for k, (a, b) in enumerate(zip(pre, post)):
        with torch.no_grad():
            for p, v, m1, m2 in zip(params, a["params"], a["exp_avg"], a["exp_avg_sq"]):
                p.copy_(v.to(hip.device))
                hip.flat.exp_avg_view(p).copy_(m1.to(hip.device))
                hip.flat.exp_avg_sq_view(p).copy_(m2.to(hip.device))
        ops.reset_device_state(hip.device_state, a["lr"])
        engine.minibatch(*engine.minibatch_rows(k % M), a["step"] + 1)
        torch.cuda.synchronize()
        kl, lr, surr, value, ent = engine.trace[:5].tolist()
        t = ora.trace[k]
        assert lr == t["lr"], (k, lr, t["lr"])
        if t["kl_mean"] is not None:
            assert abs(kl - t["kl_mean"]) <= 1e-4 * max(t["kl_mean"], 1e-6), (k, kl, t["kl_mean"])
        assert abs(value - t["value"]) <= 1e-4 * abs(t["value"]), (k, value, t["value"])
        assert abs(surr - t["surrogate"]) <= 1e-4 * max(abs(t["surrogate"]), 0.1), (k, surr, t["surrogate"])
        assert abs(ent - t["entropy"]) <= 1e-4 * abs(t["entropy"]), (k, ent, t["entropy"])
        # a sample on a clip boundary may take the other branch: its gradient term then moves the moments (and,
        # through Adam, the parameters) by about one sample's share
        ambiguous = t["clip_margin"] < AMBIGUOUS
        n_amb += ambiguous
        p_bar, m_bar = (1e-3, 1e-2) if ambiguous else (1e-4, 1e-3)
        for n, p, v, m1, m2 in zip(names, params, b["params"], b["exp_avg"], b["exp_avg_sq"]):
            err = rel_err(p, v)
            if not ambiguous:
                worst = max(worst, err)
            assert err < p_bar, (k, n, err)
            assert rel_err(hip.flat.exp_avg_view(p), m1, 1e-12) < m_bar, (k, n)
            assert rel_err(hip.flat.exp_avg_sq_view(p), m2, 1e-20) < m_bar, (k, n)
    print(f"{name}: {len(pre)} teacher-forced steps ({n_amb} with a ratio within {AMBIGUOUS:g} of a clip boundary), "
          f"worst parameter rel error on the others {worst:.2e}")


def test_state_dict_and_checkpoint_round_trip(tmp_path):
    w, over = CASES["humanoid_small_permb_adv"]
    _, _, ora, hip, _, _ = _update_both("humanoid_small_permb_adv")
    saved = hip.save()
    assert list(saved["actor_state_dict"].keys()) == list(ora.actor.state_dict().keys())
    assert list(saved["critic_state_dict"].keys()) == list(ora.critic.state_dict().keys())
    osd_h, osd_o = saved["optimizer_state_dict"], ora.optimizer.state_dict()
    assert osd_h["param_groups"][0]["params"] == osd_o["param_groups"][0]["params"]
    assert osd_h["param_groups"][0]["lr"] == osd_o["param_groups"][0]["lr"]
    # upstream-format checkpoint -> fresh plugin
    path = tmp_path / "model.pt"
    torch.save({**ora.save(), "iter": 3, "infos": None}, path)
    from tests.parity import make_hip

    fresh = make_hip(w, seed=5, **over)
    fresh.load(torch.load(path, weights_only=True), None, True)
    for (n, p_o), p_h in zip(ora.actor.named_parameters(), fresh.actor.parameters()):
        assert torch.equal(p_h.detach().cpu(), p_o.detach()), n
    for p_o, p_h in zip(ora.optimizer.param_groups[0]["params"], fresh.optimizer.param_groups[0]["params"]):
        assert torch.equal(fresh.optimizer.state[p_h]["exp_avg"].cpu(), ora.optimizer.state[p_o]["exp_avg"])
    assert fresh.learning_rate == ora.learning_rate


@pytest.mark.parametrize("name", ["humanoid", "flat48_65k", "lstm256"])
def test_full_size_update_properties(name):
    """At full size (humanoid and lstm256: 4096 envs x 24 steps; flat48_65k: 65,536 envs x 24 steps, mini-batches of
    393,216 rows; humanoid is also compared with the oracle in test_update_matches_oracle): the update runs, the losses are finite, parameters moved
    by at most 20 Adam steps' worth (the lr is clamped to [1e-5, 1e-2]), and two identical updates give bit-identical
    parameters (deterministic reductions).  lstm256 starts its sequences from random saved states."""
    from tests.parity import make_hip

    w = R.WORKLOADS[name]
    results = []
    for _ in range(2):
        hip = make_hip(w, seed=0)
        g = torch.Generator().manual_seed(7)
        st = hip.storage
        for k, v in st.observations.items():
            v.copy_(torch.randn(v.shape, generator=g))
        st.actions.copy_(torch.randn(st.actions.shape, generator=g))
        st.rewards.copy_(torch.randn(st.rewards.shape, generator=g) * 0.2)
        st.values.copy_(torch.randn(st.values.shape, generator=g))
        st.dones.copy_((torch.rand(st.dones.shape, generator=g) < 0.01).to(torch.uint8))
        mean = torch.randn(st.actions.shape, generator=g)
        st.distribution_params = (mean.to(hip.device), torch.ones_like(st.actions))
        st.actions_log_prob.copy_(torch.distributions.Normal(mean, 1.0).log_prob(st.actions.cpu()).sum(-1, keepdim=True))
        if "rnn" in w:
            H, T, N = w["rnn"]["rnn_hidden_dim"], w["steps"], w["num_envs"]
            for side in ("a", "c"):
                setattr(st, f"saved_hidden_state_{side}",
                        [(0.5 * torch.randn(T, 1, N, H, generator=g)).to(hip.device) for _ in range(2)])
        st.step = st.num_transitions_per_env
        hip.compute_returns_from(torch.randn(w["num_envs"], 1, generator=g).to(hip.device))
        params = list(hip.actor.parameters()) + list(hip.critic.parameters())
        p0 = torch.cat([p.detach().reshape(-1).clone() for p in params])
        torch.manual_seed(1)
        out = hip.update()
        p1 = torch.cat([p.detach().reshape(-1) for p in params])
        assert all(torch.isfinite(torch.tensor(v)) for v in out.values()), out
        assert torch.isfinite(p1).all()
        assert (p1 - p0).abs().max().item() <= 20 * 1e-2 * 1.01
        assert (p1 != p0).any()
        results.append(p1.cpu())
        del hip
    assert torch.equal(results[0], results[1]), "the update must be deterministic"
