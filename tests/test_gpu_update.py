"""Parity of the PPO update (all epochs x mini-batches) on the GPU against the CPU oracle.

Same seeded rollout, same initial weights, same bootstrap values, torch.manual_seed(1) before both updates.

Acceptance rule (the contract of this path):
  * exact: permutation / mini-batch rows, GAE returns, learning-rate decisions, Adam step counts;
  * advantages 1e-6 relative; losses 1e-4 relative (surrogate against max(|ref|, 0.1), its natural scale);
  * per mini-batch, every row's ratio exp(logp - old_logp) within 1e-4 of the oracle's, and its value V within 1e-4
    of the oracle's (relative to the largest |V|), for a step from the oracle's state (1e-3 along a whole update);
  * every parameter tensor within 1e-4 relative Frobenius (Adam moments 1e-3) of the oracle trajectory that takes the
    GPU's clip-branch decision on every row where the two differ, and every such row explained: its distance to the
    boundary in the oracle's evaluation is at most that row's |GPU quantity - oracle quantity| + 1e-5 (the kernels'
    own fp32 rounding), so the two evaluations lie on the two sides of the boundary;
  * in function space (actor mean and critic value on the rollout's observations; the metric of the reference's
    tests/tt/test_tt_update.py:348-351): the GPU's update differs from that branch-matched oracle's by at most 1e-4 of
    the update, and from upstream's literal evaluation by at most the listed near-boundary rows' own effect
    (d(branch-matched oracle, oracle)) + 1e-4.

Why branch-matched.  The clipped surrogate max(-A r, -A clamp(r)) and the clipped value loss have gradients that jump
at the clip boundaries: a row whose ratio lies within fp32 rounding of 1 +- clip (ulp(30) ~ 2e-6 in a 29-term
log-prob) passes -A or nothing depending on the last bits, and any two fp32 evaluations of the same formulas (the
oracle itself with its log-prob summed in another order, say) disagree on such rows now and then.  One such row moves
one step's gradient by one row's share, and Adam's normalised steps carry it on.  The oracle therefore replays the
update taking the GPU's decision on those rows (``oracle.PPO.forced_branches``; the decision is read from the GPU's
per-row output gradients, exactly zero iff the row's gradient is), lists every row where it differs from its own, and
must then agree at 1e-4.  The oracle's own spread (its fp32 log-prob sum against an fp64 one) is printed beside:
it is of the same size as the GPU's distance from the literal oracle (both are one or two such rows' effect).

Two complementary tests, both on every case (the five workloads at full size included: 4096 envs x 24 steps, and
65,536 envs x 24 steps with mini-batches of 393,216 rows):
  * test_update_matches_oracle -- the drop-in update() end to end (state threading between steps, schedule,
    normaliser update);
  * test_update_steps_teacher_forced -- every optimiser step replayed on the GPU from the oracle's exact state before
    it (parameters, Adam moments and step, learning rate) against the oracle's state after it: the numerics of every
    step without compounding.

With PPO_PARITY_RECORD=<dir> in the environment each case also writes what it measured to <dir>/<test>_<case>.json:
the rows on another clip branch and their distances, every parameter tensor's error against the branch-matched and
the literal oracle and the oracle's own spread, the function-space figures and the losses.
"""

from __future__ import annotations

import copy
import functools
import json
import os
import time
from itertools import chain

import pytest
import torch

from oracle import rollout as R
from tests.parity import (eval_observations, flipped_rows, function_deviation, hip_branch_rows, hip_quantities,
                          make_hip, oracle_logp_fp64, param_dict, quantity_gap, rel_err, unexplained_flips)
from tt_rsl_rl_amd import ops

pytestmark = pytest.mark.gpu

# the kernels' own fp32 rounding of a row's ratio (a 29-term log-prob of magnitude ~30: ulp(30) = 2e-6 per term
# order) and of its value: a row whose GPU quantity lies this close to a boundary may take either side
AMBIGUOUS = 1e-5
# the GPU's and the oracle's per-row ratio / value (relative) in a mini-batch step from the same state; over a whole
# update the two trajectories' parameters drift apart by a few 1e-6, which a 29-term log-prob with outlier actions
# turns into ratio differences of ~1e-4 on the extreme rows, hence the wider end-to-end bar
QUANTITY_BAR = 1e-4
QUANTITY_BAR_END_TO_END = 1e-3
PARAM_BAR = 1e-4
MOMENT_BAR = 1e-3
FUNCTION_BAR = 1e-4


def _lstm(num_envs: int, steps: int, hidden: int, hidden_dims: list[int], layers: int = 1, rnn_type: str = "lstm",
          **kw) -> dict:
    w = R.scaled(R.WORKLOADS["lstm256"], num_envs=num_envs, steps=steps, hidden_dims=hidden_dims)
    w["rnn"] = dict(w["rnn"], rnn_hidden_dim=hidden, rnn_num_layers=layers, rnn_type=rnn_type)
    w.update(kw)
    return w


CASES = {
    # the four single-GPU feed-forward workloads at their full size (4096 envs x 24 steps, 5 epochs x 4 mini-batches
    # of 24,576 rows; 65,536 envs: mini-batches of 393,216 rows) and the recurrent one (4096 envs, LSTM 256)
    "humanoid_full": (R.WORKLOADS["humanoid"], {}),
    "flat48_full": (R.WORKLOADS["flat48"], {}),
    "rough235_full": (R.WORKLOADS["rough235"], {}),
    "flat48_65k": (R.WORKLOADS["flat48_65k"], {}),
    "lstm256_full": (R.WORKLOADS["lstm256"], {}),
    # smaller shapes and the options off the default path
    "humanoid_1k": (R.scaled(R.WORKLOADS["humanoid"], num_envs=1024), {}),
    "rough235_512": (R.scaled(R.WORKLOADS["rough235"], num_envs=512), {}),
    "humanoid_small_permb_adv": (R.scaled(R.WORKLOADS["humanoid"], num_envs=128, steps=8, hidden_dims=[64, 32]),
                                 {"normalize_advantage_per_mini_batch": True, "num_mini_batches": 3}),
    "flat48_unclipped_fixed": (R.scaled(R.WORKLOADS["flat48"], num_envs=200, steps=5, hidden_dims=[128, 64, 32]),
                               {"use_clipped_value_loss": False, "schedule": "fixed", "num_learning_epochs": 2}),
    # a fixed std (learn_std=False): no gradient, no Adam state and no clip-norm share for the std parameter
    "humanoid_small_fixed_std": (dict(R.scaled(R.WORKLOADS["humanoid"], num_envs=128, steps=8, hidden_dims=[64, 32]),
                                      learn_std=False), {}),
    # other hidden-layer activations (rsl_rl/utils/utils.py:34-68): tanh (act' from the output), gelu (from the
    # stored input), actor relu with a softplus critic (one launch per model); the separate output-layer path
    "humanoid_small_tanh": (dict(R.scaled(R.WORKLOADS["humanoid"], num_envs=128, steps=8, hidden_dims=[64, 32]),
                                 activation="tanh"), {}),
    "flat48_small_gelu": (dict(R.scaled(R.WORKLOADS["flat48"], num_envs=256, steps=8, hidden_dims=[128, 64, 32]),
                               activation="gelu"), {}),
    "rough235_small_relu_softplus": (dict(R.scaled(R.WORKLOADS["rough235"], num_envs=128, steps=8,
                                                   hidden_dims=[64, 32]), activation="relu",
                                          critic_activation="softplus"), {}),
    # 40 actions on a 48-wide last hidden layer: outside the fused head's shapes, the separate output-layer path
    "flat48_a40_unfused": (dict(R.scaled(R.WORKLOADS["flat48"], num_envs=256, steps=8, hidden_dims=[64, 48]),
                                num_actions=40), {}),
    # recurrent (LSTM before the MLP head): env-slice mini-batches, sequences started from the saved states
    "lstm256_512": (_lstm(512, 24, 256, [256, 128]), {}),
    "lstm64_norm_carry": (_lstm(128, 16, 64, [64, 32], obs_normalization=True), {"carry_state": True}),
    "lstm32_ragged_permb_fixed": (_lstm(200, 10, 32, [32, 32, 16]),
                                  {"num_mini_batches": 3, "normalize_advantage_per_mini_batch": True,
                                   "schedule": "fixed", "use_clipped_value_loss": False, "carry_state": True}),
    # two stacked LSTM layers (layer 1 reads layer 0's h): the hidden size of the workload and a small one
    "lstm256x2_512": (_lstm(512, 24, 256, [256, 128], layers=2), {"carry_state": True}),
    "lstm32x3_ragged": (_lstm(200, 10, 32, [32, 16], layers=3), {"num_mini_batches": 3, "carry_state": True}),
    # the other optimisers upstream resolves (rsl_rl/utils/utils.py:71-96), each with torch's defaults
    "humanoid_small_adamw": (R.scaled(R.WORKLOADS["humanoid"], num_envs=128, steps=8, hidden_dims=[64, 32]),
                             {"optimizer": "adamw"}),
    "flat48_small_sgd": (R.scaled(R.WORKLOADS["flat48"], num_envs=256, steps=8, hidden_dims=[128, 64, 32]),
                         {"optimizer": "sgd", "learning_rate": 1e-2}),
    "rough235_small_rmsprop": (R.scaled(R.WORKLOADS["rough235"], num_envs=128, steps=8, hidden_dims=[64, 32]),
                               {"optimizer": "RMSprop", "schedule": "fixed", "learning_rate": 3e-4}),
    "lstm64_adamw": (_lstm(128, 16, 64, [64, 32]), {"optimizer": "adamw"}),
    # GRU (rsl_rl/modules/rnn.py:29): the workload's shape, a normalised small one, two layers on ragged slices
    "gru256_512": (_lstm(512, 24, 256, [256, 128], rnn_type="gru"), {"carry_state": True}),
    "gru64_norm": (_lstm(128, 16, 64, [64, 32], rnn_type="gru", obs_normalization=True), {}),
    "gru32x2_ragged_permb": (_lstm(200, 10, 32, [32, 16], layers=2, rnn_type="gru"),
                             {"num_mini_batches": 3, "normalize_advantage_per_mini_batch": True, "carry_state": True}),
    # the recurrent update with one launch per step (PPO_HIP_LSTM_SEQ=0: the heads' weight-grads on a second stream)
    "lstm64_per_step_launches": (_lstm(128, 16, 64, [64, 32]), {"carry_state": True, "per_step_launches": True}),
    "gru32x2_per_step_launches": (_lstm(200, 10, 32, [32, 16], layers=2, rnn_type="gru"),
                                  {"num_mini_batches": 3, "per_step_launches": True}),
}

# an oracle update of the 65,536-env workload takes ~45 s of CPU time on 16 threads, and the end-to-end test runs it
# up to three times (literal, branch-matched, fp64 log-prob spread): a limit of its own, progress lines as it goes
LONG = {"flat48_65k"}


def _cases():
    return [pytest.param(n, marks=pytest.mark.timeout(1200)) if n in LONG else n for n in CASES]


def _progress(capsys, name: str, msg: str, t0: list) -> None:
    """A progress line on the terminal for the long cases (outside pytest's capture)."""
    if name in LONG:
        with capsys.disabled():
            print(f"  [{name} +{time.time() - t0[0]:.0f}s] {msg}", flush=True)


def _record(test: str, name: str, data: dict) -> None:
    """Write a case's measured figures to $PPO_PARITY_RECORD/<test>_<name>.json (nothing without the variable)."""
    out = os.environ.get("PPO_PARITY_RECORD")
    if not out:
        return
    os.makedirs(out, exist_ok=True)
    with open(os.path.join(out, f"{test}_{name}.json"), "w") as f:
        json.dump(data, f, indent=1, sort_keys=True)

# cases whose output layers fall outside the fused head (more than 32 actions, or a last hidden width that is not a
# multiple of 16)
UNFUSED = {"flat48_a40_unfused", "humanoid_small_tanh", "flat48_small_gelu", "rough235_small_relu_softplus"}


@functools.lru_cache(maxsize=None)
def _rollout(name: str):
    """The oracle (before its update) and its recorded rollout, generated once per case for both tests."""
    w, over = CASES[name]
    over = dict(over)
    carry = over.pop("carry_state", False)
    over.pop("per_step_launches", None)
    ora, roll = R.generate(w, 0, carry_state=carry, **over)
    with torch.inference_mode():
        last_values = ora.critic(roll.last_obs).detach()
    ora.compute_returns(roll.last_obs, last_values=last_values)
    return ora, roll, last_values


def _pair(name: str):
    """A fresh copy of the case's oracle and a HIP plugin with the same weights, rollout and returns."""
    w, over = CASES[name]
    per_step = over.get("per_step_launches", False)
    over = {k: v for k, v in over.items() if k not in ("carry_state", "per_step_launches")}
    ora0, roll, last_values = _rollout(name)
    ora = copy.deepcopy(ora0)
    hip = make_hip(w, 0, **over)
    with torch.no_grad():
        hip.actor.load_state_dict(roll.init_state["actor"])
        hip.critic.load_state_dict(roll.init_state["critic"])
    R.feed(hip.storage, roll)
    hip.compute_returns_from(last_values.to(hip.device).contiguous())
    if per_step:  # the recurrent engine reads the switch when it is built: one launch per step, head dw beside them
        old = os.environ.get("PPO_HIP_LSTM_SEQ")
        os.environ["PPO_HIP_LSTM_SEQ"] = "0"
        try:
            assert hip._get_engine().lstm_sync is None
        finally:
            if old is None:
                del os.environ["PPO_HIP_LSTM_SEQ"]
            else:
                os.environ["PPO_HIP_LSTM_SEQ"] = old
    return w, ora, hip


def _table_order(ora, hip) -> torch.Tensor:
    """Storage row of every packed-table row: the oracle's permutation (feed-forward) or, for the recurrent update,
    each env slice's rows t-major (what upstream's recurrent generator yields as [T, E] blocks)."""
    engine = hip._get_engine()
    if engine.recurrent:
        return engine.order.cpu()
    return torch.cat([t["indices"] for t in ora.trace[:ora.num_mini_batches]])


@pytest.mark.parametrize("name", _cases())
def test_update_matches_oracle(name, capsys):
    t0 = [time.time()]
    w, ora, hip = _pair(name)
    _progress(capsys, name, "rollout and returns ready", t0)
    st_o, st_h = ora.storage, hip.storage
    assert torch.equal(st_h.returns.cpu(), st_o.returns), "GAE returns must be bit-exact"
    adv_err = rel_err(st_h.advantages, st_o.advantages)
    assert adv_err < 1e-6
    p0 = param_dict(ora)
    ev = eval_observations(ora)
    lp64, shadow = copy.deepcopy(ora), copy.deepcopy(ora)
    torch.manual_seed(1)
    ref = ora.update()
    _progress(capsys, name, "oracle update done", t0)
    with oracle_logp_fp64():
        torch.manual_seed(1)
        lp64.update()
    _progress(capsys, name, "oracle update with fp64 log-prob sums done", t0)

    # the drop-in update(), with each mini-batch's clip-branch decisions read back
    engine = hip._get_engine()
    if engine.recurrent:  # one optimiser launch where one weight-grad launch holds every layer's and head's problems
        n_rnn = len(engine.lay_a) + len(engine.lay_c)
        n_head = len(hip.actor.linears) + len(hip.critic.linears)
        from tt_rsl_rl_amd import _lib as L

        fits = engine.lstm_sync is not None and 2 * n_rnn + n_head <= L.MAX_LINEAR_PROBLEMS
        assert (engine.rnn_norm is not None) == fits, name
    std_param = hip.actor.distribution.param
    rows: list[dict] = []
    quantities: list[dict] = []
    std_before = [std_param.detach().clone()]

    def hook(e, r0, r1):
        rows.append(hip_branch_rows(e, r1 - r0))
        quantities.append(hip_quantities(e, r0, r1, std_before[-1]))
        std_before.append(std_param.detach().clone())  # the std parameter the next step starts from

    engine.step_hook = hook
    torch.manual_seed(1)
    out = hip.update()
    torch.cuda.synchronize()
    engine.step_hook = None
    assert len(rows) == len(ora.trace)
    _progress(capsys, name, "GPU update done", t0)

    # the oracle trajectory with the GPU's decisions on the rows where they differ (where the GPU took the oracle's
    # own decision on every row of every step, forcing changes nothing: that trajectory is the oracle's, bit for bit)
    same = all(torch.equal(r[kind], own) for r, t in zip(rows, ora.trace) for kind, own in t["branches"].own.items())
    if same:
        shadow, ref_s = ora, ref
    else:
        shadow.forced_branches = rows
        torch.manual_seed(1)
        ref_s = shadow.update()
        _progress(capsys, name, "branch-matched oracle update done", t0)
    flips = flipped_rows(shadow.trace)
    gaps = []
    for k, (t, q) in enumerate(zip(shadow.trace, quantities)):
        gap = quantity_gap(t["branches"], q)
        gaps.append(gap)
        for kind, d in gap.items():
            assert d < QUANTITY_BAR_END_TO_END, (name, k, kind, d)
        bad = unexplained_flips(t["branches"], q, AMBIGUOUS)
        assert not bad, (name, k, bad)

    # permutation / mini-batch rows: the packed table holds storage rows in oracle permutation order
    B = w["num_envs"] * w["steps"]
    perm = _table_order(ora, hip)
    lay = engine.layout
    A = w["num_actions"]
    acts = engine.table[:, lay.actions:lay.actions + A].cpu()
    assert torch.equal(acts, ora.storage.actions.flatten(0, 1)[perm]), "mini-batch rows must be bit-exact"
    assert perm.numel() == B
    assert engine.fused_head == (name not in UNFUSED), name
    # learning-rate decisions
    assert [t["lr"] for t in hip.last_trace] == [t["lr"] for t in shadow.trace] == [t["lr"] for t in ora.trace]
    assert hip.learning_rate == ora.learning_rate
    # losses, against both oracle trajectories
    for r in (ref, ref_s):
        for k, scale in (("value", 0.0), ("surrogate", 0.1), ("entropy", 0.0)):
            assert abs(out[k] - r[k]) <= 1e-4 * max(abs(r[k]), scale), (k, out[k], r[k])
    # parameters and optimiser moments against the branch-matched oracle
    worst, tensors = 0.0, {}
    for tag, model_h, model_s, model_o, model_64 in (("actor", hip.actor, shadow.actor, ora.actor, lp64.actor),
                                                     ("critic", hip.critic, shadow.critic, ora.critic, lp64.critic)):
        for (name_p, p_s), p_h, p_o, p_64 in zip(model_s.named_parameters(), model_h.parameters(),
                                                 model_o.parameters(), model_64.parameters()):
            err = rel_err(p_h, p_s)
            worst = max(worst, err)
            if not p_s.requires_grad:  # (learn_std=False: untouched, and no optimiser state on either side)
                assert not p_h.requires_grad and torch.equal(p_h.detach().cpu(), p_s.detach()), name_p
                assert p_s not in shadow.optimizer.state and p_h not in hip.optimizer.state, name_p
                continue
            # the optimiser's state (Adam / AdamW: exp_avg, exp_avg_sq; RMSprop: square_avg; SGD: none), same keys
            s_s, s_h = shadow.optimizer.state.get(p_s, {}), hip.optimizer.state.get(p_h, {})
            assert set(s_h) == set(s_s), (name_p, set(s_h), set(s_s))
            rec = {"vs_branch_matched": err, "vs_literal_oracle": rel_err(p_h, p_o),
                   "oracle_spread_lp64_vs_oracle": rel_err(p_64, p_o)}
            for key in sorted(k for k in s_s if k != "step"):
                rec[f"{key}_vs_branch_matched"] = rel_err(s_h[key], s_s[key], _STATE_FLOOR.get(key, 1e-20))
                assert rec[f"{key}_vs_branch_matched"] < MOMENT_BAR, (name_p, key)
            tensors[f"{tag}.{name_p}"] = rec
            print(f"{tag}.{name_p:28s} vs branch-matched oracle {err:.2e}   vs oracle {rel_err(p_h, p_o):.2e}   "
                  f"(oracle's own spread: lp64 vs oracle {rel_err(p_64, p_o):.2e})")
            assert err < PARAM_BAR, name_p
            if "step" in s_s:
                assert float(s_h["step"]) == float(s_s["step"])
    # function space
    p_h, p_s, p_o, p_64 = param_dict(hip), param_dict(shadow), param_dict(ora), param_dict(lp64)
    d_hs = function_deviation(p_h, p_s, p0, ora, ev)
    d_ho = function_deviation(p_h, p_o, p0, ora, ev)
    d_so = function_deviation(p_s, p_o, p0, ora, ev)
    spread = function_deviation(p_64, p_o, p0, ora, ev)
    worst_gap = {kind: max(g.get(kind, 0.0) for g in gaps) for kind in ("surrogate", "value")}
    _record("update", name, {
        "case": name, "rows": B, "mini_batches": len(rows), "returns_bit_exact": True, "advantages_rel_err": adv_err,
        "rows_on_another_branch": [{"step": k, "kind": kind, "row": i, "distance_to_boundary": d}
                                   for k, kind, i, d in flips],
        "branch_matched_oracle_replayed": not same,
        "worst_param_err_vs_branch_matched": worst, "tensors": tensors,
        "largest_ratio_gap": worst_gap["surrogate"], "largest_value_gap": worst_gap["value"],
        "function_space": {t: {"gpu_vs_branch_matched": d_hs[t], "gpu_vs_literal_oracle": d_ho[t],
                               "branch_matched_vs_literal_oracle": d_so[t], "oracle_spread_lp64_vs_oracle": spread[t]}
                           for t in ("actor", "critic")},
        "losses": {"gpu": out, "literal_oracle": ref, "branch_matched_oracle": ref_s},
        "learning_rates_equal": True, "final_learning_rate": hip.learning_rate})
    print(f"{name}: {len(flips)} row(s) on another branch {[(k, kind, round(d, 9)) for k, kind, _, d in flips]}; "
          f"worst parameter error {worst:.2e}; largest ratio gap "
          f"{worst_gap['surrogate']:.2e}, value gap {worst_gap['value']:.2e}")
    for t in ("actor", "critic"):
        print(f"  {t}: d(gpu, branch-matched) {d_hs[t]:.2e}  d(gpu, oracle) {d_ho[t]:.2e}  "
              f"d(branch-matched, oracle) {d_so[t]:.2e}  oracle spread d(lp64, oracle) {spread[t]:.2e}")
        assert d_hs[t] <= FUNCTION_BAR, (t, d_hs[t])
        assert d_ho[t] <= d_so[t] + FUNCTION_BAR, (t, d_ho[t], d_so[t])
    # normaliser statistics (updated after the epochs from all stored observations)
    if w["obs_normalization"]:
        for m_h, m_o in ((hip.actor, ora.actor), (hip.critic, ora.critic)):
            n_h, n_o = m_h.obs_normalizer, m_o.obs_normalizer
            assert int(n_h.count) == int(n_o.count)
            assert rel_err(n_h._mean, n_o._mean) < 1e-6
            assert rel_err(n_h._var, n_o._var) < 1e-6


@pytest.mark.parametrize("name", ["humanoid_full", "flat48_65k"])
def test_compute_returns_with_own_bootstrap_full_size(name):
    """compute_returns as the runner calls it (ppo.py:166-191): the bootstrap value from the plugin's own critic
    forward on the GPU (observation normaliser included), the GAE scan and the global advantage normalisation, at
    4096 envs x 24 steps (humanoid) and 65,536 envs x 24 steps, against the oracle's compute_returns with its own CPU
    critic on the same rollout and weights: returns and advantages within 1e-6 relative (norm-wise), the bootstrap
    values within 1e-6.  The critic's state is left as it was."""
    w, over = CASES[name]
    ora0, roll, last_values = _rollout(name)  # the oracle's returns come from its own critic's bootstrap value
    hip = make_hip(w, 0, **over)
    with torch.no_grad():
        hip.actor.load_state_dict(roll.init_state["actor"])
        hip.critic.load_state_dict(roll.init_state["critic"])
    R.feed(hip.storage, roll)
    obs = {k: v.to(hip.device) for k, v in roll.last_obs.items()}
    with torch.inference_mode():
        v_h = hip.critic(obs).detach()
        hip.compute_returns(obs)
    torch.cuda.synchronize()
    st_o, st_h = ora0.storage, hip.storage
    figures = {"bootstrap_values": rel_err(v_h, last_values), "returns": rel_err(st_h.returns, st_o.returns),
               "advantages": rel_err(st_h.advantages, st_o.advantages)}
    _record("compute_returns", name, {"case": name, "envs": w["num_envs"], "steps": w["steps"], "rel_err": figures})
    print(name, figures)
    for k, v in figures.items():
        assert v < 1e-6, (k, v)


def test_recorded_launches_match_rebuilt_launches():
    """From the third update on, the engine issues each mini-batch from its recorded launch sequence (only Adam's bias
    corrections recomputed); those updates must equal, bit for bit, updates whose every launch is rebuilt in Python:
    parameters, Adam moments, losses and learning rate, over several consecutive updates (obs normalisation on, so the
    frozen normaliser statistics and the normaliser update are exercised too)."""
    from tests.parity import make_pair

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


def _update_both(algs, seed: int) -> list[dict]:
    outs = []
    for alg in algs:
        alg.storage.step = alg.storage.num_transitions_per_env
        torch.manual_seed(seed)
        outs.append(alg.update())
    torch.cuda.synchronize()
    return outs


def _assert_same_state(a, b, where) -> None:
    assert a.learning_rate == b.learning_rate, where
    assert a._opt_steps == b._opt_steps, where
    for name in ("param", "exp_avg", "exp_avg_sq"):
        assert torch.equal(getattr(a.flat, name), getattr(b.flat, name)), (where, name)
    for ma, mb in ((a.actor, b.actor), (a.critic, b.critic)):
        if ma.obs_normalization:
            na, nb = ma.obs_normalizer, mb.obs_normalizer
            for k in ("_mean", "_var", "_std", "count"):
                assert torch.equal(getattr(na, k), getattr(nb, k)), (where, k)
            assert na._host_count == nb._host_count == int(na.count), where


def test_recorded_launches_follow_a_new_storage():
    """A RolloutStorage of the same shape swapped in between updates (upstream's update reads whatever alg.storage
    is): the recorded launches hold the old storage's addresses, so they must be dropped and the updates after the
    swap read the new storage -- bit for bit the updates of a twin whose every launch is rebuilt -- and record again.
    The old storages stay alive, so the new ones cannot take their addresses."""
    from tests.parity import make_pair
    from tt_rsl_rl_amd.storage import RolloutStorage

    w = R.scaled(R.WORKLOADS["humanoid"], num_envs=256, steps=8, hidden_dims=[64, 32])
    _, a, _ = make_pair(w, seed=0)
    _, b, _ = make_pair(w, seed=0)
    a._get_engine().replay, b._get_engine().replay = True, False
    for rep in range(3):
        _update_both((a, b), 1 + rep)
    _assert_same_state(a, b, "before the swap")
    replays = a._engine.replays
    assert replays > 0
    _, roll2 = R.generate(w, 5)
    old = [a.storage, b.storage]
    g = torch.Generator().manual_seed(9)
    last = torch.randn(w["num_envs"], 1, generator=g)
    for alg in (a, b):
        st = RolloutStorage("rl", w["num_envs"], w["steps"], R.zero_obs(w), [w["num_actions"]], alg.device)
        R.feed(st, roll2)
        alg.storage = st
        alg.compute_returns_from(last.to(alg.device))
    assert all(x.observations["policy"].data_ptr() != y.storage.observations["policy"].data_ptr()
               for x, y in zip(old, (a, b)))
    for rep in range(3):
        outs = _update_both((a, b), 10 + rep)
        assert outs[0] == outs[1], rep
        _assert_same_state(a, b, f"update {rep} after the swap")
    assert a._engine.replays > replays, "the updates after the swap record and replay again"
    assert b._engine.replays == 0


def test_failed_update_is_rolled_back():
    """An error raised while an update's launches are issued -- here the library rejecting a weight-grad launch of the
    third mini-batch (asked for -1 rows) after two mini-batches' Adam steps and the normaliser update have run --
    leaves the algorithm as it was before the update: parameters, Adam moments and step count, learning rate, the
    observation normalisers' statistics and sample counts (the host mirror the `until` check reads included).  The
    same update then runs normally and equals, bit for bit, the update of a twin that never failed."""
    from tests.parity import make_pair

    w = R.scaled(R.WORKLOADS["humanoid"], num_envs=256, steps=8, hidden_dims=[64, 32])
    assert w["obs_normalization"]
    _, a, _ = make_pair(w, seed=0)
    _, b, _ = make_pair(w, seed=0)
    for alg in (a, b):
        for m in (alg.actor, alg.critic):
            m.obs_normalizer.until = 10 ** 9
    _update_both((a, b), 1)
    _assert_same_state(a, b, "after the first update")
    engine = a._get_engine()
    real, calls = engine.weight_grads, [0]

    def failing(dw, rows, *args, **kw):
        calls[0] += 1
        return real(dw, -1 if calls[0] == 3 else rows, *args, **kw)

    engine.weight_grads = failing
    a.storage.step = a.storage.num_transitions_per_env
    torch.manual_seed(2)
    with pytest.raises(ValueError):
        a.update()
    assert calls[0] == 3
    del engine.weight_grads
    torch.cuda.synchronize()
    _assert_same_state(a, b, "after the failed update")
    assert a.storage.step == a.storage.num_transitions_per_env, "the rollout is kept"
    for rep in range(2):
        outs = _update_both((a, b), 2 + rep)
        assert outs[0] == outs[1], rep
        _assert_same_state(a, b, f"update {rep} after the failure")


# denominators' floor of the state comparisons: first moments (gradient scale), second moments (squared)
_STATE_FLOOR = {"exp_avg": 1e-12}


def _opt_state(opt, p) -> tuple[dict, int]:
    """A parameter's optimiser state tensors (Adam / AdamW: exp_avg, exp_avg_sq; RMSprop: square_avg; SGD: none)
    and its step count (0 without state)."""
    st = opt.state.get(p, {})
    tensors = {k: v.detach().clone() for k, v in st.items() if k != "step" and torch.is_tensor(v)}
    return tensors, int(st["step"]) if "step" in st else 0


def _snapshot(alg) -> dict:
    params = list(chain(alg.actor.parameters(), alg.critic.parameters()))
    states = [_opt_state(alg.optimizer, p) for p in params]
    # (the optimiser's step count: a parameter without a gradient -- learn_std=False -- has no state and no count;
    # SGD keeps none at all, and only Adam's bias corrections read the count)
    return {"params": [p.detach().clone() for p in params], "lr": alg.learning_rate,
            "state": [st for st, _ in states], "step": max(n for _, n in states)}


def _load_oracle_state(ora, snap: dict) -> None:
    """Put the oracle back into a recorded state (parameters, optimiser state and step, learning rate)."""
    params = list(chain(ora.actor.parameters(), ora.critic.parameters()))
    with torch.no_grad():
        for p, v in zip(params, snap["params"]):
            p.copy_(v)
    ora.optimizer.state.clear()
    for p, st in zip(params, snap["state"]):
        if st and p.requires_grad:
            ora.optimizer.state[p] = {"step": torch.tensor(float(snap["step"])), **{k: v.clone() for k, v in st.items()}}
    ora.learning_rate = snap["lr"]
    for g in ora.optimizer.param_groups:
        g["lr"] = snap["lr"]


def _flat_state_matches(hip, p, want: dict) -> dict[str, float]:
    """The GPU's flat optimiser state of p against a recorded state (zero where the optimiser kept none)."""
    return {k: rel_err(view, want[k] if k in want else torch.zeros_like(view), _STATE_FLOOR.get(k, 1e-20))
            for k, view in hip._state_views(p).items()}


@pytest.mark.parametrize("name", _cases())
def test_update_steps_teacher_forced(name, capsys):
    t0 = [time.time()]
    w, ora, hip = _pair(name)
    snaps = []
    ora.recorder = lambda phase, alg: snaps.append((phase, _snapshot(alg)))
    # the normalisers are updated after the epochs; the steps replayed below need the statistics they ran with
    norms = [(m.obs_normalizer, copy.deepcopy(m.obs_normalizer.state_dict()))
             for m in (ora.actor, ora.critic) if m.obs_normalization]
    torch.manual_seed(1)
    ora.update()
    _progress(capsys, name, "oracle update done", t0)
    ora.recorder = None
    for norm, sd in norms:
        norm.load_state_dict(sd)
    pre = [s for ph, s in snaps if ph == "pre"]
    post = [s for ph, s in snaps if ph == "post"]
    M = ora.num_mini_batches
    assert len(pre) == len(post) == len(ora.trace) == ora.num_learning_epochs * M

    # the GPU side: the update's packed table (same permutation), then one step at a time from the oracle's state
    engine = hip._get_engine()
    engine.gather(None if engine.recurrent else _table_order(ora, hip).to(hip.device))
    params = list(chain(hip.actor.parameters(), hip.critic.parameters()))
    names = [n for n, _ in chain(ora.actor.named_parameters(), ora.critic.named_parameters())]
    torch.manual_seed(1)
    batches = ora.batches()  # the oracle's mini-batches again, for the steps it replays with the GPU's branches
    worst, replayed, n_flips, worst_gap, per_step = 0.0, 0, 0, {}, []
    for k, (a, b) in enumerate(zip(pre, post)):
        batch = next(batches)
        with torch.no_grad():
            for p, v, st in zip(params, a["params"], a["state"]):
                p.copy_(v.to(hip.device))
                for key, view in hip._state_views(p).items():
                    view.copy_(st[key].to(hip.device)) if key in st else view.zero_()
        ops.reset_device_state(hip.device_state, a["lr"])
        r0, r1 = engine.minibatch_rows(k % M)
        engine.minibatch(r0, r1, a["step"] + 1)
        torch.cuda.synchronize()
        kl, lr, surr, value, ent = engine.trace[:5].tolist()
        t = ora.trace[k]
        assert lr == t["lr"], (k, lr, t["lr"])
        if t["kl_mean"] is not None:
            assert abs(kl - t["kl_mean"]) <= 1e-4 * max(t["kl_mean"], 1e-6), (k, kl, t["kl_mean"])
        assert abs(value - t["value"]) <= 1e-4 * abs(t["value"]), (k, value, t["value"])
        assert abs(surr - t["surrogate"]) <= 1e-4 * max(abs(t["surrogate"]), 0.1), (k, surr, t["surrogate"])
        assert abs(ent - t["entropy"]) <= 1e-4 * abs(t["entropy"]), (k, ent, t["entropy"])
        # where the GPU took another clip branch on some row, the oracle's step from the same state with the GPU's
        # decisions on those rows is the reference
        rows = hip_branch_rows(engine, r1 - r0)
        q = hip_quantities(engine, r0, r1, a["params"][0])
        gap = quantity_gap(t["branches"], q)
        for kind, d in gap.items():
            worst_gap[kind] = max(worst_gap.get(kind, 0.0), d)
            assert d < QUANTITY_BAR, (k, kind, d)
        own = t["branches"].own
        step_flips = []
        if any(not torch.equal(rows[kind], own[kind]) for kind in own):
            _load_oracle_state(ora, a)
            t2 = ora.minibatch_step(batch, rows)
            bad = unexplained_flips(t2["branches"], q, AMBIGUOUS)
            assert not bad, (k, bad)
            step_flips = flipped_rows([t2])
            n_flips += len(step_flips)
            assert t2["lr"] == lr
            b = _snapshot(ora)
            replayed += 1
        step_worst = 0.0
        for n, p, v, st in zip(names, params, b["params"], b["state"]):
            err = rel_err(p, v)
            step_worst = max(step_worst, err)
            assert err < PARAM_BAR, (k, n, err)
            for key, e in _flat_state_matches(hip, p, st).items():
                assert e < MOMENT_BAR, (k, n, key, e)
        worst = max(worst, step_worst)
        per_step.append({"step": k, "worst_param_err": step_worst, "ratio_gap": gap.get("surrogate"),
                         "value_gap": gap.get("value"),
                         "rows_on_another_branch": [{"kind": kind, "row": i, "distance_to_boundary": d}
                                                    for _, kind, i, d in step_flips]})
        if k % 5 == 4:
            _progress(capsys, name, f"step {k + 1} of {len(pre)} checked", t0)
    _record("teacher_forced", name, {"case": name, "steps": len(pre), "replayed_with_gpu_branches": replayed,
                                     "rows_on_another_branch": n_flips, "worst_param_err": worst,
                                     "largest_gaps": worst_gap, "per_step": per_step})
    print(f"{name}: {len(pre)} teacher-forced steps, {replayed} with {n_flips} row(s) on another clip branch "
          f"(oracle replayed with the GPU's decisions), worst parameter rel error {worst:.2e}, largest ratio / value "
          f"gap {worst_gap}")


def test_state_dict_and_checkpoint_round_trip(tmp_path):
    w, over = CASES["humanoid_small_permb_adv"]
    _, ora, hip = _pair("humanoid_small_permb_adv")
    for alg in (ora, hip):
        torch.manual_seed(1)
        alg.update()
    saved = hip.save()
    assert list(saved["actor_state_dict"].keys()) == list(ora.actor.state_dict().keys())
    assert list(saved["critic_state_dict"].keys()) == list(ora.critic.state_dict().keys())
    osd_h, osd_o = saved["optimizer_state_dict"], ora.optimizer.state_dict()
    assert osd_h["param_groups"][0]["params"] == osd_o["param_groups"][0]["params"]
    assert osd_h["param_groups"][0]["lr"] == osd_o["param_groups"][0]["lr"]
    # upstream-format checkpoint -> fresh plugin
    path = tmp_path / "model.pt"
    torch.save({**ora.save(), "iter": 3, "infos": None}, path)
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
    393,216 rows; all three are also compared with the oracle above): the update runs, the losses are finite, parameters moved by
    at most 20 Adam steps' worth (the lr is clamped to [1e-5, 1e-2]), and two identical updates give bit-identical
    parameters (deterministic reductions).  lstm256 starts its sequences from random saved states."""

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


def test_more_epochs_between_updates_grow_the_trace():
    """num_learning_epochs raised between two updates: the per-mini-batch trace grows with it (the finalize kernels
    write no row past the buffer they are given), and the second update still follows the oracle's: same
    learning-rate decisions and losses."""
    w = R.scaled(R.WORKLOADS["humanoid"], num_envs=128, steps=8, hidden_dims=[64, 32])
    from tests.parity import make_pair

    ora, hip, _ = make_pair(w, seed=0, num_learning_epochs=1)
    for epochs, seed in ((1, 1), (6, 2)):
        outs = []
        for alg in (ora, hip):
            alg.num_learning_epochs = epochs
            alg.storage.step = alg.storage.num_transitions_per_env
            torch.manual_seed(seed)
            outs.append(alg.update())
        torch.cuda.synchronize()
        assert len(hip.last_trace) == len(ora.trace) == epochs * ora.num_mini_batches
        assert [t["lr"] for t in hip.last_trace] == [t["lr"] for t in ora.trace]
        for k in ("value", "surrogate", "entropy"):
            assert abs(outs[1][k] - outs[0][k]) <= 1e-4 * max(abs(outs[0][k]), 0.1), (epochs, k)
    assert hip._engine.trace.numel() >= 5 * 6 * hip.num_mini_batches
