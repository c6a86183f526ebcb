"""Parity harness shared by the GPU tests, smoke() and bench.py: the oracle and the HIP plugin on one rollout."""

from __future__ import annotations

import contextlib
import math
from types import SimpleNamespace

import torch

from oracle import ppo_ref as O
from oracle import rollout as R


def rel_err(a: torch.Tensor, b: torch.Tensor, floor: float = 0.0) -> float:
    """||a - b|| / max(||b||, floor), in float64."""
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    den = max(float(b.norm()), floor)
    if den == 0.0:
        return float((a - b).norm())
    return float((a - b).norm()) / den


def make_hip(workload: dict, seed: int = 0, device: str = "cuda", **alg_overrides):
    from tt_rsl_rl_amd.ppo import PPO

    torch.manual_seed(seed)
    cfg = R.train_cfg(workload, algorithm_class="tt_rsl_rl_amd.ppo:PPO", **alg_overrides)
    env = SimpleNamespace(num_envs=workload["num_envs"], num_actions=workload["num_actions"])
    alg = PPO.construct_algorithm(R.zero_obs(workload), env, cfg, device)
    alg.train_mode()
    return alg


def make_pair(workload: dict, seed: int = 0, carry_state: bool = False, **alg_overrides):
    """Oracle with a generated rollout + the HIP plugin with identical weights and the same stored rollout.
    Both have their returns / advantages computed from the same bootstrap values."""
    ora, roll = R.generate(workload, seed, carry_state=carry_state, **alg_overrides)
    hip = make_hip(workload, seed, **alg_overrides)
    with torch.no_grad():
        hip.actor.load_state_dict(roll.init_state["actor"])
        hip.critic.load_state_dict(roll.init_state["critic"])
    R.feed(hip.storage, roll)
    with torch.inference_mode():
        last_values = ora.critic(roll.last_obs).detach()
    ora.compute_returns(roll.last_obs, last_values=last_values)
    hip.compute_returns_from(last_values.to(hip.device).contiguous())
    return ora, hip, roll


def hip_branch_rows(engine, R: int) -> dict:
    """The clip-branch decisions of the GPU's last mini-batch: rows whose surrogate / value gradient is non-zero.
    The loss kernels write dloss/dmean [R, A] and dloss/dV [R] into the output layers' gradient buffers; a row's
    dloss/dmean is exactly zero iff the clipped surrogate passes no gradient to its ratio (the only term that depends
    on the mean), and dloss/dV iff the clipped value loss passes none to V."""
    dm = engine.buf_a.dz[-1][:R]
    dv = engine.buf_c.dz[-1][:R, 0]
    return {"surrogate": (dm != 0).any(1).cpu(), "value": (dv != 0).cpu()}


def hip_quantities(engine, r0: int, r1: int, std_param: torch.Tensor) -> dict:
    """The quantities the GPU's clip decisions of mini-batch rows [r0, r1) depend on, from its own outputs: the ratio
    exp(log N(a; mean, std) - old_logp) per row, evaluated in fp64 on the host from the mean the kernels computed
    and the std parameter the step started from, and the value V the kernels computed (exact)."""
    R = r1 - r0
    lay, A = engine.layout, engine.A
    tab = engine.table[r0:r1]
    a = tab[:, lay.actions:lay.actions + A].double().cpu()
    old = tab[:, lay.old_logp].double().cpu()
    mu = engine.buf_a.out[:R].double().cpu()
    dist = engine.alg.actor.distribution
    lo, hi = dist.param_range
    p = std_param.detach().double().cpu().reshape(-1).clamp(lo, hi)
    sd = p if dist.std_type == "scalar" else p.exp()
    logp = (-((a - mu) ** 2) / (2 * sd * sd) - sd.log() - 0.5 * math.log(2 * math.pi)).sum(-1)
    return {"surrogate": torch.exp(logp - old), "value": engine.buf_c.out[:R, 0].double().cpu()}


def flipped_rows(trace: list) -> list[tuple[int, str, int, float]]:
    """(step, kind, row, distance to the boundary) of every row where a forced branch differs from the oracle's own."""
    out = []
    for k, t in enumerate(trace):
        for kind, (idx, dist) in t["branches"].flips.items():
            out += [(k, kind, int(i), float(d)) for i, d in zip(idx.tolist(), dist.tolist())]
    return out


def quantity_gap(branch, hip_q: dict) -> dict[str, float]:
    """Largest per-row difference between the GPU's and the oracle's ratio (absolute) and value (relative to the
    largest |V|) in one mini-batch."""
    out = {}
    for kind, q in branch.q.items():
        d = (hip_q[kind] - q).abs().max().item()
        out[kind] = d if kind == "surrogate" else d / max(q.abs().max().item(), 1e-30)
    return out


def unexplained_flips(branch, hip_q: dict, slack: float) -> list[tuple[str, int, float, float]]:
    """Rows of one mini-batch where the GPU took another clip branch than the oracle and the two evaluations' own
    quantities do not straddle the boundary within `slack`: a row is explained when its distance to the boundary (in
    the oracle's evaluation) is at most the row's |q_gpu - q_oracle| + slack, i.e. the GPU's quantity, up to the
    kernels' own fp32 rounding, lies on the side of the boundary its decision belongs to.  For the value loss the
    other decision boundary is the equality of the two squares, |l1 - l2| / l1 <= 2 |dV| / |V - R|."""
    bad = []
    for kind, (idx, dist) in branch.flips.items():
        for i, d in zip(idx.tolist(), dist.tolist()):
            dq = abs(float(hip_q[kind][i]) - float(branch.q[kind][i]))
            ok = d <= dq + slack
            if kind == "value" and not ok:
                ex = branch.extra["value"]
                ok = float(ex["gap"][i]) <= 2.0 * dq / max(float(ex["err"][i]), 1e-30) + slack
            if not ok:
                bad.append((kind, i, d, dq))
    return bad


def param_dict(alg) -> dict[str, torch.Tensor]:
    return {f"{tag}.{n}": p.detach().cpu().clone()
            for tag, m in (("actor", alg.actor), ("critic", alg.critic)) for n, p in m.named_parameters()}


def function_outputs(params: dict, ora, eval_obs: dict) -> dict[str, torch.Tensor]:
    """Actor mean and critic value of a parameter set on a fixed set of observations: the oracle models' forward
    (torch fp32, CPU) with the given parameters substituted (normaliser statistics: the oracle model's).  Recurrent
    models run the observation sequence from the saved initial state, resetting the state at the dones."""
    out = {}
    with torch.no_grad():
        for tag, model in (("actor", ora.actor), ("critic", ora.critic)):
            p = {n[len(tag) + 1:]: v for n, v in params.items() if n.startswith(tag + ".")}
            if not model.is_recurrent:
                out[tag] = torch.func.functional_call(model, p, (eval_obs["flat"],))
                continue
            saved = model.get_hidden_state()
            h0 = eval_obs["h0_" + tag]
            state = None if h0 is None else tuple(h.clone() for h in h0)
            if state is not None and len(state) == 1:  # the GRU's state is one tensor
                state = state[0]
            model.reset(hidden_state=state)
            ys = []
            for t, obs_t in enumerate(eval_obs["seq"]):
                ys.append(torch.func.functional_call(model, p, (obs_t,)))
                model.reset(eval_obs["dones"][t])
            model.reset(hidden_state=saved)
            out[tag] = torch.cat(ys)
    return out


def eval_observations(ora, max_rows: int = 32768, max_envs: int = 1024) -> dict:
    """The rollout's stored observations as the function-space evaluation set (a fixed subset for large rollouts)."""
    st = ora.storage
    if not ora.actor.is_recurrent:
        B = st.num_envs * st.num_transitions_per_env
        idx = torch.arange(B) if B <= max_rows else torch.linspace(0, B - 1, max_rows).long()
        return {"flat": {k: v.flatten(0, 1)[idx].clone() for k, v in st.observations.items()}}
    n = min(st.num_envs, max_envs)
    ev = {"seq": [{k: v[t, :n].clone() for k, v in st.observations.items()} for t in range(st.num_transitions_per_env)],
          "dones": [st.dones[t, :n, 0].clone() for t in range(st.num_transitions_per_env)]}
    for tag, saved in (("actor", st.saved_hidden_state_a), ("critic", st.saved_hidden_state_c)):
        ev["h0_" + tag] = None if saved is None else tuple(s[0, :, :n].clone() for s in saved)
    return ev


def function_deviation(p_a: dict, p_b: dict, p_0: dict, ora, eval_obs: dict) -> dict[str, float]:
    """||f(p_a) - f(p_b)|| / ||f(p_b) - f(p_0)|| for the actor mean and the critic value: the fraction of the update
    from p_0 to p_b by which p_a's update differs (the metric of the reference's tests/tt/test_tt_update.py:348-351)."""
    fa, fb, f0 = (function_outputs(p, ora, eval_obs) for p in (p_a, p_b, p_0))
    return {t: float((fa[t] - fb[t]).double().norm() / (fb[t] - f0[t]).double().norm().clamp(min=1e-30))
            for t in ("actor", "critic")}


@contextlib.contextmanager
def oracle_logp_fp64():
    """Run the oracle with the per-action log-prob sum accumulated in fp64 and rounded once, instead of torch's
    fp32 reduction order.  Same formula, a different (more accurate) fp32 evaluation: the difference between the
    two oracles is the oracle's own rounding floor for quantities that depend on the sum of A log-prob terms."""
    orig = O.GaussianDistribution.log_prob
    O.GaussianDistribution.log_prob = lambda self, x: self._distribution.log_prob(x).double().sum(dim=-1).float()
    try:
        yield
    finally:
        O.GaussianDistribution.log_prob = orig
