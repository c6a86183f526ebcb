"""use_mixed_precision (rsl_rl/algorithms/ppo.py:222-224: torch.autocast to bfloat16 over the forward and the loss).

The HIP update's mixed-precision mode runs its linear layers' matrix products -- forward, input-gradient and
weight-gradient GEMMs of the MLP layers and of the recurrent input projection -- with bf16 operands (every operand
element rounded to nearest even) and fp32 accumulation on the bf16 matrix cores, one product per k-group instead of the
six of the fp32-accurate bf16x6 scheme.  Bias, activation and loss arithmetic, the fused output-layer head and the
recurrent cells stay fp32.

Kernel bar: the result equals fp64 arithmetic on the bf16-rounded operands to the fp32-GEMM bar (2e-6), and differs from
the fp32 product by bf16's rounding (the mode is really on).  Operands the bf16 kernels do not take run on the fp32
kernels: bit-identical to the call without the flag.

Update bar: the mixed-precision update is an approximation of upstream's update, not a restatement of autocast's
rounding (autocast also rounds every layer's output to bf16); so it is measured against the fp32 oracle in function
space (the metric of the reference's tests/tt/test_tt_update.py:348-351) and must be no farther from it than
upstream's own autocast update, run by the oracle on the same rollout, is.  Learning-rate decisions are allowed to
differ only where the oracle's KL lies within bf16 resolution of a threshold (none on these cases).
"""

from __future__ import annotations

import copy
import math

import pytest
import torch

from oracle import rollout as R
from tests.parity import eval_observations, function_deviation, make_hip, param_dict, rel_err

pytestmark = pytest.mark.gpu

GEMM_BAR = 2e-6


def _ops():
    from tt_rsl_rl_amd import _lib, ops

    _lib.load()
    return ops


def _b(t: torch.Tensor) -> torch.Tensor:
    """fp64 of t's bf16 rounding (torch's conversion rounds to nearest even, as the kernels do)."""
    return t.to(torch.bfloat16).double()


def _aligned(t: torch.Tensor, cuda, off: int = 0) -> torch.Tensor:
    """t on the device with 16-byte rows (off=0), or one float past a 16-byte boundary (off=1)."""
    rows, cols = t.shape
    buf = torch.zeros(rows, -(-cols // 4) * 4 + 4, device=cuda)
    buf[:, off:off + cols].copy_(t)
    return buf[:, off:off + cols]


def _err(out: torch.Tensor, ref64: torch.Tensor, bound: torch.Tensor) -> tuple[float, float]:
    """(relative Frobenius error, worst per-element error over its |A| |B| bound) against fp64."""
    e = out.double().cpu() - ref64.cpu()
    return float(e.norm() / ref64.norm()), float((e.abs() / bound.cpu().clamp(min=1e-300)).max())


_ELU64 = lambda z: torch.where(z > 0, z, torch.expm1(z))  # noqa: E731


@pytest.mark.parametrize("rows,fin,fout", [(24576, 96, 512), (24576, 512, 256), (1000, 256, 128), (77, 128, 32)])
def test_bf16_forward_against_rounded_fp64(cuda, rows, fin, fout):
    """z = bf16(x) bf16(w)^T + b and h = elu(z) (fp32 bias + activation epilogue) against fp64 on the rounded operands;
    and the fp32 product it is not (bf16's relative rounding ~2^-9 on each operand)."""
    from tt_rsl_rl_amd import _lib as L

    ops = _ops()
    g = torch.Generator().manual_seed(rows + fin)
    x, w = torch.randn(rows, fin, generator=g), torch.randn(fout, fin, generator=g) / math.sqrt(fin)
    b = torch.randn(fout, generator=g)
    z64 = _b(x) @ _b(w).t() + b.double()
    bound = _b(x).abs() @ _b(w).abs().t() + b.double().abs()
    z, h = torch.empty(rows, fout, device=cuda), torch.empty(rows, fout, device=cuda)
    ops.linear_fwd([(_aligned(x, cuda), w.to(cuda), b.to(cuda), z, h)], rows, act=L.ACTIVATIONS["elu"], bf16=True)
    fro, elem = _err(z, z64, bound)
    print(f"fwd {rows}x{fin}->{fout}: rel-Frobenius {fro:.2e}, per-element/bound {elem:.2e}")
    assert fro < GEMM_BAR and elem < GEMM_BAR
    assert rel_err(h, _ELU64(z64)) < GEMM_BAR
    exact = x.double() @ w.double().t() + b.double()
    assert rel_err(z, exact) > 1e-4, "the flag did not select bf16 operands"


@pytest.mark.parametrize("rows,fin,fout,act,from_output", [(24576, 512, 256, "elu", False), (1000, 128, 64, "tanh", True),
                                                         (333, 256, 32, None, False)])
def test_bf16_input_grad_against_rounded_fp64(cuda, rows, fin, fout, act, from_output):
    """dz_prev = (bf16(dz) bf16(w)) * act'(src), act' in fp32 from the activation's input or output."""
    from tt_rsl_rl_amd import _lib as L

    ops = _ops()
    g = torch.Generator().manual_seed(rows + fout)
    dz, w = torch.randn(rows, fout, generator=g), torch.randn(fout, fin, generator=g) / math.sqrt(fout)
    ref = _b(dz) @ _b(w)
    bound = _b(dz).abs() @ _b(w).abs()
    src = None
    if act is not None:
        zp = torch.randn(rows, fin, generator=g) * 2
        f = torch.tanh if act == "tanh" else _ELU64
        if from_output:  # act' from the fp32 output as passed: tanh' = 1 - h^2
            src = f(zp.double()).float()
            d = 1 - src.double() ** 2
        else:
            src = zp
            zr = zp.double().requires_grad_(True)
            d = torch.autograd.grad(f(zr).sum(), zr)[0]
        ref, bound = ref * d, bound * d.abs()
        src = src.to(cuda)
    out = torch.empty(rows, fin, device=cuda)
    ops.linear_bwd_dx([(_aligned(dz, cuda), w.to(cuda), src, out)], rows, elu_from_output=from_output,
                      act=L.ACTIVATIONS[act] if act else L.PPO_ACT_ELU, bf16=True)
    fro, elem = _err(out, ref, bound)
    print(f"dx {rows}x{fout}->{fin} {act}: rel-Frobenius {fro:.2e}, per-element/bound {elem:.2e}")
    assert fro < GEMM_BAR
    if not from_output:  # (1 - h^2 in fp32 for h within a few ulps of 1 cancels: only the norm bar there)
        assert elem < GEMM_BAR
    exact = dz.double() @ w.double()
    if act is not None:
        exact = exact * d
    assert rel_err(out, exact) > 1e-4, "the flag did not select bf16 operands"


@pytest.mark.parametrize("rows,fin,fout", [(24576, 512, 256), (24576, 96, 512), (5000, 128, 29), (100, 64, 16)])
def test_bf16_weight_grad_against_rounded_fp64(cuda, rows, fin, fout):
    """dw = bf16(dz)^T bf16(x) (k = the rows, ragged tails included), db = the column sums of the fp32 dz."""
    ops = _ops()
    g = torch.Generator().manual_seed(rows + 11 * fout)
    dz, x = torch.randn(rows, fout, generator=g), torch.randn(rows, fin, generator=g)
    ref = _b(dz).t() @ _b(x)
    bound = _b(dz).abs().t() @ _b(x).abs()
    dw, db = torch.empty(fout, fin, device=cuda), torch.empty(fout, device=cuda)
    ops.linear_bwd_dw([(_aligned(dz, cuda), _aligned(x, cuda), dw, db)], rows, bf16=True)
    fro, elem = _err(dw, ref, bound)
    print(f"dw {rows} rows {fout}x{fin}: rel-Frobenius {fro:.2e}, per-element/bound {elem:.2e}")
    assert fro < GEMM_BAR and elem < GEMM_BAR
    assert rel_err(db, dz.double().sum(0)) < 1e-6
    assert rel_err(dw, dz.double().t() @ x.double()) > 1e-4, "the flag did not select bf16 operands"


def test_bf16_flag_on_operands_outside_the_bf16_kernels_runs_fp32(cuda):
    """Rows one float off a 16-byte boundary: the fp32 kernels, bit for bit the call without the flag."""
    ops = _ops()
    g = torch.Generator().manual_seed(5)
    rows, fin, fout = 3000, 96, 256
    x, w, b = torch.randn(rows, fin, generator=g), torch.randn(fout, fin, generator=g), torch.randn(fout, generator=g)
    dz = torch.randn(rows, fout, generator=g)
    xd, dzd = _aligned(x, cuda, 1), _aligned(dz, cuda, 1)
    out = {}
    for flag in (False, True):
        z = torch.empty(rows, fout, device=cuda)
        ops.linear_fwd([(xd, w.to(cuda), b.to(cuda), z, None)], rows, act=0, bf16=flag)
        dx = torch.empty(rows, fin, device=cuda)
        ops.linear_bwd_dx([(dzd, w.to(cuda), None, dx)], rows, bf16=flag)
        dw, db = torch.empty(fout, fin, device=cuda), torch.empty(fout, device=cuda)
        ops.linear_bwd_dw([(dzd, xd, dw, db)], rows, bf16=flag)
        out[flag] = (z, dx, dw, db)
    torch.cuda.synchronize()
    for a, c in zip(out[False], out[True]):
        assert torch.equal(a, c)
    assert rel_err(out[True][0], x.double() @ w.double().t() + b.double()) < GEMM_BAR


# ---------------------------------------------------------------------------------------------------------------------
# the update
# ---------------------------------------------------------------------------------------------------------------------

def _rnn(num_envs: int, steps: int, hidden: int, hidden_dims: list[int], layers: int = 1, rnn_type: str = "lstm"):
    w = R.scaled(R.WORKLOADS["lstm256"], num_envs=num_envs, steps=steps, hidden_dims=hidden_dims)
    w["rnn"] = dict(w["rnn"], rnn_hidden_dim=hidden, rnn_num_layers=layers, rnn_type=rnn_type)
    return w


MP_CASES = {
    "humanoid_1k": (R.scaled(R.WORKLOADS["humanoid"], num_envs=1024), {}),
    "rough235_512": (R.scaled(R.WORKLOADS["rough235"], num_envs=512), {}),
    "flat48_small_fixed": (R.scaled(R.WORKLOADS["flat48"], num_envs=256, steps=8, hidden_dims=[128, 64, 32]),
                           {"schedule": "fixed"}),
    # 40 actions: the output layers outside the fused head (their own GEMMs, bf16 operands too, and the loss kernel)
    "flat48_a40_unfused_fixed": (dict(R.scaled(R.WORKLOADS["flat48"], num_envs=256, steps=8, hidden_dims=[64, 48]),
                                      num_actions=40), {"schedule": "fixed"}),
    # recurrent: autocast also runs upstream's nn.LSTM / nn.GRU in bf16 (input and recurrent products); the plugin
    # takes bf16 operands in the input projections and the heads, and keeps the recurrent product fp32
    "lstm64_512": (_rnn(512, 16, 64, [64, 32]), {}),
    "gru32x2_256_fixed": (_rnn(256, 10, 32, [32, 16], layers=2, rnn_type="gru"), {"schedule": "fixed"}),
}


def _hip_twin(w: dict, roll, last_values: torch.Tensor, **over):
    """Another plugin instance on the same weights, rollout and bootstrap values."""
    hip = make_hip(w, 0, **over)
    with torch.no_grad():
        hip.actor.load_state_dict(roll.init_state["actor"])
        hip.critic.load_state_dict(roll.init_state["critic"])
    R.feed(hip.storage, roll)
    hip.compute_returns_from(last_values.to(hip.device).contiguous())
    return hip


@pytest.mark.parametrize("name", list(MP_CASES))
def test_mixed_precision_update_against_the_oracle(name):
    """The plugin's update with use_mixed_precision against the fp32 oracle and the oracle's own autocast update
    (upstream's semantics) from the same rollout and weights: in function space the plugin's update may differ from
    the fp32 oracle's by no more than upstream's autocast update does; losses no farther from the fp32 oracle's than
    autocast's plus 1e-3 of their scale; the learning-rate decisions of the fp32 oracle; every parameter finite and
    every trained one moved; and the same update without the flag is closer to the fp32 oracle, so the switch
    reached the kernels."""
    w, over = MP_CASES[name]
    ora, roll = R.generate(w, 0, **over)
    with torch.inference_mode():  # (once: a recurrent critic's forward advances its hidden state)
        last_values = ora.critic(roll.last_obs).detach()
    ora.compute_returns(roll.last_obs, last_values=last_values)
    hip = _hip_twin(w, roll, last_values, use_mixed_precision=True, **over)
    hip32 = _hip_twin(w, roll, last_values, **over)
    assert hip.use_mixed_precision and not hip32.use_mixed_precision and not ora.use_mixed_precision
    assert torch.equal(hip32.storage.advantages, hip.storage.advantages)
    p0, ev = param_dict(ora), eval_observations(ora)
    amp = copy.deepcopy(ora)
    amp.use_mixed_precision = True
    torch.manual_seed(1)
    ref = ora.update()
    torch.manual_seed(1)
    ref_amp = amp.update()
    torch.manual_seed(1)
    out = hip.update()
    torch.manual_seed(1)
    out32 = hip32.update()
    torch.cuda.synchronize()
    p_h, p_o, p_a, p_32 = param_dict(hip), param_dict(ora), param_dict(amp), param_dict(hip32)
    d_ho = function_deviation(p_h, p_o, p0, ora, ev)
    d_ao = function_deviation(p_a, p_o, p0, ora, ev)
    d_ha = function_deviation(p_h, p_a, p0, ora, ev)
    d_32 = function_deviation(p_32, p_o, p0, ora, ev)
    lr_h, lr_o, lr_a = ([t["lr"] for t in tr] for tr in (hip.last_trace, ora.trace, amp.trace))
    print(f"{name}: learning rates gpu {lr_h}\n  fp32 oracle {lr_o}\n  autocast oracle {lr_a}")
    for t in ("actor", "critic"):
        print(f"{name} {t}: d(gpu bf16 operands, fp32 oracle) {d_ho[t]:.3e}   d(oracle autocast, fp32 oracle) "
              f"{d_ao[t]:.3e}   d(gpu bf16 operands, oracle autocast) {d_ha[t]:.3e}   d(gpu fp32, fp32 oracle) "
              f"{d_32[t]:.3e}")
    for k, scale in (("value", 0.0), ("surrogate", 0.1), ("entropy", 0.0)):
        print(f"  {k}: gpu {out[k]:.6f}  fp32 oracle {ref[k]:.6f}  autocast oracle {ref_amp[k]:.6f}  "
              f"gpu fp32 {out32[k]:.6f}")
    for t in ("actor", "critic"):
        assert d_ho[t] <= 1.1 * d_ao[t], (t, d_ho[t], d_ao[t])
        assert d_ho[t] > d_32[t], (t, d_ho[t], d_32[t])
    for k, scale in (("value", 0.0), ("surrogate", 0.1), ("entropy", 0.0)):
        slack = abs(ref_amp[k] - ref[k]) + 1e-3 * max(abs(ref[k]), scale)
        assert abs(out[k] - ref[k]) <= slack, (k, out[k], ref[k], ref_amp[k])
    assert lr_h == lr_a
    trained = {f"{tag}.{n}" for tag, m in (("actor", ora.actor), ("critic", ora.critic))
               for n, q in m.named_parameters() if q.requires_grad}
    for key, q in p_h.items():
        assert torch.isfinite(q).all(), key
        if key in trained:
            assert not torch.equal(q, p0[key]), key
