"""GPU parity of every kernel of libppo_hip.so, called through the C ABI (tt_rsl_rl_amd.ops), against the oracle.

Bars: bit-exact for data movement (gather) and for the GAE returns; 1e-6 relative for advantages and normaliser
statistics; fp32-GEMM tolerance (relative Frobenius 2e-6 against float64) for the linear layers; 2e-6 for the loss
gradients given identical network outputs; 1e-6 for Adam + clipping against torch.optim.Adam / clip_grad_norm_.
"""

from __future__ import annotations

import json
import math
import os

import pytest
import torch

from oracle import ppo_ref as O
from tests.parity import rel_err

pytestmark = pytest.mark.gpu


def _ops():
    from tt_rsl_rl_amd import _lib, ops

    _lib.load()
    return ops


# ----------------------------------------------------------------------------------------------------------------------
# A1 / A2
# ----------------------------------------------------------------------------------------------------------------------


@pytest.mark.parametrize("T,N,p_done", [(24, 4096, 0.005), (7, 333, 0.3), (1, 1, 0.0), (24, 65536, 0.01),
                                        (16, 1000, 0.02), (40, 500, 0.05)])
def test_gae_matches_oracle(cuda, T, N, p_done):
    ops = _ops()
    g = torch.Generator().manual_seed(T * 1000 + N)
    rewards = torch.randn(T, N, 1, generator=g) * 0.3
    values = torch.randn(T, N, 1, generator=g)
    dones = (torch.rand(T, N, 1, generator=g) < p_done).to(torch.uint8)
    last = torch.randn(N, 1, generator=g)
    ret_ref, adv_raw_ref = O.gae_returns(rewards, values, dones, last, 0.99, 0.95, normalize=False)
    _, adv_ref = O.gae_returns(rewards, values, dones, last, 0.99, 0.95, normalize=True)
    d = lambda t: t.to(cuda).contiguous()
    ret, adv = torch.empty(T, N, 1, device=cuda), torch.empty(T, N, 1, device=cuda)
    ops.gae(d(rewards), d(values), d(dones), d(last), ret, adv, 0.99, 0.95)
    assert torch.equal(ret.cpu(), ret_ref), "GAE returns must be bit-exact"
    assert torch.equal(adv.cpu(), adv_raw_ref), "returns - values must be bit-exact"
    if T * N > 1:
        ops.adv_normalize(adv, adv, T * N)
        err = (adv.cpu() - adv_ref).abs().max().item()
        assert err <= 1e-6 * max(1.0, adv_ref.abs().max().item()), err


def test_adv_normalize_strided(cuda):
    ops = _ops()
    x = torch.randn(5000, 3)
    out = torch.zeros(5000, 7)
    xd, od = x.to(cuda), out.to(cuda)
    ops.adv_normalize(xd[:, 1], od[:, 4], 5000, in_stride=3, out_stride=7)
    col = x[:, 1]
    ref = (col - col.mean()) / (col.std() + 1e-8)
    assert rel_err(od[:, 4], ref) < 1e-6
    assert torch.equal(od[:, :4].cpu(), out[:, :4]) and torch.equal(od[:, 5:].cpu(), out[:, 5:])


# ----------------------------------------------------------------------------------------------------------------------
# A5 gather (+ fused normaliser)
# ----------------------------------------------------------------------------------------------------------------------


def test_gather_rows_bit_exact(cuda):
    ops = _ops()
    B = 98304
    torch.manual_seed(3)
    obs = torch.randn(B, 99)
    act = torch.randn(B, 29)
    logp = torch.randn(B, 1)
    mean, std = torch.randn(1, 99), torch.rand(1, 99) + 0.5
    perm = torch.randperm(B)
    W = 140
    dst = torch.full((B, W), float("nan"), device=cuda)
    dones = (torch.rand(B, 1) < 0.3).to(torch.uint8)
    segs = [ops.Segment(obs.to(cuda), 0, mean.view(-1).to(cuda), std.view(-1).to(cuda), 1e-2),
            ops.Segment(act.to(cuda), 100), ops.Segment(logp.to(cuda), 132),
            ops.Segment(dones.to(cuda), 134, keep=True)]
    ops.gather_rows(perm.to(cuda), segs, dst)
    out = dst.cpu()
    norm = O.EmpiricalNormalization(99)
    norm._mean.copy_(mean)
    norm._std.copy_(std)
    assert torch.equal(out[:, :99], norm(obs[perm])), "normalised gather must be bit-exact"
    assert torch.equal(out[:, 100:129], act[perm])
    assert torch.equal(out[:, 132:133], logp[perm])
    assert torch.equal(out[:, 134:135], 1.0 - dones[perm].float()), "keep = 1 - done from the uint8 flags"
    assert torch.isnan(out[:, 99]).all() and torch.isnan(out[:, 129:132]).all(), "gather wrote outside its columns"
    assert torch.isnan(out[:, 133]).all() and torch.isnan(out[:, 135:]).all(), "gather wrote outside its columns"


@pytest.mark.parametrize("vec_width,odd_width", [(4, 0), (96, 99), (200, 1), (256, 130), (512, 190), (1020, 255),
                                                 (1100, 3)])
def test_gather_rows_float4_segments(cuda, vec_width, odd_width):
    """Segments that are whole 16-byte aligned float4 runs (aligned sources with a leading dimension and width that are
    multiples of 4, destination columns multiples of 4) move as float4 chunks beside segments that are not (a 99- or
    odd-wide source, a keep column): one 16-byte aligned segment with the normaliser fused, split in two, next to
    4-byte ones, for every chunk-slot class (1 to 4 slots of 64 chunks per lane, and 1100 floats: the float path);
    bit-exact against torch on a ragged row count, nothing written outside the columns."""
    ops = _ops()
    torch.manual_seed(vec_width + odd_width)
    src_rows, rows = 5003, 4999
    half = vec_width // 8 * 4
    a = torch.randn(src_rows, half + 4, device=cuda)[:, :half] if half else None     # leading dim half + 4
    b = torch.randn(src_rows, vec_width - half, device=cuda)                           # contiguous, width % 4 == 0
    mean, std = torch.randn(vec_width - half, device=cuda), torch.rand(vec_width - half, device=cuda) + 0.5
    odd = torch.randn(src_rows, odd_width, device=cuda) if odd_width else None
    dones = (torch.rand(src_rows, 1) < 0.5).to(torch.uint8).to(cuda)
    perm = torch.randperm(src_rows)[:rows].to(cuda)
    W = -(-(vec_width + odd_width + 16) // 4) * 4
    dst = torch.full((rows, W), float("nan"), device=cuda)
    segs, col, checks = [], 0, []
    if a is not None:
        segs.append(ops.Segment(a, col))
        checks.append((col, a[perm]))
        col += half
    segs.append(ops.Segment(b, col, mean, std, 1e-2))
    checks.append((col, (b[perm] - mean) / (std + 1e-2)))
    col += vec_width - half
    if odd is not None:
        col += 1  # (a column that is not a multiple of 4)
        segs.append(ops.Segment(odd, col))
        checks.append((col, odd[perm]))
        col += odd_width
    segs.append(ops.Segment(dones, col, keep=True))
    checks.append((col, 1.0 - dones[perm].float()))
    ops.gather_rows(perm, segs, dst)
    torch.cuda.synchronize()
    written = torch.zeros(W, dtype=torch.bool)
    for c, ref in checks:
        assert torch.equal(dst[:, c:c + ref.shape[1]], ref), c
        written[c:c + ref.shape[1]] = True
    assert torch.isnan(dst[:, ~written.to(cuda)]).all(), "gather wrote outside its columns"


@pytest.mark.parametrize("width", [1, 63, 64, 65, 130, 190, 250, 300, 380, 420, 511, 600, 1100])
def test_gather_rows_every_slot_count(cuda, width):
    """Rows of every width class the launcher distinguishes (1 to 8 slots of 64 floats per lane, and rows wider than
    512 floats, which take several passes): a float segment of `width` - 1 columns plus a keep column, gathered
    bit-exactly from a ragged source (5,003 rows) into a NaN-filled table, nothing written outside the columns."""
    ops = _ops()
    torch.manual_seed(width)
    src_rows, rows = 5003, 4999
    wf = max(width - 1, 1)
    xd = torch.randn(src_rows, wf + 3, device=cuda)[:, :wf]  # a strided view (leading dimension wf + 3)
    x = xd.cpu()
    dones = (torch.rand(src_rows, 1) < 0.5).to(torch.uint8)
    perm = torch.randperm(src_rows)[:rows]
    dst = torch.full((rows, wf + 8), float("nan"), device=cuda)
    ops.gather_rows(perm.to(cuda), [ops.Segment(xd, 2), ops.Segment(dones.to(cuda), wf + 4, keep=True)], dst)
    out = dst.cpu()
    assert torch.equal(out[:, 2:2 + wf], x[perm])
    assert torch.equal(out[:, wf + 4:wf + 5], 1.0 - dones[perm].float())
    assert torch.isnan(out[:, :2]).all() and torch.isnan(out[:, 2 + wf:wf + 4]).all()
    assert torch.isnan(out[:, wf + 5:]).all()


@pytest.mark.parametrize("rows", [1, 1000, 98304 + 5])
def test_interleave_columns_matches_cat(cuda, rows):
    """Column blocks of different widths and strides side by side, bit-exact (torch.cat of the same views); the
    destination's columns past them stay untouched."""
    ops = _ops()
    torch.manual_seed(rows)
    a = torch.randn(rows, 3, device=cuda)
    b = torch.randn(rows, 5, device=cuda)[:, 1:2]
    c = torch.randn(rows, 1, device=cuda)
    d = torch.randn(rows, 9, device=cuda)[:, 2:8]
    dst = torch.full((rows, 16), float("nan"), device=cuda)
    ops.interleave_columns([a, b, c, d], dst)
    assert torch.equal(dst[:, :11], torch.cat([a, b, c, d], 1))
    assert torch.isnan(dst[:, 11:]).all()


# ----------------------------------------------------------------------------------------------------------------------
# A6 linear layers
# ----------------------------------------------------------------------------------------------------------------------


def _elu64(z):
    return torch.where(z > 0, z, torch.expm1(z))


@pytest.mark.parametrize("rows,aligned_x", [(1, False), (77, False), (1000, False), (24576, False), (1000, True),
                                            (24576, True)])
def test_linear_fwd_grouped(cuda, rows, aligned_x):
    """Strided inputs (ld = in + 5, offset 2: 4-byte loads), or 16-byte aligned inputs with one weight of 96 and one of
    99 input columns in the same launch (16-byte weight loads for the first problem only, as the update's first
    layer with a 99-wide critic input issues them)."""
    ops = _ops()
    torch.manual_seed(rows)
    shapes = [(96, 512), (99, 512)] if rows != 77 else [(99, 29), (48, 1)]
    probs, refs = [], []
    for i, (fin, fout) in enumerate(shapes):
        x = torch.randn(rows, fin)
        w = torch.randn(fout, fin) / math.sqrt(fin)
        b = torch.randn(fout)
        if aligned_x:
            ld = (fin + 3) // 4 * 4 + 4
            xd = torch.zeros(rows, ld, device=cuda)
            xd[:, :fin].copy_(x)
            xv = xd[:, :fin]
        else:
            xd = torch.zeros(rows, fin + 5, device=cuda)
            xd[:, 2:2 + fin].copy_(x)
            xv = xd[:, 2:2 + fin]
        z, h = torch.empty(rows, fout, device=cuda), torch.empty(rows, fout, device=cuda)
        probs.append((xv, w.to(cuda), b.to(cuda), z, h))
        z64 = x.double() @ w.double().t() + b.double()
        refs.append((z, h, z64))
    ops.linear_fwd(probs, rows, elu=True)
    for z, h, z64 in refs:
        assert rel_err(z, z64) < 2e-6
        assert rel_err(h, _elu64(z64)) < 2e-6


_ACT64 = {  # the activations' closed forms in fp64 (torch's modules with their default arguments)
    "elu": lambda z: torch.where(z > 0, z, torch.expm1(z)),
    "selu": lambda z: 1.0507009873554805 * torch.where(z > 0, z, 1.6732632423543772 * torch.expm1(z)),
    "relu": lambda z: z.clamp(min=0),
    "crelu": lambda z: torch.where(z > 0, z, torch.expm1(z)),
    "lrelu": lambda z: torch.where(z > 0, z, 0.01 * z),
    "tanh": torch.tanh,
    "sigmoid": torch.sigmoid,
    "softplus": lambda z: torch.where(z > 20, z, torch.log1p(torch.exp(z))),
    "gelu": lambda z: 0.5 * z * (1 + torch.erf(z / math.sqrt(2))),
    "swish": lambda z: z * torch.sigmoid(z),
    "mish": lambda z: z * torch.tanh(torch.log1p(torch.exp(z))),
    "identity": lambda z: z,
}


@pytest.mark.parametrize("name", list(_ACT64))
@pytest.mark.parametrize("aligned", [True, False])
def test_linear_activations(cuda, name, aligned):
    """Every hidden-layer activation rsl_rl resolves (rsl_rl/utils/utils.py:34-68): the forward's h = act(x w^T + b)
    and the input-grad's (dz w) * act'(.) from the activation's input z and, for the monotone ones, from its output h,
    against fp64 (autograd of the closed form for act'), on the bf16x6 kernels (16-byte rows) and on the fp32-MFMA
    kernels (rows one float off 16 bytes); a plain input-grad (no activation) beside them in the forward test."""
    from tt_rsl_rl_amd import _lib as L

    ops = _ops()
    act = L.ACTIVATIONS[name]
    torch.manual_seed(act + 100 * aligned)
    rows, fin, fout = 3000, 96, 256
    x = torch.randn(rows, fin)
    w = torch.randn(fout, fin) / math.sqrt(fin) * 2
    b = torch.randn(fout)
    z64 = x.double() @ w.double().t() + b.double()
    h64 = _ACT64[name](z64)
    xd = _operand(x, "bx6" if aligned else "fp32", cuda)
    z, h = torch.empty(rows, fout, device=cuda), torch.empty(rows, fout, device=cuda)
    ops.linear_fwd([(xd, w.to(cuda), b.to(cuda), z, h)], rows, act=act)
    assert rel_err(z, z64) < 2e-6
    assert rel_err(h, h64) < 2e-6, name
    # input-grad into that layer: dz_prev = (dz w2) * act'(z)
    w2 = torch.randn(64, fout) / 8
    dz = torch.randn(rows, 64)
    zr = z.detach().double().cpu().requires_grad_(True)
    g64 = torch.autograd.grad(_ACT64[name](zr).sum(), zr)[0]
    ref = (dz.double() @ w2.double()) * g64
    sources = [(False, z)] + ([(True, h)] if act in L.ACT_FROM_OUTPUT else [])
    for from_output, src in sources:
        out = torch.empty(rows, fout, device=cuda)
        ops.linear_bwd_dx([(_operand(dz, "bx6" if aligned else "fp32", cuda), w2.to(cuda), src, out)], rows,
                          elu_from_output=from_output, act=act)
        assert rel_err(out, ref) < 2e-6, (name, from_output)


@pytest.mark.parametrize("rows", [1, 130, 24576 + 77])
@pytest.mark.parametrize("elu", [True, False])
def test_linear_fwd_narrow_inputs(cuda, rows, elu):
    """First-layer shapes: inputs of 33..104 columns with 16-byte aligned rows, widths that are not multiples of the
    k-slab (the masked tail slab; the input columns past the width hold NaN and must not reach the result), ragged rows
    and outputs, weights with and without 16-byte rows in one launch.  Checked against fp64."""
    ops = _ops()
    torch.manual_seed(rows + 7)
    shapes = [(33, 200), (48, 512), (99, 130), (104, 96)]
    probs, refs = [], []
    for fin, fout in shapes:
        x = torch.randn(rows, fin)
        w = torch.randn(fout, fin) / math.sqrt(fin)
        b = torch.randn(fout)
        ld = (fin + 3) // 4 * 4 + 8
        xd = torch.full((rows, ld), float("nan"), device=cuda)  # columns past `fin` must never reach the result
        xd[:, :fin].copy_(x)
        z = torch.empty(rows, fout, device=cuda)
        h = torch.empty(rows, fout, device=cuda) if elu else None
        probs.append((xd[:, :fin], w.to(cuda), b.to(cuda), z, h))
        refs.append((z, h, x.double() @ w.double().t() + b.double()))
    ops.linear_fwd(probs, rows, elu=elu)
    for z, h, z64 in refs:
        assert rel_err(z, z64) < 2e-6
        if elu:
            assert rel_err(h, _elu64(z64)) < 2e-6


@pytest.mark.parametrize("rows,fin,fout,act,from_output", [(24576, 512, 256, True, False), (1000, 128, 29, True, False),
                                                         (333, 256, 1, False, False), (24576, 512, 256, True, True),
                                                         (77, 99, 5, True, True)])
def test_linear_bwd_dx(cuda, rows, fin, fout, act, from_output):
    """ELU' from the input z (torch's elu_backward) or from the output h = elu(z): the same derivative."""
    ops = _ops()
    torch.manual_seed(fin + fout)
    dz = torch.randn(rows, fout)
    w = torch.randn(fout, fin) / math.sqrt(fout)
    zp = torch.randn(rows, fin) * 2 if act else None
    src = None
    if act:
        src = torch.where(zp > 0, zp, torch.expm1(zp)) if from_output else zp
    ref = dz.double() @ w.double()
    if act:
        ref = ref * torch.where(zp.double() > 0, torch.ones_like(ref), torch.exp(zp.double()))
    probs = lambda out: [(dz.to(cuda), w.to(cuda), None if src is None else src.to(cuda), out)]
    out = torch.empty(rows, fin, device=cuda)
    ops.linear_bwd_dx(probs(out), rows, elu_from_output=from_output)
    assert rel_err(out, ref) < 2e-6


@pytest.mark.parametrize("elu", [True, False])
def test_linear_persistent_walks_several_tiles(cuda, elu):
    """The persistent forward / input-grad launches (16-byte operands, k a multiple of 16): 100,003 rows give each
    resident block several tiles, the last row tile ragged; grouped problems with different k (96, 112, 48) and
    output widths (512, 12) stream their k-slabs across tile boundaries.  Output rows and columns past the problem
    (a NaN sentinel) must stay untouched: the epilogue's dropped stores land nowhere."""
    ops = _ops()
    torch.manual_seed(41 + elu)
    rows = 100_003
    shapes = [(96, 512), (112, 512), (48, 12)]
    table = torch.randn(rows, 272, device=cuda)  # inputs: column blocks of one row-major table
    probs, refs, col = [], [], 0
    for fin, fout in shapes:
        xv = table[:, col:col + fin]
        col += fin
        w = torch.randn(fout, fin, device=cuda) / math.sqrt(fin)
        b = torch.randn(fout, device=cuda)
        z = torch.full((rows + 3, fout + 4), float("nan"), device=cuda)
        h = torch.full((rows + 3, fout + 4), float("nan"), device=cuda) if elu else None
        probs.append((xv, w, b, z[:rows, :fout], None if h is None else h[:rows, :fout]))
        refs.append((z, h, xv.double() @ w.double().t() + b.double(), fout))
    ops.linear_fwd(probs, rows, elu=elu)
    for z, h, z64, fout in refs:
        for out, want in ((z, z64), (h, None if h is None else _elu64(z64))):
            if out is None:
                continue
            assert rel_err(out[:rows, :fout], want) < 2e-6
            assert torch.isnan(out[rows:]).all() and torch.isnan(out[:, fout:]).all(), "store outside the output"
    # input-grads of two layers in one launch, ELU' from the layer's output
    dx_shapes = [(512, 256), (256, 128)]
    probs, refs = [], []
    for fin, fout in dx_shapes:
        dz = torch.randn(rows, fout, device=cuda)
        w = torch.randn(fout, fin, device=cuda) / math.sqrt(fout)
        zp = torch.randn(rows, fin, device=cuda) * 2
        hp = torch.where(zp > 0, zp, torch.expm1(zp))
        out = torch.full((rows + 3, fin + 4), float("nan"), device=cuda)
        probs.append((dz, w, hp, out[:rows, :fin]))
        ref = (dz.double() @ w.double()) * torch.where(zp.double() > 0, 1.0, torch.exp(zp.double()))
        refs.append((out, ref, fin))
    ops.linear_bwd_dx(probs, rows, elu_from_output=True)
    for out, ref, fin in refs:
        assert rel_err(out[:rows, :fin], ref) < 2e-6
        assert torch.isnan(out[rows:]).all() and torch.isnan(out[:, fin:]).all(), "store outside the output"


@pytest.mark.parametrize("rows", [1, 5, 130, 24576 + 77])
def test_linear_matrix_core_path_small_and_ragged(cuda, rows):
    """Operands with 16-byte rows and k a multiple of 16 (the bf16x6 matrix-core kernels) at row counts below one
    tile, ragged and above: forward with ELU (outputs of 512 and 12 columns, the second a partial column tile),
    input-grad with ELU' from the output, weight-grad with bias sums; fp64 references, NaN in every padding column
    of the operands (it must not reach a result) and around the outputs (nothing stored outside)."""
    ops = _ops()
    torch.manual_seed(rows + 13)

    def padded(t):
        buf = torch.full((t.shape[0], -(-t.shape[1] // 4) * 4 + 4), float("nan"), device=cuda)
        buf[:, :t.shape[1]].copy_(t)
        return buf[:, :t.shape[1]]

    shapes = [(112, 512), (64, 12)]
    probs, refs = [], []
    for fin, fout in shapes:
        x = torch.randn(rows, fin)
        w = torch.randn(fout, fin) / math.sqrt(fin)
        b = torch.randn(fout)
        out = torch.full((rows + 2, fout + 4), float("nan"), device=cuda)
        probs.append((padded(x), w.to(cuda), b.to(cuda), None, out[:rows, :fout]))
        refs.append((out, fout, _elu64(x.double() @ w.double().t() + b.double())))
    ops.linear_fwd(probs, rows, elu=True)
    for out, fout, ref in refs:
        assert rel_err(out[:rows, :fout], ref) < 2e-6
        assert torch.isnan(out[rows:]).all() and torch.isnan(out[:, fout:]).all()

    dz = torch.randn(rows, 256)
    w = torch.randn(256, 128) / 16
    zp = torch.randn(rows, 128) * 2
    hp = torch.where(zp > 0, zp, torch.expm1(zp))
    out = torch.full((rows + 2, 132), float("nan"), device=cuda)
    ops.linear_bwd_dx([(padded(dz), w.to(cuda), padded(hp), out[:rows, :128])], rows, elu_from_output=True)
    ref = (dz.double() @ w.double()) * torch.where(zp.double() > 0, 1.0, torch.exp(zp.double()))
    assert rel_err(out[:rows, :128], ref) < 2e-6
    assert torch.isnan(out[rows:]).all() and torch.isnan(out[:, 128:]).all()

    dw = torch.full((256, 128), float("nan"), device=cuda)
    db = torch.full((256,), float("nan"), device=cuda)
    ops.linear_bwd_dw([(padded(dz), padded(hp), dw, db)], rows)
    assert rel_err(dw, dz.double().t() @ hp.double()) < 2e-6
    assert ((db.cpu().double() - dz.double().sum(0)).abs() / dz.double().abs().sum(0)).max().item() < 1e-6


def test_linear_fwd_h_only(cuda):
    """With ELU the pre-activation output may be omitted: h alone is written, z's buffer is untouched."""
    ops = _ops()
    torch.manual_seed(5)
    rows, fin, fout = 1000, 96, 512
    x, w, b = torch.randn(rows, fin), torch.randn(fout, fin) / math.sqrt(fin), torch.randn(fout)
    h = torch.empty(rows, fout, device=cuda)
    ops.linear_fwd([(x.to(cuda), w.to(cuda), b.to(cuda), None, h)], rows, elu=True)
    z64 = x.double() @ w.double().t() + b.double()
    assert rel_err(h, _elu64(z64)) < 2e-6


@pytest.mark.parametrize("rows,padded", [(24576, False), (1000, False), (5, False), (24576, True), (1000, True),
                                         (64, True), (5, True)])
def test_linear_bwd_dw_grouped(cuda, rows, padded):
    """Contiguous operands (widths 29, 1, 99: the fp32 kernel) or operands in rows padded to 16 bytes, as the update
    stores them (the bf16x6 kernel: whole 32-row slab pairs at 24,576 and 64 rows, a clamped and zeroed tail at 1000
    and 5); bias gradients included."""
    ops = _ops()
    torch.manual_seed(rows + 1)
    shapes = [(99, 512), (512, 256), (256, 128), (128, 29), (96, 512), (512, 256), (256, 128), (128, 1)]

    def dev(t):
        if not padded:
            return t.to(cuda)
        buf = torch.full((t.shape[0], -(-t.shape[1] // 4) * 4), float("nan"), device=cuda)
        buf[:, :t.shape[1]].copy_(t)
        return buf[:, :t.shape[1]]

    probs, refs = [], []
    for fin, fout in shapes:
        dz = torch.randn(rows, fout) / rows
        x = torch.randn(rows, fin)
        dw = torch.full((fout, fin), float("nan"), device=cuda)
        db = torch.full((fout,), float("nan"), device=cuda)
        probs.append((dev(dz), dev(x), dw, db))
        refs.append((dw, db, dz.double().t() @ x.double(), dz.double().sum(0), dz.double().abs().sum(0)))
    # the last problem without a bias gradient (db = NULL: its column sums are skipped)
    nb = probs[-1][3]
    probs[-1] = probs[-1][:3] + (None,)
    ops.linear_bwd_dw(probs, rows)
    assert torch.isnan(nb).all()
    for dw, db, rw, rb, rb_abs in refs[:-1]:
        assert rel_err(dw, rw) < 2e-6
        # a bias gradient is a sum that can cancel: bound the error by the sum of |terms| (dot-product bound)
        assert ((db.cpu().double() - rb).abs() / rb_abs).max().item() < 1e-6
    assert rel_err(refs[-1][0], refs[-1][2]) < 2e-6


@pytest.mark.parametrize("rows", [24576, 1000, 64, 5])
def test_linear_bwd_dw_narrow_tiles(cuda, rows):
    """Problems at most 64 inputs wide (the 48-wide first layers of the flat and recurrent workloads, 64, 33 and 1)
    run on 128 x 64 tiles with half the splits of the full-width problems in the same launch; operands in rows padded
    to 16 bytes with NaN in the padding, fp64 references, bias gradients included."""
    ops = _ops()
    torch.manual_seed(rows + 7)
    shapes = [(48, 512), (512, 256), (64, 1024), (33, 128), (256, 12), (1, 64)]

    def dev(t):
        buf = torch.full((t.shape[0], -(-t.shape[1] // 4) * 4), float("nan"), device=cuda)
        buf[:, :t.shape[1]].copy_(t)
        return buf[:, :t.shape[1]]

    probs, refs = [], []
    for fin, fout in shapes:
        dz = torch.randn(rows, fout) / rows
        x = torch.randn(rows, fin)
        dw = torch.full((fout, fin), float("nan"), device=cuda)
        db = torch.full((fout,), float("nan"), device=cuda)
        probs.append((dev(dz), dev(x), dw, db))
        refs.append((dw, db, dz.double().t() @ x.double(), dz.double().sum(0), dz.double().abs().sum(0)))
    ops.linear_bwd_dw(probs, rows)
    for dw, db, rw, rb, rb_abs in refs:
        assert rel_err(dw, rw) < 2e-6
        assert ((db.cpu().double() - rb).abs() / rb_abs).max().item() < 1e-6


def _gemm_errors(c: torch.Tensor, c64: torch.Tensor, bound: torch.Tensor) -> tuple[float, float]:
    """(relative Frobenius error against fp64, largest per-element error over the element's |A| |B| bound)."""
    e = (c.double() - c64).abs()
    return float(e.norm() / c64.norm()), float((e / bound.clamp(min=1e-300)).max())


def _operand(t: torch.Tensor, path: str, cuda) -> torch.Tensor:
    """t on the device in 16-byte rows (the bf16x6 matrix-core kernels) or one float past a 16-byte boundary (the
    fp32-MFMA kernels take operands the bf16x6 kernels cannot)."""
    rows, cols = t.shape
    if path == "bx6":
        buf = torch.zeros(rows, -(-cols // 4) * 4, device=cuda)
        buf[:, :cols].copy_(t)
        return buf[:, :cols]
    buf = torch.zeros(rows, cols + 4, device=cuda)
    buf[:, 1:1 + cols].copy_(t)
    return buf[:, 1:1 + cols]


def _scaled(rows: int, cols: int, wide: bool, g: torch.Generator) -> torch.Tensor:
    """N(0, 1) entries; wide: times row and column magnitudes log-uniform over [1e-6, 1e6]."""
    x = torch.randn(rows, cols, generator=g)
    if wide:
        x *= 10.0 ** (12 * torch.rand(rows, 1, generator=g) - 6) * 10.0 ** (12 * torch.rand(1, cols, generator=g) - 6)
    return x


@pytest.mark.parametrize("op,rows,wide", [("fwd", 24576, False), ("fwd", 24576, True), ("dx", 24576, False),
                                          ("dx", 24576, True), ("dw", 24576, False), ("dw", 24576, True),
                                          ("dw", 393216, False)])
def test_bx6_error_against_fp32_mfma(cuda, op, rows, wide):
    """The bf16x6 GEMMs (fp32 operands as three bf16 parts, six bf16 MFMA products, fp32 accumulation) against the
    fp32-MFMA kernels on identical problems: forward (x w^T), input-grad (dz w) and weight-grad (dz^T x, k = the rows:
    24,576, and 393,216 as in the 65,536-env mini-batches), N(0, 1) operands and operands whose row and column
    magnitudes are log-uniform over [1e-6, 1e6].  Both errors are measured against fp64 two ways (relative Frobenius;
    per element over its |A| |B| bound), and the bf16x6 error must be at most twice the fp32-MFMA one by both, and
    within the fp32-GEMM bar of 2e-6 (per element over its bound; relative Frobenius up to 24,576 rows).  The two
    results must differ in some bits (two different kernels ran)."""
    ops = _ops()
    g = torch.Generator().manual_seed(rows + 3 * wide + {"fwd": 1, "dx": 2, "dw": 3}[op])
    fin, fout = 512, 256
    out = {}
    if op == "fwd":
        x, w = _scaled(rows, fin, wide, g), _scaled(fout, fin, wide, g)
        xd, wd = x.to(cuda).double(), w.to(cuda).double()
        c64, bound = xd @ wd.t(), xd.abs() @ wd.abs().t()
        for path in ("bx6", "fp32"):
            z = torch.empty(rows, fout, device=cuda)
            ops.linear_fwd([(_operand(x, path, cuda), w.to(cuda), torch.zeros(fout, device=cuda), z, None)], rows,
                           elu=False)
            out[path] = z
    elif op == "dx":
        dz, w = _scaled(rows, fout, wide, g), _scaled(fout, fin, wide, g)
        dzd, wd = dz.to(cuda).double(), w.to(cuda).double()
        c64, bound = dzd @ wd, dzd.abs() @ wd.abs()
        for path in ("bx6", "fp32"):
            dx = torch.empty(rows, fin, device=cuda)
            ops.linear_bwd_dx([(_operand(dz, path, cuda), w.to(cuda), None, dx)], rows)
            out[path] = dx
    else:
        dz, x = _scaled(rows, fout, wide, g), _scaled(rows, fin, wide, g)
        dzd, xd = dz.to(cuda).double(), x.to(cuda).double()
        c64, bound = dzd.t() @ xd, dzd.abs().t() @ xd.abs()
        for path in ("bx6", "fp32"):
            dw, db = torch.empty(fout, fin, device=cuda), torch.empty(fout, device=cuda)
            ops.linear_bwd_dw([(_operand(dz, path, cuda), _operand(x, path, cuda), dw, db)], rows)
            out[path] = dw
    torch.cuda.synchronize()
    assert not torch.equal(out["bx6"], out["fp32"]), "both paths ran the same kernel"
    e6, e32 = _gemm_errors(out["bx6"], c64, bound), _gemm_errors(out["fp32"], c64, bound)
    print(f"{op} rows={rows} wide={wide}: bf16x6 rel-Frobenius {e6[0]:.3e} per-element/bound {e6[1]:.3e}; "
          f"fp32 MFMA {e32[0]:.3e} / {e32[1]:.3e}; ratios {e6[0] / e32[0]:.2f} / {e6[1] / e32[1]:.2f}")
    rec = os.environ.get("PPO_PARITY_RECORD")
    if rec:
        os.makedirs(rec, exist_ok=True)
        with open(os.path.join(rec, f"bx6_vs_fp32_{op}_{rows}_{'wide' if wide else 'randn'}.json"), "w") as f:
            json.dump({"op": op, "rows": rows, "wide_range": wide, "in": fin, "out": fout,
                       "bx6": {"rel_frobenius": e6[0], "per_element_over_bound": e6[1]},
                       "fp32_mfma": {"rel_frobenius": e32[0], "per_element_over_bound": e32[1]},
                       "ratio": {"rel_frobenius": e6[0] / e32[0], "per_element_over_bound": e6[1] / e32[1]}}, f,
                      indent=1)
    assert e6[0] <= 2 * e32[0], (e6, e32)
    assert e6[1] <= 2 * e32[1], (e6, e32)
    assert e6[1] < 2e-6
    if rows <= 24576:  # (a sum of 393,216 products rounds more: both kernels' relative error grows with k)
        assert e6[0] < 2e-6


@pytest.mark.parametrize("rows", [24576, 96, 64])
def test_linear_bwd_dw_partial_tiles(cuda, rows):
    """Weight-grads whose outputs (384, 300, 29) or inputs (200, 99) leave partial 128-wide tiles, beside full-width and
    narrow (48-input, 128 x 64) problems in one launch, with whole 32-row slab pairs (rows a multiple of 32: 2 splits of
    64 and 32 rows at 96); operands in rows padded to 16 bytes with NaN in the padding, fp64 references, bias
    gradients included (one problem without)."""
    ops = _ops()
    torch.manual_seed(rows + 11)
    shapes = [(200, 384), (99, 300), (96, 512), (512, 256), (48, 256), (128, 29), (256, 128)]

    def dev(t):
        buf = torch.full((t.shape[0], -(-t.shape[1] // 4) * 4), float("nan"), device=cuda)
        buf[:, :t.shape[1]].copy_(t)
        return buf[:, :t.shape[1]]

    probs, refs = [], []
    for fin, fout in shapes:
        dz = torch.randn(rows, fout) / rows
        x = torch.randn(rows, fin)
        dw = torch.full((fout, fin), float("nan"), device=cuda)
        db = torch.full((fout,), float("nan"), device=cuda)
        probs.append((dev(dz), dev(x), dw, db))
        refs.append((dw, db, dz.double().t() @ x.double(), dz.double().sum(0), dz.double().abs().sum(0)))
    probs[1] = probs[1][:3] + (None,)
    ops.linear_bwd_dw(probs, rows)
    for i, (dw, db, rw, rb, rb_abs) in enumerate(refs):
        assert rel_err(dw, rw) < 2e-6, shapes[i]
        if i == 1:
            assert torch.isnan(db).all()
        else:
            assert ((db.cpu().double() - rb).abs() / rb_abs).max().item() < 1e-6, shapes[i]


# ----------------------------------------------------------------------------------------------------------------------
# A8-A11 losses
# ----------------------------------------------------------------------------------------------------------------------


def _loss_case(rows, A, std_type, clipped, seed, ratio_spread=0.3):
    g = torch.Generator().manual_seed(seed)
    mean = torch.randn(rows, A, generator=g) * 0.5
    if std_type == "log":
        param = torch.randn(A, generator=g) * 0.3
        std = torch.exp(param)
    else:
        param = torch.rand(A, generator=g) + 0.5
        std = param.clone()
    actions = mean + std * torch.randn(rows, A, generator=g)
    old_mean = mean + ratio_spread * 0.1 * torch.randn(rows, A, generator=g)
    old_std = std * (1 + 0.05 * torch.randn(A, generator=g)).abs()
    old_std = old_std.expand(rows, A).contiguous()
    old_logp = torch.distributions.Normal(old_mean, old_std).log_prob(actions).sum(-1) + ratio_spread * torch.randn(
        rows, generator=g)
    adv = torch.randn(rows, generator=g)
    value = torch.randn(rows, generator=g)
    old_value = value + 0.3 * torch.randn(rows, generator=g)
    ret = value + torch.randn(rows, generator=g)
    return dict(mean=mean, param=param, actions=actions, old_mean=old_mean, old_std=old_std, old_logp=old_logp,
                adv=adv, value=value, old_value=old_value, ret=ret)


def _oracle_loss(c, std_type, clipped, clip=0.2, cv=1.0, ce=0.01, dtype=torch.float32):
    """The oracle's loss block (ppo_loss_terms + GaussianDistribution) with torch autograd, in `dtype`."""
    c = {k: v.to(dtype) for k, v in c.items()}
    dist = O.GaussianDistribution(c["mean"].shape[1], std_type=std_type).to(dtype)
    with torch.no_grad():
        (dist.std_param if std_type == "scalar" else dist.log_std_param).copy_(c["param"])
    mean = c["mean"].clone().requires_grad_(True)
    value = c["value"].clone().requires_grad_(True)
    dist.update(mean)
    logp = dist.log_prob(c["actions"])
    entropy = dist.entropy
    with torch.no_grad():
        kl = dist.kl_divergence((c["old_mean"], c["old_std"]), dist.params).mean()
    s, v, loss = O.ppo_loss_terms(logp, c["old_logp"].unsqueeze(-1), c["adv"].unsqueeze(-1), value, c["old_value"],
                                  c["ret"], entropy, clip, clipped, cv, ce)
    loss.backward()
    p = dist.std_param if std_type == "scalar" else dist.log_std_param
    return dict(surrogate=s.item(), value=v.item(), entropy=entropy.mean().item(), kl=kl.item(), d_mean=mean.grad,
                d_value=value.grad, d_param=p.grad)


@pytest.mark.parametrize("rows,A,std_type,clipped", [(24576, 29, "log", True), (1000, 12, "scalar", True),
                                                     (77, 1, "log", False), (1, 3, "log", True)])
def test_ppo_loss_matches_autograd(cuda, rows, A, std_type, clipped):
    ops = _ops()
    from tt_rsl_rl_amd import _lib as L

    c = _loss_case(rows, A, std_type, clipped, seed=rows + A)
    ref = _oracle_loss(c, std_type, clipped)  # fp32, upstream's own arithmetic
    ref64 = _oracle_loss(c, std_type, clipped, dtype=torch.float64)  # the same formulas in fp64
    W = 3 * A + 4
    tab = torch.zeros(rows, W)
    tab[:, 0:A], tab[:, A:2 * A], tab[:, 2 * A:3 * A] = c["actions"], c["old_mean"], c["old_std"]
    tab[:, 3 * A], tab[:, 3 * A + 1], tab[:, 3 * A + 2], tab[:, 3 * A + 3] = c["old_logp"], c["adv"], c["old_value"], \
        c["ret"]
    tab = tab.to(cuda)
    batch = {"ld": W, "actions": tab[:, 0], "old_mean": tab[:, A], "old_std": tab[:, 2 * A],
             "old_logp": tab[:, 3 * A], "advantages": tab[:, 3 * A + 1], "old_values": tab[:, 3 * A + 2],
             "returns": tab[:, 3 * A + 3]}
    mean, value, param = c["mean"].to(cuda), c["value"].to(cuda), c["param"].to(cuda)
    d_mean, d_value, d_param = torch.empty(rows, A, device=cuda), torch.empty(rows, device=cuda), torch.empty(A, device=cuda)
    if std_type == "log":
        lo, hi, st = math.log(1e-6), math.log(1e6), L.PPO_STD_LOG
    else:
        lo, hi, st = 1e-6, 1e6, L.PPO_STD_SCALAR
    args = ops.make_loss_args(rows, mean, value, batch, param, st, lo, hi, 0.2, 1.0, 0.01, clipped, d_mean, d_value)
    ws = torch.empty(ops.loss_workspace_bytes(rows, A), dtype=torch.uint8, device=cuda)
    state = ops.new_device_state(1e-3, cuda)
    trace = torch.zeros(5, dtype=torch.float64, device=cuda)
    ops.ppo_loss(args, ws)
    ops.ppo_loss_finalize(args, ws, d_param, state, True, 0.01, trace)
    tr = trace.cpu().tolist()
    assert abs(tr[2] - ref["surrogate"]) <= 2e-6 * max(1.0, abs(ref["surrogate"]))
    assert abs(tr[3] - ref["value"]) <= 2e-6 * max(1.0, abs(ref["value"]))
    assert abs(tr[4] - ref["entropy"]) <= 2e-6 * max(1.0, abs(ref["entropy"]))
    assert abs(tr[0] - ref["kl"]) <= 1e-6 * max(1e-3, abs(ref["kl"])) + 1e-7
    # gradients: within fp32 noise of the fp64 truth, and of upstream's fp32 autograd (2e-5, the loss-gradient bar)
    for key, got in (("d_mean", d_mean), ("d_value", d_value), ("d_param", d_param)):
        assert rel_err(got, ref64[key], 1e-12) < 1e-5, key
        assert rel_err(got, ref[key], 1e-12) < 2e-5, key
    lr_ref = O.adaptive_lr(torch.tensor(tr[0], dtype=torch.float32), 1e-3, 0.01)
    assert tr[1] == lr_ref


def _head_case(rows, A, ka, kc, std_type, seed):
    """Last hidden activations (ELU outputs), output layers, and a batch whose actions / old distribution sit around
    the head's own means (so the ratios straddle the clip range instead of all clipping)."""
    g = torch.Generator().manual_seed(seed)
    h_a = torch.nn.functional.elu(torch.randn(rows, ka, generator=g))
    h_c = torch.nn.functional.elu(torch.randn(rows, kc, generator=g))
    w_a = torch.randn(A, ka, generator=g) / math.sqrt(ka)
    b_a = 0.1 * torch.randn(A, generator=g)
    w_c = torch.randn(1, kc, generator=g) / math.sqrt(kc)
    b_c = 0.1 * torch.randn(1, generator=g)
    mean = (h_a.double() @ w_a.double().T + b_a.double()).float()
    value = (h_c.double() @ w_c.double().T + b_c.double()).float().squeeze(1)
    c = _loss_case(rows, A, std_type, True, seed)
    shift_m = mean - c["mean"]
    for k in ("actions", "old_mean"):
        c[k] = c[k] + shift_m
    shift_v = value - c["value"]
    for k in ("old_value", "ret"):
        c[k] = c[k] + shift_v
    c.update(mean=mean, value=value)
    return c, dict(h_a=h_a, h_c=h_c, w_a=w_a, b_a=b_a, w_c=w_c, b_c=b_c)


def _head_reference(c, net, std_type, clipped):
    """fp64 autograd through both output layers and the oracle's loss block: the gradients with respect to the last
    hidden activations, times ELU' taken from those activations (h > 0 ? 1 : h + 1)."""
    d = {k: v.double() for k, v in net.items()}
    h_a = d["h_a"].clone().requires_grad_(True)
    h_c = d["h_c"].clone().requires_grad_(True)
    dist = O.GaussianDistribution(c["mean"].shape[1], std_type=std_type).double()
    with torch.no_grad():
        (dist.std_param if std_type == "scalar" else dist.log_std_param).copy_(c["param"].double())
    mean = h_a @ d["w_a"].T + d["b_a"]
    mean.retain_grad()
    value = (h_c @ d["w_c"].T + d["b_c"]).squeeze(1)
    value.retain_grad()
    cc = {k: v.double() for k, v in c.items()}
    dist.update(mean)
    logp = dist.log_prob(cc["actions"])
    s, v, loss = O.ppo_loss_terms(logp, cc["old_logp"].unsqueeze(-1), cc["adv"].unsqueeze(-1), value,
                                  cc["old_value"], cc["ret"], dist.entropy, 0.2, clipped, 1.0, 0.01)
    loss.backward()
    elu_a = torch.where(d["h_a"] > 0, 1.0, d["h_a"] + 1.0)
    elu_c = torch.where(d["h_c"] > 0, 1.0, d["h_c"] + 1.0)
    p = dist.std_param if std_type == "scalar" else dist.log_std_param
    return dict(mean=mean.detach(), value=value.detach(), d_mean=mean.grad, d_value=value.grad,
                dz_a=h_a.grad * elu_a, dz_c=h_c.grad * elu_c, d_param=p.grad, surrogate=s.item(), value_loss=v.item())


@pytest.mark.parametrize("rows,A,ka,kc,std_type,clipped", [
    (24576, 29, 128, 128, "log", True), (1000, 12, 64, 128, "scalar", True), (33, 32, 32, 16, "log", False),
    (1, 1, 96, 48, "log", True), (4097, 7, 128, 64, "scalar", False), (50, 17, 16, 16, "log", True),
    (393216, 12, 128, 128, "log", True)])
def test_fused_head_matches_autograd_and_the_separate_launches(cuda, rows, A, ka, kc, std_type, clipped):
    """ppo_gauss_ppo_head (output layers + loss + finalize + output-layer input-grad in one launch) against fp64
    autograd of the same mathematics, and against the separate launches (linear_fwd, ppo_loss + finalize,
    linear_bwd_dx) on the same inputs."""
    ops = _ops()
    from tt_rsl_rl_amd import _lib as L

    assert ops.head_supported(A, ka, kc)
    c, net = _head_case(rows, A, ka, kc, std_type, seed=rows + A + ka)
    ref = _head_reference(c, net, std_type, clipped)
    pad = lambda n: -(-n // 4) * 4
    W = 3 * pad(A) + 4 + 4
    tab = torch.zeros(rows, W)
    o_m, o_s, o_r = pad(A), 2 * pad(A), 3 * pad(A)
    tab[:, 0:A], tab[:, o_m:o_m + A], tab[:, o_s:o_s + A] = c["actions"], c["old_mean"], c["old_std"]
    tab[:, o_r], tab[:, o_r + 1], tab[:, o_r + 2], tab[:, o_r + 3] = c["old_logp"], c["adv"], c["old_value"], c["ret"]
    tab = tab.to(cuda)
    batch = {"ld": W, "actions": tab[:, 0], "old_mean": tab[:, o_m], "old_std": tab[:, o_s],
             "old_logp": tab[:, o_r], "advantages": tab[:, o_r + 1], "old_values": tab[:, o_r + 2],
             "returns": tab[:, o_r + 3]}
    dv = {k: v.to(cuda).contiguous() for k, v in net.items()}
    param = c["param"].to(cuda)
    if std_type == "log":
        lo, hi, st = math.log(1e-6), math.log(1e6), L.PPO_STD_LOG
    else:
        lo, hi, st = 1e-6, 1e6, L.PPO_STD_SCALAR
    buf = lambda w: torch.full((rows, pad(w)), float("nan"), device=cuda)[:, :w]

    def run(fused, reps=1):
        mean, value = buf(A), buf(1)
        d_mean, d_value = buf(A), buf(1)
        dz_a, dz_c = buf(ka), buf(kc)
        d_param = torch.empty(A, device=cuda)
        state = ops.new_device_state(1e-3, cuda)
        trace = torch.zeros(5 * reps, dtype=torch.float64, device=cuda)
        args = ops.make_loss_args(rows, mean, value[:, 0], batch, param, st, lo, hi, 0.2, 1.0, 0.01, clipped, d_mean,
                                  d_value[:, 0])
        if fused:
            ws = torch.empty(ops.head_workspace_bytes(rows, A), dtype=torch.uint8, device=cuda)
            for _ in range(reps):  # (the same state: one mini-batch after another)
                ops.ppo_head(args, dv["h_a"], dv["w_a"], dv["b_a"], dv["h_c"], dv["w_c"], dv["b_c"], dz_a, dz_c, ws,
                             d_param, state, True, 0.01, trace, mean=mean, value=value[:, 0])
            torch.cuda.synchronize()
            assert ops.read_device_state(state).num_minibatches == reps
        else:
            ops.linear_fwd([(dv["h_a"], dv["w_a"], dv["b_a"], mean, None), (dv["h_c"], dv["w_c"], dv["b_c"], value,
                                                                             None)], rows, elu=False)
            ws = torch.empty(ops.loss_workspace_bytes(rows, A), dtype=torch.uint8, device=cuda)
            ops.ppo_loss(args, ws)
            ops.ppo_loss_finalize(args, ws, d_param, state, True, 0.01, trace)
            ops.linear_bwd_dx([(d_mean, dv["w_a"], dv["h_a"], dz_a), (d_value, dv["w_c"], dv["h_c"], dz_c)], rows,
                              ops.Workspace(cuda), elu_from_output=True)
        torch.cuda.synchronize()
        return dict(mean=mean, value=value[:, 0], d_mean=d_mean, d_value=d_value[:, 0], dz_a=dz_a, dz_c=dz_c,
                    d_param=d_param, trace=trace.cpu().tolist())

    got, sep = run(True), run(False)
    # three calls in a row on one state give the same losses and gradients each time, and the learning rate follows
    # the rule from call to call
    again = run(True, reps=3)
    for key in ("d_mean", "dz_a", "dz_c", "d_param"):
        assert torch.equal(again[key], got[key]), key
    lr = 1e-3
    for i in range(3):
        row = again["trace"][5 * i:5 * i + 5]
        assert row[0] == got["trace"][0] and row[2:] == got["trace"][2:], i
        lr = O.adaptive_lr(torch.tensor(row[0], dtype=torch.float32), lr, 0.01)
        assert row[1] == lr, i
    for key in ("mean", "value"):
        assert rel_err(got[key], ref[key]) < 2e-6, key
    # gradients: fp32 noise of the fp64 truth (the loss-gradient bar), and the separate launches' within the same
    for key in ("d_mean", "d_value", "dz_a", "dz_c", "d_param"):
        assert torch.isfinite(got[key]).all(), key
        assert rel_err(got[key], ref[key], 1e-12) < 1e-5, key
        assert rel_err(got[key], sep[key], 1e-12) < 2e-5, key
    tr, ts = got["trace"], sep["trace"]
    assert abs(tr[2] - ref["surrogate"]) <= 2e-6 * max(1.0, abs(ref["surrogate"]))
    assert abs(tr[3] - ref["value_loss"]) <= 2e-6 * max(1.0, abs(ref["value_loss"]))
    assert tr[4] == ts[4]  # entropy depends on the std parameter alone
    assert abs(tr[0] - ts[0]) <= 1e-5 * max(1e-3, abs(ts[0]))
    assert tr[1] == O.adaptive_lr(torch.tensor(tr[0], dtype=torch.float32), 1e-3, 0.01)


def test_kl_is_exactly_zero_for_identical_distributions(cuda):
    ops = _ops()
    from tt_rsl_rl_amd import _lib as L

    from tt_rsl_rl_amd.models import GaussianDistribution

    rows, A = 4096, 12
    c = _loss_case(rows, A, "log", True, seed=5)
    # the rollout's stored std is produced by the same device code as the update's (act() -> gauss_sample)
    dist = GaussianDistribution(A, std_type="log").to(cuda)
    with torch.no_grad():
        dist.log_std_param.copy_(c["param"])
    std_d = torch.empty(rows, A, device=cuda)
    dist.sample_from(c["mean"].to(cuda), None, c["actions"].to(cuda), None, std_d)
    std = std_d.cpu()
    W = 3 * A + 4
    tab = torch.zeros(rows, W)
    tab[:, 0:A], tab[:, A:2 * A], tab[:, 2 * A:3 * A] = c["actions"], c["mean"], std
    tab = tab.to(cuda)
    batch = {"ld": W, "actions": tab[:, 0], "old_mean": tab[:, A], "old_std": tab[:, 2 * A],
             "old_logp": tab[:, 3 * A], "advantages": tab[:, 3 * A + 1], "old_values": tab[:, 3 * A + 2],
             "returns": tab[:, 3 * A + 3]}
    mean = c["mean"].to(cuda)
    value = torch.zeros(rows, device=cuda)
    param = c["param"].to(cuda)
    # the args struct holds raw pointers: every buffer it names must stay referenced until the kernels ran
    d_mean, d_value, d_param = torch.empty(rows, A, device=cuda), torch.empty(rows, device=cuda), torch.empty(A, device=cuda)
    args = ops.make_loss_args(rows, mean, value, batch, param, L.PPO_STD_LOG, math.log(1e-6), math.log(1e6), 0.2, 1.0,
                              0.01, True, d_mean, d_value)
    ws = torch.empty(ops.loss_workspace_bytes(rows, A), dtype=torch.uint8, device=cuda)
    state = ops.new_device_state(1e-3, cuda)
    trace = torch.zeros(5, dtype=torch.float64, device=cuda)
    ops.ppo_loss(args, ws)
    ops.ppo_loss_finalize(args, ws, d_param, state, True, 0.01, trace)
    kl, lr = trace.cpu().tolist()[:2]
    assert kl == 0.0 and lr == 1e-3, "KL(p||p) must round to exactly 0 so the LR is not raised (upstream S15-S17)"


# ----------------------------------------------------------------------------------------------------------------------
# A12-A13 clip + Adam
# ----------------------------------------------------------------------------------------------------------------------


@pytest.mark.parametrize("aligned", [False, True])
def test_adam_clip_matches_torch(cuda, aligned):
    """Group sizes 181,021 / 51,329 (scalar path) or 181,024 / 51,332 (multiples of 4: the float4 path)."""
    ops = _ops()
    torch.manual_seed(11)
    shapes_a = [(32,) if aligned else (29,), (512, 96), (512,), (256, 512), (256,)]
    shapes_c = [(512, 99), (512,), (1, 128), (4,) if aligned else (1,)]
    pa = [torch.nn.Parameter(torch.randn(s) * 0.1) for s in shapes_a]
    pc = [torch.nn.Parameter(torch.randn(s) * 0.1) for s in shapes_c]
    opt = torch.optim.Adam(pa + pc, lr=1e-3)
    flat = torch.cat([p.detach().reshape(-1) for p in pa + pc]).to(cuda)
    n_a = sum(p.numel() for p in pa)
    grad = torch.zeros_like(flat)
    m, v = torch.zeros_like(flat), torch.zeros_like(flat)
    gb = torch.tensor([0, n_a, flat.numel()], dtype=torch.int64)
    state = ops.new_device_state(1e-3, cuda)
    ws = ops.Workspace(cuda)
    lrs = [1e-3, 1e-3, 6.7e-4, 2e-3, 1e-5, 1e-2, 3e-3, 1e-3]
    for step, lr in enumerate(lrs, start=1):
        scale = 10.0 if step % 3 == 0 else 0.01  # both sides of the clip threshold
        for p in pa + pc:
            p.grad = torch.randn_like(p) * scale
        grad.copy_(torch.cat([p.grad.reshape(-1) for p in pa + pc]).to(cuda))
        for group in opt.param_groups:
            group["lr"] = lr
        torch.nn.utils.clip_grad_norm_(pa, 1.0)
        torch.nn.utils.clip_grad_norm_(pc, 1.0)
        opt.step()
        ops.reset_device_state(state, lr)
        ops.adam_step(flat, grad, m, v, gb, 1.0, 0.9, 0.999, 1e-8, 1 - 0.9 ** step, (1 - 0.999 ** step) ** 0.5,
                      state, ws)
        ref = torch.cat([p.detach().reshape(-1) for p in pa + pc])
        assert rel_err(flat, ref) < 1e-6, step
        ref_m = torch.cat([opt.state[p]["exp_avg"].reshape(-1) for p in pa + pc])
        ref_v = torch.cat([opt.state[p]["exp_avg_sq"].reshape(-1) for p in pa + pc])
        assert rel_err(m, ref_m) < 1e-6 and rel_err(v, ref_v) < 1e-6
        ref_g = torch.cat([p.grad.reshape(-1) for p in pa + pc])
        assert rel_err(grad, ref_g) < 1e-6, "clipped gradients are left in the gradient buffer like upstream"


def test_adam_prenorm_matches_torch(cuda):
    """Clip norms from the weight-grad launch: ppo_linear_bwd_dw_norm writes the gradients of two models' layers
    (groups 0 and 1) and the per-group sums of squares, plus an extra range (a std parameter written beforehand);
    the partial rows sum to the gradients' squared norms, and the one-launch Adam on them matches torch's
    clip_grad_norm_ per model + Adam, with the clip active and inactive."""
    ops = _ops()
    from tt_rsl_rl_amd import _lib as L

    torch.manual_seed(12)
    rows = 1000
    layers = [[(48, 64), (64, 12)], [(48, 64), (64, 1)]]
    pad = lambda n: -(-n // 16) * 16  # noqa: E731
    shapes, offs, groups_of, off = [], [], [], 0
    std_off = off
    off += pad(12)
    bounds = [0]
    for g, model in enumerate(layers):
        for i, o in model:
            for shp in ((o, i), (o,)):
                shapes.append(shp)
                offs.append(off)
                groups_of.append(g)
                off += pad(torch.Size(shp).numel())
        bounds.append(off)
    n = off
    params = torch.randn(n) * 0.1
    ref_p = [torch.nn.Parameter(params[std_off:std_off + 12].clone())]
    ref_p += [torch.nn.Parameter(params[o:o + torch.Size(sh).numel()].view(sh).clone()) for o, sh in zip(offs, shapes)]
    group0 = [ref_p[0]] + [p for p, g in zip(ref_p[1:], groups_of) if g == 0]
    group1 = [p for p, g in zip(ref_p[1:], groups_of) if g == 1]
    opt = torch.optim.Adam(group0 + group1, lr=1e-3)
    flat = params.to(cuda)
    grad = torch.zeros(n, device=cuda)
    m, v = torch.zeros_like(flat), torch.zeros_like(flat)
    gb = torch.tensor(bounds, dtype=torch.int64)
    state = ops.new_device_state(1e-3, cuda)
    partials = ops.grad_norm_partials(cuda)
    ws = ops.Workspace(cuda)
    for step in range(1, 7):
        scale = 10.0 if step % 2 == 0 else 0.001
        grad[std_off:std_off + 12] = torch.randn(12, device=cuda) * scale
        probs, k = [], 0
        for model in layers:
            for i, o in model:
                dz, x = torch.randn(rows, o, device=cuda) * scale, torch.randn(rows, i, device=cuda)
                probs.append((dz, x, grad[offs[k]:offs[k] + o * i].view(o, i), grad[offs[k + 1]:offs[k + 1] + o]))
                k += 2
        norm = ops.GradNorm(partials, [0, 0, 1, 1], grad, ((std_off, std_off + 12, 0),))
        ops.linear_bwd_dw(probs, rows, ws, norm=norm)
        g64 = grad.double()
        for g in (0, 1):
            want = float((g64[bounds[g]:bounds[g + 1]] ** 2).sum())
            got = float(partials[:, g].sum())
            assert abs(got - want) <= 1e-12 * want, (step, g, got, want)
        assert float(partials[:, 2:].abs().sum()) == 0.0
        for p_, o in zip(ref_p, [std_off] + offs):
            p_.grad = grad[o:o + p_.numel()].view(p_.shape).cpu().clone()
        torch.nn.utils.clip_grad_norm_(group0, 1.0)
        torch.nn.utils.clip_grad_norm_(group1, 1.0)
        opt.step()
        ops.reset_device_state(state, 1e-3)
        ops.adam_step(flat, grad, m, v, gb, 1.0, 0.9, 0.999, 1e-8, 1 - 0.9 ** step, (1 - 0.999 ** step) ** 0.5,
                      state, None, prenorm=partials)
        for p_, o in zip(ref_p, [std_off] + offs):
            got = flat[o:o + p_.numel()].cpu()
            assert rel_err(got, p_.detach().reshape(-1)) < 1e-6, step
            assert rel_err(grad[o:o + p_.numel()].cpu(), p_.grad.reshape(-1)) < 1e-6, "clipped gradient kept"
    assert L.DW_NORM_BLOCKS == partials.shape[0]


def test_adam_prenorm_mirror_matches_prenorm(cuda):
    """ppo_adam_step_prenorm_mirror: the flat buffers bit-identical to ppo_adam_step_prenorm's on the same inputs, and
    each mirrored range (row-major rows x cols at any flat offset, float4 boundaries straddled) written to its
    destination rows with the updated values bit for bit, the destination's columns past cols untouched."""
    ops = _ops()
    torch.manual_seed(21)
    n = 200_003 + 1
    bounds = torch.tensor([0, 120_000, n], dtype=torch.int64)
    flat = [torch.randn(n, device=cuda) * s for s in (0.1, 0.5, 0.01)] + [torch.rand(n, device=cuda) * 1e-3]
    partials = ops.grad_norm_partials(cuda)
    partials[:, :2] = torch.rand(partials.shape[0], 2, device=cuda, dtype=torch.float64) * 1e-3
    mirrors_spec = [(1003, 512, 99, 112), (150_001, 30, 235, 240)]  # (begin, rows, cols, ld)
    a = [t.clone() for t in flat]
    b = [t.clone() for t in flat]
    dsts = [torch.full((r, ld), float("nan"), device=cuda) for _, r, _, ld in mirrors_spec]
    mirrors = [(bg, r, c, d) for (bg, r, c, _), d in zip(mirrors_spec, dsts)]
    for step in (1, 2):
        for bufs, mir in ((a, None), (b, mirrors)):
            st = ops.new_device_state(1e-3, cuda)
            ops.adam_step(*bufs, bounds, 1.0, 0.9, 0.999, 1e-8, 1 - 0.9 ** step, (1 - 0.999 ** step) ** 0.5, st, None,
                          prenorm=partials, mirrors=mir)
        for x, y in zip(a, b):
            assert torch.equal(x, y), step
        for (bg, r, c, _), d in zip(mirrors_spec, dsts):
            assert torch.equal(d[:, :c], b[0][bg:bg + r * c].view(r, c)), step
            assert torch.isnan(d[:, c:]).all(), "columns past cols written"


@pytest.mark.parametrize("name", ["adam", "adamw", "sgd", "rmsprop"])
@pytest.mark.parametrize("aligned,prenorm", [(False, False), (True, False), (True, True)])
def test_optim_step_matches_torch(cuda, name, aligned, prenorm):
    """ppo_optim_step against torch's own optimiser of that name with its defaults (rsl_rl/utils/utils.py:71-96;
    upstream passes the learning rate only), after clip_grad_norm_ per group, over learning rates the adaptive
    schedule could set: parameters, state and the clipped gradients to 1e-6.  Adam through ppo_optim_step equals
    ppo_adam_step bit for bit.  With prenorm the group norms come from partial rows summing to the same squares."""
    ops = _ops()
    from tt_rsl_rl_amd import _lib as L

    torch.manual_seed(31)
    shapes_a = [(32,) if aligned else (29,), (256, 96), (256,), (128, 256)]
    shapes_c = [(256, 99), (256,), (1, 128), (4,) if aligned else (1,)]
    pa = [torch.nn.Parameter(torch.randn(s) * 0.1) for s in shapes_a]
    pc = [torch.nn.Parameter(torch.randn(s) * 0.1) for s in shapes_c]
    cls = {"adam": torch.optim.Adam, "adamw": torch.optim.AdamW, "sgd": torch.optim.SGD,
           "rmsprop": torch.optim.RMSprop}[name]
    opt = cls(pa + pc, lr=1e-3)
    d = opt.defaults
    kind = L.OPTIMIZERS[name]
    cfg = L.OptimConfig(kind=kind, beta1=d.get("betas", (0.9, 0.999))[0], beta2=d.get("betas", (0.9, 0.999))[1],
                        eps=d.get("eps", 1e-8), weight_decay=d.get("weight_decay", 0.0), alpha=d.get("alpha", 0.0))
    flat = torch.cat([p.detach().reshape(-1) for p in pa + pc]).to(cuda)
    n_a = sum(p.numel() for p in pa)
    grad = torch.zeros_like(flat)
    s0, s1 = torch.zeros_like(flat), torch.zeros_like(flat)
    twin = [flat.clone(), grad.clone(), s0.clone(), s1.clone()]  # ppo_adam_step on the same inputs (Adam only)
    gb = torch.tensor([0, n_a, flat.numel()], dtype=torch.int64)
    state = ops.new_device_state(1e-3, cuda)
    ws = ops.Workspace(cuda)
    partials = ops.grad_norm_partials(cuda)
    lrs = [1e-3, 6.7e-4, 2e-3, 1e-5, 1e-2, 3e-3]
    for step, lr in enumerate(lrs, start=1):
        scale = 10.0 if step % 3 == 0 else 0.01  # both sides of the clip threshold
        for p in pa + pc:
            p.grad = torch.randn_like(p) * scale
        grad.copy_(torch.cat([p.grad.reshape(-1) for p in pa + pc]).to(cuda))
        twin[1].copy_(grad)
        pre = None
        if prenorm:  # each group's squared norm spread over the partial rows (in halves: exact in fp64)
            g64 = grad.double()
            partials.zero_()
            for g in (0, 1):
                sq = float((g64[gb[g]:gb[g + 1]] ** 2).sum())
                partials[0, g], partials[1, g] = sq / 2, sq - sq / 2
            pre = partials
        for group in opt.param_groups:
            group["lr"] = lr
        torch.nn.utils.clip_grad_norm_(pa, 1.0)
        torch.nn.utils.clip_grad_norm_(pc, 1.0)
        opt.step()
        bc1, bc2 = 1 - 0.9 ** step, (1 - 0.999 ** step) ** 0.5
        ops.reset_device_state(state, lr)
        ops.optim_step(cfg, flat, grad, None if name == "sgd" else s0, s1 if name in ("adam", "adamw") else None, gb,
                       1.0, bc1, bc2, state, ws, prenorm=pre)
        ref = torch.cat([p.detach().reshape(-1) for p in pa + pc])
        assert rel_err(flat, ref) < 1e-6, step
        ref_g = torch.cat([p.grad.reshape(-1) for p in pa + pc])
        assert rel_err(grad, ref_g) < 1e-6, "clipped gradients are left in the gradient buffer like upstream"
        keys = {"adam": ("exp_avg", "exp_avg_sq"), "adamw": ("exp_avg", "exp_avg_sq"), "sgd": (),
                "rmsprop": ("square_avg",)}[name]
        for buf, key in zip((s0, s1), keys):
            assert rel_err(buf, torch.cat([opt.state[p][key].reshape(-1) for p in pa + pc])) < 1e-6, (step, key)
        if name == "sgd":
            assert not any(opt.state[p] for p in pa + pc) and float(s0.abs().sum()) == 0.0
        if name == "adam":
            st = ops.new_device_state(lr, cuda)
            ops.adam_step(*twin, gb, 1.0, 0.9, 0.999, 1e-8, bc1, bc2, st, ws, prenorm=pre)
            for x, y in zip(twin, (flat, grad, s0, s1)):
                assert torch.equal(x, y), step


def test_adam_first_step_moves_by_lr(cuda):
    """tests/algorithms/test_ppo.py:492-505: the first Adam step moves every parameter by lr."""
    ops = _ops()
    p = torch.randn(1000, device=cuda)
    p0 = p.clone()
    g = torch.ones(1000, device=cuda) * 1e-3
    m, v = torch.zeros_like(p), torch.zeros_like(p)
    state = ops.new_device_state(1e-3, cuda)
    ops.adam_step(p, g, m, v, torch.tensor([0, 1000]), 1.0, 0.9, 0.999, 1e-8, 1 - 0.9, (1 - 0.999) ** 0.5, state,
                  ops.Workspace(cuda))
    assert torch.allclose((p0 - p).abs(), torch.full_like(p, 1e-3), atol=1e-6, rtol=0)


# ----------------------------------------------------------------------------------------------------------------------
# A7 normaliser
# ----------------------------------------------------------------------------------------------------------------------


def test_normalizer_update_matches_oracle(cuda):
    ops = _ops()
    torch.manual_seed(2)
    ref = O.EmpiricalNormalization(96 + 3)
    ref.train()
    mean, var, std = torch.zeros(99, device=cuda), torch.ones(99, device=cuda), torch.ones(99, device=cuda)
    count = torch.zeros((), dtype=torch.int64, device=cuda)
    ws = ops.Workspace(cuda)
    for i, rows in enumerate([98304, 4096, 33, 98304]):
        a = torch.randn(rows, 96) * (i + 1) + 3.0
        b = torch.rand(rows, 3) * 2 - 1
        ref.update(torch.cat([a, b], 1))
        ops.normalizer_update([a.to(cuda), b.to(cuda)], mean, var, std, count, ws)
        assert int(count) == int(ref.count)
        assert rel_err(mean, ref._mean.view(-1)) < 1e-6
        assert rel_err(var, ref._var.view(-1)) < 1e-6
        assert rel_err(std, ref._std.view(-1)) < 1e-6


# ----------------------------------------------------------------------------------------------------------------------
# rollout-side Gaussian head
# ----------------------------------------------------------------------------------------------------------------------


def test_gauss_sample_and_log_prob(cuda):
    _ops()
    from tt_rsl_rl_amd.models import GaussianDistribution

    torch.manual_seed(4)
    dist = GaussianDistribution(29, init_std=0.7, std_type="log").to(cuda)
    mean = torch.randn(4096, 29, device=cuda)
    noise = torch.randn(4096, 29, device=cuda)
    actions = torch.empty_like(mean)
    logp = torch.empty(4096, device=cuda)
    std = torch.empty_like(mean)
    dist.sample_from(mean, noise, actions, logp, std)
    sd = torch.exp(dist.log_std_param.detach().cpu())
    assert rel_err(std, sd.expand(4096, 29)) < 1e-7
    k_sd = std.cpu()
    assert torch.equal(k_sd, k_sd[:1].expand(4096, 29)), "the std is state-independent: one value per action"
    ref_a = noise.cpu() * k_sd + mean.cpu()  # torch.normal(mean, std): standard draw * std + mean
    assert torch.equal(actions.cpu(), ref_a)
    ref_lp = torch.distributions.Normal(mean.cpu(), k_sd).log_prob(ref_a).sum(-1)
    assert rel_err(logp, ref_lp) < 1e-6
