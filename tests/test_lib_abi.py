"""The C ABI without a GPU: libppo_hip.so loads, exports every entry point include/ppo_hip.h declares, the ctypes
binding declares exactly those, the struct layouts agree with the C compiler's, and argument validation reports
errors (these calls return before any HIP call, so no GPU is touched)."""

from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "ppo_hip.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|int64_t|size_t|const char\*)\s+(ppo_\w+)\(", text, flags=re.M)))


def test_library_loads_and_exports_every_declared_symbol():
    from tt_rsl_rl_amd import _lib

    lib = _lib.load()
    declared = _declared()
    assert len(declared) >= 19
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in ppo_hip.h but not exported"
    assert sorted(_lib.EXPORTED_SYMBOLS) == declared, "ctypes signatures must cover exactly the header"
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True).stdout
    exported = sorted(set(re.findall(r" T (ppo_\w+)$", out, flags=re.M)))
    assert exported == declared, "the library exports nothing beyond the header"


STRUCTS = {
    "ppo_gather_segment": ("GatherSegment", ["src", "src_stride", "width", "dst_col", "norm_mean", "norm_std",
                                             "norm_eps", "kind"]),
    "ppo_linear_fwd_problem": ("LinearFwdProblem", ["x", "ldx", "w", "b", "z", "ldz", "h", "ldh", "in_features",
                                                    "out_features"]),
    "ppo_linear_bwd_dx_problem": ("LinearBwdDxProblem", ["dz", "lddz", "w", "z_prev", "ldz_prev", "dz_prev",
                                                         "lddz_prev", "in_features", "out_features"]),
    "ppo_linear_bwd_dw_problem": ("LinearBwdDwProblem", ["dz", "lddz", "x", "ldx", "dw", "db", "in_features",
                                                         "out_features", "grad_norm_group", "reserved"]),
    "ppo_grad_range": ("GradRange", ["begin", "end", "group", "reserved"]),
    "ppo_param_mirror": ("ParamMirror", ["begin", "rows", "cols", "dst", "ld_dst"]),
    "ppo_column_block": ("ColumnBlock", ["src", "stride", "width"]),
    "ppo_loss_args": ("LossArgs", ["rows", "num_actions", "std_type", "mean", "ld_mean", "value", "ld_value",
                                   "actions", "old_mean", "old_std", "old_logp", "advantages", "old_values", "returns",
                                   "ld_batch", "std_param", "std_lo", "std_hi", "clip_param", "value_loss_coef",
                                   "entropy_coef", "use_clipped_value_loss", "d_mean", "ld_dmean", "d_value",
                                   "ld_dvalue"]),
    "ppo_policy_head": ("PolicyHead", ["h_actor", "ld_h_actor", "w_actor", "b_actor", "h_critic", "ld_h_critic",
                                       "w_critic", "b_critic", "dz_actor", "ld_dz_actor", "dz_critic", "ld_dz_critic",
                                       "mean", "ld_mean", "value", "ld_value", "k_actor", "k_critic"]),
    "ppo_device_state": ("DeviceState", ["learning_rate", "sum_value_loss", "sum_surrogate_loss", "sum_entropy",
                                         "last_kl_mean", "last_value_loss", "last_surrogate_loss", "last_entropy",
                                         "total_norm", "clip_coef", "num_minibatches"]),
    "ppo_lstm_pack_problem": ("LstmPackProblem", ["w_ih", "w_hh", "b_ih", "b_hh", "w_ih_g", "w_hh_g", "w_hh_gt",
                                                  "b_g", "input_size", "hidden"]),
    "ppo_lstm_seq_problem": ("LstmSeqProblem", ["w_hh_g", "w_hh_gt", "gx", "ldgx", "h0", "c0", "ld0", "keep",
                                                "keep_stride", "h", "ldh", "hs", "c", "gates", "dh", "lddh",
                                                "dgates", "dc", "hidden", "cell"]),
    "ppo_lstm_input_projection": ("LstmInputProjection", ["x", "ldx", "w_ih_g", "b_g", "input_size", "reserved"]),
    "ppo_lstm_grad_problem": ("LstmGradProblem", ["dw_ih_g", "dw_hh_g", "db_g", "dw_ih", "dw_hh", "db_ih", "db_hh",
                                                  "input_size", "hidden"]),
}


# the header's size limits and the Python mirror's copies of them
CONSTANTS = {"PPO_MAX_GATHER_SEGMENTS": "MAX_GATHER_SEGMENTS", "PPO_MAX_INTERLEAVE_FLOATS": "MAX_INTERLEAVE_FLOATS", "PPO_MAX_LINEAR_PROBLEMS": "MAX_LINEAR_PROBLEMS",
             "PPO_MAX_PARAM_GROUPS": "MAX_PARAM_GROUPS", "PPO_DW_NORM_BLOCKS": "DW_NORM_BLOCKS",
             "PPO_MAX_EXTRA_GRADS": "MAX_EXTRA_GRADS", "PPO_ADAM_STATIC_SCRATCH_DOUBLES": "ADAM_STATIC_SCRATCH_DOUBLES",
             "PPO_ADAM_STATIC_MAX_PARAMS": "ADAM_STATIC_MAX_PARAMS", "PPO_MAX_PARAM_MIRRORS": "MAX_PARAM_MIRRORS",
             "PPO_GEMM_BF16_OPERANDS": "GEMM_BF16_OPERANDS"}


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_struct_layouts_match_the_c_compiler(tmp_path):
    from tt_rsl_rl_amd import _lib

    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for cname, (_, fields) in STRUCTS.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for f in fields:
            lines.append(f'  printf("{cname}.{f} %zu\\n", offsetof({cname}, {f}));')
    for macro in CONSTANTS:
        lines.append(f'  printf("{macro} %lld\\n", (long long)({macro}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        k, v = line.rsplit(" ", 1)
        got[k] = int(v)
    for cname, (pyname, fields) in STRUCTS.items():
        cls = getattr(_lib, pyname)
        assert got[f"{cname} size"] == ctypes.sizeof(cls), cname
        for f in fields:
            assert got[f"{cname}.{f}"] == getattr(cls, f).offset, f"{cname}.{f}"
    for macro, pyname in CONSTANTS.items():
        assert got[macro] == getattr(_lib, pyname), macro


def test_argument_validation_reports_errors_without_a_gpu():
    from tt_rsl_rl_amd import _lib

    lib = _lib.load()
    assert lib.ppo_gae(None, None, None, None, None, None, 24, 4096, 0.99, 0.95, None) == _lib.PPO_EINVAL
    assert "null pointer" in _lib.last_error()
    with pytest.raises(ValueError, match="num_steps"):
        _lib.call("ppo_gae", 8, 8, 8, 8, 8, 8, 0, 4096, 0.99, 0.95, None)
    with pytest.raises(ValueError, match="count"):
        _lib.call("ppo_linear_fwd", None, 0, 10, 1, None)
    with pytest.raises(ValueError, match="num_actions"):
        args = _lib.LossArgs(rows=10, num_actions=65)
        _lib.call("ppo_gauss_ppo_loss", ctypes.byref(args), None, 0, None)
    # activations: codes in [0, PPO_ACT_COUNT), and act' from the output only for the monotone ones
    prob = _lib.LinearFwdProblem(x=16, ldx=96, w=16, b=16, z=16, ldz=256, in_features=96, out_features=256)
    with pytest.raises(ValueError, match="activation=13"):
        _lib.call("ppo_linear_fwd", ctypes.byref(prob), 1, 10, 13, None)
    dx = _lib.LinearBwdDxProblem(dz=16, lddz=64, w=16, z_prev=16, ldz_prev=256, dz_prev=16, lddz_prev=256,
                                 in_features=256, out_features=64)
    for name in ("softplus", "gelu", "swish", "mish"):
        with pytest.raises(ValueError, match="needs the activation's input"):
            _lib.call("ppo_linear_bwd_dx_act", ctypes.byref(dx), 1, 10, _lib.ACTIVATIONS[name],
                      _lib.PPO_ELU_FROM_OUTPUT, None, 0, None)
    with pytest.raises(ValueError, match="activation=0"):
        _lib.call("ppo_linear_bwd_dx_act", ctypes.byref(dx), 1, 10, 0, _lib.PPO_ELU_FROM_INPUT, None, 0, None)
    # the GEMM launch flags: PPO_GEMM_BF16_OPERANDS is the only bit, anything else is refused before any launch
    assert _lib.GEMM_BF16_OPERANDS == 1
    for flags in (2, -1, 1 | 8):
        with pytest.raises(ValueError, match=f"flags={flags}"):
            _lib.call("ppo_linear_fwd_ex", ctypes.byref(prob), 1, 10, 1, flags, None)
        with pytest.raises(ValueError, match=f"flags={flags}"):
            _lib.call("ppo_linear_bwd_dx_ex", ctypes.byref(dx), 1, 10, 1, _lib.PPO_ELU_FROM_INPUT, flags, None, 0,
                      None)
    dwp = _lib.LinearBwdDwProblem(8, 512, 8, 96, 8, 8, 96, 512, 0, 0)
    with pytest.raises(ValueError, match="flags=4"):
        _lib.call("ppo_linear_bwd_dw_ex", ctypes.byref(dwp), 1, 24576, 4, 16, 1 << 30, None, None, 0, None, None)
    rng1 = _lib.array(_lib.GradRange, [_lib.GradRange(0, 5, 0, 0)])
    with pytest.raises(ValueError, match="norm_partials"):
        _lib.call("ppo_linear_bwd_dw_ex", ctypes.byref(dwp), 1, 24576, 1, 16, 1 << 30, 16, rng1, 1, None, None)
    assert sorted(_lib.ACTIVATIONS.values()) == list(range(1, 13))
    # workspace queries are pure host arithmetic
    assert lib.ppo_adv_normalize_workspace_bytes(98304) > 0
    assert lib.ppo_loss_workspace_bytes(24576, 29) > 0
    assert lib.ppo_loss_workspace_bytes(24576, 65) == 0
    assert lib.ppo_adam_workspace_bytes(433211) >= 8 * (433211 // 4096)
    # the allocation-free Adam step checks its size against the static scratch before any HIP call
    begin = torch.tensor([0, _lib.ADAM_STATIC_MAX_PARAMS + 1], dtype=torch.int64)
    assert lib.ppo_adam_step_static(16, 16, 16, 16, begin.data_ptr(), 1, 1.0, 0.9, 0.999, 1e-8, 0.1, 0.1, 16,
                                    None) == _lib.PPO_EINVAL
    assert "static scratch" in _lib.last_error()
    assert _lib.ADAM_STATIC_MAX_PARAMS // 1024 + _lib.MAX_PARAM_GROUPS <= _lib.ADAM_STATIC_SCRATCH_DOUBLES
    # LSTM entry points: argument checks run before any launch
    seq = _lib.LstmSeqProblem(hidden=6)
    with pytest.raises(ValueError, match="hidden=6"):
        _lib.call("ppo_lstm_seq_fwd", ctypes.byref(seq), 1, 24, 64, None, 0, None)
    seq = _lib.LstmSeqProblem(hidden=256)
    with pytest.raises(ValueError, match="null pointer"):
        _lib.call("ppo_lstm_seq_bwd", ctypes.byref(seq), 1, 24, 64, None, 0, None)
    with pytest.raises(ValueError, match="count"):
        _lib.call("ppo_lstm_seq_fwd", ctypes.byref(seq), 3, 24, 64, None, 0, None)
    # the one-launch sequences' synchronisation buffer: 32 header words + one 32-word line per 64-row group and problem
    assert lib.ppo_lstm_seq_sync_words(2, 1024) == 32 + 2 * 16 * 32
    assert lib.ppo_lstm_seq_sync_words(1, 65) == 32 + 2 * 32
    assert lib.ppo_lstm_seq_sync_words(3, 64) == -1 and lib.ppo_lstm_seq_sync_words(1, 0) == -1
    full = _lib.LstmSeqProblem(w_hh_g=16, w_hh_gt=16, gx=16, ldgx=1024, h0=16, c0=16, ld0=256, keep=16,
                               keep_stride=1, h=16, ldh=256, hs=16, c=16, gates=16, hidden=256)
    with pytest.raises(ValueError, match="sync buffer"):
        _lib.call("ppo_lstm_seq_fwd", ctypes.byref(full), 1, 24, 1024, 16, 32 + 16 * 32 - 1, None)
    # with the input projection: the projections, a known flag, pointers, input size and leading dimension, all
    # checked before any launch
    with pytest.raises(ValueError, match="projections are required"):
        _lib.call("ppo_lstm_seq_fwd_proj", ctypes.byref(full), None, 1, 24, 1024, 0, None, 0, None)
    proj = _lib.LstmInputProjection(x=16, ldx=48, w_ih_g=16, b_g=16, input_size=48)
    with pytest.raises(ValueError, match="flags=2"):
        _lib.call("ppo_lstm_seq_fwd_proj", ctypes.byref(full), ctypes.byref(proj), 1, 24, 1024, 2, None, 0, None)
    for bad_proj, msg in ((_lib.LstmInputProjection(x=16, ldx=48, w_ih_g=16, b_g=None, input_size=48), "null pointer"),
                          (_lib.LstmInputProjection(x=16, ldx=32, w_ih_g=16, b_g=16, input_size=48),
                           "input_size=48 ldx=32"),
                          (_lib.LstmInputProjection(x=16, ldx=48, w_ih_g=16, b_g=16, input_size=0), "input_size=0")):
        with pytest.raises(ValueError, match=msg):
            _lib.call("ppo_lstm_seq_fwd_proj", ctypes.byref(full), ctypes.byref(bad_proj), 1, 24, 1024, 0, None, 0,
                      None)
    pack = _lib.LstmPackProblem(8, 8, 8, 8, 8, 8, 8, 8, 48, 250)
    with pytest.raises(ValueError, match="sizes"):
        _lib.call("ppo_lstm_pack", ctypes.byref(pack), 1, None)
    with pytest.raises(ValueError, match="ppo_gru_pack: problem 0 sizes"):
        _lib.call("ppo_gru_pack", ctypes.byref(pack), 1, None)
    grad = _lib.LstmGradProblem(8, 8, 8, 8, 8, 8, 8, 48, 6)
    with pytest.raises(ValueError, match="ppo_gru_unpack_grads: problem 0 sizes"):
        _lib.call("ppo_gru_unpack_grads", ctypes.byref(grad), 1, None)
    # the norm-writing unpack: partials, a group per problem in range
    ok_grad = _lib.LstmGradProblem(8, 8, 8, 8, 8, 8, 8, 48, 256)
    grp = (ctypes.c_int32 * 1)(4)
    with pytest.raises(ValueError, match="null norm_partials"):
        _lib.call("ppo_lstm_unpack_grads_norm", ctypes.byref(ok_grad), grp, 1, None, None)
    with pytest.raises(ValueError, match=r"groups\[0\]=4"):
        _lib.call("ppo_lstm_unpack_grads_norm", ctypes.byref(ok_grad), grp, 1, 8, None)
    with pytest.raises(ValueError, match="null groups"):
        _lib.call("ppo_gru_unpack_grads_norm", ctypes.byref(ok_grad), None, 1, 8, None)
    # the optimiser step: a known kind and a config
    cfg = _lib.OptimConfig(kind=7)
    with pytest.raises(ValueError, match="kind=7"):
        _lib.call("ppo_optim_step", 16, 16, 16, 16, None, 1, 1.0, ctypes.byref(cfg), 1.0, 1.0, 16, 16, None, 0, None,
                  0, None)
    with pytest.raises(ValueError, match="null config"):
        _lib.call("ppo_optim_step", 16, 16, 16, 16, None, 1, 1.0, None, 1.0, 1.0, 16, 16, None, 0, None, 0, None)
    # the cell type: LSTM (0) or GRU (1), one type per call
    bad = _lib.LstmSeqProblem(hidden=256, cell=2)
    with pytest.raises(ValueError, match="cell=2"):
        _lib.call("ppo_lstm_seq_fwd", ctypes.byref(bad), 1, 24, 64, None, 0, None)
    mixed = _lib.array(_lib.LstmSeqProblem, [full, _lib.LstmSeqProblem(hidden=256, cell=_lib.CELL_GRU)])
    with pytest.raises(ValueError, match="share the cell type"):
        _lib.call("ppo_lstm_seq_fwd", mixed, 2, 24, 64, None, 0, None)
    probs = _lib.array(_lib.LinearBwdDwProblem, [_lib.LinearBwdDwProblem(8, 512, 8, 96, 8, 8, 96, 512)])
    assert lib.ppo_linear_bwd_dw_workspace_bytes(probs, 1, 24576) >= 4 * 512 * 96
    # column interleave: at most MAX_INTERLEAVE_FLOATS per row, a destination wide enough, 32-bit element count
    wide = _lib.array(_lib.ColumnBlock, [_lib.ColumnBlock(16, 9, 9, 0), _lib.ColumnBlock(16, 8, 8, 0)])
    with pytest.raises(ValueError, match="more than 16"):
        _lib.call("ppo_interleave_columns", wide, 2, 10, 16, 32, None)
    one = _lib.array(_lib.ColumnBlock, [_lib.ColumnBlock(16, 1, 1, 0)])
    with pytest.raises(ValueError, match="dst_stride"):
        _lib.call("ppo_interleave_columns", one, 1, 10, 16, 0, None)
    with pytest.raises(ValueError, match="too many"):
        _lib.call("ppo_interleave_columns", one, 1, 1 << 31, 16, 1, None)
    # the norm-partials variant rejects a group outside [0, PPO_MAX_PARAM_GROUPS] and malformed extra ranges before
    # any launch, and needs its output buffer
    bad = _lib.array(_lib.LinearBwdDwProblem, [_lib.LinearBwdDwProblem(8, 512, 8, 96, 8, 8, 96, 512,
                                                                       _lib.MAX_PARAM_GROUPS + 1, 0)])
    with pytest.raises(ValueError, match="grad_norm_group"):
        _lib.call("ppo_linear_bwd_dw_norm", bad, 1, 24576, 16, 1 << 30, None, None, 0, 16, None)
    rng = _lib.array(_lib.GradRange, [_lib.GradRange(10, 5, 0, 0)])
    with pytest.raises(ValueError, match="extra range 0"):
        _lib.call("ppo_linear_bwd_dw_norm", probs, 1, 24576, 16, 1 << 30, 16, rng, 1, 16, None)
    with pytest.raises(ValueError, match="norm_partials"):
        _lib.call("ppo_linear_bwd_dw_norm", probs, 1, 24576, 16, 1 << 30, None, None, 0, None, None)
    with pytest.raises(ValueError, match="norm_partials"):
        _lib.call("ppo_adam_step_prenorm", 16, 16, 16, 16, None, 1, 1.0, 0.9, 0.999, 1e-8, 0.1, 0.1, 16, None, None)
    # the fused output-layer head: its shape rule, and the rejection of shapes outside it before any pointer is used
    assert lib.ppo_gauss_ppo_head_supported(29, 128, 128) == 1
    assert lib.ppo_gauss_ppo_head_supported(1, 16, 16) == 1
    for shape in ((33, 128, 128), (12, 100, 128), (12, 256, 128), (12, 128, 8), (0, 128, 128)):
        assert lib.ppo_gauss_ppo_head_supported(*shape) == 0, shape
    assert lib.ppo_head_workspace_bytes(24576, 29) == 8 * 384 * 32  # one 16-row tile per wave, 4 waves per block
    args = _lib.LossArgs(rows=10, num_actions=33)
    head = _lib.PolicyHead(k_actor=128, k_critic=128)
    with pytest.raises(ValueError, match="not supported"):
        _lib.call("ppo_gauss_ppo_head", ctypes.byref(args), ctypes.byref(head), None, 0, None, None, 0, 0.0, None,
                  0, None)
    args = _lib.LossArgs(rows=10, num_actions=12)
    with pytest.raises(ValueError, match="null pointer"):
        _lib.call("ppo_gauss_ppo_head", ctypes.byref(args), ctypes.byref(head), None, 0, None, None, 0, 0.0, None,
                  0, None)


@pytest.mark.parametrize("seed, n, pre", [(0, 1, 0), (1, 2, 0), (3, 5, 0), (5, 624, 0), (5, 625, 3), (11, 1249, 700),
                                          (7, 98304, 0), (2, 1572864, 5)])
def test_host_randperm_is_torch_randperm(seed, n, pre):
    """The update's permutation (rsl_rl/storage/rollout_storage.py:232) computed natively equals torch.randperm(n) on
    the CPU generator, and leaves the generator exactly where torch.randperm leaves it (state record and the draws
    that follow), from a freshly seeded generator and from one part-way through its stream with a cached normal."""
    from tt_rsl_rl_amd import ops

    torch.manual_seed(seed)
    if pre:
        torch.rand(pre)
        torch.randn(3)
    start = torch.get_rng_state()
    ref = torch.randperm(n)
    ref_state, ref_next = torch.get_rng_state(), torch.rand(4)
    torch.set_rng_state(start)
    got = ops.host_randperm(n)
    assert torch.equal(got, ref)
    assert torch.equal(torch.get_rng_state(), ref_state)
    assert torch.equal(torch.rand(4), ref_next)


@pytest.mark.parametrize("first_on_worker", [False, True], ids=["first_here", "first_on_worker"])
@pytest.mark.parametrize("n, split", [(98304, 24576), (1000, 0), (1000, 999), (1000, 5000), (2, 1), (1, 0),
                                      (1572864, 393216)])
def test_split_randperm_is_torch_randperm(n, split, first_on_worker):
    """The permutation drawn in two pieces (the first mini-batch's positions, on the calling thread or ahead of the
    rest on the worker thread, then the rest on the worker) equals torch.randperm(n) and leaves the generator where
    torch.randperm leaves it; positions [0, split) are final after the first piece."""
    from tt_rsl_rl_amd import ops

    torch.manual_seed(n + split)
    torch.rand(3)
    start = torch.get_rng_state()
    ref = torch.randperm(n)
    ref_state, ref_next = torch.get_rng_state(), torch.rand(4)
    torch.set_rng_state(start)
    out = torch.empty(n, dtype=torch.int64)
    sh = ops.SplitRandperm(n, out, split, first_on_worker=first_on_worker)
    sh.wait_first()
    k = sh.split
    assert torch.equal(out[:k], ref[:k]), "the first piece's positions must be final"
    got = sh.join()
    assert torch.equal(got, ref)
    assert torch.equal(torch.get_rng_state(), ref_state)
    assert torch.equal(torch.rand(4), ref_next)
    sh.join()  # idempotent


@pytest.mark.parametrize("first_on_worker", [False, True], ids=["first_here", "first_on_worker"])
def test_split_randperm_falls_back_to_torch_on_an_unknown_generator_record(monkeypatch, first_on_worker):
    """A generator record this library does not read (here: one byte longer) leaves the whole draw to torch itself:
    the permutation and the samples after it are torch's, from the same generator state."""
    from tt_rsl_rl_amd import ops

    n, split, normals = 5000, 1000, [7, 40]
    torch.manual_seed(3)
    start = torch.get_rng_state()
    ref = torch.randperm(n)
    for k in normals:
        torch.randn(k)
    ref_state = torch.get_rng_state()
    torch.set_rng_state(start)
    real = torch.get_rng_state
    monkeypatch.setattr(torch, "get_rng_state", lambda: torch.cat([real(), torch.zeros(1, dtype=torch.uint8)]))
    out = torch.empty(n, dtype=torch.int64)
    sh = ops.SplitRandperm(n, out, split, normals, first_on_worker=first_on_worker)
    sh.wait_first()
    assert sh.split == n
    assert torch.equal(sh.join(), ref)
    monkeypatch.undo()
    assert torch.equal(torch.get_rng_state(), ref_state)


def test_split_randperm_calls_on_rest_once_the_rest_is_final():
    """on_rest(self) runs on the worker thread after the second piece, with out[split:] already final (the update
    enqueues that piece's host-to-device copy from it); perm_ready() returns only after it; the permutation and the
    generator state stay torch.randperm's."""
    import threading

    from tt_rsl_rl_amd import ops

    n, split = 98304, 24576
    torch.manual_seed(11)
    start = torch.get_rng_state()
    ref = torch.randperm(n)
    ref_state = torch.get_rng_state()
    torch.set_rng_state(start)
    out = torch.empty(n, dtype=torch.int64)
    seen = {}

    def on_rest(sp):
        seen["thread"] = threading.get_ident()
        seen["split"] = sp.split
        seen["tail"] = sp.out[sp.split:].clone()

    sh = ops.SplitRandperm(n, out, split, on_rest=on_rest)
    sh.perm_ready()
    assert seen["split"] == split and seen["thread"] != threading.get_ident()
    assert torch.equal(seen["tail"], ref[split:])
    assert torch.equal(sh.join(), ref)
    assert torch.equal(torch.get_rng_state(), ref_state)


def test_host_randperm_range_validation():
    from tt_rsl_rl_amd import _lib

    lib = _lib.load()
    rec = bytearray(torch.get_rng_state().numpy().tobytes())
    buf = (ctypes.c_uint8 * len(rec)).from_buffer(rec)
    out = (ctypes.c_int64 * 10)()
    assert lib.ppo_host_randperm_range(buf, len(rec), 10, 3, 2, out) == _lib.PPO_EINVAL
    assert lib.ppo_host_randperm_range(buf, len(rec), 10, 0, 10, out) == _lib.PPO_EINVAL
    assert "outside" in _lib.last_error()
    assert lib.ppo_host_randperm_range(buf, len(rec), 10, 0, 9, out) == _lib.PPO_OK


def test_host_randperm_rejects_unknown_generator_records():
    from tt_rsl_rl_amd import _lib

    lib = _lib.load()
    rec = (ctypes.c_uint8 * 5056)()  # all zero: `seeded` is 0
    out = (ctypes.c_int64 * 4)()
    assert lib.ppo_host_randperm(rec, 5056, 4, out) == _lib.PPO_EINVAL
    assert "not recognised" in _lib.last_error()
    assert lib.ppo_host_randperm(rec, 5000, 4, out) == _lib.PPO_EINVAL


def test_sequence_wait_limit_is_set_only_through_its_entry_point(monkeypatch):
    """The whole-sequence LSTM launches' wait limit: 2 s of the 100 MHz clock by default, changed only by
    ppo_lstm_seq_wait_limit (no environment variable), which returns the limit it replaces; a negative value restores
    the default."""
    from tt_rsl_rl_amd import _lib

    lib = _lib.load()
    monkeypatch.setenv("PPO_HIP_SEQ_SPIN_TICKS", "0")  # a stray variable of an older build changes nothing
    assert lib.ppo_lstm_seq_wait_limit(-1) == 200_000_000
    assert lib.ppo_lstm_seq_wait_limit(0) == 200_000_000
    assert lib.ppo_lstm_seq_wait_limit(12345) == 0
    assert lib.ppo_lstm_seq_wait_limit(-7) == 12345
    assert lib.ppo_lstm_seq_wait_limit(-1) == 200_000_000
