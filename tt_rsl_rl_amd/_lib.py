"""ctypes binding of libppo_hip.so (the C ABI declared in include/ppo_hip.h).

The product path calls these entry points only; there is no CPU fallback.  Loading fails loudly when the library
is missing (build it with ``python -m tt_rsl_rl_amd.build``).  Status codes become Python exceptions the way
upstream rsl_rl raises them: bad arguments -> ValueError, unsupported shapes -> NotImplementedError, HIP runtime
failures -> RuntimeError.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

# PPO_HIP_LIB names another build of the same library (the host-sanitizer build of sanitize_host.py)
LIB_PATH = Path(os.environ.get("PPO_HIP_LIB") or Path(__file__).resolve().parent / "libppo_hip.so")

PPO_OK = 0
PPO_EINVAL = -1
PPO_EHIP = -2
PPO_EUNSUPPORTED = -3
PPO_ACT_NONE = 0
PPO_ACT_ELU = 1
# rsl_rl's activation names (rsl_rl/utils/utils.py:34-68) -> the library's codes
ACTIVATIONS = {"elu": 1, "selu": 2, "relu": 3, "crelu": 4, "lrelu": 5, "tanh": 6, "sigmoid": 7, "softplus": 8,
               "gelu": 9, "swish": 10, "mish": 11, "identity": 12}
# activations whose derivative the input-grad can take from the activation's output (the rest need its input)
ACT_FROM_OUTPUT = {1, 2, 3, 4, 5, 6, 7, 12}
PPO_ELU_FROM_INPUT = 0
PPO_ELU_FROM_OUTPUT = 1
PPO_STD_SCALAR = 0
PPO_STD_LOG = 1
MAX_GATHER_SEGMENTS = 16
MAX_INTERLEAVE_FLOATS = 16
MAX_LINEAR_PROBLEMS = 12
MAX_PARAM_GROUPS = 4
MAX_PARAM_MIRRORS = 2
MAX_ACTIONS = 64
DW_NORM_BLOCKS = 512
MAX_EXTRA_GRADS = 4
ADAM_STATIC_SCRATCH_DOUBLES = 8192
ADAM_STATIC_MAX_PARAMS = (ADAM_STATIC_SCRATCH_DOUBLES - MAX_PARAM_GROUPS) * 1024

f32p = C.c_void_p  # device pointers are passed as plain addresses
i64 = C.c_int64
i32 = C.c_int32


PPO_GATHER_FLOAT = 0
PPO_GATHER_KEEP_U8 = 1


class GatherSegment(C.Structure):
    _fields_ = [("src", C.c_void_p), ("src_stride", i64), ("width", i32), ("dst_col", i32),
                ("norm_mean", C.c_void_p), ("norm_std", C.c_void_p), ("norm_eps", C.c_float), ("kind", i32)]


class LinearFwdProblem(C.Structure):
    _fields_ = [("x", C.c_void_p), ("ldx", i64), ("w", C.c_void_p), ("b", C.c_void_p), ("z", C.c_void_p),
                ("ldz", i64), ("h", C.c_void_p), ("ldh", i64), ("in_features", i32), ("out_features", i32)]


class LinearBwdDxProblem(C.Structure):
    _fields_ = [("dz", C.c_void_p), ("lddz", i64), ("w", C.c_void_p), ("z_prev", C.c_void_p), ("ldz_prev", i64),
                ("dz_prev", C.c_void_p), ("lddz_prev", i64), ("in_features", i32), ("out_features", i32)]


class LinearBwdDwProblem(C.Structure):
    _fields_ = [("dz", C.c_void_p), ("lddz", i64), ("x", C.c_void_p), ("ldx", i64), ("dw", C.c_void_p),
                ("db", C.c_void_p), ("in_features", i32), ("out_features", i32), ("grad_norm_group", i32),
                ("reserved", i32)]


class GradRange(C.Structure):
    _fields_ = [("begin", i64), ("end", i64), ("group", i32), ("reserved", i32)]


class ParamMirror(C.Structure):
    _fields_ = [("begin", i64), ("rows", i32), ("cols", i32), ("dst", C.c_void_p), ("ld_dst", i64)]


class OptimConfig(C.Structure):
    _fields_ = [("kind", i32), ("reserved", i32), ("beta1", C.c_double), ("beta2", C.c_double), ("eps", C.c_double),
                ("weight_decay", C.c_double), ("alpha", C.c_double)]


OPTIM_ADAM, OPTIM_ADAMW, OPTIM_SGD, OPTIM_RMSPROP = 0, 1, 2, 3
GEMM_BF16_OPERANDS = 1
OPTIMIZERS = {"adam": OPTIM_ADAM, "adamw": OPTIM_ADAMW, "sgd": OPTIM_SGD, "rmsprop": OPTIM_RMSPROP}


class ColumnBlock(C.Structure):
    _fields_ = [("src", C.c_void_p), ("stride", i64), ("width", i32), ("reserved", i32)]


class LossArgs(C.Structure):
    _fields_ = [
        ("rows", i64), ("num_actions", i32), ("std_type", i32),
        ("mean", C.c_void_p), ("ld_mean", i64),
        ("value", C.c_void_p), ("ld_value", i64),
        ("actions", C.c_void_p), ("old_mean", C.c_void_p), ("old_std", C.c_void_p), ("old_logp", C.c_void_p),
        ("advantages", C.c_void_p), ("old_values", C.c_void_p), ("returns", C.c_void_p), ("ld_batch", i64),
        ("std_param", C.c_void_p), ("std_lo", C.c_double), ("std_hi", C.c_double),
        ("clip_param", C.c_double), ("value_loss_coef", C.c_double), ("entropy_coef", C.c_double),
        ("use_clipped_value_loss", i32), ("reserved", i32),
        ("d_mean", C.c_void_p), ("ld_dmean", i64),
        ("d_value", C.c_void_p), ("ld_dvalue", i64),
    ]


class PolicyHead(C.Structure):
    _fields_ = [("h_actor", C.c_void_p), ("ld_h_actor", i64), ("w_actor", C.c_void_p), ("b_actor", C.c_void_p),
                ("h_critic", C.c_void_p), ("ld_h_critic", i64), ("w_critic", C.c_void_p), ("b_critic", C.c_void_p),
                ("dz_actor", C.c_void_p), ("ld_dz_actor", i64), ("dz_critic", C.c_void_p), ("ld_dz_critic", i64),
                ("mean", C.c_void_p), ("ld_mean", i64), ("value", C.c_void_p), ("ld_value", i64),
                ("k_actor", i32), ("k_critic", i32)]


class DeviceState(C.Structure):
    _fields_ = [("learning_rate", C.c_double), ("sum_value_loss", C.c_double),
                ("sum_surrogate_loss", C.c_double), ("sum_entropy", C.c_double),
                ("last_kl_mean", C.c_float), ("last_value_loss", C.c_float), ("last_surrogate_loss", C.c_float),
                ("last_entropy", C.c_float), ("total_norm", C.c_float * 4), ("clip_coef", C.c_float * 4),
                ("num_minibatches", i32), ("reserved", i32 * 3)]


DEVICE_STATE_BYTES = C.sizeof(DeviceState)
MAX_LSTM_PROBLEMS = 2
CELL_LSTM, CELL_GRU = 0, 1
vp = C.c_void_p


class LstmPackProblem(C.Structure):
    _fields_ = [("w_ih", vp), ("w_hh", vp), ("b_ih", vp), ("b_hh", vp), ("w_ih_g", vp), ("w_hh_g", vp),
                ("w_hh_gt", vp), ("b_g", vp), ("input_size", i32), ("hidden", i32)]


class LstmSeqProblem(C.Structure):
    _fields_ = [("w_hh_g", vp), ("w_hh_gt", vp), ("gx", vp), ("ldgx", i64), ("h0", vp), ("c0", vp), ("ld0", i64),
                ("keep", vp), ("keep_stride", i64), ("h", vp), ("ldh", i64), ("hs", vp), ("c", vp), ("gates", vp),
                ("dh", vp), ("lddh", i64), ("dgates", vp), ("dc", vp), ("hidden", i32), ("cell", i32)]


class LstmInputProjection(C.Structure):
    _fields_ = [("x", vp), ("ldx", i64), ("w_ih_g", vp), ("b_g", vp), ("input_size", i32), ("reserved", i32)]


class LstmGradProblem(C.Structure):
    _fields_ = [("dw_ih_g", vp), ("dw_hh_g", vp), ("db_g", vp), ("dw_ih", vp), ("dw_hh", vp), ("db_ih", vp),
                ("db_hh", vp), ("input_size", i32), ("hidden", i32)]

# (name, restype, argtypes)
_SIGNATURES = [
    ("ppo_last_error", C.c_char_p, []),
    ("ppo_abi_version", C.c_int, []),
    ("ppo_gae", C.c_int, [f32p, f32p, f32p, f32p, f32p, f32p, i64, i64, C.c_float, C.c_float, C.c_void_p]),
    ("ppo_adv_normalize_workspace_bytes", C.c_size_t, [i64]),
    ("ppo_adv_normalize", C.c_int, [f32p, i64, f32p, i64, i64, C.c_float, C.c_void_p, C.c_size_t, C.c_void_p]),
    ("ppo_gather_rows", C.c_int, [C.c_void_p, i64, i64, C.POINTER(GatherSegment), i32, f32p, i64, C.c_void_p]),
    ("ppo_linear_fwd", C.c_int, [C.POINTER(LinearFwdProblem), i32, i64, i32, C.c_void_p]),
    ("ppo_lstm_pack", C.c_int, [C.POINTER(LstmPackProblem), i32, C.c_void_p]),
    ("ppo_gru_pack", C.c_int, [C.POINTER(LstmPackProblem), i32, C.c_void_p]),
    ("ppo_lstm_seq_sync_words", i64, [i32, i64]),
    ("ppo_lstm_seq_wait_limit", i64, [i64]),
    ("ppo_lstm_seq_fwd", C.c_int, [C.POINTER(LstmSeqProblem), i32, i64, i64, C.c_void_p, i64, C.c_void_p]),
    ("ppo_lstm_seq_bwd", C.c_int, [C.POINTER(LstmSeqProblem), i32, i64, i64, C.c_void_p, i64, C.c_void_p]),
    ("ppo_lstm_seq_fwd_proj", C.c_int, [C.POINTER(LstmSeqProblem), C.POINTER(LstmInputProjection), i32, i64, i64, i32,
                                        C.c_void_p, i64, C.c_void_p]),
    ("ppo_lstm_unpack_grads", C.c_int, [C.POINTER(LstmGradProblem), i32, C.c_void_p]),
    ("ppo_gru_unpack_grads", C.c_int, [C.POINTER(LstmGradProblem), i32, C.c_void_p]),
    ("ppo_lstm_unpack_grads_norm", C.c_int, [C.POINTER(LstmGradProblem), C.POINTER(i32), i32, C.c_void_p,
                                             C.c_void_p]),
    ("ppo_gru_unpack_grads_norm", C.c_int, [C.POINTER(LstmGradProblem), C.POINTER(i32), i32, C.c_void_p,
                                            C.c_void_p]),
    ("ppo_linear_bwd_dx_workspace_bytes", C.c_size_t, [C.POINTER(LinearBwdDxProblem), i32]),
    ("ppo_linear_bwd_dx", C.c_int, [C.POINTER(LinearBwdDxProblem), i32, i64, i32, C.c_void_p, C.c_size_t,
                                    C.c_void_p]),
    ("ppo_linear_bwd_dx_act", C.c_int, [C.POINTER(LinearBwdDxProblem), i32, i64, i32, i32, C.c_void_p, C.c_size_t,
                                    C.c_void_p]),
    ("ppo_linear_bwd_dw_workspace_bytes", C.c_size_t, [C.POINTER(LinearBwdDwProblem), i32, i64]),
    ("ppo_linear_bwd_dw", C.c_int, [C.POINTER(LinearBwdDwProblem), i32, i64, C.c_void_p, C.c_size_t, C.c_void_p]),
    ("ppo_interleave_columns", C.c_int, [C.POINTER(ColumnBlock), i32, i64, f32p, i64, C.c_void_p]),
    ("ppo_linear_bwd_dw_norm", C.c_int, [C.POINTER(LinearBwdDwProblem), i32, i64, C.c_void_p, C.c_size_t, f32p,
                                         C.POINTER(GradRange), i32, C.c_void_p, C.c_void_p]),
    ("ppo_linear_fwd_ex", C.c_int, [C.POINTER(LinearFwdProblem), i32, i64, i32, i32, C.c_void_p]),
    ("ppo_linear_bwd_dx_ex", C.c_int, [C.POINTER(LinearBwdDxProblem), i32, i64, i32, i32, i32, C.c_void_p,
                                       C.c_size_t, C.c_void_p]),
    ("ppo_linear_bwd_dw_ex", C.c_int, [C.POINTER(LinearBwdDwProblem), i32, i64, i32, C.c_void_p, C.c_size_t, f32p,
                                       C.POINTER(GradRange), i32, C.c_void_p, C.c_void_p]),
    ("ppo_obs_normalize", C.c_int, [f32p, i64, f32p, i64, i64, i32, f32p, f32p, C.c_float, C.c_void_p]),
    ("ppo_normalizer_update_workspace_bytes", C.c_size_t, [i64, i32]),
    ("ppo_normalizer_update", C.c_int, [C.POINTER(ColumnBlock), i32, i64, f32p, f32p, f32p, C.c_void_p, C.c_void_p,
                                        C.c_size_t, C.c_void_p]),
    ("ppo_loss_workspace_bytes", C.c_size_t, [i64, i32]),
    ("ppo_gauss_ppo_loss", C.c_int, [C.POINTER(LossArgs), C.c_void_p, C.c_size_t, C.c_void_p]),
    ("ppo_loss_finalize", C.c_int, [C.POINTER(LossArgs), C.c_void_p, C.c_size_t, f32p, C.c_void_p, i32, C.c_double,
                                    C.c_void_p, i32, C.c_void_p]),
    ("ppo_gauss_ppo_head_supported", C.c_int, [i32, i32, i32]),
    ("ppo_head_workspace_bytes", C.c_size_t, [i64, i32]),
    ("ppo_gauss_ppo_head", C.c_int, [C.POINTER(LossArgs), C.POINTER(PolicyHead), C.c_void_p, C.c_size_t, f32p,
                                     C.c_void_p, i32, C.c_double, C.c_void_p, i32, C.c_void_p]),
    ("ppo_gauss_sample", C.c_int, [f32p, i64, f32p, i32, C.c_double, C.c_double, f32p, i64, f32p, i64, f32p, f32p,
                                   i64, i64, i32, C.c_void_p]),
    ("ppo_host_randperm", C.c_int, [C.c_void_p, C.c_size_t, i64, C.c_void_p]),
    ("ppo_host_randperm_range", C.c_int, [C.c_void_p, C.c_size_t, i64, i64, i64, C.c_void_p]),
    ("ppo_host_rng_skip", C.c_int, [C.c_void_p, C.c_size_t, i64]),
    ("ppo_adam_workspace_bytes", C.c_size_t, [i64]),
    ("ppo_adam_step", C.c_int, [f32p, f32p, f32p, f32p, C.c_void_p, i32, C.c_double, C.c_double, C.c_double,
                                C.c_double, C.c_double, C.c_double, C.c_void_p, C.c_void_p, C.c_size_t,
                                C.c_void_p]),
    ("ppo_adam_step_static", C.c_int, [f32p, f32p, f32p, f32p, C.c_void_p, i32, C.c_double, C.c_double,
                                       C.c_double, C.c_double, C.c_double, C.c_double, C.c_void_p, C.c_void_p]),
    ("ppo_adam_step_prenorm", C.c_int, [f32p, f32p, f32p, f32p, C.c_void_p, i32, C.c_double, C.c_double,
                                        C.c_double, C.c_double, C.c_double, C.c_double, C.c_void_p, C.c_void_p,
                                        C.c_void_p]),
    ("ppo_adam_step_prenorm_mirror", C.c_int, [f32p, f32p, f32p, f32p, C.c_void_p, i32, C.c_double, C.c_double,
                                               C.c_double, C.c_double, C.c_double, C.c_double, C.c_void_p, C.c_void_p,
                                               C.c_void_p, i32, C.c_void_p]),
    ("ppo_optim_step", C.c_int, [f32p, f32p, f32p, f32p, C.c_void_p, i32, C.c_double, C.POINTER(OptimConfig),
                                 C.c_double, C.c_double, C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p,
                                 i32, C.c_void_p]),
]

EXPORTED_SYMBOLS = [name for name, _, _ in _SIGNATURES]
ABI_VERSION = 8

_lib: C.CDLL | None = None


def load(path: str | os.PathLike | None = None) -> C.CDLL:
    """Load libppo_hip.so (idempotent) and declare every entry point's signature."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"{p} is missing: build the HIP library first (python -m tt_rsl_rl_amd.build)")
    lib = C.CDLL(str(p))
    for name, res, args in _SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.ppo_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{p}: ABI version {lib.ppo_abi_version()} != {ABI_VERSION}; rebuild the library")
    if path is None:
        _lib = lib
    return lib


def last_error() -> str:
    return load().ppo_last_error().decode(errors="replace")


def check(status: int, what: str) -> None:
    if status == PPO_OK:
        return
    msg = f"{what}: {last_error()}"
    if status == PPO_EINVAL:
        raise ValueError(msg)
    if status == PPO_EUNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


# When set (a list), every call() is appended to it as (name, args) before it runs: a launch sequence recorded this
# way can be issued again later with the same arguments (the ctypes objects in args stay referenced by the list).
recorder: list | None = None


def call(name: str, *args) -> None:
    """Call an int-returning entry point and raise on a non-zero status."""
    if recorder is not None:
        recorder.append((name, args))
    check(getattr(load(), name)(*args), name)


def array(struct_type, items):
    arr = (struct_type * max(1, len(items)))()
    for i, it in enumerate(items):
        arr[i] = it
    return arr
