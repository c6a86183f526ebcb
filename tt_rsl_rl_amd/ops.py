"""Tensor-level wrappers over the C ABI of libppo_hip.so.

Each function validates its torch tensors (device, dtype, shape, strides), then calls the matching C entry point
with raw device pointers and the current HIP stream.  Device memory and streams come from PyTorch; every
arithmetic operation happens in the HIP kernels.  Nothing here falls back to torch or the CPU: tensors that are not
on a GPU are rejected.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib as L


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _dev(*tensors: torch.Tensor | None, dtype=torch.float32) -> None:
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("tt_rsl_rl_amd ops take GPU tensors only (no CPU path exists)")
        if dtype is not None and t.dtype != dtype:
            raise ValueError(f"expected {dtype}, got {t.dtype}")


def _row_major(t: torch.Tensor, name: str) -> int:
    """Leading dimension (floats) of a 2-D row-major view with unit column stride."""
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D view with unit column stride, got shape {tuple(t.shape)} "
                         f"strides {t.stride()}")
    return max(t.stride(0), t.shape[1])


class Workspace:
    """Grow-only device scratch buffer (one per consumer), so steady-state calls allocate nothing."""

    def __init__(self, device: torch.device | str | None = None) -> None:
        self.device = device
        self.buf: torch.Tensor | None = None

    def get(self, nbytes: int) -> torch.Tensor:
        nbytes = max(int(nbytes), 256)
        if self.buf is None or self.buf.numel() < nbytes:
            self.buf = torch.empty(nbytes, dtype=torch.uint8, device=self.device or "cuda")
        return self.buf


# ----------------------------------------------------------------------------------------------------------------------
# A1 / A2
# ----------------------------------------------------------------------------------------------------------------------


def gae(rewards, values, dones, last_values, returns, advantages, gamma: float, lam: float) -> None:
    """rewards/values/returns/advantages: [T, N] (or [T, N, 1]) contiguous fp32; dones uint8 same shape."""
    _dev(rewards, values, last_values, returns, advantages)
    _dev(dones, dtype=torch.uint8)
    T, N = rewards.shape[0], rewards.shape[1]
    for t in (rewards, values, returns, advantages, dones):
        if t.numel() != T * N or not t.is_contiguous():
            raise ValueError("gae: every [T, N] input must be contiguous with T*N elements")
    if last_values.numel() != N or not last_values.is_contiguous():
        raise ValueError("gae: last_values must hold N contiguous values")
    L.call("ppo_gae", _ptr(rewards), _ptr(values), _ptr(dones), _ptr(last_values), _ptr(returns), _ptr(advantages),
           T, N, float(gamma), float(lam), _stream())


def adv_normalize(x: torch.Tensor, out: torch.Tensor, n: int, in_stride: int = 1, out_stride: int = 1,
                  eps: float = 1e-8, ws: Workspace | None = None) -> None:
    _dev(x, out)
    lib = L.load()
    nbytes = lib.ppo_adv_normalize_workspace_bytes(n)
    buf = (ws or Workspace(x.device)).get(nbytes)
    L.call("ppo_adv_normalize", _ptr(x), in_stride, _ptr(out), out_stride, n, float(eps), buf.data_ptr(), buf.numel(),
           _stream())


# ----------------------------------------------------------------------------------------------------------------------
# A5 / A7 forward
# ----------------------------------------------------------------------------------------------------------------------


@dataclass
class Segment:
    src: torch.Tensor          # [src_rows, >= width] row-major view (float32; uint8 done flags for keep)
    dst_col: int
    norm_mean: torch.Tensor | None = None
    norm_std: torch.Tensor | None = None
    norm_eps: float = 0.0
    keep: bool = False         # src holds uint8 done flags d, written as 1 - d


def host_randperm(n: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """``torch.randperm(n)`` drawn from torch's CPU generator -- the same permutation, and the generator left in the
    same state -- computed by libppo_hip.so's native Fisher-Yates (rsl_rl/storage/rollout_storage.py:232).  ``out``:
    an int64 CPU tensor of n elements (e.g. pinned, for an asynchronous copy to the device).  A generator record of
    an unexpected layout is left to torch.randperm itself."""
    import ctypes

    if out is None:
        out = torch.empty(n, dtype=torch.int64)
    if out.dtype != torch.int64 or out.device.type != "cpu" or out.numel() != n or not out.is_contiguous():
        raise ValueError("host_randperm: out must be a contiguous int64 CPU tensor of n elements")
    rec = bytearray(torch.get_rng_state().numpy().tobytes())
    buf = (ctypes.c_uint8 * len(rec)).from_buffer(rec)
    if L.load().ppo_host_randperm(buf, len(rec), n, out.data_ptr()) != L.PPO_OK:
        out.copy_(torch.randperm(n))
        return out
    torch.set_rng_state(torch.frombuffer(rec, dtype=torch.uint8).clone())
    return out


def normal_draws(n: int) -> int | None:
    """32-bit draws torch's CPU generator gives a float ``normal_`` of n contiguous elements (what ``torch.normal`` /
    ``Normal.sample()`` take on the CPU): n >= 16 fills n uniforms and, when n % 16 != 0, redraws the last 16.  None
    below 16 elements, which go through another path (pairs of 64-bit draws with a cached sample)."""
    if n < 16:
        return None
    return n + (16 if n % 16 else 0)


class SplitRandperm:
    """Upstream's CPU-generator draws during one update, in upstream's order, computed natively.

    ``torch.randperm(n)`` (rsl_rl/storage/rollout_storage.py:232) in two pieces: iterations [0, split) of the shuffle
    now, which makes positions [0, split) final, and iterations [split, n - 1) on a worker thread (the native call
    runs without the GIL) while the caller launches work on the first rows.  Then, on the same thread, the samples
    upstream's stochastic forward draws and discards in every mini-batch (``normals``: element counts, in order;
    rsl_rl/models/mlp_model.py:103-106): skipped natively (``ppo_host_rng_skip``), or drawn with torch below 16
    elements.  n = 0: no permutation (the recurrent update).  ``join()`` waits and writes the generator state back;
    between ``__init__`` and ``join()`` nothing else may draw from the CPU generator.  The permutation and the final
    generator state are bit-identical to torch's.  A generator record of an unexpected layout falls back to torch
    itself.  ``first_on_worker``: iterations [0, split) run on the worker too, ahead of the rest, so the caller can do
    other work first; ``wait_first()`` then waits until positions [0, split) are final (and ``split`` is n after a
    fallback to torch)."""

    _pool = None

    def __init__(self, n: int, out: torch.Tensor | None, split: int, normals: list[int] | tuple = (),
                 on_rest=None, first_on_worker: bool = False) -> None:
        import ctypes

        if n > 0 and (out is None or out.dtype != torch.int64 or out.device.type != "cpu" or out.numel() != n
                      or not out.is_contiguous()):
            raise ValueError("SplitRandperm: out must be a contiguous int64 CPU tensor of n elements")
        self.n, self.out, self.normals = n, out, list(normals)
        self.on_rest = on_rest  # on_rest(self), on the worker once out[split:] is final (e.g. to enqueue its copy)
        self.split = max(0, min(int(split), n - 1)) if n > 0 else 0
        self._rec = bytearray(torch.get_rng_state().numpy().tobytes())
        self._buf = (ctypes.c_uint8 * len(self._rec)).from_buffer(self._rec)
        self._perm_future = self._future = self._first_future = None
        self._first_error = None  # (first_on_worker) the first range's error: the record is not one this library reads
        if n > 0 and first_on_worker:
            pool = self._worker()
            self._first_future = pool.submit(self._perm_first)
            if self.split < n - 1:
                self._perm_future = pool.submit(self._perm_rest)
            if self.normals:
                self._future = pool.submit(self._skips)
            return
        lib = L.load()
        if n > 0 and lib.ppo_host_randperm_range(self._buf, len(self._rec), n, 0, self.split,
                                                 out.data_ptr()) != L.PPO_OK:
            self._torch_fallback()
            return
        if (n > 0 and self.split < n - 1) or self.normals:
            pool = self._worker()
            # one worker: the skips run after the permutation's rest, in stream order
            if n > 0 and self.split < n - 1:
                self._perm_future = pool.submit(self._perm_rest)
            if self.normals:
                self._future = pool.submit(self._skips)

    @staticmethod
    def _worker():
        if SplitRandperm._pool is None:
            from concurrent.futures import ThreadPoolExecutor

            SplitRandperm._pool = ThreadPoolExecutor(max_workers=1, thread_name_prefix="ppo-host-rng")
        return SplitRandperm._pool

    def _torch_fallback(self) -> None:
        """torch itself draws the permutation and the samples (a generator record this library does not read)."""
        self.out.copy_(torch.randperm(self.n))
        for k in self.normals:
            torch.randn(k)
        self._rec = None
        self.split = self.n

    def _perm_first(self) -> None:
        if L.load().ppo_host_randperm_range(self._buf, len(self._rec), self.n, 0, self.split,
                                            self.out.data_ptr()) != L.PPO_OK:
            self._first_error = L.last_error()

    def wait_first(self) -> None:
        """(first_on_worker) Wait until positions [0, split) of the permutation are final."""
        if self._first_future is None:
            return
        self._first_future.result()
        self._first_future = None
        if self._first_error is not None:  # the queued rest and skips returned at once: torch draws everything
            for f in (self._perm_future, self._future):
                if f is not None:
                    f.result()
            self._perm_future = self._future = None
            self._torch_fallback()

    def _perm_rest(self) -> str | None:
        if self._first_error is not None:
            return None
        rc = L.load().ppo_host_randperm_range(self._buf, len(self._rec), self.n, self.split, self.n - 1,
                                              self.out.data_ptr())
        if rc != L.PPO_OK:
            return L.last_error()  # the error text is thread-local: read it here
        if self.on_rest is not None:
            self.on_rest(self)
        return None

    def _skips(self) -> str | None:
        import ctypes

        lib = L.load()
        if self._first_error is not None:
            return None  # (wait_first() hands everything to torch)
        if self._perm_future is not None and self._perm_future.result() is not None:
            return None  # the permutation failed: reported by join()
        pending = 0
        for k in self.normals:
            d = normal_draws(k)
            if d is not None:
                pending += d
                continue
            if pending and lib.ppo_host_rng_skip(self._buf, len(self._rec), pending) != L.PPO_OK:
                return L.last_error()
            pending = 0
            # a sample below 16 elements: drawn by torch on the record (nothing else uses the generator meanwhile)
            torch.set_rng_state(torch.frombuffer(self._rec, dtype=torch.uint8).clone())
            torch.randn(k)
            ctypes.memmove(self._buf, torch.get_rng_state().numpy().tobytes(), len(self._rec))
        if pending and lib.ppo_host_rng_skip(self._buf, len(self._rec), pending) != L.PPO_OK:
            return L.last_error()
        return None

    def perm_ready(self) -> torch.Tensor | None:
        """Wait for the permutation only (the skips may still run); the generator state is written back by join()."""
        if self._perm_future is not None:
            err = self._perm_future.result()
            self._perm_future = None
            if err is not None:
                self.join()
                raise RuntimeError(f"ppo_host_randperm_range: {err}")
        return self.out

    def join(self) -> torch.Tensor | None:
        errs = []
        if self._first_future is not None:
            self.wait_first()
        for f in (self._perm_future, self._future):
            if f is not None:
                e = f.result()
                if e is not None:
                    errs.append(e)
        self._perm_future = self._future = None
        if errs:
            self._rec = None
            raise RuntimeError(f"host generator draws: {errs[0]}")
        if self._rec is not None:
            torch.set_rng_state(torch.frombuffer(self._rec, dtype=torch.uint8).clone())
            self._rec = None
        return self.out


def gather_rows(perm: torch.Tensor, segments: list[Segment], dst: torch.Tensor) -> None:
    """dst[j, seg.dst_col : +width] = f(seg.src[perm[j]])  (f = identity or the obs normaliser)."""
    _dev(dst)
    _dev(perm, dtype=torch.int64)
    if not perm.is_contiguous() or perm.dim() != 1:
        raise ValueError("perm must be a contiguous int64 vector")
    ld_dst = _row_major(dst, "dst")
    if dst.shape[0] < perm.numel():
        raise ValueError("dst has fewer rows than perm")
    segs = []
    src_rows = None
    for s in segments:
        if s.keep:
            if s.src.dtype != torch.uint8 or s.src.device.type != "cuda" or s.norm_mean is not None:
                raise ValueError("a keep segment reads uint8 done flags on the GPU (no normaliser)")
        else:
            _dev(s.src)
        _dev(s.norm_mean, s.norm_std)
        ld = _row_major(s.src, "segment src")
        src_rows = s.src.shape[0] if src_rows is None else min(src_rows, s.src.shape[0])
        if s.norm_mean is not None and (s.norm_mean.numel() < s.src.shape[1] or s.norm_std is None
                                        or s.norm_std.numel() < s.src.shape[1]):
            raise ValueError("normaliser statistics narrower than the segment")
        segs.append(L.GatherSegment(s.src.data_ptr(), ld, s.src.shape[1], s.dst_col, _ptr(s.norm_mean),
                                    _ptr(s.norm_std), float(s.norm_eps),
                                    L.PPO_GATHER_KEEP_U8 if s.keep else L.PPO_GATHER_FLOAT))
    L.call("ppo_gather_rows", perm.data_ptr(), perm.numel(), int(src_rows), L.array(L.GatherSegment, segs), len(segs),
           dst.data_ptr(), ld_dst, _stream())


def interleave_columns(cols: list[torch.Tensor], dst: torch.Tensor) -> None:
    """dst[:, c:c + w_i] = cols[i] for row-major [rows, w_i] fp32 views, side by side in order."""
    _dev(dst, *cols)
    rows = dst.shape[0]
    blocks = []
    for c in cols:
        if c.dim() != 2 or c.shape[0] != rows:
            raise ValueError("interleave_columns: every block must be [rows, width]")
        blocks.append(L.ColumnBlock(c.data_ptr(), _row_major(c, "column block"), c.shape[1], 0))
    L.call("ppo_interleave_columns", L.array(L.ColumnBlock, blocks), len(blocks), rows, dst.data_ptr(),
           _row_major(dst, "dst"), _stream())


def obs_normalize(x: torch.Tensor, y: torch.Tensor, mean: torch.Tensor, std: torch.Tensor, eps: float) -> None:
    _dev(x, y, mean, std)
    ldx, ldy = _row_major(x, "x"), _row_major(y, "y")
    if x.shape != y.shape or mean.numel() < x.shape[1] or std.numel() < x.shape[1]:
        raise ValueError("obs_normalize: shape mismatch")
    L.call("ppo_obs_normalize", x.data_ptr(), ldx, y.data_ptr(), ldy, x.shape[0], x.shape[1], mean.data_ptr(),
           std.data_ptr(), float(eps), _stream())


# ----------------------------------------------------------------------------------------------------------------------
# A6
# ----------------------------------------------------------------------------------------------------------------------


def _check_weight(w: torch.Tensor, b: torch.Tensor | None) -> tuple[int, int]:
    if w.dim() != 2 or not w.is_contiguous():
        raise ValueError("weight must be a contiguous [out, in] matrix")
    out_f, in_f = w.shape
    if b is not None and (b.numel() != out_f or not b.is_contiguous()):
        raise ValueError("bias must be a contiguous [out] vector")
    return out_f, in_f


def linear_fwd(problems: list[tuple], rows: int, elu: bool = False, act: int | None = None,
               bf16: bool = False) -> None:
    """problems: (x [rows, in], w [out, in], b [out], z [rows, out] or None, h [rows, out] or None).
    act: the hidden-layer activation (an L.ACTIVATIONS code; elu=True is L.PPO_ACT_ELU), h = act(z); without one z is
    required, with one at least one of z / h.  bf16: bf16 operands (ppo_linear_fwd_ex, PPO_GEMM_BF16_OPERANDS)."""
    act = (L.PPO_ACT_ELU if elu else L.PPO_ACT_NONE) if act is None else int(act)
    elu = act != L.PPO_ACT_NONE
    items = []
    for x, w, b, z, h in problems:
        _dev(x, w, b, z, h)
        out_f, in_f = _check_weight(w, b)
        ldx = _row_major(x, "x")
        if x.shape[0] < rows or x.shape[1] < in_f:
            raise ValueError("linear_fwd: x too small")
        if z is None and not (elu and h is not None):
            raise ValueError("linear_fwd: z is required (without ELU, or without h)")
        ldz = ldh = 0
        if z is not None:
            ldz = _row_major(z, "z")
            if z.shape[0] < rows or z.shape[1] < out_f:
                raise ValueError("linear_fwd: z too small")
        if h is not None and elu:
            ldh = _row_major(h, "h")
            if h.shape[0] < rows or h.shape[1] < out_f:
                raise ValueError("linear_fwd: h too small")
        items.append(L.LinearFwdProblem(x.data_ptr(), ldx, w.data_ptr(), b.data_ptr(), _ptr(z), ldz,
                                        _ptr(h) if elu else None, ldh, in_f, out_f))
    if bf16:
        L.call("ppo_linear_fwd_ex", L.array(L.LinearFwdProblem, items), len(items), rows, act, L.GEMM_BF16_OPERANDS,
               _stream())
    else:
        L.call("ppo_linear_fwd", L.array(L.LinearFwdProblem, items), len(items), rows, act, _stream())


def _dx_problems(problems: list[tuple], rows: int):
    items = []
    for dz, w, z_prev, dz_prev in problems:
        _dev(dz, w, z_prev, dz_prev)
        out_f, in_f = _check_weight(w, None)
        lddz, ldo = _row_major(dz, "dz"), _row_major(dz_prev, "dz_prev")
        ldzp = _row_major(z_prev, "z_prev") if z_prev is not None else 0
        if dz.shape[0] < rows or dz_prev.shape[0] < rows or dz.shape[1] < out_f or dz_prev.shape[1] < in_f:
            raise ValueError("linear_bwd_dx: buffers too small")
        if z_prev is not None and (z_prev.shape[0] < rows or z_prev.shape[1] < in_f):
            raise ValueError("linear_bwd_dx: z_prev too small")
        items.append(L.LinearBwdDxProblem(dz.data_ptr(), lddz, w.data_ptr(), _ptr(z_prev), ldzp, dz_prev.data_ptr(),
                                          ldo, in_f, out_f))
    arr = L.array(L.LinearBwdDxProblem, items)
    nbytes = L.load().ppo_linear_bwd_dx_workspace_bytes(arr, len(items))
    if nbytes == 0:
        raise ValueError("linear_bwd_dx: invalid problem set")
    return arr, len(items), nbytes


def linear_bwd_dx(problems: list[tuple], rows: int, ws: Workspace | None = None, elu_from_output: bool = False,
                  act: int = L.PPO_ACT_ELU, bf16: bool = False) -> None:
    """problems: (dz [rows, out], w [out, in], src [rows, in] or None, dz_prev [rows, in]); src is the activation's
    input z of the layer below, or its output h = act(z) with elu_from_output (monotone activations only).  bf16:
    bf16 operands (ppo_linear_bwd_dx_ex, PPO_GEMM_BF16_OPERANDS)."""
    arr, count, nbytes = _dx_problems(problems, rows)
    buf = (ws or Workspace(problems[0][0].device)).get(nbytes)
    src = L.PPO_ELU_FROM_OUTPUT if elu_from_output else L.PPO_ELU_FROM_INPUT
    if bf16:
        L.call("ppo_linear_bwd_dx_ex", arr, count, rows, int(act), src, L.GEMM_BF16_OPERANDS, buf.data_ptr(),
               buf.numel(), _stream())
    else:
        L.call("ppo_linear_bwd_dx_act", arr, count, rows, int(act), src, buf.data_ptr(), buf.numel(), _stream())


@dataclass
class GradNorm:
    """Per-group sums of squares of the gradients a weight-grad launch writes, for adam_step(prenorm=...):
    `partials` [DW_NORM_BLOCKS, MAX_PARAM_GROUPS] fp64; `groups[i]` = the parameter group of problem i (None: not
    counted); `extra` = (begin, end, group) ranges of `extra_grads` (a flat fp32 buffer) that belong to a group's
    norm but are written by another launch."""
    partials: torch.Tensor
    groups: list
    extra_grads: torch.Tensor | None = None
    extra: tuple = ()


def grad_norm_partials(device) -> torch.Tensor:
    return torch.zeros(L.DW_NORM_BLOCKS, L.MAX_PARAM_GROUPS, dtype=torch.float64, device=device)


def linear_bwd_dw(problems: list[tuple], rows: int, ws: Workspace | None = None, norm: GradNorm | None = None,
                  bf16: bool = False) -> None:
    """problems: (dz [rows, out], x [rows, in], dw [out, in], db [out] or None for no bias gradient).  With `norm`
    the launch also writes the per-group sums of squares of what it stores (ppo_linear_bwd_dw_norm).  bf16: bf16
    operands (ppo_linear_bwd_dw_ex, PPO_GEMM_BF16_OPERANDS)."""
    items = []
    for i, (dz, x, dw, db) in enumerate(problems):
        _dev(dz, x, dw, db)
        out_f, in_f = _check_weight(dw, db)
        lddz, ldx = _row_major(dz, "dz"), _row_major(x, "x")
        if dz.shape[0] < rows or x.shape[0] < rows or dz.shape[1] < out_f or x.shape[1] < in_f:
            raise ValueError("linear_bwd_dw: buffers too small")
        group = 0
        if norm is not None and norm.groups[i] is not None:
            group = int(norm.groups[i]) + 1
        items.append(L.LinearBwdDwProblem(dz.data_ptr(), lddz, x.data_ptr(), ldx, dw.data_ptr(), _ptr(db), in_f,
                                          out_f, group, 0))
    arr = L.array(L.LinearBwdDwProblem, items)
    nbytes = L.load().ppo_linear_bwd_dw_workspace_bytes(arr, len(items), rows)
    if nbytes == 0:
        raise ValueError("linear_bwd_dw: invalid problem set")
    buf = (ws or Workspace(problems[0][0].device)).get(nbytes)
    if norm is None:
        if bf16:
            L.call("ppo_linear_bwd_dw_ex", arr, len(items), rows, L.GEMM_BF16_OPERANDS, buf.data_ptr(), buf.numel(),
                   None, None, 0, None, _stream())
        else:
            L.call("ppo_linear_bwd_dw", arr, len(items), rows, buf.data_ptr(), buf.numel(), _stream())
        return
    p = norm.partials
    _dev(p, dtype=torch.float64)
    if tuple(p.shape) != (L.DW_NORM_BLOCKS, L.MAX_PARAM_GROUPS) or not p.is_contiguous():
        raise ValueError("linear_bwd_dw: norm partials must be a contiguous [DW_NORM_BLOCKS, MAX_PARAM_GROUPS] fp64")
    extra = [L.GradRange(int(b), int(e), int(g), 0) for b, e, g in norm.extra]
    if extra:
        _dev(norm.extra_grads)
        if any(r.begin < 0 or r.end > norm.extra_grads.numel() for r in extra):
            raise ValueError("linear_bwd_dw: extra gradient range outside its buffer")
    if bf16:
        L.call("ppo_linear_bwd_dw_ex", arr, len(items), rows, L.GEMM_BF16_OPERANDS, buf.data_ptr(), buf.numel(),
               _ptr(norm.extra_grads) if extra else None, L.array(L.GradRange, extra) if extra else None, len(extra),
               p.data_ptr(), _stream())
    else:
        L.call("ppo_linear_bwd_dw_norm", arr, len(items), rows, buf.data_ptr(), buf.numel(),
               _ptr(norm.extra_grads) if extra else None, L.array(L.GradRange, extra) if extra else None, len(extra),
               p.data_ptr(), _stream())


# ----------------------------------------------------------------------------------------------------------------------
# A7 update
# ----------------------------------------------------------------------------------------------------------------------


def normalizer_update(columns: list[torch.Tensor], mean: torch.Tensor, var: torch.Tensor, std: torch.Tensor,
                      count: torch.Tensor, ws: Workspace | None = None) -> None:
    """columns: row-major [rows, width_i] views whose concatenation is the model latent."""
    _dev(mean, var, std, *columns)
    _dev(count, dtype=torch.int64)
    rows = columns[0].shape[0]
    blocks = []
    for c in columns:
        if c.shape[0] != rows:
            raise ValueError("normalizer_update: column blocks disagree on rows")
        blocks.append(L.ColumnBlock(c.data_ptr(), _row_major(c, "column block"), c.shape[1], 0))
    dim = sum(c.shape[1] for c in columns)
    if mean.numel() != dim or var.numel() != dim or std.numel() != dim:
        raise ValueError("normalizer_update: statistics width != concatenated width")
    for t in (mean, var, std, count):
        if not t.is_contiguous():
            raise ValueError("normalizer_update: statistics must be contiguous")
    nbytes = L.load().ppo_normalizer_update_workspace_bytes(rows, dim)
    buf = (ws or Workspace(mean.device)).get(nbytes)
    L.call("ppo_normalizer_update", L.array(L.ColumnBlock, blocks), len(blocks), rows, mean.data_ptr(),
           var.data_ptr(), std.data_ptr(), count.data_ptr(), buf.data_ptr(), buf.numel(), _stream())


# ----------------------------------------------------------------------------------------------------------------------
# A8-A11 losses, A12-A13 optimiser
# ----------------------------------------------------------------------------------------------------------------------


def new_device_state(learning_rate: float, device) -> torch.Tensor:
    st = torch.zeros(L.DEVICE_STATE_BYTES, dtype=torch.uint8, device=device)
    reset_device_state(st, learning_rate)
    return st


def reset_device_state(st: torch.Tensor, learning_rate: float, staging: torch.Tensor | None = None) -> None:
    """Zero the device state and set its learning rate.  With ``staging`` (a pinned host buffer of the state's size,
    not in use by an earlier copy still in flight) the copy is asynchronous."""
    host = L.DeviceState()
    host.learning_rate = float(learning_rate)
    if staging is None:
        st.copy_(torch.frombuffer(bytearray(bytes(host)), dtype=torch.uint8))
        return
    staging.numpy()[:] = memoryview(bytes(host))
    st.copy_(staging, non_blocking=True)


def read_device_state(st: torch.Tensor) -> L.DeviceState:
    raw = st.cpu().numpy().tobytes()
    return L.DeviceState.from_buffer_copy(raw)


def pinned_state_buffer() -> torch.Tensor:
    """Host staging buffer for an asynchronous read-back of a device state."""
    return torch.empty(L.DEVICE_STATE_BYTES, dtype=torch.uint8, pin_memory=True)


def device_state_from_host(host: torch.Tensor) -> L.DeviceState:
    return L.DeviceState.from_buffer_copy(host.numpy().tobytes())


def make_loss_args(rows: int, mean: torch.Tensor, value: torch.Tensor, batch: dict, std_param: torch.Tensor,
                   std_type: int, std_lo: float, std_hi: float, clip_param: float, value_loss_coef: float,
                   entropy_coef: float, use_clipped_value_loss: bool, d_mean: torch.Tensor,
                   d_value: torch.Tensor) -> L.LossArgs:
    """batch: dict of row-major views sharing one row stride: actions/old_mean/old_std [rows, A] and
    old_logp/advantages/old_values/returns [rows] (columns of the packed table)."""
    A = std_param.numel()
    ld_batch = batch["ld"]
    return L.LossArgs(
        rows=rows, num_actions=A, std_type=std_type,
        mean=mean.data_ptr(), ld_mean=_row_major(mean, "mean"),
        value=value.data_ptr(), ld_value=value.stride(0),
        actions=batch["actions"].data_ptr(), old_mean=batch["old_mean"].data_ptr(),
        old_std=batch["old_std"].data_ptr(), old_logp=batch["old_logp"].data_ptr(),
        advantages=batch["advantages"].data_ptr(), old_values=batch["old_values"].data_ptr(),
        returns=batch["returns"].data_ptr(), ld_batch=ld_batch,
        std_param=std_param.data_ptr(), std_lo=float(std_lo), std_hi=float(std_hi),
        clip_param=float(clip_param), value_loss_coef=float(value_loss_coef), entropy_coef=float(entropy_coef),
        use_clipped_value_loss=1 if use_clipped_value_loss else 0, reserved=0,
        d_mean=d_mean.data_ptr(), ld_dmean=_row_major(d_mean, "d_mean"),
        d_value=d_value.data_ptr(), ld_dvalue=d_value.stride(0),
    )


def ppo_loss(args: L.LossArgs, ws: torch.Tensor) -> None:
    L.call("ppo_gauss_ppo_loss", C_ref(args), ws.data_ptr(), ws.numel(), _stream())


def ppo_loss_finalize(args: L.LossArgs, ws: torch.Tensor, d_std_param: torch.Tensor, state: torch.Tensor,
                      adaptive: bool, desired_kl: float, trace: torch.Tensor | None) -> None:
    L.call("ppo_loss_finalize", C_ref(args), ws.data_ptr(), ws.numel(), d_std_param.data_ptr(), state.data_ptr(),
           1 if adaptive else 0, float(desired_kl if desired_kl is not None else 0.0), _ptr(trace), _trace_rows(trace),
           _stream())


def _trace_rows(trace: torch.Tensor | None) -> int:
    """Rows of 5 doubles a trace buffer holds (the finalize kernels write none past them)."""
    if trace is None:
        return 0
    if trace.dtype != torch.float64 or not trace.is_contiguous():
        raise ValueError("trace: a contiguous float64 buffer")
    return trace.numel() // 5


def loss_workspace_bytes(rows: int, num_actions: int) -> int:
    return int(L.load().ppo_loss_workspace_bytes(rows, num_actions))


def head_supported(num_actions: int, k_actor: int, k_critic: int) -> bool:
    """Whether ppo_gauss_ppo_head takes these output layers (host arithmetic only)."""
    return bool(L.load().ppo_gauss_ppo_head_supported(num_actions, k_actor, k_critic))


def head_workspace_bytes(rows: int, num_actions: int) -> int:
    return int(L.load().ppo_head_workspace_bytes(rows, num_actions))


def ppo_head(args: L.LossArgs, h_actor: torch.Tensor, w_actor: torch.Tensor, b_actor: torch.Tensor,
             h_critic: torch.Tensor, w_critic: torch.Tensor, b_critic: torch.Tensor, dz_actor: torch.Tensor,
             dz_critic: torch.Tensor, ws: torch.Tensor, d_std_param: torch.Tensor, state: torch.Tensor,
             adaptive: bool, desired_kl: float | None, trace: torch.Tensor | None,
             mean: torch.Tensor | None = None, value: torch.Tensor | None = None) -> None:
    """Output layers + loss + finalize + the output layers' input-grad in one call (ppo_gauss_ppo_head).  args
    carries the batch columns and d_mean / d_value; its mean / value fields are not read."""
    _dev(h_actor, w_actor, b_actor, h_critic, w_critic, b_critic, dz_actor, dz_critic, mean, value)
    R = int(args.rows)
    for name, t in (("h_actor", h_actor), ("h_critic", h_critic), ("dz_actor", dz_actor), ("dz_critic", dz_critic)):
        if t.dim() != 2 or t.shape[0] < R:
            raise ValueError(f"ppo_head: {name} must be [rows, width], got {tuple(t.shape)}")
    ka, kc = h_actor.shape[1], h_critic.shape[1]
    if tuple(w_actor.shape) != (args.num_actions, ka) or not w_actor.is_contiguous() or \
            b_actor.numel() != args.num_actions:
        raise ValueError(f"ppo_head: actor output layer {tuple(w_actor.shape)} does not map {ka} -> "
                         f"{args.num_actions}")
    if tuple(w_critic.shape) != (1, kc) or not w_critic.is_contiguous() or b_critic.numel() != 1:
        raise ValueError(f"ppo_head: critic output layer {tuple(w_critic.shape)} does not map {kc} -> 1")
    if tuple(dz_actor.shape[1:]) != (ka,) or tuple(dz_critic.shape[1:]) != (kc,):
        raise ValueError("ppo_head: dz_actor / dz_critic must match the hidden widths")
    head = L.PolicyHead(
        h_actor=h_actor.data_ptr(), ld_h_actor=_row_major(h_actor, "h_actor"), w_actor=w_actor.data_ptr(),
        b_actor=b_actor.data_ptr(), h_critic=h_critic.data_ptr(), ld_h_critic=_row_major(h_critic, "h_critic"),
        w_critic=w_critic.data_ptr(), b_critic=b_critic.data_ptr(),
        dz_actor=dz_actor.data_ptr(), ld_dz_actor=_row_major(dz_actor, "dz_actor"),
        dz_critic=dz_critic.data_ptr(), ld_dz_critic=_row_major(dz_critic, "dz_critic"),
        mean=_ptr(mean), ld_mean=_row_major(mean, "mean") if mean is not None else 0,
        value=_ptr(value), ld_value=value.stride(0) if value is not None else 0, k_actor=ka, k_critic=kc)
    L.call("ppo_gauss_ppo_head", C_ref(args), C_ref(head), ws.data_ptr(), ws.numel(), d_std_param.data_ptr(),
           state.data_ptr(), 1 if adaptive else 0, float(desired_kl if desired_kl is not None else 0.0), _ptr(trace),
           _trace_rows(trace), _stream())


def optim_step(config: "L.OptimConfig", params, grads, state0, state1, group_begin: torch.Tensor,
               max_grad_norm: float, bc1: float, bc2_sqrt: float, state: torch.Tensor, ws: Workspace | None,
               prenorm: torch.Tensor | None = None, mirrors: list[tuple] | None = None) -> None:
    """Clip + the update of config.kind (L.OPTIM_*: Adam, AdamW, SGD, RMSprop) over the flat buffers
    (ppo_optim_step): state0 / state1 are Adam's moments, RMSprop's square_avg (state1 unused), nothing for SGD (both
    unused).  prenorm / mirrors as adam_step's."""
    import ctypes

    _dev(params, grads, state0, state1)
    n = params.numel()
    for t in (grads, state0, state1):
        if t is not None and (t.numel() != n or not t.is_contiguous()):
            raise ValueError("optim_step: flat buffers must be contiguous and equally long")
    if group_begin.device.type != "cpu" or group_begin.dtype != torch.int64 or int(group_begin[-1]) != n:
        raise ValueError("optim_step: group_begin is a host int64 tensor covering the flat buffer")
    items = []
    for begin, rows, cols, dst in mirrors or []:
        _dev(dst)
        ld = _row_major(dst, "mirror dst")
        if dst.shape[0] < rows or dst.shape[1] < cols or begin < 0 or begin + rows * cols > n:
            raise ValueError("optim_step: mirror outside the flat buffer or its destination")
        items.append(L.ParamMirror(int(begin), int(rows), int(cols), dst.data_ptr(), ld))
    buf = None
    if prenorm is not None:
        _dev(prenorm, dtype=torch.float64)
        if tuple(prenorm.shape) != (L.DW_NORM_BLOCKS, L.MAX_PARAM_GROUPS) or not prenorm.is_contiguous():
            raise ValueError("optim_step: prenorm must be a contiguous [DW_NORM_BLOCKS, MAX_PARAM_GROUPS] fp64 tensor")
    else:
        buf = ws.get(L.load().ppo_adam_workspace_bytes(n))
    L.call("ppo_optim_step", params.data_ptr(), grads.data_ptr(), _ptr(state0), _ptr(state1), group_begin.data_ptr(),
           group_begin.numel() - 1, float(max_grad_norm), ctypes.byref(config), float(bc1), float(bc2_sqrt),
           state.data_ptr(), _ptr(prenorm), _ptr(buf), 0 if buf is None else buf.numel(),
           L.array(L.ParamMirror, items) if items else None, len(items), _stream())


def adam_step(params, grads, exp_avg, exp_avg_sq, group_begin: torch.Tensor, max_grad_norm: float, beta1: float,
              beta2: float, eps: float, bc1: float, bc2_sqrt: float, state: torch.Tensor, ws: Workspace | None,
              prenorm: torch.Tensor | None = None, mirrors: list[tuple] | None = None) -> None:
    """Clip + Adam over the flat buffers.  prenorm: the GradNorm partials of the weight-grad launch that wrote every
    gradient of every group (ppo_adam_step_prenorm, one launch); else the norms are computed here (two launches).
    mirrors (with prenorm): (begin, rows, cols, dst [rows, >= cols] row-major) -- the updated rows x cols parameters at
    flat offset begin are also written to dst (ppo_adam_step_prenorm_mirror)."""
    _dev(params, grads, exp_avg, exp_avg_sq)
    n = params.numel()
    for t in (grads, exp_avg, exp_avg_sq):
        if t.numel() != n or not t.is_contiguous():
            raise ValueError("adam_step: flat buffers must be contiguous and equally long")
    if group_begin.device.type != "cpu" or group_begin.dtype != torch.int64:
        raise ValueError("adam_step: group_begin is a host int64 tensor")
    groups = group_begin.numel() - 1
    if int(group_begin[-1]) != n:
        raise ValueError("adam_step: the groups must cover the flat buffer")
    if prenorm is not None:
        _dev(prenorm, dtype=torch.float64)
        if tuple(prenorm.shape) != (L.DW_NORM_BLOCKS, L.MAX_PARAM_GROUPS) or not prenorm.is_contiguous():
            raise ValueError("adam_step: prenorm must be a contiguous [DW_NORM_BLOCKS, MAX_PARAM_GROUPS] fp64 tensor")
        if mirrors:
            if len(mirrors) > L.MAX_PARAM_MIRRORS:
                raise ValueError(f"adam_step: at most {L.MAX_PARAM_MIRRORS} mirrors")
            items = []
            for begin, rows, cols, dst in mirrors:
                _dev(dst)
                ld = _row_major(dst, "mirror dst")
                if dst.shape[0] < rows or dst.shape[1] < cols or begin < 0 or begin + rows * cols > n:
                    raise ValueError("adam_step: mirror outside the flat buffer or its destination")
                items.append(L.ParamMirror(int(begin), int(rows), int(cols), dst.data_ptr(), ld))
            L.call("ppo_adam_step_prenorm_mirror", params.data_ptr(), grads.data_ptr(), exp_avg.data_ptr(),
                   exp_avg_sq.data_ptr(), group_begin.data_ptr(), groups, float(max_grad_norm), float(beta1),
                   float(beta2), float(eps), float(bc1), float(bc2_sqrt), state.data_ptr(), prenorm.data_ptr(),
                   L.array(L.ParamMirror, items), len(items), _stream())
            return
        L.call("ppo_adam_step_prenorm", params.data_ptr(), grads.data_ptr(), exp_avg.data_ptr(),
               exp_avg_sq.data_ptr(), group_begin.data_ptr(), groups, float(max_grad_norm), float(beta1),
               float(beta2), float(eps), float(bc1), float(bc2_sqrt), state.data_ptr(), prenorm.data_ptr(),
               _stream())
        return
    nbytes = L.load().ppo_adam_workspace_bytes(n)
    buf = ws.get(nbytes)
    L.call("ppo_adam_step", params.data_ptr(), grads.data_ptr(), exp_avg.data_ptr(), exp_avg_sq.data_ptr(),
           group_begin.data_ptr(), groups, float(max_grad_norm), float(beta1), float(beta2), float(eps), float(bc1),
           float(bc2_sqrt), state.data_ptr(), buf.data_ptr(), buf.numel(), _stream())


def C_ref(struct):
    import ctypes

    return ctypes.byref(struct)


# ----------------------------------------------------------------------------------------------------------------------
# A15 LSTM / GRU
# ----------------------------------------------------------------------------------------------------------------------


class LstmPacked:
    """Gate-interleaved copies of one nn.LSTM (or nn.GRU) layer's weights (row 4u + q = slot q of unit u: the LSTM's
    gates i, f, g, o; the GRU's r, z, hidden part of n, input part of n)."""

    def __init__(self, input_size: int, hidden: int, device) -> None:
        H, D = hidden, input_size
        self.input_size, self.hidden = D, H
        self.w_ih_g = torch.empty(4 * H, D, device=device)
        self.w_hh_g = torch.empty(4 * H, H, device=device)
        self.w_hh_gt = torch.empty(H, 4 * H, device=device)
        self.b_g = torch.empty(4 * H, device=device)


def lstm_pack(items: list[tuple], gru: bool = False) -> None:
    """items: (w_ih [G, D], w_hh [G, H], b_ih [G], b_hh [G], LstmPacked) with G = 4H (nn.LSTM) or, with gru, 3H
    (nn.GRU, ppo_gru_pack); any number (launches of up to MAX_LSTM_PROBLEMS each)."""
    probs = []
    for w_ih, w_hh, b_ih, b_hh, pk in items:
        _dev(w_ih, w_hh, b_ih, b_hh)
        for t in (w_ih, w_hh, b_ih, b_hh):
            if not t.is_contiguous():
                raise ValueError("lstm_pack: weights must be contiguous")
        H, D = pk.hidden, pk.input_size
        G = (3 if gru else 4) * H
        if (tuple(w_ih.shape) != (G, D) or tuple(w_hh.shape) != (G, H) or b_ih.numel() != G
                or b_hh.numel() != G):
            raise ValueError("lstm_pack: weight shapes do not match the packed buffers")
        probs.append(L.LstmPackProblem(w_ih.data_ptr(), w_hh.data_ptr(), b_ih.data_ptr(), b_hh.data_ptr(),
                                       pk.w_ih_g.data_ptr(), pk.w_hh_g.data_ptr(), pk.w_hh_gt.data_ptr(),
                                       pk.b_g.data_ptr(), pk.input_size, pk.hidden))
    name = "ppo_gru_pack" if gru else "ppo_lstm_pack"
    for i in range(0, len(probs), L.MAX_LSTM_PROBLEMS):
        part = probs[i:i + L.MAX_LSTM_PROBLEMS]
        L.call(name, L.array(L.LstmPackProblem, part), len(part), _stream())


def _seq_problem(q: dict, steps: int, envs: int, bwd: bool) -> "L.LstmSeqProblem":
    H = q["hidden"]
    gx, h0, c0, h = q["gx"], q["h0"], q["c0"], q["h"]
    keep = q["keep"]
    _dev(gx, h0, c0, h, keep, q["hs"], q["c"], q["gates"], q.get("dh"), q.get("dgates"), q.get("dc"))
    if q["packed"].hidden != H:
        raise ValueError("lstm: packed weights of another hidden size")
    if h0.stride(0) != c0.stride(0):
        raise ValueError("lstm: h0 and c0 must share a leading dimension")
    # every buffer must hold the rows and columns the kernels touch (the kernels see raw pointers only)
    R = steps * envs
    need = {"gx": (R, 4 * H), "h0": (envs, H), "c0": (envs, H), "h": (R, H), "hs": (R + envs, H), "c": (R, H),
            "gates": (R, 4 * H)}
    if bwd:
        need.update({"dh": (R, H), "dgates": (R, 4 * H), "dc": (envs, H)})
    for name, (rows, cols) in need.items():
        t = q.get(name)
        if t is None:
            raise ValueError(f"lstm: {name} is required")
        if t.dim() != 2 or t.shape[0] < rows or t.shape[1] < cols or t.stride(1) != 1:
            raise ValueError(f"lstm: {name} {tuple(t.shape)} must be a row-major view of at least [{rows}, {cols}]")
    if keep.dim() != 1 or keep.shape[0] < R:
        raise ValueError(f"lstm: keep must be a vector of at least {R} entries")
    dh = q.get("dh")
    return L.LstmSeqProblem(q["packed"].w_hh_g.data_ptr(), q["packed"].w_hh_gt.data_ptr(), gx.data_ptr(),
                            _row_major(gx, "gx"), h0.data_ptr(), c0.data_ptr(), _row_major(h0, "h0"), keep.data_ptr(),
                            keep.stride(0), h.data_ptr(), _row_major(h, "h"), q["hs"].data_ptr(), q["c"].data_ptr(),
                            q["gates"].data_ptr(), _ptr(dh), _row_major(dh, "dh") if dh is not None else 0,
                            _ptr(q.get("dgates")), _ptr(q.get("dc")), H,
                            L.CELL_GRU if q.get("gru") else L.CELL_LSTM)


def lstm_seq_wait_limit(ticks: int | None) -> int:
    """Set how long the blocks of a whole-sequence LSTM launch wait for each other (100 MHz ticks) for every later
    launch; None restores the default.  Returns the previous limit.  For tests that force the give-up path."""
    return int(L.load().ppo_lstm_seq_wait_limit(-1 if ticks is None else int(ticks)))


def lstm_seq_sync_words(count: int, envs: int) -> int:
    """int32 words of the whole-sequence launches' synchronisation buffer (word 0: sticky status)."""
    n = L.load().ppo_lstm_seq_sync_words(count, envs)
    if n < 0:
        raise ValueError(f"lstm_seq_sync_words: count={count} envs={envs}")
    return n


def _sync_args(sync: torch.Tensor | None, count: int, envs: int) -> tuple[int, int]:
    if sync is None:
        return 0, 0
    if sync.dtype != torch.int32 or not sync.is_contiguous() or sync.device.type != "cuda":
        raise ValueError("lstm sync buffer must be a contiguous int32 device tensor")
    return sync.data_ptr(), sync.numel()


def lstm_seq_fwd(problems: list[dict], steps: int, envs: int, sync: torch.Tensor | None = None,
                 proj: list[torch.Tensor] | None = None, bf16: bool = False) -> None:
    """problems: dicts with packed (LstmPacked), hidden, gx [T*E, 4H], h0 / c0 [E, H], keep [T*E] (stride = row
    step), h [T*E, H], hs [(T+1)*E, H], c [T*E, H], gates [T*E, 4H], and gru=True for a GRU (c0 = h0; c receives
    the state h).  sync: int32 device buffer of
    lstm_seq_sync_words(len(problems), envs) words (zeroed once by the caller) for the one-launch sequence, or None
    for one launch per step.  proj: each problem's layer input x [T*E, D]: the call computes gx = x w_ih_g^T + b_g
    itself (ppo_lstm_seq_fwd_proj; inside the sequence launch when it can, gx is then scratch), with bf16 operands
    when bf16."""
    arr = L.array(L.LstmSeqProblem, [_seq_problem(q, steps, envs, False) for q in problems])
    if proj is None:
        L.call("ppo_lstm_seq_fwd", arr, len(problems), steps, envs, *_sync_args(sync, len(problems), envs), _stream())
        return
    items = []
    for q, x in zip(problems, proj, strict=True):
        pk = q["packed"]
        _dev(x)
        if x.dim() != 2 or x.shape[0] < steps * envs or x.shape[1] != pk.input_size or x.stride(1) != 1:
            raise ValueError(f"lstm projection: x {tuple(x.shape)} must be a row-major view of [{steps * envs}, "
                             f"{pk.input_size}]")
        items.append(L.LstmInputProjection(x.data_ptr(), x.stride(0), pk.w_ih_g.data_ptr(), pk.b_g.data_ptr(),
                                           pk.input_size, 0))
    L.call("ppo_lstm_seq_fwd_proj", arr, L.array(L.LstmInputProjection, items), len(problems), steps, envs,
           L.GEMM_BF16_OPERANDS if bf16 else 0, *_sync_args(sync, len(problems), envs), _stream())


def lstm_seq_bwd(problems: list[dict], steps: int, envs: int, sync: torch.Tensor | None = None) -> None:
    """As lstm_seq_fwd's problems plus dh [T*E, H], dgates [T*E, 4H], dc [E, H] (scratch)."""
    arr = L.array(L.LstmSeqProblem, [_seq_problem(q, steps, envs, True) for q in problems])
    L.call("ppo_lstm_seq_bwd", arr, len(problems), steps, envs, *_sync_args(sync, len(problems), envs), _stream())


def lstm_unpack_grads(items: list[tuple], gru: bool = False, norm: tuple | None = None) -> None:
    """items: (dw_ih_g [4H, D], dw_hh_g [4H, H], db_g [4H], dw_ih, dw_hh, db_ih, db_hh (torch layout views: 4H rows,
    or 3H with gru, ppo_gru_unpack_grads)), any number (launches of up to MAX_LSTM_PROBLEMS each).  norm =
    (partials, groups): also add the sums of squares of the written gradients, item i's to parameter group groups[i],
    to the norm partials of the weight-grad launch before (ppo_lstm_unpack_grads_norm / ppo_gru_unpack_grads_norm)."""
    if norm is not None:
        partials, groups = norm
        _dev(partials, dtype=torch.float64)
        if (partials.dtype != torch.float64 or tuple(partials.shape) != (L.DW_NORM_BLOCKS, L.MAX_PARAM_GROUPS)
                or not partials.is_contiguous()):
            raise ValueError("lstm_unpack_grads: norm partials must be contiguous float64 [DW_NORM_BLOCKS, "
                             "MAX_PARAM_GROUPS]")
        if len(groups) != len(items):
            raise ValueError("lstm_unpack_grads: one parameter group per item")
    probs = []
    for dw_ih_g, dw_hh_g, db_g, dw_ih, dw_hh, db_ih, db_hh in items:
        _dev(dw_ih_g, dw_hh_g, db_g, dw_ih, dw_hh, db_ih, db_hh)
        H, D = dw_hh.shape[1], dw_ih.shape[1]
        G = (3 if gru else 4) * H
        for t, n in ((dw_ih_g, 4 * H * D), (dw_ih, G * D), (dw_hh_g, 4 * H * H), (dw_hh, G * H), (db_g, 4 * H),
                     (db_ih, G), (db_hh, G)):
            if t.numel() != n or not t.is_contiguous():
                raise ValueError("lstm_unpack_grads: gradient buffers do not match [4H, D] / [4H, H] / [4H] "
                                 "(torch layout: [G, D] / [G, H] / [G])")
        probs.append(L.LstmGradProblem(dw_ih_g.data_ptr(), dw_hh_g.data_ptr(), db_g.data_ptr(), dw_ih.data_ptr(),
                                       dw_hh.data_ptr(), db_ih.data_ptr(), db_hh.data_ptr(), dw_ih.shape[1], H))
    name = "ppo_gru_unpack_grads" if gru else "ppo_lstm_unpack_grads"
    for i in range(0, len(probs), L.MAX_LSTM_PROBLEMS):
        part = probs[i:i + L.MAX_LSTM_PROBLEMS]
        if norm is None:
            L.call(name, L.array(L.LstmGradProblem, part), len(part), _stream())
        else:
            import ctypes
            grp = (ctypes.c_int32 * len(part))(*norm[1][i:i + L.MAX_LSTM_PROBLEMS])
            L.call(name + "_norm", L.array(L.LstmGradProblem, part), grp, len(part), norm[0].data_ptr(), _stream())
