"""The PPO update on the GPU: packed-table gather, then per mini-batch forward, loss, backward and Adam kernels.

This is the device-side body of upstream's ``PPO.update`` (rsl_rl/algorithms/ppo.py:193-358) for feed-forward
actor/critic MLPs.  Everything the update computes runs in libppo_hip.so; the host only enqueues kernels and reads
the three losses and the learning rate back once, after the last mini-batch.

HBM layout of one update:
  * the packed table [B, W] fp32, rows in permutation order (one gather per update, because upstream reuses a
    single permutation for all epochs): [actor latent | critic latent | actions | old mean | old std |
    old log-prob | advantage | old value | return | per-mini-batch advantage scratch], each block 16 B aligned;
  * per model and layer: pre-activation Z and ELU output H [R, width], the output [R, out], and the backward's
    dZ [R, width] (R = rows of the largest mini-batch);
  * flat parameter / gradient / exp_avg / exp_avg_sq buffers [P] (actor block then critic block, upstream's
    parameter order), which the models' parameters and torch's Adam state view;
  * a small device state (learning rate, loss sums, clip diagnostics) and split-K / loss / Adam scratch.
"""

from __future__ import annotations

import os

import torch

from . import _lib as L
from . import ops


def _align4(n: int) -> int:
    return (n + 3) // 4 * 4


# The forward GEMM's k-slab is 16 floats: a first layer whose input width is not a multiple of 16 runs on a copy of
# its weight zero-padded to the next multiple (16-byte loads of both operands, no masked tail slab; measured on
# MI355X for 24,576 rows x 512 outputs: inputs 96 + 99 86.5 -> 75.5 us, 235 + 235 141 -> 120 us).
K_SLACK = 16


def _pad16(n: int) -> int:
    return (n + 15) // 16 * 16


class TableLayout:
    """Column blocks of the packed table.  shared_obs: the critic reads the actor's latent block (the same observation
    groups and neither model normalises: identical latents), so the gather copies each observation once."""

    def __init__(self, actor_dim: int, critic_dim: int, num_actions: int, keep: bool = False,
                 shared_obs: bool = False) -> None:
        if shared_obs and actor_dim != critic_dim:
            raise ValueError("TableLayout: shared latents need equal widths")
        c = 0
        self.xa = c
        c = _align4(c + actor_dim)
        self.shared_obs = shared_obs
        self.xc = self.xa if shared_obs else c
        if not shared_obs:
            c = _align4(c + critic_dim)
        self.actions = c
        c = _align4(c + num_actions)
        self.old_mean = c
        c = _align4(c + num_actions)
        self.old_std = c
        c = _align4(c + num_actions)
        self.old_logp, self.adv, self.old_values, self.returns, self.adv_mb = c, c + 1, c + 2, c + 3, c + 4
        self.keep = c + 5 if keep else None  # recurrent: 1 - done of the row's step
        # + K_SLACK zero columns: the first layers' GEMMs may read up to K_SLACK - 1 columns past an observation
        # block (against zero weight columns), which must stay inside the row and hold finite values
        self.width = _align4(c + (6 if keep else 5)) + K_SLACK


class ModelBuffers:
    """Activation and gradient buffers of one MLP for mini-batches of up to `rows` rows.  Rows are padded to a
    multiple of 4 floats (views keep the logical width) so every buffer can be read with 16-byte loads."""

    def __init__(self, model, rows: int, device) -> None:
        lin = model.linears
        self.widths = [l.out_features for l in lin]
        self.act = model.act_code
        # the input-grad takes act' from h = act(z) where the activation allows it (ELU and the other monotone ones);
        # the others (softplus, gelu, swish, mish) keep z as well
        self.from_output = self.act in L.ACT_FROM_OUTPUT

        def buf(w: int) -> torch.Tensor:
            return torch.empty(rows, -(-w // 4) * 4, device=device)[:, :w]

        self.out = buf(self.widths[-1])                 # output layer (no activation): mean / value
        self.h = [buf(w) for w in self.widths[:-1]]     # hidden layers' act(z)
        self.z = None if self.from_output else [buf(w) for w in self.widths[:-1]]
        self.dz = [buf(w) for w in self.widths]

    def act_src(self, i: int, R: int) -> torch.Tensor:
        """What the input-grad below hidden layer i reads for act': h (from the output) or z."""
        return (self.h if self.from_output else self.z)[i][:R]


class PhaseTimer:
    """Optional instrumentation: HIP events (torch.cuda.Event on the launch stream) around named launches."""

    def __init__(self, only: set[str] | None = None) -> None:
        self.events: dict[str, list[tuple[torch.cuda.Event, torch.cuda.Event]]] = {}
        self._open: dict[str, torch.cuda.Event] = {}
        self.enabled = True
        self.only = only  # None: every phase; else only these names get events

    def start(self, name: str) -> None:
        if self.enabled and (self.only is None or name in self.only):
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            self._open[name] = e

    def stop(self, name: str) -> None:
        if name in self._open:
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            self.events.setdefault(name, []).append((self._open.pop(name), e))

    def reset(self) -> None:
        self.events.clear()
        self._open.clear()

    def summary(self) -> dict[str, tuple[int, float]]:
        """name -> (launches, mean milliseconds); call after a device synchronisation."""
        return {k: (len(v), sum(a.elapsed_time(b) for a, b in v) / len(v)) for k, v in self.events.items()}


class _NoTimer:
    def start(self, name: str) -> None:
        pass

    def stop(self, name: str) -> None:
        pass


class _RecordingTimer:
    """Forwards to the engine's timer and appends the phase marks to the launch sequence being recorded."""

    def __init__(self, inner, entries: list) -> None:
        self.inner, self.entries = inner, entries

    def start(self, name: str) -> None:
        self.entries.append(("start", name))
        self.inner.start(name)

    def stop(self, name: str) -> None:
        self.entries.append(("stop", name))
        self.inner.stop(name)


class UpdateEngine:
    """Owns the device workspaces of the update and runs it.  Rebuilt when the rollout shape changes.

    Every buffer a launch names is allocated here once, so a mini-batch issues the same launches with the same
    arguments in every update except for Adam's bias corrections.  The second update (the first one may still grow
    the workspaces) records each mini-batch's launch sequence (C entry point + ctypes arguments, and the phase-timer
    marks between them); later updates issue
    the recorded calls directly, with the bias corrections of their own step, instead of rebuilding every argument
    in Python: the host then stays ahead of the GPU from the first mini-batch on.  The records are dropped when a
    hyperparameter or the stream changes."""

    recurrent = False

    def max_rows(self) -> int:
        return -(-self.B // self.M)

    def __init__(self, alg) -> None:
        self.alg = alg
        self.timer = _NoTimer()
        self.device = alg.device
        st = alg.storage
        self.B = st.batch_size
        self.M = alg.num_mini_batches
        if not 1 <= self.M <= self.B:
            raise ValueError("num_mini_batches must be between 1 and the rollout batch size.")
        self.R_max = self.max_rows()
        actor, critic = alg.actor, alg.critic
        self.A = actor.distribution.output_dim
        shared = (list(actor.obs_groups) == list(critic.obs_groups) and not actor.obs_normalization and
                  not critic.obs_normalization)
        self.layout = TableLayout(actor.obs_dim, critic.obs_dim, self.A, keep=self.recurrent, shared_obs=shared)
        self.table = torch.zeros(self.B, self.layout.width, device=self.device)  # padding columns stay zero
        self.scalars = torch.empty(self.B, 4, device=self.device)  # pack_scalars
        # zero-padded copies of first-layer weights whose input width is not a multiple of 16: written by every Adam
        # step beside the weight itself (mirrors of ppo_adam_step_prenorm_mirror) after a row gather at the start of
        # each update; without the one-launch Adam, refreshed by a row gather before every mini-batch's forward
        self.w0_pad: dict[int, torch.Tensor] = {}
        if not self.recurrent:
            for model in (actor, critic):
                w = model.linears[0].weight
                if w.shape[1] % 16:
                    self.w0_pad[id(model)] = torch.zeros(w.shape[0], _pad16(w.shape[1]), device=self.device)
            rows = max((w.shape[0] for w in self.w0_pad.values()), default=0)
            self.w0_rows = torch.arange(rows, dtype=torch.int64, device=self.device)
        self.grad_norm = None if self.recurrent else self._grad_norm_plan()
        self.w0_mirrors: list[tuple] = []
        self._w0_current = False  # inside run(): the copies were refreshed at its start and every Adam step keeps them
        if self.grad_norm is not None and len(self.w0_pad) <= L.MAX_PARAM_MIRRORS:
            for model in (actor, critic):
                wp = self.w0_pad.get(id(model))
                if wp is not None:
                    w = model.linears[0].weight
                    self.w0_mirrors.append((alg.flat.offsets[id(w)][0], w.shape[0], w.shape[1], wp))
        self.buf_a = ModelBuffers(actor, self.R_max, self.device)
        self.buf_c = ModelBuffers(critic, self.R_max, self.device)
        self.loss_ws = torch.empty(ops.loss_workspace_bytes(self.R_max, self.A), dtype=torch.uint8, device=self.device)
        # learn_std=False (distribution.py:166): the std parameter takes no gradient; the loss kernels' gradient for it
        # goes here instead of into the flat gradient, whose slot stays zero, so Adam leaves the parameter (and its
        # zero moments) as they are and the clip norms do not count it
        self.std_grad_sink = torch.zeros_like(actor.distribution.param)
        # the output layers, loss and their input-grad as one launch (ppo_gauss_ppo_head) where it takes the shapes
        la, lc = actor.linears, critic.linears
        self.fused_head = (len(la) >= 2 and len(la) == len(lc) and
                           actor.act_code == critic.act_code == L.PPO_ACT_ELU and  # (its ELU' of the last hidden layer)
                           ops.head_supported(self.A, la[-1].in_features, lc[-1].in_features) and
                           os.environ.get("PPO_HIP_FUSED_HEAD", "1") != "0")
        if self.fused_head:
            self.head_ws = torch.empty(ops.head_workspace_bytes(self.R_max, self.A), dtype=torch.uint8,
                                       device=self.device)
        self.dw_ws = ops.Workspace(self.device)
        self.adam_ws = ops.Workspace(self.device)
        self.dx_ws = ops.Workspace(self.device)  # the input-grad's w^T copies
        self.adv_ws = ops.Workspace(self.device)
        # the observation normalisers' statistics as the update's forward passes must see them (pre-update), in
        # buffers of their own so the recorded gathers keep pointing at them
        self._norm_frozen: dict[int, tuple[torch.Tensor, torch.Tensor]] = {}
        for model in (actor, critic):
            if model.obs_normalization:
                norm = model.obs_normalizer
                self._norm_frozen[id(norm)] = (torch.empty_like(norm._mean.view(-1)),
                                               torch.empty_like(norm._std.view(-1)))
        self._frozen = False
        self._plans: dict = {}
        self.trace = torch.zeros(0, dtype=torch.float64, device=self.device)
        self._ensure_trace()
        self._plan_key = None
        self._warm = False  # records are kept from the second run on: by then no workspace grows any more
        self.replays = 0
        self.replay = os.environ.get("PPO_HIP_LAUNCH_CACHE", "1") != "0" and not self.recurrent
        # inspection hook (None in normal use): called as step_hook(engine, r0, r1) after each mini-batch's launches
        # are enqueued, before the next mini-batch's; the buffers then hold that mini-batch's activations / gradients.
        # It must not change the parameters: within a run the padded first-layer copies follow the Adam steps only
        self.step_hook = None

    # -- one update ------------------------------------------------------------------------------------------------
    def _ensure_trace(self) -> None:
        """Per-mini-batch trace rows (5 doubles each) for every optimiser step of an update; grown (and the recorded
        launches, which hold the old buffer, dropped) when num_learning_epochs rises between updates."""
        need = 5 * self.alg.num_learning_epochs * self.M
        if self.trace.numel() < need:
            self.trace = torch.zeros(need, dtype=torch.float64, device=self.device)
            self.trace_host = torch.empty(need, dtype=torch.float64, pin_memory=True)
            self._plans.clear()

    def freeze_normalizers(self) -> None:
        """Copy the normalisers' current statistics (device to device, on the stream) for this update's gather, so
        the normaliser update (upstream runs it after the epochs, ppo.py:327-330) can be launched first and run
        while the host draws the permutation."""
        dsts, srcs = [], []
        for model in (self.alg.actor, self.alg.critic):
            if model.obs_normalization:
                norm = model.obs_normalizer
                mean, std = self._norm_frozen[id(norm)]
                dsts += [mean, std]
                srcs += [norm._mean.view(-1), norm._std.view(-1)]
        if dsts:
            torch._foreach_copy_(dsts, srcs)
        self._frozen = True

    def _norm_stats(self, norm) -> tuple[torch.Tensor, torch.Tensor]:
        if self._frozen:
            return self._norm_frozen[id(norm)]
        return norm._mean.view(-1), norm._std.view(-1)

    # -- recorded launch sequences ------------------------------------------------------------------------------------
    def _plan_signature(self):
        """What the recorded launches hold besides the engine's own buffers: the stream, the hyperparameters passed
        as values, and every storage tensor the gathers read (address, shape, strides: a storage rebound to other
        tensors of the same shape, or its distribution parameters replaced, must not replay stale addresses)."""
        a = self.alg
        return (torch.cuda.current_stream(self.device).cuda_stream, a.clip_param, a.value_loss_coef, a.entropy_coef,
                a.use_clipped_value_loss, a.desired_kl, a.schedule, a.max_grad_norm, tuple(a.betas), a.adam_eps,
                a.optim_kind, a.optim_config.weight_decay, a.optim_config.alpha,
                a.normalize_advantage_per_mini_batch, a.num_learning_epochs, a.use_mixed_precision,
                self._storage_signature())

    def _storage_signature(self) -> tuple:
        st = self.alg.storage
        ts = [*st.observations.values(), st.actions, st.actions_log_prob, st.values, st.returns, st.advantages,
              st.dones, *(st.distribution_params or ())]
        if st.act_record is not None:
            ts.append(st.act_record)
        return (id(st), self.alg.flat.param.data_ptr()) + tuple(
            (t.data_ptr(), tuple(t.shape), tuple(t.stride())) for t in ts)

    def _issue(self, key, fn, step: int | None = None) -> None:
        """Run fn (which issues launches through the C ABI) the first time for this key, recording its calls;
        afterwards issue the recorded calls directly."""
        plan = self._plans.get(key) if self.replay else None
        if plan is None:
            entries: list = []
            timer = self.timer
            L.recorder = entries
            self.timer = _RecordingTimer(timer, entries)
            try:
                fn()
            finally:
                L.recorder = None
                self.timer = timer
            if self.replay and self._warm:
                self._plans[key] = entries
            return
        self.replays += 1
        lib = L.load()
        for e in plan:
            if e[0] == "start":
                self.timer.start(e[1])
            elif e[0] == "stop":
                self.timer.stop(e[1])
            else:
                name, args = e
                if name in ("ppo_adam_step", "ppo_adam_step_prenorm", "ppo_adam_step_prenorm_mirror"):
                    bc1, bc2_sqrt = self._bias_corrections(step)
                    args = args[:10] + (float(bc1), float(bc2_sqrt)) + args[12:]
                elif name == "ppo_optim_step":
                    bc1, bc2_sqrt = self._bias_corrections(step)
                    args = args[:8] + (float(bc1), float(bc2_sqrt)) + args[10:]
                L.check(getattr(lib, name)(*args), name)

    def gather(self, perm: torch.Tensor, row0: int = 0) -> None:
        """Table rows [row0, row0 + len(perm)) = storage rows perm (from row 0: the scalar records are packed
        first)."""
        if row0 == 0:
            self.pack_scalars()
        segs = self.segments()
        dst = self.table[row0:row0 + perm.numel()]
        for i in range(0, len(segs), L.MAX_GATHER_SEGMENTS):
            ops.gather_rows(perm, segs[i:i + L.MAX_GATHER_SEGMENTS], dst)

    def segments(self) -> list[ops.Segment]:
        """The packed table's column blocks and their storage sources ([T * N, width] views)."""
        alg, st, lay = self.alg, self.alg.storage, self.layout
        segs: list[ops.Segment] = []
        models = ((alg.actor, lay.xa),) if lay.shared_obs else ((alg.actor, lay.xa), (alg.critic, lay.xc))
        for model, base in models:
            col = 0
            norm = model.obs_normalizer if model.obs_normalization else None
            for g in model.obs_groups:
                src = st.flat(st.observations[g])
                w = src.shape[1]
                if norm is not None:
                    mean, std = self._norm_stats(norm)
                    segs.append(ops.Segment(src, base + col, mean[col:col + w], std[col:col + w], norm.eps))
                else:
                    segs.append(ops.Segment(src, base + col))
                col += w
        mean, std = st.distribution_params
        if self._record_matches():
            # actions | mean | std with their padding, one contiguous record per row, in the table's column order
            segs.append(ops.Segment(st.act_record.view(self.B, -1), lay.actions))
        else:
            segs += [ops.Segment(st.flat(st.actions), lay.actions), ops.Segment(st.flat(mean), lay.old_mean),
                     ops.Segment(st.flat(std), lay.old_std)]
        # log-prob, advantage, value, return: one 16-byte record per row (pack_scalars)
        segs.append(ops.Segment(self.scalars, lay.old_logp))
        return segs

    def _record_matches(self) -> bool:
        """The storage's actions and (mean, std) are still the views of its interleaved record, laid out as the
        table's actions / old mean / old std columns."""
        st, lay = self.alg.storage, self.layout
        rec = st.act_record
        if rec is None or rec.shape[-1] != 3 * st.act_record_pad or len(st.distribution_params) != 2:
            return False
        ap = st.act_record_pad
        views = (st.actions, *st.distribution_params)
        return (all(v.data_ptr() == rec.data_ptr() + 4 * i * ap and v.stride() == rec[..., :1].stride()
                    for i, v in enumerate(views)) and
                lay.old_mean == lay.actions + ap and lay.old_std == lay.old_mean + ap)

    def pack_scalars(self) -> None:
        """scalars[r] = (log-prob, advantage, value, return) of storage row r, one coalesced pass over the four
        [T, N, 1] buffers (the rows the gather then picks at random are one 16-byte read each)."""
        st = self.alg.storage
        ops.interleave_columns([st.flat(st.actions_log_prob), st.flat(st.advantages), st.flat(st.values),
                                st.flat(st.returns)], self.scalars)

    def refresh_padded_weights(self) -> None:
        """w0_pad[:, :in] = the first layer's weight (the padding columns were zeroed at allocation)."""
        for model in (self.alg.actor, self.alg.critic):
            wp = self.w0_pad.get(id(model))
            if wp is not None:
                w = model.linears[0].weight
                ops.gather_rows(self.w0_rows[:w.shape[0]], [ops.Segment(w, 0)], wp)

    def minibatch(self, r0: int, r1: int, step: int) -> None:
        alg, lay = self.alg, self.layout
        R = r1 - r0
        tab = self.table[r0:r1]
        xa = tab[:, lay.xa:lay.xa + alg.actor.obs_dim]
        xc = tab[:, lay.xc:lay.xc + alg.critic.obs_dim]
        adv_col = self.advantage_column(tab, R)
        if not (self.w0_mirrors and self._w0_current):  # (a caller may have changed the weights since)
            self.refresh_padded_weights()
        fa, wa0 = self._first_layer(alg.actor, tab, lay.xa, xa)
        fc, wc0 = self._first_layer(alg.critic, tab, lay.xc, xc)
        self.head_forward(fa, fc, R, w0=(wa0, wc0))
        self.loss(tab, R, adv_col)
        self.head_backward(R)
        self.weight_grads(self.head_dw(xa, xc, R), R, norm=self.grad_norm)
        self.adam(step, prenorm=self.grad_norm.partials if self.grad_norm is not None else None)

    # -- pieces shared with the recurrent engine ----------------------------------------------------------------------
    def advantage_column(self, tab: torch.Tensor, R: int) -> int:
        lay = self.layout
        if self.alg.normalize_advantage_per_mini_batch and R > 1:
            ops.adv_normalize(tab[:, lay.adv], tab[:, lay.adv_mb], R, in_stride=lay.width, out_stride=lay.width,
                              ws=self.adv_ws)
            return lay.adv_mb
        return lay.adv

    def _layers(self):
        la, lc = self.alg.actor.linears, self.alg.critic.linears
        if len(lc) != len(la):
            raise NotImplementedError("actor and critic must have the same number of layers")
        return la, lc

    def head_forward(self, xa: torch.Tensor, xc: torch.Tensor, R: int, w0: tuple | None = None) -> None:
        """The MLPs, actor and critic grouped layer by layer (hidden layers keep only elu(z)).  w0: the first layer's
        (actor, critic) weights to use in place of the parameters (zero-padded copies, with inputs as wide)."""
        la, lc = self._layers()
        ba, bc = self.buf_a, self.buf_c
        nl = len(la)
        tm = self.timer
        ins_a, ins_c = [xa], [xc]
        for i in range(nl - 1 if self.fused_head else nl):
            last = i == nl - 1
            wa, wc = w0 if i == 0 and w0 is not None else (la[i].weight, lc[i].weight)
            probs = []
            for b, x, w, lin in ((ba, ins_a[-1], wa, la[i]), (bc, ins_c[-1], wc, lc[i])):
                z = b.out[:R] if last else (b.z[i][:R] if b.z is not None else None)
                probs.append((x, w, lin.bias, z, None if last else b.h[i][:R]))
            tm.start(f"fwd{i}")
            bf16 = self.alg.use_mixed_precision
            if last:
                ops.linear_fwd(probs, R, act=L.PPO_ACT_NONE, bf16=bf16)
            elif ba.act == bc.act:
                ops.linear_fwd(probs, R, act=ba.act, bf16=bf16)
            else:  # (actor and critic with different activations: one launch each)
                ops.linear_fwd(probs[:1], R, act=ba.act, bf16=bf16)
                ops.linear_fwd(probs[1:], R, act=bc.act, bf16=bf16)
            tm.stop(f"fwd{i}")
            if not last:
                ins_a.append(ba.h[i][:R])
                ins_c.append(bc.h[i][:R])

    def _grad_norm_plan(self) -> ops.GradNorm | None:
        """The clip norms from the weight-grad launch (ppo_linear_bwd_dw_norm + ppo_adam_step_prenorm, one Adam launch
        instead of two), when that launch writes every linear layer's gradients and the few other gradients (the
        distribution's std parameter) fit as extra ranges; else None (ppo_adam_step computes the norms itself)."""
        f = self.alg.flat
        la, lc = self._layers()
        linear = {id(p) for lin in (*la, *lc) for p in (lin.weight, lin.bias)}
        if 2 * len(la) > L.MAX_LINEAR_PROBLEMS or any(lin.bias is None for lin in (*la, *lc)):
            return None
        bounds = f.group_begin.tolist()
        group = lambda off: max(i for i in range(len(bounds) - 1) if bounds[i] <= off)  # noqa: E731
        extra = []
        for p in f.params:
            if id(p) not in linear and p.requires_grad:  # (a fixed std takes no gradient: not in the norms)
                off, k = f.offsets[id(p)]
                extra.append((off, off + k, group(off)))
        if len(extra) > L.MAX_EXTRA_GRADS or len(bounds) - 1 > L.MAX_PARAM_GROUPS:
            return None
        groups = [group(f.offsets[id(lin.weight)][0]) for lin in la] + [group(f.offsets[id(lin.weight)][0]) for lin in lc]
        return ops.GradNorm(ops.grad_norm_partials(self.device), groups, f.grad, tuple(extra))

    def _first_layer(self, model, tab: torch.Tensor, col: int, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(input, weight) of the model's first forward GEMM: the padded weight copy and the table block read
        as wide as it, where the model has one."""
        wp = self.w0_pad.get(id(model))
        if wp is None:
            return x, model.linears[0].weight
        return tab[:, col:col + wp.shape[1]], wp

    def loss(self, tab: torch.Tensor, R: int, adv_col: int) -> None:
        """Losses + per-row output gradients, then the device-side reduction / LR rule / std-parameter gradient.
        With the fused head the output layers' forward and input-grad run in the same launch."""
        alg, lay = self.alg, self.layout
        ba, bc = self.buf_a, self.buf_c
        dist = alg.actor.distribution
        lo, hi = dist.param_range
        batch = {"ld": lay.width, "actions": tab[:, lay.actions], "old_mean": tab[:, lay.old_mean],
                 "old_std": tab[:, lay.old_std], "old_logp": tab[:, lay.old_logp], "advantages": tab[:, adv_col],
                 "old_values": tab[:, lay.old_values], "returns": tab[:, lay.returns]}
        args = ops.make_loss_args(R, ba.out[:R], bc.out[:R, 0], batch, dist.param, dist.kernel_std_type, lo, hi,
                                  alg.clip_param, alg.value_loss_coef, alg.entropy_coef, alg.use_clipped_value_loss,
                                  ba.dz[-1][:R], bc.dz[-1][:R, 0])
        tm = self.timer
        adaptive = alg.desired_kl is not None and alg.schedule == "adaptive"
        std_grad = alg.flat.grad_view(dist.param) if dist.param.requires_grad else self.std_grad_sink
        if self.fused_head:
            la, lc = self._layers()
            tm.start("head")
            ops.ppo_head(args, ba.h[-1][:R], la[-1].weight, la[-1].bias, bc.h[-1][:R], lc[-1].weight, lc[-1].bias,
                         ba.dz[-2][:R], bc.dz[-2][:R], self.head_ws, std_grad,
                         alg.device_state, adaptive, alg.desired_kl, self.trace, mean=ba.out[:R],
                         value=bc.out[:R, 0])
            tm.stop("head")
            return
        tm.start("loss")
        ops.ppo_loss(args, self.loss_ws)
        ops.ppo_loss_finalize(args, self.loss_ws, std_grad, alg.device_state, adaptive,
                              alg.desired_kl if alg.desired_kl is not None else 0.0, self.trace)
        tm.stop("loss")

    def dx_layers(self, R: int) -> list[tuple[int, list[tuple], bool, int]]:
        """The head's input-gradients, top layer first: (layer, grouped actor / critic problems, act' taken from the
        layer below's output, the activation).  Layer 0 has none (no gradient into the observations)."""
        la, lc = self._layers()
        ba, bc = self.buf_a, self.buf_c
        top = len(la) - 2 if self.fused_head else len(la) - 1  # the fused head produced the output layer's
        out = []
        for i in range(top, 0, -1):
            pa = (ba.dz[i][:R], la[i].weight, ba.act_src(i - 1, R), ba.dz[i - 1][:R])
            pc = (bc.dz[i][:R], lc[i].weight, bc.act_src(i - 1, R), bc.dz[i - 1][:R])
            if (ba.act, ba.from_output) == (bc.act, bc.from_output):
                out.append((i, [pa, pc], ba.from_output, ba.act))
            else:
                out += [(i, [pa], ba.from_output, ba.act), (i, [pc], bc.from_output, bc.act)]
        return out

    def head_backward(self, R: int) -> None:
        """Input gradients down the chain (actor and critic grouped)."""
        tm = self.timer
        for i, probs, from_output, act in self.dx_layers(R):
            tm.start(f"dx{i}")
            ops.linear_bwd_dx(probs, R, self.dx_ws, elu_from_output=from_output, act=act,
                              bf16=self.alg.use_mixed_precision)
            tm.stop(f"dx{i}")

    def head_dw(self, xa: torch.Tensor, xc: torch.Tensor, R: int) -> list[tuple]:
        la, lc = self._layers()
        grad = self.alg.flat.grad_view
        dw = []
        for buf, lins, x0 in ((self.buf_a, la, xa), (self.buf_c, lc, xc)):
            for i in range(len(lins)):
                x = x0 if i == 0 else buf.h[i - 1][:R]
                dw.append((buf.dz[i][:R], x, grad(lins[i].weight), grad(lins[i].bias)))
        return dw

    def weight_grads(self, dw: list[tuple], R: int, phase: str = "dw", ws: ops.Workspace | None = None,
                     norm: ops.GradNorm | None = None) -> None:
        """Weight gradients, as few grouped launches as the problem limit allows (with `norm`: one launch that also
        sums the squares for the clip norms)."""
        tm = self.timer
        tm.start(phase)
        bf16 = self.alg.use_mixed_precision
        if norm is not None:
            if len(dw) > L.MAX_LINEAR_PROBLEMS:
                raise RuntimeError("weight_grads: the norm partials need all problems in one launch")
            ops.linear_bwd_dw(dw, R, ws if ws is not None else self.dw_ws, norm=norm, bf16=bf16)
        else:
            for i in range(0, len(dw), L.MAX_LINEAR_PROBLEMS):
                ops.linear_bwd_dw(dw[i:i + L.MAX_LINEAR_PROBLEMS], R, ws if ws is not None else self.dw_ws, bf16=bf16)
        tm.stop(phase)

    def _bias_corrections(self, step: int) -> tuple[float, float]:
        """torch.optim.Adam's 1 - b1^t and sqrt(1 - b2^t), in Python floats as torch computes them."""
        b1, b2 = self.alg.betas
        return 1 - b1 ** step, (1 - b2 ** step) ** 0.5

    def adam(self, step: int, prenorm: torch.Tensor | None = None) -> None:
        """Per-model clip + Adam over the flat buffers (prenorm: the norm partials of this mini-batch's weight-grad
        launch)."""
        alg = self.alg
        b1, b2 = alg.betas
        bc1, bc2_sqrt = self._bias_corrections(step)
        f = alg.flat
        tm = self.timer
        tm.start("adam")
        mirrors = self.w0_mirrors if prenorm is not None else None
        if alg.optim_kind == L.OPTIM_ADAM:
            ops.adam_step(f.param, f.grad, f.exp_avg, f.exp_avg_sq, f.group_begin, alg.max_grad_norm, b1, b2,
                          alg.adam_eps, bc1, bc2_sqrt, alg.device_state, self.adam_ws, prenorm=prenorm, mirrors=mirrors)
        else:  # AdamW / SGD / RMSprop: the same launches with their update rule
            s0 = None if alg.optim_kind == L.OPTIM_SGD else f.exp_avg
            s1 = f.exp_avg_sq if alg.optim_kind == L.OPTIM_ADAMW else None
            ops.optim_step(alg.optim_config, f.param, f.grad, s0, s1, f.group_begin, alg.max_grad_norm, bc1, bc2_sqrt,
                           alg.device_state, self.adam_ws, prenorm=prenorm, mirrors=mirrors)
        tm.stop("adam")

    def minibatch_rows(self, i: int) -> tuple[int, int]:
        return i * self.B // self.M, (i + 1) * self.B // self.M

    def discard_sizes(self) -> list[int]:
        """Elements of the Normal sample upstream's stochastic forward draws (and discards) in each mini-batch of an
        update, in its order: epoch after epoch, mini-batch after mini-batch, rows x actions."""
        sizes = [(r1 - r0) * self.A for r0, r1 in (self.minibatch_rows(i) for i in range(self.M))]
        return sizes * self.alg.num_learning_epochs

    # the feed-forward update has no device-side failure; the recurrent one overrides these
    can_fail = False

    def read_status(self) -> None:
        """Queue the read-back of device-side error words (none on the feed-forward path)."""

    def failure(self) -> str | None:
        """The error a read-back status word reports (after the stream was synchronised), else None."""
        return None

    def clear_status(self) -> None:
        """Reset the device-side error words after a failure was reported."""

    def run(self, perm: torch.Tensor, first_step: int, ready: int | None = None, rest=None) -> int:
        """All epochs x mini-batches.  Returns the number of optimiser steps taken.  With ``rest``, only
        ``perm[:ready]`` is final at the call: those rows are gathered first, and ``rest()`` (which completes
        ``perm``) is called once the first mini-batch is enqueued, before any row past ``ready`` is needed."""
        self._ensure_trace()
        sig = self._plan_signature()
        if sig != self._plan_key:
            self._plans.clear()
            self._plan_key = sig
        first = perm if rest is None else perm[:ready]

        def gather_first():
            self.timer.start("gather")
            self.gather(first)
            self.timer.stop("gather")

        self._issue(("gather", 0, None if perm is None else first.numel(), None if perm is None else perm.data_ptr()),
                    gather_first)
        if self.w0_mirrors:  # (then every Adam step of this run keeps the copies current)
            self.refresh_padded_weights()
            self._w0_current = True
        # (no clearing of the trace: the finalize of mini-batch i writes all 5 values of row i, and the host reads
        # back only the rows of this update's mini-batches)
        step = first_step
        try:
            for _ in range(self.alg.num_learning_epochs):
                for i in range(self.M):
                    r0, r1 = self.minibatch_rows(i)
                    if rest is not None and r1 > ready:
                        rest()
                        rest = None

                        def gather_rest():
                            self.timer.start("gather")
                            self.gather(perm[ready:], ready)
                            self.timer.stop("gather")

                        self._issue(("gather", ready, perm.numel() - ready, perm.data_ptr()), gather_rest)
                    step += 1
                    self._issue(("minibatch", r0, r1), lambda: self.minibatch(r0, r1, step), step)
                    if self.step_hook is not None:
                        self.step_hook(self, r0, r1)
        finally:
            self._frozen = False
            self._w0_current = False
        self._warm = True
        return step - first_step


class LstmBuffers:
    """Sequence buffers of one LSTM or GRU layer for mini-batches of up to ``rows`` = T x envs rows (t-major); the
    GRU's state h takes the place of the LSTM's cell state c."""

    def __init__(self, rnn, layer: int, rows: int, envs: int, device) -> None:
        H, D = rnn.hidden_size, rnn.layer_input_size(layer)
        self.layer = layer
        self.gru = rnn.gru
        e = lambda *shape: torch.empty(*shape, device=device)
        self.packed = ops.LstmPacked(D, H, device)
        self.gx, self.gates, self.dgates = e(rows, 4 * H), e(rows, 4 * H), e(rows, 4 * H)
        self.h, self.c, self.dh = e(rows, H), e(rows, H), e(rows, H)
        self.hs = e(rows + envs, H)  # the state entering each step, then h of the last step
        self.dc = e(envs, H)
        self.zero = torch.zeros(envs, H, device=device)
        self.dw_ih_g, self.dw_hh_g = e(4 * H, D), e(4 * H, H)
        self.db_g = e(4 * H)  # the gates' bias gradient (column sums of dgates), once for b_ih and b_hh


class RecurrentUpdateEngine(UpdateEngine):
    """The recurrent update (upstream ppo.py:204-236 with rollout_storage.py:262-331 and rnn.py:35-52), for LSTM and
    GRU models of one or more layers.

    Upstream splits each env's rollout at dones, pads the trajectories, runs nn.LSTM from the hidden state saved at
    each trajectory start and unpads.  Here every env of a mini-batch is ONE sequence of T steps started from the
    state saved at step 0, with the state multiplied by (1 - done) after each step: the state saved at a trajectory
    start after a done is exactly that zero (``reset(dones)`` zeroes it before the next step), so both give the same
    outputs on the same T x E valid steps.  Mini-batch i is the env slice [i N / M, (i + 1) N / M), all steps, the
    same slices every epoch (no permutation; the host generator is not drawn).  The packed table holds those rows
    t-major per slice, so a mini-batch is one contiguous row block and step t of it is E consecutive rows."""

    def __init__(self, alg) -> None:
        actor, critic = alg.actor, alg.critic
        if not (actor.is_recurrent and critic.is_recurrent):
            raise NotImplementedError("recurrent PPO on the HIP path needs a recurrent actor AND critic")
        st = alg.storage
        self.T, self.N = st.num_transitions_per_env, st.num_envs
        M = alg.num_mini_batches
        if not 1 <= M <= self.N:
            raise ValueError("num_mini_batches must be between 1 and the number of environments.")
        self.E_max = -(-self.N // M)
        super().__init__(alg)
        # the heads' weight-grads run on a second stream (default priority) beside the LSTM backward steps
        self.side = torch.cuda.Stream(device=self.device)
        self.side_dw_ws = ops.Workspace(self.device)
        # per layer, bottom first; seq_a / seq_c: the top layers, whose outputs feed the heads
        self.lay_a = [LstmBuffers(actor.rnn, k, self.R_max, self.E_max, self.device)
                      for k in range(actor.rnn.num_layers)]
        self.lay_c = [LstmBuffers(critic.rnn, k, self.R_max, self.E_max, self.device)
                      for k in range(critic.rnn.num_layers)]
        self.seq_a, self.seq_c = self.lay_a[-1], self.lay_c[-1]
        # synchronisation words of the one-launch sequences (word 0: sticky status, read back with every update);
        # PPO_HIP_LSTM_SEQ=0 selects one launch per step (same results)
        self.lstm_sync = None
        if os.environ.get("PPO_HIP_LSTM_SEQ", "1") != "0":
            self.lstm_sync = torch.zeros(ops.lstm_seq_sync_words(2, self.E_max), dtype=torch.int32,
                                         device=self.device)
            self._status_host = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        # one clip + optimiser launch (prenorm): the weight-grad launch of the recurrent layers and heads writes the
        # norm partials of the heads' gradients and the extra ranges, the gradient unpack adds the recurrent layers'.
        # Only with the one-launch sequences, where the heads' weight-grads share that launch
        self.rnn_norm = self._recurrent_norm_plan() if self.lstm_sync is not None else None
        # row order of the table: per env slice, t-major
        order = []
        idx = torch.arange(self.T * self.N).view(self.T, self.N)
        for i in range(M):
            e0, e1 = self.env_slice(i)
            order.append(idx[:, e0:e1].reshape(-1))
        self.order = torch.cat(order).to(self.device)

    recurrent = True

    def _recurrent_norm_plan(self) -> dict | None:
        """The clip norms from the weight-grad launch and the gradient unpack (one optimiser launch), when that one
        launch holds both weight-grads of every recurrent layer and every head layer, and the remaining gradients
        (the std parameter) fit as extra ranges; else None (the optimiser computes the norms itself)."""
        alg, f = self.alg, self.alg.flat
        la, lc = self._layers()
        n_rnn = len(self.lay_a) + len(self.lay_c)
        if 2 * n_rnn + len(la) + len(lc) > L.MAX_LINEAR_PROBLEMS or any(lin.bias is None for lin in (*la, *lc)):
            return None
        bounds = f.group_begin.tolist()
        if len(bounds) - 1 > L.MAX_PARAM_GROUPS:
            return None
        group = lambda off: max(i for i in range(len(bounds) - 1) if bounds[i] <= off)  # noqa: E731
        covered = {id(p) for lin in (*la, *lc) for p in (lin.weight, lin.bias)}
        rnn = {}
        for m, lays in ((alg.actor, self.lay_a), (alg.critic, self.lay_c)):
            for b in lays:
                ps = m.rnn.layer_weights(b.layer)
                covered |= {id(p) for p in ps}
                gs = {group(f.offsets[id(p)][0]) for p in ps}
                if len(gs) != 1:
                    return None
                rnn[id(b)] = gs.pop()
        extra = []
        for p in f.params:
            if id(p) not in covered and p.requires_grad:
                off, k = f.offsets[id(p)]
                extra.append((off, off + k, group(off)))
        if len(extra) > L.MAX_EXTRA_GRADS:
            return None
        head = [group(f.offsets[id(lin.weight)][0]) for lin in (*la, *lc)]
        return {"partials": ops.grad_norm_partials(self.device), "head": head, "extra": tuple(extra), "rnn": rnn}

    def max_rows(self) -> int:
        return self.T * self.E_max

    def env_slice(self, i: int) -> tuple[int, int]:
        return i * self.N // self.M, (i + 1) * self.N // self.M

    def minibatch_rows(self, i: int) -> tuple[int, int]:
        e0, e1 = self.env_slice(i)
        return self.T * e0, self.T * e1

    def gather(self, perm: torch.Tensor | None = None) -> None:
        super().gather(self.order if perm is None else perm)

    def segments(self) -> list[ops.Segment]:
        # keep = 1 - done of each row's step, converted from the stored uint8 dones by the gather itself
        return super().segments() + [ops.Segment(self.alg.storage.dones.reshape(-1, 1), self.layout.keep,
                                                 keep=True)]

    def _initial_state(self, side: str, e0: int, e1: int, buf: LstmBuffers):
        saved = getattr(self.alg.storage, f"saved_hidden_state_{side}")
        if saved is None:  # no state was recorded (a first rollout of one step): nn.LSTM's zero default
            return buf.zero[:e1 - e0], buf.zero[:e1 - e0]
        # [T, layers, N, H]: the state of this layer before step 0 (the GRU's h is also the kernels' c0)
        h0 = saved[0][0, buf.layer, e0:e1]
        return (h0, h0) if buf.gru else (h0, saved[1][0, buf.layer, e0:e1])

    def _seq(self, model, side: str, buf: LstmBuffers, e0: int, e1: int, tab: torch.Tensor) -> dict:
        R = self.T * (e1 - e0)
        h0, c0 = self._initial_state(side, e0, e1, buf)
        return dict(packed=buf.packed, hidden=model.rnn.hidden_size, gx=buf.gx[:R], h0=h0, c0=c0,
                    keep=tab[:, self.layout.keep], h=buf.h[:R], hs=buf.hs[:R + e1 - e0], c=buf.c[:R],
                    gates=buf.gates[:R], dh=buf.dh[:R], dgates=buf.dgates[:R], dc=buf.dc[:e1 - e0], gru=buf.gru)

    def dx_layers(self, R: int) -> list[tuple[int, list[tuple], bool]]:
        """As the feed-forward head's, plus layer 0: it has no activation below it, so a plain input-gradient into
        the LSTM outputs' gradient dh."""
        la, lc = self._layers()
        return super().dx_layers(R) + [(0, [(self.buf_a.dz[0][:R], la[0].weight, None, self.seq_a.dh[:R]),
                                            (self.buf_c.dz[0][:R], lc[0].weight, None, self.seq_c.dh[:R])], False,
                                        L.PPO_ACT_ELU)]

    @property
    def can_fail(self) -> bool:
        return self.lstm_sync is not None

    def read_status(self) -> None:
        if self.lstm_sync is not None:
            self._status_host.copy_(self.lstm_sync[:1], non_blocking=True)

    def failure(self) -> str | None:
        if self.lstm_sync is not None and int(self._status_host[0]) != 0:
            return ("LSTM sequence launch: blocks stopped waiting for each other (another whole-sequence launch "
                    "overlapped on this GPU?)")
        return None

    def clear_status(self) -> None:
        if self.lstm_sync is not None:
            self.lstm_sync.zero_()

    def _grouped(self, fn, qs: list[dict], E: int) -> None:
        """One launch for the actor's and the critic's sequences of one layer when their hidden sizes and cell types
        agree."""
        if len(qs) == 2 and qs[0]["hidden"] == qs[1]["hidden"] and qs[0]["gru"] == qs[1]["gru"]:
            fn(qs, self.T, E, self.lstm_sync)
        else:
            for q in qs:
                fn([q], self.T, E, self.lstm_sync)

    def _grouped_fwd(self, qs: list[dict], xs: list[torch.Tensor], E: int, bf16: bool) -> None:
        """The forward sequences of one layer with their input projections (x_i: problem i's layer input), grouped
        as _grouped groups them."""
        if len(qs) == 2 and qs[0]["hidden"] == qs[1]["hidden"] and qs[0]["gru"] == qs[1]["gru"]:
            ops.lstm_seq_fwd(qs, self.T, E, self.lstm_sync, proj=xs, bf16=bf16)
        else:
            for q, x in zip(qs, xs):
                ops.lstm_seq_fwd([q], self.T, E, self.lstm_sync, proj=[x], bf16=bf16)

    def _layer_inputs(self, xa: torch.Tensor, xc: torch.Tensor, R: int) -> list[list[tuple]]:
        """Per layer k (bottom first): (model, side, buffers, the layer's input rows) of each model that has layer k;
        layer 0 reads the observations, layer k > 0 the h of layer k - 1."""
        alg = self.alg
        out = []
        for k in range(max(len(self.lay_a), len(self.lay_c))):
            row = []
            for model, side, lays, x in ((alg.actor, "a", self.lay_a, xa), (alg.critic, "c", self.lay_c, xc)):
                if k < len(lays):
                    row.append((model, side, lays[k], x if k == 0 else lays[k - 1].h[:R]))
            out.append(row)
        return out

    def minibatch(self, r0: int, r1: int, step: int) -> None:
        alg, lay, tm = self.alg, self.layout, self.timer
        actor, critic = alg.actor, alg.critic
        R = r1 - r0
        E = R // self.T
        e0 = r0 // self.T
        tab = self.table[r0:r1]
        xa = tab[:, lay.xa:lay.xa + actor.obs_dim]
        xc = tab[:, lay.xc:lay.xc + critic.obs_dim]
        sa, sc = self.seq_a, self.seq_c
        adv_col = self.advantage_column(tab, R)

        # LSTM forward, layer after layer: packed weights, input projection for all T x E rows at once, then the T
        # recurrent steps
        tm.start("lstm_fwd")
        packs = [(m, b) for m, lays in ((actor, self.lay_a), (critic, self.lay_c)) for b in lays]
        for gru in (False, True):
            items = [(*m.rnn.layer_weights(b.layer), b.packed) for m, b in packs if b.gru == gru]
            if items:
                ops.lstm_pack(items, gru=gru)
        layers = self._layer_inputs(xa, xc, R)
        seqs = []
        for row in layers:
            # the input projection gx = x w_ih_g^T + b_g goes with the sequence call (inside the one-launch sequence
            # for narrow inputs, else its own launch first: the same values either way)
            qs = [self._seq(m, side, b, e0, e0 + E, tab) for m, side, b, _ in row]
            self._grouped_fwd(qs, [x for _, _, _, x in row], E, alg.use_mixed_precision)
            seqs.append(qs)
        tm.stop("lstm_fwd")

        self.head_forward(sa.h[:R], sc.h[:R], R)
        self.loss(tab, R, adv_col)
        self.head_backward(R)
        # the heads' weight gradients need only their dz and inputs.  Beside one launch per LSTM step they run on a
        # side stream (Adam waits for both); the whole-sequence backward keeps every CU's LDS for its whole run, so
        # there they join the LSTM weight gradients' grouped launch after it
        main = torch.cuda.current_stream()
        head_dw = self.head_dw(sa.h[:R], sc.h[:R], R)
        if self.lstm_sync is None:
            self.side.wait_stream(main)
            with torch.cuda.stream(self.side):
                self.weight_grads(head_dw, R, ws=self.side_dw_ws)
            head_dw = []
        # LSTM backward, top layer first: each layer's sequence, then the input-gradient of its projection into the
        # outputs' gradient dh of the layer below (no activation between the layers)
        tm.start("lstm_bwd")
        below = {"a": self.lay_a, "c": self.lay_c}
        for k in range(len(layers) - 1, -1, -1):
            self._grouped(ops.lstm_seq_bwd, seqs[k], E)
            if k > 0:
                ops.linear_bwd_dx([(b.dgates[:R], b.packed.w_ih_g, None, below[side][k - 1].dh[:R])
                                   for _, side, b, _ in layers[k]], R, self.dx_ws, bf16=alg.use_mixed_precision)
        tm.stop("lstm_bwd")

        dw = []
        for row in layers:
            for _, _, b, x in row:
                dw.append((b.dgates[:R], b.hs[:R], b.dw_hh_g, b.db_g))
                dw.append((b.dgates[:R], x, b.dw_ih_g, None))  # same operand dgates: its column sums once
        rn = self.rnn_norm
        norm = None if rn is None else ops.GradNorm(rn["partials"], [None] * len(dw) + rn["head"], alg.flat.grad,
                                                    rn["extra"])
        self.weight_grads(dw + head_dw, R, "lstm_dw", norm=norm)
        grad = alg.flat.grad_view
        for gru in (False, True):
            sel = [(m, b) for m, b in packs if b.gru == gru]
            items = [(b.dw_ih_g, b.dw_hh_g, b.db_g, *(grad(p) for p in m.rnn.layer_weights(b.layer))) for m, b in sel]
            if items:
                ops.lstm_unpack_grads(items, gru=gru,
                                      norm=None if rn is None else (rn["partials"], [rn["rnn"][id(b)] for _, b in sel]))
        if self.lstm_sync is None:
            main.wait_stream(self.side)
        self.adam(step, prenorm=None if rn is None else rn["partials"])
