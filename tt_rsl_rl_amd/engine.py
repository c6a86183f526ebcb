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

import torch

from . import _lib as L
from . import ops


def _align4(n: int) -> int:
    return (n + 3) // 4 * 4


class TableLayout:
    def __init__(self, actor_dim: int, critic_dim: int, num_actions: int) -> None:
        c = 0
        self.xa = c
        c = _align4(c + actor_dim)
        self.xc = c
        c = _align4(c + critic_dim)
        self.actions = c
        c = _align4(c + num_actions)
        self.old_mean = c
        c = _align4(c + num_actions)
        self.old_std = c
        c = _align4(c + num_actions)
        self.old_logp, self.adv, self.old_values, self.returns, self.adv_mb = c, c + 1, c + 2, c + 3, c + 4
        self.width = _align4(c + 5)


class ModelBuffers:
    """Activation and gradient buffers of one MLP for mini-batches of up to `rows` rows.  Rows are padded to a
    multiple of 4 floats (views keep the logical width) so every buffer can be read with 16-byte loads."""

    def __init__(self, model, rows: int, device) -> None:
        lin = model.linears
        self.widths = [l.out_features for l in lin]

        def buf(w: int) -> torch.Tensor:
            return torch.empty(rows, -(-w // 4) * 4, device=device)[:, :w]

        self.out = buf(self.widths[-1])                 # output layer (no activation): mean / value
        self.h = [buf(w) for w in self.widths[:-1]]     # hidden layers keep only elu(z); ELU' is taken from it
        self.dz = [buf(w) for w in self.widths]


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


class UpdateEngine:
    """Owns the device workspaces of the update and runs it.  Rebuilt when the rollout shape changes."""

    def __init__(self, alg) -> None:
        self.alg = alg
        self.timer = _NoTimer()
        self.device = alg.device
        st = alg.storage
        self.B = st.batch_size
        self.M = alg.num_mini_batches
        if not 1 <= self.M <= self.B:
            raise ValueError("num_mini_batches must be between 1 and the rollout batch size.")
        self.R_max = -(-self.B // self.M)
        actor, critic = alg.actor, alg.critic
        self.A = actor.distribution.output_dim
        self.layout = TableLayout(actor.obs_dim, critic.obs_dim, self.A)
        self.table = torch.empty(self.B, self.layout.width, device=self.device)
        self.buf_a = ModelBuffers(actor, self.R_max, self.device)
        self.buf_c = ModelBuffers(critic, self.R_max, self.device)
        self.loss_ws = torch.empty(ops.loss_workspace_bytes(self.R_max, self.A), dtype=torch.uint8, device=self.device)
        self.dw_ws = ops.Workspace(self.device)
        self.adam_ws = ops.Workspace(self.device)
        self.dx_ws = ops.Workspace(self.device)
        self.adv_ws = ops.Workspace(self.device)
        self.trace = torch.zeros(5 * alg.num_learning_epochs * self.M, dtype=torch.float64, device=self.device)

    # -- one update ------------------------------------------------------------------------------------------------
    def gather(self, perm: torch.Tensor) -> None:
        alg, st, lay = self.alg, self.alg.storage, self.layout
        segs: list[ops.Segment] = []
        for model, base in ((alg.actor, lay.xa), (alg.critic, lay.xc)):
            col = 0
            norm = model.obs_normalizer if model.obs_normalization else None
            for g in model.obs_groups:
                src = st.flat(st.observations[g])
                w = src.shape[1]
                if norm is not None:
                    segs.append(ops.Segment(src, base + col, norm._mean.view(-1)[col:col + w],
                                            norm._std.view(-1)[col:col + w], norm.eps))
                else:
                    segs.append(ops.Segment(src, base + col))
                col += w
        mean, std = st.distribution_params
        segs += [ops.Segment(st.flat(st.actions), lay.actions), ops.Segment(st.flat(mean), lay.old_mean),
                 ops.Segment(st.flat(std), lay.old_std), ops.Segment(st.flat(st.actions_log_prob), lay.old_logp),
                 ops.Segment(st.flat(st.advantages), lay.adv), ops.Segment(st.flat(st.values), lay.old_values),
                 ops.Segment(st.flat(st.returns), lay.returns)]
        for i in range(0, len(segs), L.MAX_GATHER_SEGMENTS):
            ops.gather_rows(perm, segs[i:i + L.MAX_GATHER_SEGMENTS], self.table)

    def minibatch(self, r0: int, r1: int, step: int) -> None:
        alg, lay = self.alg, self.layout
        R = r1 - r0
        tab = self.table[r0:r1]
        actor, critic = alg.actor, alg.critic
        la, lc = actor.linears, critic.linears
        ba, bc = self.buf_a, self.buf_c
        nl = len(la)
        if len(lc) != nl:
            raise NotImplementedError("actor and critic must have the same number of layers")
        xa = tab[:, lay.xa:lay.xa + actor.obs_dim]
        xc = tab[:, lay.xc:lay.xc + critic.obs_dim]

        adv_col = lay.adv
        if alg.normalize_advantage_per_mini_batch and R > 1:
            ops.adv_normalize(tab[:, lay.adv], tab[:, lay.adv_mb], R, in_stride=lay.width, out_stride=lay.width,
                              ws=self.adv_ws)
            adv_col = lay.adv_mb

        # forward, actor and critic grouped layer by layer
        tm = self.timer
        ins_a, ins_c = [xa], [xc]
        for i in range(nl):
            last = i == nl - 1
            probs = [(ins_a[-1], la[i].weight, la[i].bias, ba.out[:R] if last else None, None if last else ba.h[i][:R]),
                     (ins_c[-1], lc[i].weight, lc[i].bias, bc.out[:R] if last else None, None if last else bc.h[i][:R])]
            tm.start(f"fwd{i}")
            ops.linear_fwd(probs, R, elu=not last)
            tm.stop(f"fwd{i}")
            if not last:
                ins_a.append(ba.h[i][:R])
                ins_c.append(bc.h[i][:R])

        # losses + per-row gradients, then the device-side reduction / LR rule / std-parameter gradient
        dist = actor.distribution
        lo, hi = dist.param_range
        batch = {"ld": lay.width, "actions": tab[:, lay.actions], "old_mean": tab[:, lay.old_mean],
                 "old_std": tab[:, lay.old_std], "old_logp": tab[:, lay.old_logp], "advantages": tab[:, adv_col],
                 "old_values": tab[:, lay.old_values], "returns": tab[:, lay.returns]}
        args = ops.make_loss_args(R, ba.out[:R], bc.out[:R, 0], batch, dist.param, dist.kernel_std_type, lo, hi,
                                  alg.clip_param, alg.value_loss_coef, alg.entropy_coef, alg.use_clipped_value_loss,
                                  ba.dz[-1][:R], bc.dz[-1][:R, 0])
        tm.start("loss")
        ops.ppo_loss(args, self.loss_ws)
        adaptive = alg.desired_kl is not None and alg.schedule == "adaptive"
        ops.ppo_loss_finalize(args, self.loss_ws, alg.flat.grad_view(dist.param), alg.device_state, adaptive,
                              alg.desired_kl if alg.desired_kl is not None else 0.0, self.trace)
        tm.stop("loss")

        # backward: input gradients down the chain (grouped), then every weight gradient in one launch
        for i in range(nl - 1, 0, -1):
            tm.start(f"dx{i}")
            ops.linear_bwd_dx([(ba.dz[i][:R], la[i].weight, ba.h[i - 1][:R], ba.dz[i - 1][:R]),
                               (bc.dz[i][:R], lc[i].weight, bc.h[i - 1][:R], bc.dz[i - 1][:R])], R, self.dx_ws,
                              elu_from_output=True)
            tm.stop(f"dx{i}")
        dw = []
        for model, buf, lins, x0 in ((actor, ba, la, xa), (critic, bc, lc, xc)):
            for i in range(nl):
                x = x0 if i == 0 else buf.h[i - 1][:R]
                dw.append((buf.dz[i][:R], x, alg.flat.grad_view(lins[i].weight), alg.flat.grad_view(lins[i].bias)))
        tm.start("dw")
        ops.linear_bwd_dw(dw, R, self.dw_ws)
        tm.stop("dw")

        # per-model clip + Adam over the flat buffers
        b1, b2 = alg.betas
        bc1 = 1 - b1 ** step
        bc2_sqrt = (1 - b2 ** step) ** 0.5
        f = alg.flat
        tm.start("adam")
        ops.adam_step(f.param, f.grad, f.exp_avg, f.exp_avg_sq, f.group_begin, alg.max_grad_norm, b1, b2, alg.adam_eps,
                      bc1, bc2_sqrt, alg.device_state, self.adam_ws)
        tm.stop("adam")

    def run(self, perm: torch.Tensor, first_step: int) -> int:
        """All epochs x mini-batches.  Returns the number of optimiser steps taken."""
        self.timer.start("gather")
        self.gather(perm)
        self.timer.stop("gather")
        self.trace.zero_()
        step = first_step
        for _ in range(self.alg.num_learning_epochs):
            for i in range(self.M):
                r0 = i * self.B // self.M
                r1 = (i + 1) * self.B // self.M
                step += 1
                self.minibatch(r0, r1, step)
        return step - first_step
