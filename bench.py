#!/usr/bin/env python3
"""PPO update throughput on one MI355X: samples/s and ms per update (fwd + bwd + Adam over all epochs).

Workload (default): the humanoid-scale update -- actor obs 96 -> [512, 256, 128] ELU -> 29 actions, critic obs 99
-> [512, 256, 128] ELU -> 1, observation normalisation, 4096 envs x 24 steps, 5 epochs x 4 mini-batches.
A synthetic rollout (obs ~ N(0,1), rewards ~ N(0, 0.2^2), dones ~ Bernoulli(0.01), actions sampled from the
policy) is collected once with the plugin's own act() on the GPU, returns are computed, and then `--steps` updates
are timed on the resident rollout (each update = one step; inputs already in HBM).

Prints ONE JSON line.  Alongside the GPU figure it reports:
  * roofline: the dominant kernel's algorithmic FLOP rate (HIP events on the launch stream, timed region) against
    its MFMA ceiling (bf16x6 kernel: the dense bf16 MFMA peak over six; fp32-MFMA kernel: the fp32 MFMA peak), and
    the HBM traffic per launch measured with rocprofv3 counters (profiles/, else null);
  * cpu_baseline: the CPU oracle's update() on this host's cores on the same workload (a bounded sample).
"""

from __future__ import annotations

import argparse
import gc
import json
import os
import statistics
import sys
import time
from pathlib import Path
from types import SimpleNamespace

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "PPO update samples/s (fwd+bwd+Adam) and ms/update at 4096 envs×24 steps, 1 GPU"
PEAK_FP32_MFMA_TFLOPS = 157.3
# The bf16x6 GEMMs compute each fp32 product from six bf16 MFMA products of the operands' three-part splits: their
# ceiling, in algorithmic fp32 FLOP/s, is the dense bf16 MFMA peak (2.5 PFLOP/s) over six.
PEAK_BF16_MFMA_TFLOPS = 2500.0
PEAK_BX6_TFLOPS = PEAK_BF16_MFMA_TFLOPS / 6
PEAK_HBM_GBS = 8000.0


def dw_arith(engine, R: int) -> str:
    """Arithmetic of the weight-grad launch: the bf16x6 kernel runs when every problem's operands (dz and the layer
    input) have 16-byte aligned rows, else the fp32-MFMA kernel (the library's own rule, restated on the operands the
    engine passes)."""
    tab = engine.table[:R]
    lay = engine.layout
    alg = engine.alg
    xa = tab[:, lay.xa:lay.xa + alg.actor.obs_dim]
    xc = tab[:, lay.xc:lay.xc + alg.critic.obs_dim]
    if engine.recurrent:
        ops = [(b.dgates[:R], h) for row in engine._layer_inputs(xa, xc, R) for _, _, b, x in row
               for h in (b.hs[:R], x)]
        if engine.lstm_sync is not None:
            ops += [(dz, x) for dz, x, *_ in engine.head_dw(engine.seq_a.h[:R], engine.seq_c.h[:R], R)]
    else:
        ops = [(dz, x) for dz, x, *_ in engine.head_dw(xa, xc, R)]
    aligned = all(t.data_ptr() % 16 == 0 and t.stride(0) % 4 == 0 for pair in ops for t in pair)
    return "bf16x6" if aligned else "fp32"


def _sample_obs(workload, n, device, gen):
    import torch

    out = {}
    for name, (kind, width) in workload["obs"].items():
        if kind == "normal":
            out[name] = torch.randn(n, width, device=device, generator=gen)
        else:
            out[name] = torch.rand(n, width, device=device, generator=gen) * 2.0 - 1.0
    return out


def build_gpu_alg(workload, seed: int = 0, mixed_precision: bool = False):
    """Construct the plugin the way upstream's runner does and collect one synthetic rollout on the GPU."""
    import torch

    from tt_rsl_rl_amd import workloads as W
    from tt_rsl_rl_amd.ppo import PPO

    dev = torch.device("cuda:0")
    torch.manual_seed(seed)
    cfg = W.train_cfg(workload, **({"use_mixed_precision": True} if mixed_precision else {}))
    env = SimpleNamespace(num_envs=workload["num_envs"], num_actions=workload["num_actions"])
    n = workload["num_envs"]
    obs0 = {k: torch.zeros(n, w) for k, (_, w) in workload["obs"].items()}
    alg = PPO.construct_algorithm(obs0, env, cfg, str(dev))
    alg.train_mode()
    gen = torch.Generator(device=dev).manual_seed(seed)
    rollout_ms = []
    with torch.inference_mode():
        for _ in range(2):  # the second rollout is timed (act + process_env_step per env step) and kept
            alg.storage.clear()
            obs = _sample_obs(workload, n, dev, gen)
            env_s = [_sample_obs(workload, n, dev, gen) for _ in range(workload["steps"])]
            rewards = workload["reward_std"] * torch.randn(workload["steps"], n, device=dev, generator=gen)
            dones = (torch.rand(workload["steps"], n, device=dev, generator=gen) < workload["p_done"]).float()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for t in range(workload["steps"]):
                alg.act(obs)
                obs = env_s[t]
                alg.process_env_step(obs, rewards[t], dones[t], {})
            torch.cuda.synchronize()
            rollout_ms.append((time.perf_counter() - t0) / workload["steps"] * 1e3)
        alg.compute_returns(obs)
    torch.cuda.synchronize()
    alg.bench_rollout_ms = rollout_ms[-1]
    alg.bench_last_obs = obs
    return alg


def phase_flops(workload, R: int) -> dict[str, float]:
    """Algorithmic FLOPs of one launch of each GEMM phase (both models share a launch)."""
    from tt_rsl_rl_amd import workloads as W

    shapes = W.linear_shapes(workload)
    nl = len(shapes[0])
    out = {}
    for i in range(nl):
        out[f"fwd{i}"] = sum(2.0 * R * s[i][0] * s[i][1] for s in shapes)
    for i in range(1, nl):
        out[f"dx{i}"] = sum(2.0 * R * s[i][0] * s[i][1] for s in shapes)
    out["dw"] = sum(2.0 * R * i_ * o_ for s in shapes for i_, o_ in s)
    # the fused head: the output layers' forward and input-grad (with the loss) in one launch
    out["head"] = out[f"fwd{nl - 1}"] + out[f"dx{nl - 1}"]
    if "rnn" in workload:
        # recurrent: R = T x E rows; one LSTM (hidden H on D observation columns) before each head
        H = workload["rnn"]["rnn_hidden_dim"]
        E = R // workload["steps"]
        dims = [sum(workload["obs"][g][1] for g in workload["obs_groups"][m]) for m in ("actor", "critic")]
        out["dx0"] = sum(2.0 * R * s[0][0] * s[0][1] for s in shapes)
        out["lstm_fwd"] = sum(2.0 * R * 4 * H * (D + H) for D in dims)   # input projection + T recurrent steps
        out["lstm_bwd"] = sum(2.0 * (R - E) * 4 * H * H for _ in dims)    # recurrent input-grad, T - 1 steps
        out["lstm_dw"] = sum(2.0 * R * 4 * H * (D + H) for D in dims)
    return out


def graph_ms(fn, reps: int = 50) -> float:
    """Mean GPU time of fn's launches: `reps` calls captured in one HIP graph (kernels only) and replayed, so the
    host's launch overhead is not in the measurement."""
    import torch

    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    del graph
    return e0.elapsed_time(e1) / reps


def hbm_kernels(alg, engine, phases, workload, R: int) -> dict:
    """Achieved bandwidth of the HBM-bound kernels against the 8 TB/s peak: algorithmic bytes per launch / mean launch
    time.  GAE, the permutation gather and clip + Adam are timed standalone on the resident data by HIP-graph replay
    (this runs after the timed updates; Adam steps the parameters further); the loss (+ finalize) time is the
    instrumented pass's HIP events."""
    import torch

    from tt_rsl_rl_amd import ops

    st = alg.storage
    T, N = st.num_transitions_per_env, st.num_envs
    B = T * N
    A = workload["num_actions"]
    ka, kc = alg.actor.linears[-1].in_features, alg.critic.linears[-1].in_features
    # the rows' algorithmic floats: every observation group once, actions, old mean, the four per-transition scalars
    # (the state-independent std counts once per rollout); the kernel copies every segment it is given, the std and
    # the 16-byte padding of the action records included
    groups = {g for m in (alg.actor, alg.critic) for g in m.obs_groups}
    width = sum(st.observations[g].shape[-1] for g in groups) + 2 * A + 4
    copied = sum(seg.src.shape[1] for seg in engine.segments())
    nbytes = {
        "gather": B * (2 * 4 * width + 8),                        # every float read + written once, int64 index
        "loss": R * 4 * (4 * A + 6) + R * 4 * (A + 1),            # per-row inputs + per-row output gradients
        # fused head: last hidden activations in, their gradients out, batch columns in, mean / value and their
        # gradients out
        "head": R * 4 * (2 * (ka + kc) + 3 * A + 4 + 2 * (A + 1)),
        # p, g, m, v read and written (+ a 4 B norm pass without the weight-grad launch's norm partials)
        "adam": alg.flat.param.numel() * (32 if engine.grad_norm is not None else 36),
        "gae": B * (4 + 4 + 1 + 4 + 4) + 4 * N,                   # r, V, done in; returns, advantages out
    }
    last = torch.randn(N, 1, device=alg.device)
    rets, advs = torch.empty_like(st.returns), torch.empty_like(st.advantages)
    perm = torch.randperm(B).to(alg.device)
    f = alg.flat
    b1, b2 = alg.betas
    ms = {
        "gae": graph_ms(lambda: ops.gae(st.rewards, st.values, st.dones, last, rets, advs, alg.gamma, alg.lam)),
        "gather": graph_ms(lambda: engine.gather(perm)),
        "adam": graph_ms(lambda: ops.adam_step(f.param, f.grad, f.exp_avg, f.exp_avg_sq, f.group_begin,
                                               alg.max_grad_norm, b1, b2, alg.adam_eps, 0.5, 0.5, alg.device_state,
                                               engine.adam_ws, prenorm=None if engine.grad_norm is None
                                               else engine.grad_norm.partials)),
    }
    for k in ("loss", "head"):
        if k in phases:
            ms[k] = phases[k][1]
    out = {}
    for k, b in nbytes.items():
        if k in ms:
            gbs = b / (ms[k] * 1e-3) / 1e9
            out[k] = {"bytes": b, "mean_us": round(ms[k] * 1e3, 2), "GB/s": round(gbs, 1),
                      "frac": round(gbs / PEAK_HBM_GBS, 4)}
    if "gather" in out:
        out["gather"]["row_floats"] = width
        out["gather"]["copied_bytes"] = B * (2 * 4 * copied + 8)
    # Single-launch floor at these sizes: one plain streaming kernel (torch's elementwise y = x * 1, half the bytes
    # read, half written) moving the same bytes as the kernel, and an empty launch (one element), both by graph replay
    empty = torch.ones(1, device=alg.device)
    out["floor"] = {"empty_launch_us": round(graph_ms(lambda: torch.mul(empty, 1.0, out=empty)) * 1e3, 2)}
    for k in ("gae", "adam", "gather"):
        n = max(1, (out["gather"]["copied_bytes"] if k == "gather" else nbytes[k]) // 8)
        x, y = torch.ones(n, device=alg.device), torch.empty(n, device=alg.device)
        us = graph_ms(lambda: torch.mul(x, 1.0, out=y)) * 1e3
        gbs = 8 * n / (us * 1e-6) / 1e9
        out["floor"][k] = {"copy_bytes": 8 * n, "copy_us": round(us, 2), "GB/s": round(gbs, 1),
                           "frac": round(gbs / PEAK_HBM_GBS, 4)}
        del x, y
    return out


def load_traffic(workload_name: str, kernel_phase: str):
    """HBM bytes per launch of the dominant kernel from the workload's committed rocprofv3 counter summary
    (profiles/traffic_<workload>.json), else None."""
    p = ROOT / "profiles" / f"traffic_{workload_name}.json"
    if not p.exists():
        return None
    try:
        d = json.loads(p.read_text())
        return d.get(kernel_phase)
    except (OSError, ValueError):
        return None


def cpu_baseline(workload, reps: int) -> dict:
    """The oracle (upstream's update restated in CPU torch) on this host's cores, same workload, same statistics."""
    import torch

    from oracle import rollout as R

    threads = torch.get_num_threads()
    ora, roll = R.generate(workload, seed=0)
    with torch.inference_mode():  # as upstream's runner collects (the recurrent states are inference tensors)
        ora.compute_returns(roll.last_obs)
    B = workload["num_envs"] * workload["steps"]
    steps_total = ora.num_learning_epochs * ora.num_mini_batches
    # Bounded sample: above ~100k transitions a whole CPU update takes minutes, so only the first `k` mini-batch
    # steps (plus the observation-normaliser update) are timed and scaled to the update's steps.
    k = steps_total if B <= 100_000 else 2
    ora.max_steps = k if k < steps_total else None
    times = []
    for i in range(reps + 1):
        ora.storage.step = ora.storage.num_transitions_per_env
        torch.manual_seed(1)
        t0 = time.perf_counter()
        ora.update()
        dt = time.perf_counter() - t0
        if i > 0:
            times.append(dt * steps_total / k)
    med = statistics.median(times)
    scope = ("the whole update" if k == steps_total else
             f"the first {k} of its {steps_total} mini-batch steps, scaled by {steps_total}/{k}")
    return {"value": B / med, "unit": "samples/s", "cores": threads, "kind": "port",
            "sample": f"oracle PPO.update (upstream restated in CPU torch) on the same workload, {scope}; median of "
                      f"{reps} after 1 warm-up, {threads} torch threads, cpu_count={os.cpu_count()}",
            "cpu_model": cpu_model(), "ms_per_update": med * 1e3}


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or "unknown"."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


class FenceFreeTimer:
    """The engine's phase-timer interface (start / stop / summary / reset) on HIP events created with
    hipEventDisableSystemFence, recorded on the stream the kernels use.  Such events only time: recording one skips
    the system-scope cache write-back and invalidate that a default event performs, which otherwise adds a few
    microseconds of idle GPU before and after every timed launch.  Read only after a device synchronisation.
    `every`: events around every every-th occurrence of a phase (the phase's launches are identical from mini-batch
    to mini-batch; each event pair still leaves ~2 us of idle GPU around its launch)."""

    FLAGS = 0x20000000  # hipEventDisableSystemFence (hip_runtime_api.h)

    def __init__(self, only: set[str], every: int = 1) -> None:
        import ctypes

        import torch
        from tt_rsl_rl_amd import _lib

        self.ct, self.torch = ctypes, torch
        self.hip = _lib.load()  # dlsym through libppo_hip.so reaches the HIP runtime it (and torch) already loaded
        self.hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.only, self.enabled, self.every = only, True, max(1, every)
        self._seen: dict[str, int] = {}
        self.events: dict[str, list[tuple[int, int]]] = {}
        self._open: dict[str, int] = {}
        self._pool: list[int] = []

    def _record(self) -> int:
        ev = self._pool.pop() if self._pool else None
        if ev is None:
            h = self.ct.c_void_p()
            if self.hip.hipEventCreateWithFlags(self.ct.byref(h), self.FLAGS) != 0:
                raise RuntimeError("hipEventCreateWithFlags failed")
            ev = h.value
        if self.hip.hipEventRecord(ev, self.torch.cuda.current_stream().cuda_stream) != 0:
            raise RuntimeError("hipEventRecord failed")
        return ev

    def start(self, name: str) -> None:
        if self.enabled and name in self.only:
            k = self._seen.get(name, 0)
            self._seen[name] = k + 1
            if k % self.every == 0:
                self._open[name] = self._record()

    def stop(self, name: str) -> None:
        if name in self._open:
            self.events.setdefault(name, []).append((self._open.pop(name), self._record()))

    def reset(self) -> None:
        for pairs in self.events.values():
            for a, b in pairs:
                self._pool += [a, b]
        self.events.clear()
        self._open.clear()
        self._seen.clear()

    def summary(self) -> dict[str, tuple[int, float]]:
        out = {}
        for k, pairs in self.events.items():
            tot = 0.0
            for a, b in pairs:
                ms = self.ct.c_float()
                if self.hip.hipEventElapsedTime(self.ct.byref(ms), a, b) != 0:
                    raise RuntimeError("hipEventElapsedTime failed")
                tot += ms.value
            out[k] = (len(pairs), tot / len(pairs))
        return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="humanoid")
    ap.add_argument("--cpu-baseline", choices=("on", "off"), default="on")
    ap.add_argument("--cpu-reps", type=int, default=None,
                    help="timed oracle updates for cpu_baseline (default 3; 1 for recurrent workloads)")
    ap.add_argument("--no-phase-events", action="store_true", help="do not record per-launch HIP events")
    ap.add_argument("--mixed-precision", action="store_true",
                    help="upstream's use_mixed_precision: the layers' GEMMs with bf16 operands (not the default "
                         "configuration: a separate line, dtype bf16)")
    ap.add_argument("--census", type=int, default=None, metavar="N",
                    help="only collect the rollout and run N updates (no timing; for a kernel census under rocprofv3: "
                         "the kernels of N updates = this run's minus the run with N = 0)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB (counter calibration) and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch

        n = args.copy_calibration * (1 << 20) // 4
        x = torch.ones(n, device="cuda")
        y = torch.empty_like(x)
        torch.cuda.synchronize()
        y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": 4 * n}))
        return 0

    if args.gpus != 1:
        print(f"bench.py: this build runs the PPO update on ONE GPU; --gpus {args.gpus} is not supported "
              "(multi-GPU data parallelism is not implemented)", file=sys.stderr)
        return 2

    import torch

    from tt_rsl_rl_amd import workloads as W
    from tt_rsl_rl_amd.engine import PhaseTimer

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 2
    workload = W.WORKLOADS[args.workload]
    alg = build_gpu_alg(workload, mixed_precision=args.mixed_precision)
    B = workload["num_envs"] * workload["steps"]
    M = alg.num_mini_batches
    R = B // M if "rnn" not in workload else workload["steps"] * (workload["num_envs"] // M)

    def one_update():
        alg.storage.step = alg.storage.num_transitions_per_env
        torch.manual_seed(1)
        return alg.update()

    if args.census is not None:
        torch.cuda.synchronize()
        for _ in range(args.census):
            one_update()
        torch.cuda.synchronize()
        print(json.dumps({"census_updates": args.census, "workload": args.workload}))
        return 0

    for _ in range(args.warmup):
        one_update()
    engine = alg._engine
    flops = phase_flops(workload, R)

    # Untimed instrumented pass: HIP events around every launch group, for the per-phase breakdown and to find
    # the dominant GEMM kernel.
    full = PhaseTimer()
    engine.timer = full
    for _ in range(2):
        one_update()
    torch.cuda.synchronize()
    phases = full.summary()
    if "lstm_dw" in phases and "dw" not in phases:
        flops["lstm_dw"] += flops["dw"]  # the heads' weight-grads share the LSTM weight-grads' launch
    total_ms = {k: n * t for k, (n, t) in phases.items()}
    phase_report = {}
    for k, (n, t) in phases.items():
        entry = {"launches": n, "mean_ms": round(t, 5)}
        if k in flops:
            entry["tflops"] = round(flops[k] / (t * 1e-3) / 1e12, 2)
        phase_report[k] = entry
    gemm_phases = [k for k in phases if k in flops and k != "head"]  # the fused head is HBM-bound
    dom = max(gemm_phases, key=lambda k: total_ms[k])

    # Timed region: events only around the dominant kernel's launches (on the stream the kernels use).  The Python heap
    # is collected and frozen first, so a collection of the objects built so far does not land inside it.  The GPU
    # idles through that collection and comes back at a lower clock: one more untimed update restores its working
    # clock (without it the first timed update took 16.2 ms against 13.9 for the rest).
    timer = FenceFreeTimer(only={dom}, every=4)
    timer.enabled = not args.no_phase_events
    engine.timer = timer
    gc.collect()
    gc.freeze()
    one_update()
    torch.cuda.synchronize()
    timer.reset()
    t0 = time.perf_counter()
    per = []
    for _ in range(args.steps):
        s0 = time.perf_counter()
        losses = one_update()
        per.append(time.perf_counter() - s0)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = elapsed / args.steps * 1e3
    value = B / (elapsed / args.steps)

    roofline = None
    if timer.enabled:
        n, t = timer.summary()[dom]
        ach = flops[dom] / (t * 1e-3) / 1e12
        arith = dw_arith(engine, R) if dom in ("dw", "lstm_dw") else "fp32"
        if arith == "bf16x6" and args.mixed_precision:
            arith = "bf16"  # (the same kernels at one bf16 product per k-group)
        peak = {"bf16x6": PEAK_BX6_TFLOPS, "bf16": PEAK_BF16_MFMA_TFLOPS}.get(arith, PEAK_FP32_MFMA_TFLOPS)
        roofline = {"bound": "mfma", "achieved": round(ach, 2), "peak": round(peak, 2), "unit": "TFLOP/s",
                    "frac": round(ach / peak, 4), "traffic": load_traffic(args.workload, dom), "kernel": dom,
                    "arith": arith, "peak_basis": {"bf16x6": "bf16 dense MFMA 2.5 PFLOP/s / 6 products per fp32 "
                                                             "product", "bf16": "bf16 dense MFMA 2.5 PFLOP/s"}.get(
                                                       arith, "fp32 dense MFMA"),
                    "frac_of_fp32_mfma_peak": round(ach / PEAK_FP32_MFMA_TFLOPS, 4),
                    "flops_per_launch": flops[dom], "mean_launch_ms": round(t, 5), "launches_timed": n}
    # compute_returns() (bootstrap critic forward, GAE, advantage normalisation) on the stored rollout, timed after
    # the updates (it rewrites the same returns / advantages each call), as the runner calls it: in inference mode
    cr = []
    with torch.inference_mode():
        for i in range(12):
            torch.cuda.synchronize()
            s0 = time.perf_counter()
            alg.compute_returns(alg.bench_last_obs)
            torch.cuda.synchronize()
            if i >= 2:
                cr.append(time.perf_counter() - s0)
    cr_ms = statistics.median(cr) * 1e3
    hbm = hbm_kernels(alg, engine, phases, workload, R)
    gemm_total = W.gemm_flops_per_update(workload, alg.num_learning_epochs)
    lstm = ""
    if "rnn" in workload:
        lstm = (f"LSTM {workload['rnn']['rnn_hidden_dim']} on the observations (sequences of {workload['steps']} "
                f"steps per env, env-slice mini-batches), then ")

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "samples/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16" if args.mixed_precision else "fp32", "data": "synthetic",
        "gemm_arith": ("use_mixed_precision: the layers' GEMMs with bf16 operands (rounded to nearest even), one bf16 "
                       "MFMA product, fp32 accumulation and results; loss, head and optimiser in fp32"
                       if args.mixed_precision else
                       "fp32 operands and results; GEMMs with 16-byte aligned operand rows as bf16x6 (three bf16 "
                       "parts per operand, six bf16 MFMA products, fp32 accumulation), the rest on fp32 MFMA"),
        "config": {"workload": f"{args.workload}: {lstm}{len(W.linear_shapes(workload)[0])}-layer actor/critic MLPs "
                               f"{W.linear_shapes(workload)}, {workload['num_envs']} envs x {workload['steps']} steps, "
                               f"{alg.num_learning_epochs} epochs x {M} mini-batches of {R} rows, "
                               f"obs normalisation {workload['obs_normalization']}",
                   "num_envs": workload["num_envs"], "steps_per_env": workload["steps"], "mini_batch_rows": R,
                   "parallelism": "single GPU"},
        "ms_per_update_median": round(statistics.median(per) * 1e3, 3),
        "ms_per_update_min_p90_max": [round(min(per) * 1e3, 3), round(sorted(per)[int(0.9 * (len(per) - 1))] * 1e3, 3),
                                      round(max(per) * 1e3, 3)],
        "sample_visits_per_s": round(value * alg.num_learning_epochs, 1),
        "compute_returns_ms_median": round(cr_ms, 3),
        "compute_returns_plus_update_ms": round(cr_ms + statistics.median(per) * 1e3, 3),
        "update_gemm_tflops": round(gemm_total / (ms * 1e-3) / 1e12, 2),
        "update_gemm_frac_of_fp32_mfma_peak": round(gemm_total / (ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4),
        "update_gemm_frac_of_bf16x6_peak": round(gemm_total / (ms * 1e-3) / 1e12 / PEAK_BX6_TFLOPS, 4),
        "phases": phase_report,
        "roofline": roofline,
        "hbm_kernels": hbm,
        "rollout": {"ms_per_env_step": round(alg.bench_rollout_ms, 4),
                    "transitions_per_s": round(workload["num_envs"] / (alg.bench_rollout_ms * 1e-3), 1),
                    "note": "act() + process_env_step() for all envs, observations already on the GPU"},
        "losses": losses,
        "cpu_baseline": None,
    }
    if args.cpu_baseline == "on":
        reps = args.cpu_reps if args.cpu_reps is not None else (1 if "rnn" in workload else 3)
        line["cpu_baseline"] = cpu_baseline(workload, reps)
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
