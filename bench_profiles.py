"""Summaries of rocprofv3 runs of bench.py for profiles/ (text a few KB long; the raw output stays where the profiler
wrote it).  Every summary names the commands that made it; they run bench.py and this file only.

usage (repository root; D = the directory the rocprofv3 runs wrote into, one sub-directory per run):
  python bench_profiles.py kernels D <workload>   # D/stats_<w>/ (--kernel-trace --stats) + D/stats_<w>.log
  python bench_profiles.py traffic D <workload>   # D/fetch_<w>/, D/write_<w>/ (--pmc FETCH_SIZE / WRITE_SIZE),
                                                  # D/cfetch/, D/cwrite/ (the same on bench.py --copy-calibration 256)
  python bench_profiles.py mfma D <workload>      # D/mfma_<w>/ (--pmc MfmaUtil VALUBusy LdsUtil)
  python bench_profiles.py census D <workload> N  # D/census<N>_<w>/, D/census0_<w>/ (--kernel-trace --stats)
  python bench_profiles.py parity D               # D/*.json written by the GPU parity tests with PPO_PARITY_RECORD=D
Writes D/<mode>_<w>.txt (and D/traffic_<w>.json; parity: D/parity.md); copy them into profiles/.
"""

from __future__ import annotations

import csv
import json
import sys
from collections import defaultdict
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from tt_rsl_rl_amd.workloads import WORKLOADS, linear_shapes  # noqa: E402

DESC = {
    "humanoid": "humanoid PPO update (actor 96 -> [512, 256, 128] -> 29, critic 99 -> [512, 256, 128] -> 1, obs "
                "normalisation; 4096 envs x 24 steps, 5 epochs x 4 mini-batches of 24,576 rows)",
    "flat48": "flat48 PPO update (actor / critic 48 -> [512, 256, 128] -> 12 / 1; 4096 envs x 24 steps, 5 epochs x 4 "
              "mini-batches of 24,576 rows)",
    "rough235": "rough235 PPO update (actor / critic 235 -> [512, 256, 128] -> 12 / 1; 4096 envs x 24 steps, 5 epochs x "
                "4 mini-batches of 24,576 rows)",
    "flat48_65k": "flat48_65k PPO update (actor / critic 48 -> [512, 256, 128] -> 12 / 1; 65,536 envs x 24 steps, 5 "
                  "epochs x 4 mini-batches of 393,216 rows)",
    "lstm256": "lstm256 recurrent PPO update (LSTM 48 -> 256 + MLP [256, 128] -> 12 / 1; 4096 envs x 24 steps, 5 epochs "
               "x 4 env-slice mini-batches of 1024 envs)",
}
# the kernels each candidate dominant phase launches once per mini-batch (name prefix; the largest grid of that name)
PHASES_MLP = {"dw": ["gemm_tn_bx6_kernel", "dw_reduce_kernel"]}
PHASES_LSTM = {"lstm_fwd": ["lstm_pack_kernel", "gemm_nt_bx6_kernel", "lstm_seq_fwd_kernel"],
               "lstm_bwd": ["lstm_seq_bwd_kernel"],
               "lstm_dw": ["gemm_tn_bx6_kernel", "dw_reduce_kernel", "lstm_unpack_kernel"]}
BENCH = "python3 $R/bench.py --workload {w} --cpu-baseline off --steps 2 --warmup 1 --no-phase-events"


def short(name: str) -> str:
    """A kernel's name without its argument list and namespaces (64 characters at most)."""
    n = name.replace("void ", "").replace("ppo::(anonymous namespace)::", "")
    depth, out = 0, []
    for ch in n:
        if ch == "(" and depth == 0 and out and out[-1] not in " <":
            break
        depth += ch == "<"
        depth -= ch == ">"
        out.append(ch)
    return "".join(out)[:64]


def _csv(d: Path, pattern: str) -> Path:
    found = sorted(d.glob(pattern))
    if not found:
        raise SystemExit(f"no {pattern} under {d}")
    return found[0]


def _pmc(path: Path) -> dict:
    """(kernel, grid) -> counter -> [(value, duration ns)] per dispatch."""
    rows: dict = defaultdict(lambda: defaultdict(list))
    for r in csv.DictReader(open(path)):
        dur = float(r["End_Timestamp"]) - float(r["Start_Timestamp"])
        rows[(short(r["Kernel_Name"]), int(r["Grid_Size"]))][r["Counter_Name"]].append((float(r["Counter_Value"]), dur))
    return rows


def _header(kind: str, w: str, commands: list[str]) -> list[str]:
    return [f"# {kind} -- {DESC[w]}", "#", "# commands (GPU box, repository root R):"] + [f"#   {c}" for c in commands]


def kernels(d: Path, w: str) -> None:
    stats = _csv(d / f"stats_{w}", "*kernel_stats.csv")
    line = [x for x in open(d / f"stats_{w}.log") if x.startswith("{")][-1]
    b = json.loads(line)
    r = b.get("roofline") or {}
    lines = _header("rocprofv3 kernel statistics", w, [
        f"cd /tmp && TMPDIR=/tmp rocprofv3 --kernel-trace --stats --output-format csv -d $R/gpurun_out/prof/stats_{w} "
        f"-o run -- python3 $R/bench.py --workload {w} --cpu-baseline off --steps 10 --warmup 2",
        f"python bench_profiles.py kernels $R/gpurun_out/prof {w}"])
    lines += ["# 10 timed + 2 warm-up + instrumented updates and the GPU rollout of bench.py.",
              f"# bench line under the profiler: value {b['value']:.0f} samples/s, ms/update median "
              f"{b['ms_per_update_median']}",
              f"# roofline: dominant phase {r.get('kernel')} ({r.get('arith')}): {r.get('achieved')} TFLOP/s, mean "
              f"launch {r.get('mean_launch_ms')} ms (HIP events); peak {r.get('peak')} TFLOP/s ({r.get('peak_basis')})",
              "#", f"{'share':>6s} {'calls':>6s} {'avg_us':>9s} {'total_ms':>9s}  kernel"]
    for k, row in enumerate(csv.DictReader(open(stats))):
        if k >= 36:
            break
        lines.append(f"{float(row['Percentage']):5.1f}% {int(row['Calls']):6d} {float(row['AverageNs']) / 1e3:9.1f} "
                     f"{float(row['TotalDurationNs']) / 1e6:9.2f}  {short(row['Name'])}")
    (d / f"kernels_{w}.txt").write_text("\n".join(lines) + "\n")


def _calibration(d: Path, which: str) -> float:
    """Counter KiB of the plain 256 MiB copy -> bytes per counted KiB."""
    f = _csv(d / f"c{which}", "*counter_collection.csv")
    vals = [float(r["Counter_Value"]) for r in csv.DictReader(open(f)) if "copy" in r["Kernel_Name"].lower()]
    return (256 << 20) / (max(vals) * 1024)


def traffic(d: Path, w: str) -> None:
    f_cal, w_cal = _calibration(d, "fetch"), _calibration(d, "write")
    fetch = _pmc(_csv(d / f"fetch_{w}", "*counter_collection.csv"))
    write = _pmc(_csv(d / f"write_{w}", "*counter_collection.csv"))
    mean = lambda rec, c: sum(v for v, _ in rec[c]) / len(rec[c])  # noqa: E731
    phases = PHASES_LSTM if "rnn" in WORKLOADS[w] else PHASES_MLP
    out, detail = {}, {}
    for ph, pats in phases.items():
        tot, ks = 0.0, []
        for pat in pats:
            cands = [kg for kg in fetch if kg[0].startswith(pat)]
            if not cands:
                raise SystemExit(f"{w}: no dispatch of {pat}")
            kg = max(cands, key=lambda x: x[1])
            fb = mean(fetch[kg], "FETCH_SIZE") * 1024 * f_cal
            wb = mean(write[kg], "WRITE_SIZE") * 1024 * w_cal
            tot += fb + wb
            ks.append({"kernel": kg[0], "grid": kg[1], "fetch_bytes": round(fb), "write_bytes": round(wb),
                       "launches_measured": len(fetch[kg]["FETCH_SIZE"])})
        out[ph] = round(tot)
        detail[ph] = {"kernels": ks, "fetch_calibration": f_cal, "write_calibration": w_cal}
        if ph == "dw":
            R = WORKLOADS[w]["num_envs"] * WORKLOADS[w]["steps"] // 4
            detail[ph]["algorithmic_operand_bytes"] = 4 * R * sum(i + o for m in linear_shapes(WORKLOADS[w])
                                                                  for i, o in m)
    out["_detail"] = detail
    (d / f"traffic_{w}.json").write_text(json.dumps(out, indent=1) + "\n")
    lines = _header("HBM traffic per launch from rocprofv3 counters", w, [
        f"cd /tmp && TMPDIR=/tmp rocprofv3 --pmc FETCH_SIZE --output-format csv -d $R/gpurun_out/prof/fetch_{w} -o pmc "
        f"-- {BENCH.format(w=w)}",
        f"(the same with WRITE_SIZE into prof/write_{w})",
        "calibration, a plain 256 MiB device-to-device copy under the same counters: python3 $R/bench.py "
        "--copy-calibration 256 (FETCH_SIZE -> prof/cfetch, WRITE_SIZE -> prof/cwrite)",
        f"python bench_profiles.py traffic $R/gpurun_out/prof {w}"])
    lines.append(f"# copy of 268435456 B: fetch factor {f_cal:.5f}, write factor {w_cal:.5f}")
    lines.append("# per phase (bench.py's roofline.traffic for that phase = the sum over its kernels, one launch each "
                 "per mini-batch):")
    for ph, v in out.items():
        if ph != "_detail":
            lines.append(f"#   {ph}: {v / 1e6:.2f} MB per launch = " + " + ".join(
                f"{x['kernel']} ({(x['fetch_bytes'] + x['write_bytes']) / 1e6:.2f})" for x in detail[ph]["kernels"]))
    if "dw" in detail:
        lines.append(f"#   dw algorithmic operand bytes (R x sum(in + out) x 4): "
                     f"{detail['dw']['algorithmic_operand_bytes'] / 1e6:.2f} MB")
    lines += ["#", f"{'kernel':64s} {'grid':>8s} {'counter':10s} {'launches':>8s} {'KiB/launch':>12s} "
                   f"{'MB/launch (calibrated)':>24s}"]
    rows = []
    for cname, tab, cal in (("FETCH_SIZE", fetch, f_cal), ("WRITE_SIZE", write, w_cal)):
        for (k, g), rec in tab.items():
            n = len(rec[cname])
            kib = mean(rec, cname)
            rows.append((kib * n, k, g, cname, n, kib, kib * 1024 * cal / 1e6))
    for _, k, g, c, n, kib, mb in sorted(rows, reverse=True)[:28]:
        lines.append(f"{k:64s} {g:8d} {c:10s} {n:8d} {kib:12.1f} {mb:24.2f}")
    (d / f"traffic_{w}.txt").write_text("\n".join(lines) + "\n")


def mfma(d: Path, w: str) -> None:
    """Per kernel: MfmaUtil (MFMA-busy cycles of all SIMDs over the dispatch's GPU-active cycles times the SIMDs),
    VALUBusy and LdsUtil, rocprofv3's derived counters, averaged over the dispatches (the profiler runs them one at a
    time), with the mean dispatch time under the counters."""
    rec = _pmc(_csv(d / f"mfma_{w}", "*counter_collection.csv"))
    lines = _header("MFMA / VALU / LDS utilisation per kernel from rocprofv3 counters", w, [
        f"cd /tmp && TMPDIR=/tmp rocprofv3 --pmc MfmaUtil VALUBusy LdsUtil --output-format csv "
        f"-d $R/gpurun_out/prof/mfma_{w} -o pmc -- {BENCH.format(w=w)}",
        f"python bench_profiles.py mfma $R/gpurun_out/prof {w}"])
    lines += ["# MfmaUtil = sum over SIMDs of SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x SIMDs): the fraction of the",
              "# dispatch's cycles the matrix cores were busy; VALUBusy = SQ_ACTIVE_INST_VALU per CU over the same cycles;",
              "# LdsUtil = SQ_LDS_IDX_ACTIVE per CU over the same cycles.  Kernels sorted by their share of the run's",
              "# dispatch time under the counters (dispatches are serialised there).", "#",
              f"{'kernel':64s} {'grid':>8s} {'launches':>8s} {'us/launch':>10s} {'MfmaUtil%':>10s} {'VALUBusy%':>10s} "
              f"{'LdsUtil%':>9s}"]
    rows = []
    for (k, g), c in rec.items():
        n = len(c.get("MfmaUtil", []))
        if n == 0:
            continue
        avg = lambda name: sum(v for v, _ in c.get(name, [(0.0, 0.0)])) / max(len(c.get(name, [])), 1)  # noqa: E731
        us = sum(t for _, t in c["MfmaUtil"]) / n / 1e3
        rows.append((us * n, k, g, n, us, avg("MfmaUtil"), avg("VALUBusy"), avg("LdsUtil")))
    for _, k, g, n, us, m, v, l in sorted(rows, reverse=True)[:30]:
        lines.append(f"{k:64s} {g:8d} {n:8d} {us:10.1f} {m:10.1f} {v:10.1f} {l:9.1f}")
    (d / f"mfma_{w}.txt").write_text("\n".join(lines) + "\n")


def census(d: Path, w: str, n: int) -> None:
    def calls(sub: str) -> dict:
        f = _csv(d / sub, "*kernel_stats.csv")
        return {short(r["Name"]): (int(r["Calls"]), float(r["TotalDurationNs"])) for r in csv.DictReader(open(f))}

    a, b = calls(f"census{n}_{w}"), calls(f"census0_{w}")
    rows = []
    for k, (c, t) in a.items():
        c0, t0 = b.get(k, (0, 0.0))
        if c - c0 > 0:
            rows.append((k, (c - c0) / n, (t - t0) / n / 1e3))
    rows.sort(key=lambda r: -r[2])
    torch_rows = [r for r in rows if "at::" in r[0] or "native" in r[0]]
    lines = _header("Kernel census of update()", w, [
        f"cd /tmp && TMPDIR=/tmp rocprofv3 --kernel-trace --stats --output-format csv "
        f"-d $R/gpurun_out/prof/census{n}_{w} -o run -- python3 $R/bench.py --workload {w} --census {n}",
        f"(the same with --census 0 into prof/census0_{w})",
        f"python bench_profiles.py census $R/gpurun_out/prof {w} {n}"])
    lines += ["# the kernels of N updates = the run with --census N minus the run with --census 0 (the same construction",
              "# and GPU rollout, no update)",
              f"# per update: {sum(r[1] for r in rows):.0f} launches, {sum(r[2] for r in rows) / 1e3:.2f} ms of kernel "
              f"time; torch (at::native) kernels among them: {len(torch_rows)}",
              "#", f"{'launches/update':>16s} {'us/update':>10s}  kernel"]
    lines += [f"{c:16.1f} {t:10.1f}  {k}" for k, c, t in rows]
    (d / f"census_{w}.txt").write_text("\n".join(lines) + "\n")


def parity(d: Path) -> None:
    """The GPU parity tests' records (tests/test_gpu_update.py, tests/test_gpu_kernels.py) as tables."""
    load = lambda f: json.loads(f.read_text())  # noqa: E731
    lines = ["# GPU parity against the CPU oracle -- the figures the GPU parity tests measured", "#",
             "# command (GPU box, repository root R):",
             "#   PPO_PARITY_RECORD=$R/gpurun_out/parity python -m pytest tests/test_gpu_update.py tests/test_gpu_kernels.py "
             "-m gpu -k 'update or compute_returns or bx6_error'",
             "#   python bench_profiles.py parity $R/gpurun_out/parity", "",
             "## Whole update, end to end (test_update_matches_oracle)", "",
             "Rows on another clip branch than the literal oracle's (step, kind, distance of the oracle's ratio or value "
             "to the boundary); parameters against the oracle that takes the GPU's branch on those rows (worst tensor, "
             "relative Frobenius); function space ||f(p) - f(q)|| / ||f(q) - f(p0)|| of the actor mean / critic value; "
             "the oracle's own spread = the same oracle with its log-prob sums in fp64.", "",
             "| case | rows on another branch | worst param err vs branch-matched | d(gpu, branch-matched) actor / critic "
             "| d(gpu, literal oracle) actor | d(branch-matched, literal) actor | oracle spread actor | largest ratio gap "
             "| advantages rel err |", "|---|---|---|---|---|---|---|---|---|"]
    for f in sorted(d.glob("update_*.json")):
        r = load(f)
        fl = r["rows_on_another_branch"]
        fls = f"{len(fl)}" + (" (" + ", ".join(f"{x['step']}:{x['distance_to_boundary']:.1e}" for x in fl[:6]) +
                              (", ..." if len(fl) > 6 else "") + ")" if fl else "")
        fs = r["function_space"]
        lines.append(f"| {r['case']} | {fls} | {r['worst_param_err_vs_branch_matched']:.1e} | "
                     f"{fs['actor']['gpu_vs_branch_matched']:.1e} / {fs['critic']['gpu_vs_branch_matched']:.1e} | "
                     f"{fs['actor']['gpu_vs_literal_oracle']:.1e} | {fs['actor']['branch_matched_vs_literal_oracle']:.1e} | "
                     f"{fs['actor']['oracle_spread_lp64_vs_oracle']:.1e} | {r['largest_ratio_gap']:.1e} | "
                     f"{r['advantages_rel_err']:.1e} |")
    lines += ["", "Per parameter tensor (worst case of each kind over the cases above): against the branch-matched "
              "oracle / against the literal oracle / the oracle's own spread.", ""]
    for f in sorted(d.glob("update_*.json")):
        r = load(f)
        worst = max(r["tensors"].items(), key=lambda kv: kv[1]["vs_branch_matched"])
        lit = max(r["tensors"].items(), key=lambda kv: kv[1]["vs_literal_oracle"])
        lines.append(f"* {r['case']}: worst vs branch-matched {worst[0]} {worst[1]['vs_branch_matched']:.1e}; worst vs "
                     f"literal {lit[0]} {lit[1]['vs_literal_oracle']:.1e} (its oracle spread "
                     f"{lit[1]['oracle_spread_lp64_vs_oracle']:.1e})")
    lines += ["", "## Every optimiser step from the oracle's state (test_update_steps_teacher_forced)", "",
              "| case | steps | steps replayed with the GPU's branches | rows on another branch | worst param err | "
              "largest ratio gap | largest value gap |", "|---|---|---|---|---|---|---|"]
    for f in sorted(d.glob("teacher_forced_*.json")):
        r = load(f)
        g = r["largest_gaps"]
        lines.append(f"| {r['case']} | {r['steps']} | {r['replayed_with_gpu_branches']} | {r['rows_on_another_branch']} "
                     f"| {r['worst_param_err']:.1e} | {g.get('surrogate', 0):.1e} | {g.get('value', 0):.1e} |")
    cr = sorted(d.glob("compute_returns_*.json"))
    if cr:
        lines += ["", "## compute_returns with the plugin's own bootstrap forward (relative, norm-wise)", "",
                  "| case | envs x steps | bootstrap values | returns | advantages |", "|---|---|---|---|---|"]
        for f in cr:
            r = load(f)
            e = r["rel_err"]
            lines.append(f"| {r['case']} | {r['envs']} x {r['steps']} | {e['bootstrap_values']:.1e} | {e['returns']:.1e} "
                         f"| {e['advantages']:.1e} |")
    bx = sorted(d.glob("bx6_vs_fp32_*.json"))
    if bx:
        lines += ["", "## bf16x6 against the fp32-MFMA kernels, both against fp64 (test_bx6_error_against_fp32_mfma)", "",
                  "| op | rows | operands | bf16x6 rel-Frobenius | fp32 MFMA rel-Frobenius | ratio | bf16x6 per-element / "
                  "bound | fp32 MFMA per-element / bound | ratio |", "|---|---|---|---|---|---|---|---|---|"]
        for f in bx:
            r = load(f)
            lines.append(f"| {r['op']} | {r['rows']} | {'log-uniform 1e-6..1e6' if r['wide_range'] else 'N(0, 1)'} | "
                         f"{r['bx6']['rel_frobenius']:.2e} | {r['fp32_mfma']['rel_frobenius']:.2e} | "
                         f"{r['ratio']['rel_frobenius']:.2f} | {r['bx6']['per_element_over_bound']:.2e} | "
                         f"{r['fp32_mfma']['per_element_over_bound']:.2e} | {r['ratio']['per_element_over_bound']:.2f} |")
    (d / "parity.md").write_text("\n".join(lines) + "\n")


if __name__ == "__main__":
    if sys.argv[1] == "parity":
        parity(Path(sys.argv[2]))
        print(f"wrote {sys.argv[2]}/parity.md")
        sys.exit(0)
    mode, d, w = sys.argv[1], Path(sys.argv[2]), sys.argv[3]
    if mode == "census":
        census(d, w, int(sys.argv[4]))
    else:
        {"kernels": kernels, "traffic": traffic, "mfma": mfma}[mode](d, w)
    print(f"wrote {d}/{mode}_{w}.txt")
