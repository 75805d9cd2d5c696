"""Reduce rocprofv3 output of ``bench.py`` runs into the ``profiles/*.md`` summaries.

Usage (on the directories the rocprofv3 runs wrote)::

    python -m mingru_amd.profiling --workload C2 --stats DIR --fetch DIR --write DIR \\
        --bench BENCH_JSON [--counters DIR ...] --out profiles/linear_scan_C2.md \\
        --command "rocprofv3 ..." [--command ...]

* ``--stats``: a ``rocprofv3 --kernel-trace --stats -f csv -o run`` directory
  (``run_kernel_stats.csv``) of ``bench.py --only <workload>``.
* ``--fetch`` / ``--write``: ``rocprofv3 --pmc FETCH_SIZE`` / ``--pmc WRITE_SIZE``
  directories (``run_counter_collection.csv``) of a ``bench.py --copy-probe`` run
  covering the workload.  Each counter (KiB per dispatch) is averaged over the
  dispatches of every kernel a C-ABI call launches and summed over those kernels,
  then scaled by what the same counter reads for the copy probe's plain 1 GiB
  device-to-device copy in the same run, so the figures are HBM bytes.
* ``--counters``: further ``--pmc`` directories; their counters are tabulated per
  kernel (average per dispatch).
* ``--valu``: a ``--pmc`` directory with ``SQ_INSTS_VALU``; adds each call's VALU issue
  floor (``valu`` lines, read by ``bench.py``).
* ``--bench``: the JSON line an unprofiled ``bench.py`` run printed, for the HIP-event
  timings and the step time (rocprofv3's own tracing adds to the step).

Kernels are attributed to C-ABI entry points by name (``ENTRIES``), independent of
tile-size template arguments; an entry point with no matching dispatch is an error,
never a zero.
"""

from __future__ import annotations

import argparse
import collections
import csv
import json
import os
import re
import statistics

# workload -> [(entry point, kernel-name pattern)], matched against the demangled
# name with its argument list removed.
ENTRIES = {
    "C2": [("mg_linear_scan_fwd", r"\bew_fwd_kernel<"),
           ("mg_linear_scan_bwd", r"\blinear_bwd_kernel<")],
    # gate kernels: <columns per lane, steps per wave, waves, gate kind, decay[, launch form]>
    "C2g": [("mg_signed_gate_scan_fwd", r"\bgate_fwd_kernel<\d+, \d+, \d+, [01], false(, \d)?>"),
            ("mg_signed_gate_scan_bwd", r"\bgate_bwd_kernel<\d+, \d+, \d+, [01], false(, \d)?>")],
    "C2gd": [("mg_signed_gate_scan_decay_fwd",
              r"\bgate_fwd_kernel<\d+, \d+, \d+, [01], true(, \d)?>"),
             ("mg_signed_gate_scan_decay_bwd",
              r"\bgate_bwd_kernel<\d+, \d+, \d+, [01], true(, \d)?>")],
    "C1g": [("mg_mingru_gate_scan_fwd", r"\bgate_fwd_kernel<\d+, \d+, \d+, 2, false(, \d)?>"),
            ("mg_mingru_gate_scan_bwd", r"\bgate_bwd_kernel<\d+, \d+, \d+, 2, false(, \d)?>")],
    "C1": [("mg_log_scan_fwd", r"\blog_fwd_kernel<"), ("mg_log_scan_bwd", r"\blog_bwd_kernel<")],
    "C3": [("mg_affine_scan_fwd", r"\baffine_fwd_kernel<2, 1,"),
           ("mg_affine_scan_bwd", r"\baffine_bwd_kernel<2, 1,")],
    "C4": [("mg_angle_scan_fwd", r"\bangle_fwd_\w+<|\bangle_group_\w+<\d+, false>"),
           ("mg_angle_scan_bwd",
            r"\bangle_bwd_\w+<|\bangle_group_\w+<\d+, true>|\bangle_group_offsets<")],
    # brick-wall schedule with the gated heads: pass kernels <K, schedule, scale, decay, gated>
    "C4g": [("mg_angle_scan_gated_fwd", r"\bangle_fwd_\w+<"),
            ("mg_angle_scan_gated_bwd", r"\bangle_bwd_\w+<")],
    "C5": [("mg_delta_fwd", r"\bdwb_fwd_\w+<false>"), ("mg_delta_bwd", r"\bdwb_bwd_\w+<false>")],
    "C5d": [("mg_delta_gated_fwd", r"\bdwb_fwd_\w+<true>"),
            ("mg_delta_gated_bwd", r"\bdwb_bwd_\w+<true>")],
    "C5dp": [("mg_delta_gated_fwd", r"\bdwb_fwd_\w+<true>"),
             ("mg_delta_gated_bwd", r"\bdwb_bwd_\w+<true>")],
}

COPY_PROBE_BYTES = 1 << 30  # bench.py --copy-probe: one 1 GiB device-to-device copy

# VALU issue floor: a wave64 fp32 VALU instruction occupies a 16-lane SIMD for 4
# cycles; MI355X has 256 CUs x 4 SIMDs at a 2.4 GHz peak engine clock.
VALU_CYCLES_PER_INST = 4
SIMDS = 1024
CLOCK_MHZ = 2400


def valu_floor_us(wave_insts: float) -> float:
    """Time the SIMDs need just to issue `wave_insts` wave64 VALU instructions."""
    return wave_insts * VALU_CYCLES_PER_INST / SIMDS / CLOCK_MHZ


def short_name(name: str) -> str:
    """``void (anonymous namespace)::ew_fwd_kernel<4, 16, 8>(float const*, ...)`` ->
    ``ew_fwd_kernel<4, 16, 8>``."""
    n = name.replace("(anonymous namespace)::", "")
    n = re.sub(r"^void ", "", n)
    depth = 0
    for i, ch in enumerate(n):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            n = n[:i]
            break
    head, sep, rest = n.partition("<")
    return head.rsplit("::", 1)[-1] + sep + rest


def read_counters(directory: str) -> dict:
    """``{counter: {kernel short name: [value per dispatch, ...]}}`` of one --pmc run."""
    path = os.path.join(directory, "run_counter_collection.csv")
    out: dict = collections.defaultdict(lambda: collections.defaultdict(list))
    with open(path) as f:
        for r in csv.DictReader(f):
            out[r["Counter_Name"]][short_name(r["Kernel_Name"])].append(float(r["Counter_Value"]))
    return out


def copy_scale(per_kernel: dict) -> float:
    """Bytes per counter unit: the copy probe's 1 GiB over its median counter reading.

    The probe's copy runs as the runtime's blit kernel; its dispatches are the ones of
    that kernel reading at least a quarter of the probe size (smaller blits are torch's
    own host<->device copies)."""
    vals = [v for k, vs in per_kernel.items() if "copyBuffer" in k for v in vs
            if v * 1024 >= COPY_PROBE_BYTES / 8]
    if not vals:
        raise SystemExit("no copy-probe dispatch in the counter run (run bench.py --copy-probe)")
    return COPY_PROBE_BYTES / (statistics.median(vals) * 1024)


def entry_sum(per_kernel: dict, pattern: str, what: str) -> float:
    """Counter per call of one entry point: per-kernel dispatch averages, summed."""
    rx = re.compile(pattern)
    hits = {k: v for k, v in per_kernel.items() if rx.search(k)}
    if not hits:
        raise SystemExit(f"{what}: no dispatch matches {pattern!r}")
    return sum(sum(v) / len(v) for v in hits.values())


def entry_bytes(per_kernel: dict, pattern: str, scale: float, what: str) -> float:
    """Counter bytes per call of one entry point: per-kernel dispatch averages, summed."""
    rx = re.compile(pattern)
    hits = {k: v for k, v in per_kernel.items() if rx.search(k)}
    if not hits:
        raise SystemExit(f"{what}: no dispatch matches {pattern!r}")
    total = sum(sum(v) / len(v) for v in hits.values()) * 1024 * scale
    if total <= 0:
        raise SystemExit(f"{what}: counter reads zero for {sorted(hits)}")
    return total


def kernel_stats(directory: str, limit: int = 10) -> list:
    path = os.path.join(directory, "run_kernel_stats.csv")
    with open(path) as f:
        rows = list(csv.DictReader(f))
    return [
        (short_name(r["Name"]), int(r["Calls"]), float(r["AverageNs"]) / 1e3,
         float(r["MinNs"]) / 1e3, float(r["MaxNs"]) / 1e3, float(r["Percentage"]))
        for r in rows[:limit]
    ]


def _fmt(x: float) -> str:
    return f"{x:.3g}" if abs(x) >= 1e4 or (0 < abs(x) < 1e-2) else f"{x:.4g}"


def counter_table(dirs: list, patterns: list) -> list:
    """Markdown rows: per kernel matching any entry pattern, every counter's average per
    dispatch, plus the waiting share when SQ_WAIT_ANY and SQ_WAVE_CYCLES are present."""
    merged: dict = {}
    for d in dirs:
        for ctr, per in read_counters(d).items():
            merged[ctr] = per
    kernels = []
    for per in merged.values():
        for k in per:
            if any(re.search(p, k) for p in patterns) and k not in kernels:
                kernels.append(k)
    ctrs = sorted(merged)
    head = ["kernel"] + ctrs
    derived = "SQ_WAIT_ANY" in merged and "SQ_WAVE_CYCLES" in merged
    if derived:
        head.append("waiting")
    lines = ["| " + " | ".join(head) + " |", "|" + "---|" + "---:|" * (len(head) - 1)]
    for k in kernels:
        avg = {c: (sum(merged[c][k]) / len(merged[c][k]) if merged[c].get(k) else None)
               for c in ctrs}
        cells = [f"`{k}`"] + ["—" if avg[c] is None else _fmt(avg[c]) for c in ctrs]
        if derived:
            w, cyc = avg["SQ_WAIT_ANY"], avg["SQ_WAVE_CYCLES"]
            cells.append(f"{100 * w / cyc:.0f}%" if w is not None and cyc else "—")
        lines.append("| " + " | ".join(cells) + " |")
    return lines


def summarize(args) -> str:
    entries = ENTRIES[args.workload]
    bench = json.loads(open(args.bench).read().strip().splitlines()[-1])
    ops = bench.get("ops", {}).get(args.workload, {})
    fetch = read_counters(args.fetch)["FETCH_SIZE"]
    write = read_counters(args.write)["WRITE_SIZE"]
    fs, ws = copy_scale(fetch), copy_scale(write)
    L = [f"# {args.title}", "",
         "Kernel durations and HBM traffic of the HIP path on one MI355X (gfx950), measured with",
         "rocprofv3 while `bench.py` ran the workload's forward + backward steps.", "",
         "Commands (run from `/tmp` with `TMPDIR=/tmp`; `$R` is the repository root), then this "
         "summary:", "", "```", *args.command,
         f"python3 -m mingru_amd.profiling {' '.join(args.argv)}", "```", "",
         "## Kernel statistics (`run_kernel_stats.csv`)", "",
         "| kernel | calls | avg µs | min µs | max µs | share |", "|---|---:|---:|---:|---:|---:|"]
    for name, calls, avg, lo, hi, pct in kernel_stats(args.stats):
        L.append(f"| `{name}` | {calls} | {avg:.2f} | {lo:.2f} | {hi:.2f} | {pct:.1f}% |")
    L += ["", "## HIP-event timing in `bench.py` (per C-ABI call)", "",
          "From an unprofiled `bench.py` run (the first command above), not from the rocprofv3 "
          "runs.", "",
          "| entry point | avg µs | algorithmic bytes | achieved GB/s |", "|---|---:|---:|---:|"]
    for e, k in ops.get("kernels", {}).items():
        L.append(f"| `{e}` | {k['avg_us']:.1f} | {k['algorithmic_bytes']:,} | "
                 f"{k['achieved_GBs']:.0f} |")
    if ops:
        L += ["", f"Step: {ops['ms_per_step']:.3f} ms fwd+bwd, {ops['tokens_per_s']:.4g} tokens/s, "
              f"{ops['achieved_TBs']:.3f} TB/s algorithmic "
              f"({100 * ops['frac_of_hbm_peak']:.1f}% of 8 TB/s)."]
    L += ["", "## HBM traffic per C-ABI call (rocprof counters)", "",
          "`FETCH_SIZE` and `WRITE_SIZE` (KiB per dispatch), averaged per kernel and summed over "
          "the kernels of the call, times the bytes per counter unit that the copy probe's 1 GiB "
          f"device copy gives in the same runs: fetch x{fs:.3f}, write x{ws:.3f}.", "",
          "| entry point | fetch MB | write MB | total MB | algorithmic MB |",
          "|---|---:|---:|---:|---:|"]
    traffic = []
    for entry, pat in entries:
        f = entry_bytes(fetch, pat, fs, f"{args.workload}:{entry} FETCH_SIZE")
        w = entry_bytes(write, pat, ws, f"{args.workload}:{entry} WRITE_SIZE")
        alg = ops.get("kernels", {}).get(entry, {}).get("algorithmic_bytes")
        L.append(f"| `{entry}` | {f / 1e6:.1f} | {w / 1e6:.1f} | {(f + w) / 1e6:.1f} | "
                 f"{'—' if alg is None else f'{alg / 1e6:.1f}'} |")
        traffic.append(f"traffic {args.workload}:{entry} {int(f)} {int(w)}")
    L += ["", "Machine-readable lines read by `bench.py` "
          "(`traffic <workload>:<entry> <fetch bytes> <write bytes>`):", "", "```", *traffic, "```"]
    if args.valu:
        insts = read_counters(args.valu).get("SQ_INSTS_VALU")
        if not insts:
            raise SystemExit(f"{args.valu}: no SQ_INSTS_VALU counter")
        L += ["", "## VALU issue floor per C-ABI call (`SQ_INSTS_VALU`)", "",
              f"Wave64 VALU instructions per call (per-kernel dispatch averages, summed) times "
              f"{VALU_CYCLES_PER_INST} cycles each, spread over {SIMDS} SIMDs at {CLOCK_MHZ} MHz: "
              "the time the SIMDs need only to issue them.", "",
              "| entry point | VALU wave instructions | floor µs | measured µs | share of floor |",
              "|---|---:|---:|---:|---:|"]
        lines = []
        for entry, pat in entries:
            n = entry_sum(insts, pat, f"{args.workload}:{entry} SQ_INSTS_VALU")
            fl = valu_floor_us(n)
            meas = ops.get("kernels", {}).get(entry, {}).get("avg_us")
            L.append(f"| `{entry}` | {n:.4g} | {fl:.1f} | "
                     f"{'—' if meas is None else f'{meas:.1f}'} | "
                     f"{'—' if not meas else f'{100 * fl / meas:.0f}%'} |")
            lines.append(f"valu {args.workload}:{entry} {int(n)}")
        L += ["", "Machine-readable lines read by `bench.py` "
              "(`valu <workload>:<entry> <VALU wave instructions per call>`):", "", "```",
              *lines, "```"]
    if args.counters:
        L += ["", "## Issue and memory counters per kernel (average per dispatch)", "",
              *counter_table(args.counters, [p for _, p in entries])]
    return "\n".join(L) + "\n"


def main(argv=None):
    import sys

    argv = list(sys.argv[1:] if argv is None else argv)
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--workload", required=True, choices=sorted(ENTRIES))
    ap.add_argument("--title", required=True)
    ap.add_argument("--stats", required=True)
    ap.add_argument("--fetch", required=True)
    ap.add_argument("--write", required=True)
    ap.add_argument("--bench", required=True)
    ap.add_argument("--counters", nargs="*", default=[])
    ap.add_argument("--valu", default=None,
                    help="a --pmc run with SQ_INSTS_VALU: adds the VALU issue floor per call")
    ap.add_argument("--command", action="append", default=[])
    ap.add_argument("--out", required=True)
    args = ap.parse_args(argv)
    # The summary records how it was made, minus the rocprof commands themselves.
    shown = []
    skip = False
    for a in argv:
        if skip:
            skip = False
            continue
        if a == "--command":
            skip = True
            continue
        shown.append(f'"{a}"' if " " in a else a)
    args.argv = shown
    text = summarize(args)
    with open(args.out, "w") as f:
        f.write(text)
    print(f"wrote {args.out}")


if __name__ == "__main__":
    main()
