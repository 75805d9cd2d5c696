"""Parity, benchmark and memory artefacts in the reference's JSON schemas.

Counterpart of the reference's ``scripts/bench_scans.py`` for the HIP backend, so
that tooling which reads the reference's ``experiments/bench/`` artefacts reads
these too.  ``python -m mingru_amd.bench_scans [--check] [--bench] [--memory]
[--out DIR] [--quick]`` writes, under ``DIR`` (default ``experiments/bench``):

* ``--check``  -> ``scan_parity.json`` / ``.md``: ``{"meta": {...}, "rows": [...]}``,
  one row per gated case over the reference's grid (every scan op at T in {1, 13,
  64, 128, 1024} x B in {2, 128}; ``matrix_affine_scan`` over the whole k x v
  envelope), with the reference's keys (``src/mingru/triton_scans.py:
  2634-2679``): ``op, shape, dtype, direction ("fwd" | "grad"), gate_atol,
  gate_rtol, max_abs_err, max_rel_err, pass, ref_fp64_dev``.  Each case runs the
  HIP path on fp32 inputs and the package's eager path in float64 on the same
  inputs; ``ref_fp64_dev`` is the eager fp32 path's own deviation from float64.
* ``--bench``  -> ``scan_bench.json`` / ``.md``: rows ``{op, impl, shape, dtype,
  direction ("fwd" | "fwdbwd"), us_per_iter}`` (``scripts/bench_scans.py:522-529``)
  for the four scan ops at the reference's lab (B=128, T=64, d=64, k=8) and
  long-T (B=16, T=1024) shapes.  ``impl`` is ``"hip"`` (this backend) or
  ``"eager"`` (the torch path on the GPU); the reference's ``"triton"`` and
  ``"torch_compile"`` rows have no counterpart here.
* ``--memory`` -> ``scan_memory.json`` / ``.md``: peak bytes of one
  GivensMinGRU forward+backward at the lab shape, angle-fused HIP path against
  the generic eager ``matrix_affine_scan`` path.

Without a GPU every mode prints a loud skip and exits 0, as the reference does.
Exit status 1 means a gated parity case failed or a bench case could not run.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import subprocess
from datetime import datetime, timezone
from pathlib import Path

import torch
import torch.nn.functional as F

FWD_ATOL = 1e-4
GRAD_ATOL = 1e-3

# The reference's parity grid (``src/mingru/triton_scans.py:2753-2754``) and its
# block envelope (``:183``).
PARITY_TS = (1, 13, 64, 128, 1024)
PARITY_BS = (2, 128)
AFFINE_ENVELOPE = (1, 2, 4, 8, 16)

LAB_SHAPE = {"label": "lab", "B": 128, "T": 64, "d": 64, "k": 8, "warmup": 10, "reps": 30}
LONGT_SHAPE = {"label": "long-T", "B": 16, "T": 1024, "d": 64, "k": 8, "warmup": 5, "reps": 10}
OPS = ("linear_scan", "matrix_scan", "matrix_affine_scan", "parallel_scan_log")
IMPLS = ("hip", "eager")
DIRECTIONS = ("fwd", "fwdbwd")

PARITY_KEYS = ("op", "shape", "dtype", "direction", "gate_atol", "gate_rtol", "max_abs_err",
               "max_rel_err", "pass", "ref_fp64_dev")
BENCH_KEYS = ("op", "impl", "shape", "dtype", "direction", "us_per_iter")


# ---------------------------------------------------------------------------
# inputs (seeded CPU generator; contractive transitions keep long products finite)
# ---------------------------------------------------------------------------


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def op_inputs(op: str, B: int, T: int, d: int, k: int, seed: int = 0):
    """Inputs of one scan op in the shape a mixer hands it, and the op's schema shape dict.

    ``matrix_scan`` is RotationMinGRU's k = 2 path (``d // 2`` blocks) and
    ``matrix_affine_scan`` GivensMinGRU's (``d // k`` blocks of ``k``, ``v = 1``),
    as in the reference's bench configuration.
    """
    from .min_gru import g as g_act

    gen = _gen(seed)
    if op == "linear_scan":
        a = torch.tanh(2 * torch.randn(B, T, d, generator=gen))
        return (a, torch.randn(B, T, d, generator=gen)), {"B": B, "T": T, "D": d}
    if op == "parallel_scan_log":
        z = torch.randn(B, T, d, generator=gen)
        x = torch.randn(B, T, d, generator=gen)
        h0 = g_act(torch.randn(B, 1, d, generator=gen))
        lv = torch.cat([h0.log(), F.logsigmoid(z) + torch.log(g_act(x))], dim=1)
        return (F.logsigmoid(-z), lv), {"B": B, "T": T, "D": d}
    if op == "matrix_scan":
        n = d // 2
        M = torch.randn(B, T, n, 2, 2, generator=gen) * (0.5 / math.sqrt(2))
        return (M, torch.randn(B, T, n, 2, generator=gen)), {"B": B, "T": T, "n": n, "k": 2,
                                                             "v": 1}
    if op == "matrix_affine_scan":
        n = d // k
        A = torch.randn(B, T, n, k, k, generator=gen) * (0.5 / math.sqrt(k))
        return (A, torch.randn(B, T, n, k, 1, generator=gen)), {"B": B, "T": T, "n": n, "k": k,
                                                                "v": 1}
    raise ValueError(f"unknown op {op!r}")


def affine_inputs(B: int, T: int, n: int, k: int, v: int, seed: int = 0):
    """``matrix_affine_scan`` inputs for a generic (k, v): k x k transitions scaled to
    spectral norm below 1 (so long products stay finite) and N(0, 1) offsets."""
    gen = _gen(seed)
    A = torch.randn(B, T, n, k, k, generator=gen, dtype=torch.float64)
    A = A / torch.linalg.matrix_norm(A, ord=2)[..., None, None]
    A = (A * torch.rand(B, T, n, 1, 1, generator=gen, dtype=torch.float64)).float()
    Bm = torch.randn(B, T, n, k, v, generator=gen)
    return (A, Bm), {"B": B, "T": T, "n": n, "k": k, "v": v}


def _op_fn(op: str):
    from . import min_gru

    return getattr(min_gru, op)


class _ScanMode:
    """Sets ``MINGRU_SCAN`` for a block and restores the previous value."""

    def __init__(self, mode: str):
        self.mode = mode

    def __enter__(self):
        self.saved = os.environ.get("MINGRU_SCAN")
        os.environ["MINGRU_SCAN"] = self.mode

    def __exit__(self, *exc):
        if self.saved is None:
            os.environ.pop("MINGRU_SCAN", None)
        else:
            os.environ["MINGRU_SCAN"] = self.saved
        return False


# ---------------------------------------------------------------------------
# rows, meta and markdown (schema helpers; CPU-testable)
# ---------------------------------------------------------------------------


def parity_row(op, shape, dtype, direction, gate_atol, gate_rtol, max_abs_err, max_rel_err,
               passed, ref_fp64_dev=None) -> dict:
    return {"op": op, "shape": shape, "dtype": str(dtype).replace("torch.", ""),
            "direction": direction, "gate_atol": gate_atol, "gate_rtol": gate_rtol,
            "max_abs_err": max_abs_err, "max_rel_err": max_rel_err, "pass": bool(passed),
            "ref_fp64_dev": ref_fp64_dev}


def bench_row(op, impl, shape: dict, direction, us_per_iter) -> dict:
    return {"op": op, "impl": impl, "shape": shape, "dtype": "float32", "direction": direction,
            "us_per_iter": us_per_iter}


def parity_counts(rows: list[dict]) -> dict:
    def count(rs):
        return {"total": len(rs), "passed": sum(r["pass"] for r in rs),
                "failed": sum(not r["pass"] for r in rs)}

    out = count(rows)
    out["by_direction"] = {d: count([r for r in rows if r["direction"] == d])
                           for d in ("fwd", "grad")}
    return out


def _git_commit() -> str | None:
    try:
        here = Path(__file__).resolve().parent
        r = subprocess.run(["git", "rev-parse", "HEAD"], capture_output=True, text=True,
                           cwd=here, timeout=10, check=True)
        return r.stdout.strip()
    except Exception:  # noqa: BLE001 - metadata only
        return None


def run_meta(rows: list[dict]) -> dict:
    cuda = torch.cuda.is_available()
    return {
        "gpu_name": torch.cuda.get_device_name(0) if cuda else None,
        "driver_version": getattr(torch.version, "hip", None),
        "torch_version": torch.__version__,
        "triton_version": None,
        "hip_version": getattr(torch.version, "hip", None),
        "git_commit": _git_commit(),
        "timestamp": datetime.now(timezone.utc).isoformat(),
        "counts": parity_counts(rows),
    }


def parity_markdown(rows: list[dict], meta: dict) -> str:
    lines = ["# Scan kernel parity conformance (HIP backend)", "",
             f"torch {meta['torch_version']}, HIP {meta['hip_version']}, device "
             f"{meta['gpu_name']}, commit {meta['git_commit']}, generated {meta['timestamp']}.", "",
             "| op | shape | dtype | direction | gate atol | gate rtol | max abs err | max rel err "
             "| ref fp32-vs-fp64 dev | pass |",
             "| --- | --- | --- | --- | --- | --- | --- | --- | --- | --- |"]

    def e(x):
        return "n/a" if x is None else f"{x:.2e}"

    for r in rows:
        lines.append(f"| {r['op']} | {r['shape']} | {r['dtype']} | {r['direction']} | "
                     f"{r['gate_atol']:.0e} | {r['gate_rtol']:.0e} | {e(r['max_abs_err'])} | "
                     f"{e(r['max_rel_err'])} | {e(r['ref_fp64_dev'])} | "
                     f"{'PASS' if r['pass'] else 'FAIL'} |")
    lines += ["", f"Counts: {json.dumps(meta['counts'])}"]
    return "\n".join(lines) + "\n"


def bench_markdown(rows: list[dict], meta: dict) -> str:
    lines = ["# Scan kernel benchmark (HIP backend)", "",
             f"torch {meta['torch_version']}, device {meta['device_name']}. "
             f"Warmup/reps per shape: {json.dumps(meta['warmup_reps'])}.", "",
             "| op | shape | direction | hip (us) | eager (us) | hip speedup vs eager |",
             "| --- | --- | --- | --- | --- | --- |"]
    by_key: dict = {}
    for r in rows:
        key = (r["op"], json.dumps(r["shape"], sort_keys=True), r["direction"])
        by_key.setdefault(key, {})[r["impl"]] = r["us_per_iter"]
    for (op, shape_json, direction), impls in by_key.items():
        hip, eager = impls.get("hip"), impls.get("eager")
        sp = f"{eager / hip:.2f}x" if hip and eager else "n/a"
        f = (lambda v: "n/a" if v is None else f"{v:.2f}")
        lines.append(f"| {op} | {json.dumps(json.loads(shape_json))} | {direction} | {f(hip)} | "
                     f"{f(eager)} | {sp} |")
    return "\n".join(lines) + "\n"


def _write(out: Path, stem: str, payload: dict, md: str) -> None:
    out.mkdir(parents=True, exist_ok=True)
    (out / f"{stem}.json").write_text(json.dumps(payload, indent=2) + "\n")
    (out / f"{stem}.md").write_text(md)
    print(f"wrote {out / (stem + '.json')} and {out / (stem + '.md')}")


def _loud_skip(reason: str) -> int:
    print(f"mingru_amd.bench_scans SKIPPED (loud): {reason}")
    return 0


def _gpu_status():
    if not torch.cuda.is_available():
        return "no GPU visible"
    from . import hip_scans

    return hip_scans.available()


# ---------------------------------------------------------------------------
# --check
# ---------------------------------------------------------------------------


def _outputs(out):
    return out if isinstance(out, tuple) else (out,)


def _max_err(got, ref):
    abs_err = max(float((g.double().cpu() - r.double().cpu()).abs().max()) if g.numel() else 0.0
                  for g, r in zip(got, ref))
    scale = max(float(r.double().abs().max()) if r.numel() else 0.0 for r in ref)
    return abs_err, abs_err / max(scale, 1e-30)


def _run_case(fn, ins, gouts_seed):
    """Forward outputs and input gradients (sum of <gout, out>) of ``fn`` on ``ins``."""
    leaves = [t.detach().clone().requires_grad_(True) for t in ins]
    outs = _outputs(fn(*leaves))
    gen = _gen(gouts_seed)
    gouts = [torch.randn(o.shape, generator=gen).to(o.device, o.dtype) for o in outs]
    grads = torch.autograd.grad(outs, leaves, gouts, allow_unused=True)
    grads = [torch.zeros_like(x) if g is None else g for g, x in zip(grads, leaves)]
    return [o.detach() for o in outs], [g.detach() for g in grads]


def _gate_rows(op, shape, fn_hip, fn_ref, ins, dev, rows, seed):
    """Run one case three ways (HIP fp32, eager fp32, eager fp64) and append fwd/grad rows."""
    with _ScanMode("hip"):
        o_h, g_h = _run_case(fn_hip, [t.to(dev) for t in ins], seed)
    with _ScanMode("eager"):
        o_64, g_64 = _run_case(fn_ref, [t.double().to(dev) for t in ins], seed)
        o_32, g_32 = _run_case(fn_ref, [t.to(dev) for t in ins], seed)
    for direction, got, ref, e32, atol in (("fwd", o_h, o_64, o_32, FWD_ATOL),
                                           ("grad", g_h, g_64, g_32, GRAD_ATOL)):
        abs_err, rel_err = _max_err(got, ref)
        dev32, _ = _max_err(e32, ref)
        rows.append(parity_row(op, shape, torch.float32, direction, atol, 0.0, abs_err, rel_err,
                               abs_err <= atol, dev32))


def _module_fn(module):
    def fn(x, *rest):
        m = module.to(x.device, x.dtype)
        return m(x, *rest)

    return fn


def run_check(out: Path, quick: bool = False) -> int:
    status = _gpu_status()
    if status is not True:
        return _loud_skip(f"--check needs the HIP backend on a GPU: {status}")
    from .min_gru import DeltaMinGRU, GivensMinGRU, MinGRU, SignedMinGRU

    dev = torch.device("cuda")
    rows: list[dict] = []
    Ts, Bs = ((1, 13, 64), (2,)) if quick else (PARITY_TS, PARITY_BS)
    envelope = (1, 2, 8, 16) if quick else AFFINE_ENVELOPE
    seed = 0

    def case(op, ins, shp):
        nonlocal seed
        seed += 1
        tag = " ".join(f"{key}={v}" for key, v in shp.items())
        print(f"  {op} {tag}", flush=True)
        fn = _op_fn(op)
        _gate_rows(op, tag, fn, fn, ins, dev, rows, seed)

    # The reference's sweep: every scan op over T x B; matrix_affine_scan over the
    # whole (k, v) envelope with one plane, then k = 8, v = 4 with three planes.
    for B in Bs:
        for T in Ts:
            case("parallel_scan_log", *op_inputs("parallel_scan_log", B, T, 64, 1, seed))
            case("linear_scan", *op_inputs("linear_scan", B, T, 64, 1, seed))
            case("matrix_scan", *op_inputs("matrix_scan", B, T, 8, 2, seed))
            for k in envelope:
                for v in envelope:
                    case("matrix_affine_scan", *affine_inputs(B, T, 1, k, v, seed))
            case("matrix_affine_scan", *affine_inputs(B, T, 3, 8, 4, seed))
    # Mixer-level paths: the fused gate scans, the angle-fused Givens scan and the
    # chunked-WY delta rule (plain and decay-gated), each against its eager module.
    mixers = [
        ("MinGRU", lambda: MinGRU(8, 32), None),
        ("SignedMinGRU", lambda: SignedMinGRU(8, 32, coupled=True), None),
        ("GivensMinGRU", lambda: GivensMinGRU(8, 32, block_size=8), None),
        ("DeltaMinGRU", lambda: DeltaMinGRU(8, 32, n_heads=2, nh=2, chunk_size=16), None),
        ("DeltaMinGRU decay", lambda: DeltaMinGRU(8, 32, n_heads=2, chunk_size=16,
                                                  decay="learnable"), "dt"),
    ]
    for name, make, extra in mixers:
        for B, T in ((2, 40), (3, 129)) if not quick else ((2, 40),):
            seed += 1
            torch.manual_seed(seed)
            m = make()
            gen = _gen(seed)
            ins = [torch.randn(B, T, 8, generator=gen)]
            tag = f"B={B} T={T} in=8 hidden=32"
            if extra == "dt":
                dt = torch.rand(B, T, generator=gen)
                fn_h = (lambda mod, dtv: lambda x: mod.to(x.device, x.dtype)(
                    x, delta_t=dtv.to(x.device, x.dtype)))(m, dt)
                fn_r = fn_h
            else:
                fn_h = fn_r = _module_fn(m)
            _gate_rows(f"{name}.forward", tag, fn_h, fn_r, ins, dev, rows, seed)
    meta = run_meta(rows)
    _write(out, "scan_parity", {"meta": meta, "rows": rows}, parity_markdown(rows, meta))
    c = meta["counts"]
    print(f"parity: {c['passed']}/{c['total']} passed")
    return 0 if c["failed"] == 0 else 1


# ---------------------------------------------------------------------------
# --bench
# ---------------------------------------------------------------------------


def _time_us(fn, warmup: int, reps: int) -> float:
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) * 1000.0 / reps


def run_bench(out: Path, quick: bool = False) -> int:
    status = _gpu_status()
    if status is not True:
        return _loud_skip(f"--bench needs the HIP backend on a GPU: {status}")
    dev = torch.device("cuda")
    rows: list[dict] = []
    failed = 0
    shapes = (LAB_SHAPE, LONGT_SHAPE)
    for shape in shapes:
        warmup, reps = (2, 3) if quick else (shape["warmup"], shape["reps"])
        for op in OPS:
            fn = _op_fn(op)
            ins, shp = op_inputs(op, shape["B"], shape["T"], shape["d"], shape["k"])
            ins = [t.to(dev) for t in ins]
            for direction in DIRECTIONS:
                for impl in IMPLS:
                    try:
                        with _ScanMode(impl):
                            if direction == "fwd":
                                def step():
                                    with torch.no_grad():
                                        fn(*ins)
                            else:
                                leaves = [t.clone().requires_grad_(True) for t in ins]

                                def step():
                                    for x in leaves:
                                        x.grad = None
                                    outs = _outputs(fn(*leaves))
                                    sum(o.float().sum() for o in outs).backward()
                            us = _time_us(step, warmup, reps)
                    except (RuntimeError, torch.cuda.OutOfMemoryError) as exc:
                        print(f"  [skip] {op}/{shape['label']}/{impl}/{direction}: {exc}")
                        failed += 1
                        continue
                    print(f"  [ok]   {op}/{shape['label']}/{impl}/{direction}: {us:.2f} us/iter")
                    rows.append(bench_row(op, impl, shp, direction, us))
    meta = {"torch_version": torch.__version__, "device_name": torch.cuda.get_device_name(0),
            "warmup_reps": {s["label"]: {"warmup": s["warmup"], "reps": s["reps"]}
                            for s in shapes},
            "counts": {"attempted": len(rows) + failed, "succeeded": len(rows),
                       "failed": failed, "excluded_unavailable": 0}}
    _write(out, "scan_bench", {"meta": meta, "rows": rows}, bench_markdown(rows, meta))
    return 0 if failed == 0 else 1


# ---------------------------------------------------------------------------
# --memory
# ---------------------------------------------------------------------------


def run_memory(out: Path) -> int:
    status = _gpu_status()
    if status is not True:
        return _loud_skip(f"--memory needs the HIP backend on a GPU: {status}")
    from .min_gru import GivensMinGRU

    B, T, d, k = LAB_SHAPE["B"], LAB_SHAPE["T"], LAB_SHAPE["d"], LAB_SHAPE["k"]
    torch.manual_seed(0)
    m = GivensMinGRU(d, d, block_size=k, rounds=3).cuda()
    x = torch.randn(B, T, d, device="cuda")

    def once(mode):
        with _ScanMode(mode):
            m.zero_grad(set_to_none=True)
            m(x).float().sum().backward()
            m.zero_grad(set_to_none=True)
        torch.cuda.synchronize()

    def peak(mode):
        # Bytes allocated during one forward+backward above what was already live
        # when the window opened (the module, its input and anything an earlier
        # mode of this process left behind), plus the module and input themselves,
        # which a fresh process measuring only this step would hold too.
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        once(mode)
        return torch.cuda.max_memory_allocated() - base + own

    own = sum(p.numel() * p.element_size() for p in m.parameters()) + x.numel() * x.element_size()
    once("eager")
    once("hip")
    eager_b, hip_b = peak("eager"), peak("hip")
    shape = {"B": B, "T": T, "d": d, "k": k}
    rows = [{"impl": impl, "op": "GivensMinGRU.forward+backward", "shape": shape,
             "peak_bytes": b, "peak_mb": b / 2**20}
            for impl, b in (("eager_phase1_generic", eager_b), ("angle_fused_hip", hip_b))]
    md = ("# GivensMinGRU backward peak memory (angle-fused HIP vs generic eager)\n\n"
          f"Shape: {shape}\n\n"
          "Peak bytes allocated by one forward+backward above the allocations live when "
          "the measurement window opens, plus the module's parameters and its input.\n\n"
          "| impl | peak MB |\n| --- | --- |\n"
          + "".join(f"| {r['impl']} | {r['peak_mb']:.2f} |\n" for r in rows))
    _write(out, "scan_memory", {"rows": rows}, md)
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--check", action="store_true", help="gated parity cases -> scan_parity")
    ap.add_argument("--bench", action="store_true", help="timing matrix -> scan_bench")
    ap.add_argument("--memory", action="store_true", help="GivensMinGRU peak memory")
    ap.add_argument("--out", default="experiments/bench", help="artefact directory")
    ap.add_argument("--quick", action="store_true", help="fewer cases and reps (smoke runs)")
    args = ap.parse_args(argv)
    if not (args.check or args.bench or args.memory):
        ap.error("at least one of --check, --bench, --memory is required")
    out = Path(args.out)
    rc = 0
    if args.check:
        rc |= run_check(out, args.quick)
    if args.bench:
        rc |= run_bench(out, args.quick)
    if args.memory:
        rc |= run_memory(out)
    return rc


if __name__ == "__main__":
    raise SystemExit(main())
