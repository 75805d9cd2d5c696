"""The artefact driver writes the reference's schemas (``scripts/bench_scans.py``,
``src/mingru/triton_scans.py:2634-2679``).  CPU tests cover the row builders,
markdown, input shapes and the loud skip; the GPU test runs every mode once."""

import json

import pytest
import torch

from mingru_amd import bench_scans as bs

# Key sets of the reference's artefact rows, copied from its row builders.
REF_PARITY_KEYS = {"op", "shape", "dtype", "direction", "gate_atol", "gate_rtol", "max_abs_err",
                   "max_rel_err", "pass", "ref_fp64_dev"}
REF_BENCH_KEYS = {"op", "impl", "shape", "dtype", "direction", "us_per_iter"}
REF_MEMORY_KEYS = {"impl", "op", "shape", "peak_bytes", "peak_mb"}


def test_row_builders_match_reference_schemas():
    r = bs.parity_row("linear_scan", "B=2 T=3 D=4", torch.float32, "fwd", 1e-4, 0.0, 1e-7, 1e-8,
                      True, 2e-7)
    assert set(r) == REF_PARITY_KEYS and r["dtype"] == "float32" and r["pass"] is True
    b = bs.bench_row("linear_scan", "hip", {"B": 1, "T": 2, "D": 3}, "fwdbwd", 12.5)
    assert set(b) == REF_BENCH_KEYS and b["dtype"] == "float32"
    rows = [r, dict(r, direction="grad", **{"pass": False})]
    c = bs.parity_counts(rows)
    assert c["total"] == 2 and c["failed"] == 1
    assert c["by_direction"]["grad"] == {"total": 1, "passed": 0, "failed": 1}
    meta = bs.run_meta(rows)
    md = bs.parity_markdown(rows, meta)
    assert "| linear_scan | B=2 T=3 D=4 | float32 | fwd |" in md and "FAIL" in md
    bmd = bs.bench_markdown([b, dict(b, impl="eager", us_per_iter=25.0)],
                            {"torch_version": "x", "device_name": "y", "warmup_reps": {}})
    assert "2.00x" in bmd


@pytest.mark.parametrize("op", bs.OPS)
def test_op_inputs_have_mixer_shapes(op):
    ins, shape = bs.op_inputs(op, 2, 5, 16, 8)
    out = getattr(__import__("mingru_amd"), op)(*ins)  # eager on the CPU
    assert all(torch.isfinite(o).all() for o in (out if isinstance(out, tuple) else (out,)))
    assert shape["B"] == 2 and shape["T"] == 5


@pytest.mark.skipif(torch.cuda.is_available(), reason="the loud skip is the no-GPU behaviour")
def test_cpu_run_is_a_loud_skip(tmp_path, capsys):
    assert bs.main(["--check", "--bench", "--memory", "--out", str(tmp_path)]) == 0
    assert "SKIPPED (loud)" in capsys.readouterr().out
    assert not any(tmp_path.iterdir())


@pytest.mark.gpu
def test_gpu_artefacts(tmp_path):
    print("[gpu] bench_scans --check --bench --memory --quick", flush=True)
    rc = bs.main(["--check", "--bench", "--memory", "--quick", "--out", str(tmp_path)])
    par = json.loads((tmp_path / "scan_parity.json").read_text())
    assert all(set(r) == REF_PARITY_KEYS for r in par["rows"])
    failed = [r for r in par["rows"] if not r["pass"]]
    assert not failed, failed
    bench = json.loads((tmp_path / "scan_bench.json").read_text())
    assert all(set(r) == REF_BENCH_KEYS for r in bench["rows"])
    assert len(bench["rows"]) == 2 * len(bs.OPS) * 2 * 2  # shapes x ops x directions x impls
    mem = json.loads((tmp_path / "scan_memory.json").read_text())
    assert all(set(r) == REF_MEMORY_KEYS for r in mem["rows"])
    assert rc == 0


def test_affine_inputs_cover_the_envelope():
    """The parity sweep's generic (k, v) inputs: shapes, and transitions of spectral
    norm below 1 so products over the longest grid length stay finite."""
    assert bs.AFFINE_ENVELOPE == (1, 2, 4, 8, 16)
    assert bs.PARITY_TS == (1, 13, 64, 128, 1024) and bs.PARITY_BS == (2, 128)
    (A, Bm), shape = bs.affine_inputs(2, 5, 3, 16, 4, seed=1)
    assert A.shape == (2, 5, 3, 16, 16) and Bm.shape == (2, 5, 3, 16, 4)
    assert shape == {"B": 2, "T": 5, "n": 3, "k": 16, "v": 4}
    assert float(torch.linalg.matrix_norm(A.double(), ord=2).max()) < 1.0
