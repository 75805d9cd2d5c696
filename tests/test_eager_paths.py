"""CPU tests of eager helpers the benchmark times and of the profile summarizer."""

import json
import os

import numpy as np
import pytest
import torch

from mingru_amd import profiling
from mingru_amd import workloads as wl
from mingru_amd.min_gru import GivensMinGRU, angle_scan_eager
from oracle import scans as orc


def _schedules():
    lex = wl.c4_inputs(2, 9, 3, 8)
    m = GivensMinGRU(4, 24, block_size=8, rounds=3)
    perm, sgn, p2p = m._angle_plane_meta(torch.device("cpu"))
    brick_theta = torch.randn(2, 9, 3, 3, 4, generator=torch.Generator().manual_seed(3))
    return {
        "lexicographic": (lex["theta"], lex["perm"], lex["sgn"], lex["p2p"]),
        "brick": (brick_theta, perm, sgn, p2p),
    }


@pytest.mark.parametrize("sched", ["lexicographic", "brick"])
@pytest.mark.parametrize("has_scale,has_decay", [(0, 1), (1, 0), (1, 1)])
def test_angle_scan_eager_matches_oracle(sched, has_scale, has_decay):
    """The materialised-M eager angle path (the C4 CPU baseline) against the float64
    oracle's step-by-step rotation scan and its adjoint, in float64."""
    theta, perm, sgn, p2p = _schedules()[sched]
    g = torch.Generator().manual_seed(11)
    Bn, T, n = theta.shape[:3]
    k = perm.shape[1]
    xs = {
        "theta": theta.double(),
        "scale": 0.5 + torch.rand(Bn, T, n, generator=g, dtype=torch.float64),
        "gamma": torch.rand(Bn, T, n, generator=g, dtype=torch.float64),
        "b": torch.randn(Bn, T, n, k, generator=g, dtype=torch.float64),
        "h0": torch.randn(Bn, n, k, generator=g, dtype=torch.float64),
    }
    gh = torch.randn(Bn, T, n, k, generator=g, dtype=torch.float64)
    req = {name: t.clone().requires_grad_(True) for name, t in xs.items()}
    h = angle_scan_eager(req["theta"], req["scale"], req["gamma"], req["b"], req["h0"], perm,
                         sgn, p2p, has_scale=has_scale, has_decay=has_decay)
    grads = torch.autograd.grad(h, list(req.values()), gh, allow_unused=True)
    args = [xs[n_].numpy() for n_ in ("theta", "scale", "gamma", "b", "h0")]
    args += [perm.numpy(), sgn.numpy(), p2p.numpy()]
    ref = orc.angle_scan(*args, has_scale, has_decay)
    np.testing.assert_allclose(h.detach().numpy(), ref, atol=1e-12)
    rg = orc.angle_scan_bwd(*args, has_scale, has_decay, gh.numpy())
    for name, got, want in zip(req, grads, rg):
        if (name == "scale" and not has_scale) or (name == "gamma" and not has_decay):
            assert got is None or float(got.abs().max()) == 0.0
            continue
        np.testing.assert_allclose(got.numpy(), want, atol=1e-11, err_msg=name)


def _write_counters(d, counter, rows):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "run_counter_collection.csv"), "w") as f:
        f.write('"Dispatch_Id","Kernel_Name","Counter_Name","Counter_Value"\n')
        for i, (name, val) in enumerate(rows):
            f.write(f'{i},"{name}","{counter}",{val}\n')


def test_profile_summary_attributes_traffic(tmp_path):
    """Kernels are attributed to entry points whatever their tile template arguments,
    counters are scaled by the copy probe, and an unmatched entry point is an error."""
    fwd = "void (anonymous namespace)::ew_fwd_kernel<4, 16, 8>(float const*, float*)"
    bwd = "void (anonymous namespace)::linear_bwd_kernel<4, 8, 8>(float const*, float*)"
    copy = "__amd_rocclr_copyBuffer"
    _write_counters(tmp_path / "f", "FETCH_SIZE",
                    [(copy, 524288.0), (copy, 3.0), (fwd, 100.0), (fwd, 300.0), (bwd, 50.0)])
    _write_counters(tmp_path / "w", "WRITE_SIZE", [(copy, 1048576.0), (fwd, 10.0), (bwd, 20.0)])
    os.makedirs(tmp_path / "s")
    with open(tmp_path / "s" / "run_kernel_stats.csv", "w") as f:
        f.write('"Name","Calls","TotalDurationNs","AverageNs","Percentage","MinNs","MaxNs"\n')
        f.write(f'"{bwd}",2,600,300.0,60.0,290,310\n"{fwd}",2,400,200.0,40.0,190,210\n')
    bench = {"ops": {"C2": {"kernels": {"mg_linear_scan_fwd": {
        "avg_us": 200.0, "algorithmic_bytes": 1000, "achieved_GBs": 5.0}},
        "ms_per_step": 0.5, "tokens_per_s": 1.0, "achieved_TBs": 1.0, "frac_of_hbm_peak": 0.1}}}
    (tmp_path / "b.json").write_text(json.dumps(bench) + "\n")
    out = tmp_path / "p.md"
    base = ["--workload", "C2", "--title", "t", "--stats", str(tmp_path / "s"),
            "--fetch", str(tmp_path / "f"), "--write", str(tmp_path / "w"),
            "--bench", str(tmp_path / "b.json"), "--out", str(out)]
    profiling.main(base + ["--command", "rocprofv3 x"])
    text = out.read_text()
    # fetch: probe reads 524288 KiB for 1 GiB -> x2; fwd averages 200 KiB -> 409600 bytes
    assert "traffic C2:mg_linear_scan_fwd 409600 10240" in text
    assert "traffic C2:mg_linear_scan_bwd 102400 20480" in text
    assert "ew_fwd_kernel<4, 16, 8>" in text and "rocprofv3 x" in text
    _write_counters(tmp_path / "v", "SQ_INSTS_VALU", [(fwd, 1000.0), (fwd, 3000.0), (bwd, 614400.0)])
    profiling.main(base + ["--valu", str(tmp_path / "v")])
    text = out.read_text()
    # per-call averages: fwd 2000, bwd 614400 wave instructions; the bwd floor is
    # 614400 * 4 cycles / 1024 SIMDs / 2400 MHz = 1.0 us
    assert "valu C2:mg_linear_scan_fwd 2000" in text
    assert "valu C2:mg_linear_scan_bwd 614400" in text
    assert profiling.valu_floor_us(614400) == pytest.approx(1.0)
    _write_counters(tmp_path / "w", "WRITE_SIZE", [(copy, 1048576.0), (fwd, 10.0)])
    with pytest.raises(SystemExit, match="linear_bwd"):
        profiling.main(base)


def test_profile_entry_patterns_split_angle_walk_kernels():
    """The angle scan's walk kernels are attributed by their direction argument, and the
    gate kernels by their gate kind and decay flag whatever their launch form."""
    import re

    sfwd, sbwd = (p for _, p in profiling.ENTRIES["C2g"])
    dfwd, dbwd = (p for _, p in profiling.ENTRIES["C2gd"])
    mfwd, mbwd = (p for _, p in profiling.ENTRIES["C1g"])
    pats = (sfwd, sbwd, dfwd, dbwd, mfwd, mbwd)
    for name, pat in (("gate_fwd_kernel<4, 16, 8, 0, false>", sfwd),
                      ("gate_fwd_kernel<4, 16, 8, 1, false, 2>", sfwd),
                      ("gate_bwd_kernel<1, 4, 8, 0, false, 1>", sbwd),
                      ("gate_fwd_kernel<4, 16, 8, 1, true, 3>", dfwd),
                      ("gate_bwd_kernel<2, 4, 8, 0, true>", dbwd),
                      ("gate_fwd_kernel<1, 8, 8, 2, false, 1>", mfwd),
                      ("gate_bwd_kernel<4, 4, 8, 2, false>", mbwd)):
        assert [bool(re.search(p, name)) for p in pats] == [p is pat for p in pats], name

    fwd, bwd = (p for _, p in profiling.ENTRIES["C4"])
    for name in ("angle_fwd_reduce<8, 1, false, true>", "angle_fwd_scan<8>",
                 "angle_group_walk_fill<8, false>", "angle_group_fill<8, false>"):
        assert re.search(fwd, name) and not re.search(bwd, name), name
    for name in ("angle_bwd_final<8, 1, false, true>", "angle_bwd_scan<8>",
                 "angle_group_walk_fill<8, true>", "angle_group_fill<8, true>",
                 "angle_group_offsets<8>"):
        assert re.search(bwd, name) and not re.search(fwd, name), name


def test_bench_reads_profile_lines(tmp_path, monkeypatch):
    """bench.py takes traffic and the VALU floor from the committed summaries' lines."""
    import importlib
    import sys

    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    bench = importlib.import_module("bench")
    (tmp_path / "profiles").mkdir()
    (tmp_path / "profiles" / "x.md").write_text(
        "text\n```\ntraffic C4:mg_angle_scan_fwd 300 200\nvalu C4:mg_angle_scan_fwd 614400\n```\n")
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    assert bench._traffic("C4:mg_angle_scan_fwd") == 500
    assert bench._valu_floor_us("C4:mg_angle_scan_fwd") == pytest.approx(1.0)
    assert bench._traffic("C4:mg_angle_scan_bwd") is None
    assert bench._valu_floor_us("C2:mg_linear_scan_fwd") is None
