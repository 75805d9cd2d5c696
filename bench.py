#!/usr/bin/env python3
"""Benchmark of the minGRU scan hot path on one MI355X.

Metric: fwd+bwd tokens/s and achieved HBM TB/s (% of peak) per
scan op.  The headline JSON line is workload C2 (``linear_scan`` fwd+bwd,
B=16 T=4096 D=1024 fp32, BASELINE.json ``configs[1]``); the other workloads
are reported under ``"ops"`` in the same line.

A step is one forward + backward pass of the op through the public API
(``torch.autograd.grad`` on the HIP autograd Function) over one batch of
synthetic inputs already resident in HBM.  ``--warmup`` untimed steps, then
exactly ``--steps`` timed steps between two ``torch.cuda.synchronize()``.
Per-kernel device durations come from HIP events recorded around every C-ABI
launch on the launch stream; achieved bandwidth = algorithmic bytes per launch
/ that duration.  The CPU baseline times this package's eager path (the
reference algorithm on CPU tensors, all host threads) on a bounded batch slice
of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only C2,...]
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense bf16 (the delta kernels' MFMA type at C5)
MFMA_FP32_PEAK_TFLOPS = 157.3  # dense fp32 (the gated delta kernels' MFMA type)
HEADLINE = "C2"  # the workload BASELINE.json's metric is quoted on

METRIC = "fwd+bwd tokens/s + achieved HBM TB/s (% of peak) per scan op, 1 MI355X"


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", type=str, default="")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-eager", action="store_true",
                    help="skip the GPU comparison paths (eager delta loop, unfused gate path); "
                         "used under rocprof")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also time a plain 1 GiB device copy (rocprof counter calibration)")
    return ap.parse_args()


def _profile_line(kind: str, name: str):
    """Integers of the line ``<kind> <name> <int> ...`` in the committed rocprof
    summaries ``profiles/*.md``; ``None`` when no summary has one."""
    import glob
    import re

    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.md"))):
        with open(path) as f:
            for line in f:
                m = re.match(rf"^{kind} (\S+)((?: \d+)+)\s*$", line)
                if m and m.group(1) == name:
                    return [int(x) for x in m.group(2).split()]
    return None


def _traffic(name: str):
    """HBM bytes per C-ABI call (fetch + write) from the summaries' lines
    ``traffic <workload>:<entry> <fetch bytes> <write bytes>``."""
    v = _profile_line("traffic", name)
    return None if v is None else v[0] + v[1]


def _valu_floor_us(name: str):
    """VALU issue floor of one C-ABI call, from the summaries' lines
    ``valu <workload>:<entry> <wave64 VALU instructions per call>``: 4 cycles per
    instruction over MI355X's 1024 SIMDs at 2.4 GHz."""
    v = _profile_line("valu", name)
    return None if v is None else v[0] * 4 / 1024 / 2400


class Op:
    """One benchmark workload: input builder, one fwd+bwd step, byte (or FLOP) accounting."""

    def __init__(self, key, workload, tokens, fwd_entry, bwd_entry, fwd_bytes, bwd_bytes,
                 fwd_flops=None, bwd_flops=None, mfma=("bf16", MFMA_BF16_PEAK_TFLOPS)):
        self.key = key
        self.mfma = mfma  # (operand type, dense peak TFLOP/s) the FLOP figures are priced at
        self.workload = workload
        self.tokens = tokens
        self.fwd_entry = fwd_entry
        self.bwd_entry = bwd_entry
        self.fwd_bytes = fwd_bytes
        self.bwd_bytes = bwd_bytes
        self.fwd_flops = fwd_flops
        self.bwd_flops = bwd_flops


def build_ops(torch, wl):
    ops = {}

    # C2: linear_scan (headline)
    c = wl.C2
    N = c["B"] * c["T"] * c["D"]
    ops["C2"] = Op("C2", "C2 SignedMinGRU linear_scan fwd+bwd", c["B"] * c["T"],
                   "mg_linear_scan_fwd", "mg_linear_scan_bwd", 4 * N * 4, 6 * N * 4)
    # C2g: SignedMinGRU gates + linear_scan + h0 fused (same shape as C2).  Forward
    # reads s, z, hpre and writes h; backward reads s, z, hpre, dL/dh and writes
    # ds, dz, dhpre (h is read only at sub-chunk starts).
    ops["C2g"] = Op("C2g", "C2g SignedMinGRU fused gates + linear_scan fwd+bwd (C2 shape)",
                    c["B"] * c["T"], "mg_signed_gate_scan_fwd", "mg_signed_gate_scan_bwd",
                    4 * N * 4, 7 * N * 4)
    # C2gd: C2g with time decay, a = exp(-lam dt) tanh(s) formed in the kernel; dt (B,T)
    # and lam (D) add B*T + D floats, and the backward writes dL/dlam and dL/ddt partial
    # rows (B*chunks*D + ceil(D/64)*B*T floats).
    c = wl.C2
    bt = c["B"] * c["T"]
    part = (c["B"] * -(-c["T"] // 32) * c["D"] + -(-c["D"] // 64) * bt) * 4
    ops["C2gd"] = Op("C2gd", "C2gd SignedMinGRU fused gates with time decay + linear_scan "
                     "fwd+bwd (C2 shape)", bt, "mg_signed_gate_scan_decay_fwd",
                     "mg_signed_gate_scan_decay_bwd", 4 * N * 4 + (bt + c["D"]) * 4,
                     7 * N * 4 + (bt + c["D"]) * 4 + part)
    # C1: parallel_scan_log
    c = wl.C1
    N = c["B"] * c["T"] * c["D"]
    N1 = c["B"] * (c["T"] + 1) * c["D"]
    ops["C1"] = Op("C1", "C1 MinGRU parallel_scan_log fwd+bwd", c["B"] * c["T"],
                   "mg_log_scan_fwd", "mg_log_scan_bwd", (2 * N + N1) * 4, (3 * N + 2 * N1) * 4)
    # C1g: MinGRU log-space gates + parallel_scan_log fused (C1 shape).  Forward reads
    # k, hpre and writes h; backward reads k, hpre, dL/dh and writes dk, dhpre.
    ops["C1g"] = Op("C1g", "C1g MinGRU fused gates + parallel_scan_log fwd+bwd (C1 shape)",
                    c["B"] * c["T"], "mg_mingru_gate_scan_fwd", "mg_mingru_gate_scan_bwd",
                    3 * N * 4, 5 * N * 4)
    # C3: 2x2 matrix_affine_scan and matrix_scan (b = 0)
    c = wl.C3
    P = c["B"] * c["T"] * c["n"]
    ops["C3"] = Op("C3", "C3 RotationMinGRU 2x2 matrix_affine_scan fwd+bwd", c["B"] * c["T"],
                   "mg_affine_scan_fwd", "mg_affine_scan_bwd", 12 * P * 4, 18 * P * 4)
    ops["C3m"] = Op("C3m", "C3 matrix_scan (b=0) fwd+bwd", c["B"] * c["T"],
                    "mg_affine_scan_fwd", "mg_affine_scan_bwd", 12 * P * 4, 18 * P * 4)
    # C4: angle-fused Givens, 28 lexicographic rotations, decay
    c = wl.C4
    L = c["B"] * c["T"] * c["n"]
    h0b = c["B"] * c["n"] * c["k"] * 4
    ops["C4"] = Op("C4", "C4 GivensMinGRU angle-fused (28 lexicographic rotations) fwd+bwd",
                   c["B"] * c["T"], "mg_angle_scan_fwd", "mg_angle_scan_bwd",
                   180 * L + h0b, 328 * L + 2 * h0b)
    # C4g: GivensMinGRU's brick-wall scan (k=8, 3 rounds) at the C4 shape with the heads
    # b = sigmoid(z) * hpre formed in the kernel and decay.  Per block-token: forward reads
    # theta (12 floats), gamma, z, hpre (8 each) and writes h; backward reads theta, gamma,
    # z, hpre, h, dL/dh and writes dtheta, dgamma, dz, dhpre.
    c = wl.C4
    L = c["B"] * c["T"] * c["n"]
    h0b = c["B"] * c["n"] * c["k"] * 4
    ops["C4g"] = Op("C4g", "C4g GivensMinGRU brick-wall (k=8, 3 rounds) with the gated heads "
                    "in the kernel, decay, fwd+bwd (C4 shape)", c["B"] * c["T"],
                    "mg_angle_scan_gated_fwd", "mg_angle_scan_gated_bwd",
                    (12 + 1 + 8 + 8 + 8) * 4 * L + h0b, (12 + 1 + 8 + 8 + 8 + 8 + 12 + 1 + 8 + 8)
                    * 4 * L + 2 * h0b)
    # C5: DeltaMinGRU chunked-WY, bf16 inputs.  FLOP floor: per (b, h) and chunk of
    # C tokens, six C x C x d products and one triangular solve (C^3), i.e.
    # 6 * 2 C^3 + C^3 = 13 C^3 at C = d = 64; the backward is counted as 2x the
    # forward (fwd+bwd = 3x fwd), the convention of the reference's delta probe.
    c = wl.C5
    n_chunk = c["B"] * c["H"] * (c["T"] // c["chunk"])
    f_fwd = 13 * c["chunk"] ** 3 * n_chunk
    bt = c["B"] * c["H"] * c["T"] * c["d"] * 2  # one bf16 (B,H,T,d) tensor
    ops["C5"] = Op("C5", "C5 DeltaMinGRU chunked-WY fwd+bwd (bf16 in, fp32 state)",
                   c["B"] * c["T"], "mg_delta_fwd", "mg_delta_bwd",
                   4 * bt + bt // c["d"], 7 * bt + 2 * bt // c["d"], f_fwd, 2 * f_fwd)
    # C5d: C5 with per-token decay on the gated kernels (bf16 in, fp32 state and decay).
    # Bytes: as C5 plus log_gamma (fp32, (B,H,T)) read forward and backward and dlog_gamma
    # written.  Same FLOP floor as C5.
    lgb = c["B"] * c["H"] * c["T"] * 4
    ops["C5d"] = Op("C5d", "C5d DeltaMinGRU decay-gated chunked-WY fwd+bwd (C5 shape, bf16 in)",
                    c["B"] * c["T"], "mg_delta_gated_fwd", "mg_delta_gated_bwd",
                    4 * bt + bt // c["d"] + lgb, 7 * bt + 2 * bt // c["d"] + 2 * lgb, f_fwd,
                    2 * f_fwd)
    # C5dp: C5d with nh = 2 micro-steps per token (DeltaProduct), bf16: K, V, beta carry
    # two micro-steps per token; the kernels tile 32 tokens (64 micro-steps) per chunk.
    # FLOP floor as C5's per 64-micro-step tile (twice the tiles of C5).
    nh = 2
    bk = bt * nh  # one bf16 (B,H,T,nh,d) tensor
    ops["C5dp"] = Op("C5dp", "C5dp DeltaMinGRU decay-gated DeltaProduct nh=2 fwd+bwd (C5 shape, "
                     "bf16 in)", c["B"] * c["T"], "mg_delta_gated_fwd", "mg_delta_gated_bwd",
                     2 * bt + 2 * bk + bk // c["d"] + lgb,
                     3 * bt + 4 * bk + 2 * bk // c["d"] + 2 * lgb, nh * f_fwd, 2 * nh * f_fwd)
    return ops


def make_step(key, torch, wl, dev):
    """Returns (step_fn, cpu_step_fn(batch_slice) or None)."""
    import mingru_amd as mg

    if key == "C2":
        inp = wl.c2_inputs(**wl.C2)
        a = inp["a"].to(dev).requires_grad_(True)
        b = inp["b"].to(dev).requires_grad_(True)
        gA, gB = inp["grad_A"].to(dev), inp["grad_Bc"].to(dev)

        def step():
            A, Bc = mg.linear_scan(a, b)
            return torch.autograd.grad((A, Bc), (a, b), (gA, gB))

        def cpu(bs):
            ac = inp["a"][:bs].clone().requires_grad_(True)
            bc = inp["b"][:bs].clone().requires_grad_(True)
            A, Bc = mg.linear_scan(ac, bc)
            torch.autograd.grad((A, Bc), (ac, bc), (inp["grad_A"][:bs], inp["grad_Bc"][:bs]))

        return step, cpu, wl.C2["B"]
    if key == "C2g":
        from mingru_amd.min_gru import _dispatch_signed_gate_scan

        inp = wl.c2g_inputs(**wl.C2)
        xs = [inp[k].to(dev).requires_grad_(True) for k in ("s", "z", "hpre")]
        h0 = inp["h0"].to(dev)
        gh = inp["grad_h"].to(dev)

        def step():
            h = _dispatch_signed_gate_scan(*xs, h0, coupled=False)
            return torch.autograd.grad(h, xs, gh)

        return step, None, wl.C2["B"]
    if key == "C2gd":
        from mingru_amd.min_gru import _dispatch_signed_gate_scan

        inp = wl.c2gd_inputs(**wl.C2)
        xs = [inp[k].to(dev).requires_grad_(True) for k in ("s", "z", "hpre")]
        h0 = inp["h0"].to(dev)
        dt, lam = inp["dt"].to(dev), inp["lam"].to(dev).requires_grad_(True)
        gh = inp["grad_h"].to(dev)

        def step():
            h = _dispatch_signed_gate_scan(*xs, h0, coupled=False, dt=dt, lam=lam)
            return torch.autograd.grad(h, xs + [lam], gh)

        return step, None, wl.C2["B"]
    if key == "C4g":
        from mingru_amd import hip_scans

        inp = wl.c4g_inputs(**wl.C4)
        th, gm, z, hp, h0 = (inp[k].to(dev).requires_grad_(True)
                             for k in ("theta", "gamma", "z", "hpre", "h0"))
        meta = [t.to(dev) for t in hip_scans._brick_tables(wl.C4["k"], 3)]
        gh = inp["grad_h"].to(dev)

        def step():
            h = hip_scans.angle_gated_scan_impl(th, None, gm, z, hp, h0, *meta, has_scale=0,
                                                has_decay=1)
            return torch.autograd.grad(h, (th, gm, z, hp, h0), gh)

        return step, None, wl.C4["B"]
    if key == "C1g":
        from mingru_amd.min_gru import _dispatch_mingru_gate_scan

        inp = wl.c1g_inputs(**wl.C1)
        xs = [inp[k].to(dev).requires_grad_(True) for k in ("k", "hpre")]
        lh0 = inp["log_h0"].to(dev)
        gh = inp["grad_h"].to(dev)

        def step():
            h = _dispatch_mingru_gate_scan(*xs, lh0)
            return torch.autograd.grad(h, xs, gh)

        return step, None, wl.C1["B"]
    if key == "C1":
        inp = wl.c1_inputs(**wl.C1)
        lc = inp["log_coeffs"].to(dev).requires_grad_(True)
        lv = inp["log_values"].to(dev).requires_grad_(True)
        gh = inp["grad_h"].to(dev)

        def step():
            h = mg.parallel_scan_log(lc, lv)
            return torch.autograd.grad(h, (lc, lv), gh)

        def cpu(bs):
            lcc = inp["log_coeffs"][:bs].clone().requires_grad_(True)
            lvc = inp["log_values"][:bs].clone().requires_grad_(True)
            h = mg.parallel_scan_log(lcc, lvc)
            torch.autograd.grad(h, (lcc, lvc), inp["grad_h"][:bs])

        return step, cpu, wl.C1["B"]
    if key in ("C3", "C3m"):
        inp = wl.c3_inputs(**wl.C3)
        A = inp["A"].to(dev).requires_grad_(True)
        if key == "C3":
            Bm = inp["Bm"].to(dev).requires_grad_(True)
            gA, gB = inp["grad_Abar"].to(dev), inp["grad_Bbar"].to(dev)

            def step():
                Abar, Bbar = mg.matrix_affine_scan(A, Bm)
                return torch.autograd.grad((Abar, Bbar), (A, Bm), (gA, gB))

            def cpu(bs):
                Ac = inp["A"][:bs].clone().requires_grad_(True)
                Bc = inp["Bm"][:bs].clone().requires_grad_(True)
                Abar, Bbar = mg.matrix_affine_scan(Ac, Bc)
                torch.autograd.grad((Abar, Bbar), (Ac, Bc),
                                    (inp["grad_Abar"][:bs], inp["grad_Bbar"][:bs]))
        else:
            b0 = torch.zeros(inp["Bm"].shape[:-1], device=dev).requires_grad_(True)
            gA, gB = inp["grad_Abar"].to(dev), inp["grad_Bbar"][..., 0].to(dev)

            def step():
                Abar, Bc = mg.matrix_scan(A, b0)
                return torch.autograd.grad((Abar, Bc), (A, b0), (gA, gB))

            def cpu(bs):
                Ac = inp["A"][:bs].clone().requires_grad_(True)
                bc = torch.zeros(inp["Bm"][:bs].shape[:-1]).requires_grad_(True)
                Abar, Bc = mg.matrix_scan(Ac, bc)
                torch.autograd.grad((Abar, Bc), (Ac, bc),
                                    (inp["grad_Abar"][:bs], inp["grad_Bbar"][:bs, ..., 0]))
        return step, cpu, wl.C3["B"]
    if key == "C4":
        from mingru_amd import hip_scans

        inp = wl.c4_inputs(**wl.C4)
        th = inp["theta"].to(dev).requires_grad_(True)
        gm = inp["gamma"].to(dev).requires_grad_(True)
        bb = inp["b"].to(dev).requires_grad_(True)
        h0 = inp["h0"].to(dev).requires_grad_(True)
        sc = inp["scale"].to(dev)
        meta = [inp[k].to(dev) for k in ("perm", "sgn", "p2p")]
        gh = inp["grad_h"].to(dev)

        def step():
            h = hip_scans.angle_scan_impl(th, sc, gm, bb, h0, *meta, has_scale=0, has_decay=1)
            return torch.autograd.grad(h, (th, gm, bb, h0), gh)

        def cpu(bs):
            # The eager path: every 8x8 transition materialised from its 28 angles,
            # then the eager matrix_affine_scan (reference GivensMinGRU fallback).
            from mingru_amd.min_gru import angle_scan_eager

            xc = [inp[k][:bs].clone().requires_grad_(True) for k in ("theta", "gamma", "b", "h0")]
            h = angle_scan_eager(xc[0], inp["scale"][:bs], xc[1], xc[2], xc[3], inp["perm"],
                                 inp["sgn"], inp["p2p"], has_scale=0, has_decay=1)
            torch.autograd.grad(h, xc, inp["grad_h"][:bs])

        return step, cpu, wl.C4["B"]
    if key == "C5":
        from mingru_amd import hip_scans

        inp = wl.c5_inputs(**wl.C5)
        xs = [inp[k].to(dev).requires_grad_(True) for k in ("Q", "K", "V", "beta", "H0")]
        gy = inp["grad_y"].to(dev).to(torch.bfloat16)
        gH = inp["grad_HT"].to(dev)
        C = inp["chunk_size"]

        def step():
            y, HT = hip_scans.delta_scan_impl(*xs, chunk_size=C)
            return torch.autograd.grad((y, HT), xs, (gy, gH))

        def cpu(bs):
            from mingru_amd.min_gru import delta_chunked_eager

            xc = [inp[k][:bs].float().clone().requires_grad_(True)
                  for k in ("Q", "K", "V", "beta", "H0")]
            y, HT = delta_chunked_eager(*xc, C)
            torch.autograd.grad((y, HT), xc, (inp["grad_y"][:bs].permute(0, 2, 1, 3),
                                              inp["grad_HT"][:bs]))

        return step, cpu, wl.C5["B"]
    if key in ("C5d", "C5dp"):
        from mingru_amd import hip_scans

        inp = wl.c5d_inputs(**wl.C5, nh=2 if key == "C5dp" else 1)
        names = ("Q", "K", "V", "beta", "log_gamma", "H0")
        xs = [inp[k].to(dev).requires_grad_(True) for k in names]
        gy = inp["grad_y"].to(dev).to(inp["Q"].dtype)
        gH = inp["grad_HT"].to(dev)
        C = inp["chunk_size"]

        def step():
            y, HT = hip_scans.delta_gated_scan_impl(*xs, chunk_size=C)
            return torch.autograd.grad((y, HT), xs, (gy, gH))

        return step, None, wl.C5["B"]
    raise KeyError(key)


def gate_unfused_gpu_ms(key, torch, wl, dev, steps):
    """The unfused mixer path that a fused gate op replaces, fwd+bwd, ms per step over
    `steps` steps.  C2g: SignedMinGRU's eager gates on the GPU, the HIP linear_scan,
    then h = A * h0 + Bc; C2gd the same with the decay exp(-lam dt) applied eagerly.
    C1g: MinGRU's eager log-space gates, the concatenation with log h0 and the HIP
    parallel_scan_log.  C4g: GivensMinGRU's eager b = sigmoid(z) * hpre and the HIP
    angle scan."""
    import torch.nn.functional as F

    import mingru_amd as mg
    from mingru_amd.min_gru import log_g

    if key == "C2g":
        inp = wl.c2g_inputs(**wl.C2)
        s, z, hp = (inp[k].to(dev).requires_grad_(True) for k in ("s", "z", "hpre"))
        h0 = inp["h0"].to(dev)
        gh = inp["grad_h"].to(dev)

        def step():
            sg = torch.sigmoid(z)
            A, Bc = mg.linear_scan(torch.tanh(s), sg * hp)
            torch.autograd.grad(A * h0 + Bc, (s, z, hp), gh)
    elif key == "C2gd":
        inp = wl.c2gd_inputs(**wl.C2)
        s, z, hp = (inp[k].to(dev).requires_grad_(True) for k in ("s", "z", "hpre"))
        h0 = inp["h0"].to(dev)
        dt, lam = inp["dt"].to(dev), inp["lam"].to(dev).requires_grad_(True)
        gh = inp["grad_h"].to(dev)

        def step():
            a = torch.exp(-lam * dt.unsqueeze(-1)) * torch.tanh(s)
            A, Bc = mg.linear_scan(a, torch.sigmoid(z) * hp)
            torch.autograd.grad(A * h0 + Bc, (s, z, hp, lam), gh)
    elif key == "C4g":
        from mingru_amd import hip_scans

        inp = wl.c4g_inputs(**wl.C4)
        th, gm, z, hp, h0 = (inp[k].to(dev).requires_grad_(True)
                             for k in ("theta", "gamma", "z", "hpre", "h0"))
        meta = [t.to(dev) for t in hip_scans._brick_tables(wl.C4["k"], 3)]
        ones = torch.ones(gm.shape, device=dev)
        gh = inp["grad_h"].to(dev)

        def step():
            b = torch.sigmoid(z) * hp
            h = hip_scans.angle_scan_impl(th, ones, gm, b, h0, *meta, has_scale=0, has_decay=1)
            torch.autograd.grad(h, (th, gm, z, hp, h0), gh)
    else:
        inp = wl.c1g_inputs(**wl.C1)
        k, hp = (inp[n].to(dev).requires_grad_(True) for n in ("k", "hpre"))
        lh0 = inp["log_h0"].to(dev)
        gh = inp["grad_h"].to(dev)

        def step():
            lv = torch.cat([lh0, -F.softplus(-k) + log_g(hp)], dim=1)
            h = mg.parallel_scan_log(-F.softplus(k), lv)
            torch.autograd.grad(h, (k, hp), gh)

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def delta_eager_gpu_ms(torch, wl, dev, reps=3):
    """The eager chunked-WY loop (torch ops on the GPU, fp32 since the triangular
    solve has no bf16 kernel) fwd+bwd at C5; returns the median ms per step."""
    from mingru_amd.min_gru import delta_chunked_eager

    inp = wl.c5_inputs(**wl.C5)
    xs = [inp[k].to(dev).float().requires_grad_(True) for k in ("Q", "K", "V", "beta", "H0")]
    gy = inp["grad_y"].to(dev).float().permute(0, 2, 1, 3)
    gH = inp["grad_HT"].to(dev)

    def step():
        y, HT = delta_chunked_eager(*xs, inp["chunk_size"])
        torch.autograd.grad((y, HT), xs, (gy, gH))

    step()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        step()
        torch.cuda.synchronize()
        ts.append((time.perf_counter() - t0) * 1e3)
    ts.sort()
    return ts[len(ts) // 2]


def delta_gated_fp32_kernels_ms(torch, wl, dev, steps, nh=1):
    """The decay-gated workload with fp32 inputs, i.e. on the fp32-operand gated kernels,
    fwd+bwd; ms per step over `steps` steps."""
    from mingru_amd import hip_scans

    inp = wl.c5d_inputs(**wl.C5, nh=nh)
    names = ("Q", "K", "V", "beta", "log_gamma", "H0")
    xs = [inp[k].to(dev).float().requires_grad_(True) for k in names]
    gy = inp["grad_y"].to(dev)
    gH = inp["grad_HT"].to(dev)

    def step():
        y, HT = hip_scans.delta_gated_scan_impl(*xs, chunk_size=inp["chunk_size"])
        torch.autograd.grad((y, HT), xs, (gy, gH))

    for _ in range(2):
        step()
    return _timed(step, steps, torch)


def delta_gated_eager_gpu_ms(torch, wl, dev, reps=3):
    """The eager decay-gated chunked-WY loop (the module's ``_forward_chunked_gated``,
    torch ops on the GPU, fp32 since the triangular solve has no bf16 kernel) fwd+bwd
    at C5d; returns the median ms per step."""
    from mingru_amd.min_gru import delta_chunked_gated_eager

    inp = wl.c5d_inputs(**wl.C5)
    names = ("Q", "K", "V", "beta", "log_gamma", "H0")
    xs = [inp[k].to(dev).float().requires_grad_(True) for k in names]
    gy = inp["grad_y"].to(dev).permute(0, 2, 1, 3)
    gH = inp["grad_HT"].to(dev)

    def step():
        y, HT = delta_chunked_gated_eager(*xs, inp["chunk_size"])
        torch.autograd.grad((y, HT), xs, (gy, gH))

    step()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        step()
        torch.cuda.synchronize()
        ts.append((time.perf_counter() - t0) * 1e3)
    ts.sort()
    return ts[len(ts) // 2]


def decode_bench(torch, wl, dev, steps):
    """Streaming decode: one recurrent step per call, fused kernel vs the eager step body on
    the GPU (the same arithmetic as the mixers' step()), median over `steps` calls.

    D5: DeltaMinGRU state update at C5's heads (B=8, H=8, d_k=d_v=64, nh=1, with decay);
        bytes = the state read and written plus q, k, v, beta.
    D2: SignedMinGRU step at C2's width (B=16, D=1024); bytes = s, z, hpre, h_prev in, h out.
    """
    from mingru_amd import hip_scans

    g = torch.Generator().manual_seed(1099)
    out = {}
    c = wl.C5
    B, Hh, d = c["B"], c["H"], c["d"]
    H = torch.randn(B, Hh, d, d, generator=g).to(dev)
    q = torch.randn(B, Hh, d, generator=g).to(dev)
    K = torch.nn.functional.normalize(torch.randn(B, Hh, 1, d, generator=g), dim=-1).to(dev)
    V = torch.randn(B, Hh, 1, d, generator=g).to(dev)
    beta = torch.rand(B, Hh, 1, generator=g).to(dev)
    lg = -torch.rand(B, Hh, generator=g).to(dev)

    def fused5():
        return hip_scans.delta_step_impl(H, q, K, V, beta, lg)

    def eager5():
        Hx = torch.exp(lg)[..., None, None] * H
        k, v, bt = K[:, :, 0], V[:, :, 0], beta[:, :, 0]
        kH = torch.einsum("bhk,bhkv->bhv", k, Hx)
        Hx = Hx + bt[..., None, None] * torch.einsum("bhk,bhv->bhkv", k, v - kH)
        return torch.einsum("bhk,bhkv->bhv", q, Hx), Hx

    b5 = 2 * H.numel() * 4 + (q.numel() + K.numel() + V.numel() + beta.numel() + lg.numel()) * 4
    c2 = wl.C2
    n = c2["B"] * c2["D"]
    s_, z_, hp_, h_ = (torch.randn(c2["B"], c2["D"], generator=g).to(dev) for _ in range(4))

    def fused2():
        return hip_scans.gate_step_impl("signed", s_, z_, hp_, None, h_)

    def eager2():
        return torch.tanh(s_) * h_ + torch.sigmoid(z_) * hp_

    for key, fused, eager, nbytes, tok in (("D5", fused5, eager5, b5, B),
                                            ("D2", fused2, eager2, 5 * n * 4, c2["B"])):
        res = {}
        for name, fn in (("fused", fused), ("eager", eager)):
            with torch.no_grad():
                for _ in range(5):
                    fn()
                torch.cuda.synchronize()
                # latency: one step, then wait for it (a decode loop that reads each result)
                ts = []
                for _ in range(steps):
                    t0 = time.perf_counter()
                    fn()
                    torch.cuda.synchronize()
                    ts.append((time.perf_counter() - t0) * 1e6)
                # throughput: 10 * steps calls queued back to back, one wait at the end
                t0 = time.perf_counter()
                for _ in range(10 * steps):
                    fn()
                torch.cuda.synchronize()
                tput = (time.perf_counter() - t0) * 1e6 / (10 * steps)
            ts.sort()
            res[f"{name}_us_per_step"] = ts[len(ts) // 2]
            res[f"{name}_us_per_step_queued"] = tput
        res["speedup_vs_eager"] = res["eager_us_per_step"] / res["fused_us_per_step"]
        res["speedup_vs_eager_queued"] = (res["eager_us_per_step_queued"]
                                          / res["fused_us_per_step_queued"])
        res["bytes_per_step"] = nbytes
        res["tokens_per_step"] = tok
        out[key] = res
    return out


def _timed(step, steps, torch):
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def graphed_ms(step, torch, steps):
    """ms per step of ``step`` (forward + autograd.grad) captured once in a HIP graph and
    replayed: the launch-bound workloads' kernels with no host dispatch between them.  The
    warm-up runs on the capture stream, so the scan workspace of that stream exists before
    capture and nothing is allocated or filled inside it.  The first replay's gradients are
    checked against an eager step before timing."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = step()
    g.replay()
    ref = step()
    torch.cuda.synchronize()
    for x, r in zip(out, ref):
        if not torch.allclose(x, r, rtol=1e-5, atol=1e-6):
            raise RuntimeError("graph replay disagrees with the eager step")
    return _timed(g.replay, steps, torch)


def run_op(op, torch, wl, dev, steps, warmup, hip_scans, headline=False):
    """Times `steps` steps after `warmup` untimed ones.  Per-kernel durations come
    from HIP events recorded around every C-ABI call.  For the headline workload
    the events are recorded inside the timed region itself (its GPU time hides
    their host cost).  For the others the timed steps run uninstrumented and a
    second, instrumented pass of the same length supplies the kernel durations:
    recording an event costs tens of microseconds of host time, which would
    dominate a launch-bound step such as C1."""
    step, cpu_step, B = make_step(op.key, torch, wl, dev)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    n = steps
    if not headline:
        # A workload whose step takes microseconds is timed over at least ~50 ms of
        # steps (at most 2000), after as many warm-up steps again: a 20-step window of
        # such a step measures the GPU's wake-up from the idle CPU-baseline phase
        # before it rather than the steady state.
        est = _timed(step, 5, torch)
        n = max(steps, min(2000, int(50.0 / max(est, 1e-3))))
        if n > steps:
            _timed(step, n, torch)
    ms_plain = None if headline else _timed(step, n, torch)
    with hip_scans.kernel_timer(prealloc=2 * n + 16) as timer:
        ms_instr = _timed(step, n, torch)
    ms = ms_instr if headline else ms_plain
    durs = timer.durations_ms()
    kern = {}
    for entry, nbytes, nflops in ((op.fwd_entry, op.fwd_bytes, op.fwd_flops),
                                  (op.bwd_entry, op.bwd_bytes, op.bwd_flops)):
        d = durs.get(entry, [])
        if not d:
            continue
        d = sorted(d)
        avg = sum(d) / len(d)
        kern[entry] = {
            "avg_us": avg * 1e3,
            "median_us": d[len(d) // 2] * 1e3,
            "algorithmic_bytes": nbytes,
            "achieved_GBs": nbytes / (avg * 1e-3) / 1e9,
        }
        if nflops is not None:
            kern[entry]["algorithmic_flops"] = nflops
            kern[entry]["achieved_TFLOPs"] = nflops / (avg * 1e-3) / 1e12
    total_bytes = op.fwd_bytes + op.bwd_bytes
    res = {
        "workload": op.workload,
        "tokens_per_s": op.tokens / (ms * 1e-3),
        "ms_per_step": ms,
        "algorithmic_bytes": total_bytes,
        "achieved_TBs": total_bytes / (ms * 1e-3) / 1e12,
        "frac_of_hbm_peak": total_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "kernels": kern,
        "ms_per_step_instrumented": ms_instr,
        "timed_steps": n,
    }
    if op.key in ("C1", "C1g"):  # host-bound: also the GPU-side rate, replayed from a graph
        gms = graphed_ms(step, torch, steps)
        res["graph_ms_per_step"] = gms
        res["graph_tokens_per_s"] = op.tokens / (gms * 1e-3)
    if op.fwd_flops is not None:
        fl = op.fwd_flops + op.bwd_flops
        res["algorithmic_flops"] = fl
        res["achieved_TFLOPs"] = fl / (ms * 1e-3) / 1e12
        res[f"frac_of_{op.mfma[0]}_mfma_peak"] = res["achieved_TFLOPs"] / op.mfma[1]
    return res, cpu_step, B


def cpu_baseline(cpu_step, B_full, tokens_full, torch, budget_s=12.0):
    """Time the eager CPU path (this package's restatement of the reference's eager
    algorithm, run on CPU tensors with every host thread) on a batch slice of the
    same inputs: the slice doubles until one step takes >= 1 s (or is the whole
    batch), then 1 warm-up and up to 5 timed reps within ``budget_s``."""
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    prev = os.environ.get("MINGRU_SCAN")
    os.environ["MINGRU_SCAN"] = "eager"
    try:
        bs = 1
        while True:
            t0 = time.perf_counter()
            cpu_step(bs)  # warm-up at this slice
            warm = time.perf_counter() - t0
            if warm >= 1.0 or bs >= B_full:
                break
            bs = min(B_full, 2 * bs)
        reps = max(1, min(5, int(budget_s / max(warm, 1e-3))))
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            cpu_step(bs)
            times.append(time.perf_counter() - t0)
    finally:
        if prev is None:
            os.environ.pop("MINGRU_SCAN", None)
        else:
            os.environ["MINGRU_SCAN"] = prev
    times.sort()
    med = times[len(times) // 2]
    tokens_slice = tokens_full * bs // B_full
    return {
        "value": tokens_slice / med,
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"eager torch CPU fwd+bwd on batch slice {bs}/{B_full} of the same inputs "
                  f"(1 warm-up, median of {reps}; min {tokens_slice / times[0]:.4g} tokens/s); "
                  f"os.cpu_count()={os.cpu_count()}, cpu={_cpu_model()}",
    }


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def copy_probe(torch, dev, nbytes=1 << 30, reps=20):
    """A plain device-to-device copy of ``nbytes``: the streaming ceiling of this
    GPU, and the known-size kernel that calibrates rocprof's FETCH_SIZE /
    WRITE_SIZE counters."""
    src = torch.randn(nbytes // 4, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record()
    for _ in range(reps):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / reps
    return {"bytes_read": nbytes, "bytes_written": nbytes, "avg_us": us,
            "achieved_GBs": 2 * nbytes / (us * 1e-6) / 1e9}


def main():
    args = _parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1 "
                          "(the scan path would shard over batch rows and lanes with no "
                          "communication between GPUs)"}))
        sys.exit(2)
    import torch

    from mingru_amd import hip_scans
    from mingru_amd import workloads as wl

    status = hip_scans.available()
    if status is not True:
        raise SystemExit(f"HIP backend unavailable: {status}")
    os.environ["MINGRU_SCAN"] = "hip"
    dev = torch.device("cuda:0")
    ops = build_ops(torch, wl)
    order = ["C2", "C2g", "C2gd", "C1", "C1g", "C3", "C3m", "C4", "C4g", "C5", "C5d", "C5dp"]
    if args.only:
        order = [k for k in order if k in args.only.split(",")]
    results = {}
    cpu = None
    for key in order:
        if key not in ops:
            continue
        res, cpu_step, B = run_op(ops[key], torch, wl, dev, args.steps, args.warmup, hip_scans,
                                  headline=(key == HEADLINE))
        results[key] = res
        floors = {e: _valu_floor_us(f"{key}:{e}") for e in res["kernels"]}
        if floors and all(v is not None for v in floors.values()):
            for e, fl in floors.items():
                res["kernels"][e]["valu_floor_us"] = fl
            res["valu_floor_ms"] = sum(floors.values()) / 1e3
            res["frac_of_valu_floor"] = res["valu_floor_ms"] / res["ms_per_step"]
        print(f"# {key}: {res['tokens_per_s']:.4g} tok/s, {res['ms_per_step']:.3f} ms/step, "
              f"{res['achieved_TBs']:.3f} TB/s ({100 * res['frac_of_hbm_peak']:.1f}% of peak)",
              file=sys.stderr, flush=True)
        for kname, kres in res["kernels"].items():
            print(f"#   {kname}: {kres['avg_us']:.1f} us, {kres['achieved_GBs']:.0f} GB/s",
                  file=sys.stderr, flush=True)
        if "graph_ms_per_step" in res:
            print(f"#   replayed from a HIP graph: {res['graph_ms_per_step']:.3f} ms/step, "
                  f"{res['graph_tokens_per_s']:.4g} tok/s", file=sys.stderr, flush=True)
        if key in ("C2g", "C2gd", "C1g", "C4g") and not args.no_eager:
            uf = gate_unfused_gpu_ms(key, torch, wl, dev, args.steps)
            res["unfused_ms_per_step"] = uf
            res["speedup_vs_unfused"] = uf / res["ms_per_step"]
            scan = {"C2g": "linear_scan + A*h0+Bc", "C2gd": "linear_scan + A*h0+Bc",
                    "C1g": "parallel_scan_log", "C4g": "angle scan"}[key]
            print(f"#   unfused (eager gates + HIP {scan}): {uf:.3f} ms/step "
                  f"({res['speedup_vs_unfused']:.2f}x the fused time)", file=sys.stderr,
                  flush=True)
        if key == "C5dp" and not args.no_eager:
            # The same workload on the fp32-operand gated kernels (what bf16 DeltaProduct
            # inputs ran on before the bf16 kernels took nh > 1).
            f32 = delta_gated_fp32_kernels_ms(torch, wl, dev, args.steps, nh=2)
            res["fp32_kernels_ms_per_step"] = f32
            res["speedup_vs_fp32_kernels"] = f32 / res["ms_per_step"]
            print(f"#   fp32-operand gated kernels: {f32:.3f} ms/step "
                  f"({res['speedup_vs_fp32_kernels']:.2f}x the bf16 time)", file=sys.stderr,
                  flush=True)
        if key in ("C5", "C5d") and not args.no_eager:
            eg = (delta_eager_gpu_ms if key == "C5" else delta_gated_eager_gpu_ms)(torch, wl, dev)
            res["eager_gpu_ms_per_step"] = eg
            res["speedup_vs_eager_gpu"] = eg / res["ms_per_step"]
            print(f"#   eager GPU chunked-WY: {eg:.2f} ms/step "
                  f"({res['speedup_vs_eager_gpu']:.1f}x slower than HIP)", file=sys.stderr,
                  flush=True)
        if cpu_step is not None and not args.no_cpu:
            cb = cpu_baseline(cpu_step, B, ops[key].tokens, torch)
            res["cpu_eager_tokens_per_s"] = cb["value"]
            res["cpu_eager_sample"] = cb["sample"]
            print(f"#   CPU eager ({cb['cores']} threads): {cb['value']:.4g} tok/s "
                  f"({res['tokens_per_s'] / cb['value']:.0f}x slower than HIP)", file=sys.stderr,
                  flush=True)
            if key == "C2":
                cpu = cb
        torch.cuda.empty_cache()
    decode = None
    if not args.only or "decode" in args.only.split(","):
        decode = dec = decode_bench(torch, wl, dev, max(args.steps, 20))
        for k, r in dec.items():
            print(f"# {k} decode step: fused {r['fused_us_per_step']:.1f} us, eager "
                  f"{r['eager_us_per_step']:.1f} us ({r['speedup_vs_eager']:.1f}x); queued: fused "
                  f"{r['fused_us_per_step_queued']:.1f} us, eager "
                  f"{r['eager_us_per_step_queued']:.1f} us ({r['speedup_vs_eager_queued']:.1f}x)",
                  file=sys.stderr, flush=True)
    copy = None
    if args.copy_probe:
        copy = copy_probe(torch, dev)
        print(f"# copy probe: {copy['achieved_GBs']:.0f} GB/s ({copy['avg_us']:.1f} us per "
              "1 GiB copy)", file=sys.stderr, flush=True)

    if not results:  # --only decode
        print(json.dumps({"decode": decode}))
        return
    head = results.get(HEADLINE) or next(iter(results.values()))
    head_key = HEADLINE if HEADLINE in results else next(iter(results))
    op = ops[head_key]
    # Dominant kernel: the one with the largest device time per step.
    dom_name, dom = max(head["kernels"].items(), key=lambda kv: kv[1]["avg_us"])
    roofline = {
        "bound": "hbm",
        "kernel": dom_name,
        "achieved": dom["achieved_GBs"],
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": dom["achieved_GBs"] / HBM_PEAK_GBS,
        "traffic": _traffic(f"{head_key}:{dom_name}"),
    }
    line = {
        "metric": METRIC,
        "value": head["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded CPU generator, BASELINE.json workload shapes)",
        "config": {"workload": op.workload, **{"C1": wl.C1, "C1g": wl.C1, "C2": wl.C2, "C2g": wl.C2,
                                               "C2gd": wl.C2, "C3": wl.C3, "C3m": wl.C3,
                                               "C4": wl.C4, "C4g": wl.C4, "C5": wl.C5,
                                               "C5d": wl.C5, "C5dp": wl.C5}.get(head_key, {})},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "achieved_TBs": head["achieved_TBs"],
        "frac_of_hbm_peak": head["frac_of_hbm_peak"],
        "ops": results,
    }
    if copy is not None:
        line["copy_probe"] = copy
    if decode is not None:
        line["decode"] = decode
    print(json.dumps(line))


if __name__ == "__main__":
    main()
