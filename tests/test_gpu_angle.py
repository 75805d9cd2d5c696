"""GPU parity: HIP angle-fused rotation scan vs the fp64 oracle, and the module paths.

Bars: fp32 forward max abs err <= 1e-4, gradients <= 1e-3 against float64 on
the C4 workload.  The synthetic stress cases include schedules without decay,
where the state random-walks to |h| ~ 25 over the sequence; there the bar is
scaled by max(1, max|ref| / 4), i.e. the same bar relative to the state size.
"""

import os

import numpy as np
import pytest
import torch

import mingru_amd as mg
from mingru_amd import hip_scans
from mingru_amd import workloads as wl
from oracle import scans as orc

FWD_TOL = 1e-4
GRAD_TOL = 1e-3

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _force_hip(monkeypatch):
    monkeypatch.setenv("MINGRU_SCAN", "hip")


def _maxerr(x, ref):
    return float(np.max(np.abs(x.detach().double().cpu().numpy() - ref))) if ref.size else 0.0


def _brick_meta(k, R):
    layer = mg.GivensMinGRU(4, k, block_size=k, rounds=R)
    return layer._angle_plane_meta(torch.device("cpu"))


def _inputs(B, T, n, k, R, half, seed, std=0.7):
    g = torch.Generator().manual_seed(seed)
    theta = std * torch.randn(B, T, n, R, half, generator=g)
    scale = torch.tanh(torch.randn(B, T, n, generator=g))
    gamma = torch.sigmoid(torch.randn(B, T, n, generator=g))
    b = torch.randn(B, T, n, k, generator=g)
    h0 = torch.randn(B, n, k, generator=g)
    gh = torch.randn(B, T, n, k, generator=g)
    return theta, scale, gamma, b, h0, gh


def _check(cuda, theta, scale, gamma, b, h0, gh, perm, sgn, p2p, hs, hd):
    ts = [t.to(cuda).requires_grad_(True) for t in (theta, scale, gamma, b, h0)]
    h = hip_scans.angle_scan_impl(*ts, perm.to(cuda), sgn.to(cuda), p2p.to(cuda),
                                  has_scale=hs, has_decay=hd)
    assert type(h.grad_fn).__name__.startswith(("_AngleScanFn", "_AngleTablesFn"))
    h.backward(gh.to(cuda))
    torch.cuda.synchronize()
    npy = [t.numpy() for t in (theta, scale, gamma, b, h0)]
    ref = orc.angle_scan(*npy, perm.numpy(), sgn.numpy(), p2p.numpy(), hs, hd)
    rgrads = orc.angle_scan_bwd(*npy, perm.numpy(), sgn.numpy(), p2p.numpy(), hs, hd, gh.numpy())
    def bar(tol, r):
        return tol * max(1.0, float(np.max(np.abs(r))) / 4.0)

    assert _maxerr(h, ref) <= bar(FWD_TOL, ref)
    names = ["theta", "scale", "gamma", "b", "h0"]
    for name, t, r in zip(names, ts, rgrads):
        if name == "scale" and not hs:
            continue
        if name == "gamma" and not hd:
            continue
        err = _maxerr(t.grad, r)
        assert err <= bar(GRAD_TOL, r), f"d{name}: {err}"


BRICK_CASES = [
    # B, T, n, k, R, has_scale, has_decay
    (2, 1, 3, 8, 3, 0, 0),
    (2, 37, 5, 8, 3, 0, 1),
    (2, 100, 70, 8, 3, 0, 0),
    (1, 65, 9, 8, 2, 0, 1),
    (2, 50, 33, 4, 3, 0, 1),
    (2, 80, 40, 4, 1, 0, 0),
    (2, 90, 65, 2, 1, 1, 0),
    (2, 71, 12, 2, 1, 1, 1),
    (1, 40, 7, 2, 3, 0, 1),
    # exactly 16 chunks of 16 tokens: the last sequence length walked chunk by chunk
    (1, 256, 6, 8, 3, 0, 1),
    # more than 16 chunks of 16 tokens: the two-level boundary walk, last group partial
    (2, 300, 5, 8, 3, 0, 1),
    (1, 530, 3, 2, 1, 1, 1),
    (1, 260, 4, 4, 2, 0, 0),
    # more than 16 groups of 8 chunks (T > 2048): the group walk and the fill as two
    # launches instead of one
    (1, 2200, 3, 4, 2, 0, 1),
]


@pytest.mark.parametrize("case", BRICK_CASES)
def test_brick_schedule_matches_oracle(cuda, case):
    B, T, n, k, R, hs, hd = case
    print(f"[gpu] angle brick case={case}", flush=True)
    perm, sgn, p2p = _brick_meta(k, R)
    theta, scale, gamma, b, h0, gh = _inputs(B, T, n, k, R, k // 2, seed=T * 13 + n + k)
    _check(cuda, theta, scale, gamma, b, h0, gh, perm, sgn, p2p, hs, hd)


LEX_CASES = [(2, 33, 10, 8, 1), (1, 120, 64, 8, 1), (2, 45, 20, 4, 1), (2, 30, 66, 8, 0),
             (1, 400, 6, 8, 1), (1, 2100, 2, 8, 1)]


@pytest.mark.parametrize("case", LEX_CASES)
def test_lexicographic_schedule_matches_oracle(cuda, case):
    B, T, n, k, hd = case
    print(f"[gpu] angle lex case={case}", flush=True)
    perm, sgn, p2p = wl.lexicographic_schedule(k)
    R = k * (k - 1) // 2
    theta, scale, gamma, b, h0, gh = _inputs(B, T, n, k, R, 1, seed=7 * T + n, std=0.5)
    _check(cuda, theta, scale, gamma, b, h0, gh, perm, sgn, p2p, 0, hd)


TABLE_CASES = [
    # B, T, n, k, R, half, schedule, has_scale, has_decay
    (2, 50, 3, 16, 3, 8, "brick", 0, 1),
    (1, 70, 2, 16, 5, 8, "brick", 0, 0),
    (2, 20, 2, 16, 120, 1, "lex", 0, 1),
    (2, 40, 5, 8, 5, 6, "random", 1, 1),  # two of six angles unused per round
    (1, 33, 4, 4, 7, 2, "random_inactive", 0, 1),
    (2, 25, 3, 2, 2, 1, "random", 1, 0),
    (1, 1, 2, 16, 3, 8, "brick", 1, 1),
    (2, 30, 4, 8, 70, 4, "random", 0, 1),  # more rounds than the compiled kernels take
    (1, 300, 3, 16, 3, 8, "brick", 0, 1),  # many chunks: the boundary walks
    (2, 129, 2, 8, 4, 4, "random", 1, 0),
]


def _tables(k, R, half, kind, seed):
    from test_dispatch import _random_tables

    if kind == "brick":
        return _brick_meta(k, R)
    if kind == "lex":
        return wl.lexicographic_schedule(k)
    return _random_tables(k, R, half, seed, inactive=kind == "random_inactive")


@pytest.mark.parametrize("case", TABLE_CASES)
def test_plane_table_kernel_matches_oracle(cuda, case, monkeypatch):
    """The table-driven kernel (k = 16, any valid plane tables, any round count) against
    the float64 oracle, fwd and all gradients."""
    B, T, n, k, R, half, kind, hs, hd = case
    print(f"[gpu] angle tables case={case}", flush=True)
    perm, sgn, p2p = _tables(k, R, half, kind, seed=T + k + R)
    theta, scale, gamma, b, h0, gh = _inputs(B, T, n, k, R, half, seed=3 * T + n + k, std=0.6)
    used = []
    real = hip_scans._AngleTablesFn.apply

    def spy(*a):
        used.append(True)
        return real(*a)

    monkeypatch.setattr(hip_scans._AngleTablesFn, "apply", spy)
    _check(cuda, theta, scale, gamma, b, h0, gh, perm, sgn, p2p, hs, hd)
    assert used, "the table-driven kernel did not run"


def test_givens_block16_module_matches_fp64(cuda, monkeypatch):
    """GivensMinGRU(block_size=16) under MINGRU_SCAN=hip (table-driven angle kernel)."""
    torch.manual_seed(5)
    _module_vs_fp64(cuda, mg.GivensMinGRU(12, 48, block_size=16), torch.randn(2, 60, 12),
                    monkeypatch)


def test_c4_full_size(cuda):
    print("[gpu] angle C4 full size", flush=True)
    inp = wl.c4_inputs(**wl.C4)
    keys = ("theta", "scale", "gamma", "b", "h0")
    ts = [inp[k].to(cuda).requires_grad_(True) for k in keys]
    h = hip_scans.angle_scan_impl(*ts, inp["perm"].to(cuda), inp["sgn"].to(cuda),
                                  inp["p2p"].to(cuda), has_scale=0, has_decay=1)
    h.backward(inp["grad_h"].to(cuda))
    torch.cuda.synchronize()
    for r in (0, wl.C4["B"] - 1):
        sl = slice(r, r + 1)
        npy = [inp[k][sl].numpy() for k in keys]
        meta = (inp["perm"].numpy(), inp["sgn"].numpy(), inp["p2p"].numpy())
        ref = orc.angle_scan(*npy, *meta, 0, 1)
        rg = orc.angle_scan_bwd(*npy, *meta, 0, 1, inp["grad_h"][sl].numpy())
        assert _maxerr(h[sl], ref) <= FWD_TOL
        for name, t, g in zip(keys, ts, rg):
            if name == "scale":
                continue
            assert _maxerr(t.grad[sl], g) <= GRAD_TOL, name


def test_c4_norm_preserved_full_size(cuda):
    """At the full C4 shape, rotations alone (gamma = 1, b = 0) keep |h_t| = |h_0| at every
    token: a size-independent property of the special-orthogonal transition (the
    reference checks M M^T = I, tests/test_mixers.py:244-251).  In fp32 each rotation
    keeps the norm to about 6e-8 relative; unbiased over the 2048 x 28 rotations a state
    sees, that is a drift near sqrt(57344) x 6e-8 = 1.4e-5 (measured: 8.7e-6).  The bar,
    1e-4, fails a sin/cos whose c^2 + s^2 is biased by more than about 2e-9."""
    print("[gpu] angle C4 norm preservation", flush=True)
    inp = wl.c4_inputs(**wl.C4)
    theta, scale, h0 = (inp[k].to(cuda) for k in ("theta", "scale", "h0"))
    B, T, n = theta.shape[:3]
    k = h0.shape[-1]
    gamma = torch.ones(B, T, n, device=cuda)
    b = torch.zeros(B, T, n, k, device=cuda)
    with torch.no_grad():
        h = hip_scans.angle_scan_impl(theta, scale, gamma, b, h0, inp["perm"].to(cuda),
                                      inp["sgn"].to(cuda), inp["p2p"].to(cuda),
                                      has_scale=0, has_decay=1)
    torch.cuda.synchronize()
    nrm = h.double().norm(dim=-1)
    ref = h0.double().norm(dim=-1)[:, None, :]
    drift = ((nrm - ref).abs() / ref).max().item()
    print(f"[gpu] angle C4 max relative norm drift {drift:.3e}", flush=True)
    assert drift <= 1e-4


def _graph_has(t, name, depth=4):
    """Whether an autograd node named ``name`` lies within ``depth`` steps of ``t``."""
    frontier = [t.grad_fn]
    for _ in range(depth):
        nxt = []
        for f in frontier:
            if f is None:
                continue
            if name in type(f).__name__:
                return True
            nxt += [g for g, _ in f.next_functions]
        frontier = nxt
    return False


def _module_vs_fp64(cuda, layer, x, monkeypatch, dt=None, kernel=None):
    """A mixer under MINGRU_SCAN=hip on the GPU (fp32) against a float64 copy of it on
    the CPU eager path: output within 1e-4 and the input and parameter gradients within
    1e-3, each relative to max(1, max |ref|) (the undecayed rotation state grows to
    |h| ~ 10 over a sequence).  ``kernel`` names the autograd node the GPU forward must
    have run (the gated-heads kernel or the plain one)."""
    import copy

    ref = copy.deepcopy(layer).double()
    xr = x.double().requires_grad_(True)
    dtr = None if dt is None else dt.double()
    monkeypatch.setenv("MINGRU_SCAN", "eager")
    yr = ref(xr, delta_t=dtr)
    yr.square().sum().backward()
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    lg = layer.to(cuda)
    xg = x.to(cuda).requires_grad_(True)
    y = lg(xg, delta_t=None if dt is None else dt.to(cuda))
    if kernel is not None:
        assert _graph_has(y, kernel), f"{kernel} did not run"
    y.square().sum().backward()
    torch.cuda.synchronize()

    def rel(a, r):
        return (a.double().cpu() - r).abs().max().item() / max(1.0, r.abs().max().item())

    assert rel(y, yr) <= FWD_TOL, f"output {rel(y, yr):.2e}"
    assert rel(xg.grad, xr.grad) <= GRAD_TOL
    gp = dict(ref.named_parameters())
    for name, p in lg.named_parameters():
        assert rel(p.grad, gp[name].grad) <= GRAD_TOL, name


def test_givens_module_matches_eager(cuda, monkeypatch):
    torch.manual_seed(0)
    _module_vs_fp64(cuda, mg.GivensMinGRU(16, 64), torch.randn(3, 64, 16), monkeypatch,
                    kernel="AngleGatedFn")


def test_givens_module_decay_matches_eager(cuda, monkeypatch):
    torch.manual_seed(1)
    layer = mg.GivensMinGRU(16, 32, decay="learnable")
    _module_vs_fp64(cuda, layer, torch.randn(2, 40, 16), monkeypatch, dt=torch.rand(2, 40),
                    kernel="AngleGatedFn")


@pytest.mark.parametrize("k, rounds", [(2, 1), (4, 5)])
def test_givens_module_small_blocks_gated_heads(cuda, monkeypatch, k, rounds):
    """Block sizes 2 and 4 on the gated-heads kernel, one with decay."""
    torch.manual_seed(5 + k)
    layer = mg.GivensMinGRU(12, 24, block_size=k, rounds=rounds,
                            decay="fixed" if k == 4 else None)
    dt = torch.rand(2, 300) if k == 4 else None
    _module_vs_fp64(cuda, layer, torch.randn(2, 300, 12), monkeypatch, dt=dt,
                    kernel="AngleGatedFn")


def test_givens_module_block16_keeps_the_table_kernel(cuda, monkeypatch):
    """k = 16 runs on the run-time-table kernel, with the heads formed eagerly."""
    torch.manual_seed(6)
    _module_vs_fp64(cuda, mg.GivensMinGRU(12, 32, block_size=16), torch.randn(2, 50, 12),
                    monkeypatch, kernel="AngleTablesFn")


@pytest.mark.parametrize("snap", [None, (2, 3, 4, 6)], ids=["nosnap", "default_snap"])
def test_rotation_module_matches_eager(cuda, monkeypatch, snap):
    torch.manual_seed(2)
    _module_vs_fp64(cuda, mg.RotationMinGRU(16, 32, snap=snap), torch.randn(3, 64, 16),
                    monkeypatch, kernel="AngleGatedFn")


@pytest.mark.parametrize("decay", ["fixed", "learnable"])
def test_rotation_module_decay_matches_eager(cuda, monkeypatch, decay):
    torch.manual_seed(3)
    layer = mg.RotationMinGRU(16, 32, decay=decay)
    _module_vs_fp64(cuda, layer, torch.randn(2, 500, 16), monkeypatch,
                    dt=torch.rand(2, 500) * 2, kernel="AngleGatedFn")


@pytest.mark.parametrize("has_decay", [0, 1])
def test_gated_heads_match_the_plain_kernel_full_size(cuda, has_decay):
    """At the C4 size (B=8, T=2048, 64 blocks of 8, brick-wall rounds as GivensMinGRU):
    the gated-heads kernel against the plain kernel fed sigmoid(z) * hpre computed by
    torch, forward and every gradient (through torch's autograd for the plain path)."""
    B, T, n, k, R = 8, 2048, 64, 8, 3
    print(f"[gpu] gated heads vs plain kernel, C4 size, has_decay={has_decay}", flush=True)
    g = torch.Generator(device=cuda).manual_seed(9)
    theta = (0.5 * torch.randn(B, T, n, R, k // 2, device=cuda, generator=g))
    z = torch.randn(B, T, n, k, device=cuda, generator=g)
    hp = torch.randn(B, T, n, k, device=cuda, generator=g)
    gamma = torch.sigmoid(torch.randn(B, T, n, device=cuda, generator=g))
    h0 = torch.randn(B, n, k, device=cuda, generator=g)
    gh = torch.randn(B, T, n, k, device=cuda, generator=g)
    perm, sgn, p2p = (t.to(cuda) for t in hip_scans._brick_tables(k, R))
    a = [t.clone().requires_grad_(True) for t in (theta, z, hp, gamma, h0)]
    h1 = hip_scans.angle_gated_scan_impl(a[0], None, a[3], a[1], a[2], a[4], perm, sgn, p2p,
                                         has_scale=0, has_decay=has_decay)
    assert "AngleGatedFn" in type(h1.grad_fn).__name__
    h1.backward(gh)
    b_ = [t.clone().requires_grad_(True) for t in (theta, z, hp, gamma, h0)]
    bb = torch.sigmoid(b_[1]) * b_[2]
    ones = torch.ones(B, T, n, device=cuda)
    h2 = hip_scans.angle_scan_impl(b_[0], ones, b_[3], bb, b_[4], perm, sgn, p2p, has_scale=0,
                                   has_decay=has_decay)
    h2.backward(gh)
    torch.cuda.synchronize()
    # The two differ only in how sigmoid(z) is evaluated (the kernel's exp2/rcp against
    # torch's), about 1e-7 relative per token; without decay |h| grows to ~25 over the
    # sequence, so the bar is relative to the largest magnitude.
    assert (h1 - h2).abs().max().item() / max(1.0, h2.abs().max().item()) <= 1e-5
    for name, x, y in zip(("theta", "z", "hpre", "gamma", "h0"), a, b_):
        if name == "gamma" and not has_decay:
            continue
        err = (x.grad - y.grad).abs().max().item() / max(1.0, y.grad.abs().max().item())
        assert err <= 1e-5, f"d{name} {err:.2e}"
