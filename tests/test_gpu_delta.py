"""GPU parity: HIP DeltaMinGRU chunked-WY forward/backward vs the fp64 oracle.

Bars: fp32 inputs -- forward max abs err <= 1e-4, gradients <= 1e-3 against
the float64 oracle (``oracle.scans.delta_chunked`` / ``delta_chunked_bwd``);
bf16 inputs -- max abs err <= 2e-2 of the largest reference magnitude, with the
oracle fed the same bf16-rounded values, for the bf16 outputs (y, dQ, dK, dV,
dbeta), and <= 1e-4 of max(1, largest reference magnitude) for the fp32 ones
(H_T, dH0).  The full-size C5 workload is checked
on two heads at full length (heads are independent).
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from mingru_amd import DeltaMinGRU, hip_scans
from mingru_amd import workloads as wl
from oracle import scans as orc

FWD_TOL = 1e-4
GRAD_TOL = 1e-3
BF16_REL = 2e-2
SPLIT_REL = 1e-4  # fp32 outputs of the bf16-input path

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _force_hip(monkeypatch):
    monkeypatch.setenv("MINGRU_SCAN", "hip")


def _inputs(B, H, T, nh, dk, dv, seed, beta_scale=2.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    Q = torch.randn(B, H, T, dk, generator=g)
    K = F.normalize(torch.randn(B, H, T, nh, dk, generator=g), dim=-1)
    V = torch.randn(B, H, T, nh, dv, generator=g)
    beta = beta_scale * torch.sigmoid(torch.randn(B, H, T, nh, generator=g))
    H0 = 0.3 * torch.randn(B, H, dk, dv, generator=g)
    dy = torch.randn(B, H, T, dv, generator=g)
    dHT = torch.randn(B, H, dk, dv, generator=g)
    Q, K, V, beta = (t.to(dtype) for t in (Q, K, V, beta))
    return Q, K, V, beta, H0, dy.to(dtype), dHT


def _np(t):
    return t.detach().double().cpu().numpy()


def _run(Q, K, V, beta, H0, dy, dHT, chunk, cuda):
    ts = [t.to(cuda).requires_grad_(True) for t in (Q, K, V, beta, H0)]
    y, HT = hip_scans.delta_scan_impl(*ts, chunk_size=chunk)
    assert "DeltaScanFn" in type(y.grad_fn).__name__, "HIP path did not run"
    torch.autograd.backward([y, HT], [dy.to(cuda), dHT.to(cuda)])
    torch.cuda.synchronize()
    return y, HT, [t.grad for t in ts]


CASES = [
    # B, H, T, nh, dk, dv, chunk
    (1, 1, 1, 1, 4, 4, 4),
    (2, 2, 100, 1, 16, 16, 16),
    (1, 3, 128, 1, 64, 64, 64),
    (2, 1, 130, 1, 32, 48, 32),
    (1, 2, 77, 2, 24, 24, 20),
    (2, 2, 33, 3, 8, 5, 7),
    (1, 1, 300, 1, 64, 64, 64),
    (1, 2, 95, 4, 64, 64, 16),
    # nh * chunk above one 64-micro-step kernel tile, up to the reference's 128
    (2, 2, 1024, 2, 16, 16, 64),
    (2, 2, 1024, 2, 64, 64, 64),
    (1, 2, 130, 3, 32, 32, 42),
    (1, 1, 70, 64, 8, 8, 2),
]


@pytest.mark.parametrize("case", CASES)
def test_delta_fp32_matches_oracle(cuda, case):
    B, H, T, nh, dk, dv, C = case
    print(f"[gpu] delta fp32 case={case}", flush=True)
    Q, K, V, beta, H0, dy, dHT = _inputs(B, H, T, nh, dk, dv, seed=11 + T)
    y, HT, grads = _run(Q, K, V, beta, H0, dy, dHT, C, cuda)
    ry, rHT, _ = orc.delta_chunked(_np(Q), _np(K), _np(V), _np(beta), _np(H0), C)
    assert np.max(np.abs(_np(y) - ry)) <= FWD_TOL
    assert np.max(np.abs(_np(HT) - rHT)) <= FWD_TOL
    rg = orc.delta_chunked_bwd(_np(Q), _np(K), _np(V), _np(beta), _np(H0), C, _np(dy),
                               _np(dHT))
    for name, gk, rk in zip(("dQ", "dK", "dV", "dbeta", "dH0"), grads, rg):
        err = np.max(np.abs(_np(gk) - rk))
        assert err <= GRAD_TOL, f"{name} max abs err {err:.3e}"


def _rel(x, ref):
    return float(np.max(np.abs(_np(x) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def _rel1(x, ref):
    """Max abs error relative to max(1, max |ref|): the fp32 bar, scaled for large values."""
    return float(np.max(np.abs(_np(x) - ref)) / max(np.max(np.abs(ref)), 1.0))


# The bf16 inputs run their own kernels (bf16 MFMA, split operands): every
# fp32 case again (ragged d_k / d_v, nh > 1, partial chunks, T = 1), plus two.
BF16_CASES = CASES + [(2, 2, 200, 1, 64, 64, 64), (1, 2, 70, 2, 32, 32, 32)]


@pytest.mark.parametrize("case", BF16_CASES)
def test_delta_bf16_matches_oracle(cuda, case):
    B, H, T, nh, dk, dv, C = case
    print(f"[gpu] delta bf16 case={case}", flush=True)
    Q, K, V, beta, H0, dy, dHT = _inputs(B, H, T, nh, dk, dv, seed=5 + T, dtype=torch.bfloat16)
    y, HT, grads = _run(Q, K, V, beta, H0, dy, dHT, C, cuda)
    assert y.dtype == torch.bfloat16 and grads[0].dtype == torch.bfloat16
    ry, rHT, _ = orc.delta_chunked(_np(Q), _np(K), _np(V), _np(beta), _np(H0), C)
    assert _rel(y, ry) <= BF16_REL
    # H_T and dH0 stay fp32: with split (hi/lo) bf16 operands every product keeps
    # about 16 significant bits, so they match the fp64 oracle to fp32 level.
    assert _rel1(HT, rHT) <= SPLIT_REL, f"H_T rel err {_rel1(HT, rHT):.3e}"
    rg = orc.delta_chunked_bwd(_np(Q), _np(K), _np(V), _np(beta), _np(H0), C, _np(dy),
                               _np(dHT))
    for name, gk, rk in zip(("dQ", "dK", "dV", "dbeta", "dH0"), grads, rg):
        err = _rel1(gk, rk) if name == "dH0" else _rel(gk, rk)
        bar = SPLIT_REL if name == "dH0" else BF16_REL
        assert err <= bar, f"{name} rel err {err:.3e}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_delta_interleaved_calls(cuda, dtype):
    """Two forwards before either backward (as two layers' forwards run before their
    backwards): each backward must read its own forward's saved state -- the chunk-entry
    states and, for bf16, the chunk inverses -- while the second forward and the first
    backward have rewritten the shared workspace.  Bitwise equal to separate runs."""
    B, H, T, nh, dk, dv, C = 2, 2, 200, 1, 64, 64, 64
    print(f"[gpu] delta interleaved calls dtype={dtype}", flush=True)
    xa = _inputs(B, H, T, nh, dk, dv, seed=31, dtype=dtype)
    xb = _inputs(B, H, T, nh, dk, dv, seed=32, dtype=dtype)
    ref = [_run(*x, C, cuda) for x in (xa, xb)]
    leaves, outs = [], []
    for x in (xa, xb):
        ts = [t.to(cuda).requires_grad_(True) for t in x[:5]]
        leaves.append(ts)
        outs.append(hip_scans.delta_scan_impl(*ts, chunk_size=C))
    for (y, HT), x in zip(outs[::-1], (xb, xa)):  # second call's backward first
        torch.autograd.backward([y, HT], [x[5].to(cuda), x[6].to(cuda)])
    torch.cuda.synchronize()
    for (y, HT), ts, (ry, rHT, rg) in zip(outs, leaves, ref):
        assert torch.equal(y, ry) and torch.equal(HT, rHT)
        for g, rgk in zip((t.grad for t in ts), rg):
            assert torch.equal(g, rgk)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("gated", [False, True])
def test_delta_c_abi_buffers_stay_in_bounds(cuda, dtype, gated):
    """Through the C ABI with buffers of exactly the reported sizes plus a canary tail:
    the saved state (chunk-entry states and the packed chunk inverses) and the workspace
    are written only inside mg_delta_state_bytes / the workspace size, and the results
    equal the autograd wrapper's bitwise.  Ragged last chunk (T = 130, chunk 64)."""
    import ctypes

    from mingru_amd import _native

    B, H, T, nh, dk, dv, C = 1, 2, 130, 1, 64, 64, 64
    print(f"[gpu] delta C ABI buffer bounds dtype={dtype} gated={gated}", flush=True)
    lib = _native.load()
    Q, K, V, beta, H0, dy, dHT = (t.to(cuda).contiguous()
                                  for t in _inputs(B, H, T, nh, dk, dv, seed=61, dtype=dtype))
    lg = (-0.5 * torch.rand(B, H, T, generator=torch.Generator().manual_seed(62))).to(cuda)
    tag = 1 if dtype == torch.bfloat16 else 0
    dims = (B, H, T, nh, dk, dv, C)
    canary = 4096  # floats after each buffer
    pattern = 1234.5
    nstate = lib.mg_delta_state_bytes(*dims) // 4
    wsb = (lib.mg_delta_gated_workspace_bytes if gated else lib.mg_delta_workspace_bytes)(*dims)
    Hb = torch.full((nstate + canary,), pattern, device=cuda)
    ws = torch.full((wsb // 4 + canary,), pattern, device=cuda)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    y = torch.empty(B, H, T, dv, dtype=dtype, device=cuda)
    HT = torch.empty(B, H, dk, dv, device=cuda)
    dQ, dK, dV, dbeta = (torch.empty_like(t) for t in (Q, K, V, beta))
    dH0 = torch.empty_like(H0)
    if gated:
        dlg = torch.empty_like(lg)
        assert lib.mg_delta_gated_fwd(p(Q), p(K), p(V), p(beta), p(lg), p(H0), p(y), p(HT), p(Hb),
                                      *dims, tag, p(ws), wsb, stream) == 0
        assert lib.mg_delta_gated_bwd(p(Q), p(K), p(V), p(beta), p(lg), p(Hb), p(dy), p(dHT),
                                      p(dQ), p(dK), p(dV), p(dbeta), p(dlg), p(dH0), *dims, tag,
                                      p(ws), wsb, stream) == 0
    else:
        assert lib.mg_delta_fwd(p(Q), p(K), p(V), p(beta), p(H0), p(y), p(HT), p(Hb), *dims, tag,
                                p(ws), wsb, stream) == 0
        assert lib.mg_delta_bwd(p(Q), p(K), p(V), p(beta), p(Hb), p(dy), p(dHT), p(dQ), p(dK),
                                p(dV), p(dbeta), p(dH0), *dims, tag, p(ws), wsb, stream) == 0
    torch.cuda.synchronize()
    assert bool((Hb[nstate:] == pattern).all()), "saved state written past mg_delta_state_bytes"
    assert bool((ws[wsb // 4:] == pattern).all()), "workspace written past its size"
    ts = [t.clone().requires_grad_(True) for t in ((Q, K, V, beta, lg, H0) if gated
                                                   else (Q, K, V, beta, H0))]
    if gated:
        ry, rHT = hip_scans.delta_gated_scan_impl(*ts, chunk_size=C)
    else:
        ry, rHT = hip_scans.delta_scan_impl(*ts, chunk_size=C)
    torch.autograd.backward([ry, rHT], [dy, dHT])
    torch.cuda.synchronize()
    assert torch.equal(y, ry) and torch.equal(HT, rHT)
    mine = (dQ, dK, dV, dbeta, dlg, dH0) if gated else (dQ, dK, dV, dbeta, dH0)
    for g, t in zip(mine, ts):
        assert torch.equal(g, t.grad)


def test_delta_c5_full_size(cuda):
    """C5 (B=8, H=8, T=8192, d=64, chunk 64, bf16): two heads at full length vs the
    oracle, from the first and the second half of the 64 (batch, head) pairs."""
    print("[gpu] delta C5 full size", flush=True)
    inp = wl.c5_inputs(**wl.C5)
    Q, K, V, beta, H0 = (inp[k] for k in ("Q", "K", "V", "beta", "H0"))
    dy = inp["grad_y"].to(torch.bfloat16)
    dHT = inp["grad_HT"]
    y, HT, grads = _run(Q, K, V, beta, H0, dy, dHT, inp["chunk_size"], cuda)
    assert torch.isfinite(y.float()).all() and all(torch.isfinite(g.float()).all() for g in grads)
    for sel in ((slice(3, 4), slice(2, 3)), (slice(6, 7), slice(5, 6))):  # pairs 26 and 53
        sub = [_np(t[sel]) for t in (Q, K, V, beta, H0)]
        ry, rHT, _ = orc.delta_chunked(*sub, inp["chunk_size"])
        assert _rel(y[sel], ry) <= BF16_REL
        assert _rel(HT[sel], rHT) <= BF16_REL
        rg = orc.delta_chunked_bwd(*sub, inp["chunk_size"], _np(dy[sel]), _np(dHT[sel]))
        for name, gk, rk in zip(("dQ", "dK", "dV", "dbeta", "dH0"), grads, rg):
            assert _rel(gk[sel], rk) <= BF16_REL, f"{name} rel err {_rel(gk[sel], rk):.3e}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_delta_chaining_at_misaligned_boundary(cuda, dtype):
    """Running [0, T1) and then [T1, T) with the first call's H_T as the second's H_0
    gives the single run's y and H_T, at a split that is not a chunk boundary (the
    reference's chaining property, tests/test_mixers.py:834-854).  The runs differ only
    by chunk association, so the bars are the parity bars: fp32 y and H_T within twice
    the 1e-4 fp64 bar; bf16 y within the bf16 bar; the fp32 state within 2e-4 relative."""
    B, H, T, C, T1 = 2, 2, 150, 32, 77
    print(f"[gpu] delta chaining dtype={dtype}", flush=True)
    Q, K, V, beta, H0, _, _ = _inputs(B, H, T, 1, 64, 64, seed=41, dtype=dtype)
    seq = [t.to(cuda) for t in (Q, K, V, beta)]
    h0 = H0.to(cuda)
    with torch.no_grad():
        y, HT = hip_scans.delta_scan_impl(*seq, h0, chunk_size=C)
        ya, Ha = hip_scans.delta_scan_impl(*(t[:, :, :T1] for t in seq), h0, chunk_size=C)
        yb, Hb = hip_scans.delta_scan_impl(*(t[:, :, T1:] for t in seq), Ha, chunk_size=C)
    torch.cuda.synchronize()
    ys = torch.cat([ya, yb], dim=2)
    if dtype == torch.float32:
        assert (ys - y).abs().max().item() <= 2 * FWD_TOL
        assert (Hb - HT).abs().max().item() <= 2 * FWD_TOL
    else:
        assert _rel(ys, _np(y)) <= BF16_REL
        assert _rel(Hb, _np(HT)) <= 2 * SPLIT_REL


@pytest.mark.parametrize("nh,chunks", [(1, (1, 3, 40, 64)), (2, (1, 5, 32))])
def test_delta_chunk_size_invariance(cuda, nh, chunks):
    """One input set at several chunk sizes (1, ragged, T and > T) gives the same outputs
    and gradients as chunk 16, within the fp32 bars (the reference's chunk-size
    invariance, tests/test_mixers.py:748-775)."""
    B, H, T, dk, dv = 2, 2, 40, 16, 24
    Q, K, V, beta, H0, dy, dHT = _inputs(B, H, T, nh, dk, dv, seed=77 + nh)
    print(f"[gpu] delta chunk invariance nh={nh} chunks={chunks}", flush=True)
    y0, H0T, g0 = _run(Q, K, V, beta, H0, dy, dHT, 16, cuda)
    for C in chunks:
        y, HT, grads = _run(Q, K, V, beta, H0, dy, dHT, C, cuda)
        assert (y - y0).abs().max().item() <= FWD_TOL, f"chunk {C}: y"
        assert (HT - H0T).abs().max().item() <= FWD_TOL, f"chunk {C}: H_T"
        for name, gk, rk in zip(("dQ", "dK", "dV", "dbeta", "dH0"), grads, g0):
            assert (gk - rk).abs().max().item() <= GRAD_TOL, f"chunk {C}: {name}"


def test_delta_deterministic(cuda):
    Q, K, V, beta, H0, dy, dHT = _inputs(2, 2, 257, 1, 64, 64, seed=3)
    a = _run(Q, K, V, beta, H0, dy, dHT, 64, cuda)
    b = _run(Q, K, V, beta, H0, dy, dHT, 64, cuda)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    for ga, gb in zip(a[2], b[2]):
        assert torch.equal(ga, gb)


def test_delta_module_matches_eager(cuda, monkeypatch):
    """DeltaMinGRU on the GPU (HIP) vs the same module in float64 on the CPU (eager)."""
    torch.manual_seed(0)
    m = DeltaMinGRU(24, 32, n_heads=2, chunk_size=16)
    x = torch.randn(3, 100, 24)
    ref = m.double()
    xr = x.double().requires_grad_(True)
    monkeypatch.setenv("MINGRU_SCAN", "eager")
    out_r = ref(xr)
    out_r.sum().backward()
    gx_r = xr.grad.clone()
    gp_r = {n: p.grad.clone() for n, p in ref.named_parameters()}
    ref.zero_grad()
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    mg = m.float().to(cuda)
    xg = x.to(cuda).requires_grad_(True)
    out = mg(xg)
    out.sum().backward()
    assert np.max(np.abs(_np(out) - _np(out_r))) <= FWD_TOL
    assert np.max(np.abs(_np(xg.grad) - _np(gx_r))) <= GRAD_TOL
    for n, p in mg.named_parameters():
        ref_g = _np(gp_r[n])
        err = np.max(np.abs(_np(p.grad) - ref_g))
        # parameter grads sum over B*T tokens: gate relative to their magnitude
        assert err <= GRAD_TOL * max(1.0, float(np.max(np.abs(ref_g)))), f"{n}: {err:.3e}"


def test_delta_golden_fixture_hip(cuda, monkeypatch):
    """The reference's golden DeltaMinGRU vector (nh=2 at the default chunk_size=64)
    through the module on the GPU under MINGRU_SCAN=hip: output within 1e-4, the input
    gradient and all 16 parameter gradients within 1e-3."""
    import golden_fixture as gf

    fx = gf.load()
    layer = gf.module(fx).to(cuda)
    print("[gpu] delta golden fixture (B=2, T=5, nh=2, chunk 64)", flush=True)
    called = []
    real = hip_scans._DeltaScanFn.apply

    def spy(*a):
        called.append(a[-1])
        return real(*a)

    monkeypatch.setattr(hip_scans._DeltaScanFn, "apply", spy)
    out, gx, gp = gf.run(layer, torch.tensor(fx["x"], device=cuda))
    torch.cuda.synchronize()
    assert called == [32], f"HIP kernel chunk tiles: {called}"
    assert np.max(np.abs(_np(out) - np.asarray(fx["output"]))) <= FWD_TOL
    assert np.max(np.abs(_np(gx) - np.asarray(fx["x_grad"]))) <= GRAD_TOL
    assert sorted(gp) == sorted(fx["param_grads"])
    for name, ref in fx["param_grads"].items():
        ref = np.asarray(ref)
        err = np.max(np.abs(_np(gp[name]) - ref))
        assert err <= GRAD_TOL * max(1.0, float(np.max(np.abs(ref)))), f"{name}: {err:.3e}"
