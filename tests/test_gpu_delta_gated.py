"""GPU parity: HIP decay-gated DeltaMinGRU chunked-WY forward/backward vs the fp64 oracle.

The oracle is the token-by-token gated recurrence and its hand-derived adjoint
(``oracle.scans.delta_gated_sequential`` / ``_bwd``), pinned on the CPU by the
ungated golden-pinned rule at log_gamma = 0, the beta = 0 closed form, the module's
span-sum chunked forward and finite differences.  Bars (fp32 kernels against
float64): forward max abs err <= 1e-4; gradients <= 1e-3 absolute, and for
dlog_gamma (a sum over a whole chunk's span products) <= 1e-3 of the largest
reference magnitude when that exceeds 1.
"""

import copy

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from mingru_amd import DeltaMinGRU, hip_scans
from oracle import scans as orc

FWD_TOL = 1e-4
GRAD_TOL = 1e-3

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _force_hip(monkeypatch):
    monkeypatch.setenv("MINGRU_SCAN", "hip")


def _inputs(B, H, T, nh, dk, dv, seed, lg_kind):
    g = torch.Generator().manual_seed(seed)
    Q = torch.randn(B, H, T, dk, generator=g)
    K = F.normalize(torch.randn(B, H, T, nh, dk, generator=g), dim=-1)
    V = torch.randn(B, H, T, nh, dv, generator=g)
    beta = 2.0 * torch.sigmoid(torch.randn(B, H, T, nh, generator=g))
    H0 = 0.3 * torch.randn(B, H, dk, dv, generator=g)
    dy = torch.randn(B, H, T, dv, generator=g)
    dHT = torch.randn(B, H, dk, dv, generator=g)
    lg = -0.5 * torch.rand(B, H, T, generator=g)
    if lg_kind == "zero":
        lg.zero_()
    elif lg_kind == "spikes":
        # gaps that drive gamma to (or below) fp32 underflow inside a chunk
        lg[..., 3::17] = -60.0
        lg[..., 9::29] = -300.0
    elif lg_kind == "weak":
        lg *= 0.02
    return Q, K, V, beta, lg, H0, dy, dHT


def _np(t):
    return t.detach().double().cpu().numpy()


def _run(ins, dy, dHT, chunk, cuda):
    ts = [t.to(cuda).requires_grad_(True) for t in ins]
    y, HT = hip_scans.delta_gated_scan_impl(*ts, chunk_size=chunk)
    assert "DeltaGatedScanFn" in type(y.grad_fn).__name__, "HIP path did not run"
    torch.autograd.backward([y, HT], [dy.to(cuda), dHT.to(cuda)])
    torch.cuda.synchronize()
    return y, HT, [t.grad for t in ts]


CASES = [
    # B, H, T, nh, dk, dv, chunk, log-gamma kind
    (1, 1, 1, 1, 4, 4, 4, "mod"),
    (2, 2, 100, 1, 16, 16, 16, "mod"),
    (1, 3, 128, 1, 64, 64, 64, "mod"),
    (2, 1, 130, 1, 32, 48, 32, "spikes"),
    (1, 2, 77, 2, 24, 24, 20, "mod"),
    (2, 2, 33, 3, 8, 5, 7, "spikes"),
    (1, 1, 300, 1, 64, 64, 64, "weak"),
    (1, 2, 95, 4, 64, 64, 16, "mod"),
    (1, 2, 200, 1, 64, 64, 64, "spikes"),
    # nh * chunk above one 64-micro-step kernel tile (the reference allows 128)
    (1, 2, 150, 2, 32, 32, 64, "mod"),
    (1, 1, 90, 3, 16, 16, 40, "spikes"),
]


@pytest.mark.parametrize("case", CASES)
def test_delta_gated_matches_oracle(cuda, case):
    B, H, T, nh, dk, dv, C, kind = case
    print(f"[gpu] delta gated case={case}", flush=True)
    Q, K, V, beta, lg, H0, dy, dHT = _inputs(B, H, T, nh, dk, dv, seed=23 + T, lg_kind=kind)
    y, HT, grads = _run((Q, K, V, beta, lg, H0), dy, dHT, C, cuda)
    ref = [_np(t) for t in (Q, K, V, beta, lg, H0)]
    ry, rHT = orc.delta_gated_sequential(*ref)
    assert np.max(np.abs(_np(y) - ry)) <= FWD_TOL
    assert np.max(np.abs(_np(HT) - rHT)) <= FWD_TOL
    rg = orc.delta_gated_sequential_bwd(*ref, _np(dy), _np(dHT))
    for name, gk, gr in zip(("dQ", "dK", "dV", "dbeta", "dlog_gamma", "dH0"), grads, rg):
        assert torch.isfinite(gk).all(), name
        bar = GRAD_TOL * max(1.0, float(np.max(np.abs(gr)))) if name == "dlog_gamma" else GRAD_TOL
        err = float(np.max(np.abs(_np(gk) - gr)))
        assert err <= bar, f"{name} max abs err {err:.3e} (bar {bar:.1e})"


def test_delta_gated_zero_decay_equals_ungated_kernel(cuda):
    """log gamma = 0 turns every decay factor into exactly 1: the gated kernels give the
    ungated kernels' y, H_T and gradients to fp32 rounding (the two sum some terms in a
    different order): max abs difference <= 1e-5 of the largest magnitude."""
    print("[gpu] delta gated zero decay vs ungated", flush=True)
    Q, K, V, beta, lg, H0, dy, dHT = _inputs(2, 2, 150, 2, 32, 32, seed=5, lg_kind="zero")
    y, HT, grads = _run((Q, K, V, beta, lg, H0), dy, dHT, 24, cuda)
    ts = [t.to(cuda).requires_grad_(True) for t in (Q, K, V, beta, H0)]
    y0, HT0 = hip_scans.delta_scan_impl(*ts, chunk_size=24)
    torch.autograd.backward([y0, HT0], [dy.to(cuda), dHT.to(cuda)])
    torch.cuda.synchronize()
    pairs = [("y", y, y0), ("H_T", HT, HT0)]
    pairs += list(zip(("dQ", "dK", "dV", "dbeta"), grads[:4], [t.grad for t in ts[:4]]))
    pairs.append(("dH0", grads[5], ts[4].grad))
    for name, a, b in pairs:
        bar = 1e-5 * max(1.0, b.abs().max().item())
        assert (a - b).abs().max().item() <= bar, name


@pytest.mark.parametrize("decay", ["fixed", "learnable"])
def test_delta_module_with_decay_runs_gated_kernel(cuda, decay, monkeypatch):
    """DeltaMinGRU with decay takes the gated kernel on the GPU; output, input and
    parameter gradients (incl. the learnable decay rate) match the float64 eager
    module on the CPU."""
    print(f"[gpu] DeltaMinGRU module decay={decay}", flush=True)
    torch.manual_seed(11)
    m = DeltaMinGRU(12, 32, n_heads=2, nh=2, chunk_size=16, decay=decay)
    m_ref = copy.deepcopy(m).double()
    x = torch.randn(2, 70, 12)
    dt = torch.rand(2, 70) * 1.5
    dt[:, 20] = 80.0
    gy = torch.randn(2, 70, 32)
    mg_ = m.to(cuda)
    xg = x.to(cuda).requires_grad_(True)
    y = mg_(xg, delta_t=dt.to(cuda))
    assert any("DeltaGatedScanFn" in type(n).__name__
               for n in _graph_nodes(y.grad_fn)), "gated kernel did not run"
    y.backward(gy.to(cuda))
    torch.cuda.synchronize()
    monkeypatch.setenv("MINGRU_SCAN", "eager")
    xr = x.double().requires_grad_(True)
    yr = m_ref(xr, delta_t=dt.double())
    yr.backward(gy.double())
    assert (y.detach().double().cpu() - yr.detach()).abs().max().item() <= FWD_TOL
    assert (xg.grad.double().cpu() - xr.grad).abs().max().item() <= GRAD_TOL
    for (name, p), (_, pr) in zip(mg_.named_parameters(), m_ref.named_parameters()):
        if pr.grad is None:
            assert p.grad is None, name
            continue
        err = (p.grad.double().cpu() - pr.grad).abs().max().item()
        assert err <= GRAD_TOL * max(1.0, pr.grad.abs().max().item()), f"{name} grad err {err:.3e}"


def _graph_nodes(fn, seen=None):
    seen = set() if seen is None else seen
    stack = [fn]
    while stack:
        f = stack.pop()
        if f is None or f in seen:
            continue
        seen.add(f)
        yield f
        stack.extend(n for n, _ in f.next_functions)


# bf16 Q, K, V, beta run the gated bf16-MFMA kernels (any nh).  Bars as for the
# ungated bf16 path: bf16 outputs (y, dQ, dK, dV, dbeta) within 2e-2 of the largest
# reference magnitude (the oracle sees the same bf16-rounded inputs); the fp32
# outputs (H_T, dH0, dlog_gamma) within 1e-4 of it.
BF16_REL = 2e-2
SPLIT_REL = 1e-4

BF16_CASES = [
    # B, H, T, nh, dk, dv, chunk, log-gamma kind
    (1, 1, 1, 1, 4, 4, 4, "mod"),
    (2, 2, 100, 1, 16, 16, 16, "mod"),
    (1, 3, 128, 1, 64, 64, 64, "mod"),
    (2, 1, 130, 1, 32, 48, 32, "spikes"),
    (1, 2, 300, 1, 64, 64, 64, "weak"),
    (2, 2, 200, 1, 64, 64, 64, "spikes"),
    (1, 2, 70, 1, 24, 40, 20, "zero"),
    # DeltaProduct: nh micro-steps per token on the bf16 kernels, the decay applied
    # once per token before them; 64 micro-steps per kernel tile (nh = 2 at chunk 64
    # runs 32-token tiles), ragged last tiles, saturating gaps.
    (2, 2, 150, 2, 64, 64, 32, "mod"),
    (1, 2, 200, 2, 64, 64, 64, "spikes"),
    (2, 1, 97, 3, 32, 48, 21, "weak"),
    (1, 3, 64, 3, 16, 16, 8, "spikes"),
    (1, 1, 1, 2, 8, 8, 4, "mod"),
    (1, 2, 40, 4, 64, 64, 16, "zero"),
]


def _rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(_np(got) - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.mark.parametrize("case", BF16_CASES)
def test_delta_gated_bf16_matches_oracle(cuda, case):
    B, H, T, nh, dk, dv, C, kind = case
    print(f"[gpu] delta gated bf16 case={case}", flush=True)
    Q, K, V, beta, lg, H0, dy, dHT = _inputs(B, H, T, nh, dk, dv, seed=41 + T + nh, lg_kind=kind)
    Q, K, V, beta, dy = (t.to(torch.bfloat16) for t in (Q, K, V, beta, dy))
    y, HT, grads = _run((Q, K, V, beta, lg, H0), dy, dHT, C, cuda)
    assert y.dtype == torch.bfloat16 and grads[0].dtype == torch.bfloat16
    assert grads[4].dtype == torch.float32
    # The bf16 kernels ran: y is the op's own bf16 output (an fp32 compute would end in
    # a cast, whose graph node _run's check on y.grad_fn would have rejected).
    ref = [_np(t) for t in (Q, K, V, beta, lg, H0)]
    ry, rHT = orc.delta_gated_sequential(*ref)
    assert _rel(y, ry) <= BF16_REL
    assert _rel(HT, rHT) <= SPLIT_REL, f"H_T rel err {_rel(HT, rHT):.3e}"
    rg = orc.delta_gated_sequential_bwd(*ref, _np(dy), _np(dHT))
    for name, gk, gr in zip(("dQ", "dK", "dV", "dbeta", "dlog_gamma", "dH0"), grads, rg):
        assert torch.isfinite(gk.float()).all(), name
        bar = SPLIT_REL if name in ("dlog_gamma", "dH0") else BF16_REL
        assert _rel(gk, gr) <= bar, f"{name} rel err {_rel(gk, gr):.3e}"


@pytest.mark.parametrize("nh", [1, 2])
def test_delta_gated_bf16_interleaved_calls(cuda, nh):
    """Two gated bf16 forwards before either backward: each backward reads its own
    forward's saved chunk states and chunk inverses while the shared workspace has been
    rewritten in between.  Bitwise equal to separate runs."""
    B, H, T, dk, dv, C = 2, 2, 150, 64, 64, 64 // nh
    print(f"[gpu] delta gated bf16 interleaved calls nh={nh}", flush=True)
    xs = []
    for seed in (51, 52):
        Q, K, V, beta, lg, H0, dy, dHT = _inputs(B, H, T, nh, dk, dv, seed=seed, lg_kind="mod")
        Q, K, V, beta, dy = (t.to(torch.bfloat16) for t in (Q, K, V, beta, dy))
        xs.append(((Q, K, V, beta, lg, H0), dy, dHT))
    ref = [_run(ins, dy, dHT, C, cuda) for ins, dy, dHT in xs]
    leaves, outs = [], []
    for ins, _, _ in xs:
        ts = [t.to(cuda).requires_grad_(True) for t in ins]
        leaves.append(ts)
        outs.append(hip_scans.delta_gated_scan_impl(*ts, chunk_size=C))
    for (y, HT), (_, dy, dHT) in zip(outs[::-1], xs[::-1]):  # second call's backward first
        torch.autograd.backward([y, HT], [dy.to(cuda), dHT.to(cuda)])
    torch.cuda.synchronize()
    for (y, HT), ts, (ry, rHT, rg) in zip(outs, leaves, ref):
        assert torch.equal(y, ry) and torch.equal(HT, rHT)
        for g, rgk in zip((t.grad for t in ts), rg):
            assert torch.equal(g, rgk)


def test_delta_gated_bf16_c5_heads(cuda):
    """The C5d workload in bf16 (B=8, H=8, T=8192, d=64, chunk 64): two heads at full
    length against the oracle, from the first and the second half of the 64 (batch,
    head) pairs."""
    from mingru_amd import workloads as wl

    print("[gpu] delta gated bf16 C5 heads", flush=True)
    inp = wl.c5d_inputs(**wl.C5)
    Q, K, V, beta = (inp[k].to(torch.bfloat16) for k in ("Q", "K", "V", "beta"))
    lg, H0 = inp["log_gamma"], inp["H0"]
    dy, dHT = inp["grad_y"].to(torch.bfloat16), inp["grad_HT"]
    y, HT, grads = _run((Q, K, V, beta, lg, H0), dy, dHT, inp["chunk_size"], cuda)
    for sel in ((slice(1, 2), slice(6, 7)), (slice(5, 6), slice(1, 2))):  # pairs 14 and 41
        sub = [_np(t[sel]) for t in (Q, K, V, beta, lg, H0)]
        ry, rHT = orc.delta_gated_sequential(*sub)
        assert _rel(y[sel], ry) <= BF16_REL
        assert _rel(HT[sel], rHT) <= BF16_REL
        rg = orc.delta_gated_sequential_bwd(*sub, _np(dy[sel]), _np(dHT[sel]))
        for name, gk, gr in zip(("dQ", "dK", "dV", "dbeta", "dlog_gamma", "dH0"), grads, rg):
            assert _rel(gk[sel], gr) <= BF16_REL, f"{name} rel err {_rel(gk[sel], gr):.3e}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_delta_gated_chaining_at_misaligned_boundary(cuda, dtype):
    """Gated chaining: [0, T1) then [T1, T) with the first call's H_T as the second's H_0
    gives the single run's y and H_T at a split inside a chunk, including decay spikes
    (the reference's chaining property, tests/test_mixers.py:834-854, with the decay of
    _forward_chunked_gated).  Bars as the parity bars: fp32 within twice 1e-4, bf16 y
    within the bf16 bar, the fp32 state within 2e-4 relative."""
    B, H, T, C, T1 = 2, 2, 150, 32, 77
    print(f"[gpu] delta gated chaining dtype={dtype}", flush=True)
    Q, K, V, beta, lg, H0, _, _ = _inputs(B, H, T, 1, 64, 64, seed=43, lg_kind="spikes")
    seq = [t.to(dtype).to(cuda) for t in (Q, K, V, beta)]
    lg, h0 = lg.to(cuda), H0.to(cuda)
    with torch.no_grad():
        y, HT = hip_scans.delta_gated_scan_impl(*seq, lg, h0, chunk_size=C)
        ya, Ha = hip_scans.delta_gated_scan_impl(*(t[:, :, :T1] for t in seq), lg[:, :, :T1], h0,
                                                 chunk_size=C)
        yb, Hb = hip_scans.delta_gated_scan_impl(*(t[:, :, T1:] for t in seq), lg[:, :, T1:], Ha,
                                                 chunk_size=C)
    torch.cuda.synchronize()
    ys = torch.cat([ya, yb], dim=2)
    if dtype == torch.float32:
        assert (ys - y).abs().max().item() <= 2 * FWD_TOL
        assert (Hb - HT).abs().max().item() <= 2 * FWD_TOL
    else:
        assert _rel(ys, _np(y)) <= BF16_REL
        assert _rel(Hb, _np(HT)) <= 2 * SPLIT_REL
