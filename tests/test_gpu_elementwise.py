"""GPU parity: HIP ``linear_scan`` / ``parallel_scan_log`` vs the fp64 oracle.

Bars (stated for the hot path): fp32 forward max abs err <= 1e-4 and gradients
<= 1e-3 against the float64 oracle on identical seeded inputs.  Full-size
workloads are checked on a subset of batch rows (lanes are independent) plus
size-independent properties.
"""

import numpy as np
import pytest
import torch

from mingru_amd import linear_scan, parallel_scan_log
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


def _run_linear(a, b, gA, gB, cuda):
    ag = a.to(cuda).requires_grad_(True)
    bg = b.to(cuda).requires_grad_(True)
    A, Bc = linear_scan(ag, bg)
    assert "LinearScanFn" in type(A.grad_fn).__name__, "HIP path did not run"
    torch.autograd.backward([A, Bc], [gA.to(cuda), gB.to(cuda)])
    torch.cuda.synchronize()
    return A, Bc, ag.grad, bg.grad


LINEAR_SHAPES = [
    (1, 1, 1),
    (2, 5, 3),
    (2, 13, 64),
    (3, 64, 256),
    (2, 65, 257),
    (2, 1000, 128),
    (1, 4097, 1024),
    (4, 333, 12),
    # the launch picks 4 columns per lane here, 2 at D=128 below, 1 for the small shapes
    (8, 2048, 512),
    (32, 1024, 128),
    # launch forms (64-step chunks both ways; at most 32 chunks and 32 MB of inputs run
    # as two launches): both directions two-launch; forward two-launch with a look-back
    # backward (its four input arrays pass 32 MB); both look-back
    (2, 2048, 64),
    (2, 2048, 640),
    (2, 4097, 64),
]


@pytest.mark.parametrize("shape", LINEAR_SHAPES)
def test_linear_scan_matches_oracle(cuda, shape):
    B, T, D = shape
    print(f"[gpu] linear_scan shape={shape}", flush=True)
    g = torch.Generator().manual_seed(7 + T + D)
    a = torch.tanh(2 * torch.randn(B, T, D, generator=g))
    b = torch.randn(B, T, D, generator=g)
    gA = torch.randn(B, T, D, generator=g)
    gB = torch.randn(B, T, D, generator=g)
    A, Bc, da, db = _run_linear(a, b, gA, gB, cuda)
    rA, rB = orc.linear_scan(a.numpy(), b.numpy())
    rda, rdb = orc.linear_scan_bwd(a.numpy(), b.numpy(), gA.numpy(), gB.numpy())
    assert _maxerr(A, rA) <= FWD_TOL
    assert _maxerr(Bc, rB) <= FWD_TOL
    assert _maxerr(da, rda) <= GRAD_TOL
    assert _maxerr(db, rdb) <= GRAD_TOL


def test_linear_scan_c2_full_size(cuda):
    print("[gpu] linear_scan C2 full size", flush=True)
    inp = wl.c2_inputs(**wl.C2)
    a, b, gA, gB = inp["a"], inp["b"], inp["grad_A"], inp["grad_Bc"]
    A, Bc, da, db = _run_linear(a, b, gA, gB, cuda)
    rows = [0, wl.C2["B"] - 1]
    for r in rows:
        sl = slice(r, r + 1)
        rA, rB = orc.linear_scan(a[sl].numpy(), b[sl].numpy())
        rda, rdb = orc.linear_scan_bwd(a[sl].numpy(), b[sl].numpy(), gA[sl].numpy(),
                                       gB[sl].numpy())
        assert _maxerr(A[sl], rA) <= FWD_TOL
        assert _maxerr(Bc[sl], rB) <= FWD_TOL
        assert _maxerr(da[sl], rda) <= GRAD_TOL
        assert _maxerr(db[sl], rdb) <= GRAD_TOL
    # size-independent: the last step of every lane satisfies the recurrence exactly
    last = Bc[:, -1]
    prev = Bc[:, -2]
    rec = a[:, -1].to(cuda) * prev + b[:, -1].to(cuda)
    assert torch.allclose(last, rec, atol=1e-5)
    assert torch.isfinite(da).all() and torch.isfinite(db).all()


def test_linear_scan_identity_is_cumsum(cuda):
    B, T, D = 2, 3000, 256
    b = torch.randn(B, T, D, generator=torch.Generator().manual_seed(3))
    A, Bc = linear_scan(torch.ones(B, T, D, device=cuda), b.to(cuda))
    assert torch.equal(A, torch.ones_like(A))
    ref = np.cumsum(b.double().numpy(), axis=1)
    assert _maxerr(Bc, ref) <= 1e-3  # cumsum of 3000 N(0,1): fp32 rounding of |x| ~ 50


def test_linear_scan_long_sequence_exact(cuda):
    """T = 2**20 (about 8,000 look-back chunks along T; C2 has 32) with a = 1 and integer
    b, gB in [-2, 2]: every partial sum is an integer below 2**21, exact in fp32 under any
    association, so the scan must equal the fp64 closed forms bit for bit: A = 1,
    Bc = cumsum(b), db = reverse cumsum(gB) and da_t = db_t * Bc_{t-1} (one rounding)."""
    B, T, D = 1, 1 << 20, 64
    print(f"[gpu] linear_scan long sequence T={T}", flush=True)
    gen = torch.Generator(device=cuda).manual_seed(12)
    b = torch.randint(-2, 3, (B, T, D), device=cuda, generator=gen).float()
    gB = torch.randint(-2, 3, (B, T, D), device=cuda, generator=gen).float()
    a = torch.ones(B, T, D, device=cuda, requires_grad=True)
    bg = b.clone().requires_grad_(True)
    A, Bc = linear_scan(a, bg)
    torch.autograd.backward([A, Bc], [torch.zeros_like(A), gB])
    torch.cuda.synchronize()
    assert torch.equal(A, torch.ones_like(A))
    ref = b.double().cumsum(1)
    assert torch.equal(Bc.double(), ref)
    y = gB.double().flip(1).cumsum(1).flip(1)
    assert torch.equal(bg.grad.double(), y)
    prev = torch.cat([torch.zeros_like(ref[:, :1]), ref[:, :-1]], dim=1)
    assert torch.equal(a.grad, (y * prev).float())


def _run_log(lc, lv, gh, cuda):
    lcg = lc.to(cuda).requires_grad_(True)
    lvg = lv.to(cuda).requires_grad_(True)
    h = parallel_scan_log(lcg, lvg)
    assert "LogScanFn" in type(h.grad_fn).__name__, "HIP path did not run"
    h.backward(gh.to(cuda))
    torch.cuda.synchronize()
    return h, lcg.grad, lvg.grad


# Launch forms (64-step chunks): up to 32 chunks per sequence and 32 MB of inputs run
# as two launches (chunk aggregates, then every chunk folds its predecessors'), the
# rest as one look-back launch.  (2, 2048, 64) is the longest two-launch sequence and
# (2, 2049, 64) / (1, 2049, 512) the shortest look-back ones; (8, 2048, 512) and
# (32, 1024, 128) take the look-back form by size.
LOG_SHAPES = [(1, 1, 1), (2, 7, 5), (3, 64, 64), (2, 200, 130), (4, 1024, 256), (2, 2048, 64),
              (2, 2049, 64), (1, 2049, 512), (8, 2048, 512), (32, 1024, 128)]


@pytest.mark.parametrize("shape", LOG_SHAPES)
def test_parallel_scan_log_matches_oracle(cuda, shape):
    B, T, D = shape
    print(f"[gpu] parallel_scan_log shape={shape}", flush=True)
    inp = wl.c1_inputs(B, T, D)
    lc, lv, gh = inp["log_coeffs"], inp["log_values"], inp["grad_h"]
    h, dlc, dlv = _run_log(lc, lv, gh, cuda)
    rh = orc.parallel_scan_log(lc.numpy(), lv.numpy())
    rdlc, rdlv = orc.parallel_scan_log_bwd(lc.numpy(), lv.numpy(), gh.numpy())
    assert _maxerr(h, rh) <= FWD_TOL
    assert _maxerr(dlc, rdlc) <= GRAD_TOL
    assert _maxerr(dlv, rdlv) <= GRAD_TOL


def test_parallel_scan_log_beats_fp32_eager_accuracy(cuda):
    """The linear-space kernel is closer to fp64 than the fp32 log-space eager body."""
    inp = wl.c1_inputs(**wl.C1)
    lc, lv = inp["log_coeffs"], inp["log_values"]
    rh = orc.parallel_scan_log(lc.numpy(), lv.numpy())
    h = parallel_scan_log(lc.to(cuda), lv.to(cuda))
    import os

    os.environ["MINGRU_SCAN"] = "eager"
    h_eager = parallel_scan_log(lc, lv)
    os.environ["MINGRU_SCAN"] = "hip"
    assert _maxerr(h, rh) <= _maxerr(h_eager, rh)


def test_non_contiguous_inputs(cuda):
    """Strided views (a transposed base tensor) give the same results as contiguous copies."""
    print("[gpu] linear_scan / parallel_scan_log non-contiguous views", flush=True)
    g = torch.Generator().manual_seed(99)
    base_a = torch.tanh(torch.randn(2, 48, 130, generator=g)).to(cuda)  # (B, D, T)
    base_b = torch.randn(2, 48, 130, generator=g).to(cuda)
    a, b = base_a.transpose(1, 2), base_b.transpose(1, 2)  # (B, T, D), non-contiguous
    assert not a.is_contiguous()
    A, Bc = linear_scan(a, b)
    A2, Bc2 = linear_scan(a.contiguous(), b.contiguous())
    assert torch.allclose(A, A2, rtol=1e-5, atol=1e-6) and torch.allclose(Bc, Bc2, rtol=1e-5, atol=1e-5)
    rA, rB = orc.linear_scan(a.double().cpu().numpy(), b.double().cpu().numpy())
    assert _maxerr(A, rA) <= FWD_TOL and _maxerr(Bc, rB) <= FWD_TOL
    lc = -torch.nn.functional.softplus(base_a).transpose(1, 2)
    lv = torch.randn(2, 48, 131, generator=g).to(cuda).transpose(1, 2) * 0.1
    h = parallel_scan_log(lc, lv)
    rh = orc.parallel_scan_log(lc.double().cpu().numpy(), lv.double().cpu().numpy())
    assert _maxerr(h, rh) <= FWD_TOL


def test_parallel_scan_log_long_sequence(cuda):
    """T = 2**20 with log a = 0: h_t = h_0 + sum_{s<=t} b_s with b_s = exp(lv_s) > 0, a sum of
    positive terms (no cancellation), checked against the fp64 cumulative sum to 1e-5
    relative at every step."""
    B, T, D = 1, 1 << 20, 64
    print(f"[gpu] parallel_scan_log long sequence T={T}", flush=True)
    gen = torch.Generator(device=cuda).manual_seed(13)
    lc = torch.zeros(B, T, D, device=cuda)
    lv = -2.0 + 0.5 * torch.randn(B, T + 1, D, device=cuda, generator=gen)
    h = parallel_scan_log(lc, lv)
    torch.cuda.synchronize()
    ref = lv.double().exp().cumsum(1)[:, 1:]
    rel = ((h.double() - ref).abs() / ref).max().item()
    print(f"[gpu] parallel_scan_log long sequence max rel err {rel:.3e}", flush=True)
    assert rel <= 1e-5


# ---------------------------------------------------------------------------
# parallel_scan_log over the whole fp32 log domain
# ---------------------------------------------------------------------------

FLT_MAX = float(np.finfo(np.float32).max)
FLT_MIN = float(np.finfo(np.float32).tiny)


def _heinsen_fp64(lc, lv):
    """The reference's log-space formula (src/mingru/min_gru.py:804-807) in float64:
    a* = pad(cumsum(lc)), h = exp(a* + logcumsumexp(lv - a*))[1:]."""
    lc = np.asarray(lc, np.float64)
    lv = np.asarray(lv, np.float64)
    a_star = np.concatenate([np.zeros_like(lc[:, :1]), np.cumsum(lc, axis=1)], axis=1)
    log_h = a_star + np.logaddexp.accumulate(lv - a_star, axis=1)
    return np.exp(log_h)[:, 1:]


def _assert_extended_close(x, ref, rtol, what):
    """Elementwise check of an fp32 result against a float64 reference that may lie
    outside fp32's range: +-inf where the reference overflows fp32, |err| <= 2 FLT_MIN
    where it underflows, and relative error <= rtol (plus rtol times the column's
    largest finite magnitude, for sums with cancellation) elsewhere."""
    x = x.detach().double().cpu().numpy()
    ref = np.asarray(ref, np.float64)
    big = np.abs(ref) > FLT_MAX * (1 + 1e-6)
    assert np.all(np.isinf(x[big]) & (np.sign(x[big]) == np.sign(ref[big]))), f"{what}: overflow"
    tiny = np.abs(ref) < FLT_MIN
    assert np.all(np.abs(x[tiny] - ref[tiny]) <= 2 * FLT_MIN), f"{what}: underflow"
    mid = ~big & ~tiny & (np.abs(ref) < FLT_MAX * (1 - 1e-6))
    scale = np.where(np.isfinite(ref) & ~big, np.abs(ref), 0.0).max(axis=1, keepdims=True)
    bound = rtol * (np.abs(ref) + 1e-3 * scale)
    err = np.abs(x - ref)
    worst = float(np.max(np.where(mid, err / np.maximum(bound, 1e-300), 0.0)))
    assert np.all(err[mid] <= bound[mid]), f"{what}: worst err/bound {worst:.3g}"


EXTREME_CASES = {
    # e^-150 initial state grown by e per step: h_199 = e^50 (5.18e21) although
    # h_-1 and every b_t underflow fp32.
    "grow_from_underflow": (1.0, -150.0, -200.0),
    # e^120 initial state (overflows fp32) decaying by e^-1 per step towards the
    # small inputs: h_199 = 0.0107.
    "decay_from_overflow": (-1.0, 120.0, -5.0),
}


@pytest.mark.parametrize("case", sorted(EXTREME_CASES))
def test_parallel_scan_log_extended_range(cuda, case):
    """Inputs whose exponentials leave fp32's range while the outputs (or part of them)
    stay inside it: fwd and grads against the float64 oracle, and the forward also
    against the reference's float64 log-space formula."""
    c, v0, v = EXTREME_CASES[case]
    B, T, D = 2, 200, 70
    print(f"[gpu] parallel_scan_log extended range case={case}", flush=True)
    g = torch.Generator().manual_seed(31)
    lc = torch.full((B, T, D), c) + 0.01 * torch.randn(B, T, D, generator=g)
    lv = torch.full((B, T + 1, D), v) + 0.5 * torch.randn(B, T + 1, D, generator=g)
    lv[:, 0] = v0 + 0.5 * torch.randn(B, D, generator=g)
    gh = torch.randn(B, T, D, generator=g)
    h, dlc, dlv = _run_log(lc, lv, gh, cuda)
    rh = orc.parallel_scan_log(lc.numpy(), lv.numpy())
    np.testing.assert_allclose(rh, _heinsen_fp64(lc.numpy(), lv.numpy()), rtol=1e-9)
    if case == "grow_from_underflow":
        assert 1e20 < rh[0, -1, 0] < 1e23
    else:
        assert 0.005 < rh[0, -1, 0] < 0.03 and np.isinf(np.float32(rh[0, 0, 0]))
    rdlc, rdlv = orc.parallel_scan_log_bwd(lc.numpy(), lv.numpy(), gh.numpy())
    _assert_extended_close(h, rh, 2e-5, "h")
    _assert_extended_close(dlc, rdlc, 1e-4, "dlc")
    _assert_extended_close(dlv, rdlv, 1e-4, "dlv")


def test_parallel_scan_log_backward_without_state_record(cuda):
    """The C ABI's backward with no forward record (hstate = NULL) restarts from the fp32
    outputs: same gradients as with the record for inputs inside fp32's range."""
    import ctypes

    from mingru_amd import _native

    print("[gpu] parallel_scan_log backward with hstate = NULL", flush=True)
    lib = _native.load()
    inp = wl.c1_inputs(3, 517, 96)
    lc, lv, gh = (inp[k].to(cuda).contiguous() for k in ("log_coeffs", "log_values", "grad_h"))
    B, T, D = lc.shape
    p = lambda t: ctypes.c_void_p(t.data_ptr() if t is not None else 0)  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ws = torch.zeros(lib.mg_log_scan_workspace_bytes(B, T, D), dtype=torch.uint8, device=cuda)
    hs = torch.empty(lib.mg_log_scan_state_bytes(B, T, D) // 4, device=cuda)
    h = torch.empty_like(lc)
    assert lib.mg_log_scan_fwd(p(lc), p(lv), p(h), p(hs), B, T, D, p(ws), ws.numel(), stream) == 0
    grads = []
    for state in (hs, None):
        dlc, dlv = torch.empty_like(lc), torch.empty_like(lv)
        assert lib.mg_log_scan_bwd(p(lc), p(lv), p(h), p(state), p(gh), p(dlc), p(dlv), B, T, D,
                                   p(ws), ws.numel(), stream) == 0
        grads.append((dlc, dlv))
    torch.cuda.synchronize()
    rdlc, rdlv = orc.parallel_scan_log_bwd(*(inp[k].numpy() for k in ("log_coeffs", "log_values",
                                                                     "grad_h")))
    for dlc, dlv in grads:
        assert _maxerr(dlc, rdlc) <= GRAD_TOL and _maxerr(dlv, rdlv) <= GRAD_TOL
    assert int(ws[8:12].view(torch.int32).item()) == 0


# Small problems (at most 32 chunks per sequence and 32 MB of inputs) run as one launch
# whose workgroups publish their chunk aggregates and fold their predecessors' (when the
# whole grid is resident, as at these shapes), or as two launches (aggregates, then the
# fold).  MINGRU_HIP_EW_FORM=two forces the second form, so both are checked here.
SMALL_FORM_SHAPES = [(4, 1024, 256), (2, 2048, 64), (2, 777, 136), (3, 64, 64), (1, 5, 3)]


@pytest.mark.parametrize("form", ["auto", "two"])
@pytest.mark.parametrize("shape", SMALL_FORM_SHAPES)
def test_small_problem_launch_forms(cuda, shape, form, monkeypatch):
    B, T, D = shape
    print(f"[gpu] launch form {form}: linear_scan + parallel_scan_log shape={shape}", flush=True)
    monkeypatch.setenv("MINGRU_HIP_EW_FORM", form)
    g = torch.Generator().manual_seed(5 + T + D)
    a = torch.tanh(2 * torch.randn(B, T, D, generator=g))
    b = torch.randn(B, T, D, generator=g)
    gA = torch.randn(B, T, D, generator=g)
    gB = torch.randn(B, T, D, generator=g)
    A, Bc, da, db = _run_linear(a, b, gA, gB, cuda)
    rA, rB = orc.linear_scan(a.numpy(), b.numpy())
    rda, rdb = orc.linear_scan_bwd(a.numpy(), b.numpy(), gA.numpy(), gB.numpy())
    assert _maxerr(A, rA) <= FWD_TOL and _maxerr(Bc, rB) <= FWD_TOL
    assert _maxerr(da, rda) <= GRAD_TOL and _maxerr(db, rdb) <= GRAD_TOL
    inp = wl.c1_inputs(B, T, D)
    lc, lv, gh = inp["log_coeffs"], inp["log_values"], inp["grad_h"]
    h, dlc, dlv = _run_log(lc, lv, gh, cuda)
    rh = orc.parallel_scan_log(lc.numpy(), lv.numpy())
    rdlc, rdlv = orc.parallel_scan_log_bwd(lc.numpy(), lv.numpy(), gh.numpy())
    assert _maxerr(h, rh) <= FWD_TOL
    assert _maxerr(dlc, rdlc) <= GRAD_TOL and _maxerr(dlv, rdlv) <= GRAD_TOL
