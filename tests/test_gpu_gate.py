"""GPU parity: the fused SignedMinGRU gate scan (gates + linear_scan + h0 in one kernel).

The reference is the mixer's own arithmetic (``src/mingru/min_gru.py:1788-1857``):
a = tanh(s) (times 1 - sigmoid(z) when coupled), b = sigmoid(z) * hpre,
h_t = a_t h_{t-1} + b_t from h0, run as a sequential float64 recurrence on the CPU
and differentiated by torch autograd, so the forward and all four input gradients
are checked against an independent derivation.  Bars: forward max abs err <= 1e-4,
gradients <= 1e-3 (float64 reference, fp32 kernels).
"""

import copy

import pytest
import torch

from mingru_amd import SignedMinGRU, hip_scans

FWD_TOL = 1e-4
GRAD_TOL = 1e-3

pytestmark = pytest.mark.gpu


def _ref(s, z, hp, h0, coupled):
    sg, th = torch.sigmoid(z), torch.tanh(s)
    a = (1 - sg) * th if coupled else th
    b = sg * hp
    h, out = h0[:, 0], []
    for t in range(s.shape[1]):
        h = a[:, t] * h + b[:, t]
        out.append(h)
    return torch.stack(out, 1)


CASES = [
    # B, T, D, coupled
    (2, 777, 136, False),
    (2, 777, 136, True),
    (3, 1, 64, False),
    (1, 300, 7, True),
    (4, 1024, 256, False),
    (2, 65, 260, True),
    (8, 2048, 512, False),  # 4 columns per lane
    (32, 1024, 128, True),  # 2 columns per lane
    # The backward's 32-step chunks: 32 per sequence still run as two launches,
    # 33 as one look-back launch.
    (2, 1024, 64, False),
    (2, 1025, 64, True),
]


@pytest.mark.parametrize("case", CASES)
def test_signed_gate_scan_matches_fp64(cuda, case):
    B, T, D, coupled = case
    print(f"[gpu] signed gate scan case={case}", flush=True)
    g = torch.Generator().manual_seed(31 + T + D)
    s, z, hp = (torch.randn(B, T, D, generator=g) for _ in range(3))
    h0 = torch.randn(B, 1, D, generator=g)
    gh = torch.randn(B, T, D, generator=g)
    ins = [t.to(cuda).requires_grad_(True) for t in (s, z, hp, h0)]
    h = hip_scans.signed_gate_scan_impl(*ins, coupled=coupled)
    assert "SignedGateScanFn" in type(h.grad_fn).__name__, "HIP path did not run"
    h.backward(gh.to(cuda))
    torch.cuda.synchronize()
    refs = [t.double().requires_grad_(True) for t in (s, z, hp, h0)]
    hr = _ref(*refs, coupled)
    hr.backward(gh.double())
    assert (h.detach().double().cpu() - hr.detach()).abs().max().item() <= FWD_TOL
    for name, x, xr in zip(("ds", "dz", "dhpre", "dh0"), ins, refs):
        err = (x.grad.double().cpu() - xr.grad).abs().max().item()
        assert err <= GRAD_TOL, f"{name} max abs err {err:.3e}"


@pytest.mark.parametrize("coupled", [False, True])
def test_signed_mingru_module_runs_fused_and_matches_fp64(cuda, coupled, monkeypatch):
    """The module takes the fused path on the GPU; output, input and parameter
    gradients match the float64 eager module on the CPU."""
    print(f"[gpu] SignedMinGRU module fused coupled={coupled}", flush=True)
    torch.manual_seed(7)
    m = SignedMinGRU(24, 48, coupled=coupled, learnable_h0=True)
    m_ref = copy.deepcopy(m).double()
    x = torch.randn(3, 200, 24)
    gy = torch.randn(3, 200, 48)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    mg = m.to(cuda)
    xg = x.to(cuda).requires_grad_(True)
    y = mg(xg)
    assert "SignedGateScanFn" in type(y.grad_fn).__name__, "fused path did not run"
    y.backward(gy.to(cuda))
    torch.cuda.synchronize()
    monkeypatch.setenv("MINGRU_SCAN", "eager")
    xr = x.double().requires_grad_(True)
    yr = m_ref(xr)
    yr.backward(gy.double())
    assert (y.detach().double().cpu() - yr.detach()).abs().max().item() <= FWD_TOL
    assert (xg.grad.double().cpu() - xr.grad).abs().max().item() <= GRAD_TOL
    for (name, p), (_, pr) in zip(mg.named_parameters(), m_ref.named_parameters()):
        err = (p.grad.double().cpu() - pr.grad).abs().max().item()
        assert err <= GRAD_TOL, f"{name} grad max abs err {err:.3e}"


def _ref_decay(s, z, hp, h0, dt, lam, coupled):
    """The mixer's decay-active coefficients (a times exp(-lam dt)) and the sequential
    recurrence, differentiable in every input."""
    sg, th = torch.sigmoid(z), torch.tanh(s)
    a = ((1 - sg) * th if coupled else th) * torch.exp(-lam * dt.unsqueeze(-1))
    b = sg * hp
    h, out = h0[:, 0], []
    for t in range(s.shape[1]):
        h = a[:, t] * h + b[:, t]
        out.append(h)
    return torch.stack(out, 1)


DECAY_CASES = [
    # B, T, D, coupled, per-channel rate
    (2, 777, 136, False, True),
    (3, 300, 70, True, False),  # a scalar rate; 70 columns: a partial 64-column tile
    (4, 1024, 256, True, True),
    (2, 3000, 512, False, True),  # the look-back launch
    (1, 1, 8, False, True),
]


@pytest.mark.parametrize("case", DECAY_CASES)
def test_signed_gate_scan_decay_matches_fp64(cuda, case):
    """The decay-active fused kernel against float64 autograd: h and the gradients of
    s, z, hpre, h0, dt and lam (dt with a saturating gap and zeros)."""
    B, T, D, coupled, per_channel = case
    print(f"[gpu] signed gate scan with decay case={case}", flush=True)
    g = torch.Generator().manual_seed(41 + T + D)
    s, z, hp = (torch.randn(B, T, D, generator=g) for _ in range(3))
    h0 = torch.randn(B, 1, D, generator=g)
    dt = torch.rand(B, T, generator=g) * 2
    dt[:, T // 2] = 0.0
    if T > 2:
        dt[0, 1] = 60.0  # gamma underflows to zero there
    lam = (torch.rand(D, generator=g) + 0.1) if per_channel else torch.tensor(0.8)
    gh = torch.randn(B, T, D, generator=g)
    ins = [t.to(cuda).requires_grad_(True) for t in (s, z, hp, h0, dt, lam)]
    h = hip_scans.signed_gate_scan_impl(*ins[:4], coupled=coupled, dt=ins[4], lam=ins[5])
    assert "SignedGateScanFn" in type(h.grad_fn).__name__, "HIP path did not run"
    h.backward(gh.to(cuda))
    torch.cuda.synchronize()
    refs = [t.double().requires_grad_(True) for t in (s, z, hp, h0, dt, lam)]
    hr = _ref_decay(*refs, coupled)
    hr.backward(gh.double())
    assert (h.detach().double().cpu() - hr.detach()).abs().max().item() <= FWD_TOL
    for name, x, xr in zip(("ds", "dz", "dhpre", "dh0", "ddt", "dlam"), ins, refs):
        scale = max(1.0, xr.grad.abs().max().item()) if name in ("ddt", "dlam") else 1.0
        err = (x.grad.double().cpu() - xr.grad).abs().max().item() / scale
        assert err <= GRAD_TOL, f"{name} max abs err {err:.3e} (scale {scale:.3g})"


@pytest.mark.parametrize("decay", ["fixed", "learnable"])
@pytest.mark.parametrize("coupled", [False, True])
def test_signed_mingru_decay_module_runs_fused_and_matches_fp64(cuda, decay, coupled,
                                                                monkeypatch):
    """With decay the module runs the fused kernel; output, input, delta_t and parameter
    gradients (the learnable rate's rho included) match the float64 eager module."""
    print(f"[gpu] SignedMinGRU module decay={decay} coupled={coupled}", flush=True)
    torch.manual_seed(11)
    m = SignedMinGRU(24, 48, coupled=coupled, learnable_h0=True, decay=decay, decay_rate=0.6)
    m_ref = copy.deepcopy(m).double()
    x = torch.randn(3, 200, 24)
    dt = torch.rand(3, 200) * 3
    dt[1, 7] = float("nan")  # normalised to 0 by the module
    gy = torch.randn(3, 200, 48)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    mg = m.to(cuda)
    xg = x.to(cuda).requires_grad_(True)
    dtg = dt.to(cuda).requires_grad_(True)
    y = mg(xg, delta_t=dtg)
    assert "SignedGateScanFn" in type(y.grad_fn).__name__, "fused path did not run"
    y.backward(gy.to(cuda))
    torch.cuda.synchronize()
    monkeypatch.setenv("MINGRU_SCAN", "eager")
    xr = x.double().requires_grad_(True)
    dtr = dt.double().requires_grad_(True)
    yr = m_ref(xr, delta_t=dtr)
    yr.backward(gy.double())
    assert (y.detach().double().cpu() - yr.detach()).abs().max().item() <= FWD_TOL
    assert (xg.grad.double().cpu() - xr.grad).abs().max().item() <= GRAD_TOL
    sc = max(1.0, dtr.grad.abs().max().item())
    assert (dtg.grad.double().cpu() - dtr.grad).abs().max().item() / sc <= GRAD_TOL
    for (name, p), (_, pr) in zip(mg.named_parameters(), m_ref.named_parameters()):
        sc = max(1.0, pr.grad.abs().max().item())
        err = (p.grad.double().cpu() - pr.grad).abs().max().item() / sc
        assert err <= GRAD_TOL, f"{name} grad max abs err {err:.3e} (scale {sc:.3g})"


@pytest.mark.parametrize("case", [(2, 777, 136, False), (4, 1024, 256, True), (2, 1024, 64, False)])
def test_small_problem_two_launch_form(cuda, case, monkeypatch):
    """The same parity on the two-launch form (MINGRU_HIP_EW_FORM=two); by default these
    shapes run as one launch whose workgroups fold their predecessors' aggregates."""
    monkeypatch.setenv("MINGRU_HIP_EW_FORM", "two")
    test_signed_gate_scan_matches_fp64(cuda, case)
