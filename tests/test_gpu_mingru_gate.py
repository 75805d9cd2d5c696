"""GPU parity: the fused MinGRU gate scan (log-space gates + parallel_scan_log in one kernel).

The reference is the mixer's own log-space arithmetic (``src/mingru/min_gru.py:
1366-1397``): log(1 - z) = -softplus(k), log z = -softplus(-k), log h~ = log_g(hpre),
h = exp(parallel_scan_log(log(1 - z), [log h0, log z + log h~])), evaluated in float64
on the CPU with the eager log-space scan (logcumsumexp) and differentiated by torch
autograd.  The kernel runs the linear recurrence instead, so this checks the
log-space/linear equivalence as well as the forward and all three input gradients.
Bars: forward max abs err <= 1e-4, gradients <= 1e-3 (float64 reference, fp32 kernels).
"""

import copy

import pytest
import torch
import torch.nn.functional as F

from mingru_amd import MinGRU, hip_scans
from mingru_amd import min_gru as mg

FWD_TOL = 1e-4
GRAD_TOL = 1e-3

pytestmark = pytest.mark.gpu


def _ref(k, hp, log_h0):
    log_coeffs = -F.softplus(k)
    log_values = torch.cat([log_h0, -F.softplus(-k) + mg.log_g(hp)], dim=1)
    a_star = F.pad(torch.cumsum(log_coeffs, dim=1), (0, 0, 1, 0))
    log_h = a_star + torch.logcumsumexp(log_values - a_star, dim=1)
    return torch.exp(log_h)[:, 1:]


CASES = [
    # B, T, D, input scale
    (2, 777, 136, 2.0),
    (3, 1, 64, 1.0),
    (1, 300, 7, 3.0),
    (4, 1024, 256, 1.0),
    (2, 65, 260, 2.0),
    (2, 129, 64, 30.0),  # saturated gates: z and g at 0/1, sigmoid(-k) underflowing
    (8, 2048, 512, 1.0),  # 4 columns per lane
    (32, 1024, 128, 2.0),  # 2 columns per lane
    # The backward's 32-step chunks: 32 per sequence still run as two launches,
    # 33 as one look-back launch.
    (2, 1024, 64, 1.0),
    (2, 1025, 64, 1.0),
]


@pytest.mark.parametrize("case", CASES)
def test_mingru_gate_scan_matches_fp64(cuda, case):
    B, T, D, scale = case
    print(f"[gpu] MinGRU gate scan case={case}", flush=True)
    g = torch.Generator().manual_seed(17 + T + D)
    k = torch.randn(B, T, D, generator=g) * scale
    hp = torch.randn(B, T, D, generator=g) * scale
    log_h0 = torch.rand(B, 1, D, generator=g).clamp_min(0.05).log()
    gh = torch.randn(B, T, D, generator=g)
    ins = [t.to(cuda).requires_grad_(True) for t in (k, hp, log_h0)]
    h = hip_scans.mingru_gate_scan_impl(*ins)
    assert "MinGRUGateScanFn" in type(h.grad_fn).__name__, "HIP path did not run"
    h.backward(gh.to(cuda))
    torch.cuda.synchronize()
    refs = [t.double().requires_grad_(True) for t in (k, hp, log_h0)]
    hr = _ref(*refs)
    hr.backward(gh.double())
    assert (h.detach().double().cpu() - hr.detach()).abs().max().item() <= FWD_TOL
    for name, x, xr in zip(("dk", "dhpre", "dlog_h0"), ins, refs):
        assert torch.isfinite(x.grad).all(), name
        err = (x.grad.double().cpu() - xr.grad).abs().max().item()
        assert err <= GRAD_TOL, f"{name} max abs err {err:.3e}"


@pytest.mark.parametrize("given_h0", [False, True])
def test_mingru_module_runs_fused_and_matches_fp64(cuda, given_h0, monkeypatch):
    """The module takes the fused path on the GPU, with the learned default h0 or a
    caller's h_0; output, input and parameter gradients match the float64 eager
    module on the CPU."""
    print(f"[gpu] MinGRU module fused given_h0={given_h0}", flush=True)
    torch.manual_seed(5)
    m = MinGRU(24, 48, learnable_h0=True)
    with torch.no_grad():
        m.h0_pre.normal_()
    m_ref = copy.deepcopy(m).double()
    x = torch.randn(3, 200, 24)
    gy = torch.randn(3, 200, 48)
    h0 = torch.rand(3, 1, 48) if given_h0 else None
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    mg_ = m.to(cuda)
    xg = x.to(cuda).requires_grad_(True)
    y = mg_(xg, None if h0 is None else h0.to(cuda))
    assert "MinGRUGateScanFn" in type(y.grad_fn).__name__, "fused path did not run"
    y.backward(gy.to(cuda))
    torch.cuda.synchronize()
    monkeypatch.setenv("MINGRU_SCAN", "eager")
    xr = x.double().requires_grad_(True)
    yr = m_ref(xr, None if h0 is None else h0.double())
    yr.backward(gy.double())
    assert (y.detach().double().cpu() - yr.detach()).abs().max().item() <= FWD_TOL
    assert (xg.grad.double().cpu() - xr.grad).abs().max().item() <= GRAD_TOL
    for (name, p), (_, pr) in zip(mg_.named_parameters(), m_ref.named_parameters()):
        if pr.grad is None:  # h0_pre is unused when the caller passes h_0
            assert p.grad is None, name
            continue
        err = (p.grad.double().cpu() - pr.grad).abs().max().item()
        assert err <= GRAD_TOL, f"{name} grad max abs err {err:.3e}"


def _ref_decay(k, hp, log_h0, dt, lam):
    """The mixer's log-space coefficients with the decay term -lam dt on log(1 - z)
    (reference ``:1383-1393``), scanned in log space in float64."""
    log_coeffs = -F.softplus(k) - lam * dt.unsqueeze(-1)
    log_values = torch.cat([log_h0, -F.softplus(-k) + mg.log_g(hp)], dim=1)
    a_star = F.pad(torch.cumsum(log_coeffs, dim=1), (0, 0, 1, 0))
    log_h = a_star + torch.logcumsumexp(log_values - a_star, dim=1)
    return torch.exp(log_h)[:, 1:]


DECAY_CASES = [
    # B, T, D, input scale, per-channel rate
    (2, 777, 136, 2.0, True),
    (3, 300, 70, 1.0, False),
    (4, 1024, 256, 1.0, True),
    (2, 3000, 512, 1.0, True),
    (1, 1, 8, 1.0, True),
]


@pytest.mark.parametrize("case", DECAY_CASES)
def test_mingru_gate_scan_decay_matches_fp64(cuda, case):
    """The decay-active fused kernel against the float64 log-space reference: h and the
    gradients of k, hpre, log_h0, dt and lam."""
    B, T, D, scale, per_channel = case
    print(f"[gpu] MinGRU gate scan with decay case={case}", flush=True)
    g = torch.Generator().manual_seed(23 + T + D)
    k = torch.randn(B, T, D, generator=g) * scale
    hp = torch.randn(B, T, D, generator=g) * scale
    log_h0 = torch.rand(B, 1, D, generator=g).clamp_min(0.05).log()
    dt = torch.rand(B, T, generator=g) * 2
    dt[:, T // 2] = 0.0
    lam = (torch.rand(D, generator=g) + 0.1) if per_channel else torch.tensor(0.8)
    gh = torch.randn(B, T, D, generator=g)
    ins = [t.to(cuda).requires_grad_(True) for t in (k, hp, log_h0, dt, lam)]
    h = hip_scans.mingru_gate_scan_impl(*ins)
    assert "MinGRUGateScanFn" in type(h.grad_fn).__name__, "HIP path did not run"
    h.backward(gh.to(cuda))
    torch.cuda.synchronize()
    refs = [t.double().requires_grad_(True) for t in (k, hp, log_h0, dt, lam)]
    hr = _ref_decay(*refs)
    hr.backward(gh.double())
    assert (h.detach().double().cpu() - hr.detach()).abs().max().item() <= FWD_TOL
    for name, x, xr in zip(("dk", "dhpre", "dlog_h0", "ddt", "dlam"), ins, refs):
        sc = max(1.0, xr.grad.abs().max().item()) if name in ("ddt", "dlam") else 1.0
        err = (x.grad.double().cpu() - xr.grad).abs().max().item() / sc
        assert err <= GRAD_TOL, f"{name} max abs err {err:.3e} (scale {sc:.3g})"


@pytest.mark.parametrize("decay", ["fixed", "learnable"])
def test_mingru_decay_module_runs_fused_and_matches_fp64(cuda, decay, monkeypatch):
    """With decay the module runs the fused kernel; output, input, delta_t and parameter
    gradients match the float64 eager module."""
    print(f"[gpu] MinGRU module decay={decay}", flush=True)
    torch.manual_seed(13)
    m = MinGRU(24, 48, learnable_h0=True, decay=decay, decay_rate=0.6)
    m_ref = copy.deepcopy(m).double()
    x = torch.randn(3, 200, 24)
    dt = torch.rand(3, 200) * 3
    gy = torch.randn(3, 200, 48)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    mg_ = m.to(cuda)
    xg = x.to(cuda).requires_grad_(True)
    dtg = dt.to(cuda).requires_grad_(True)
    y = mg_(xg, delta_t=dtg)
    assert "MinGRUGateScanFn" in type(y.grad_fn).__name__, "fused path did not run"
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
    for (name, p), (_, pr) in zip(mg_.named_parameters(), m_ref.named_parameters()):
        sc = max(1.0, pr.grad.abs().max().item())
        err = (p.grad.double().cpu() - pr.grad).abs().max().item() / sc
        assert err <= GRAD_TOL, f"{name} grad max abs err {err:.3e} (scale {sc:.3g})"


@pytest.mark.parametrize("case", [(2, 777, 136, 2.0), (4, 1024, 256, 1.0), (2, 1024, 64, 1.0)])
def test_small_problem_two_launch_form(cuda, case, monkeypatch):
    """The same parity on the two-launch form (MINGRU_HIP_EW_FORM=two); by default these
    shapes run as one launch whose workgroups fold their predecessors' aggregates."""
    monkeypatch.setenv("MINGRU_HIP_EW_FORM", "two")
    test_mingru_gate_scan_matches_fp64(cuda, case)
