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


def test_mingru_with_decay_keeps_the_unfused_scan(cuda, monkeypatch):
    """Decay adds -lambda dt to log(1 - z): the module computes the log coefficients
    eagerly and runs the HIP parallel_scan_log instead of the fused kernel."""
    print("[gpu] MinGRU decay path", flush=True)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    torch.manual_seed(3)
    m = MinGRU(8, 16, decay="fixed").to(cuda)
    x = torch.randn(2, 50, 8, device=cuda)
    dt = torch.rand(2, 50, device=cuda)
    y = m(x, delta_t=dt)
    assert "MinGRUGateScanFn" not in type(y.grad_fn).__name__
    assert torch.isfinite(y).all()


@pytest.mark.parametrize("case", [(2, 777, 136, 2.0), (4, 1024, 256, 1.0), (2, 1024, 64, 1.0)])
def test_small_problem_two_launch_form(cuda, case, monkeypatch):
    """The same parity on the two-launch form (MINGRU_HIP_EW_FORM=two); by default these
    shapes run as one launch whose workgroups fold their predecessors' aggregates."""
    monkeypatch.setenv("MINGRU_HIP_EW_FORM", "two")
    test_mingru_gate_scan_matches_fp64(cuda, case)
