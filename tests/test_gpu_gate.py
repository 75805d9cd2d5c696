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


def test_signed_mingru_with_decay_keeps_the_unfused_scan(cuda, monkeypatch):
    """Decay multiplies a by gamma(dt): the module computes the coefficients eagerly
    and runs the HIP linear_scan instead of the fused kernel."""
    print("[gpu] SignedMinGRU decay path", flush=True)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    torch.manual_seed(3)
    m = SignedMinGRU(8, 16, decay="fixed").to(cuda)
    x = torch.randn(2, 50, 8, device=cuda)
    dt = torch.rand(2, 50, device=cuda)
    y = m(x, delta_t=dt)
    assert "SignedGateScanFn" not in type(y.grad_fn).__name__
    assert torch.isfinite(y).all()


@pytest.mark.parametrize("case", [(2, 777, 136, False), (4, 1024, 256, True), (2, 1024, 64, False)])
def test_small_problem_two_launch_form(cuda, case, monkeypatch):
    """The same parity on the two-launch form (MINGRU_HIP_EW_FORM=two); by default these
    shapes run as one launch whose workgroups fold their predecessors' aggregates."""
    monkeypatch.setenv("MINGRU_HIP_EW_FORM", "two")
    test_signed_gate_scan_matches_fp64(cuda, case)
