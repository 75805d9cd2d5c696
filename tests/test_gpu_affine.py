"""GPU parity: HIP ``matrix_scan`` / ``matrix_affine_scan`` vs the fp64 oracle.

fp32 forward max abs err <= 1e-4, gradients <= 1e-3 against float64.
"""

import numpy as np
import pytest
import torch

from mingru_amd import matrix_affine_scan, matrix_scan
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


def _contractive(B, T, n, k, g):
    """Random k x k transitions scaled to spectral norm < 1."""
    A = torch.randn(B, T, n, k, k, generator=g)
    A = A / torch.linalg.matrix_norm(A, ord=2)[..., None, None] * torch.rand(B, T, n, 1, 1, generator=g)
    return A


CASES = [
    (2, 1, 1, 2, 1),
    (2, 13, 3, 2, 1),
    (2, 100, 64, 2, 1),
    (3, 257, 130, 2, 1),
    (2, 77, 65, 1, 1),
    (2, 50, 33, 2, 2),
    (2, 40, 20, 2, 16),
    (2, 60, 70, 4, 1),
    (2, 33, 17, 4, 4),
    (2, 45, 66, 8, 1),
    (1, 19, 9, 8, 16),
    (1, 1000, 64, 1, 4),
    # 2x2 blocks with re-read offsets, several chunks (look-back)
    (2, 300, 70, 2, 4),
    (2, 300, 70, 2, 8),
    # 8x8 and 16x16 blocks on the matrix cores: odd plane counts (a half-empty
    # 16x16 block for k = 8), single steps, ragged and multi-chunk lengths
    (2, 300, 5, 8, 4),
    (1, 1000, 4, 8, 2),
    (2, 1, 1, 16, 4),
    (2, 100, 3, 16, 1),
    (1, 257, 2, 16, 16),
    (3, 70, 7, 16, 8),
    (1, 130, 1, 16, 2),
]


@pytest.mark.parametrize("case", CASES)
def test_matrix_affine_scan_matches_oracle(cuda, case):
    B, T, n, k, v = case
    print(f"[gpu] matrix_affine_scan case={case}", flush=True)
    g = torch.Generator().manual_seed(11 * T + 7 * n + k + v)
    A = _contractive(B, T, n, k, g)
    Bm = torch.randn(B, T, n, k, v, generator=g)
    gA = torch.randn(B, T, n, k, k, generator=g)
    gB = torch.randn(B, T, n, k, v, generator=g)
    Ag = A.to(cuda).requires_grad_(True)
    Bg = Bm.to(cuda).requires_grad_(True)
    Abar, Bbar = matrix_affine_scan(Ag, Bg)
    assert "AffineScanFn" in type(Abar.grad_fn).__name__
    torch.autograd.backward([Abar, Bbar], [gA.to(cuda), gB.to(cuda)])
    torch.cuda.synchronize()
    rA, rB = orc.affine_scan(A.numpy(), Bm.numpy())
    rdA, rdB = orc.affine_scan_bwd(A.numpy(), Bm.numpy(), gA.numpy(), gB.numpy())
    assert _maxerr(Abar, rA) <= FWD_TOL
    assert _maxerr(Bbar, rB) <= FWD_TOL
    assert _maxerr(Ag.grad, rdA) <= GRAD_TOL
    assert _maxerr(Bg.grad, rdB) <= GRAD_TOL


def test_matrix_scan_public_op(cuda):
    g = torch.Generator().manual_seed(5)
    M = _contractive(2, 300, 40, 2, g)
    b = torch.randn(2, 300, 40, 2, generator=g)
    A, Bc = matrix_scan(M.to(cuda), b.to(cuda))
    rA, rB = orc.affine_scan(M.numpy(), b.unsqueeze(-1).numpy())
    assert A.shape == (2, 300, 40, 2, 2) and Bc.shape == (2, 300, 40, 2)
    assert _maxerr(A, rA) <= FWD_TOL
    assert _maxerr(Bc, rB[..., 0]) <= FWD_TOL


def test_matrix_affine_scan_c3_full_size(cuda):
    print("[gpu] matrix_affine_scan C3 full size", flush=True)
    inp = wl.c3_inputs(**wl.C3)
    A, Bm, gA, gB = inp["A"], inp["Bm"], inp["grad_Abar"], inp["grad_Bbar"]
    Ag = A.to(cuda).requires_grad_(True)
    Bg = Bm.to(cuda).requires_grad_(True)
    Abar, Bbar = matrix_affine_scan(Ag, Bg)
    torch.autograd.backward([Abar, Bbar], [gA.to(cuda), gB.to(cuda)])
    torch.cuda.synchronize()
    for r in (0, wl.C3["B"] - 1):
        sl = slice(r, r + 1)
        rA, rB = orc.affine_scan(A[sl].numpy(), Bm[sl].numpy())
        rdA, rdB = orc.affine_scan_bwd(A[sl].numpy(), Bm[sl].numpy(), gA[sl].numpy(),
                                       gB[sl].numpy())
        assert _maxerr(Abar[sl], rA) <= FWD_TOL
        assert _maxerr(Bbar[sl], rB) <= FWD_TOL
        assert _maxerr(Ag.grad[sl], rdA) <= GRAD_TOL
        assert _maxerr(Bg.grad[sl], rdB) <= GRAD_TOL


def test_identity_transitions_give_cumsum(cuda):
    B, T, n = 2, 2000, 64
    Bm = torch.randn(B, T, n, 2, 1, generator=torch.Generator().manual_seed(1))
    A = torch.eye(2).expand(B, T, n, 2, 2).contiguous()
    Abar, Bbar = matrix_affine_scan(A.to(cuda), Bm.to(cuda))
    assert torch.equal(Abar.cpu(), A)
    assert _maxerr(Bbar, np.cumsum(Bm.double().numpy(), axis=1)) <= 1e-3


def test_identity_transitions_long_sequence_exact(cuda):
    """T = 2**20 with identity transitions and integer B in [-2, 2]: Abar = I and
    Bbar = cumsum(B) exactly (integer partial sums below 2**21 are exact in fp32 under any
    association), across about 8,000 look-back chunks along T."""
    B, T, n = 1, 1 << 20, 16
    print(f"[gpu] matrix_affine_scan long sequence T={T}", flush=True)
    gen = torch.Generator(device=cuda).manual_seed(14)
    Bm = torch.randint(-2, 3, (B, T, n, 2, 1), device=cuda, generator=gen).float()
    A = torch.eye(2, device=cuda).expand(B, T, n, 2, 2).contiguous()
    Abar, Bbar = matrix_affine_scan(A, Bm)
    torch.cuda.synchronize()
    assert torch.equal(Abar, A)
    assert torch.equal(Bbar.double(), Bm.double().cumsum(1))


@pytest.mark.parametrize("case", [(1, 257, 2, 16, 16), (2, 300, 5, 8, 4)])
def test_matrix_affine_scan_mfma_repeatable(cuda, case):
    """Matrix-core blocks: five runs of one multi-chunk case agree to rounding in
    outputs and gradients (the look-back consumes a predecessor's map only once the
    whole wave sees it published, so no lane mixes in a stale part of it; a stale
    mix showed up as errors of order 1).  Not bitwise: which predecessors have
    published their inclusive maps when a chunk looks back decides the association."""
    B, T, n, k, v = case
    print(f"[gpu] matrix_affine_scan repeatable case={case}", flush=True)
    g = torch.Generator().manual_seed(3)
    A = _contractive(B, T, n, k, g).to(cuda)
    Bm = torch.randn(B, T, n, k, v, generator=g).to(cuda)
    gA = torch.randn(B, T, n, k, k, generator=g).to(cuda)
    gB = torch.randn(B, T, n, k, v, generator=g).to(cuda)
    runs = []
    for _ in range(5):
        Ag = A.clone().requires_grad_(True)
        Bg = Bm.clone().requires_grad_(True)
        Abar, Bbar = matrix_affine_scan(Ag, Bg)
        torch.autograd.backward([Abar, Bbar], [gA, gB])
        runs.append([Abar.detach(), Bbar.detach(), Ag.grad, Bg.grad])
    torch.cuda.synchronize()
    for r in runs[1:]:
        for x, y in zip(r, runs[0]):
            scale = max(1.0, y.abs().max().item())
            assert (x - y).abs().max().item() <= 1e-5 * scale
    rdA, _ = orc.affine_scan_bwd(A.cpu().numpy(), Bm.cpu().numpy(), gA.cpu().numpy(),
                                 gB.cpu().numpy())
    assert _maxerr(runs[0][2], rdA) <= GRAD_TOL
