"""GPU tests of the scan workspace protocol: a workspace zero-filled once is reused
by every stream-ordered scan call, each launch tagging its look-back slots with a
fresh epoch kept in the workspace header (no clearing between calls)."""

import ctypes

import numpy as np
import pytest
import torch

from mingru_amd import _native, hip_scans, linear_scan, matrix_affine_scan, parallel_scan_log
from oracle import scans as orc

pytestmark = pytest.mark.gpu

H_TICKET0, H_TICKET1, H_ERROR, H_EPOCH = 0, 1, 2, 3


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def test_epoch_advances_and_results_repeat(cuda):
    """Direct C-ABI calls on one zeroed workspace: every launch advances the epoch by one,
    the ticket counter of the next epoch is reset, no spin overflows are recorded, and the
    outputs agree on every reuse."""
    print("[gpu] workspace epochs", flush=True)
    lib = _native.load()
    g = torch.Generator().manual_seed(5)
    B, T, D = 3, 4225, 136  # 67 chunks per sequence: the look-back launch (tickets, epochs)
    a = torch.tanh(torch.randn(B, T, D, generator=g)).to(cuda)
    b = torch.randn(B, T, D, generator=g).to(cuda)
    nbytes = lib.mg_linear_scan_workspace_bytes(B, T, D)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=cuda)
    A, Bc = torch.empty_like(a), torch.empty_like(a)
    first = None
    for i in range(1, 41):
        rc = lib.mg_linear_scan_fwd(_p(a), _p(b), _p(A), _p(Bc), B, T, D, _p(ws), nbytes, _stream())
        assert rc == 0
        torch.cuda.synchronize()
        hdr = ws[:16].view(torch.int32).cpu().numpy()
        assert hdr[H_EPOCH] == i
        assert hdr[H_TICKET0 + ((i + 1) & 1)] == 0  # counter of the next epoch is ready
        assert hdr[H_ERROR] == 0
        # The decoupled look-back composes whatever its predecessors have published
        # when it looks, so the association of the carry (not its value) can vary
        # between launches: results agree to rounding, not bitwise.
        if first is None:
            first = (A.clone(), Bc.clone())
        else:
            assert torch.allclose(A, first[0], rtol=1e-5, atol=1e-6)
            assert torch.allclose(Bc, first[1], rtol=1e-5, atol=1e-5)
    rA, rB = orc.linear_scan(a.double().cpu().numpy(), b.double().cpu().numpy())
    assert np.max(np.abs(A.double().cpu().numpy() - rA)) <= 1e-4
    assert np.max(np.abs(Bc.double().cpu().numpy() - rB)) <= 1e-4


def test_mixed_ops_and_sizes_share_one_workspace(cuda, monkeypatch):
    """Interleaved linear / log / affine calls of different sizes through the public ops
    (one cached workspace per stream) all match the oracle."""
    print("[gpu] workspace shared across ops and sizes", flush=True)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    g = torch.Generator().manual_seed(17)
    for rep in range(3):
        for (B, T, D) in [(2, 4097, 512), (1, 33, 8), (4, 1000, 260)]:
            a = torch.tanh(torch.randn(B, T, D, generator=g))
            b = torch.randn(B, T, D, generator=g)
            A, Bc = linear_scan(a.to(cuda), b.to(cuda))
            rA, rB = orc.linear_scan(a.double().numpy(), b.double().numpy())
            assert np.max(np.abs(A.double().cpu().numpy() - rA)) <= 1e-4
            assert np.max(np.abs(Bc.double().cpu().numpy() - rB)) <= 1e-4
            lc = -torch.nn.functional.softplus(torch.randn(B, T, D, generator=g))
            lv = 0.1 * torch.randn(B, T + 1, D, generator=g)
            h = parallel_scan_log(lc.to(cuda), lv.to(cuda))
            rh = orc.parallel_scan_log(lc.double().numpy(), lv.double().numpy())
            assert np.max(np.abs(h.double().cpu().numpy() - rh)) <= 1e-4
        Am = 0.9 * torch.linalg.qr(torch.randn(2, 300, 70, 2, 2, generator=g))[0]
        Bm = torch.randn(2, 300, 70, 2, 1, generator=g)
        Abar, Bbar = matrix_affine_scan(Am.to(cuda), Bm.to(cuda))
        rAb, rBb = orc.affine_scan(Am.double().numpy(), Bm.double().numpy())
        assert np.max(np.abs(Abar.double().cpu().numpy() - rAb)) <= 1e-4
        assert np.max(np.abs(Bbar.double().cpu().numpy() - rBb)) <= 1e-4


def test_side_stream_gets_its_own_workspace(cuda, monkeypatch):
    print("[gpu] workspace per stream", flush=True)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    g = torch.Generator().manual_seed(23)
    a = torch.tanh(torch.randn(2, 513, 64, generator=g)).to(cuda)
    b = torch.randn(2, 513, 64, generator=g).to(cuda)
    A0, B0 = linear_scan(a, b)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        A1, B1 = linear_scan(a, b)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.allclose(A0, A1, rtol=1e-5, atol=1e-6)
    assert torch.allclose(B0, B1, rtol=1e-5, atol=1e-5)
    keys = [k for k in hip_scans._scan_ws if k[0] == cuda.index]
    assert (cuda.index, side.cuda_stream) in keys
    assert (cuda.index, torch.cuda.current_stream().cuda_stream) in keys


def test_broken_workspace_is_reported_not_silent(cuda, monkeypatch):
    """A workspace whose ticket counter already lies past the grid (as after a protocol
    violation) makes every workgroup record an error and retire at once -- no wait, no
    fault -- and the error is visible through mg_scan_workspace_errors and, under
    MINGRU_HIP_CHECK=1, as a LookbackError.  The workspace is private to this test."""
    print("[gpu] broken workspace reporting", flush=True)
    lib = _native.load()
    B, T, D = 2, 4225, 64  # 67 chunks per sequence: the look-back launch, which takes tickets
    a = torch.rand(B, T, D, device=cuda)
    b = torch.randn(B, T, D, device=cuda)
    nbytes = lib.mg_linear_scan_workspace_bytes(B, T, D)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=cuda)
    # A zeroed workspace's first launch runs epoch 1, whose tickets come from counter 1.
    ws[:16].view(torch.int32)[H_TICKET1] = 1 << 30
    A, Bc = torch.empty_like(a), torch.empty_like(a)
    rc = lib.mg_linear_scan_fwd(_p(a), _p(b), _p(A), _p(Bc), B, T, D, _p(ws), nbytes, _stream())
    assert rc == 0
    torch.cuda.synchronize()
    hdr = ws[:16].view(torch.int32).cpu().numpy()
    assert hdr[H_ERROR] > 0
    assert hdr[H_EPOCH] == 0  # no workgroup held the last ticket
    cnt = ctypes.c_uint(0)
    assert lib.mg_scan_workspace_errors(_p(ws), ctypes.byref(cnt), _stream()) == 0
    assert cnt.value == hdr[H_ERROR]
    monkeypatch.setenv("MINGRU_HIP_CHECK", "1")
    with pytest.raises(hip_scans.LookbackError):
        hip_scans._check_workspace(ws, a)
    monkeypatch.setenv("MINGRU_HIP_CHECK", "0")
    hip_scans._check_workspace(ws, a)  # check mode off: nothing is read


def test_check_mode_passes_on_healthy_workspaces(cuda, monkeypatch):
    """MINGRU_HIP_CHECK=1 through the public ops: every call synchronises, reads its
    workspace's error count (zero) and returns the same results."""
    print("[gpu] check mode on healthy workspaces", flush=True)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    monkeypatch.setenv("MINGRU_HIP_CHECK", "1")
    g = torch.Generator().manual_seed(29)
    a = torch.tanh(torch.randn(2, 700, 96, generator=g)).to(cuda).requires_grad_()
    b = torch.randn(2, 700, 96, generator=g).to(cuda).requires_grad_()
    A, Bc = linear_scan(a, b)
    (A.sum() + Bc.sum()).backward()
    lc = -torch.nn.functional.softplus(torch.randn(2, 700, 96, generator=g)).to(cuda)
    lv = torch.randn(2, 701, 96, generator=g).to(cuda)
    h = parallel_scan_log(lc.requires_grad_(), lv.requires_grad_())
    h.sum().backward()
    torch.cuda.synchronize()
    assert hip_scans.workspace_errors() == 0
    rA, rB = orc.linear_scan(a.detach().double().cpu().numpy(), b.detach().double().cpu().numpy())
    assert np.max(np.abs(Bc.detach().double().cpu().numpy() - rB)) <= 1e-4
