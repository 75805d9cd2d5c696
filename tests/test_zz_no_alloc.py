"""The allocation-free linear_scan forward (``mg_linear_scan_fwd_noalloc``) against the
existing entry point (``mg_linear_scan_fwd`` with a caller workspace), through the C ABI.

The entry point keeps its look-back workspace in a static device array of the library
(``MG_NOALLOC_SCRATCH_BYTES`` per GPU), so it must give the same results as the
workspace entry point on consecutive calls of different sizes, and reject a problem
whose workspace would not fit before touching the device.  After every call the array's
look-back error word (``mg_linear_scan_noalloc_errors``) must read 0: a wait that gave
up would have left a partial carry."""

import ctypes
import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest
import torch

from mingru_amd import _native
from oracle import scans as orc

pytestmark = pytest.mark.gpu

FWD_TOL = 1e-4  # fp32 forward bar against the float64 oracle
MG_ERR_TOO_LARGE = 4
MG_ERR_CAPTURE = 6
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _noalloc_errors(lib):
    n = ctypes.c_uint(123)
    assert lib.mg_linear_scan_noalloc_errors(ctypes.byref(n), _stream()) == 0
    return n.value


def _inputs(B, T, D, seed, cuda):
    g = torch.Generator().manual_seed(seed)
    a = torch.tanh(2 * torch.randn(B, T, D, generator=g))
    b = torch.randn(B, T, D, generator=g)
    return a.to(cuda), b.to(cuda)


def test_noalloc_matches_workspace_entry_point(cuda):
    lib = _native.load()
    # Two calls in a row, the second smaller (and with a narrower lane width).
    for (B, T, D), seed in (((4, 3000, 512), 1), ((2, 777, 96), 2)):
        print(f"[gpu] mg_linear_scan_fwd_noalloc B={B} T={T} D={D}", flush=True)
        a, b = _inputs(B, T, D, seed, cuda)
        A0, B0 = torch.empty_like(a), torch.empty_like(a)
        A1, B1 = torch.full_like(a, float("nan")), torch.full_like(a, float("nan"))
        nbytes = lib.mg_linear_scan_workspace_bytes(B, T, D)
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=cuda)
        assert lib.mg_linear_scan_fwd(_p(a), _p(b), _p(A0), _p(B0), B, T, D, _p(ws), nbytes,
                                      _stream()) == 0
        assert lib.mg_linear_scan_fwd_noalloc(_p(a), _p(b), _p(A1), _p(B1), B, T, D,
                                              _stream()) == 0
        torch.cuda.synchronize()
        assert _noalloc_errors(lib) == 0, "a look-back wait of the static array gave up"
        assert torch.isfinite(A1).all() and torch.isfinite(B1).all()
        assert float((A1 - A0).abs().max()) <= FWD_TOL
        assert float((B1 - B0).abs().max()) <= FWD_TOL
        rA, rB = orc.linear_scan(a[:1].double().cpu().numpy(), b[:1].double().cpu().numpy())
        assert np.max(np.abs(A1[:1].double().cpu().numpy() - rA)) <= FWD_TOL
        assert np.max(np.abs(B1[:1].double().cpu().numpy() - rB)) <= FWD_TOL


def test_noalloc_accepts_the_headline_shape(cuda):
    """The headline linear_scan shape (B=16, T=4096, D=1024: 2^26 elements) fits the static
    array and gives the workspace entry point's results."""
    B, T, D = 16, 4096, 1024
    print(f"[gpu] mg_linear_scan_fwd_noalloc B={B} T={T} D={D}", flush=True)
    lib = _native.load()
    g = torch.Generator(device=cuda).manual_seed(3)
    a = torch.tanh(2 * torch.randn(B, T, D, generator=g, device=cuda))
    b = torch.randn(B, T, D, generator=g, device=cuda)
    A0, B0 = torch.empty_like(a), torch.empty_like(a)
    A1, B1 = torch.full_like(a, float("nan")), torch.full_like(a, float("nan"))
    nbytes = lib.mg_linear_scan_workspace_bytes(B, T, D)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=cuda)
    assert lib.mg_linear_scan_fwd(_p(a), _p(b), _p(A0), _p(B0), B, T, D, _p(ws), nbytes,
                                  _stream()) == 0
    assert lib.mg_linear_scan_fwd_noalloc(_p(a), _p(b), _p(A1), _p(B1), B, T, D,
                                          _stream()) == 0
    torch.cuda.synchronize()
    assert _noalloc_errors(lib) == 0, "a look-back wait of the static array gave up"
    assert float((A1 - A0).abs().max()) <= FWD_TOL
    assert float((B1 - B0).abs().max()) <= FWD_TOL


def test_noalloc_rejects_problems_beyond_the_scratch(cuda):
    """B*T*D = 2^28 needs more look-back slots than the static array holds: status 4,
    nothing launched (the pointers are never dereferenced)."""
    print("[gpu] mg_linear_scan_fwd_noalloc size limit", flush=True)
    lib = _native.load()
    x = torch.zeros(16, device=cuda)
    rc = lib.mg_linear_scan_fwd_noalloc(_p(x), _p(x), _p(x), _p(x), 64, 4096, 1024, _stream())
    assert rc == MG_ERR_TOO_LARGE
    assert lib.mg_linear_scan_fwd_noalloc(None, _p(x), _p(x), _p(x), 1, 4, 4, _stream()) == 1


_CAPTURE_SCRIPT = textwrap.dedent("""
    import ctypes, sys
    import torch
    sys.path.insert(0, sys.argv[1])
    from mingru_amd import _native
    lib = _native.load()
    dev = torch.device("cuda:0")
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    B, T, D = 2, 4225, 64   # 34 forward chunks per sequence: the look-back launch
    gen = torch.Generator(device=dev).manual_seed(5)
    sa = torch.tanh(torch.randn(B, T, D, device=dev, generator=gen))
    sb = torch.randn(B, T, D, device=dev, generator=gen)
    A, Bc = torch.empty_like(sa), torch.empty_like(sa)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        rc_first = lib.mg_linear_scan_fwd_noalloc(p(sa), p(sb), p(A), p(Bc), B, T, D,
                                                  ctypes.c_void_p(s.cuda_stream))
    print("first call under capture:", rc_first, flush=True)
    assert rc_first == 6, rc_first
    # the set-up runs eagerly, then a captured call replays on new data
    cur = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.mg_linear_scan_fwd_noalloc(p(sa), p(sb), p(A), p(Bc), B, T, D, cur) == 0
    torch.cuda.synchronize()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        rc = lib.mg_linear_scan_fwd_noalloc(p(sa), p(sb), p(A), p(Bc), B, T, D,
                                            ctypes.c_void_p(s.cuda_stream))
    assert rc == 0, rc
    nbytes = lib.mg_linear_scan_workspace_bytes(B, T, D)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    A0, B0 = torch.empty_like(sa), torch.empty_like(sa)
    for rep in range(3):
        sa.copy_(torch.tanh(2 * torch.randn(B, T, D, device=dev, generator=gen)))
        sb.copy_(torch.randn(B, T, D, device=dev, generator=gen))
        g.replay()
        assert lib.mg_linear_scan_fwd(p(sa), p(sb), p(A0), p(B0), B, T, D, p(ws), nbytes,
                                      cur) == 0
        torch.cuda.synchronize()
        n = ctypes.c_uint(7)
        assert lib.mg_linear_scan_noalloc_errors(ctypes.byref(n), cur) == 0
        assert n.value == 0, n.value
        ea, eb = float((A - A0).abs().max()), float((Bc - B0).abs().max())
        print(f"replay {rep}: max |A| err {ea:.2e}, max |Bc| err {eb:.2e}", flush=True)
        assert ea <= 1e-4 and eb <= 1e-4
    print("capture ok", flush=True)
""")


def test_noalloc_first_call_under_capture_is_refused(cuda):
    """In a fresh process, a first call made under stream capture returns status 6 and
    records nothing; after an eager first call, a captured call replays correctly on new
    data (three replays against the workspace entry point, error word 0 each time)."""
    print("[gpu] mg_linear_scan_fwd_noalloc first call under capture (subprocess)", flush=True)
    res = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT, ROOT], capture_output=True,
                         text=True, timeout=300)
    print(res.stdout, res.stderr[-2000:], flush=True)
    assert res.returncode == 0
    assert "capture ok" in res.stdout
