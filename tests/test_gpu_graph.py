"""HIP-graph capture: captured C-ABI launches replay correctly.

The look-back scans keep an epoch in their workspace header and bump it on the
device, so a captured launch replays with fresh slot tags and needs no clearing
between replays; the decode kernels use no workspace.  Each test captures once,
then replays several times on new data copied into the static inputs, with eager
calls of the same ops (on the default stream, with their own workspace) and
synchronisations between the replays, and checks every replay against eager.
"""

import pytest
import torch

from mingru_amd import hip_scans, linear_scan, parallel_scan_log
from mingru_amd.min_gru import _dispatch_mingru_gate_scan

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _force_hip(monkeypatch):
    monkeypatch.setenv("MINGRU_SCAN", "hip")


def _capture(fn, warm_args):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn(*warm_args)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn(*warm_args)
    return g, out


# (2, 777, 136) runs as two launches (chunk aggregates, then the fold); (2, 4225, 64) has
# 34 forward chunks per sequence and runs the look-back launch, whose epoch advances on
# the device at every replay.
@pytest.mark.parametrize("shape", [(2, 777, 136), (2, 4225, 64)], ids=["two_launch", "lookback"])
def test_linear_scan_graph_replays(cuda, shape):
    print(f"[gpu] graph: linear_scan shape={shape}", flush=True)
    gen = torch.Generator(device=cuda).manual_seed(0)
    sa = torch.empty(shape, device=cuda)
    sb = torch.empty(shape, device=cuda)
    sa.copy_(torch.tanh(torch.randn(shape, device=cuda, generator=gen)))
    sb.copy_(torch.randn(shape, device=cuda, generator=gen))
    g, (A_s, B_s) = _capture(linear_scan, (sa, sb))
    for rep in range(4):
        na = torch.tanh(2 * torch.randn(shape, device=cuda, generator=gen))
        nb = torch.randn(shape, device=cuda, generator=gen)
        sa.copy_(na)
        sb.copy_(nb)
        g.replay()
        A_e, B_e = linear_scan(na, nb)
        torch.cuda.synchronize()
        assert torch.allclose(A_s, A_e, rtol=1e-5, atol=1e-6), f"replay {rep}: A"
        assert torch.allclose(B_s, B_e, rtol=1e-5, atol=1e-5), f"replay {rep}: Bc"


def test_mingru_gate_scan_graph_replays(cuda):
    print("[gpu] graph: fused MinGRU gate scan", flush=True)
    gen = torch.Generator(device=cuda).manual_seed(1)
    B, T, D = 3, 500, 64
    sk = torch.randn(B, T, D, device=cuda, generator=gen)
    sh = torch.randn(B, T, D, device=cuda, generator=gen)
    lh0 = torch.full((B, 1, D), 0.5, device=cuda).log()

    def fn(k, hp):
        with torch.no_grad():
            return _dispatch_mingru_gate_scan(k, hp, lh0)

    g, h_s = _capture(fn, (sk, sh))
    for rep in range(4):
        nk = 2 * torch.randn(B, T, D, device=cuda, generator=gen)
        nh = torch.randn(B, T, D, device=cuda, generator=gen)
        sk.copy_(nk)
        sh.copy_(nh)
        g.replay()
        h_e = fn(nk, nh)
        torch.cuda.synchronize()
        assert torch.allclose(h_s, h_e, rtol=1e-5, atol=1e-6), f"replay {rep}"


def test_delta_step_graph_replays(cuda):
    print("[gpu] graph: DeltaMinGRU decode step", flush=True)
    gen = torch.Generator(device=cuda).manual_seed(2)
    B, nH, d = 4, 2, 64
    H = torch.randn(B, nH, d, d, device=cuda, generator=gen)
    q = torch.randn(B, nH, d, device=cuda, generator=gen)
    K = torch.nn.functional.normalize(torch.randn(B, nH, 1, d, device=cuda, generator=gen), dim=-1)
    V = torch.randn(B, nH, 1, d, device=cuda, generator=gen)
    beta = torch.rand(B, nH, 1, device=cuda, generator=gen)
    lg = -torch.rand(B, nH, device=cuda, generator=gen)

    def fn(H, q):
        with torch.no_grad():
            return hip_scans.delta_step_impl(H, q, K, V, beta, lg)

    g, (y_s, H_s) = _capture(fn, (H, q))
    for rep in range(4):
        nH_ = torch.randn(B, nH, d, d, device=cuda, generator=gen)
        nq = torch.randn(B, nH, d, device=cuda, generator=gen)
        H.copy_(nH_)
        q.copy_(nq)
        g.replay()
        y_e, H_e = fn(nH_, nq)
        torch.cuda.synchronize()
        assert torch.equal(y_s, y_e) and torch.equal(H_s, H_e), f"replay {rep}"


def test_log_scan_fwd_bwd_graph_replays(cuda):
    """Forward and backward (autograd.grad) of parallel_scan_log captured together, the
    way a launch-bound caller runs them; every replay on new data against eager."""
    print("[gpu] graph: parallel_scan_log fwd+bwd", flush=True)
    gen = torch.Generator(device=cuda).manual_seed(3)
    B, T, D = 2, 700, 96
    lc = torch.empty(B, T, D, device=cuda).requires_grad_(True)
    lv = torch.empty(B, T + 1, D, device=cuda).requires_grad_(True)
    gh = torch.empty(B, T, D, device=cuda)

    def fill():
        with torch.no_grad():
            lc.copy_(torch.nn.functional.logsigmoid(torch.randn(B, T, D, device=cuda, generator=gen)))
            lv.copy_(torch.randn(B, T + 1, D, device=cuda, generator=gen) - 1.0)
            gh.copy_(torch.randn(B, T, D, device=cuda, generator=gen))

    def fn():
        h = parallel_scan_log(lc, lv)
        return (h,) + torch.autograd.grad(h, (lc, lv), gh)

    fill()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = fn()
    for rep in range(4):
        fill()
        g.replay()
        ref = fn()
        torch.cuda.synchronize()
        for name, x, r in zip(("h", "dlc", "dlv"), out, ref):
            assert torch.allclose(x, r, rtol=1e-5, atol=1e-6), f"replay {rep}: {name}"
