"""GPU parity: the streaming decode kernels (one recurrent step per call).

* The DeltaMinGRU step op is checked against the float64 gated oracle run for one
  token (``oracle.scans.delta_gated_sequential`` with T = 1, pinned on the CPU).
* The mixers' ``step()`` on the GPU (fused kernels; Rotation and Givens run the
  angle-fused scan for one token) is checked against the same
  module's float64 eager ``step()`` on the CPU, which follows the reference's step
  bodies (``src/mingru/min_gru.py:1399-1448, 3611-3688``).
* Running the fused step token by token reproduces the fused chunked forward, the
  reference's forward == step property (``tests/test_mixers.py:94, 153, 350``).
Bars: max abs err <= 1e-4 against float64 (fp32 kernels).
"""

import copy

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from mingru_amd import DeltaMinGRU, GivensMinGRU, MinGRU, RotationMinGRU, SignedMinGRU, hip_scans
from oracle import scans as orc

TOL = 1e-4

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _force_hip(monkeypatch):
    monkeypatch.setenv("MINGRU_SCAN", "hip")


@pytest.mark.parametrize("B,nH,nh,dk,dv,decay", [
    (4, 3, 1, 64, 64, True), (2, 2, 2, 24, 40, False), (5, 1, 3, 7, 5, True), (1, 4, 1, 64, 17, False),
])
def test_delta_step_op_matches_oracle(cuda, B, nH, nh, dk, dv, decay):
    print(f"[gpu] delta step op B={B} nH={nH} nh={nh} dk={dk} dv={dv} decay={decay}", flush=True)
    g = torch.Generator().manual_seed(B * 100 + dk)
    H = torch.randn(B, nH, dk, dv, generator=g)
    q = torch.randn(B, nH, dk, generator=g)
    K = F.normalize(torch.randn(B, nH, nh, dk, generator=g), dim=-1)
    V = torch.randn(B, nH, nh, dv, generator=g)
    beta = 2 * torch.sigmoid(torch.randn(B, nH, nh, generator=g))
    lg = -torch.rand(B, nH, generator=g) if decay else None
    ins = [t.to(cuda) if t is not None else None for t in (H, q, K, V, beta, lg)]
    y, Hn = hip_scans.delta_step_impl(*ins)
    torch.cuda.synchronize()
    assert torch.equal(ins[0].cpu(), H), "the input state must not be modified"
    lg0 = np.zeros((B, nH, 1)) if lg is None else lg.double().numpy()[..., None]
    ry, rH = orc.delta_gated_sequential(q.double().numpy()[:, :, None], K.double().numpy()[:, :, None],
                                        V.double().numpy()[:, :, None],
                                        beta.double().numpy()[:, :, None], lg0, H.double().numpy())
    assert np.max(np.abs(y.double().cpu().numpy() - ry[:, :, 0])) <= TOL
    assert np.max(np.abs(Hn.double().cpu().numpy() - rH)) <= TOL


def _module_cases():
    return [
        ("mingru", lambda: MinGRU(12, 40), False),
        ("mingru-decay-h0", lambda: MinGRU(12, 40, learnable_h0=True, decay="learnable"), True),
        ("signed", lambda: SignedMinGRU(12, 40), False),
        ("signed-coupled-decay", lambda: SignedMinGRU(12, 40, coupled=True, decay="fixed"), True),
        ("delta", lambda: DeltaMinGRU(12, 32, n_heads=2, nh=2), False),
        ("delta-decay", lambda: DeltaMinGRU(12, 64, n_heads=1, decay="learnable"), True),
        ("rotation", lambda: RotationMinGRU(12, 40), False),
        ("rotation-decay", lambda: RotationMinGRU(12, 40, decay="fixed"), True),
        ("givens", lambda: GivensMinGRU(12, 32, block_size=8), False),
        ("givens-decay", lambda: GivensMinGRU(12, 32, block_size=4, decay="learnable"), True),
    ]


@pytest.mark.parametrize("name,make,decay", _module_cases())
def test_module_step_fused_matches_fp64_eager(cuda, name, make, decay, monkeypatch):
    """Three steps of the fused GPU step() against the float64 eager step() on the CPU,
    state carried between steps (the first from the module's default state)."""
    print(f"[gpu] module step {name}", flush=True)
    torch.manual_seed(3)
    m = make()
    if getattr(m, "h0_pre", None) is not None:
        with torch.no_grad():
            m.h0_pre.normal_()
    m_ref = copy.deepcopy(m).double()
    mg = m.to(cuda)
    xs = torch.randn(3, 5, 12)
    dts = torch.rand(3, 5) * 2 if decay else [None] * 3
    is_delta = isinstance(m, DeltaMinGRU)
    h = hr = None
    for t in range(3):
        dt = dts[t] if decay else None
        out = mg.step(xs[t].to(cuda), h, delta_t=None if dt is None else dt.to(cuda))
        monkeypatch.setenv("MINGRU_SCAN", "eager")
        ref = m_ref.step(xs[t].double(), hr, delta_t=None if dt is None else dt.double())
        monkeypatch.setenv("MINGRU_SCAN", "hip")
        if is_delta:
            (y, h), (yr, hr) = out, ref
            assert (y.double().cpu() - yr).abs().max().item() <= TOL
        else:
            h, hr = out, ref
        assert (h.double().cpu() - hr).abs().max().item() <= TOL


@pytest.mark.parametrize("make", [lambda: MinGRU(8, 24), lambda: SignedMinGRU(8, 24, coupled=True),
                                  lambda: DeltaMinGRU(8, 32, n_heads=2, nh=2, chunk_size=8),
                                  lambda: RotationMinGRU(8, 24),
                                  lambda: GivensMinGRU(8, 24, block_size=8)])
def test_fused_step_loop_reproduces_fused_forward(cuda, make):
    """forward == step: the fused step run over T tokens gives the fused forward's outputs."""
    torch.manual_seed(9)
    m = make().to(cuda)
    print(f"[gpu] step loop vs forward {type(m).__name__}", flush=True)
    x = torch.randn(2, 40, 8, device=cuda)
    with torch.no_grad():
        y_fwd = m(x)
        h, ys = None, []
        for t in range(x.shape[1]):
            out = m.step(x[:, t], h)
            if isinstance(m, DeltaMinGRU):
                y, h = out
                ys.append(y)
            else:
                h = out
                ys.append(h)
    assert (torch.stack(ys, 1) - y_fwd).abs().max().item() <= TOL
