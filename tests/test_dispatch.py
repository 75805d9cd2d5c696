"""CPU-only contract tests for the ``MINGRU_SCAN`` seam and the HIP backend's
envelope (reference behaviour: ``src/mingru/min_gru.py:85-668``,
``src/mingru/triton_scans.py:166-177, 335-452``; the reference's own seam
tests are ``tests/test_dispatch.py``).

No GPU is touched: a stand-in object reports ``is_cuda = True`` to reach the
GPU branches, the real backend then declines because no device is visible,
and a fake backend module injected into ``sys.modules`` pins the value-level
layout round trip of the DeltaMinGRU seam.
"""

import subprocess
import sys
import types
import warnings

import pytest
import torch
import torch.nn.functional as F

import mingru_amd
from mingru_amd import DeltaMinGRU, GivensMinGRU, MinGRU, SignedMinGRU, hip_scans, linear_scan
from mingru_amd import min_gru as mg

BACKEND = "mingru_amd.hip_scans"


class _FakeCudaTensor:
    """Reports GPU residency; the seam reads only ``.is_cuda`` before the backend declines."""

    is_cuda = True


@pytest.fixture(autouse=True)
def _isolate(monkeypatch):
    monkeypatch.delenv("MINGRU_SCAN", raising=False)
    for flag in ("_warned_scan_fallback", "_warned_angle_fallback", "_warned_delta_fallback",
                 "_warned_delta_decay_fallback", "_warned_gate_fallback",
                 "_warned_mingru_gate_fallback", "_warned_step_fallback"):
        monkeypatch.setattr(mg, flag, False)


def _fresh_python(code: str) -> str:
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                         timeout=300, cwd=mingru_amd.__path__[0] + "/..")
    assert out.returncode == 0, out.stderr
    return out.stdout.strip()


# ---------------------------------------------------------------- modes


def test_invalid_mode_raises_value_error(monkeypatch):
    monkeypatch.setenv("MINGRU_SCAN", "cuda")
    a = torch.rand(1, 3, 2)
    with pytest.raises(ValueError, match="MINGRU_SCAN"):
        linear_scan(a, a)


@pytest.mark.parametrize("mode", [None, "auto", "eager"])
def test_cpu_paths_stay_eager_without_warning(monkeypatch, mode):
    if mode:
        monkeypatch.setenv("MINGRU_SCAN", mode)
    a, b = torch.rand(2, 9, 3), torch.randn(2, 9, 3)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        A, Bc = linear_scan(a, b)
    assert A.grad_fn is None or "LinearScanFn" not in type(A.grad_fn).__name__


@pytest.mark.parametrize("mode", ["auto", "eager"])
def test_cpu_never_imports_backend(mode):
    """``import mingru_amd`` and CPU scans under auto/eager never load the backend."""
    code = (
        "import os, sys; os.environ['MINGRU_SCAN'] = %r\n"
        "import torch, mingru_amd\n"
        "a = torch.rand(1, 5, 4)\n"
        "mingru_amd.linear_scan(a, a); mingru_amd.parallel_scan_log(a.log(), torch.zeros(1, 6, 4))\n"
        "m = mingru_amd.DeltaMinGRU(4, 8, n_heads=2, chunk_size=2); m(torch.randn(1, 9, 4))\n"
        "print(%r in sys.modules)" % (mode, BACKEND)
    )
    assert _fresh_python(code) == "False"


def test_lazy_backend_names_resolve():
    code = (
        "import sys, mingru_amd\n"
        "before = %r in sys.modules\n"
        "fb = mingru_amd.ScanFallback\n"
        "print(before, %r in sys.modules, fb.__name__, callable(mingru_amd.delta_scan_impl))"
        % (BACKEND, BACKEND)
    )
    assert _fresh_python(code) == "False True ScanFallback True"


@pytest.mark.parametrize("mode", ["hip", "triton"])
def test_forcing_mode_raises_with_reason(monkeypatch, mode):
    monkeypatch.setenv("MINGRU_SCAN", mode)
    with pytest.raises(RuntimeError, match="device not available"):
        mg._dispatch_scan("linear_scan", _FakeCudaTensor(), _FakeCudaTensor())


def test_auto_gpu_fallback_warns_once_and_returns_none(monkeypatch):
    monkeypatch.setenv("MINGRU_SCAN", "auto")
    with pytest.warns(UserWarning, match="fell back to the eager scan"):
        assert mg._dispatch_scan("linear_scan", _FakeCudaTensor(), _FakeCudaTensor()) is None
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        assert mg._dispatch_scan("matrix_scan", _FakeCudaTensor(), _FakeCudaTensor()) is None


def test_angle_and_delta_fallbacks_warn_independently(monkeypatch):
    monkeypatch.setenv("MINGRU_SCAN", "auto")
    f = _FakeCudaTensor()
    with pytest.warns(UserWarning, match="angle-fused"):
        assert mg._dispatch_angle_scan(f, f, f, f, f, f, f, f, has_scale=0, has_decay=0) is None
    with pytest.warns(UserWarning, match="DeltaMinGRU"):
        assert mg._dispatch_delta_scan(f, [], [], [], f, chunk_size=4) is None
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        assert mg._dispatch_delta_scan(f, [], [], [], f, chunk_size=4) is None


def test_delta_auto_region_gate(monkeypatch):
    monkeypatch.setenv("MINGRU_SCAN", "auto")
    assert mg._delta_scan_should_try(True, T=128, chunk_size=64, d_k=64)
    assert not mg._delta_scan_should_try(True, T=100, chunk_size=64, d_k=64)
    assert not mg._delta_scan_should_try(True, T=4096, chunk_size=64, d_k=128)
    assert not mg._delta_scan_should_try(False, T=4096, chunk_size=64, d_k=64)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    assert mg._delta_scan_should_try(True, T=3, chunk_size=64, d_k=128)
    monkeypatch.setenv("MINGRU_SCAN", "eager")
    assert not mg._delta_scan_should_try(True, T=4096, chunk_size=64, d_k=64)


def test_delta_decay_seam_keeps_the_reference_guard_contract(monkeypatch):
    """A backend without the gated kernel declines: the forcing mode raises, CUDA
    ``auto`` warns once and runs eager, CPU ``auto`` stays silent (reference
    ``_delta_decay_dispatch_guard``, ``src/mingru/min_gru.py:612-668``)."""
    _fake_backend(monkeypatch)
    f = _FakeCudaTensor()
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    with pytest.raises(RuntimeError, match="decay"):
        mg._dispatch_delta_gated_scan(f, [f], [f], [f], f, f, chunk_size=4)
    monkeypatch.setenv("MINGRU_SCAN", "auto")
    with pytest.warns(UserWarning, match="decay"):
        assert mg._dispatch_delta_gated_scan(f, [f], [f], [f], f, f, chunk_size=4) is None
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        assert mg._dispatch_delta_gated_scan(f, [f], [f], [f], f, f, chunk_size=4) is None
        c = torch.zeros(1)
        assert mg._dispatch_delta_gated_scan(c, [c], [c], [c], c, c, chunk_size=4) is None


def test_delta_decay_seam_hands_gated_layouts_to_backend(monkeypatch):
    """DeltaMinGRU with decay passes the kernel layouts plus log_gamma = -lambda dt
    (B, n_heads, T) to ``delta_gated_scan_impl`` and maps its y back through out_proj."""
    seen = {}

    def fake_gated(Q, K, V, beta, log_gamma, H0, *, chunk_size):
        seen.update(Q=tuple(Q.shape), K=tuple(K.shape), V=tuple(V.shape),
                    beta=tuple(beta.shape), lg=log_gamma.detach().clone(), H0=tuple(H0.shape),
                    chunk=chunk_size)
        return torch.zeros(Q.shape[:3] + (V.shape[-1],)), H0 + 1.0

    _fake_backend(monkeypatch, delta_gated_scan_impl=fake_gated)
    m = DeltaMinGRU(6, 12, n_heads=3, nh=2, chunk_size=5, decay="fixed", decay_rate=0.7)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    x = torch.randn(2, 9, 6)
    dt = torch.rand(2, 9)
    y, HT = m(x, delta_t=dt, return_state=True)
    assert seen["Q"] == (2, 3, 9, 4) and seen["K"] == (2, 3, 9, 2, 4)
    assert seen["V"] == (2, 3, 9, 2, 4) and seen["beta"] == (2, 3, 9, 2)
    assert seen["H0"] == (2, 3, 4, 4) and seen["chunk"] == 5
    lam = m._decay_lambda().reshape(1, -1, 1)  # one value under decay="fixed"
    assert seen["lg"].shape == (2, 3, 9)
    assert torch.allclose(seen["lg"], (-lam * dt.unsqueeze(1)).expand(2, 3, 9))
    with torch.no_grad():
        assert torch.allclose(y, m.out_proj(torch.zeros(2, 9, 12)))
    assert torch.equal(HT, torch.ones(2, 1, 48))


# ---------------------------------------------------------------- backend envelope


def test_backend_declines_without_gpu():
    assert hip_scans.available() is not True
    a = torch.rand(1, 4, 3)
    with pytest.raises(hip_scans.ScanFallback):
        hip_scans.SCAN_IMPLS["linear_scan"](a, a)


_OK = dict(is_cuda=True, q_dtype=torch.bfloat16, k_dtype=torch.bfloat16, v_dtype=torch.bfloat16,
           beta_dtype=torch.bfloat16, h0_dtype=torch.float32, d_k=64, d_v=64, chunk_size=64, nh=1)

_VIOLATIONS = {
    "non_gpu": dict(is_cuda=False),
    "q": dict(q_dtype=torch.float64),
    "k": dict(k_dtype=torch.int32),
    "v": dict(v_dtype=torch.float64),
    "beta": dict(beta_dtype=torch.float64),
    "h0": dict(h0_dtype=torch.float64),
    "dk": dict(d_k=65),
    "dv": dict(d_v=0),
    "chunk": dict(chunk_size=65),
    "micro": dict(nh=3, chunk_size=43),
    "nh_tile": dict(nh=65, chunk_size=1),
}


def test_delta_envelope_in_range_is_none():
    assert hip_scans._delta_envelope_reason(**_OK) is None
    assert hip_scans._delta_envelope_reason(**{**_OK, "d_k": 5, "d_v": 48, "nh": 4,
                                               "chunk_size": 16}) is None
    # the reference's micro-step bound (nh * chunk_size <= 128), e.g. nh=2 at the
    # module's default chunk_size=64
    assert hip_scans._delta_envelope_reason(**{**_OK, "nh": 2, "chunk_size": 64}) is None
    assert hip_scans._delta_envelope_reason(**{**_OK, "nh": 64, "chunk_size": 2}) is None


@pytest.mark.parametrize("nh,chunk,tile", [(1, 64, 64), (1, 7, 7), (2, 64, 32), (2, 20, 20),
                                           (3, 42, 21), (5, 25, 12), (64, 2, 1)])
def test_delta_tile_chunk(nh, chunk, tile):
    """Chunks of more than 64 micro-steps run as tiles of floor(64 / nh) tokens."""
    assert hip_scans._delta_tile_chunk(nh, chunk) == tile
    assert nh * hip_scans._delta_tile_chunk(nh, chunk) <= 64


def test_delta_envelope_reasons_are_distinct():
    reasons = {}
    for name, bad in _VIOLATIONS.items():
        r = hip_scans._delta_envelope_reason(**{**_OK, **bad})
        assert r is not None, name
        reasons[name] = r
    assert len(set(reasons.values())) == len(reasons)


def test_delta_validate_envelope_shapes():
    Q = torch.zeros(1, 2, 5, 4)
    K = torch.zeros(1, 2, 5, 1, 4)
    V = torch.zeros(1, 2, 5, 1, 3)
    b = torch.zeros(1, 2, 5, 1)
    H0 = torch.zeros(1, 2, 4, 3)
    with pytest.raises(hip_scans.ScanFallback, match="ranks"):
        hip_scans._delta_validate_envelope(Q[0], K, V, b, H0, 4)
    with pytest.raises(hip_scans.ScanFallback, match="shapes disagree"):
        hip_scans._delta_validate_envelope(Q, K, V, b, torch.zeros(1, 2, 3, 3), 4)
    with pytest.raises(hip_scans.ScanFallback, match="GPU tensors"):
        hip_scans._delta_validate_envelope(Q, K, V, b, H0, 4)


def test_angle_schedule_classifier():
    from mingru_amd import workloads as wl

    perm, sgn, p2p = wl.lexicographic_schedule(8)
    assert hip_scans._classify_schedule(perm, sgn, p2p, 8, 28, 1) == (hip_scans._SCHED_LEX, 28)
    bp, bs, bq = hip_scans._brick_tables(8, 3)
    assert hip_scans._classify_schedule(bp, bs, bq, 8, 3, 4) == (hip_scans._SCHED_BRICK, 3)
    bad = perm.clone()
    bad[0, 0], bad[0, 1] = 0, 1
    with pytest.raises(hip_scans.ScanFallback, match="schedule"):
        hip_scans._classify_schedule(bad, sgn, p2p, 8, 28, 1)


# ---------------------------------------------------------------- delta layout round trip


def test_delta_seam_layout_round_trip(monkeypatch):
    """A fake backend sees the kernel layouts and its (B, H, T, d_v) output comes back as
    (B, T, H, d_v): the whole module forward then equals the eager chunked forward."""
    seen = {}

    class FakeFallback(Exception):
        pass

    def fake_delta(Q, K, V, beta, H0, *, chunk_size):
        seen["shapes"] = (tuple(Q.shape), tuple(K.shape), tuple(V.shape), tuple(beta.shape),
                          tuple(H0.shape), chunk_size)
        y, HT = mg.delta_chunked_eager(Q, K, V, beta, H0, chunk_size)
        return y.permute(0, 2, 1, 3), HT

    fake = types.ModuleType(BACKEND)
    fake.ScanFallback = FakeFallback
    fake.available = lambda: True
    fake.SCAN_IMPLS = {}
    fake.delta_scan_impl = fake_delta
    monkeypatch.setitem(sys.modules, BACKEND, fake)
    monkeypatch.setattr(mingru_amd, "hip_scans", fake, raising=False)

    torch.manual_seed(3)
    m = DeltaMinGRU(6, 12, n_heads=3, nh=2, chunk_size=5).double()
    x = torch.randn(2, 13, 6, dtype=torch.float64)
    monkeypatch.setenv("MINGRU_SCAN", "eager")
    ref, Href = m(x, return_state=True)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    out, H = m(x, return_state=True)
    assert seen["shapes"] == ((2, 3, 13, 4), (2, 3, 13, 2, 4), (2, 3, 13, 2, 4), (2, 3, 13, 2),
                              (2, 3, 4, 4), 5)
    torch.testing.assert_close(out, ref, rtol=0, atol=1e-12)
    torch.testing.assert_close(H, Href, rtol=0, atol=1e-12)


def test_angle_seam_reaches_backend(monkeypatch):
    """GivensMinGRU's fused path hands (B, T, n, R, half) angles to the backend."""
    seen = {}

    class FakeFallback(Exception):
        pass

    def fake_angle(theta, scale, gamma, b, h0, perm, sgn, p2p, *, has_scale, has_decay):
        seen["theta"] = tuple(theta.shape)
        raise FakeFallback("declined by the fake backend")

    fake = types.ModuleType(BACKEND)
    fake.ScanFallback = FakeFallback
    fake.available = lambda: True
    fake.SCAN_IMPLS = {}
    fake.angle_scan_impl = fake_angle
    monkeypatch.setitem(sys.modules, BACKEND, fake)
    monkeypatch.setattr(mingru_amd, "hip_scans", fake, raising=False)
    m = GivensMinGRU(6, 16, block_size=8)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    with pytest.raises(RuntimeError, match="declined by the fake backend"):
        m(torch.randn(2, 7, 6))
    assert seen["theta"][:3] == (2, 7, 2)


def _fake_backend(monkeypatch, **attrs):
    class FakeFallback(Exception):
        pass

    fake = types.ModuleType(BACKEND)
    fake.ScanFallback = FakeFallback
    fake.available = lambda: True
    fake.SCAN_IMPLS = {}
    for k, v in attrs.items():
        setattr(fake, k, v)
    monkeypatch.setitem(sys.modules, BACKEND, fake)
    monkeypatch.setattr(mingru_amd, "hip_scans", fake, raising=False)
    return fake


def test_signed_gate_seam_hands_preactivations_to_backend(monkeypatch):
    """SignedMinGRU's fused path passes (s, z, hpre) pre-activations and a (B, 1, D) h0,
    and returns the backend's h unchanged."""
    seen = {}

    def fake_gate(s, z, hpre, h0, *, coupled):
        seen.update(s=tuple(s.shape), h0=tuple(h0.shape), coupled=coupled)
        return torch.full(s.shape, 7.0)

    _fake_backend(monkeypatch, signed_gate_scan_impl=fake_gate)
    m = SignedMinGRU(5, 6, coupled=True)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    y = m(torch.randn(2, 9, 5))
    assert seen == {"s": (2, 9, 6), "h0": (2, 1, 6), "coupled": True}
    assert torch.equal(y, torch.full((2, 9, 6), 7.0))


def test_signed_gate_seam_fuses_the_decay(monkeypatch):
    """With decay the fused call carries the normalised dt and the rate lambda; the
    eager coefficients and the scan seam do not run."""
    seen = {}

    def fake_gate(s, z, hpre, h0, *, coupled, dt=None, lam=None):
        seen.update(dt=dt, lam=lam, coupled=coupled)
        return torch.full(s.shape, 3.0)

    def fake_linear(a, b):
        raise AssertionError("the scan seam must not run when the fused path takes decay")

    _fake_backend(monkeypatch, signed_gate_scan_impl=fake_gate,
                  SCAN_IMPLS={"linear_scan": fake_linear})
    m = SignedMinGRU(4, 5, decay="fixed", decay_rate=0.7)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    dt = torch.rand(2, 6)
    dt[0, 1] = float("nan")
    y = m(torch.randn(2, 6, 4), delta_t=dt)
    assert torch.equal(y, torch.full((2, 6, 5), 3.0))
    assert seen["coupled"] is False
    assert torch.equal(seen["dt"], dt.nan_to_num(0.0))  # normalised by the module
    assert float(seen["lam"]) == pytest.approx(0.7)


def test_signed_gate_decay_decline_raises_in_forcing_mode(monkeypatch):
    """A declined fused call under decay raises in the forcing mode, naming the reason
    (auto would fall back to the eager coefficients and the scan seam)."""
    calls = []

    def fake_gate(*args, **kwargs):
        calls.append("gate")
        raise sys.modules[BACKEND].ScanFallback("declined by the fake backend")

    def fake_linear(a, b):
        calls.append("linear_scan")
        return torch.cumprod(a, 1), _seq_bc(a, b)

    _fake_backend(monkeypatch, signed_gate_scan_impl=fake_gate,
                  SCAN_IMPLS={"linear_scan": fake_linear})
    m = SignedMinGRU(4, 5, decay="fixed")
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    with pytest.raises(RuntimeError, match="declined by the fake backend"):
        m(torch.randn(2, 6, 4), delta_t=torch.rand(2, 6))
    assert calls == ["gate"]


def test_mingru_gate_seam_fuses_the_decay(monkeypatch):
    seen = {}

    def fake_gate(k, hpre, log_h0, dt=None, lam=None):
        seen.update(dt=dt, lam=lam)
        return torch.full(k.shape, 2.0)

    _fake_backend(monkeypatch, mingru_gate_scan_impl=fake_gate)
    m = MinGRU(4, 5, decay="learnable", decay_rate=0.5)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    dt = torch.rand(2, 6)
    y = m(torch.randn(2, 6, 4), delta_t=dt)
    assert torch.equal(y, torch.full((2, 6, 5), 2.0))
    assert torch.equal(seen["dt"], dt)
    assert seen["lam"].shape == (5,) and torch.allclose(seen["lam"], torch.full((5,), 0.5))


def _seq_bc(a, b):
    h, out = torch.zeros_like(a[:, 0]), []
    for t in range(a.shape[1]):
        h = a[:, t] * h + b[:, t]
        out.append(h)
    return torch.stack(out, 1)


def test_signed_gate_auto_fallback_warns_once_and_runs_eager(monkeypatch):
    def fake_gate(*args, **kwargs):
        raise sys.modules[BACKEND].ScanFallback("declined by the fake backend")

    _fake_backend(monkeypatch, signed_gate_scan_impl=fake_gate)
    f = _FakeCudaTensor()
    monkeypatch.setenv("MINGRU_SCAN", "auto")
    with pytest.warns(UserWarning, match="fused gate path"):
        assert mg._dispatch_signed_gate_scan(f, f, f, f, coupled=False) is None
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        assert mg._dispatch_signed_gate_scan(f, f, f, f, coupled=False) is None
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    with pytest.raises(RuntimeError, match="declined by the fake backend"):
        mg._dispatch_signed_gate_scan(f, f, f, f, coupled=False)


def test_mingru_gate_seam_hands_preactivations_to_backend(monkeypatch):
    """MinGRU's fused path passes the (k, hpre) pre-activations and log h0 = log 0.5
    (B, 1, D), and returns the backend's h unchanged."""
    seen = {}

    def fake_gate(k, hpre, log_h0):
        seen.update(k=tuple(k.shape), hpre=tuple(hpre.shape), log_h0=log_h0.clone())
        return torch.full(k.shape, 3.0)

    _fake_backend(monkeypatch, mingru_gate_scan_impl=fake_gate)
    m = MinGRU(5, 6)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    x = torch.randn(2, 9, 5)
    y = m(x)
    assert seen["k"] == seen["hpre"] == (2, 9, 6)
    assert torch.allclose(seen["log_h0"], torch.full((2, 1, 6), 0.5).log())
    assert torch.equal(y, torch.full((2, 9, 6), 3.0))


def test_mingru_gate_auto_fallback_warns_once_and_runs_eager(monkeypatch):
    def fake_gate(*args, **kwargs):
        raise sys.modules[BACKEND].ScanFallback("declined by the fake backend")

    _fake_backend(monkeypatch, mingru_gate_scan_impl=fake_gate)
    f = _FakeCudaTensor()
    monkeypatch.setenv("MINGRU_SCAN", "auto")
    with pytest.warns(UserWarning, match="MinGRU coefficients"):
        assert mg._dispatch_mingru_gate_scan(f, f, f) is None
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        assert mg._dispatch_mingru_gate_scan(f, f, f) is None
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    with pytest.raises(RuntimeError, match="declined by the fake backend"):
        mg._dispatch_mingru_gate_scan(f, f, f)


def test_mingru_linear_recurrence_equals_log_space_forward():
    """The linear recurrence the fused kernel runs, h_t = sigmoid(-k) h_{t-1} +
    sigmoid(k) g(hpre) from h_0 = exp(log h0), equals the log-space forward
    (reference ``src/mingru/min_gru.py:1366-1397``) in float64, incl. a learned h0."""
    torch.manual_seed(3)
    m = MinGRU(4, 6, learnable_h0=True).double()
    with torch.no_grad():
        m.h0_pre.normal_()
    x = torch.randn(2, 11, 4, dtype=torch.float64) * 3
    ref = m(x)
    k, hpre = m.linear_z(x), m.linear_h(x)
    h = mg.g(m.h0_pre).expand(2, 1, 6)[:, 0]
    out = []
    for t in range(x.shape[1]):
        h = torch.sigmoid(-k[:, t]) * h + torch.sigmoid(k[:, t]) * mg.g(hpre[:, t])
        out.append(h)
    assert torch.allclose(torch.stack(out, 1), ref, rtol=1e-12, atol=1e-12)


def test_delta_module_forward_equals_step_recurrence():
    """Eager chunked forward == token-by-token ``step`` (reference tests/test_mixers.py:350-363)."""
    torch.manual_seed(1)
    m = DeltaMinGRU(5, 8, n_heads=2, nh=2, chunk_size=3).double()
    x = torch.randn(2, 10, 5, dtype=torch.float64)
    y = m(x)
    h = None
    ys = []
    for t in range(10):
        yt, h = m.step(x[:, t], h)
        ys.append(yt)
    torch.testing.assert_close(y, torch.stack(ys, 1), rtol=0, atol=1e-12)
    assert F.mse_loss(y, y).item() == 0.0


# ------------------------------------------------------------ streaming decode seams


def test_mingru_step_hands_preactivations_to_gate_step(monkeypatch):
    seen = {}

    def fake_step(kind, p0, p1, p2, gamma, h_prev):
        seen.update(kind=kind, p0=tuple(p0.shape), p2=p2, gamma=gamma, hp=h_prev.clone())
        return torch.full(h_prev.shape, 2.0)

    _fake_backend(monkeypatch, gate_step_impl=fake_step)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    m = MinGRU(5, 6)
    h = m.step(torch.randn(3, 5))
    assert seen["kind"] == "mingru" and seen["p0"] == (3, 6)
    assert seen["p2"] is None and seen["gamma"] is None
    assert torch.equal(seen["hp"], torch.full((3, 6), 0.5))  # g(0) default state
    assert torch.equal(h, torch.full((3, 6), 2.0))


def test_signed_step_passes_decay_gamma_and_kind(monkeypatch):
    seen = {}

    def fake_step(kind, p0, p1, p2, gamma, h_prev):
        seen.update(kind=kind, gamma=gamma)
        return h_prev + 1

    _fake_backend(monkeypatch, gate_step_impl=fake_step)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    m = SignedMinGRU(4, 5, coupled=True, decay="fixed", decay_rate=0.3)
    dt = torch.rand(2)
    m.step(torch.randn(2, 4), torch.zeros(2, 5), delta_t=dt)
    assert seen["kind"] == "signed_coupled"
    assert torch.allclose(seen["gamma"].expand(2, 5), torch.exp(-0.3 * dt)[:, None].expand(2, 5))


def test_delta_step_hands_stacked_layouts(monkeypatch):
    seen = {}

    def fake_step(H, q, K, V, beta, log_gamma):
        seen.update(H=tuple(H.shape), q=tuple(q.shape), K=tuple(K.shape), V=tuple(V.shape),
                    beta=tuple(beta.shape), lg=None if log_gamma is None else log_gamma.clone())
        return torch.zeros(q.shape[0], q.shape[1], V.shape[-1]), H + 1

    _fake_backend(monkeypatch, delta_step_impl=fake_step)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    m = DeltaMinGRU(6, 12, n_heads=3, nh=2, decay="fixed", decay_rate=0.5)
    dt = torch.rand(2)
    y, H = m.step(torch.randn(2, 6), delta_t=dt)
    assert seen["H"] == (2, 3, 4, 4) and seen["q"] == (2, 3, 4)
    assert seen["K"] == (2, 3, 2, 4) and seen["V"] == (2, 3, 2, 4) and seen["beta"] == (2, 3, 2)
    assert torch.allclose(seen["lg"], (-0.5 * dt)[:, None].expand(2, 3))
    assert torch.equal(H, torch.ones(2, 48))
    with torch.no_grad():
        assert torch.allclose(y, m.out_proj(torch.zeros(2, 12)))


def test_step_auto_fallback_warns_once(monkeypatch):
    def fake_step(*args):
        raise sys.modules[BACKEND].ScanFallback("declined by the fake backend")

    _fake_backend(monkeypatch, gate_step_impl=fake_step)
    f = _FakeCudaTensor()
    monkeypatch.setenv("MINGRU_SCAN", "auto")
    with pytest.warns(UserWarning, match="step"):
        assert mg._dispatch_gate_step("mingru", f, f, None, None, f) is None
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        assert mg._dispatch_gate_step("mingru", f, f, None, None, f) is None
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    with pytest.raises(RuntimeError, match="declined by the fake backend"):
        mg._dispatch_gate_step("mingru", f, f, None, None, f)


def test_givens_step_runs_the_angle_scan_for_one_token(monkeypatch):
    """GivensMinGRU.step on the GPU path hands a T = 1 angle problem with h_prev as the
    carried state to the angle-fused kernel and returns its single output row."""
    seen = {}

    def fake_angle(theta, scale, gamma, b, h0, perm, sgn, p2p, *, has_scale, has_decay):
        seen.update(theta=tuple(theta.shape), h0=h0.clone(), has_decay=has_decay)
        return torch.full(b.shape, 4.0)

    _fake_backend(monkeypatch, angle_scan_impl=fake_angle)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    m = GivensMinGRU(6, 16, block_size=8, decay="fixed")
    hp = torch.randn(3, 16)
    h = m.step(torch.randn(3, 6), hp, delta_t=torch.rand(3))
    assert seen["theta"][:3] == (3, 1, 2) and seen["has_decay"] == 1
    assert torch.equal(seen["h0"], hp.reshape(3, 2, 8))
    assert torch.equal(h, torch.full((3, 16), 4.0))


# ---------------------------------------------------------------- angle plane tables


def _random_tables(k, R, half, seed, inactive=False):
    """Random disjoint plane rotations per round: a random pairing of the positions,
    random signs and random angle indices (shared by partners)."""
    g = torch.Generator().manual_seed(seed)
    perm = torch.arange(k).repeat(R, 1)
    sgn = torch.zeros(R, k)
    p2p = torch.zeros(R, k, dtype=torch.int64)
    for r in range(R):
        order = torch.randperm(k, generator=g)
        npairs = k // 2 - (1 if inactive else 0)
        angles = torch.randperm(half, generator=g)  # one distinct angle per plane
        assert npairs <= half
        for m in range(npairs):
            i, j = int(order[2 * m]), int(order[2 * m + 1])
            s = 1.0 if torch.rand(1, generator=g).item() < 0.5 else -1.0
            a = int(angles[m])
            perm[r, i], perm[r, j] = j, i
            sgn[r, i], sgn[r, j] = s, -s
            p2p[r, i] = p2p[r, j] = a
    return perm.to(torch.int32), sgn, p2p.to(torch.int32)


def test_plane_tables_accepted():
    for k, R in ((2, 1), (8, 3), (16, 3)):
        perm, sgn, p2p = hip_scans._brick_tables(k, R)
        assert hip_scans._table_reason(perm, sgn, p2p, k, k // 2) is None
    from mingru_amd import workloads as wl

    perm, sgn, p2p = wl.lexicographic_schedule(16)
    assert hip_scans._table_reason(perm.long(), sgn.double(), p2p.long(), 16, 1) is None
    perm, sgn, p2p = _random_tables(8, 5, 3, seed=1, inactive=True)
    assert hip_scans._table_reason(perm.long(), sgn.double(), p2p.long(), 8, 3) is None


def test_plane_tables_rejected_with_distinct_reasons():
    base = [t.clone() for t in hip_scans._brick_tables(8, 2)]
    bad = {}
    p, s, q = (t.clone() for t in base)
    p[0, 0] = 9
    bad["range"] = (p, s, q)
    p, s, q = (t.clone() for t in base)
    p[0, 0], p[0, 1] = 2, 0  # 0 -> 2 but 2 -> 3
    bad["involution"] = (p, s, q)
    p, s, q = (t.clone() for t in base)
    q[0, 0] = 3
    bad["angle"] = (p, s, q)
    p, s, q = (t.clone() for t in base)
    s[0, 0] = 1.0  # same sign as its partner
    bad["sign"] = (p, s, q)
    p, s, q = (t.clone() for t in base)
    q[0, 0] = q[0, 1] = 7
    bad["p2p range"] = (p, s, q)
    p, s, q = (t.clone() for t in base)
    q[0, 2] = q[0, 3] = 0  # planes (0,1) and (2,3) both driven by angle 0
    bad["shared angle"] = (p, s, q)
    reasons = {name: hip_scans._table_reason(*t, 8, 4) for name, t in bad.items()}
    assert all(r is not None for r in reasons.values()), reasons
    assert len(set(reasons.values())) == len(reasons)


def test_plane_table_angle_cover():
    perm, sgn, p2p = hip_scans._brick_tables(8, 3)
    assert hip_scans._tables_cover_all_angles(perm, p2p, 4)
    assert not hip_scans._tables_cover_all_angles(perm, p2p, 5)  # angle 4 unused
    perm, sgn, p2p = _random_tables(4, 3, 2, seed=2, inactive=True)
    assert not hip_scans._tables_cover_all_angles(perm.long(), p2p.long(), 2)


def test_plane_table_cache_sees_new_sgn_and_p2p_objects():
    """The validated-table cache must not serve stale tables when the same ``perm`` object
    comes back with new ``sgn``/``p2p`` tensors (fresh objects start at ``_version`` 0 and
    may reuse an address), nor after an in-place change to any of the three."""
    perm, sgn, p2p = hip_scans._brick_tables(8, 2)
    t1 = hip_scans._device_tables(perm, sgn, p2p, 8, 4, torch.device("cpu"))
    assert hip_scans._device_tables(perm, sgn, p2p, 8, 4, torch.device("cpu")) is t1
    # same perm object, new p2p contents (each plane driven by another angle)
    p2p_new = (3 - p2p).to(p2p.dtype)
    t2 = hip_scans._device_tables(perm, sgn, p2p_new, 8, 4, torch.device("cpu"))
    assert torch.equal(t2[2].long(), p2p_new.long())
    # same perm object, new sgn (every plane's sign flipped)
    sgn_new = -sgn
    t3 = hip_scans._device_tables(perm, sgn_new, p2p_new, 8, 4, torch.device("cpu"))
    assert torch.equal(t3[1], sgn_new.float())
    # in-place change of the cached sgn object
    sgn_new.neg_()
    t4 = hip_scans._device_tables(perm, sgn_new, p2p_new, 8, 4, torch.device("cpu"))
    assert torch.equal(t4[1], sgn_new.float())


def test_rotation_gated_heads_reach_backend(monkeypatch):
    """RotationMinGRU's fast path hands the snapped angle (B, T, n, 1, 1), u (B, T, n),
    and z, h~ (B, T, n, 2) pre-activations to the gated-heads kernel; its result is the
    module's output."""
    seen = {}

    def fake_gated(theta, u, gamma, z, hpre, h0, perm, sgn, p2p, *, has_scale, has_decay):
        seen.update(theta=tuple(theta.shape), u=tuple(u.shape), z=tuple(z.shape),
                    hpre=tuple(hpre.shape), gamma=gamma, has_scale=has_scale,
                    has_decay=has_decay)
        return torch.full(z.shape, 4.0)

    def fake_plain(*args, **kwargs):
        raise AssertionError("the plain angle kernel must not run when the gated one does")

    _fake_backend(monkeypatch, angle_gated_scan_impl=fake_gated, angle_scan_impl=fake_plain)
    m = mg.RotationMinGRU(5, 6)
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    y = m(torch.randn(2, 7, 5))
    assert torch.equal(y, torch.full((2, 7, 6), 4.0))
    assert seen == {"theta": (2, 7, 3, 1, 1), "u": (2, 7, 3), "z": (2, 7, 3, 2),
                    "hpre": (2, 7, 3, 2), "gamma": None, "has_scale": 1, "has_decay": 0}


def test_givens_gated_heads_decline_runs_the_plain_kernel(monkeypatch):
    """A declined gated call is silent: the plain angle seam then runs with eager heads,
    under its own mode rules."""
    calls = []

    def fake_gated(*args, **kwargs):
        calls.append("gated")
        raise sys.modules[BACKEND].ScanFallback("schedule not covered")

    def fake_plain(theta, scale, gamma, b, h0, perm, sgn, p2p, *, has_scale, has_decay):
        calls.append("plain")
        assert tuple(b.shape) == (2, 7, 2, 8) and has_decay == 1
        return torch.zeros(b.shape)

    _fake_backend(monkeypatch, angle_gated_scan_impl=fake_gated, angle_scan_impl=fake_plain)
    m = GivensMinGRU(6, 16, block_size=8, decay="fixed")
    monkeypatch.setenv("MINGRU_SCAN", "hip")
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        y = m(torch.randn(2, 7, 6), delta_t=torch.rand(2, 7))
    assert calls == ["gated", "plain"]
    assert torch.equal(y, torch.zeros(2, 7, 16))
