"""GPU contract of the scan entry points beyond fp32 parity.

* Half-precision inputs (bf16, fp16) run the fp32 kernels on upcast copies and come
  back in the input dtype, as the eager ops do: outputs and gradients equal the fp32
  kernel's results on the upcast inputs, rounded once to the input dtype (the
  look-back carry may associate differently between the two runs, hence one ulp of
  slack on top of that rounding).
* float64 inputs decline (the kernels compute in fp32): under MINGRU_SCAN=hip the call
  raises RuntimeError naming the reason; under auto it warns once and returns the
  eager float64 result (reference seam behaviour, src/mingru/min_gru.py:255-319).
"""

import pytest
import torch

import mingru_amd as mg
from mingru_amd import linear_scan, matrix_affine_scan, parallel_scan_log

pytestmark = pytest.mark.gpu

HALF = [torch.bfloat16, torch.float16]


def _ulp_close(x, ref, dtype):
    eps = torch.finfo(dtype).eps
    ref = ref.to(dtype).float()
    return bool(((x.float() - ref).abs() <= 2 * eps * ref.abs() + 1e-6).all())


def _inputs(kind, dtype, cuda):
    g = torch.Generator().manual_seed(7)
    if kind == "linear":
        a = torch.tanh(2 * torch.randn(2, 300, 40, generator=g))
        b = torch.randn(2, 300, 40, generator=g)
        gs = (torch.randn(2, 300, 40, generator=g), torch.randn(2, 300, 40, generator=g))
        xs = (a, b)
    elif kind == "log":
        xs = (torch.nn.functional.logsigmoid(torch.randn(2, 300, 40, generator=g)),
              torch.randn(2, 301, 40, generator=g) - 1.0)
        gs = (torch.randn(2, 300, 40, generator=g),)
    else:
        A = 0.7 * torch.randn(2, 200, 12, 2, 2, generator=g)
        Bm = torch.randn(2, 200, 12, 2, 1, generator=g)
        xs = (A, Bm)
        gs = (torch.randn(2, 200, 12, 2, 2, generator=g), torch.randn(2, 200, 12, 2, 1, generator=g))
    return [x.to(dtype).to(cuda) for x in xs], [t.to(dtype).to(cuda) for t in gs]


def _run(kind, xs, gs):
    xs = [x.detach().clone().requires_grad_(True) for x in xs]
    fn = {"linear": linear_scan, "log": parallel_scan_log, "affine": matrix_affine_scan}[kind]
    out = fn(*xs)
    out = out if isinstance(out, tuple) else (out,)
    grads = torch.autograd.grad(out, xs, gs)
    torch.cuda.synchronize()
    return out, grads


@pytest.fixture
def _hip(monkeypatch):
    monkeypatch.setenv("MINGRU_SCAN", "hip")


@pytest.mark.parametrize("dtype", HALF)
@pytest.mark.parametrize("kind", ["linear", "log", "affine"])
def test_half_inputs_run_fp32_kernels_and_keep_dtype(cuda, _hip, kind, dtype):
    print(f"[gpu] contract half inputs {kind} {dtype}", flush=True)
    xs, gs = _inputs(kind, dtype, cuda)
    out, grads = _run(kind, xs, gs)
    out32, grads32 = _run(kind, [x.float() for x in xs], [t.float() for t in gs])
    for o, o32 in zip(out, out32):
        assert o.dtype == dtype
        assert _ulp_close(o, o32, dtype)
    for d, d32 in zip(grads, grads32):
        assert d.dtype == dtype
        assert _ulp_close(d, d32, dtype)


def test_float64_declines_loudly_under_hip(cuda, _hip):
    a = torch.rand(2, 16, 8, dtype=torch.float64, device=cuda)
    with pytest.raises(RuntimeError, match="fp32"):
        linear_scan(a, a)


def test_float64_falls_back_to_eager_under_auto(cuda, monkeypatch):
    monkeypatch.setenv("MINGRU_SCAN", "auto")
    monkeypatch.setattr(mg.min_gru, "_warned_scan_fallback", False)
    g = torch.Generator().manual_seed(8)
    a = torch.tanh(torch.randn(2, 40, 8, generator=g, dtype=torch.float64)).to(cuda)
    b = torch.randn(2, 40, 8, generator=g, dtype=torch.float64).to(cuda)
    with pytest.warns(UserWarning, match="fell back"):
        A, Bc = linear_scan(a, b)
    assert A.dtype == torch.float64 and Bc.dtype == torch.float64
    monkeypatch.setenv("MINGRU_SCAN", "eager")
    A_e, B_e = linear_scan(a, b)
    assert torch.equal(A, A_e) and torch.equal(Bc, B_e)
