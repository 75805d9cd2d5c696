"""GPU parity of whole ``MinGRUStack`` models under ``MINGRU_SCAN=hip``.

Each case builds one stack, runs it in float32 on the GPU with the HIP scans
forced (a decline raises, so no eager fallback can hide), and compares the
output, every block's returned state, the input gradient and every parameter
gradient with a float64 copy of the same model run through the CPU eager path.
Bars, each relative to max(1, max |ref|): 1e-4 on outputs and states, 1e-3 on
gradients.
Block/stack contract: reference ``src/mingru/min_gru.py:3698-4336``.
"""

import copy
import os
import warnings

import pytest
import torch

from mingru_amd import MinGRUStack

pytestmark = pytest.mark.gpu

FWD_TOL = 1e-4
GRAD_TOL = 1e-3

CASES = {
    "log": ("log", None),
    "signed": ("signed", None),
    "rotation_snap": ("rotation", None),  # default snap=(2, 3, 4, 6)
    "rotation_nosnap": ("rotation", {"snap": None}),
    "givens": ("givens", None),
    "givens_k4_r5": ("givens", {"block_size": 4, "rounds": 5}),
    "delta": ("delta", {"n_heads": 2}),
    "mixed": (["log", "signed", "rotation", "givens", "delta"], {"delta": {"n_heads": 2}}),
}


def _run(model, x, mode):
    os.environ["MINGRU_SCAN"] = mode
    try:
        out, state = model(x)
        loss = out.square().sum() + sum(s.sum() for s in state)
        loss.backward()
    finally:
        os.environ["MINGRU_SCAN"] = "auto"
    return out, state


@pytest.mark.parametrize("case", sorted(CASES))
def test_stack_hip_matches_fp64_eager(cuda, case):
    mixer, kwargs = CASES[case]
    n_layers = len(mixer) if isinstance(mixer, list) else 2
    torch.manual_seed(7)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        model = MinGRUStack(input_size=24, d_model=64, n_layers=n_layers, mixer=mixer,
                            mixer_kwargs=kwargs)
    ref = copy.deepcopy(model).double()
    gpu = model.to(cuda)
    x = torch.randn(2, 130, 24)
    x_ref = x.double().requires_grad_()
    x_gpu = x.to(cuda).requires_grad_()
    print(f"[gpu] stack case={case} B=2 T=130 d_model=64 layers={n_layers}", flush=True)

    out_r, st_r = _run(ref, x_ref, "eager")
    out_g, st_g = _run(gpu, x_gpu, "hip")
    torch.cuda.synchronize()

    def gerr(g, r):
        return (g.double().cpu() - r).abs().max().item() / max(1.0, r.abs().max().item())

    # The final LayerNorm keeps the output at unit scale; a block's state is its raw
    # recurrence value, which grows to |h| ~ 10 without decay (rotation mixers), so its
    # bar is relative to max(1, |h|) like the gradients'.
    e = gerr(out_g, out_r)
    es = max(gerr(a, b) for a, b in zip(st_g, st_r))
    print(f"[gpu] stack {case}: out err {e:.2e} state rel err {es:.2e} "
          f"(max |state| {max(b.abs().max().item() for b in st_r):.2f})", flush=True)
    assert e <= FWD_TOL and es <= FWD_TOL

    worst = gerr(x_gpu.grad, x_ref.grad)
    assert worst <= GRAD_TOL, f"x.grad {worst:.2e}"
    ref_params = dict(ref.named_parameters())
    for name, p in gpu.named_parameters():
        r = ref_params[name].grad
        assert (p.grad is None) == (r is None), name
        if r is None:
            continue
        eg = gerr(p.grad, r)
        worst = max(worst, eg)
        assert eg <= GRAD_TOL, f"{name}: {eg:.2e}"
    print(f"[gpu] stack {case}: worst relative grad err {worst:.2e}", flush=True)


def test_stack_hip_step_matches_forward(cuda):
    """Streaming decode through every mixer type on the GPU equals the parallel forward."""
    torch.manual_seed(3)
    mixer, kwargs = CASES["mixed"]
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        model = MinGRUStack(input_size=24, d_model=64, n_layers=len(mixer), mixer=mixer,
                            mixer_kwargs=kwargs).to(cuda)
    x = torch.randn(2, 40, 24, device=cuda)
    os.environ["MINGRU_SCAN"] = "hip"
    try:
        with torch.no_grad():
            out, st = model(x)
            state = model.init_state()
            outs = []
            for t in range(x.shape[1]):
                y, state = model.step(x[:, t], state)
                outs.append(y)
    finally:
        os.environ["MINGRU_SCAN"] = "auto"
    seq = torch.stack(outs, dim=1)
    e = (seq - out).abs().max().item()
    print(f"[gpu] stack step vs forward err {e:.2e}", flush=True)
    assert e <= 1e-4
    for a, b in zip(state, st):
        assert (a - b[:, 0]).abs().max().item() <= 1e-4 * max(1.0, b.abs().max().item())
