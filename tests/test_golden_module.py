"""The reference's golden DeltaMinGRU vector through the module on the CPU eager path:
output, input gradient and all 16 parameter gradients (reference
``tests/test_mixers.py:496-511``; the fixture's nh=2 with the default chunk_size=64
is 128 micro-steps per chunk)."""

import os

import pytest
import torch

import golden_fixture as gf


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_golden_delta_module_eager(dtype, monkeypatch):
    monkeypatch.setenv("MINGRU_SCAN", "eager")
    fx = gf.load()
    layer = gf.module(fx, dtype)
    assert layer.chunk_size == 64 and layer.nh == 2
    out, gx, gp = gf.run(layer, torch.tensor(fx["x"], dtype=dtype))
    assert torch.allclose(out, torch.tensor(fx["output"], dtype=dtype), atol=1e-5)
    assert torch.allclose(gx, torch.tensor(fx["x_grad"], dtype=dtype), atol=1e-4)
    assert sorted(gp) == sorted(fx["param_grads"])
    for name, ref in fx["param_grads"].items():
        assert torch.allclose(gp[name], torch.tensor(ref, dtype=dtype), atol=1e-4), name


def test_golden_fixture_is_data_only():
    """The fixture holds numbers and names only (it is loaded with json, never unpickled)."""
    fx = gf.load()
    assert set(fx) >= {"state_dict", "x", "output", "x_grad", "param_grads"}
    assert os.path.getsize(gf.PATH) < 64 * 1024
