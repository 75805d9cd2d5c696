"""Loader for the reference's golden DeltaMinGRU fixture (JSON data only).

``tests/golden/delta_mingru_decay_none_golden.json`` is the reference's
``tests/fixtures/delta_mingru_decay_none_golden.json``: a ``DeltaMinGRU``
(D_IN=8, D_H=6, n_heads=2, nh=2, default chunk_size=64, decay=None) state_dict,
an input ``x`` and, for the loss ``output.sum()``, the output, ``x_grad`` and the
gradient of every parameter (pinned by the reference's
``tests/test_mixers.py:496-511``).
"""

import json
import os

import torch

from mingru_amd import DeltaMinGRU

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                    "delta_mingru_decay_none_golden.json")


def load():
    with open(PATH) as f:
        return json.load(f)


def module(fx, dtype=torch.float32):
    """The fixture's layer with its state_dict loaded (constructor defaults otherwise)."""
    layer = DeltaMinGRU(fx["D_IN"], fx["D_H"], n_heads=fx["n_heads"], nh=fx["nh"])
    sd = {k: torch.tensor(v, dtype=dtype) for k, v in fx["state_dict"].items()}
    layer = layer.to(dtype)
    layer.load_state_dict(sd)
    return layer


def run(layer, x):
    """``(output, x_grad, {param: grad})`` for the fixture's loss ``output.sum()``."""
    x = x.detach().clone().requires_grad_(True)
    layer.zero_grad(set_to_none=True)
    out = layer(x)
    out.sum().backward()
    return out.detach(), x.grad.detach(), {n: p.grad.detach() for n, p in layer.named_parameters()}
