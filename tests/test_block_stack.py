"""CPU tests of ``MinGRUBlock`` / ``MinGRUStack``: the ``(output, state)``
contract, list mixers and their kwargs schema, streaming ``step`` == ``forward``,
chunked chaining through the returned state, and the block wiring recomputed
from the stack's own submodules.

Contract followed: reference ``src/mingru/min_gru.py:3698-4336``; the
reference's own checks of it are ``tests/test_mixers.py:614-720, 866-983``.
"""

import copy
import warnings

import pytest
import torch

from mingru_amd import MinGRUBlock, MinGRUStack

SEED = 42
B, T, D_IN, D_H = 2, 5, 8, 6

# d_model 8 keeps every mixer's shape constraint satisfied (rotation: even;
# givens: a multiple of its block size 4; delta with two heads: d_k = d_v = 4).
MIXER_KW = {
    "log": None,
    "signed": None,
    "rotation": None,
    "givens": {"block_size": 4},
    "delta": {"n_heads": 2},
}
D_ALL = 8


def _stack(mixer, n_layers=2, d_model=D_ALL, **kw):
    torch.manual_seed(SEED)
    if isinstance(mixer, str):
        mk = MIXER_KW[mixer]
    else:
        mk = {m: MIXER_KW[m] for m in set(mixer) if MIXER_KW[m]} or None
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        return MinGRUStack(input_size=D_IN, d_model=d_model, n_layers=n_layers,
                           mixer=mixer, mixer_kwargs=mk, **kw)


def _state_numel(block, d_model):
    m = block.mingru
    if getattr(m, "carries_matrix_state", False):
        return m.n_heads * m.d_k * m.d_v
    return d_model


# ---------------------------------------------------------------------------
# (output, state) contract
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("mixer", sorted(MIXER_KW))
def test_block_output_and_state_shapes(mixer):
    torch.manual_seed(SEED)
    block = MinGRUBlock(d_model=D_ALL, mixer=mixer, mixer_kwargs=MIXER_KW[mixer])
    x = torch.randn(B, T, D_ALL)
    out, state = block(x)
    assert out.shape == (B, T, D_ALL)
    assert state.shape == (B, 1, _state_numel(block, D_ALL))
    if not getattr(block.mingru, "carries_matrix_state", False):
        # a vector-state mixer's state is the mixer's last output, before the residual
        h_seq = block.mingru(block.norm1(x))
        assert torch.equal(state, h_seq[:, -1:])


def test_block_unknown_mixer_lists_valid_names():
    with pytest.raises(ValueError, match=r"delta"):
        MinGRUBlock(d_model=D_H, mixer="nope")


def test_block_without_mlp():
    torch.manual_seed(SEED)
    block = MinGRUBlock(d_model=D_H, mixer="signed", mlp_expansion=0)
    assert block.mlp is None and block.norm2 is None
    x = torch.randn(B, T, D_H)
    out, _ = block(x)
    assert torch.allclose(out, x + block.mingru(block.norm1(x)), atol=1e-6)


def test_stack_shapes_and_state_length():
    model = _stack("log", n_layers=3, d_model=D_H)
    out, state = model(torch.randn(B, T, D_IN))
    assert out.shape == (B, T, D_H)
    assert len(state) == 3 and all(s.shape == (B, 1, D_H) for s in state)
    assert model.init_state() == [None, None, None]


def test_stack_identity_in_proj_when_sizes_match():
    torch.manual_seed(SEED)
    model = MinGRUStack(input_size=D_H, d_model=D_H, n_layers=1)
    assert isinstance(model.in_proj, torch.nn.Identity)


def test_stack_list_mixer_and_per_type_kwargs():
    model = _stack(["signed", "delta", "givens"], n_layers=3)
    kinds = [type(b.mingru).__name__ for b in model.blocks]
    assert kinds == ["SignedMinGRU", "DeltaMinGRU", "GivensMinGRU"]
    assert model.blocks[1].mingru.n_heads == 2
    assert model.blocks[2].mingru.k == 4
    out, state = model(torch.randn(B, T, D_IN))
    assert out.shape == (B, T, D_ALL)
    assert [s.shape[-1] for s in state] == [_state_numel(b, D_ALL) for b in model.blocks]


@pytest.mark.parametrize(
    "mixer,kwargs,match",
    [
        (["log", "signed"], None, r"length"),  # list length != n_layers (3)
        (["log", "signed", "bogus"], None, r"bogus"),
        (["log", "signed", "log"], {"delta": {"n_heads": 2}}, r"delta"),  # key not present
        ("log", {"signed": {}}, r"signed"),  # str mixer given the list-mixer schema
        (3, None, r"str or list"),
    ],
)
def test_stack_spec_errors(mixer, kwargs, match):
    with pytest.raises(ValueError, match=match):
        MinGRUStack(input_size=D_IN, d_model=D_ALL, n_layers=3, mixer=mixer, mixer_kwargs=kwargs)


def test_stack_decay_layers_validation():
    with pytest.raises(ValueError, match=r"decay_layers"):
        MinGRUStack(input_size=D_IN, d_model=D_H, n_layers=2, decay_layers="first")


def test_stack_decay_layers_last_strips_decay_below_the_top():
    torch.manual_seed(SEED)
    model = MinGRUStack(input_size=D_IN, d_model=D_H, n_layers=3, mixer="signed",
                        mixer_kwargs={"decay": "learnable"}, decay_layers="last")
    assert [b.mingru.decay is not None for b in model.blocks] == [False, False, True]
    x = torch.randn(B, T, D_IN)
    dt = torch.rand(B, T)
    out, _ = model(x, delta_t=dt)
    assert out.shape == (B, T, D_H)


def test_multi_rotation_stack_warns_once():
    torch.manual_seed(SEED)
    with warnings.catch_warnings(record=True) as records:
        warnings.simplefilter("always")
        MinGRUStack(input_size=D_IN, d_model=D_H, n_layers=3, mixer="rotation")
    assert len([w for w in records if issubclass(w.category, UserWarning)]) == 1


# ---------------------------------------------------------------------------
# streaming, chaining and gradients
# ---------------------------------------------------------------------------


STACK_CASES = [*sorted(MIXER_KW), ("signed", "delta"), ("log", "rotation", "givens")]


def _case_id(c):
    return c if isinstance(c, str) else "+".join(c)


@pytest.mark.parametrize("mixer", STACK_CASES, ids=_case_id)
def test_stack_step_matches_forward(mixer):
    spec = mixer if isinstance(mixer, str) else list(mixer)
    model = _stack(spec, n_layers=2 if isinstance(mixer, str) else len(mixer))
    x = torch.randn(B, T, D_IN)
    out_par, state_par = model(x)
    state = model.init_state()
    outs = []
    for t in range(T):
        y, state = model.step(x[:, t], state)
        outs.append(y)
    assert torch.allclose(out_par, torch.stack(outs, dim=1), atol=1e-5)
    for s_seq, s_par in zip(state, state_par):
        assert torch.allclose(s_seq, s_par[:, 0], atol=1e-5)


@pytest.mark.parametrize("mixer", STACK_CASES, ids=_case_id)
def test_stack_chunked_forward_chains_through_state(mixer):
    """Running the sequence in two pieces, the second seeded with the state the
    first returned, reproduces the one-piece run (every block's state is its
    recurrence's last value, so it is a valid h_0 for the next piece)."""
    spec = mixer if isinstance(mixer, str) else list(mixer)
    model = _stack(spec, n_layers=2 if isinstance(mixer, str) else len(mixer))
    x = torch.randn(B, 9, D_IN)
    full, s_full = model(x)
    first, s1 = model(x[:, :4])
    second, s2 = model(x[:, 4:], s1)
    assert torch.allclose(torch.cat([first, second], dim=1), full, atol=1e-5)
    for a, b in zip(s2, s_full):
        assert torch.allclose(a, b, atol=1e-5)


@pytest.mark.parametrize("mixer", STACK_CASES, ids=_case_id)
def test_stack_matches_hand_wired_blocks(mixer):
    """The stack recomputed from its submodules alone: in_proj, then per block
    x + mixer(LN1 x) and x + MLP(LN2 x), then the final LayerNorm."""
    spec = mixer if isinstance(mixer, str) else list(mixer)
    model = _stack(spec, n_layers=2 if isinstance(mixer, str) else len(mixer)).double()
    x = torch.randn(B, T, D_IN, dtype=torch.float64)
    out, _ = model(x)
    h = model.in_proj(x)
    for blk in model.blocks:
        y = blk.mingru(blk.norm1(h))
        h = h + (y[0] if isinstance(y, tuple) else y)
        h = h + blk.mlp[3](blk.mlp[1](blk.mlp[0](blk.norm2(h))))
    assert torch.allclose(out, model.norm_out(h), atol=1e-12)


@pytest.mark.parametrize("mixer", STACK_CASES, ids=_case_id)
def test_stack_gradient_flow(mixer):
    spec = mixer if isinstance(mixer, str) else list(mixer)
    model = _stack(spec, n_layers=2 if isinstance(mixer, str) else len(mixer))
    x = torch.randn(B, T, D_IN, requires_grad=True)
    out, _ = model(x)
    out.square().sum().backward()
    assert x.grad is not None and x.grad.abs().sum() > 0
    grads = [p.grad for p in model.parameters() if p.requires_grad]
    assert all(g is not None for g in grads)
    assert any(g.abs().sum() > 0 for g in grads)


def test_stack_gradcheck_float64():
    """Finite differences through a two-block mixed stack (tiny shapes, float64)."""
    model = _stack(["signed", "delta"], n_layers=2).double()
    model.eval()
    x = torch.randn(1, 3, D_IN, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda inp: model(inp)[0], (x,), eps=1e-6, atol=1e-5)


def test_block_step_signed_regression_pin():
    """Known-answer pin of one streaming block step (seed 42, signed mixer, d_model 6).

    The expected values are the ones the reference's own test holds
    (``tests/test_mixers.py:948-978``); they pin the parameter construction
    order, the pre-norm wiring and the residual/MLP path of ``step``.
    """
    torch.manual_seed(SEED)
    block = MinGRUBlock(d_model=6, mixer="signed")
    x_t = torch.randn(2, 6)
    out, state = block.step(x_t, None)
    expected_out = torch.tensor(
        [
            [-0.1164, -0.5916, 0.7359, 1.1987, -0.2292, -0.7409],
            [0.9475, -0.2558, -0.1918, -0.8776, -1.5433, 0.8536],
        ]
    )
    expected_state = torch.tensor(
        [
            [-0.2117, -0.1494, -0.0530, -0.0080, -0.3067, -0.5182],
            [0.1409, 0.5886, -0.3198, -0.0620, 0.1942, 0.8264],
        ]
    )
    assert torch.allclose(out, expected_out, atol=1e-4)
    assert torch.allclose(state, expected_state, atol=1e-4)
    assert torch.allclose(state, block.mingru.step(block.norm1(x_t), None), atol=1e-6)


def test_block_step_matches_forward_for_delta_state():
    torch.manual_seed(SEED)
    block = MinGRUBlock(d_model=D_ALL, mixer="delta", mixer_kwargs={"n_heads": 2})
    x = torch.randn(B, T, D_ALL)
    out_par, state_par = block(x)
    state, outs = None, []
    for t in range(T):
        y, state = block.step(x[:, t], state)
        outs.append(y)
    assert torch.allclose(out_par, torch.stack(outs, dim=1), atol=1e-5)
    assert torch.allclose(state, state_par[:, 0], atol=1e-5)


def test_stack_deepcopy_double_is_independent():
    """The fp64 copy used as the GPU tests' reference shares no storage with the
    fp32 model it came from."""
    model = _stack("signed")
    ref = copy.deepcopy(model).double()
    p0 = next(model.parameters())
    p1 = next(ref.parameters())
    assert p0.dtype == torch.float32 and p1.dtype == torch.float64
    assert p0.data_ptr() != p1.data_ptr()
