"""Pins the fp64 oracle (CPU only) so a plausible mistake in it fails a check.

Each oracle function is checked against something independent of its own
formula: closed forms, invariants, the reference's own (different) formulas
evaluated in float64, brute-force matrix materialisation, central finite
differences, and the reference's golden DeltaMinGRU fixture.
"""

import json
import math
import os

import numpy as np
import pytest
import torch

from mingru_amd import workloads as wl
from oracle import scans as orc

HERE = os.path.dirname(os.path.abspath(__file__))
RNG = np.random.default_rng(1234)


def _fd(f, args, idx, gout, eps=1e-6, n_probe=12):
    """Central finite-difference check of <gout, d f / d args[idx]> at random coordinates."""
    x = args[idx]
    probes = RNG.choice(x.size, size=min(n_probe, x.size), replace=False)
    out = []
    for p in probes:
        xp = x.copy().reshape(-1)
        xm = x.copy().reshape(-1)
        xp[p] += eps
        xm[p] -= eps
        ap = list(args)
        am = list(args)
        ap[idx] = xp.reshape(x.shape)
        am[idx] = xm.reshape(x.shape)
        fp, fm = f(*ap), f(*am)
        if not isinstance(fp, tuple):
            fp, fm = (fp,), (fm,)
        out.append(sum(np.sum(g * (a - b)) for g, a, b in zip(gout, fp, fm)) / (2 * eps))
    return probes, np.array(out)


# ---------------------------------------------------------------- linear_scan


def test_linear_scan_closed_forms():
    a = RNG.uniform(-1, 1, (2, 9, 3))
    b = RNG.normal(size=(2, 9, 3))
    A, Bc = orc.linear_scan(a, b)
    np.testing.assert_allclose(A, np.cumprod(a, axis=1), rtol=1e-12)
    _, Bc1 = orc.linear_scan(np.ones_like(a), b)
    np.testing.assert_allclose(Bc1, np.cumsum(b, axis=1), rtol=1e-12)
    A1, B1 = orc.linear_scan(a[:, :1], b[:, :1])
    np.testing.assert_array_equal(A1, a[:, :1])
    np.testing.assert_array_equal(B1, b[:, :1])


def test_linear_scan_matches_hillis_steele_formula():
    """The reference's eager doubling recurrence (src/mingru/min_gru.py:1501-1510) in fp64."""
    a = RNG.uniform(-1, 1, (2, 37, 4))
    b = RNG.normal(size=(2, 37, 4))
    A, Bc, step, T = a.copy(), b.copy(), 1, a.shape[1]
    while step < T:
        Ap = np.concatenate([np.ones((2, step, 4)), A[:, : T - step]], axis=1)
        Bp = np.concatenate([np.zeros((2, step, 4)), Bc[:, : T - step]], axis=1)
        Bc = A * Bp + Bc
        A = A * Ap
        step *= 2
    rA, rB = orc.linear_scan(a, b)
    np.testing.assert_allclose(rA, A, atol=1e-12)
    np.testing.assert_allclose(rB, Bc, atol=1e-12)


def test_linear_scan_bwd_finite_differences():
    a = RNG.uniform(-1, 1, (2, 11, 3))
    b = RNG.normal(size=(2, 11, 3))
    gA, gB = RNG.normal(size=a.shape), RNG.normal(size=a.shape)
    da, db = orc.linear_scan_bwd(a, b, gA, gB)
    for idx, grad in ((0, da), (1, db)):
        probes, fd = _fd(orc.linear_scan, (a, b), idx, (gA, gB))
        np.testing.assert_allclose(grad.reshape(-1)[probes], fd, rtol=1e-6, atol=1e-7)


# ---------------------------------------------------------- parallel_scan_log


def _heinsen(lc, lv):
    """Reference formula (src/mingru/min_gru.py:804-807) evaluated in float64."""
    cum = np.concatenate([np.zeros_like(lc[:, :1]), np.cumsum(lc, axis=1)], axis=1)
    lse = np.logaddexp.accumulate(lv - cum, axis=1)
    return np.exp(cum + lse)[:, 1:]


def test_parallel_scan_log_matches_heinsen():
    inp = wl.c1_inputs(2, 50, 6)
    lc, lv = inp["log_coeffs"].double().numpy(), inp["log_values"].double().numpy()
    np.testing.assert_allclose(orc.parallel_scan_log(lc, lv), _heinsen(lc, lv), rtol=1e-10)


def test_parallel_scan_log_t1_closed_form():
    lc = RNG.normal(size=(3, 1, 4))
    lv = RNG.normal(size=(3, 2, 4))
    ref = np.exp(lc[:, 0] + lv[:, 0]) + np.exp(lv[:, 1])
    np.testing.assert_allclose(orc.parallel_scan_log(lc, lv)[:, 0], ref, rtol=1e-13)


def test_parallel_scan_log_bwd_finite_differences():
    lc = -np.abs(RNG.normal(size=(2, 9, 3)))
    lv = RNG.normal(size=(2, 10, 3)) * 0.5
    gh = RNG.normal(size=(2, 9, 3))
    dlc, dlv = orc.parallel_scan_log_bwd(lc, lv, gh)
    for idx, grad in ((0, dlc), (1, dlv)):
        probes, fd = _fd(orc.parallel_scan_log, (lc, lv), idx, (gh,))
        np.testing.assert_allclose(grad.reshape(-1)[probes], fd, rtol=1e-6, atol=1e-7)


# ------------------------------------------------------------- affine scans


def test_affine_identity_is_cumsum_and_k2_matches_matrix_scan_formula():
    B, T, n = 2, 13, 3
    Bm = RNG.normal(size=(B, T, n, 2, 1))
    A = np.broadcast_to(np.eye(2), (B, T, n, 2, 2))
    Abar, Bbar = orc.affine_scan(A, Bm)
    np.testing.assert_allclose(Bbar, np.cumsum(Bm, axis=1), atol=1e-12)
    np.testing.assert_allclose(Abar, A, atol=0)
    # reference matrix_scan doubling (src/mingru/min_gru.py:1570-1581), fp64
    M = RNG.normal(size=(B, T, n, 2, 2)) * 0.5
    b = RNG.normal(size=(B, T, n, 2))
    Ah, Bh, step = M.copy(), b.copy(), 1
    while step < T:
        Ap = np.concatenate([np.broadcast_to(np.eye(2), (B, step, n, 2, 2)), Ah[:, : T - step]], 1)
        Bp = np.concatenate([np.zeros((B, step, n, 2)), Bh[:, : T - step]], 1)
        Bh = np.einsum("btnij,btnj->btni", Ah, Bp) + Bh
        Ah = Ah @ Ap
        step *= 2
    rA, rB = orc.affine_scan(M, b[..., None])
    np.testing.assert_allclose(rA, Ah, atol=1e-12)
    np.testing.assert_allclose(rB[..., 0], Bh, atol=1e-12)


@pytest.mark.parametrize("k,v", [(2, 1), (3, 2), (4, 4)])
def test_affine_bwd_finite_differences(k, v):
    A = RNG.normal(size=(2, 7, 2, k, k)) * 0.4
    Bm = RNG.normal(size=(2, 7, 2, k, v))
    gA, gB = RNG.normal(size=A.shape), RNG.normal(size=Bm.shape)
    dA, dB = orc.affine_scan_bwd(A, Bm, gA, gB)
    for idx, grad in ((0, dA), (1, dB)):
        probes, fd = _fd(orc.affine_scan, (A, Bm), idx, (gA, gB))
        np.testing.assert_allclose(grad.reshape(-1)[probes], fd, rtol=1e-6, atol=1e-7)


# ------------------------------------------------------------- angle scan


def _brick(k, R):
    from mingru_amd import GivensMinGRU

    return [t.numpy() for t in GivensMinGRU(4, k, block_size=k, rounds=R)._angle_plane_meta("cpu")]


def test_givens_plane_meta_matches_reference_row_update():
    """Materialising M from perm/sgn/p2p equals GivensMinGRU._coeffs' row-update product."""
    from mingru_amd import GivensMinGRU

    torch.manual_seed(0)
    layer = GivensMinGRU(5, 16, block_size=8, rounds=3).double()
    x = torch.randn(2, 4, 5, dtype=torch.float64)
    M_ref, _ = layer._coeffs(x)
    theta, _, _, _ = layer._angle_heads(x, None)
    perm, sgn, p2p = [t.numpy() for t in layer._angle_plane_meta("cpu")]
    M = orc.angle_transition_matrices(theta.detach().numpy(), None, None, perm, sgn, p2p, 0, 0)
    np.testing.assert_allclose(M, M_ref.detach().numpy(), atol=1e-13)


@pytest.mark.parametrize("sched", ["brick", "lex"])
def test_angle_scan_equals_materialised_sequential(sched):
    k = 8
    if sched == "brick":
        perm, sgn, p2p = _brick(k, 3)
        R, half = 3, 4
    else:
        perm, sgn, p2p = [t.numpy() for t in wl.lexicographic_schedule(k)]
        R, half = 28, 1
    B, T, n = 2, 9, 3
    theta = RNG.normal(size=(B, T, n, R, half)) * 0.7
    gamma = RNG.uniform(0.2, 1, size=(B, T, n))
    b = RNG.normal(size=(B, T, n, k))
    h0 = RNG.normal(size=(B, n, k))
    h = orc.angle_scan(theta, None, gamma, b, h0, perm, sgn, p2p, 0, 1)
    M = orc.angle_transition_matrices(theta, None, gamma, perm, sgn, p2p, 0, 1)
    cur = h0
    for t in range(T):
        cur = np.einsum("bnij,bnj->bni", M[:, t], cur) + b[:, t]
        np.testing.assert_allclose(h[:, t], cur, atol=1e-12)
    # every transition / gamma is special orthogonal
    R_ = M / gamma[..., None, None]
    eye = np.eye(k)
    np.testing.assert_allclose(R_ @ np.swapaxes(R_, -1, -2), np.broadcast_to(eye, R_.shape),
                               atol=1e-12)
    np.testing.assert_allclose(np.linalg.det(R_), 1.0, atol=1e-10)


def test_angle_scan_norm_preserved_without_decay_or_input():
    perm, sgn, p2p = [t.numpy() for t in wl.lexicographic_schedule(8)]
    theta = RNG.normal(size=(1, 50, 2, 28, 1))
    h0 = RNG.normal(size=(1, 2, 8))
    h = orc.angle_scan(theta, None, None, np.zeros((1, 50, 2, 8)), h0, perm, sgn, p2p, 0, 0)
    np.testing.assert_allclose(np.linalg.norm(h, axis=-1),
                               np.broadcast_to(np.linalg.norm(h0, axis=-1)[:, None], (1, 50, 2)),
                               rtol=1e-12)


def test_rotation_meta_matches_rotation_coeffs():
    from mingru_amd import RotationMinGRU

    torch.manual_seed(2)
    layer = RotationMinGRU(5, 6, snap=None).double()
    x = torch.randn(2, 3, 5, dtype=torch.float64)
    M_ref, _ = layer._coeffs(x)
    theta, scale, _, _ = layer._angle_heads(x, None)
    perm, sgn, p2p = [t.numpy() for t in layer._angle_plane_meta("cpu")]
    M = orc.angle_transition_matrices(theta.detach().numpy(), scale.detach().numpy(), None, perm,
                                      sgn, p2p, 1, 0)
    np.testing.assert_allclose(M, M_ref.detach().numpy(), atol=1e-13)


@pytest.mark.parametrize("sched,hs,hd", [("brick", 0, 1), ("lex", 0, 1), ("rot", 1, 1),
                                         ("brick2", 0, 0)])
def test_angle_bwd_finite_differences(sched, hs, hd):
    if sched == "brick":
        k, (perm, sgn, p2p), R, half = 8, _brick(8, 3), 3, 4
    elif sched == "brick2":
        k, (perm, sgn, p2p), R, half = 4, _brick(4, 2), 2, 2
    elif sched == "lex":
        k, R, half = 4, 6, 1
        perm, sgn, p2p = [t.numpy() for t in wl.lexicographic_schedule(4)]
    else:
        k, (perm, sgn, p2p), R, half = 2, _brick(2, 1), 1, 1
    B, T, n = 2, 6, 2
    theta = RNG.normal(size=(B, T, n, R, half))
    scale = RNG.uniform(-1, 1, size=(B, T, n))
    gamma = RNG.uniform(0.3, 1, size=(B, T, n))
    b = RNG.normal(size=(B, T, n, k))
    h0 = RNG.normal(size=(B, n, k))
    gh = RNG.normal(size=(B, T, n, k))

    def f(th, sc, gm, bb, hz):
        return orc.angle_scan(th, sc, gm, bb, hz, perm, sgn, p2p, hs, hd)

    grads = orc.angle_scan_bwd(theta, scale, gamma, b, h0, perm, sgn, p2p, hs, hd, gh)
    args = (theta, scale, gamma, b, h0)
    for idx, grad in enumerate(grads):
        if (idx == 1 and not hs) or (idx == 2 and not hd):
            continue
        probes, fd = _fd(f, args, idx, (gh,))
        np.testing.assert_allclose(grad.reshape(-1)[probes], fd, rtol=1e-6, atol=1e-7)


# ------------------------------------------------------------- delta rule


def _delta_inputs(B=2, H=2, T=11, nh=1, dk=4, dv=3, seed=0):
    r = np.random.default_rng(seed)
    Q = r.normal(size=(B, H, T, dk))
    K = r.normal(size=(B, H, T, nh, dk))
    K /= np.linalg.norm(K, axis=-1, keepdims=True)
    V = r.normal(size=(B, H, T, nh, dv))
    beta = 2 / (1 + np.exp(-r.normal(size=(B, H, T, nh))))
    H0 = r.normal(size=(B, H, dk, dv)) * 0.3
    return Q, K, V, beta, H0


@pytest.mark.parametrize("nh", [1, 2])
@pytest.mark.parametrize("chunk", [1, 3, 4, 11, 16])
def test_delta_chunked_equals_sequential(nh, chunk):
    Q, K, V, beta, H0 = _delta_inputs(nh=nh)
    y_s, H_s = orc.delta_sequential(Q, K, V, beta, H0)
    y_c, H_c, _ = orc.delta_chunked(Q, K, V, beta, H0, chunk)
    np.testing.assert_allclose(y_c, y_s, atol=1e-11)
    np.testing.assert_allclose(H_c, H_s, atol=1e-11)


def test_delta_householder_reflection_special_case():
    """beta = 2 with unit k: one micro-step is an exact reflection (I - 2 k k^T) H."""
    Q, K, V, beta, H0 = _delta_inputs(T=1)
    beta[:] = 2.0
    V[:] = 0.0
    _, HT, _ = orc.delta_chunked(Q, K, V, beta, H0, 4)
    k = K[:, :, 0, 0]
    refl = np.eye(4) - 2 * np.einsum("bhi,bhj->bhij", k, k)
    np.testing.assert_allclose(HT, refl @ H0, atol=1e-13)


@pytest.mark.parametrize("nh,chunk", [(1, 4), (2, 3), (1, 16)])
def test_delta_bwd_finite_differences(nh, chunk):
    Q, K, V, beta, H0 = _delta_inputs(T=9, nh=nh, seed=3)
    r = np.random.default_rng(9)
    dy = r.normal(size=(2, 2, 9, 3))
    dHT = r.normal(size=(2, 2, 4, 3))

    def f(q, k, v, bt, h0):
        y, HT, _ = orc.delta_chunked(q, k, v, bt, h0, chunk)
        return y, HT

    grads = orc.delta_chunked_bwd(Q, K, V, beta, H0, chunk, dy, dHT)
    for idx, grad in enumerate(grads):
        probes, fd = _fd(f, (Q, K, V, beta, H0), idx, (dy, dHT))
        np.testing.assert_allclose(grad.reshape(-1)[probes], fd, rtol=1e-6, atol=1e-7)


def test_delta_golden_fixture():
    """The reference's golden DeltaMinGRU vector (tests/fixtures/...decay_none_golden.json)."""
    with open(os.path.join(HERE, "golden", "delta_mingru_decay_none_golden.json")) as f:
        fx = json.load(f)
    sd = {k: np.asarray(v, np.float64) for k, v in fx["state_dict"].items()}
    x = np.asarray(fx["x"], np.float64)
    nh, Hn = fx["nh"], fx["n_heads"]
    B, T, _ = x.shape
    dk = sd["linear_q.weight"].shape[0] // Hn

    def lin(name, inp):
        return inp @ sd[f"{name}.weight"].T + sd[f"{name}.bias"]

    q = lin("linear_q", x).reshape(B, T, Hn, dk)
    ks = [lin(f"linear_k.{j}", x).reshape(B, T, Hn, dk) for j in range(nh)]
    ks = [k / np.linalg.norm(k, axis=-1, keepdims=True) for k in ks]
    vs = [lin(f"linear_v.{j}", x).reshape(B, T, Hn, -1) for j in range(nh)]
    bs = [2 / (1 + np.exp(-lin(f"linear_beta.{j}", x))) for j in range(nh)]
    Q = q.transpose(0, 2, 1, 3)
    K = np.stack(ks, 2).transpose(0, 3, 1, 2, 4)
    V = np.stack(vs, 2).transpose(0, 3, 1, 2, 4)
    beta = np.stack(bs, 2).transpose(0, 3, 1, 2)
    H0 = np.zeros((B, Hn, dk, V.shape[-1]))
    y, _ = orc.delta_sequential(Q, K, V, beta, H0)
    out = lin("out_proj", y.transpose(0, 2, 1, 3).reshape(B, T, -1))
    np.testing.assert_allclose(out, np.asarray(fx["output"]), atol=1e-5)
    y2, _, _ = orc.delta_chunked(Q, K, V, beta, H0, 2)
    out2 = lin("out_proj", y2.transpose(0, 2, 1, 3).reshape(B, T, -1))
    np.testing.assert_allclose(out2, np.asarray(fx["output"]), atol=1e-5)
    # golden output gradient: loss = output.sum(), so dL/d(out_proj.bias) = B*T
    np.testing.assert_allclose(np.asarray(fx["param_grads"]["out_proj.bias"]), B * T, atol=1e-4)
    assert math.isfinite(float(np.sum(out)))


# -------------------------------------------------------- gated delta rule


def _gated_lg(B=2, H=2, T=11, seed=5, scale=0.6):
    return -scale * np.random.default_rng(seed).random(size=(B, H, T))


def test_delta_gated_zero_decay_is_the_ungated_rule():
    """log gamma = 0: the gated recurrence is the golden-pinned ungated one."""
    Q, K, V, beta, H0 = _delta_inputs(nh=2)
    y0, H0T = orc.delta_sequential(Q, K, V, beta, H0)
    y, HT = orc.delta_gated_sequential(Q, K, V, beta, np.zeros(Q.shape[:3]), H0)
    np.testing.assert_allclose(y, y0, atol=1e-13)
    np.testing.assert_allclose(HT, H0T, atol=1e-13)


def test_delta_gated_beta_zero_is_pure_decay():
    """beta = 0: H_t = exp(sum_{s<=t} l_s) H0 and y_t = H_t^T q_t in closed form."""
    Q, K, V, beta, H0 = _delta_inputs(T=7)
    beta[:] = 0.0
    lg = _gated_lg(T=7)
    y, HT = orc.delta_gated_sequential(Q, K, V, beta, lg, H0)
    G = np.exp(np.cumsum(lg, axis=-1))
    np.testing.assert_allclose(HT, G[..., -1, None, None] * H0, atol=1e-13)
    ref = G[..., None] * np.einsum("bhtk,bhkv->bhtv", Q, H0)
    np.testing.assert_allclose(y, ref, atol=1e-13)


@pytest.mark.parametrize("nh,chunk", [(1, 4), (2, 3), (1, 16), (3, 5)])
def test_delta_gated_matches_module_span_sum_forward(nh, chunk):
    """The module's eager decay-active forward (span-sum chunked form of the
    reference ``_forward_chunked_gated``) equals the token-by-token oracle in float64."""
    from mingru_amd import DeltaMinGRU

    torch.manual_seed(nh * 10 + chunk)
    m = DeltaMinGRU(5, 8, n_heads=2, nh=nh, chunk_size=chunk, decay="learnable").double()
    x = torch.randn(2, 13, 5, dtype=torch.float64)
    dt = torch.rand(2, 13, dtype=torch.float64) * 2
    dt[:, 4] = 40.0  # one gap that drives gamma to ~0 for every span containing it
    with torch.no_grad():
        y, HT = m(x, delta_t=dt, return_state=True)
        q, ks, vs, betas = m._coeffs(x)
        Q, K, V, beta = (t.numpy() for t in m._layouts(q, ks, vs, betas))
        lg = (-m._decay_lambda().reshape(1, -1, 1) * dt.unsqueeze(1)).numpy()
    yo, HTo = orc.delta_gated_sequential(Q, K, V, beta, lg, np.zeros((2, 2, 4, 4)))
    with torch.no_grad():
        ref = m.out_proj(torch.from_numpy(yo).permute(0, 2, 1, 3).reshape(2, 13, 8))
    np.testing.assert_allclose(y.numpy(), ref.numpy(), atol=1e-11)
    np.testing.assert_allclose(HT.numpy().reshape(HTo.shape), HTo, atol=1e-11)


@pytest.mark.parametrize("nh", [1, 2])
def test_delta_gated_bwd_finite_differences(nh):
    Q, K, V, beta, H0 = _delta_inputs(T=8, nh=nh, seed=7)
    lg = _gated_lg(T=8, seed=8)
    r = np.random.default_rng(10)
    dy = r.normal(size=(2, 2, 8, 3))
    dHT = r.normal(size=(2, 2, 4, 3))
    grads = orc.delta_gated_sequential_bwd(Q, K, V, beta, lg, H0, dy, dHT)
    args = (Q, K, V, beta, lg, H0)
    for idx, grad in enumerate(grads):
        probes, fd = _fd(orc.delta_gated_sequential, args, idx, (dy, dHT))
        np.testing.assert_allclose(grad.reshape(-1)[probes], fd, rtol=1e-6, atol=1e-7)
