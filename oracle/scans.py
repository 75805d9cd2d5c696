"""fp64 CPU oracle for the minGRU scan hot path (TEST INFRASTRUCTURE ONLY).

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import it.
Every function is a sequential (time-step by time-step) restatement in numpy
float64 of the reference algorithm it cites, with hand-derived adjoints for
the backward.  Loops run over time only and are vectorised over all lanes.

How each function is pinned (see ``tests/test_oracle.py``):

* linear_scan / linear_scan_bwd -- ``src/mingru/min_gru.py:1454-1510``;
  pinned by A = cumprod(a), a == 1 => Bc = cumsum(b), the T = 1 closed form,
  the reference's Hillis-Steele formula evaluated independently in fp64, and
  central finite differences for the adjoint.
* parallel_scan_log / _bwd -- ``src/mingru/min_gru.py:755-807``; pinned by the
  reference's Heinsen formula (cumsum + logcumsumexp) evaluated in fp64, the
  T = 1 closed form and finite differences.
* affine_scan / _bwd -- ``src/mingru/min_gru.py:1513-1655``; pinned by
  identity transitions => cumsum, k = 2, v = 1 == matrix_scan, the
  Hillis-Steele einsum formula, and finite differences.
* angle_scan / _bwd -- ``src/mingru/triton_scans.py:1039-1291`` (round
  semantics) and ``src/mingru/min_gru.py:2552-2602`` (row-update rule);
  pinned by brute-force materialisation of each transition matrix,
  orthogonality / determinant +1, norm preservation at gamma = 1, b = 0, and
  finite differences.
* delta_sequential / delta_chunked / delta_chunked_bwd --
  ``src/mingru/min_gru.py:3103-3255, 3611-3688`` and
  ``src/mingru/triton_scans.py:473-605``; pinned by the reference golden
  fixture (``tests/golden/``), sequential == chunked for every chunk size,
  and finite differences.
* delta_gated_sequential / _bwd -- the decay-active delta rule of ``step``
  (``src/mingru/min_gru.py:3611-3688``: decay the state, then the token's
  micro-steps); pinned by log_gamma = 0 == delta_sequential, the beta = 0
  closed form, the module's span-sum chunked forward (reference structure
  ``:3257-3448``) in float64, and finite differences.
"""

from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------------------
# linear_scan
# ---------------------------------------------------------------------------


def linear_scan(a: np.ndarray, b: np.ndarray):
    """``h_t = a_t h_{t-1} + b_t``: returns ``(A, Bc)`` (running product, zero-start)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    A = np.empty_like(a)
    Bc = np.empty_like(b)
    pa = np.ones_like(a[:, 0])
    pb = np.zeros_like(b[:, 0])
    for t in range(a.shape[1]):
        pa = a[:, t] * pa
        pb = a[:, t] * pb + b[:, t]
        A[:, t] = pa
        Bc[:, t] = pb
    return A, Bc


def linear_scan_bwd(a, b, gA, gB):
    """Adjoint of :func:`linear_scan`: ``x_t = g_t + a_{t+1} x_{t+1}``;
    ``da_t = xA_t A_{t-1} + xB_t Bc_{t-1}``, ``db_t = xB_t``."""
    a = np.asarray(a, np.float64)
    A, Bc = linear_scan(a, b)
    T = a.shape[1]
    xa = np.zeros_like(a[:, 0])
    xb = np.zeros_like(a[:, 0])
    da = np.empty_like(a)
    db = np.empty_like(a)
    for t in range(T - 1, -1, -1):
        if t + 1 < T:
            xa = gA[:, t] + a[:, t + 1] * xa
            xb = gB[:, t] + a[:, t + 1] * xb
        else:
            xa = np.asarray(gA[:, t], np.float64).copy()
            xb = np.asarray(gB[:, t], np.float64).copy()
        Ap = A[:, t - 1] if t > 0 else np.ones_like(xa)
        Bp = Bc[:, t - 1] if t > 0 else np.zeros_like(xb)
        da[:, t] = xa * Ap + xb * Bp
        db[:, t] = xb
    return da, db


# ---------------------------------------------------------------------------
# parallel_scan_log
# ---------------------------------------------------------------------------


def parallel_scan_log(lc, lv):
    """``h_t = exp(lc_t) h_{t-1} + exp(lv_{t+1})`` with ``h_{-1} = exp(lv_0)``; returns h (B,T,D)."""
    lc = np.asarray(lc, np.float64)
    lv = np.asarray(lv, np.float64)
    a = np.exp(lc)
    bv = np.exp(lv)
    h = np.empty_like(lc)
    cur = bv[:, 0]
    for t in range(lc.shape[1]):
        cur = a[:, t] * cur + bv[:, t + 1]
        h[:, t] = cur
    return h


def parallel_scan_log_bwd(lc, lv, gh):
    """Adjoint of :func:`parallel_scan_log`: returns ``(dlc (B,T,D), dlv (B,T+1,D))``."""
    lc = np.asarray(lc, np.float64)
    lv = np.asarray(lv, np.float64)
    gh = np.asarray(gh, np.float64)
    a = np.exp(lc)
    bv = np.exp(lv)
    h = parallel_scan_log(lc, lv)
    T = lc.shape[1]
    dlc = np.empty_like(lc)
    dlv = np.empty_like(lv)
    x = np.zeros_like(lc[:, 0])
    for t in range(T - 1, -1, -1):
        x = gh[:, t] + (a[:, t + 1] * x if t + 1 < T else 0.0)
        hp = h[:, t - 1] if t > 0 else bv[:, 0]
        dlc[:, t] = x * a[:, t] * hp
        dlv[:, t + 1] = x * bv[:, t + 1]
    dlv[:, 0] = (a[:, 0] * x * bv[:, 0]) if T > 0 else 0.0
    return dlc, dlv


# ---------------------------------------------------------------------------
# matrix_scan / matrix_affine_scan
# ---------------------------------------------------------------------------


def affine_scan(A, Bm):
    """``H_t = A_t H_{t-1} + B_t`` per (b, n): returns ``(Abar, Bbar)``."""
    A = np.asarray(A, np.float64)
    Bm = np.asarray(Bm, np.float64)
    Bn, T, n, k, _ = A.shape
    Abar = np.empty_like(A)
    Bbar = np.empty_like(Bm)
    Pa = np.broadcast_to(np.eye(k), (Bn, n, k, k)).copy()
    Pb = np.zeros_like(Bm[:, 0])
    for t in range(T):
        Pa = A[:, t] @ Pa
        Pb = A[:, t] @ Pb + Bm[:, t]
        Abar[:, t] = Pa
        Bbar[:, t] = Pb
    return Abar, Bbar


def affine_scan_bwd(A, Bm, gAbar, gBbar):
    """Adjoint of :func:`affine_scan`.

    ``X_t = G_t + A_{t+1}^T X_{t+1}`` (both streams);
    ``dA_t = XA_t Abar_{t-1}^T + XB_t Bbar_{t-1}^T``, ``dB_t = XB_t``.
    """
    A = np.asarray(A, np.float64)
    Abar, Bbar = affine_scan(A, Bm)
    gAbar = np.asarray(gAbar, np.float64)
    gBbar = np.asarray(gBbar, np.float64)
    Bn, T, n, k, _ = A.shape
    dA = np.empty_like(A)
    dB = np.empty_like(np.asarray(Bm, np.float64))
    XA = np.zeros_like(gAbar[:, 0])
    XB = np.zeros_like(gBbar[:, 0])
    eye = np.broadcast_to(np.eye(k), (Bn, n, k, k))
    for t in range(T - 1, -1, -1):
        if t + 1 < T:
            At = np.swapaxes(A[:, t + 1], -1, -2)
            XA = gAbar[:, t] + At @ XA
            XB = gBbar[:, t] + At @ XB
        else:
            XA = gAbar[:, t].copy()
            XB = gBbar[:, t].copy()
        Ap = Abar[:, t - 1] if t > 0 else eye
        Bp = Bbar[:, t - 1] if t > 0 else np.zeros_like(XB)
        dA[:, t] = XA @ np.swapaxes(Ap, -1, -2) + XB @ np.swapaxes(Bp, -1, -2)
        dB[:, t] = XB
    return dA, dB


# ---------------------------------------------------------------------------
# angle-fused rotation scan
# ---------------------------------------------------------------------------


def angle_round_tables(perm, sgn, p2p):
    """Per-round index arrays; a position whose partner is itself is left untouched."""
    perm = np.asarray(perm, np.int64)
    sgn = np.asarray(sgn, np.float64)
    p2p = np.asarray(p2p, np.int64)
    active = perm != np.arange(perm.shape[1])[None, :]
    return perm, sgn, p2p, active


def _round_apply(v, c, s, perm_r, sgn_r, act_r):
    """One round: ``v'[p] = c_p v[p] + sgn_p s_p v[perm_p]`` on active positions."""
    out = c * v + sgn_r * s * v[..., perm_r]
    return np.where(act_r, out, v)


def angle_scan(theta, scale, gamma, b, h0, perm, sgn, p2p, has_scale, has_decay):
    """``h_t = gamma_t R(theta_t) S_t h_{t-1} + b_t`` (reference kernel semantics).

    ``theta`` ``(B,T,n,R,half)``, ``scale``/``gamma`` ``(B,T,n)``, ``b`` ``(B,T,n,k)``,
    ``h0`` ``(B,n,k)``; ``S_t`` multiplies coordinate 1 by ``scale`` when
    ``has_scale``.  Returns h ``(B,T,n,k)``.
    """
    theta = np.asarray(theta, np.float64)
    perm, sgn, p2p, act = angle_round_tables(perm, sgn, p2p)
    R = theta.shape[3]
    b = np.asarray(b, np.float64)
    k = b.shape[-1]
    v = np.asarray(h0, np.float64).copy()
    out = np.empty_like(b)
    for t in range(theta.shape[1]):
        if has_scale:
            v[..., 1] = v[..., 1] * scale[:, t]
        for r in range(R):
            ang = theta[:, t, :, r, :][..., p2p[r]]
            v = _round_apply(v, np.cos(ang), np.sin(ang), perm[r], sgn[r], act[r])
        if has_decay:
            v = v * np.asarray(gamma[:, t], np.float64)[..., None]
        v = v + b[:, t]
        out[:, t] = v
    assert out.shape[-1] == k
    return out


def angle_transition_matrices(theta, scale, gamma, perm, sgn, p2p, has_scale, has_decay):
    """Brute-force materialisation of every ``M_t`` ``(B,T,n,k,k)`` by applying the rounds
    to the identity (row-update rule of ``src/mingru/min_gru.py:2583-2602``)."""
    theta = np.asarray(theta, np.float64)
    perm, sgn, p2p, act = angle_round_tables(perm, sgn, p2p)
    Bn, T, n, R, _ = theta.shape
    k = perm.shape[1]
    M = np.broadcast_to(np.eye(k), (Bn, T, n, k, k)).copy()
    if has_scale:
        M[..., 1] = M[..., 1] * np.asarray(scale, np.float64)[..., None]
    for r in range(R):
        ang = theta[:, :, :, r, :][..., p2p[r]]  # (B,T,n,k)
        c = np.cos(ang)[..., None]
        s = np.sin(ang)[..., None]
        rows = M[..., perm[r], :]
        new = c * M + (sgn[r][:, None] * s) * rows
        M = np.where(act[r][:, None], new, M)
    if has_decay:
        M = M * np.asarray(gamma, np.float64)[..., None, None]
    return M


def angle_scan_bwd(theta, scale, gamma, b, h0, perm, sgn, p2p, has_scale, has_decay, gh):
    """Adjoint of :func:`angle_scan`: ``(dtheta, dscale, dgamma, db, dh0)``."""
    theta = np.asarray(theta, np.float64)
    scale = np.asarray(scale, np.float64)
    gamma = np.asarray(gamma, np.float64)
    h0 = np.asarray(h0, np.float64)
    gh = np.asarray(gh, np.float64)
    perm, sgn, p2p, act = angle_round_tables(perm, sgn, p2p)
    Bn, T, n, R, half = theta.shape
    h = angle_scan(theta, scale, gamma, b, h0, perm, sgn, p2p, has_scale, has_decay)
    dtheta = np.zeros_like(theta)
    dscale = np.zeros_like(scale)
    dgamma = np.zeros_like(gamma)
    db = np.empty_like(h)
    ghat = np.zeros_like(h0)
    for t in range(T - 1, -1, -1):
        hp = h[:, t - 1] if t > 0 else h0
        vs = [hp.copy()]
        if has_scale:
            vs[0][..., 1] = vs[0][..., 1] * scale[:, t]
        for r in range(R):
            ang = theta[:, t, :, r, :][..., p2p[r]]
            vs.append(_round_apply(vs[r], np.cos(ang), np.sin(ang), perm[r], sgn[r], act[r]))
        gbar = gh[:, t] + ghat
        db[:, t] = gbar
        if has_decay:
            dgamma[:, t] = np.sum(gbar * vs[R], axis=-1)
            adj = gamma[:, t][..., None] * gbar
        else:
            adj = gbar
        for r in range(R - 1, -1, -1):
            ang = theta[:, t, :, r, :][..., p2p[r]]
            c, s = np.cos(ang), np.sin(ang)
            v = vs[r]
            vp = v[..., perm[r]]
            g_pos = np.where(act[r], adj * (-s * v + sgn[r] * c * vp), 0.0)
            for m in range(half):
                dtheta[:, t, :, r, m] = np.sum(np.where(p2p[r] == m, g_pos, 0.0), axis=-1)
            tmp = np.where(act[r], sgn[r] * s * adj, 0.0)
            back = np.zeros_like(adj)
            # adjoint of v[perm[p]] reads: scatter tmp[p] into position perm[p]
            for p in range(perm.shape[1]):
                back[..., perm[r, p]] += tmp[..., p]
            adj = np.where(act[r], c * adj, adj) + back
        if has_scale:
            dscale[:, t] = adj[..., 1] * hp[..., 1]
            adj = adj.copy()
            adj[..., 1] = adj[..., 1] * scale[:, t]
        ghat = adj
    return dtheta, dscale, dgamma, db, ghat


# ---------------------------------------------------------------------------
# DeltaMinGRU delta rule
# ---------------------------------------------------------------------------


def delta_sequential(Q, K, V, beta, H0):
    """Token-by-token delta rule on kernel layouts (reference ``step``, ``:3611-3688``).

    ``Q`` ``(B,h,T,dk)``, ``K`` ``(B,h,T,nh,dk)``, ``V`` ``(B,h,T,nh,dv)``,
    ``beta`` ``(B,h,T,nh)``, ``H0`` ``(B,h,dk,dv)``.  Returns ``y (B,h,T,dv)``, ``H_T``.
    """
    Q, K, V, beta = (np.asarray(x, np.float64) for x in (Q, K, V, beta))
    H = np.asarray(H0, np.float64).copy()
    Bn, nhd, T, dk = Q.shape
    nh = K.shape[3]
    y = np.empty(V.shape[:3] + (V.shape[-1],))
    for t in range(T):
        for j in range(nh):
            k = K[:, :, t, j]
            v = V[:, :, t, j]
            bt = beta[:, :, t, j][..., None, None]
            kH = np.einsum("bhk,bhkv->bhv", k, H)
            H = H + bt * np.einsum("bhk,bhv->bhkv", k, v - kH)
        y[:, :, t] = np.einsum("bhk,bhkv->bhv", Q[:, :, t], H)
    return y, H


def _solve_unit_lower(Tm, R):
    """Forward substitution for unit-lower-triangular ``Tm`` (batched)."""
    X = np.array(R, np.float64, copy=True)
    M = Tm.shape[-1]
    for i in range(M):
        if i:
            X[..., i, :] -= np.einsum("...l,...lv->...v", Tm[..., i, :i], X[..., :i, :])
    return X


def _solve_unit_upper(Tm, R):
    X = np.array(R, np.float64, copy=True)
    M = Tm.shape[-1]
    for i in range(M - 1, -1, -1):
        if i < M - 1:
            X[..., i, :] -= np.einsum("...l,...lv->...v", Tm[..., i, i + 1:], X[..., i + 1:, :])
    return X


def _chunk(K, V, beta, Q, s, e):
    Bn, nhd, _, nh, dk = K.shape
    dv = V.shape[-1]
    C = e - s
    M = nh * C
    Kc = K[:, :, s:e].reshape(Bn, nhd, M, dk)
    Vc = V[:, :, s:e].reshape(Bn, nhd, M, dv)
    bc = beta[:, :, s:e].reshape(Bn, nhd, M)
    Qc = Q[:, :, s:e]
    strict = np.tril(np.ones((M, M)), -1)
    read = np.repeat(np.tril(np.ones((C, C))), nh, axis=1)
    return Kc, Vc, bc, Qc, strict, read


def delta_chunked(Q, K, V, beta, H0, chunk_size):
    """Chunked-WY forward (reference ``_forward_chunked``, ``:3152-3255``).

    Returns ``y (B,h,T,dv)``, ``H_T`` and the start-of-chunk states ``Hbound``.
    """
    Q, K, V, beta = (np.asarray(x, np.float64) for x in (Q, K, V, beta))
    H = np.asarray(H0, np.float64).copy()
    T = Q.shape[2]
    ys, bounds = [], []
    for s in range(0, T, chunk_size):
        e = min(s + chunk_size, T)
        Kc, Vc, bc, Qc, strict, read = _chunk(K, V, beta, Q, s, e)
        bounds.append(H.copy())
        Tm = np.eye(Kc.shape[2]) + (Kc @ np.swapaxes(Kc, -1, -2)) * bc[..., None, :] * strict
        U = _solve_unit_lower(Tm, Vc - Kc @ H)
        y = Qc @ H + ((Qc @ np.swapaxes(Kc, -1, -2)) * bc[..., None, :] * read) @ U
        H = H + np.swapaxes(Kc, -1, -2) @ (bc[..., None] * U)
        ys.append(y)
    return np.concatenate(ys, axis=2), H, np.stack(bounds, axis=2)


def delta_chunked_bwd(Q, K, V, beta, H0, chunk_size, dy, dHT):
    """Reverse-chunk backward (reference ``_delta_backward_torch``, ``triton_scans.py:473-605``).

    Returns ``(dQ, dK, dV, dbeta, dH0)``.
    """
    Q, K, V, beta, dy, dHT = (np.asarray(x, np.float64) for x in (Q, K, V, beta, dy, dHT))
    _, _, Hb = delta_chunked(Q, K, V, beta, H0, chunk_size)
    Bn, nhd, T, dk = Q.shape
    nh = K.shape[3]
    dv = V.shape[-1]
    tr = lambda x: np.swapaxes(x, -1, -2)  # noqa: E731
    dQ = np.zeros_like(Q)
    dK = np.zeros_like(K)
    dV = np.zeros_like(V)
    dbeta = np.zeros_like(beta)
    dH = dHT.copy()
    n_chunks = Hb.shape[2]
    for c in range(n_chunks - 1, -1, -1):
        s = c * chunk_size
        e = min(s + chunk_size, T)
        C = e - s
        M = nh * C
        Kc, Vc, bc, Qc, strict, read = _chunk(K, V, beta, Q, s, e)
        Hc = Hb[:, :, c]
        dyc = dy[:, :, s:e]
        KK = Kc @ tr(Kc)
        Tm = np.eye(M) + KK * bc[..., None, :] * strict
        U = _solve_unit_lower(Tm, Vc - Kc @ Hc)
        S = Qc @ tr(Kc)
        P = S * bc[..., None, :] * read
        dQc = dyc @ tr(Hc)
        dHc = tr(Qc) @ dyc
        dP = dyc @ tr(U)
        dU = tr(P) @ dyc
        dK_loc = (bc[..., None] * U) @ tr(dH)
        dbU = Kc @ dH
        dU = dU + bc[..., None] * dbU
        db_loc = np.sum(U * dbU, axis=-1)
        dHc = dHc + dH
        dS = dP * bc[..., None, :] * read
        db_loc = db_loc + np.sum(dP * S * read, axis=-2)
        dQc = dQc + dS @ Kc
        dK_loc = dK_loc + tr(dS) @ Qc
        G = _solve_unit_upper(tr(Tm), dU)
        dT = -(G @ tr(U))
        dK_loc = dK_loc - G @ tr(Hc)
        dHc = dHc - tr(Kc) @ G
        dKK = dT * bc[..., None, :] * strict
        db_loc = db_loc + np.sum(dT * KK * strict, axis=-2)
        dK_loc = dK_loc + dKK @ Kc + tr(dKK) @ Kc
        dQ[:, :, s:e] = dQc
        dK[:, :, s:e] = dK_loc.reshape(Bn, nhd, C, nh, dk)
        dV[:, :, s:e] = G.reshape(Bn, nhd, C, nh, dv)
        dbeta[:, :, s:e] = db_loc.reshape(Bn, nhd, C, nh)
        dH = dHc
    return dQ, dK, dV, dbeta, dH


def delta_gated_sequential(Q, K, V, beta, log_gamma, H0, return_states=False):
    """Decay-active delta rule, token by token (reference ``step``, ``:3611-3688``).

    Per token ``t``: ``H <- exp(log_gamma[..., t]) H``, then the ``nh`` micro-steps
    ``H <- H + beta k (v - H^T k)^T``, then ``y_t = H^T q_t``.  Layouts as
    ``delta_sequential`` plus ``log_gamma`` ``(B,h,T)``.  Returns ``y``, ``H_T``
    (and, with ``return_states``, the state before every token's decay,
    ``(B,h,T,dk,dv)``).
    """
    Q, K, V, beta, lg = (np.asarray(x, np.float64) for x in (Q, K, V, beta, log_gamma))
    H = np.asarray(H0, np.float64).copy()
    T = Q.shape[2]
    nh = K.shape[3]
    y = np.empty(V.shape[:3] + (V.shape[-1],))
    states = np.empty(H.shape[:2] + (T,) + H.shape[2:]) if return_states else None
    for t in range(T):
        if return_states:
            states[:, :, t] = H
        H = np.exp(lg[:, :, t])[..., None, None] * H
        for j in range(nh):
            k = K[:, :, t, j]
            bt = beta[:, :, t, j][..., None, None]
            u = V[:, :, t, j] - np.einsum("bhk,bhkv->bhv", k, H)
            H = H + bt * np.einsum("bhk,bhv->bhkv", k, u)
        y[:, :, t] = np.einsum("bhk,bhkv->bhv", Q[:, :, t], H)
    return (y, H, states) if return_states else (y, H)


def delta_gated_sequential_bwd(Q, K, V, beta, log_gamma, H0, dy, dHT):
    """Adjoint of ``delta_gated_sequential``: ``(dQ, dK, dV, dbeta, dlog_gamma, dH0)``.

    Reverse over tokens: ``dH += q_t dy_t^T`` (``dq_t = H_t dy_t``), then the
    micro-steps in reverse, with ``H' = H + beta k u^T``, ``u = v - H^T k``:
    ``dv = beta dH'^T k``, ``dbeta = k^T dH' u``,
    ``dk = beta (dH' u - H dH'^T k)``, ``dH = dH' - beta k (k^T dH')``; then the
    decay: ``dlog_gamma_t = gamma_t <dH, H_{t-1}>``, ``dH_{t-1} = gamma_t dH``.
    """
    Q, K, V, beta, lg, dy, dHT = (np.asarray(x, np.float64)
                                  for x in (Q, K, V, beta, log_gamma, dy, dHT))
    _, _, states = delta_gated_sequential(Q, K, V, beta, lg, H0, return_states=True)
    T = Q.shape[2]
    nh = K.shape[3]
    dQ, dK, dV, dbeta, dlg = (np.zeros_like(x) for x in (Q, K, V, beta, lg))
    dH = dHT.copy()
    for t in range(T - 1, -1, -1):
        g = np.exp(lg[:, :, t])[..., None, None]
        # Recompute the token's micro-step inputs from the state before its decay.
        Hs = [g * states[:, :, t]]
        for j in range(nh):
            k = K[:, :, t, j]
            u = V[:, :, t, j] - np.einsum("bhk,bhkv->bhv", k, Hs[-1])
            Hs.append(Hs[-1] + beta[:, :, t, j][..., None, None] * np.einsum("bhk,bhv->bhkv", k, u))
        dQ[:, :, t] = np.einsum("bhkv,bhv->bhk", Hs[-1], dy[:, :, t])
        dH = dH + np.einsum("bhk,bhv->bhkv", Q[:, :, t], dy[:, :, t])
        for j in range(nh - 1, -1, -1):
            H = Hs[j]
            k = K[:, :, t, j]
            bt = beta[:, :, t, j]
            u = V[:, :, t, j] - np.einsum("bhk,bhkv->bhv", k, H)
            dHk = np.einsum("bhkv,bhk->bhv", dH, k)  # dH'^T k
            dV[:, :, t, j] = bt[..., None] * dHk
            dbeta[:, :, t, j] = np.einsum("bhv,bhv->bh", dHk, u)
            dK[:, :, t, j] = bt[..., None] * (np.einsum("bhkv,bhv->bhk", dH, u)
                                              - np.einsum("bhkv,bhv->bhk", H, dHk))
            dH = dH - bt[..., None, None] * np.einsum("bhk,bhv->bhkv", k, dHk)
        dlg[:, :, t] = g[..., 0, 0] * np.einsum("bhkv,bhkv->bh", dH, states[:, :, t])
        dH = g * dH
    return dQ, dK, dV, dbeta, dlg, dH
