"""Seeded synthetic inputs for the five benchmark workloads of the scan hot path.

Every tensor is drawn on the CPU from a ``torch.Generator`` seeded with
``1000 + i`` for workload ``Ci`` (upstream gradients from ``2000 + i``) and can
then be copied to the GPU, so CPU and GPU paths see identical inputs.

C1  MinGRU ``parallel_scan_log``            B=4  T=1024 D=256              fp32
C2  SignedMinGRU ``linear_scan``            B=16 T=4096 D=1024             fp32
C3  RotationMinGRU 2x2 ``matrix_affine_scan`` B=16 T=4096 n=256 (and b=0 ``matrix_scan``)
C4  GivensMinGRU angle-fused, 28 lexicographic rotations  B=8 T=2048 n=64 k=8
C5  DeltaMinGRU chunked-WY  B=8 H=8 d_k=d_v=64 T=8192 C=64, bf16 inputs, fp32 state
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

C1 = dict(B=4, T=1024, D=256)
C2 = dict(B=16, T=4096, D=1024)
C3 = dict(B=16, T=4096, n=256)
C4 = dict(B=8, T=2048, n=64, k=8)
C5 = dict(B=8, H=8, T=8192, d=64, chunk=64)


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def _g(x: torch.Tensor) -> torch.Tensor:
    return torch.where(x >= 0, x + 0.5, torch.sigmoid(x))


def c1_inputs(B=4, T=1024, D=256):
    """log-coefficients / log-values as ``MinGRU.forward`` builds them
    (reference ``src/mingru/min_gru.py:1383-1397``) plus an upstream grad."""
    g = _gen(1001)
    z = torch.randn(B, T, D, generator=g)
    x = torch.randn(B, T, D, generator=g)
    h0 = _g(torch.randn(B, 1, D, generator=g))
    lc = F.logsigmoid(-z)
    lv = torch.cat([h0.log(), F.logsigmoid(z) + torch.log(_g(x))], dim=1)
    gh = torch.randn(B, T, D, generator=_gen(2001))
    return dict(log_coeffs=lc, log_values=lv, grad_h=gh)


def c1g_inputs(B=4, T=1024, D=256):
    """MinGRU pre-activations at the C1 shape for the fused gate scan:
    ``k, hpre ~ N(0,1)``, ``log h0 = log g(N(0,1))`` (B, 1, D), upstream
    ``dL/dh ~ N(0,1)``; the same distributions ``c1_inputs`` forms its log
    coefficients from."""
    g = _gen(1011)
    k = torch.randn(B, T, D, generator=g)
    hpre = torch.randn(B, T, D, generator=g)
    log_h0 = _g(torch.randn(B, 1, D, generator=g)).log()
    gh = torch.randn(B, T, D, generator=_gen(2011))
    return dict(k=k, hpre=hpre, log_h0=log_h0, grad_h=gh)


def c2_inputs(B=16, T=4096, D=1024):
    """Signed coefficients ``a = tanh(2 N(0,1))``, ``b ~ N(0,1)``, ``h0 = 0``."""
    g = _gen(1002)
    a = torch.tanh(2.0 * torch.randn(B, T, D, generator=g))
    b = torch.randn(B, T, D, generator=g)
    gh = torch.randn(B, T, D, generator=_gen(2002))
    # h = A * h0 + Bc with h0 = 0: dL/dA = gh * h0 (materialised zeros), dL/dBc = gh.
    return dict(a=a, b=b, grad_A=torch.zeros_like(gh), grad_Bc=gh)


def c2g_inputs(B=16, T=4096, D=1024):
    """SignedMinGRU pre-activations at the C2 shape for the fused gate scan:
    ``s = 2 N(0,1)`` (so ``a = tanh(s)`` is distributed as C2's), ``z, hpre ~ N(0,1)``,
    ``h0 = 0`` (B, 1, D), upstream ``dL/dh ~ N(0,1)``."""
    g = _gen(1012)
    s = 2.0 * torch.randn(B, T, D, generator=g)
    z = torch.randn(B, T, D, generator=g)
    hpre = torch.randn(B, T, D, generator=g)
    gh = torch.randn(B, T, D, generator=_gen(2012))
    return dict(s=s, z=z, hpre=hpre, h0=torch.zeros(B, 1, D), grad_h=gh)


def c3_inputs(B=16, T=4096, n=256):
    """``A = sigmoid(N) R(theta)``, theta ~ U(-pi, pi); ``b ~ N``; ``h0 ~ N``."""
    g = _gen(1003)
    theta = (torch.rand(B, T, n, generator=g) * 2 - 1) * math.pi
    s = torch.sigmoid(torch.randn(B, T, n, generator=g))
    c, sn = torch.cos(theta), torch.sin(theta)
    A = torch.stack([torch.stack([c, -sn], -1), torch.stack([sn, c], -1)], -2) * s[..., None, None]
    b = torch.randn(B, T, n, 2, 1, generator=g)
    h0 = torch.randn(B, n, 2, generator=g)
    gh = torch.randn(B, T, n, 2, generator=_gen(2003))
    # h_t = Abar_t h0 + Bbar_t: dL/dAbar_t = gh_t h0^T, dL/dBbar_t = gh_t.
    gA = gh[..., :, None] * h0[:, None, :, None, :]
    return dict(A=A, Bm=b, h0=h0, grad_Abar=gA, grad_Bbar=gh[..., None])


def lexicographic_schedule(k: int = 8):
    """``(perm, sgn, p2p)`` for one rotation per round over all pairs i<j in
    lexicographic order; positions outside a round's plane are left untouched
    (their partner is themselves)."""
    pairs = [(i, j) for i in range(k) for j in range(i + 1, k)]
    R = len(pairs)
    perm = torch.arange(k, dtype=torch.int32).repeat(R, 1)
    sgn = torch.zeros(R, k, dtype=torch.float32)
    p2p = torch.zeros(R, k, dtype=torch.int32)
    for r, (i, j) in enumerate(pairs):
        perm[r, i], perm[r, j] = j, i
        sgn[r, i], sgn[r, j] = -1.0, 1.0
    return perm, sgn, p2p


def c4_inputs(B=8, T=2048, n=64, k=8):
    """28 angles per block-token (std 0.5), decay ``sigmoid(N)``, ``b ~ N``, ``h0 ~ N``."""
    g = _gen(1004)
    R = k * (k - 1) // 2
    theta = 0.5 * torch.randn(B, T, n, R, 1, generator=g)
    gamma = torch.sigmoid(torch.randn(B, T, n, generator=g))
    b = torch.randn(B, T, n, k, generator=g)
    h0 = torch.randn(B, n, k, generator=g)
    gh = torch.randn(B, T, n, k, generator=_gen(2004))
    perm, sgn, p2p = lexicographic_schedule(k)
    return dict(theta=theta, scale=torch.ones(B, T, n), gamma=gamma, b=b, h0=h0, perm=perm,
                sgn=sgn, p2p=p2p, grad_h=gh)


def c4g_inputs(B=8, T=2048, n=64, k=8, rounds=3):
    """GivensMinGRU's brick-wall heads at the C4 shape (its default 3 rounds): angles
    ``0.5 N(0,1)`` (B, T, n, rounds, k/2), ``gamma = sigmoid(N)``, the gate and candidate
    pre-activations ``z, hpre ~ N(0,1)`` (B, T, n, k) (so ``b = sigmoid(z) * hpre``),
    ``h0 ~ N``, upstream ``dL/dh ~ N``."""
    g = _gen(1014)
    theta = 0.5 * torch.randn(B, T, n, rounds, k // 2, generator=g)
    gamma = torch.sigmoid(torch.randn(B, T, n, generator=g))
    z = torch.randn(B, T, n, k, generator=g)
    hpre = torch.randn(B, T, n, k, generator=g)
    h0 = torch.randn(B, n, k, generator=g)
    gh = torch.randn(B, T, n, k, generator=_gen(2014))
    return dict(theta=theta, gamma=gamma, z=z, hpre=hpre, h0=h0, grad_h=gh)


def c2gd_inputs(B=16, T=4096, D=1024):
    """C2g's pre-activations plus time decay: ``dt ~ U(0, 2)`` (B, T) and a per-channel
    rate ``lam ~ U(0.1, 1.1)`` (D,)."""
    inp = c2g_inputs(B, T, D)
    g = _gen(1013)
    inp["dt"] = 2.0 * torch.rand(B, T, generator=g)
    inp["lam"] = 0.1 + torch.rand(D, generator=g)
    return inp


def c5_inputs(B=8, H=8, T=8192, d=64, chunk=64, dtype=torch.bfloat16, nh=1):
    """Delta-rule heads on the kernel layouts, bf16 inputs, ``H0 = 0``; ``nh``
    micro-steps per token (DeltaProduct) give K, V (B, H, T, nh, d) and beta
    (B, H, T, nh)."""
    g = _gen(1005)
    q = torch.randn(B, H, T, d, generator=g)
    k = F.normalize(torch.randn(B, H, T, nh, d, generator=g), dim=-1)
    v = torch.randn(B, H, T, nh, d, generator=g)
    beta = torch.sigmoid(torch.randn(B, H, T, nh, generator=g))
    g2 = _gen(2005)
    dy = torch.randn(B, H, T, d, generator=g2)
    dHT = torch.randn(B, H, d, d, generator=g2)
    return dict(Q=q.to(dtype), K=k.to(dtype), V=v.to(dtype), beta=beta.to(dtype),
                H0=torch.zeros(B, H, d, d), chunk_size=chunk, grad_y=dy, grad_HT=dHT)


def c5d_inputs(B=8, H=8, T=8192, d=64, chunk=64, dtype=torch.bfloat16, nh=1):
    """C5 heads (bf16, as C5) with per-token decay for the gated delta kernels:
    ``log gamma = -0.5 U(0, 1)`` per (head, token) in fp32, the span a fixed decay
    rate of 0.5 gives over unit-scale gaps."""
    inp = c5_inputs(B, H, T, d, chunk, dtype=dtype, nh=nh)
    inp["log_gamma"] = -0.5 * torch.rand(B, H, T, generator=_gen(1015))
    return inp
