"""minGRU mixers, scan primitives and the ``MINGRU_SCAN`` dispatch seam.

This module is the public, eager half of the package.  It keeps the surface of
chris-santiago/minGRU (``src/mingru/min_gru.py``) unchanged -- the five mixers,
``MinGRUBlock``/``MinGRUStack`` and the four scan primitives keep their names,
signatures, shapes and error behaviour -- while the GPU backend behind the seam
is :mod:`mingru_amd.hip_scans`: hand-written HIP kernels for gfx950 reached
through a C-ABI shared library.

Dispatch contract (reference ``src/mingru/min_gru.py:85-118, 149-319``):

* ``MINGRU_SCAN`` is read from the environment on every call.
* ``"auto"`` (default): GPU tensors run the HIP kernel when the backend is
  available and the call is inside the kernel envelope; otherwise the eager
  implementation runs after a once-per-process warning naming the reason.
  CPU tensors always run eager and never import the backend.
* ``"eager"``: always the eager implementation; the backend is never imported.
* ``"hip"`` (``"triton"`` is accepted as an alias so scripts written for the
  reference keep working): always the HIP kernel; a decline raises
  ``RuntimeError`` instead of downgrading silently.

The eager implementations below are the CPU path and the reference semantics
the kernels are tested against: Heinsen's log-space scan for
``parallel_scan_log`` and Hillis-Steele doubling over the affine monoid for the
other three scans (reference ``:755-807, 1454-1655``).
"""

from __future__ import annotations

import math
import os
import warnings
from typing import Literal

import torch
import torch.nn as nn
import torch.nn.functional as F

__all__ = [
    "MinGRU",
    "SignedMinGRU",
    "RotationMinGRU",
    "GivensMinGRU",
    "DeltaMinGRU",
    "MinGRUBlock",
    "MinGRUStack",
    "parallel_scan_log",
    "linear_scan",
    "matrix_scan",
    "matrix_affine_scan",
]

Decay = Literal["fixed", "learnable"] | None

# ---------------------------------------------------------------------------
# Dispatch seam
# ---------------------------------------------------------------------------

#: Forcing mode name of this backend.  ``"triton"`` is kept as an alias.
_NATIVE_MODE = "hip"
_VALID_SCAN_MODES = ("auto", "eager", _NATIVE_MODE, "triton")
_BACKEND_MODULE = "mingru_amd.hip_scans"

_warned_scan_fallback = False
_warned_angle_fallback = False
_warned_delta_fallback = False
_warned_delta_decay_fallback = False
_warned_gate_fallback = False
_warned_mingru_gate_fallback = False
_warned_step_fallback = False

# DeltaMinGRU ``auto`` region.  The HIP chunked-WY kernel beats the eager GPU
# loop from a handful of chunks upward at every head size of its envelope, so
# ``auto`` engages it whenever the sequence spans at least
# ``_DELTA_AUTO_MIN_T_CHUNKS`` chunks and ``d_k`` is at most
# ``_DELTA_AUTO_MAX_DK`` (the envelope maximum).  Reference counterpart:
# ``src/mingru/min_gru.py:145-146`` (whose region is narrower because its
# Triton kernel only won at d_k <= 16).
_DELTA_AUTO_MIN_T_CHUNKS = 2
_DELTA_AUTO_MAX_DK = 64


def _resolve_scan_mode(is_cuda: bool) -> str | None:
    """Validate ``MINGRU_SCAN`` and apply the eager / CPU-``auto`` short-circuit.

    Mirrors ``src/mingru/min_gru.py:149-187``.  Returns ``"auto"`` or the
    forcing mode if a native path should be attempted, ``None`` if the caller
    should run its eager implementation (``eager``, or ``auto`` on CPU: no
    import, no warning).

    Raises
    ------
    ValueError
        If ``MINGRU_SCAN`` is not a recognised mode.
    """
    mode = os.environ.get("MINGRU_SCAN", "auto")
    if mode not in _VALID_SCAN_MODES:
        raise ValueError(f"MINGRU_SCAN must be one of {_VALID_SCAN_MODES} (got {mode!r})")
    if mode == "eager":
        return None
    if mode == "auto" and not is_cuda:
        return None
    return mode


def _resolve_native_dispatch(mode: str, op_label: str, call) -> tuple[object | None, str | None]:
    """Lazy backend import, per-op call and ``ScanFallback`` funnel.

    Counterpart of ``_resolve_triton_dispatch`` (``src/mingru/min_gru.py:190-252``).
    ``call(backend)`` performs the availability checks and the kernel call and
    raises only ``backend.ScanFallback`` on decline.  Returns
    ``(result, None)`` when a kernel ran and ``(None, reason)`` when it did not
    (``auto`` only); the forcing mode raises ``RuntimeError`` instead.
    """
    reason = None
    try:
        from mingru_amd import hip_scans
    except ImportError as exc:
        reason = f"hip_scans not importable: {exc}"
    else:
        try:
            return call(hip_scans), None
        except hip_scans.ScanFallback as exc:
            reason = str(exc)
    if mode != "auto":
        raise RuntimeError(
            f"MINGRU_SCAN={mode} requested for {op_label} but the HIP backend is unavailable: "
            f"{reason}"
        )
    return None, reason


# Reference name, kept so code written against the reference seam still resolves.
_resolve_triton_dispatch = _resolve_native_dispatch


def _dispatch_scan(name: str, *args: torch.Tensor):
    """Run the HIP kernel registered for scan ``name``, or return ``None``.

    Called as the first statement of each of the four scan functions
    (``src/mingru/min_gru.py:255-319``).  A non-``None`` return is the scan's
    result; ``None`` means "run the eager body".
    """
    mode = _resolve_scan_mode(args[0].is_cuda)
    if mode is None:
        return None

    def _call(backend):
        status = backend.available()
        if status is not True:
            raise backend.ScanFallback(str(status))
        if name not in backend.SCAN_IMPLS:
            raise backend.ScanFallback(f"no HIP kernel registered for {name!r}")
        return backend.SCAN_IMPLS[name](*args)

    result, reason = _resolve_native_dispatch(mode, repr(name), _call)
    if reason is None:
        return result
    global _warned_scan_fallback
    if not _warned_scan_fallback:
        warnings.warn(
            f"MINGRU_SCAN=auto fell back to the eager scan implementation for {name!r} "
            f"despite CUDA inputs: {reason}",
            stacklevel=3,
        )
        _warned_scan_fallback = True
    return None


def _angle_scan_should_try(is_cuda: bool) -> bool:
    """Import-free pre-gate for the angle-fused module path (reference ``:322-350``)."""
    return _resolve_scan_mode(is_cuda) is not None


def _dispatch_angle_scan(
    theta: torch.Tensor,
    scale: torch.Tensor,
    gamma: torch.Tensor,
    b: torch.Tensor,
    h0: torch.Tensor,
    perm: torch.Tensor,
    sgn: torch.Tensor,
    p2p: torch.Tensor,
    *,
    has_scale: int,
    has_decay: int,
):
    """Run the angle-fused rotation scan, or return ``None`` for the eager forward.

    Same contract as ``src/mingru/min_gru.py:353-439``: ``theta``
    ``(B, T, n, R, half)``, ``scale``/``gamma`` ``(B, T, n)``, ``b``
    ``(B, T, n, k)``, ``h0`` ``(B, n, k)`` and plane metadata
    ``perm``/``sgn``/``p2p`` ``(R, k)``.  Returns ``h`` ``(B, T, n, k)``.
    """
    mode = _resolve_scan_mode(theta.is_cuda)
    if mode is None:
        return None

    def _call(backend):
        status = backend.available()
        if status is not True:
            raise backend.ScanFallback(str(status))
        if not hasattr(backend, "angle_scan_impl"):
            raise backend.ScanFallback("no angle-fused HIP kernel registered")
        return backend.angle_scan_impl(
            theta, scale, gamma, b, h0, perm, sgn, p2p, has_scale=has_scale, has_decay=has_decay
        )

    result, reason = _resolve_native_dispatch(mode, "the angle-fused mixer path", _call)
    if reason is None:
        return result
    global _warned_angle_fallback
    if not _warned_angle_fallback:
        warnings.warn(
            "MINGRU_SCAN=auto fell back to the eager mixer forward (angle-fused path) "
            f"despite CUDA inputs: {reason}",
            stacklevel=3,
        )
        _warned_angle_fallback = True
    return None


def _dispatch_angle_gated_scan(theta, u, gamma, z, hpre, h0, perm, sgn, p2p, *, has_scale: int,
                               has_decay: int):
    """Run the angle-fused scan with the mixer's heads (``b = sigmoid(z) * hpre``,
    ``scale = tanh(u)``) formed in the kernel, or return ``None``.

    No reference counterpart: the reference forms the heads eagerly
    (``src/mingru/min_gru.py:2261-2262, 2719``) and calls ``_dispatch_angle_scan``
    (``:353-439``), which is what ``None`` leads to.  Any decline (a schedule the
    fused heads do not cover, a missing backend) returns ``None`` silently in every
    mode: the caller's ``_dispatch_angle_scan`` then applies the mode's rules.
    """
    mode = _resolve_scan_mode(theta.is_cuda)
    if mode is None:
        return None
    try:
        from mingru_amd import hip_scans as backend
    except ImportError:
        return None
    if not hasattr(backend, "angle_gated_scan_impl") or backend.available() is not True:
        return None
    try:
        return backend.angle_gated_scan_impl(theta, u, gamma, z, hpre, h0, perm, sgn, p2p,
                                             has_scale=has_scale, has_decay=has_decay)
    except backend.ScanFallback:
        return None


def _dispatch_signed_gate_scan(
    s: torch.Tensor, z: torch.Tensor, hpre: torch.Tensor, h0: torch.Tensor, *, coupled: bool,
    dt: torch.Tensor | None = None, lam: torch.Tensor | None = None,
):
    """Run SignedMinGRU's coefficients and scan as one fused kernel, or return ``None``.

    The reference has no fused path here; its mixer computes ``a, b`` eagerly
    and calls ``linear_scan`` (``src/mingru/min_gru.py:1788-1857``), which is
    what ``None`` falls back to.  With time decay, ``dt`` (B, T) and the rate
    ``lam`` give ``a * exp(-lam * dt)`` (``:1807-1813``) inside the kernel.  Mode
    handling follows the other fast paths: ``eager`` and CPU ``auto`` return
    ``None`` silently, ``auto`` warns once on a decline, the forcing mode raises.
    Returns ``h`` ``(B, T, D)``.
    """
    mode = _resolve_scan_mode(s.is_cuda)
    if mode is None:
        return None

    def _call(backend):
        status = backend.available()
        if status is not True:
            raise backend.ScanFallback(str(status))
        if not hasattr(backend, "signed_gate_scan_impl"):
            raise backend.ScanFallback("no fused SignedMinGRU gate kernel registered")
        if dt is None:
            return backend.signed_gate_scan_impl(s, z, hpre, h0, coupled=coupled)
        return backend.signed_gate_scan_impl(s, z, hpre, h0, coupled=coupled, dt=dt, lam=lam)

    result, reason = _resolve_native_dispatch(mode, "the fused SignedMinGRU gate path", _call)
    if reason is None:
        return result
    global _warned_gate_fallback
    if not _warned_gate_fallback:
        warnings.warn(
            "MINGRU_SCAN=auto fell back to the eager SignedMinGRU coefficients "
            f"(fused gate path) despite CUDA inputs: {reason}",
            stacklevel=3,
        )
        _warned_gate_fallback = True
    return None


def _dispatch_mingru_gate_scan(k: torch.Tensor, hpre: torch.Tensor, log_h0: torch.Tensor,
                               dt: torch.Tensor | None = None, lam: torch.Tensor | None = None):
    """Run MinGRU's log-space coefficients and scan as one fused kernel, or return ``None``.

    The reference has no fused path here; its mixer forms ``-softplus(k)``,
    ``-softplus(-k) + log_g(hpre)`` eagerly and calls ``parallel_scan_log``
    (``src/mingru/min_gru.py:1366-1397``), which is what ``None`` falls back
    to.  With time decay the log coefficient gains ``-lam * dt`` (``:1383-1393``)
    inside the kernel.  Mode handling as for ``_dispatch_signed_gate_scan``.
    Returns ``h`` ``(B, T, D)``.
    """
    mode = _resolve_scan_mode(k.is_cuda)
    if mode is None:
        return None

    def _call(backend):
        status = backend.available()
        if status is not True:
            raise backend.ScanFallback(str(status))
        if not hasattr(backend, "mingru_gate_scan_impl"):
            raise backend.ScanFallback("no fused MinGRU gate kernel registered")
        if dt is None:
            return backend.mingru_gate_scan_impl(k, hpre, log_h0)
        return backend.mingru_gate_scan_impl(k, hpre, log_h0, dt, lam)

    result, reason = _resolve_native_dispatch(mode, "the fused MinGRU gate path", _call)
    if reason is None:
        return result
    global _warned_mingru_gate_fallback
    if not _warned_mingru_gate_fallback:
        warnings.warn(
            "MINGRU_SCAN=auto fell back to the eager MinGRU coefficients "
            f"(fused gate path) despite CUDA inputs: {reason}",
            stacklevel=3,
        )
        _warned_mingru_gate_fallback = True
    return None


def _dispatch_step(what: str, is_cuda: bool, call):
    """Shared mode handling of the streaming decode kernels: run ``call(backend)`` or
    return ``None`` for the eager step body.

    The reference's ``step()`` bodies are eager only (``src/mingru/min_gru.py:
    1399-1448, 3611-3688``).  ``eager`` and CPU ``auto`` stay eager silently;
    CUDA ``auto`` warns once on a decline; the forcing mode raises.
    """
    mode = _resolve_scan_mode(is_cuda)
    if mode is None:
        return None

    def _call(backend):
        status = backend.available()
        if status is not True:
            raise backend.ScanFallback(str(status))
        return call(backend)

    result, reason = _resolve_native_dispatch(mode, what, _call)
    if reason is None:
        return result
    global _warned_step_fallback
    if not _warned_step_fallback:
        warnings.warn(
            f"MINGRU_SCAN=auto ran the eager step() despite CUDA inputs ({what}): {reason}",
            stacklevel=4,
        )
        _warned_step_fallback = True
    return None


def _dispatch_gate_step(kind: str, p0, p1, p2, gamma, h_prev):
    """One fused decode step ``h = gamma a h_prev + b`` (MinGRU / SignedMinGRU), or
    ``None`` for the eager body."""

    def call(backend):
        if not hasattr(backend, "gate_step_impl"):
            raise backend.ScanFallback("no gate step kernel registered")
        return backend.gate_step_impl(kind, p0, p1, p2, gamma, h_prev)

    return _dispatch_step("the fused gate step", h_prev.is_cuda, call)


def _dispatch_delta_step(H, q, ks, vs, betas, log_gamma):
    """One fused DeltaMinGRU decode step on ``(B, n_heads, ...)`` layouts, returning
    ``(y (B, n_heads, d_v), H_new)``, or ``None`` for the eager body."""

    def call(backend):
        if not hasattr(backend, "delta_step_impl"):
            raise backend.ScanFallback("no DeltaMinGRU step kernel registered")
        K = torch.stack(ks, dim=2)
        V = torch.stack(vs, dim=2)
        beta = torch.stack(betas, dim=2)
        return backend.delta_step_impl(H, q, K, V, beta, log_gamma)

    return _dispatch_step("the fused DeltaMinGRU step", H.is_cuda, call)


def _delta_scan_should_try(is_cuda: bool, *, T: int, chunk_size: int, d_k: int) -> bool:
    """Import-free pre-gate for the DeltaMinGRU chunked-WY kernel (reference ``:442-500``).

    Under ``auto`` the kernel is tried only inside the region described at
    ``_DELTA_AUTO_MIN_T_CHUNKS``; out-of-region ``auto`` stays eager silently.
    The forcing mode ignores the region.
    """
    mode = _resolve_scan_mode(is_cuda)
    if mode is None:
        return False
    if mode == "auto" and not (
        T >= _DELTA_AUTO_MIN_T_CHUNKS * chunk_size and d_k <= _DELTA_AUTO_MAX_DK
    ):
        return False
    return True


def _dispatch_delta_scan(
    q: torch.Tensor,
    ks: list[torch.Tensor],
    vs: list[torch.Tensor],
    betas: list[torch.Tensor],
    H: torch.Tensor,
    *,
    chunk_size: int,
) -> tuple[torch.Tensor, torch.Tensor] | None:
    """Run the DeltaMinGRU chunked-WY kernel, or return ``None`` for eager.

    Owns the layout change in both directions (reference ``:503-609``):
    ``q`` ``(B, T, n_heads, d_k)`` and the ``nh`` per-micro-step lists become
    ``Q`` ``(B, n_heads, T, d_k)``, ``K`` ``(B, n_heads, T, nh, d_k)``,
    ``V`` ``(B, n_heads, T, nh, d_v)``, ``beta`` ``(B, n_heads, T, nh)``; the
    kernel's ``y`` ``(B, n_heads, T, d_v)`` is returned as
    ``(B, T, n_heads, d_v)`` together with ``H_T`` ``(B, n_heads, d_k, d_v)``.
    """
    mode = _resolve_scan_mode(q.is_cuda)
    if mode is None:
        return None

    def _call(backend):
        status = backend.available()
        if status is not True:
            raise backend.ScanFallback(str(status))
        if not hasattr(backend, "delta_scan_impl"):
            raise backend.ScanFallback("no DeltaMinGRU HIP kernel registered")
        K = torch.stack(ks, dim=2).permute(0, 3, 1, 2, 4)
        V = torch.stack(vs, dim=2).permute(0, 3, 1, 2, 4)
        beta = torch.stack(betas, dim=2).permute(0, 3, 1, 2)
        Q = q.permute(0, 2, 1, 3)
        y, H_T = backend.delta_scan_impl(Q, K, V, beta, H, chunk_size=chunk_size)
        return y.permute(0, 2, 1, 3), H_T

    result, reason = _resolve_native_dispatch(mode, "the DeltaMinGRU chunked-WY path", _call)
    if reason is None:
        return result
    global _warned_delta_fallback
    if not _warned_delta_fallback:
        warnings.warn(
            "MINGRU_SCAN=auto fell back to the eager DeltaMinGRU forward (chunked-WY path) "
            f"despite CUDA inputs: {reason}",
            stacklevel=3,
        )
        _warned_delta_fallback = True
    return None


def _dispatch_delta_gated_scan(
    q: torch.Tensor,
    ks: list[torch.Tensor],
    vs: list[torch.Tensor],
    betas: list[torch.Tensor],
    log_gamma: torch.Tensor,
    H: torch.Tensor,
    *,
    chunk_size: int,
) -> tuple[torch.Tensor, torch.Tensor] | None:
    """Run DeltaMinGRU's decay-active forward on the gated chunked-WY kernel, or
    return ``None`` for the eager ``_forward_chunked_gated``.

    The reference has no kernel here; its guard (``src/mingru/min_gru.py:612-668``)
    raises under the forcing mode and warns once under CUDA ``auto``.  This seam
    keeps that contract for a backend that declines: the forcing mode raises, CUDA
    ``auto`` warns once and runs eager, ``eager`` and CPU ``auto`` run eager
    silently.  Layouts as ``_dispatch_delta_scan``, plus ``log_gamma``
    ``(B, n_heads, T)`` (``log gamma_t = -lambda f(dt_t)`` per head and token).
    """
    mode = _resolve_scan_mode(q.is_cuda)
    if mode is None:
        return None

    def _call(backend):
        status = backend.available()
        if status is not True:
            raise backend.ScanFallback(str(status))
        if not hasattr(backend, "delta_gated_scan_impl"):
            raise backend.ScanFallback("decay has no HIP kernel registered")
        K = torch.stack(ks, dim=2).permute(0, 3, 1, 2, 4)
        V = torch.stack(vs, dim=2).permute(0, 3, 1, 2, 4)
        beta = torch.stack(betas, dim=2).permute(0, 3, 1, 2)
        Q = q.permute(0, 2, 1, 3)
        y, H_T = backend.delta_gated_scan_impl(Q, K, V, beta, log_gamma, H,
                                               chunk_size=chunk_size)
        return y.permute(0, 2, 1, 3), H_T

    result, reason = _resolve_native_dispatch(
        mode, "DeltaMinGRU's decay-active forward (gated chunked-WY path)", _call
    )
    if reason is None:
        return result
    global _warned_delta_decay_fallback
    if not _warned_delta_decay_fallback:
        warnings.warn(
            "MINGRU_SCAN=auto is running DeltaMinGRU's decay-active forward eagerly on CUDA "
            f"input: {reason}",
            stacklevel=3,
        )
        _warned_delta_decay_fallback = True
    return None


def _cached_plane_meta_per_device(obj, attr: str, device: torch.device, build):
    """Per-instance, per-device cache of constant plane metadata (reference ``:671-703``)."""
    cache = getattr(obj, attr, None)
    if cache is not None and cache[0].device == device:
        return cache
    meta = tuple(t.to(device) for t in build())
    setattr(obj, attr, meta)
    return meta


# ---------------------------------------------------------------------------
# Positive activation and the four scan primitives (eager bodies)
# ---------------------------------------------------------------------------


def g(x: torch.Tensor) -> torch.Tensor:
    """``x + 0.5`` for ``x >= 0``, ``sigmoid(x)`` below (reference ``:706-724``)."""
    return torch.where(x >= 0, x + 0.5, torch.sigmoid(x))


def log_g(x: torch.Tensor) -> torch.Tensor:
    """``log(g(x))`` with finite values and gradients everywhere (reference ``:727-752``).

    The unselected ``x >= 0`` branch is fed a clamped copy so ``log`` never
    sees a negative argument (``torch.where`` evaluates both branches).
    """
    pos = x >= 0
    x_pos = torch.where(pos, x, torch.zeros_like(x))
    return torch.where(pos, torch.log(x_pos + 0.5), -F.softplus(-x))


def parallel_scan_log(log_coeffs: torch.Tensor, log_values: torch.Tensor) -> torch.Tensor:
    """Heinsen log-space scan for ``h_t = a_t h_{t-1} + b_t`` with positive terms.

    Parameters
    ----------
    log_coeffs : torch.Tensor
        ``(B, T, D)``, ``log(a_t)``.
    log_values : torch.Tensor
        ``(B, T + 1, D)``; slot 0 is ``log(h_0)``, slots ``1..T`` are ``log(b_t)``.

    Returns
    -------
    torch.Tensor
        ``(B, T, D)``, the states ``h_1..h_T``.

    Reference: ``src/mingru/min_gru.py:755-807``.  On GPU the HIP kernel runs the
    same recurrence in linear space with fp32 state (all terms are positive, so
    no cancellation), which is closer to fp64 than the fp32 log-space body.
    """
    result = _dispatch_scan("parallel_scan_log", log_coeffs, log_values)
    if result is not None:
        return result
    cum = F.pad(torch.cumsum(log_coeffs, dim=1), (0, 0, 1, 0))
    log_h = cum + torch.logcumsumexp(log_values - cum, dim=1)
    return torch.exp(log_h)[:, 1:]


def linear_scan(a: torch.Tensor, b: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Scan ``h_t = a_t h_{t-1} + b_t`` with signed coefficients.

    Returns ``(A, Bc)``, each ``(B, T, D)``: ``A_t`` is the running product of
    ``a`` and ``Bc_t`` the ``h_0 = 0`` solution, so ``h_t = A_t h_0 + Bc_t``.
    Eager body: Hillis-Steele doubling over ``(A1,B1) o (A2,B2) = (A2 A1, A2 B1 + B2)``
    (reference ``src/mingru/min_gru.py:1454-1510``).
    """
    result = _dispatch_scan("linear_scan", a, b)
    if result is not None:
        return result
    T = a.size(1)
    A, Bc = a, b
    step = 1
    while step < T:
        A_shift = F.pad(A, (0, 0, step, 0), value=1.0)[:, :T]
        B_shift = F.pad(Bc, (0, 0, step, 0), value=0.0)[:, :T]
        Bc = A * B_shift + Bc
        A = A * A_shift
        step *= 2
    return A, Bc


def matrix_scan(M: torch.Tensor, b: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Scan ``h_t = M_t h_{t-1} + b_t`` over 2x2 blocks.

    ``M`` ``(B, T, n, 2, 2)``, ``b`` ``(B, T, n, 2)``.  Returns ``(A, Bc)`` with
    ``A_t = M_t ... M_1`` and ``Bc_t`` the ``h_0 = 0`` solution (reference
    ``src/mingru/min_gru.py:1513-1581``).
    """
    result = _dispatch_scan("matrix_scan", M, b)
    if result is not None:
        return result
    Bn, T, n = M.shape[:3]
    eye = torch.eye(2, dtype=M.dtype, device=M.device)
    A, Bc = M, b
    step = 1
    while step < T:
        A_prev = torch.cat([eye.expand(Bn, step, n, 2, 2), A[:, : T - step]], dim=1)
        B_prev = torch.cat([b.new_zeros(Bn, step, n, 2), Bc[:, : T - step]], dim=1)
        Bc = torch.einsum("btnij,btnj->btni", A, B_prev) + Bc
        A = A @ A_prev
        step *= 2
    return A, Bc


def matrix_affine_scan(A: torch.Tensor, Bm: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Scan ``H_t = A_t H_{t-1} + B_t`` with ``k x k`` transitions and ``k x v`` injections.

    ``A`` ``(B, T, n, k, k)``, ``Bm`` ``(B, T, n, k, v)``.  Returns
    ``(Abar, Bbar)`` of the same shapes (reference ``src/mingru/min_gru.py:1584-1655``).
    """
    result = _dispatch_scan("matrix_affine_scan", A, Bm)
    if result is not None:
        return result
    Ab, Bb = A, Bm
    T = A.size(1)
    step = 1
    while step < T:
        newA = torch.einsum("btnij,btnjk->btnik", Ab[:, step:], Ab[:, :-step])
        newB = torch.einsum("btnij,btnjv->btniv", Ab[:, step:], Bb[:, :-step]) + Bb[:, step:]
        Ab = torch.cat([Ab[:, :step], newA], dim=1)
        Bb = torch.cat([Bb[:, :step], newB], dim=1)
        step *= 2
    return Ab, Bb


# ---------------------------------------------------------------------------
# Time decay (shared by all mixers)
# ---------------------------------------------------------------------------

_DELTA_T_POSINF_CAP = 1e10
_DECAY_MIXER_KWARGS = ("decay", "decay_rate", "log1p_delta")
_DECAY_SATURATION_WARN_THRESHOLD = 1e4


def _match_delta_t_dtype(delta_t: torch.Tensor | None, module: nn.Module) -> torch.Tensor | None:
    """Cast ``delta_t`` to ``module``'s parameter dtype (reference ``:917-945``)."""
    if delta_t is None:
        return None
    dtype = next(module.parameters()).dtype
    return delta_t if delta_t.dtype == dtype else delta_t.to(dtype)


def _normalize_delta_t(
    delta_t: torch.Tensor, canonical_ndim: int, log1p_delta: bool = False
) -> tuple[torch.Tensor, bool]:
    """Squeeze, sanitise (NaN->0, +inf->cap, negatives->0) and optionally ``log1p``.

    Returns the normalised tensor and, on CPU only, whether invalid entries were
    present (reference ``:948-1015``).
    """
    if delta_t.dim() == canonical_ndim + 1:
        if delta_t.size(-1) != 1:
            raise ValueError(
                f"delta_t with {delta_t.dim()} dims must have a trailing size-1 dimension to "
                f"squeeze (got shape {tuple(delta_t.shape)})"
            )
        delta_t = delta_t.squeeze(-1)
    elif delta_t.dim() != canonical_ndim:
        raise ValueError(
            f"delta_t must have {canonical_ndim} dims (or {canonical_ndim + 1} with a trailing "
            f"size-1 dim to squeeze); got shape {tuple(delta_t.shape)}"
        )
    has_invalid = False
    if delta_t.device.type == "cpu":
        has_invalid = bool(((delta_t < 0) | delta_t.isnan() | delta_t.isinf()).any())
    delta_t = delta_t.nan_to_num(nan=0.0, posinf=_DELTA_T_POSINF_CAP).clamp(min=0)
    if log1p_delta:
        delta_t = torch.log1p(delta_t)
    return delta_t, has_invalid


def _validate_delta_t_pairing(decay: Decay, delta_t: torch.Tensor | None) -> None:
    """Decay on <=> ``delta_t`` given (reference ``:1018-1044``)."""
    if decay is not None and delta_t is None:
        raise ValueError(f"decay={decay!r} requires delta_t to be provided.")
    if decay is None and delta_t is not None:
        raise ValueError(
            "delta_t was provided but decay is disabled (decay=None); construct the mixer "
            "with decay='fixed' or decay='learnable' to use delta_t."
        )


def _warn_once_invalid_delta_t(module: nn.Module, has_invalid: bool) -> None:
    if has_invalid and not module._warned_negative_dt:
        warnings.warn(
            "delta_t contains negative, NaN, or infinite entries (likely out-of-order or "
            "corrupted timestamps); sanitizing to finite, non-negative values.",
            stacklevel=3,
        )
        module._warned_negative_dt = True


class DecayMixin:
    """``gamma = exp(-lambda * f(delta_t))`` decay contract (reference ``:1016-1210``).

    ``_init_decay`` is called last in each mixer's ``__init__`` and draws no
    random numbers, so ``decay=None`` modules have the same parameters, in the
    same order, as modules without decay.
    """

    def _init_decay(self, decay: Decay, decay_rate: float, log1p_delta: bool, num_channels: int):
        if decay not in (None, "fixed", "learnable"):
            raise ValueError(f"decay must be None, 'fixed', or 'learnable' (got {decay!r})")
        if decay is not None and decay_rate <= 0:
            raise ValueError(
                f"decay_rate must be > 0 when decay={decay!r} is enabled (got {decay_rate!r}); "
                "lambda must be strictly positive so gamma stays in (0, 1]."
            )
        self.decay = decay
        self.decay_rate = decay_rate
        self.log1p_delta = log1p_delta
        self._warned_negative_dt = False
        if decay == "fixed":
            self.register_buffer("decay_rate_buf", torch.full((), decay_rate))
        elif decay == "learnable":
            self.rho = nn.Parameter(torch.full((num_channels,), math.log(math.expm1(decay_rate))))

    def _decay_lambda(self) -> torch.Tensor:
        if self.decay == "fixed":
            return self.decay_rate_buf
        return F.softplus(self.rho)

    def _decay_gamma(self, dt: torch.Tensor) -> torch.Tensor:
        return torch.exp(-self._decay_lambda() * dt.unsqueeze(-1))

    def _prepare_decay(self, delta_t: torch.Tensor | None, canonical_ndim: int):
        _validate_delta_t_pairing(self.decay, delta_t)
        if delta_t is None:
            return None
        dt, has_invalid = _normalize_delta_t(delta_t, canonical_ndim, self.log1p_delta)
        _warn_once_invalid_delta_t(self, has_invalid)
        return dt


# ---------------------------------------------------------------------------
# Mixers
# ---------------------------------------------------------------------------


class MinGRU(DecayMixin, nn.Module):
    """Log-space minGRU (reference ``src/mingru/min_gru.py:1213-1451``).

    ``z = sigmoid(Linear_z x)``, ``h~ = g(Linear_h x)``,
    ``h_t = (1 - z_t) h_{t-1} + z_t h~_t``, run through ``parallel_scan_log``.
    ``h_0`` is a real, non-negative state (default ``g(0) = 0.5``).
    """

    def __init__(
        self,
        input_size: int,
        hidden_size: int,
        bias: bool = True,
        learnable_h0: bool = False,
        decay: Decay = None,
        decay_rate: float = 1.0,
        log1p_delta: bool = False,
    ):
        super().__init__()
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.linear_z = nn.Linear(input_size, hidden_size, bias=bias)
        self.linear_h = nn.Linear(input_size, hidden_size, bias=bias)
        self.h0_pre = nn.Parameter(torch.zeros(1, 1, hidden_size)) if learnable_h0 else None
        self._init_decay(decay, decay_rate, log1p_delta, hidden_size)

    def _default_log_h0(self, B: int, x: torch.Tensor) -> torch.Tensor:
        if self.h0_pre is not None:
            return log_g(self.h0_pre).expand(B, 1, self.hidden_size)
        return torch.full((B, 1, self.hidden_size), 0.5, dtype=x.dtype, device=x.device).log()

    def forward(self, x, h_0=None, delta_t=None):
        B = x.size(0)
        if h_0 is None:
            log_h_0 = self._default_log_h0(B, x)
        else:
            torch._assert_async(
                (h_0 >= 0).all(),
                "h_0 must be a non-negative real hidden state (an output of forward()/step()), "
                "not a pre-activation.",
            )
            log_h_0 = h_0.clamp_min(torch.finfo(h_0.dtype).tiny).log()
        k = self.linear_z(x)
        dt = self._prepare_decay(delta_t, canonical_ndim=2)
        h_pre = self.linear_h(x)
        # Coefficients (with the decay, if any) and scan in one kernel where the native
        # backend takes it.
        if dt is None:
            h = _dispatch_mingru_gate_scan(k, h_pre, log_h_0)
        else:
            h = _dispatch_mingru_gate_scan(k, h_pre, log_h_0, dt, self._decay_lambda())
        if h is not None:
            return h
        log_z = -F.softplus(-k)
        log_coeffs = -F.softplus(k)
        if dt is not None:
            log_coeffs = log_coeffs - self._decay_lambda() * dt.unsqueeze(-1)
        log_tilde_h = log_g(h_pre)
        return parallel_scan_log(log_coeffs, torch.cat([log_h_0, log_z + log_tilde_h], dim=1))

    @torch.no_grad()
    def step(self, x_t, h_prev=None, delta_t=None):
        if h_prev is None:
            if self.h0_pre is not None:
                h_prev = g(self.h0_pre)[:, 0].expand(x_t.size(0), self.hidden_size)
            else:
                h_prev = x_t.new_full((x_t.size(0), self.hidden_size), 0.5)
        k = self.linear_z(x_t)
        h_pre = self.linear_h(x_t)
        dt = self._prepare_decay(delta_t, canonical_ndim=1)
        gamma = self._decay_gamma(dt) if dt is not None else None
        h = _dispatch_gate_step("mingru", k, h_pre, None, gamma, h_prev)
        if h is not None:
            return h
        z = torch.sigmoid(k)
        h_tilde = g(h_pre)
        a = 1 - z
        if gamma is not None:
            a = gamma * a
        return a * h_prev + z * h_tilde

    def extra_repr(self) -> str:
        return f"input_size={self.input_size}, hidden_size={self.hidden_size}"


class SignedMinGRU(DecayMixin, nn.Module):
    """Signed diagonal minGRU on ``linear_scan`` (reference ``:1658-1906``).

    ``a = tanh(Linear_s x)`` (times ``1 - z`` when ``coupled``),
    ``b = sigmoid(Linear_z x) * Linear_h x``; ``h = A * h_0 + Bc``.
    """

    def __init__(
        self,
        input_size: int,
        hidden_size: int,
        bias: bool = True,
        learnable_h0: bool = False,
        coupled: bool = False,
        decay: Decay = None,
        decay_rate: float = 1.0,
        log1p_delta: bool = False,
    ):
        super().__init__()
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.coupled = coupled
        self.linear_z = nn.Linear(input_size, hidden_size, bias=bias)
        self.linear_h = nn.Linear(input_size, hidden_size, bias=bias)
        self.linear_s = nn.Linear(input_size, hidden_size, bias=bias)
        self.h0 = nn.Parameter(torch.zeros(1, 1, hidden_size)) if learnable_h0 else None
        self._init_decay(decay, decay_rate, log1p_delta, hidden_size)

    def _coeffs(self, x, dt=None):
        return self._coeffs_from(self.linear_z(x), self.linear_h(x), self.linear_s(x), dt)

    def _coeffs_from(self, z_pre, h_pre, s_pre, dt=None):
        z = torch.sigmoid(z_pre)
        tanh_s = torch.tanh(s_pre)
        a = (1 - z) * tanh_s if self.coupled else tanh_s
        b = z * h_pre
        if dt is not None:
            a = self._decay_gamma(dt) * a
        return a, b

    def forward(self, x, h_0=None, delta_t=None):
        if h_0 is None:
            h_0 = (
                self.h0.expand(x.size(0), 1, self.hidden_size)
                if self.h0 is not None
                else x.new_zeros(x.size(0), 1, self.hidden_size)
            )
        dt = self._prepare_decay(delta_t, canonical_ndim=2)
        z_pre, h_pre, s_pre = self.linear_z(x), self.linear_h(x), self.linear_s(x)
        # GPU fast path: gates (with the decay, if any), scan and h = A h0 + Bc in one
        # fused kernel.
        if dt is None:
            h = _dispatch_signed_gate_scan(s_pre, z_pre, h_pre, h_0, coupled=self.coupled)
        else:
            h = _dispatch_signed_gate_scan(s_pre, z_pre, h_pre, h_0, coupled=self.coupled,
                                           dt=dt, lam=self._decay_lambda())
        if h is not None:
            return h
        a, b = self._coeffs_from(z_pre, h_pre, s_pre, dt)
        A, Bc = linear_scan(a, b)
        return A * h_0 + Bc

    @torch.no_grad()
    def step(self, x_t, h_prev=None, delta_t=None):
        if h_prev is None:
            h_prev = (
                self.h0[:, 0].expand(x_t.size(0), self.hidden_size)
                if self.h0 is not None
                else x_t.new_zeros(x_t.size(0), self.hidden_size)
            )
        dt = self._prepare_decay(delta_t, canonical_ndim=1)
        z_pre, h_pre, s_pre = self.linear_z(x_t), self.linear_h(x_t), self.linear_s(x_t)
        gamma = self._decay_gamma(dt) if dt is not None else None
        kind = "signed_coupled" if self.coupled else "signed"
        h = _dispatch_gate_step(kind, s_pre, z_pre, h_pre, gamma, h_prev)
        if h is not None:
            return h
        a, b = self._coeffs_from(z_pre, h_pre, s_pre, dt)
        return a * h_prev + b

    def extra_repr(self) -> str:
        return (
            f"input_size={self.input_size}, hidden_size={self.hidden_size}, coupled={self.coupled}"
        )


class RotationMinGRU(DecayMixin, nn.Module):
    """2x2 block-rotation minGRU (reference ``:1909-2362``).

    Per block ``M_t = R(theta_t) diag(1, tanh(u_t))`` (times ``gamma_t`` with
    decay), ``b_t = sigmoid(Linear_z x) * Linear_h x``; optional straight-through
    angle snapping to multiples of ``2 pi / K``.  On GPU the angle-fused kernel
    runs it from the angles without materialising ``M``.
    """

    def __init__(
        self,
        input_size: int,
        hidden_size: int,
        bias: bool = True,
        snap: tuple[int, ...] | None = (2, 3, 4, 6),
        decay: Decay = None,
        decay_rate: float = 1.0,
        log1p_delta: bool = False,
    ):
        super().__init__()
        if hidden_size % 2 != 0:
            raise ValueError(
                f"RotationMinGRU requires an even hidden_size (got {hidden_size}); "
                "state is n = hidden_size / 2 planar 2D blocks."
            )
        if snap is not None and (len(snap) == 0 or any(k < 1 for k in snap)):
            raise ValueError(f"snap must be None or a non-empty tuple of positive ints (got {snap!r})")
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.n_blocks = hidden_size // 2
        self.snap = snap
        self.linear_z = nn.Linear(input_size, hidden_size, bias=bias)
        self.linear_h = nn.Linear(input_size, hidden_size, bias=bias)
        self.linear_theta = nn.Linear(input_size, self.n_blocks, bias=bias)
        self.linear_u = nn.Linear(input_size, self.n_blocks, bias=bias)
        self.h0 = nn.Parameter(torch.randn(1, 1, hidden_size) * 0.5)
        if snap is not None:
            self.register_buffer(
                "snap_step",
                torch.tensor([2 * math.pi / snap[j % len(snap)] for j in range(self.n_blocks)]),
            )
        self._init_decay(decay, decay_rate, log1p_delta, self.n_blocks)

    def _angle(self, x):
        theta = self.linear_theta(x)
        if self.snap is not None:
            snapped = torch.round(theta / self.snap_step) * self.snap_step
            theta = theta + (snapped - theta).detach()
        return theta

    def _coeffs(self, x, dt=None):
        theta = self._angle(x)
        c, s = torch.cos(theta), torch.sin(theta)
        d = torch.tanh(self.linear_u(x))
        M = torch.stack(
            [torch.stack([c, -s * d], dim=-1), torch.stack([s, c * d], dim=-1)], dim=-2
        )
        if dt is not None:
            M = self._decay_gamma(dt).unsqueeze(-1).unsqueeze(-1) * M
        z = torch.sigmoid(self.linear_z(x))
        b = (z * self.linear_h(x)).reshape(*x.shape[:-1], self.n_blocks, 2)
        return M, b

    def forward(self, x, h_0=None, delta_t=None):
        B, T, _ = x.shape
        if h_0 is None:
            h_0 = self.h0.expand(B, 1, self.hidden_size)
        h0_blocks = h_0.reshape(B, self.n_blocks, 2)
        dt = self._prepare_decay(delta_t, canonical_ndim=2)
        fused = self._angle_fused_forward(x, h0_blocks, dt)
        if fused is not None:
            return fused
        M, b = self._coeffs(x, dt)
        A, Bc = matrix_scan(M, b)
        h = torch.einsum("btnij,bnj->btni", A, h0_blocks) + Bc
        return h.reshape(B, T, self.hidden_size)

    def _angle_plane_meta(self, device):
        """One plane per round: position 0 pairs with 1, ``R(theta)`` sign convention."""

        def build():
            return (
                torch.tensor([[1, 0]], dtype=torch.int32),
                torch.tensor([[-1.0, 1.0]], dtype=torch.float32),
                torch.tensor([[0, 0]], dtype=torch.int32),
            )

        return _cached_plane_meta_per_device(self, "_angle_meta_cache", device, build)

    def _angle_heads(self, x, dt):
        """``theta (B,T,n,1,1)``, ``scale = tanh(u) (B,T,n)``, ``gamma (B,T,n)``, ``b (B,T,n,2)``."""
        B, T, _ = x.shape
        n = self.n_blocks
        theta = self._angle(x).view(B, T, n, 1, 1)
        scale = torch.tanh(self.linear_u(x))
        b = (torch.sigmoid(self.linear_z(x)) * self.linear_h(x)).reshape(B, T, n, 2)
        if dt is not None:
            gamma = self._decay_gamma(dt).expand(B, T, n)
        else:
            gamma = torch.ones(B, T, n, dtype=x.dtype, device=x.device)
        return theta, scale, gamma, b

    def _angle_fused_forward(self, x, h0_blocks, dt):
        if not _angle_scan_should_try(x.is_cuda):
            return None
        B, T, _ = x.shape
        n = self.n_blocks
        perm, sgn, p2p = self._angle_plane_meta(x.device)
        # The heads' nonlinearities in the kernel: angle (snapped here), tanh(u) scale,
        # sigmoid(z) * h~ input.
        gamma = self._decay_gamma(dt).expand(B, T, n) if dt is not None else None
        h = _dispatch_angle_gated_scan(
            self._angle(x).view(B, T, n, 1, 1), self.linear_u(x), gamma,
            self.linear_z(x).view(B, T, n, 2), self.linear_h(x).view(B, T, n, 2), h0_blocks,
            perm, sgn, p2p, has_scale=1, has_decay=1 if dt is not None else 0,
        )
        if h is not None:
            return h.reshape(B, T, self.hidden_size)
        theta, scale, gamma, b = self._angle_heads(x, dt)
        h = _dispatch_angle_scan(
            theta, scale, gamma, b, h0_blocks, perm, sgn, p2p,
            has_scale=1, has_decay=1 if dt is not None else 0,
        )
        if h is None:
            return None
        return h.reshape(B, T, self.hidden_size)

    @torch.no_grad()
    def step(self, x_t, h_prev=None, delta_t=None):
        B = x_t.size(0)
        if h_prev is None:
            h_prev = self.h0.expand(B, 1, self.hidden_size)[:, 0]
        hp = h_prev.reshape(B, self.n_blocks, 2)
        dt = self._prepare_decay(delta_t, canonical_ndim=1)
        # Decode on the angle-fused kernel: one token with h_prev as the carried state.
        fused = self._angle_fused_forward(x_t.unsqueeze(1), hp, None if dt is None else dt[:, None])
        if fused is not None:
            return fused[:, 0]
        M, b = self._coeffs(x_t, dt)
        return (torch.einsum("bnij,bnj->bni", M, hp) + b).reshape(B, self.hidden_size)

    def extra_repr(self) -> str:
        return f"input_size={self.input_size}, hidden_size={self.hidden_size}, snap={self.snap}"


class GivensMinGRU(DecayMixin, nn.Module):
    """k-dim block rotations from brick-wall Givens rounds (reference ``:2365-2824``).

    ``M_t = G_{R-1} ... G_0``; even rounds rotate planes ``(0,1),(2,3),...``,
    odd rounds ``(1,2),...,(k-1,0)``; a rotation of plane ``(i, j)`` by
    ``theta`` maps ``row_i <- c row_i - s row_j``, ``row_j <- s row_i + c row_j``.
    """

    def __init__(
        self,
        input_size: int,
        hidden_size: int,
        bias: bool = True,
        block_size: int = 8,
        rounds: int = 3,
        decay: Decay = None,
        decay_rate: float = 1.0,
        log1p_delta: bool = False,
    ):
        super().__init__()
        if block_size % 2 != 0:
            raise ValueError(
                f"GivensMinGRU requires an even block_size (got {block_size}); brick-wall "
                "Givens rounds pair the k state dims into k/2 disjoint planes."
            )
        if hidden_size % block_size != 0:
            raise ValueError(
                f"GivensMinGRU requires hidden_size ({hidden_size}) divisible by block_size "
                f"({block_size})."
            )
        if rounds < 1:
            raise ValueError(f"GivensMinGRU requires rounds >= 1 (got {rounds}).")
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.k = block_size
        self.n_blocks = hidden_size // block_size
        self.rounds = rounds
        half = block_size // 2
        self.linear_theta = nn.Linear(input_size, self.n_blocks * rounds * half, bias=bias)
        self.linear_z = nn.Linear(input_size, hidden_size, bias=bias)
        self.linear_h = nn.Linear(input_size, hidden_size, bias=bias)
        self.h0 = nn.Parameter(torch.randn(1, 1, hidden_size) * 0.5)
        for r in range(rounds):
            first = torch.arange(r % 2, block_size, 2) % block_size
            self.register_buffer(f"_pi{r}", first)
            self.register_buffer(f"_pj{r}", (first + 1) % block_size)
        self._init_decay(decay, decay_rate, log1p_delta, self.n_blocks)

    def _coeffs(self, x, dt=None):
        lead = x.shape[:-1]
        half = self.k // 2
        theta = self.linear_theta(x).view(*lead, self.n_blocks, self.rounds, half)
        M = torch.eye(self.k, dtype=x.dtype, device=x.device).expand(
            *lead, self.n_blocks, self.k, self.k
        ).clone()
        for r in range(self.rounds):
            ii = getattr(self, f"_pi{r}")
            jj = getattr(self, f"_pj{r}")
            c = torch.cos(theta[..., r, :]).unsqueeze(-1)
            s = torch.sin(theta[..., r, :]).unsqueeze(-1)
            row_i = M[..., ii, :]
            row_j = M[..., jj, :]
            M = M.clone()
            M[..., ii, :] = c * row_i - s * row_j
            M[..., jj, :] = s * row_i + c * row_j
        if dt is not None:
            M = self._decay_gamma(dt).unsqueeze(-1).unsqueeze(-1) * M
        z = torch.sigmoid(self.linear_z(x))
        b = (z * self.linear_h(x)).reshape(*lead, self.n_blocks, self.k)
        return M, b

    def forward(self, x, h_0=None, delta_t=None):
        B, T, _ = x.shape
        if h_0 is None:
            h_0 = self.h0.expand(B, 1, self.hidden_size)
        h0_blocks = h_0.reshape(B, self.n_blocks, self.k)
        dt = self._prepare_decay(delta_t, canonical_ndim=2)
        fused = self._angle_fused_forward(x, h0_blocks, dt)
        if fused is not None:
            return fused
        M, b = self._coeffs(x, dt)
        Abar, Bbar = matrix_affine_scan(M, b.unsqueeze(-1))
        h = torch.einsum("btnij,bnj->btni", Abar, h0_blocks) + Bbar.squeeze(-1)
        return h.reshape(B, T, self.hidden_size)

    def _angle_plane_meta(self, device):
        """``perm`` (partner), ``sgn`` (-1 first member, +1 second), ``p2p`` (angle slot)."""

        def build():
            R, k = self.rounds, self.k
            perm = torch.empty(R, k, dtype=torch.int32)
            sgn = torch.empty(R, k, dtype=torch.float32)
            p2p = torch.empty(R, k, dtype=torch.int32)
            for r in range(R):
                ii = getattr(self, f"_pi{r}").cpu().tolist()
                jj = getattr(self, f"_pj{r}").cpu().tolist()
                for m, (i, j) in enumerate(zip(ii, jj)):
                    perm[r, i], perm[r, j] = j, i
                    sgn[r, i], sgn[r, j] = -1.0, 1.0
                    p2p[r, i] = p2p[r, j] = m
            return perm, sgn, p2p

        return _cached_plane_meta_per_device(self, "_angle_meta_cache", device, build)

    def _angle_heads(self, x, dt):
        """``theta (B,T,n,R,k/2)``, unit ``scale``, ``gamma (B,T,n)``, ``b (B,T,n,k)``."""
        B, T, _ = x.shape
        n, k, R = self.n_blocks, self.k, self.rounds
        theta = self.linear_theta(x).view(B, T, n, R, k // 2)
        b = (torch.sigmoid(self.linear_z(x)) * self.linear_h(x)).reshape(B, T, n, k)
        if dt is not None:
            gamma = self._decay_gamma(dt).expand(B, T, n)
        else:
            gamma = torch.ones(B, T, n, dtype=x.dtype, device=x.device)
        scale = torch.ones(B, T, n, dtype=x.dtype, device=x.device)
        return theta, scale, gamma, b

    def _angle_fused_forward(self, x, h0_blocks, dt):
        if not _angle_scan_should_try(x.is_cuda):
            return None
        B, T, _ = x.shape
        n, k, R = self.n_blocks, self.k, self.rounds
        perm, sgn, p2p = self._angle_plane_meta(x.device)
        # The sigmoid(z) * h~ input formed in the kernel (brick-wall k <= 8).
        gamma = self._decay_gamma(dt).expand(B, T, n) if dt is not None else None
        h = _dispatch_angle_gated_scan(
            self.linear_theta(x).view(B, T, n, R, k // 2), None, gamma,
            self.linear_z(x).view(B, T, n, k), self.linear_h(x).view(B, T, n, k), h0_blocks,
            perm, sgn, p2p, has_scale=0, has_decay=1 if dt is not None else 0,
        )
        if h is not None:
            return h.reshape(B, T, self.hidden_size)
        theta, scale, gamma, b = self._angle_heads(x, dt)
        h = _dispatch_angle_scan(
            theta, scale, gamma, b, h0_blocks, perm, sgn, p2p,
            has_scale=0, has_decay=1 if dt is not None else 0,
        )
        if h is None:
            return None
        return h.reshape(B, T, self.hidden_size)

    @torch.no_grad()
    def step(self, x_t, h_prev=None, delta_t=None):
        B = x_t.size(0)
        if h_prev is None:
            h_prev = self.h0.expand(B, 1, self.hidden_size)[:, 0]
        hp = h_prev.reshape(B, self.n_blocks, self.k)
        dt = self._prepare_decay(delta_t, canonical_ndim=1)
        # Decode on the angle-fused kernel: one token with h_prev as the carried state.
        fused = self._angle_fused_forward(x_t.unsqueeze(1), hp, None if dt is None else dt[:, None])
        if fused is not None:
            return fused[:, 0]
        M, b = self._coeffs(x_t, dt)
        return (torch.einsum("bnij,bnj->bni", M, hp) + b).reshape(B, self.hidden_size)

    def extra_repr(self) -> str:
        return (
            f"input_size={self.input_size}, hidden_size={self.hidden_size}, "
            f"block_size={self.k}, rounds={self.rounds}"
        )


class DeltaMinGRU(DecayMixin, nn.Module):
    """DeltaNet / DeltaProduct delta-rule mixer (reference ``:2827-3695``).

    Per head and token, for micro-steps ``j = 1..nh``:
    ``H <- (I - beta k k^T) H + beta k v^T`` with ``k`` L2-normalised and
    ``beta = 2 sigmoid(.) in (0, 2)``; readout ``y_t = H_t^T q_t``, heads
    concatenated and projected by ``out_proj``.  ``forward`` runs the
    chunked-WY (UT-transform) form; ``step`` the sequential recurrence.
    """

    carries_matrix_state: bool = True

    def __init__(
        self,
        input_size: int,
        hidden_size: int,
        bias: bool = True,
        n_heads: int = 4,
        nh: int = 1,
        d_k: int | None = None,
        d_v: int | None = None,
        chunk_size: int = 64,
        decay: Decay = None,
        decay_rate: float = 1.0,
        log1p_delta: bool = False,
    ):
        super().__init__()
        if n_heads <= 0:
            raise ValueError(f"n_heads must be positive (got {n_heads})")
        if nh <= 0:
            raise ValueError(f"nh must be positive (got {nh})")
        if chunk_size <= 0:
            raise ValueError(f"chunk_size must be positive (got {chunk_size})")
        if d_k is None and hidden_size % n_heads != 0:
            raise ValueError(
                f"hidden_size ({hidden_size}) must be divisible by n_heads ({n_heads}) when d_k "
                "is not given explicitly; d_k defaults to hidden_size // n_heads."
            )
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.n_heads = n_heads
        self.nh = nh
        self.d_k = d_k if d_k is not None else hidden_size // n_heads
        self.d_v = d_v if d_v is not None else self.d_k
        self.chunk_size = chunk_size
        self.linear_q = nn.Linear(input_size, n_heads * self.d_k, bias=bias)
        self.linear_k = nn.ModuleList(
            nn.Linear(input_size, n_heads * self.d_k, bias=bias) for _ in range(nh)
        )
        self.linear_v = nn.ModuleList(
            nn.Linear(input_size, n_heads * self.d_v, bias=bias) for _ in range(nh)
        )
        self.linear_beta = nn.ModuleList(nn.Linear(input_size, n_heads, bias=bias) for _ in range(nh))
        self.out_proj = nn.Linear(n_heads * self.d_v, hidden_size, bias=bias)
        self._warned_fp32_decay_saturation = False
        self._init_decay(decay, decay_rate, log1p_delta, num_channels=self.n_heads)

    def _coeffs(self, x):
        lead = x.shape[:-1]
        q = self.linear_q(x).view(*lead, self.n_heads, self.d_k)
        ks = [F.normalize(lin(x).view(*lead, self.n_heads, self.d_k), dim=-1) for lin in self.linear_k]
        vs = [lin(x).view(*lead, self.n_heads, self.d_v) for lin in self.linear_v]
        betas = [2 * torch.sigmoid(lin(x)) for lin in self.linear_beta]
        return q, ks, vs, betas

    @staticmethod
    def _contract_state(vec, H):
        return torch.einsum("...hk,...hkv->...hv", vec, H)

    def _micro_step(self, H, k, v, beta):
        kH = self._contract_state(k, H)
        beta = beta.unsqueeze(-1).unsqueeze(-1)
        H = H - beta * torch.einsum("...hk,...hv->...hkv", k, kH)
        return H + beta * torch.einsum("...hk,...hv->...hkv", k, v)

    @staticmethod
    def _layouts(q, ks, vs, betas):
        K = torch.stack(ks, dim=2).permute(0, 3, 1, 2, 4)
        V = torch.stack(vs, dim=2).permute(0, 3, 1, 2, 4)
        beta = torch.stack(betas, dim=2).permute(0, 3, 1, 2)
        return q.permute(0, 2, 1, 3), K, V, beta

    def _forward_chunked(self, x, H):
        """Chunked-WY forward (reference ``:3152-3255``).

        Per chunk of ``C`` tokens (``M = nh C`` micro-steps, token-major):
        ``T = I + strict_lower(K K^T * beta_col)``, ``U = T^-1 (V - K H)``,
        ``y = Q H + (Q K^T * beta_col * read_mask) U``, ``H += K^T (beta U)``.
        """
        q, ks, vs, betas = self._coeffs(x)
        Q, K, V, beta = self._layouts(q, ks, vs, betas)
        return delta_chunked_eager(Q, K, V, beta, H, self.chunk_size)

    @staticmethod
    def _span_log_decay(log_gamma):
        C = log_gamma.shape[-1]
        rows = log_gamma.unsqueeze(-2).expand(*log_gamma.shape[:-1], C, C)
        tail = torch.tril(rows).flip(-1).cumsum(-1).flip(-1)
        span = torch.cat([tail[..., 1:], tail.new_zeros(*tail.shape[:-1], 1)], dim=-1)
        return span, tail[..., 0]

    def _forward_chunked_gated(self, x, H, dt):
        """Decay-gated chunked-WY forward with span-sum factors (reference ``:3257-3448``)."""
        q, ks, vs, betas = self._coeffs(x)
        Q_all, K_all, V_all, beta_all = self._layouts(q, ks, vs, betas)
        lam = self._decay_lambda()
        log_gamma = -lam.reshape(1, -1, 1) * dt.unsqueeze(1)
        if (
            log_gamma.dtype != torch.float64
            and not self._warned_fp32_decay_saturation
            and log_gamma.device.type == "cpu"
            and bool((log_gamma < -_DECAY_SATURATION_WARN_THRESHOLD).any())
        ):
            warnings.warn(
                "delta_t gaps are large enough that lambda*delta_t exceeds "
                f"{_DECAY_SATURATION_WARN_THRESHOLD:g}, saturating the gated float32 forward; "
                "pass log1p_delta=True or rescale delta_t.",
                stacklevel=2,
            )
            self._warned_fp32_decay_saturation = True
        return delta_chunked_gated_eager(Q_all, K_all, V_all, beta_all, log_gamma, H,
                                         self.chunk_size)

    def forward(self, x, h_0=None, delta_t=None, return_state=False):
        delta_t = _match_delta_t_dtype(delta_t, self)
        dt = self._prepare_decay(delta_t, canonical_ndim=2)
        B, T, _ = x.shape
        expected = (B, 1, self.n_heads * self.d_k * self.d_v)
        if h_0 is None:
            H = x.new_zeros(B, self.n_heads, self.d_k, self.d_v)
        else:
            if tuple(h_0.shape) != expected:
                raise ValueError(f"h_0 must have shape {expected} (got {tuple(h_0.shape)})")
            H = h_0.reshape(B, self.n_heads, self.d_k, self.d_v)
        if T == 0:
            _resolve_scan_mode(x.is_cuda)
            y = x.new_zeros(B, 0, self.n_heads * self.d_v)
            H = H.clone()
        elif dt is not None:
            fused = self._delta_gated_fused_forward(x, H, dt)
            y, H = fused if fused is not None else self._forward_chunked_gated(x, H, dt)
        else:
            fused = self._delta_fused_forward(x, H)
            y, H = fused if fused is not None else self._forward_chunked(x, H)
        y = self.out_proj(y.reshape(B, T, self.n_heads * self.d_v))
        if return_state:
            return y, H.reshape(*expected)
        return y

    def _delta_gated_fused_forward(self, x, H, dt):
        if not _delta_scan_should_try(
            x.is_cuda, T=x.shape[1], chunk_size=self.chunk_size, d_k=self.d_k
        ):
            return None
        q, ks, vs, betas = self._coeffs(x)
        B, T = dt.shape
        # lambda is per head ("learnable") or one value ("fixed"): (B, n_heads, T) either way.
        log_gamma = (-self._decay_lambda().reshape(1, -1, 1) * dt.unsqueeze(1)).expand(
            B, self.n_heads, T
        )
        return _dispatch_delta_gated_scan(q, ks, vs, betas, log_gamma, H,
                                          chunk_size=self.chunk_size)

    def _delta_fused_forward(self, x, H):
        if not _delta_scan_should_try(
            x.is_cuda, T=x.shape[1], chunk_size=self.chunk_size, d_k=self.d_k
        ):
            return None
        q, ks, vs, betas = self._coeffs(x)
        return _dispatch_delta_scan(q, ks, vs, betas, H, chunk_size=self.chunk_size)

    @torch.no_grad()
    def step(self, x_t, h_prev=None, delta_t=None):
        delta_t = _match_delta_t_dtype(delta_t, self)
        dt = self._prepare_decay(delta_t, canonical_ndim=1)
        B = x_t.size(0)
        expected = (B, self.n_heads * self.d_k * self.d_v)
        if h_prev is None:
            H = x_t.new_zeros(B, self.n_heads, self.d_k, self.d_v)
        else:
            if tuple(h_prev.shape) != expected:
                raise ValueError(f"h_prev must have shape {expected} (got {tuple(h_prev.shape)})")
            H = h_prev.reshape(B, self.n_heads, self.d_k, self.d_v)
        q, ks, vs, betas = self._coeffs(x_t)
        log_gamma = None
        if dt is not None:
            log_gamma = (-self._decay_lambda() * dt.unsqueeze(-1)).expand(B, self.n_heads)
        fused = _dispatch_delta_step(H, q, ks, vs, betas, log_gamma)
        if fused is not None:
            y, H = fused
            y = self.out_proj(y.reshape(B, self.n_heads * self.d_v))
            return y, H.reshape(*expected)
        if dt is not None:
            H = self._decay_gamma(dt).unsqueeze(-1).unsqueeze(-1) * H
        for j in range(self.nh):
            H = self._micro_step(H, ks[j], vs[j], betas[j])
        y = self.out_proj(self._contract_state(q, H).reshape(B, self.n_heads * self.d_v))
        return y, H.reshape(*expected)

    def extra_repr(self) -> str:
        return (
            f"input_size={self.input_size}, hidden_size={self.hidden_size}, "
            f"n_heads={self.n_heads}, nh={self.nh}, d_k={self.d_k}, "
            f"d_v={self.d_v}, chunk_size={self.chunk_size}"
        )


def angle_scan_eager(theta, scale, gamma, b, h0, perm, sgn, p2p, *, has_scale, has_decay):
    """Angle-fused scan contract evaluated eagerly by materialising every transition.

    ``theta`` ``(B, T, n, R, half)``, ``scale``/``gamma`` ``(B, T, n)``, ``b``
    ``(B, T, n, k)``, ``h0`` ``(B, n, k)`` and the plane tables ``perm``/``sgn``/``p2p``
    ``(R, k)`` of ``_angle_plane_meta``.  Builds ``M_t = gamma_t R(theta_t) S_t``
    ``(B, T, n, k, k)`` by the modules' row-update rule (round r maps
    ``row_p <- c row_p + sgn_p s row_perm(p)`` on every position whose partner is not
    itself; reference ``src/mingru/min_gru.py:2583-2602``), runs ``matrix_affine_scan``
    and returns ``h = Abar h0 + Bbar`` ``(B, T, n, k)``: the path the reference's
    Givens/Rotation modules take when the angle kernel declines, for any schedule.
    """
    Bn, T, n, R, _ = theta.shape
    k = perm.shape[1]
    M = torch.eye(k, dtype=theta.dtype, device=theta.device).expand(Bn, T, n, k, k)
    if has_scale:
        col = torch.ones(k, dtype=theta.dtype, device=theta.device)
        col[1] = 0.0
        M = M * (col + (1.0 - col) * scale[..., None]).unsqueeze(-2)
    perm_l = perm.to(device=theta.device, dtype=torch.long)
    p2p_l = p2p.to(device=theta.device, dtype=torch.long)
    sgn_f = sgn.to(device=theta.device, dtype=theta.dtype)
    pos = torch.arange(k, device=theta.device)
    for r in range(R):
        ang = theta[:, :, :, r, :].index_select(-1, p2p_l[r]).unsqueeze(-1)
        rows = M.index_select(-2, perm_l[r])
        rotated = torch.cos(ang) * M + sgn_f[r][:, None] * torch.sin(ang) * rows
        M = torch.where((perm_l[r] != pos)[:, None], rotated, M)
    if has_decay:
        M = M * gamma[..., None, None]
    Abar, Bbar = matrix_affine_scan(M, b.unsqueeze(-1))
    return torch.einsum("btnij,bnj->btni", Abar, h0) + Bbar.squeeze(-1)


def delta_chunked_eager(Q, K, V, beta, H, chunk_size):
    """Chunked-WY delta rule on the kernel layouts (eager, any device/dtype).

    ``Q`` ``(B, h, T, d_k)``, ``K`` ``(B, h, T, nh, d_k)``, ``V``
    ``(B, h, T, nh, d_v)``, ``beta`` ``(B, h, T, nh)``, ``H`` ``(B, h, d_k, d_v)``.
    Returns ``y`` ``(B, T, h, d_v)`` and ``H_T``.  This is the loop body of
    ``DeltaMinGRU._forward_chunked`` (reference ``src/mingru/min_gru.py:3228-3255``),
    shared with the benchmark's eager-GPU leg.
    """
    B, n_heads, T, d_k = Q.shape
    nh = K.shape[3]
    d_v = V.shape[4]
    ys = []
    for s in range(0, T, chunk_size):
        e = min(s + chunk_size, T)
        C = e - s
        M = nh * C
        Kc = K[:, :, s:e].reshape(B, n_heads, M, d_k)
        Vc = V[:, :, s:e].reshape(B, n_heads, M, d_v)
        bc = beta[:, :, s:e].reshape(B, n_heads, M)
        Qc = Q[:, :, s:e]
        strict = torch.tril(Kc.new_ones(M, M), diagonal=-1)
        eye = torch.eye(M, dtype=Kc.dtype, device=Kc.device)
        T_mat = eye + (Kc @ Kc.transpose(-1, -2)) * bc.unsqueeze(-2) * strict
        U = torch.linalg.solve_triangular(T_mat, Vc - Kc @ H, upper=False, unitriangular=True)
        read = torch.tril(Qc.new_ones(C, C)).repeat_interleave(nh, dim=1)
        y = Qc @ H + ((Qc @ Kc.transpose(-1, -2)) * bc.unsqueeze(-2) * read) @ U
        H = H + Kc.transpose(-1, -2) @ (bc.unsqueeze(-1) * U)
        ys.append(y)
    return torch.cat(ys, dim=2).permute(0, 2, 1, 3), H


def delta_chunked_gated_eager(Q_all, K_all, V_all, beta_all, log_gamma, H, chunk_size):
    """Decay-gated chunked-WY delta rule on the kernel layouts (eager, any device/dtype).

    Layouts as ``delta_chunked_eager`` plus ``log_gamma`` ``(B, h, T)`` (or
    broadcastable to it).  Returns ``y`` ``(B, T, h, d_v)`` and ``H_T``.  This is the
    loop of ``DeltaMinGRU._forward_chunked_gated`` (reference
    ``src/mingru/min_gru.py:3257-3448``): every decay factor is ``exp`` of a span sum
    taken from its own terms, shared with the benchmark's eager-GPU leg.
    """
    B, n_heads, T, d_k = Q_all.shape
    nh = K_all.shape[3]
    d_v = V_all.shape[4]
    ys = []
    for s in range(0, T, chunk_size):
        e = min(s + chunk_size, T)
        C = e - s
        M = nh * C
        K = K_all[:, :, s:e].reshape(B, n_heads, M, d_k)
        V = V_all[:, :, s:e].reshape(B, n_heads, M, d_v)
        beta = beta_all[:, :, s:e].reshape(B, n_heads, M)
        Q = Q_all[:, :, s:e]
        span, logP = DeltaMinGRU._span_log_decay(log_gamma[:, :, s:e])
        span_cm = span.repeat_interleave(nh, dim=-1)
        span_mm = span_cm.repeat_interleave(nh, dim=-2)
        P_tok = torch.exp(logP)
        P_micro = P_tok.repeat_interleave(nh, dim=-1)
        strict = torch.tril(K.new_ones(M, M), diagonal=-1)
        eye = torch.eye(M, dtype=K.dtype, device=K.device)
        dec_lower = torch.exp(span_mm.masked_fill(strict == 0, float("-inf")))
        T_mat = eye + (K @ K.transpose(-1, -2)) * beta.unsqueeze(-2) * dec_lower
        U = torch.linalg.solve_triangular(
            T_mat, V - P_micro.unsqueeze(-1) * (K @ H), upper=False, unitriangular=True
        )
        read = torch.tril(Q.new_ones(C, C)).repeat_interleave(nh, dim=1)
        dec_read = torch.exp(span_cm.masked_fill(read == 0, float("-inf")))
        y = P_tok.unsqueeze(-1) * (Q @ H) + (
            (Q @ K.transpose(-1, -2)) * beta.unsqueeze(-2) * dec_read
        ) @ U
        carry = torch.exp(span_cm[:, :, -1, :])
        P_C = P_tok[:, :, -1].unsqueeze(-1).unsqueeze(-1)
        H = P_C * H + K.transpose(-1, -2) @ ((carry * beta).unsqueeze(-1) * U)
        ys.append(y)
    return torch.cat(ys, dim=2).permute(0, 2, 1, 3), H


# ---------------------------------------------------------------------------
# Block and stack
# ---------------------------------------------------------------------------


class MinGRUBlock(nn.Module):
    """Pre-norm residual block: LN -> mixer -> +x, then LN -> MLP -> +x (reference ``:3698-4008``)."""

    _MIXER_CLASSES: dict[str, tuple[type[nn.Module], bool]] = {
        "log": (MinGRU, True),
        "signed": (SignedMinGRU, True),
        "rotation": (RotationMinGRU, False),
        "givens": (GivensMinGRU, False),
        "delta": (DeltaMinGRU, False),
    }

    def __init__(
        self,
        d_model: int,
        mlp_expansion: int = 4,
        dropout: float = 0.0,
        learnable_h0: bool = False,
        mixer: str = "log",
        mixer_kwargs: dict | None = None,
    ):
        super().__init__()
        if mixer not in self._MIXER_CLASSES:
            raise ValueError(f"unknown mixer {mixer!r}; expected one of {sorted(self._MIXER_CLASSES)}")
        mixer_kwargs = dict(mixer_kwargs) if mixer_kwargs else {}
        self.norm1 = nn.LayerNorm(d_model)
        cls, accepts_h0 = self._MIXER_CLASSES[mixer]
        if accepts_h0:
            mixer_kwargs["learnable_h0"] = learnable_h0
        self.mingru = cls(d_model, d_model, **mixer_kwargs)
        self.drop = nn.Dropout(dropout)
        if mlp_expansion > 0:
            self.norm2 = nn.LayerNorm(d_model)
            self.mlp = nn.Sequential(
                nn.Linear(d_model, mlp_expansion * d_model),
                nn.GELU(),
                nn.Dropout(dropout),
                nn.Linear(mlp_expansion * d_model, d_model),
            )
        else:
            self.norm2 = None
            self.mlp = None

    def forward(self, x, h_0=None, delta_t=None):
        delta_t = _match_delta_t_dtype(delta_t, self.mingru)
        if getattr(self.mingru, "carries_matrix_state", False):
            h_seq, state = self.mingru(self.norm1(x), h_0, delta_t, return_state=True)
        else:
            h_seq = self.mingru(self.norm1(x), h_0, delta_t)
            state = h_seq[:, -1:]
        x = x + self.drop(h_seq)
        if self.mlp is not None:
            x = x + self.mlp(self.norm2(x))
        return x, state

    @torch.no_grad()
    def step(self, x_t, h_prev, delta_t=None):
        delta_t = _match_delta_t_dtype(delta_t, self.mingru)
        if getattr(self.mingru, "carries_matrix_state", False):
            y_t, state = self.mingru.step(self.norm1(x_t), h_prev, delta_t)
        else:
            y_t = self.mingru.step(self.norm1(x_t), h_prev, delta_t)
            state = y_t
        x_t = x_t + y_t
        if self.mlp is not None:
            x_t = x_t + self.mlp(self.norm2(x_t))
        return x_t, state


def _resolve_stack_mixer_spec(mixer, mixer_kwargs, n_layers):
    """Normalise ``MinGRUStack``'s ``mixer``/``mixer_kwargs`` pair (reference ``:4011-4088``)."""
    valid = MinGRUBlock._MIXER_CLASSES
    if isinstance(mixer, str):
        if mixer_kwargs:
            hits = sorted(k for k in mixer_kwargs if k in valid)
            if hits:
                raise ValueError(
                    f"mixer={mixer!r} is a single mixer name, so mixer_kwargs must be a flat dict "
                    f"of that mixer's constructor kwargs; got key(s) matching a mixer type name "
                    f"instead ({hits!r}), which is the schema for a list mixer."
                )
        return [mixer] * n_layers, {mixer: mixer_kwargs}
    if isinstance(mixer, list):
        if len(mixer) != n_layers:
            raise ValueError(f"mixer list length ({len(mixer)}) must equal n_layers ({n_layers})")
        unknown = sorted({m for m in mixer if m not in valid})
        if unknown:
            raise ValueError(
                f"unknown mixer name(s) {unknown!r} in mixer list; expected one of {sorted(valid)}"
            )
        present = set(mixer)
        if mixer_kwargs is None:
            return list(mixer), {m: None for m in present}
        bad = sorted(k for k in mixer_kwargs if k not in valid or k not in present)
        if bad:
            raise ValueError(
                f"mixer_kwargs keys must name a mixer type present in mixer={mixer!r} (one of "
                f"{sorted(present)}); got unexpected key(s) {bad!r}."
            )
        return list(mixer), {m: mixer_kwargs.get(m) for m in present}
    raise ValueError(f"mixer must be a str or list[str] (got {type(mixer).__name__})")


class MinGRUStack(nn.Module):
    """``in_proj`` -> N ``MinGRUBlock`` -> final LayerNorm (reference ``:4091-4336``)."""

    def __init__(
        self,
        input_size: int,
        d_model: int,
        n_layers: int,
        mlp_expansion: int = 4,
        dropout: float = 0.0,
        learnable_h0: bool = False,
        mixer: str | list[str] = "log",
        mixer_kwargs: dict | None = None,
        decay_layers: str = "all",
    ):
        super().__init__()
        if decay_layers not in ("all", "last"):
            raise ValueError(f"decay_layers must be 'all' or 'last' (got {decay_layers!r})")
        self.decay_layers = decay_layers
        self.in_proj = nn.Linear(input_size, d_model) if input_size != d_model else nn.Identity()
        names, kw_by_type = _resolve_stack_mixer_spec(mixer, mixer_kwargs, n_layers)
        stripped = {
            m: ({k: v for k, v in kw.items() if k not in _DECAY_MIXER_KWARGS}
                if decay_layers == "last" and kw else kw)
            for m, kw in kw_by_type.items()
        }
        n_rot = names.count("rotation")
        if n_rot > 1:
            warnings.warn(
                f"stack contains more than one 'rotation' block ({n_rot} of {n_layers}): the "
                "straight-through snap discontinuity can compound across rotation layers; "
                "multi-rotation stacks are validated only at L=2; proceeding anyway.",
                stacklevel=2,
            )
        blocks = []
        for i, name in enumerate(names):
            kw = kw_by_type[name] if i == n_layers - 1 else stripped[name]
            blocks.append(MinGRUBlock(d_model, mlp_expansion, dropout, learnable_h0, name, kw))
        self.blocks = nn.ModuleList(blocks)
        self.norm_out = nn.LayerNorm(d_model)

    def _check_delta_t_has_decay(self, delta_t):
        if not any(b.mingru.decay is not None for b in self.blocks):
            _validate_delta_t_pairing(None, delta_t)

    def forward(self, x, state=None, delta_t=None):
        if state is None:
            state = self.init_state()
        self._check_delta_t_has_decay(delta_t)
        x = self.in_proj(x)
        new_state = []
        for block, h_0 in zip(self.blocks, state):
            x, h_last = block(x, h_0, delta_t if block.mingru.decay is not None else None)
            new_state.append(h_last)
        return self.norm_out(x), new_state

    def init_state(self):
        return [None] * len(self.blocks)

    @torch.no_grad()
    def step(self, x_t, state, delta_t=None):
        self._check_delta_t_has_decay(delta_t)
        x_t = self.in_proj(x_t)
        new_state = []
        for block, h_prev in zip(self.blocks, state):
            x_t, h = block.step(x_t, h_prev, delta_t if block.mingru.decay is not None else None)
            new_state.append(h)
        return self.norm_out(x_t), new_state
