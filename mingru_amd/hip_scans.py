"""HIP backend for the ``MINGRU_SCAN`` seam (replaces the reference's ``triton_scans``).

Backend contract (reference ``src/mingru/triton_scans.py:166-177, 460,
2403-2590``), kept name for name so the seam in :mod:`mingru_amd.min_gru`
and code written against the reference work unchanged:

* ``available() -> True | str`` -- ``True`` when a gfx950 GPU is visible and
  ``libmingru_hip.so`` loads; otherwise the reason.
* ``ScanFallback`` -- the one exception a decline raises (out-of-envelope
  shape or dtype, launch failure).  The seam turns it into a warn-once eager
  fallback under ``auto`` and a ``RuntimeError`` under the forcing mode.
* ``SCAN_IMPLS[name](*args)`` -- same signature and return as the eager scan
  ``name``, differentiable through ``torch.autograd.Function`` wrappers whose
  forward and backward are single C-ABI calls.
* ``angle_scan_impl`` and ``delta_scan_impl`` -- module fast paths for
  ``RotationMinGRU``/``GivensMinGRU`` and ``DeltaMinGRU``.

Launches are asynchronous on torch's current stream; outputs and workspaces
come from torch's caching allocator on the input's device.  Double backward
is not supported (``once_differentiable``).
"""

from __future__ import annotations

import ctypes
import os
import weakref

import torch
from torch.autograd.function import once_differentiable

__all__ = [
    "available",
    "ScanFallback",
    "SCAN_IMPLS",
    "angle_scan_impl",
    "delta_scan_impl",
    "delta_gated_scan_impl",
    "signed_gate_scan_impl",
    "mingru_gate_scan_impl",
    "gate_step_impl",
    "delta_step_impl",
    "workspace_errors",
    "LookbackError",
]


class ScanFallback(Exception):
    """The HIP path declines this call; the seam falls back to eager (or raises)."""


# Block sizes the matrix kernels are compiled for (k x k transitions, k x v
# injections): the reference's envelope (``src/mingru/triton_scans.py:183``).
# k <= 4 run one plane per thread; k = 8 and 16 run one 16x16 block (two 8x8
# planes or one 16x16 plane) per wave on the matrix cores.
_AFFINE_K = frozenset({1, 2, 4, 8, 16})
_AFFINE_V = frozenset({1, 2, 4, 8, 16})

# Angle-fused kernels.  The compiled-schedule kernels (brick-wall and
# lexicographic rounds, chunk-parallel) take k in {2, 4, 8} and up to 64 rounds;
# the table-driven kernel takes any valid plane tables for k up to 16 (the
# reference's envelope, ``src/mingru/triton_scans.py:1791``).
_ANGLE_K = frozenset({2, 4, 8})
_ANGLE_MAX_ROT = 64
_ANGLE_TABLE_K = frozenset({2, 4, 8, 16})
_ANGLE_TABLE_MAX_HALF = 64
_ANGLE_TABLE_MAX_ROUNDS = 128

# DeltaMinGRU envelope (reference ``src/mingru/triton_scans.py:294-300``): chunks
# of at most 64 tokens and nh * chunk_size <= 128 micro-steps.  The kernels
# zero-pad every chunk matrix to 64 x 64, so any d_k, d_v up to 64 runs (d_k need
# not equal d_v) and one kernel tile holds at most 64 micro-steps.  A requested
# chunk with more micro-steps than that runs as tiles of floor(64 / nh) tokens
# (``_delta_tile_chunk``): the chunked-WY result does not depend on the chunk
# size in exact arithmetic (reference ``tests/test_mixers.py:767-775``), so the
# tiling changes only the rounding, which the parity bars against float64 cover.
_DELTA_MAX_DIM = 64
_DELTA_MAX_CHUNK = 64
_DELTA_MAX_MICROSTEPS = 128
_DELTA_TILE_MICROSTEPS = 64
_DELTA_DTYPES = (torch.float32, torch.bfloat16, torch.float16)

_SUPPORTED_ARCH = "gfx950"


from . import _native

_loaded = None


def _lib():
    global _loaded
    if _loaded is None:
        _loaded = _native.load()
    return _loaded


_avail_cache: dict = {}


def available() -> bool | str:
    """``True`` if the HIP kernels can run in this process, else the reason."""
    if _loaded is not None and _avail_cache.get(torch.cuda.current_device()) == _SUPPORTED_ARCH:
        return True  # this device was checked before and the library is loaded
    if not torch.cuda.is_available():
        return "CUDA/HIP device not available"
    if torch.version.hip is None:
        return "torch is not a ROCm build"
    try:
        _lib()
    except (ImportError, OSError) as exc:
        return f"HIP library not loadable: {exc}"
    dev = torch.cuda.current_device()
    arch = _avail_cache.get(dev)
    if arch is None:
        arch = torch.cuda.get_device_properties(dev).gcnArchName.split(":")[0]
        _avail_cache[dev] = arch
    if arch != _SUPPORTED_ARCH:
        return f"HIP kernels are built for {_SUPPORTED_ARCH} (device is {arch})"
    return True


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------


def _ptr(t: torch.Tensor | None) -> int:
    # Plain ints: the ctypes signatures declare void*, which converts them directly.
    return t.data_ptr() if t is not None else 0


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor) -> int:
    """torch's current stream on ``t``'s device, as the raw ``hipStream_t`` value."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def _workspace(nbytes: int, device) -> torch.Tensor:
    """Scratch whose contents on entry do not matter (the delta kernels)."""
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


# Look-back workspaces of the scan kernels, one per (device, stream).  The C ABI
# asks for a workspace that was zero-filled once and is then reused only by
# calls ordered on one stream: every launch tags its slots with a fresh epoch
# kept in the workspace header, so nothing is cleared between calls.  A larger
# request replaces the buffer with a new zero-filled one (the old one returns to
# torch's caching allocator, ordered after the work already queued on the stream).
_scan_ws: dict = {}
# Failed look-back waits recorded by workspaces since replaced by larger ones.
_retired_errors = [0]
# Workspaces created under HIP graph capture.  Their zero fill is itself captured,
# so it runs before the scan at every replay and not at capture time: such a
# workspace serves only the captured calls (never later eager calls on the stream),
# and stays alive as long as the process, since the graph may replay at any time.
_capture_ws: list = []


def _scan_workspace(nbytes: int, device) -> torch.Tensor:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    raw = _raw_stream(idx) if _raw_stream is not None else torch.cuda.current_stream(idx).cuda_stream
    key = (idx, raw)
    ws = _scan_ws.get(key)
    if ws is not None and ws.numel() >= nbytes:
        return ws
    fresh = torch.zeros(max(int(nbytes), 1 << 20), dtype=torch.uint8, device=device)
    if torch.cuda.is_current_stream_capturing():
        _capture_ws.append(fresh)
        return fresh
    if ws is not None:
        # Keep the count of waits the outgoing workspace saw give up (one stream sync,
        # only when a workspace grows).
        _retired_errors[0] += _ws_error_count(ws)
    _scan_ws[key] = fresh
    return fresh


class LookbackError(RuntimeError):
    """A look-back scan reported a failed wait (raised only under ``MINGRU_HIP_CHECK=1``)."""


def _ws_error_count(ws: torch.Tensor) -> int:
    """Failed look-back waits recorded in a scan workspace; synchronises its stream."""
    cnt = ctypes.c_uint(0)
    rc = _lib().mg_scan_workspace_errors(_ptr(ws), ctypes.byref(cnt), _stream(ws))
    _native.check(rc, "mg_scan_workspace_errors")
    return int(cnt.value)


def workspace_errors() -> int:
    """Failed look-back waits recorded so far in this process's cached scan workspaces.

    Every look-back wait is bounded: one that gives up counts an error in its
    workspace header and the kernel finishes with a partial carry, so a nonzero
    count means some result was wrong.  Synchronises each workspace's stream.
    """
    live = list(_scan_ws.values()) + list(_capture_ws)
    return _retired_errors[0] + sum(_ws_error_count(ws) for ws in live)


def _check_workspace(ws: torch.Tensor, t: torch.Tensor) -> None:
    """Under ``MINGRU_HIP_CHECK=1``: wait for the call just queued and raise
    ``LookbackError`` if its workspace recorded a failed look-back wait.  The
    workspace is then dropped, so later calls start from a fresh one."""
    if os.environ.get("MINGRU_HIP_CHECK", "0") in ("", "0"):
        return
    n = _ws_error_count(ws)
    if n:
        for key, cached in list(_scan_ws.items()):
            if cached is ws:
                del _scan_ws[key]
        raise LookbackError(
            f"HIP look-back scan on {t.device} recorded {n} failed wait(s): the results of the "
            "calls since its workspace was created are not to be trusted"
        )


class kernel_timer:
    """Context manager recording HIP events around every C-ABI launch.

    Events are recorded on the stream each call is enqueued on (torch's current
    stream), so ``records`` yields per-call device durations:
    ``[(entry_point_name, start_event, stop_event), ...]``.  Used by the
    benchmark; inactive otherwise.
    """

    active = None

    def __init__(self, prealloc: int = 512):
        self.records = []
        # Events are created here, outside any timed loop: creating one costs
        # several microseconds of host time, recording one far less.
        self._pool = [torch.cuda.Event(enable_timing=True) for _ in range(prealloc)]

    def _event(self):
        return self._pool.pop() if self._pool else torch.cuda.Event(enable_timing=True)

    def __enter__(self):
        kernel_timer.active = self
        return self

    def __exit__(self, *exc):
        kernel_timer.active = None
        return False

    def durations_ms(self):
        out: dict = {}
        for name, a, b in self.records:
            out.setdefault(name, []).append(a.elapsed_time(b))
        return out


_sizes: dict = {}


def _size(fn_name: str, *args) -> int:
    """A size query of the C ABI (workspace or state bytes), cached per arguments: the
    answer depends only on them, and each ctypes call costs microseconds of host time
    on every step of a launch-bound workload."""
    key = (fn_name,) + args
    v = _sizes.get(key)
    if v is None:
        if len(_sizes) >= 4096:
            _sizes.clear()
        v = _sizes[key] = int(getattr(_lib(), fn_name)(*args))
    return v


def _call(fn_name: str, *args) -> None:
    timer = kernel_timer.active
    if timer is not None:
        start = timer._event()
        stop = timer._event()
        start.record()
        rc = getattr(_lib(), fn_name)(*args)
        stop.record()
        timer.records.append((fn_name, start, stop))
    else:
        rc = getattr(_lib(), fn_name)(*args)
    _native.check(rc, fn_name)


def _as_f32(*ts: torch.Tensor):
    """Contiguous fp32 views of the inputs (half types are upcast; fp64 declines)."""
    out = []
    for t in ts:
        if t.dtype == torch.float64:
            raise ScanFallback("HIP scans compute in fp32; float64 inputs stay on the eager path")
        if not t.dtype.is_floating_point:
            raise ScanFallback(f"HIP scans need floating-point inputs (got {t.dtype})")
        t = t.to(torch.float32).contiguous()
        if t.data_ptr() % 16:
            t = t.clone()  # kernels use 16-byte vector accesses
        out.append(t)
    return out


def _same_device(*ts: torch.Tensor) -> None:
    dev = ts[0].device
    if dev.type != "cuda":
        raise ScanFallback("HIP scans need GPU tensors")
    for t in ts[1:]:
        if t.device != dev:
            raise ScanFallback("HIP scan inputs live on different devices")


def _funnel(what: str, fn, *args):
    """Run ``fn`` and turn any launch-side failure into ``ScanFallback``."""
    try:
        return fn(*args)
    except (ScanFallback, LookbackError):
        raise
    except Exception as exc:  # noqa: BLE001 - every launch failure becomes a decline
        raise ScanFallback(f"{what} HIP kernel failed: {exc}") from exc


# ---------------------------------------------------------------------------
# linear_scan
# ---------------------------------------------------------------------------


class _LinearScanFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, b):
        out_dtype = a.dtype
        a32, b32 = _as_f32(a, b)
        Bn, T, D = a32.shape
        A = torch.empty_like(a32)
        Bc = torch.empty_like(a32)
        ws = _scan_workspace(_size("mg_linear_scan_workspace_bytes", Bn, T, D), a32.device)
        _call("mg_linear_scan_fwd", _ptr(a32), _ptr(b32), _ptr(A), _ptr(Bc), Bn, T, D,
              _ptr(ws), ws.numel(), _stream(a32))
        _check_workspace(ws, a32)
        ctx.save_for_backward(a32, b32, A, Bc)
        ctx.out_dtype = out_dtype
        if out_dtype != torch.float32:
            return A.to(out_dtype), Bc.to(out_dtype)
        return A, Bc

    @staticmethod
    @once_differentiable
    def backward(ctx, gA, gB):
        a32, b32, A, Bc = ctx.saved_tensors
        Bn, T, D = a32.shape
        gA32, gB32 = _as_f32(gA, gB)
        da = torch.empty_like(a32)
        db = torch.empty_like(a32)
        ws = _scan_workspace(_size("mg_linear_scan_workspace_bytes", Bn, T, D), a32.device)
        _call("mg_linear_scan_bwd", _ptr(a32), _ptr(b32), _ptr(A), _ptr(Bc), _ptr(gA32),
              _ptr(gB32), _ptr(da), _ptr(db), Bn, T, D, _ptr(ws), ws.numel(), _stream(a32))
        _check_workspace(ws, a32)
        return da.to(ctx.out_dtype), db.to(ctx.out_dtype)


def _linear_scan_impl(a: torch.Tensor, b: torch.Tensor):
    """``SCAN_IMPLS['linear_scan']``: same contract as the eager ``linear_scan``."""
    if a.ndim != 3 or b.ndim != 3 or a.shape != b.shape:
        raise ScanFallback(
            f"linear_scan (a={tuple(a.shape)}, b={tuple(b.shape)}) outside the HIP envelope: "
            "need matching (B, T, D) a and b"
        )
    _same_device(a, b)
    if a.numel() == 0:
        return a.new_empty(a.shape), b.new_empty(b.shape)
    return _funnel("linear_scan", _LinearScanFn.apply, a, b)


# ---------------------------------------------------------------------------
# fused SignedMinGRU gates + linear_scan
# ---------------------------------------------------------------------------


def _decay_partials(dims, need_lam: bool, need_dt: bool, device):
    """Partial-sum buffers of the decay gradients (the kernel writes every row; the
    caller sums them), or None where the gradient is not needed."""
    Bn, T, D = dims
    dlam = (torch.empty(_lib().mg_gate_decay_dlam_rows(Bn, T, D), D, dtype=torch.float32,
                        device=device) if need_lam else None)
    ddt = (torch.empty(_lib().mg_gate_decay_ddt_rows(Bn, T, D), Bn, T, dtype=torch.float32,
                       device=device) if need_dt else None)
    return dlam, ddt


def _decay_args(dt, lam, like: torch.Tensor):
    """fp32 contiguous ``dt`` (B, T) and ``lam`` (D,) for the decay kernels."""
    Bn, T, D = like.shape
    dt32 = dt.to(torch.float32).contiguous()
    lam32 = lam.to(torch.float32).expand(D).contiguous()
    return dt32, lam32


class _SignedGateScanFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, s, z, hpre, h0, dt, lam, coupled):
        out_dtype = s.dtype
        s32, z32, hp32, h032 = _as_f32(s, z, hpre, h0)
        Bn, T, D = s32.shape
        h = torch.empty_like(s32)
        ws = _scan_workspace(_size("mg_signed_gate_scan_workspace_bytes", Bn, T, D), s32.device)
        if dt is None:
            _call("mg_signed_gate_scan_fwd", _ptr(s32), _ptr(z32), _ptr(hp32), _ptr(h032),
                  _ptr(h), Bn, T, D, int(coupled), _ptr(ws), ws.numel(), _stream(s32))
            dt32 = lam32 = None
        else:
            dt32, lam32 = _decay_args(dt, lam, s32)
            _call("mg_signed_gate_scan_decay_fwd", _ptr(s32), _ptr(z32), _ptr(hp32), _ptr(h032),
                  _ptr(dt32), _ptr(lam32), _ptr(h), Bn, T, D, int(coupled), _ptr(ws),
                  ws.numel(), _stream(s32))
        _check_workspace(ws, s32)
        ctx.save_for_backward(s32, z32, hp32, h032, h, dt32, lam32)
        ctx.coupled = bool(coupled)
        ctx.dtypes = (out_dtype, None if dt is None else dt.dtype,
                      None if lam is None else lam.dtype)
        return h if out_dtype == torch.float32 else h.to(out_dtype)

    @staticmethod
    @once_differentiable
    def backward(ctx, gh):
        s32, z32, hp32, h032, h, dt32, lam32 = ctx.saved_tensors
        Bn, T, D = s32.shape
        (gh32,) = _as_f32(gh)
        ds, dz, dhp = (torch.empty_like(s32) for _ in range(3))
        dh0 = torch.empty_like(h032)
        ws = _scan_workspace(_size("mg_signed_gate_scan_workspace_bytes", Bn, T, D), s32.device)
        od, dtd, lamd = ctx.dtypes
        if dt32 is None:
            _call("mg_signed_gate_scan_bwd", _ptr(s32), _ptr(z32), _ptr(hp32), _ptr(h032),
                  _ptr(h), _ptr(gh32), _ptr(ds), _ptr(dz), _ptr(dhp), _ptr(dh0), Bn, T, D,
                  int(ctx.coupled), _ptr(ws), ws.numel(), _stream(s32))
            _check_workspace(ws, s32)
            return ds.to(od), dz.to(od), dhp.to(od), dh0.to(od), None, None, None
        need = ctx.needs_input_grad
        dlam, ddt = _decay_partials((Bn, T, D), need[5], need[4], s32.device)
        _call("mg_signed_gate_scan_decay_bwd", _ptr(s32), _ptr(z32), _ptr(hp32), _ptr(h032),
              _ptr(dt32), _ptr(lam32), _ptr(h), _ptr(gh32), _ptr(ds), _ptr(dz), _ptr(dhp),
              _ptr(dh0), _ptr(dlam), _ptr(ddt), Bn, T, D, int(ctx.coupled), _ptr(ws),
              ws.numel(), _stream(s32))
        _check_workspace(ws, s32)
        g_dt = ddt.sum(0).to(dtd) if ddt is not None else None
        g_lam = dlam.sum(0).to(lamd) if dlam is not None else None
        return ds.to(od), dz.to(od), dhp.to(od), dh0.to(od), g_dt, g_lam, None


def _check_decay(what: str, like: torch.Tensor, dt, lam) -> None:
    if (dt is None) != (lam is None):
        raise ScanFallback(f"{what}: dt and lam must be given together")
    if dt is None:
        return
    Bn, T, D = like.shape
    if tuple(dt.shape) != (Bn, T) or not (lam.ndim == 0 or tuple(lam.shape) in ((1,), (D,))):
        raise ScanFallback(
            f"{what} decay (dt={tuple(dt.shape)}, lam={tuple(lam.shape)}) outside the HIP "
            f"envelope: need dt (B, T) and lam () or (D,)"
        )
    _same_device(like, dt, lam)


def signed_gate_scan_impl(s: torch.Tensor, z: torch.Tensor, hpre: torch.Tensor,
                          h0: torch.Tensor, *, coupled: bool, dt: torch.Tensor | None = None,
                          lam: torch.Tensor | None = None):
    """Fused SignedMinGRU coefficients + ``linear_scan``: ``h`` (B, T, D).

    No reference kernel fuses these; the arithmetic is the mixer's
    (``src/mingru/min_gru.py:1788-1857``): ``a = tanh(s)`` (times
    ``1 - sigmoid(z)`` when ``coupled``), ``b = sigmoid(z) * hpre`` and
    ``h = A * h0 + Bc`` with ``(A, Bc) = linear_scan(a, b)``, for pre-activations
    ``s, z, hpre`` (B, T, D) and ``h0`` (B, 1, D).  With time decay (the module's
    ``delta_t``, reference ``:1807-1813``) ``a`` is multiplied by
    ``exp(-lam * dt)`` inside the kernel, for the normalised ``dt`` (B, T) and the
    rate ``lam`` (a scalar, or (D,) per channel).  Differentiable in every input.
    """
    if (
        s.ndim != 3
        or z.shape != s.shape
        or hpre.shape != s.shape
        or tuple(h0.shape) != (s.shape[0], 1, s.shape[2])
    ):
        raise ScanFallback(
            f"signed gate scan (s={tuple(s.shape)}, z={tuple(z.shape)}, hpre={tuple(hpre.shape)}, "
            f"h0={tuple(h0.shape)}) outside the HIP envelope: need (B, T, D) pre-activations "
            "and a (B, 1, D) h0"
        )
    _same_device(s, z, hpre, h0)
    _check_decay("signed gate scan", s, dt, lam)
    if s.numel() == 0:
        return s.new_empty(s.shape)
    return _funnel("signed gate scan", _SignedGateScanFn.apply, s, z, hpre, h0, dt, lam,
                   bool(coupled))


# ---------------------------------------------------------------------------
# fused MinGRU gates + parallel_scan_log
# ---------------------------------------------------------------------------


class _MinGRUGateScanFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, k, hpre, log_h0, dt, lam):
        out_dtype = k.dtype
        k32, hp32, lh032 = _as_f32(k, hpre, log_h0)
        Bn, T, D = k32.shape
        h = torch.empty_like(k32)
        ws = _scan_workspace(_size("mg_mingru_gate_scan_workspace_bytes", Bn, T, D), k32.device)
        if dt is None:
            _call("mg_mingru_gate_scan_fwd", _ptr(k32), _ptr(hp32), _ptr(lh032), _ptr(h),
                  Bn, T, D, _ptr(ws), ws.numel(), _stream(k32))
            dt32 = lam32 = None
        else:
            dt32, lam32 = _decay_args(dt, lam, k32)
            _call("mg_mingru_gate_scan_decay_fwd", _ptr(k32), _ptr(hp32), _ptr(lh032),
                  _ptr(dt32), _ptr(lam32), _ptr(h), Bn, T, D, _ptr(ws), ws.numel(),
                  _stream(k32))
        _check_workspace(ws, k32)
        ctx.save_for_backward(k32, hp32, lh032, h, dt32, lam32)
        ctx.dtypes = (out_dtype, None if dt is None else dt.dtype,
                      None if lam is None else lam.dtype)
        return h if out_dtype == torch.float32 else h.to(out_dtype)

    @staticmethod
    @once_differentiable
    def backward(ctx, gh):
        k32, hp32, lh032, h, dt32, lam32 = ctx.saved_tensors
        Bn, T, D = k32.shape
        (gh32,) = _as_f32(gh)
        dk, dhp = torch.empty_like(k32), torch.empty_like(k32)
        dlh0 = torch.empty_like(lh032)
        ws = _scan_workspace(_size("mg_mingru_gate_scan_workspace_bytes", Bn, T, D), k32.device)
        od, dtd, lamd = ctx.dtypes
        if dt32 is None:
            _call("mg_mingru_gate_scan_bwd", _ptr(k32), _ptr(hp32), _ptr(lh032), _ptr(h),
                  _ptr(gh32), _ptr(dk), _ptr(dhp), _ptr(dlh0), Bn, T, D,
                  _ptr(ws), ws.numel(), _stream(k32))
            _check_workspace(ws, k32)
            return dk.to(od), dhp.to(od), dlh0.to(od), None, None
        need = ctx.needs_input_grad
        dlam, ddt = _decay_partials((Bn, T, D), need[4], need[3], k32.device)
        _call("mg_mingru_gate_scan_decay_bwd", _ptr(k32), _ptr(hp32), _ptr(lh032), _ptr(dt32),
              _ptr(lam32), _ptr(h), _ptr(gh32), _ptr(dk), _ptr(dhp), _ptr(dlh0), _ptr(dlam),
              _ptr(ddt), Bn, T, D, _ptr(ws), ws.numel(), _stream(k32))
        _check_workspace(ws, k32)
        g_dt = ddt.sum(0).to(dtd) if ddt is not None else None
        g_lam = dlam.sum(0).to(lamd) if dlam is not None else None
        return dk.to(od), dhp.to(od), dlh0.to(od), g_dt, g_lam


def mingru_gate_scan_impl(k: torch.Tensor, hpre: torch.Tensor, log_h0: torch.Tensor,
                          dt: torch.Tensor | None = None, lam: torch.Tensor | None = None):
    """Fused MinGRU coefficients + ``parallel_scan_log``: ``h`` (B, T, D).

    No reference kernel fuses these; the arithmetic is the mixer's
    (``src/mingru/min_gru.py:1366-1397``): ``log(1 - z) = -softplus(k)``,
    ``log z = -softplus(-k)``, ``log h~ = log_g(hpre)`` and
    ``h = exp(parallel_scan_log(log(1 - z), [log_h0, log z + log h~]))``, run as
    the equivalent linear recurrence ``h_t = sigmoid(-k) h_{t-1} +
    sigmoid(k) g(hpre)`` from ``h_0 = exp(log_h0)`` (all terms positive).
    ``k, hpre`` are (B, T, D) pre-activations, ``log_h0`` is (B, 1, D).  With
    time decay the log coefficient gains ``-lam * dt`` (reference ``:1383-1393``):
    the kernel multiplies ``sigmoid(-k)`` by ``exp(-lam * dt)`` for the normalised
    ``dt`` (B, T) and the rate ``lam`` (a scalar, or (D,)).  Differentiable in every
    input.
    """
    if k.ndim != 3 or hpre.shape != k.shape or tuple(log_h0.shape) != (k.shape[0], 1, k.shape[2]):
        raise ScanFallback(
            f"MinGRU gate scan (k={tuple(k.shape)}, hpre={tuple(hpre.shape)}, "
            f"log_h0={tuple(log_h0.shape)}) outside the HIP envelope: need (B, T, D) "
            "pre-activations and a (B, 1, D) log_h0"
        )
    _same_device(k, hpre, log_h0)
    _check_decay("MinGRU gate scan", k, dt, lam)
    if k.numel() == 0:
        return k.new_empty(k.shape)
    return _funnel("MinGRU gate scan", _MinGRUGateScanFn.apply, k, hpre, log_h0, dt, lam)


# ---------------------------------------------------------------------------
# parallel_scan_log
# ---------------------------------------------------------------------------


class _LogScanFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, log_coeffs, log_values):
        out_dtype = log_coeffs.dtype
        lc, lv = _as_f32(log_coeffs, log_values)
        Bn, T, D = lc.shape
        h = torch.empty_like(lc)
        # Extended-range states at every 8-step boundary, kept for the backward so it
        # can restart from values an fp32 h under- or overflows.
        hstate = None
        if any(ctx.needs_input_grad):
            nfloat = _size("mg_log_scan_state_bytes", Bn, T, D) // 4
            hstate = torch.empty(nfloat, dtype=torch.float32, device=lc.device)
        ws = _scan_workspace(_size("mg_log_scan_workspace_bytes", Bn, T, D), lc.device)
        _call("mg_log_scan_fwd", _ptr(lc), _ptr(lv), _ptr(h), _ptr(hstate), Bn, T, D, _ptr(ws),
              ws.numel(), _stream(lc))
        _check_workspace(ws, lc)
        ctx.save_for_backward(lc, lv, h, hstate)
        ctx.out_dtype = out_dtype
        return h if out_dtype == torch.float32 else h.to(out_dtype)

    @staticmethod
    @once_differentiable
    def backward(ctx, gh):
        lc, lv, h, hstate = ctx.saved_tensors
        Bn, T, D = lc.shape
        (gh32,) = _as_f32(gh)
        dlc = torch.empty_like(lc)
        dlv = torch.empty_like(lv)
        ws = _scan_workspace(_size("mg_log_scan_workspace_bytes", Bn, T, D), lc.device)
        _call("mg_log_scan_bwd", _ptr(lc), _ptr(lv), _ptr(h), _ptr(hstate), _ptr(gh32),
              _ptr(dlc), _ptr(dlv), Bn, T, D, _ptr(ws), ws.numel(), _stream(lc))
        _check_workspace(ws, lc)
        return dlc.to(ctx.out_dtype), dlv.to(ctx.out_dtype)


def _parallel_scan_log_impl(log_coeffs: torch.Tensor, log_values: torch.Tensor):
    """``SCAN_IMPLS['parallel_scan_log']``: same contract as the eager op."""
    if (
        log_coeffs.ndim != 3
        or log_values.ndim != 3
        or log_values.shape
        != (log_coeffs.shape[0], log_coeffs.shape[1] + 1, log_coeffs.shape[2])
    ):
        raise ScanFallback(
            f"parallel_scan_log (log_coeffs={tuple(log_coeffs.shape)}, "
            f"log_values={tuple(log_values.shape)}) outside the HIP envelope: need (B, T, D) "
            "log_coeffs and (B, T+1, D) log_values"
        )
    _same_device(log_coeffs, log_values)
    if log_coeffs.numel() == 0:
        return log_coeffs.new_empty(log_coeffs.shape)
    return _funnel("parallel_scan_log", _LogScanFn.apply, log_coeffs, log_values)


# ---------------------------------------------------------------------------
# matrix_scan / matrix_affine_scan
# ---------------------------------------------------------------------------


class _AffineScanFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, A, Bm):
        out_dtype = A.dtype
        A32, B32 = _as_f32(A, Bm)
        Bn, T, n, k, _ = A32.shape
        v = B32.shape[-1]
        Abar = torch.empty_like(A32)
        Bbar = torch.empty_like(B32)
        ws = _scan_workspace(_size("mg_affine_scan_workspace_bytes", Bn, T, n, k, v), A32.device)
        _call("mg_affine_scan_fwd", _ptr(A32), _ptr(B32), _ptr(Abar), _ptr(Bbar), Bn, T, n, k, v,
              _ptr(ws), ws.numel(), _stream(A32))
        _check_workspace(ws, A32)
        ctx.save_for_backward(A32, B32, Abar, Bbar)
        ctx.out_dtype = out_dtype
        if out_dtype != torch.float32:
            return Abar.to(out_dtype), Bbar.to(out_dtype)
        return Abar, Bbar

    @staticmethod
    @once_differentiable
    def backward(ctx, gAbar, gBbar):
        A32, B32, Abar, Bbar = ctx.saved_tensors
        Bn, T, n, k, _ = A32.shape
        v = B32.shape[-1]
        gA32, gB32 = _as_f32(gAbar, gBbar)
        dA = torch.empty_like(A32)
        dB = torch.empty_like(B32)
        ws = _scan_workspace(_size("mg_affine_scan_workspace_bytes", Bn, T, n, k, v), A32.device)
        _call("mg_affine_scan_bwd", _ptr(A32), _ptr(B32), _ptr(Abar), _ptr(Bbar), _ptr(gA32),
              _ptr(gB32), _ptr(dA), _ptr(dB), Bn, T, n, k, v, _ptr(ws), ws.numel(), _stream(A32))
        _check_workspace(ws, A32)
        return dA.to(ctx.out_dtype), dB.to(ctx.out_dtype)


def _matrix_affine_scan_impl(A: torch.Tensor, Bm: torch.Tensor):
    """``SCAN_IMPLS['matrix_affine_scan']``: generic k x k transitions, k x v injections."""
    if A.ndim != 5 or Bm.ndim != 5:
        raise ScanFallback(
            f"matrix_affine_scan (A={tuple(A.shape)}, Bm={tuple(Bm.shape)}) outside the HIP "
            "envelope: need 5-D (B, T, n, k, k) A and (B, T, n, k, v) Bm"
        )
    k = A.shape[-1]
    v = Bm.shape[-1]
    if (
        k not in _AFFINE_K
        or v not in _AFFINE_V
        or A.shape[-2] != k
        or Bm.shape[-2] != k
        or A.shape[:3] != Bm.shape[:3]
    ):
        raise ScanFallback(
            f"matrix_affine_scan (A={tuple(A.shape)}, Bm={tuple(Bm.shape)}) outside the HIP "
            f"envelope: need k in {sorted(_AFFINE_K)}, v in {sorted(_AFFINE_V)}, a square A and "
            "A/Bm sharing the (B, T, n) lane grid"
        )
    _same_device(A, Bm)
    if A.numel() == 0:
        return A.new_empty(A.shape), Bm.new_empty(Bm.shape)
    return _funnel("matrix_affine_scan", _AffineScanFn.apply, A, Bm)


def _matrix_scan_impl(M: torch.Tensor, b: torch.Tensor):
    """``SCAN_IMPLS['matrix_scan']``: the k = 2, v = 1 case, ``b`` viewed as (..., 2, 1)."""
    if (
        M.ndim != 5
        or b.ndim != 4
        or tuple(M.shape[-2:]) != (2, 2)
        or b.shape[-1] != 2
        or M.shape[:3] != b.shape[:3]
    ):
        raise ScanFallback(
            f"matrix_scan (M={tuple(M.shape)}, b={tuple(b.shape)}) outside the HIP envelope: "
            "need (B, T, n, 2, 2) M and (B, T, n, 2) b sharing the (B, T, n) lane grid"
        )
    _same_device(M, b)
    if M.numel() == 0:
        return M.new_empty(M.shape), b.new_empty(b.shape)

    def run():
        Abar, Bbar = _AffineScanFn.apply(M, b.unsqueeze(-1))
        return Abar, Bbar.squeeze(-1)

    return _funnel("matrix_scan", run)


# ---------------------------------------------------------------------------
# angle-fused rotation scan
# ---------------------------------------------------------------------------

_SCHED_BRICK = 0
_SCHED_LEX = 1
# id(perm) -> (weakref to perm, validity key, (sched, rounds)).  Tensors cannot be
# dictionary keys by value (their == is elementwise), hence the identity key.
_sched_cache: dict = {}


def _brick_tables(k: int, R: int):
    perm = torch.arange(k, dtype=torch.int64).repeat(R, 1)
    sgn = torch.zeros(R, k, dtype=torch.float64)
    p2p = torch.zeros(R, k, dtype=torch.int64)
    for r in range(R):
        for m in range(k // 2):
            i = (r % 2 + 2 * m) % k
            j = (i + 1) % k
            perm[r, i], perm[r, j] = j, i
            sgn[r, i], sgn[r, j] = -1.0, 1.0
            p2p[r, i] = p2p[r, j] = m
    return perm, sgn, p2p


def _classify_schedule(perm, sgn, p2p, k: int, R: int, half: int):
    """Map the plane metadata onto a compiled schedule: ``(sched, rounds)``.

    Recognised: brick-wall rounds (even rounds pair (0,1),(2,3)...; odd rounds
    (1,2),...,(k-1,0); ``half = k/2`` angles per round) and one-plane rounds
    over all pairs i<j in lexicographic order (``half = 1``).  A position whose
    partner is itself is untouched by its round.  Anything else declines.
    """
    key = (perm._version, sgn.data_ptr(), sgn._version, p2p.data_ptr(), p2p._version, k, R, half)
    hit = _sched_cache.get(id(perm))
    if hit is not None and hit[0]() is perm and hit[1] == key:
        return hit[2]
    pc = perm.detach().to("cpu", torch.int64)
    sc = sgn.detach().to("cpu", torch.float64)
    qc = p2p.detach().to("cpu", torch.int64)
    result = None
    if half == k // 2:
        bp, bs, bq = _brick_tables(k, R)
        if torch.equal(pc, bp) and torch.equal(sc, bs) and torch.equal(qc, bq):
            result = (_SCHED_BRICK, R)
    if result is None and half == 1 and R == k * (k - 1) // 2:
        ok = True
        r = 0
        for i in range(k):
            for j in range(i + 1, k):
                exp = torch.arange(k)
                exp[i], exp[j] = j, i
                if not (torch.equal(pc[r], exp) and sc[r, i] == -1.0 and sc[r, j] == 1.0
                        and qc[r, i] == 0 and qc[r, j] == 0):
                    ok = False
                r += 1
        if ok:
            result = (_SCHED_LEX, R)
    if result is None:
        raise ScanFallback(
            "angle-fused HIP kernel supports brick-wall rounds and the lexicographic all-pairs "
            "schedule; the given perm/sgn/p2p plane metadata is neither"
        )
    if len(_sched_cache) > 256:
        for dead in [i for i, v in _sched_cache.items() if v[0]() is None]:
            del _sched_cache[dead]
    _sched_cache[id(perm)] = (weakref.ref(perm), key, result)
    return result


_SCHED_TABLES = 2
# id(perm) -> (weakref to perm, validity key, device tables) for the table-driven kernel.
_table_cache: dict = {}


def _table_reason(perm, sgn, p2p, k: int, half: int) -> str | None:
    """Why the tables do not describe disjoint plane rotations, or ``None``.

    Per round: ``perm`` is an involution on 0..k-1; a position paired with another
    shares its partner's angle index (in 0..half-1) and has the opposite sign, -1
    or +1; a position paired with itself is left untouched.
    """
    idx = torch.arange(k)
    if perm.min() < 0 or perm.max() >= k:
        return "perm entries must lie in [0, k)"
    if not torch.equal(torch.gather(perm, 1, perm), idx.expand_as(perm)):
        return "every round's perm must be an involution (partners pair up)"
    act = perm != idx
    part_q = torch.gather(p2p, 1, perm)
    part_s = torch.gather(sgn, 1, perm)
    if bool((act & ((p2p < 0) | (p2p >= half))).any()):
        return "p2p entries of paired positions must lie in [0, half)"
    if bool((act & (part_q != p2p)).any()):
        return "paired positions must share one angle (equal p2p)"
    if bool((act & ((sgn.abs() != 1) | (part_s != -sgn))).any()):
        return "paired positions must carry opposite unit signs (sgn -1/+1)"
    for r in range(perm.shape[0]):
        firsts = act[r] & (sgn[r] < 0)  # one member of each plane
        used = p2p[r][firsts]
        if used.numel() != torch.unique(used).numel():
            return "an angle may drive at most one plane per round"
    return None


def _tables_cover_all_angles(perm, p2p, half: int) -> bool:
    """Whether every angle index of every round drives a plane (then the backward
    writes every dtheta element; otherwise the unused ones must start at zero)."""
    act = perm != torch.arange(perm.shape[1])
    for r in range(perm.shape[0]):
        if torch.unique(p2p[r][act[r]]).numel() != half:
            return False
    return True


def _device_tables(perm, sgn, p2p, k: int, half: int, device):
    """Validated int32/fp32 copies of the plane tables on ``device``, cached while the
    same three tensor objects (held by weak reference) are passed unmodified: a new
    ``sgn`` or ``p2p`` object, even at a reused address, or an in-place change to any
    of the three (its ``_version``) validates and copies again."""
    key = (perm._version, sgn._version, p2p._version, k, half, str(device))
    hit = _table_cache.get(id(perm))
    if (hit is not None and hit[0]() is perm and hit[1]() is sgn and hit[2]() is p2p
            and hit[3] == key):
        return hit[4]
    pc = perm.detach().to("cpu", torch.int64)
    sc = sgn.detach().to("cpu", torch.float64)
    qc = p2p.detach().to("cpu", torch.int64)
    reason = _table_reason(pc, sc, qc, k, half)
    if reason is not None:
        raise ScanFallback(f"angle-fused HIP kernel: plane tables rejected: {reason}")
    tables = (pc.to(device, torch.int32).contiguous(), sc.to(device, torch.float32).contiguous(),
              qc.to(device, torch.int32).contiguous(), _tables_cover_all_angles(pc, qc, half))
    if len(_table_cache) > 256:
        for dead in [i for i, v in _table_cache.items() if v[0]() is None]:
            del _table_cache[dead]
    _table_cache[id(perm)] = (weakref.ref(perm), weakref.ref(sgn), weakref.ref(p2p), key, tables)
    return tables


class _AngleTablesFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, theta, scale, gamma, b, h0, perm, sgn, p2p, cover, flags):
        out_dtype = b.dtype
        th, sc, gm, b32, h032 = _as_f32(theta, scale, gamma, b, h0)
        Bn, T, n, k = b32.shape
        R, half = th.shape[3], th.shape[4]
        h = torch.empty_like(b32)
        # Chunk products P_c, saved for the backward (whose chunk maps are P_c^T).
        prod = torch.empty(max(_size("mg_angle_scan_tables_state_bytes", Bn, T, n, k), 16) // 4,
                           dtype=torch.float32, device=b32.device)
        ws = _workspace(_size("mg_angle_scan_tables_workspace_bytes", Bn, T, n, k), b32.device)
        _call("mg_angle_scan_tables_fwd", _ptr(th), _ptr(sc), _ptr(gm), _ptr(b32), _ptr(h032),
              _ptr(perm), _ptr(sgn), _ptr(p2p), _ptr(h), _ptr(prod), Bn, T, n, k, R, half, flags,
              _ptr(ws), ws.numel(), _stream(b32))
        ctx.save_for_backward(th, sc, gm, h032, h, prod, perm, sgn, p2p)
        ctx.meta = (flags, cover, out_dtype, theta.dtype, scale.dtype, gamma.dtype, h0.dtype)
        return h if out_dtype == torch.float32 else h.to(out_dtype)

    @staticmethod
    @once_differentiable
    def backward(ctx, gh):
        th, sc, gm, h032, h, prod, perm, sgn, p2p = ctx.saved_tensors
        flags, cover, out_dtype, tdt, sdt, gdt, hdt = ctx.meta
        Bn, T, n, k = h.shape
        R, half = th.shape[3], th.shape[4]
        (gh32,) = _as_f32(gh)
        need = ctx.needs_input_grad
        # dtheta of an angle no plane uses is zero; the kernel writes only used ones.
        dth = torch.empty_like(th) if cover else torch.zeros_like(th)
        dsc = (torch.empty_like(sc) if flags & 1 else torch.zeros_like(sc)) \
            if (flags & 1 or need[1]) else None
        dgm = (torch.empty_like(gm) if flags & 2 else torch.zeros_like(gm)) \
            if (flags & 2 or need[2]) else None
        db = torch.empty_like(h)
        dh0 = torch.empty_like(h032)
        ws = _workspace(_size("mg_angle_scan_tables_workspace_bytes", Bn, T, n, k), h.device)
        _call("mg_angle_scan_tables_bwd", _ptr(th), _ptr(sc), _ptr(gm), _ptr(h032), _ptr(h),
              _ptr(prod), _ptr(gh32), _ptr(perm), _ptr(sgn), _ptr(p2p), _ptr(dth), _ptr(dsc),
              _ptr(dgm), _ptr(db), _ptr(dh0), Bn, T, n, k, R, half, flags, _ptr(ws), ws.numel(),
              _stream(h))
        return (dth.to(tdt), None if dsc is None else dsc.to(sdt),
                None if dgm is None else dgm.to(gdt), db.to(out_dtype), dh0.to(hdt),
                None, None, None, None, None)


class _AngleScanFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, theta, scale, gamma, b, h0, sched, rounds, flags):
        out_dtype = b.dtype
        th, sc, gm, b32, h032 = _as_f32(theta, scale, gamma, b, h0)
        Bn, T, n, k = b32.shape
        h = torch.empty_like(b32)
        # Chunk products P_c (and, past 16 chunks, the group products), saved for the
        # backward, whose chunk and group maps are their transposes.
        prod = torch.empty(max(_size("mg_angle_scan_state_bytes", Bn, T, n, k), 16) // 4,
                           dtype=torch.float32, device=b32.device)
        ws = _workspace(_size("mg_angle_scan_workspace_bytes", Bn, T, n, k), b32.device)
        _call("mg_angle_scan_fwd", _ptr(th), _ptr(sc), _ptr(gm), _ptr(b32), _ptr(h032), _ptr(h),
              _ptr(prod), Bn, T, n, k, sched, rounds, flags, _ptr(ws), ws.numel(), _stream(b32))
        ctx.save_for_backward(th, sc, gm, h032, h, prod)
        ctx.meta = (sched, rounds, flags, out_dtype, theta.dtype, scale.dtype, gamma.dtype,
                    h0.dtype)
        return h if out_dtype == torch.float32 else h.to(out_dtype)

    @staticmethod
    @once_differentiable
    def backward(ctx, gh):
        th, sc, gm, h032, h, prod = ctx.saved_tensors
        sched, rounds, flags, out_dtype, tdt, sdt, gdt, hdt = ctx.meta
        Bn, T, n, k = h.shape
        (gh32,) = _as_f32(gh)
        dth = torch.empty_like(th)
        need = ctx.needs_input_grad
        # An enabled scale / decay channel has every element of its grad written by the
        # kernel; a disabled one's grad is zero (the kernel never touches it).
        dsc = (torch.empty_like(sc) if flags & 1 else torch.zeros_like(sc)) \
            if (flags & 1 or need[1]) else None
        dgm = (torch.empty_like(gm) if flags & 2 else torch.zeros_like(gm)) \
            if (flags & 2 or need[2]) else None
        db = torch.empty_like(h)
        dh0 = torch.empty_like(h032)
        ws = _workspace(_size("mg_angle_scan_workspace_bytes", Bn, T, n, k), h.device)
        _call("mg_angle_scan_bwd", _ptr(th), _ptr(sc), _ptr(gm), _ptr(h032), _ptr(h), _ptr(prod),
              _ptr(gh32), _ptr(dth), _ptr(dsc), _ptr(dgm), _ptr(db), _ptr(dh0), Bn, T, n, k,
              sched, rounds, flags, _ptr(ws), ws.numel(), _stream(h))
        return (dth.to(tdt), None if dsc is None else dsc.to(sdt),
                None if dgm is None else dgm.to(gdt), db.to(out_dtype), dh0.to(hdt),
                None, None, None)


def angle_scan_impl(theta, scale, gamma, b, h0, perm, sgn, p2p, *, has_scale: int,
                    has_decay: int):
    """Envelope-checked angle-fused rotation scan; returns ``h`` ``(B, T, n, k)``.

    Same contract as the reference entry point (``src/mingru/triton_scans.py:1743-1812``):
    ``theta`` ``(B, T, n, R, half)``, ``scale``/``gamma`` ``(B, T, n)``, ``b``
    ``(B, T, n, k)``, ``h0`` ``(B, n, k)``, ``perm``/``sgn``/``p2p`` ``(R, k)``.
    """
    if theta.ndim != 5 or b.ndim != 4:
        raise ScanFallback(
            f"angle-fused kernel (theta={tuple(theta.shape)}, b={tuple(b.shape)}) outside the "
            "envelope: need 5-D (B, T, n, R, half) theta and 4-D (B, T, n, k) b"
        )
    Bn, T, n, R, half = theta.shape
    k = b.shape[-1]
    if (
        k not in _ANGLE_TABLE_K
        or half > _ANGLE_TABLE_MAX_HALF
        or R > _ANGLE_TABLE_MAX_ROUNDS
        or tuple(b.shape[:3]) != (Bn, T, n)
        or tuple(scale.shape) != (Bn, T, n)
        or tuple(gamma.shape) != (Bn, T, n)
        or tuple(h0.shape) != (Bn, n, k)
        or tuple(perm.shape) != (R, k)
        or tuple(sgn.shape) != (R, k)
        or tuple(p2p.shape) != (R, k)
    ):
        raise ScanFallback(
            f"angle-fused kernel (theta={tuple(theta.shape)}, scale={tuple(scale.shape)}, "
            f"gamma={tuple(gamma.shape)}, b={tuple(b.shape)}, h0={tuple(h0.shape)}, "
            f"perm={tuple(perm.shape)}) outside the envelope: need k in "
            f"{sorted(_ANGLE_TABLE_K)}, at most {_ANGLE_TABLE_MAX_HALF} angles per round, at "
            f"most {_ANGLE_TABLE_MAX_ROUNDS} rounds and shapes agreeing on (B, T, n, R, k)"
        )
    _same_device(theta, scale, gamma, b, h0)
    flags = (1 if has_scale else 0) | (2 if has_decay else 0)
    sched = None
    if k in _ANGLE_K and R <= _ANGLE_MAX_ROT:
        try:
            sched, rounds = _classify_schedule(perm, sgn, p2p, k, R, half)
        except ScanFallback:
            sched = None
    if sched is None:
        # Any other schedule, more rounds, or k = 16: the table-driven kernel.
        tables = _device_tables(perm, sgn, p2p, k, half, b.device)
        if T == 0:
            return b.new_empty(b.shape)
        return _funnel("angle-fused (plane tables)", _AngleTablesFn.apply, theta, scale, gamma,
                       b, h0, *tables, flags)
    if T == 0:
        return b.new_empty(b.shape)
    return _funnel("angle-fused", _AngleScanFn.apply, theta, scale, gamma, b, h0, sched, rounds,
                   flags)


class _AngleGatedFn(torch.autograd.Function):
    """The brick-wall angle scan with the mixers' heads formed in the kernel: b =
    sigmoid(z) * hpre and, with a scale, tanh(u)."""

    @staticmethod
    def forward(ctx, theta, u, gamma, z, hpre, h0, rounds, flags):
        out_dtype = z.dtype
        th, z32, hp32, h032 = _as_f32(theta, z, hpre, h0)
        u32 = _as_f32(u)[0] if u is not None else None
        gm = _as_f32(gamma)[0] if gamma is not None else None
        Bn, T, n, k = z32.shape
        h = torch.empty_like(z32)
        prod = torch.empty(max(_size("mg_angle_scan_state_bytes", Bn, T, n, k), 16) // 4,
                           dtype=torch.float32, device=z32.device)
        ws = _workspace(_size("mg_angle_scan_workspace_bytes", Bn, T, n, k), z32.device)
        _call("mg_angle_scan_gated_fwd", _ptr(th), _ptr(u32), _ptr(gm), _ptr(z32), _ptr(hp32),
              _ptr(h032), _ptr(h), _ptr(prod), Bn, T, n, k, rounds, flags, _ptr(ws), ws.numel(),
              _stream(z32))
        ctx.save_for_backward(th, u32, gm, z32, hp32, h032, h, prod)
        ctx.meta = (rounds, flags, out_dtype, theta.dtype,
                    None if u is None else u.dtype, None if gamma is None else gamma.dtype,
                    hpre.dtype, h0.dtype)
        return h if out_dtype == torch.float32 else h.to(out_dtype)

    @staticmethod
    @once_differentiable
    def backward(ctx, gh):
        th, u32, gm, z32, hp32, h032, h, prod = ctx.saved_tensors
        rounds, flags, out_dtype, tdt, udt, gdt, hdt, h0dt = ctx.meta
        Bn, T, n, k = h.shape
        (gh32,) = _as_f32(gh)
        dth = torch.empty_like(th)
        du = torch.empty_like(u32) if u32 is not None else None
        dgm = torch.empty_like(gm) if gm is not None else None
        dz, dhp = torch.empty_like(z32), torch.empty_like(hp32)
        dh0 = torch.empty_like(h032)
        ws = _workspace(_size("mg_angle_scan_workspace_bytes", Bn, T, n, k), h.device)
        _call("mg_angle_scan_gated_bwd", _ptr(th), _ptr(u32), _ptr(gm), _ptr(z32), _ptr(hp32),
              _ptr(h032), _ptr(h), _ptr(prod), _ptr(gh32), _ptr(dth), _ptr(du), _ptr(dgm),
              _ptr(dz), _ptr(dhp), _ptr(dh0), Bn, T, n, k, rounds, flags, _ptr(ws), ws.numel(),
              _stream(h))
        return (dth.to(tdt), None if du is None else du.to(udt),
                None if dgm is None else dgm.to(gdt), dz.to(out_dtype), dhp.to(hdt),
                dh0.to(h0dt), None, None)


def angle_gated_scan_impl(theta, u, gamma, z, hpre, h0, perm, sgn, p2p, *, has_scale: int,
                          has_decay: int):
    """The angle-fused scan with RotationMinGRU's / GivensMinGRU's heads formed in the
    kernel; returns ``h`` ``(B, T, n, k)``.

    No reference kernel fuses the heads: the reference computes ``scale =
    tanh(linear_u x)`` and ``b = sigmoid(linear_z x) * linear_h x`` eagerly
    (``src/mingru/min_gru.py:2261-2262, 2719``) and hands them to the angle scan.
    Here ``u`` ``(B, T, n)`` (used when ``has_scale``), ``z`` and ``hpre``
    ``(B, T, n, k)`` go to the kernel instead; ``theta``, ``gamma`` (when
    ``has_decay``), ``h0`` and the plane tables as for ``angle_scan_impl``.  Only
    the compiled brick-wall schedules (k in {2, 4, 8}) take this form; anything
    else raises ``ScanFallback`` and the caller runs the heads eagerly.
    """
    if theta.ndim != 5 or z.ndim != 4:
        raise ScanFallback("gated angle scan: need 5-D theta and 4-D z")
    Bn, T, n, R, half = theta.shape
    k = z.shape[-1]
    if (
        k not in _ANGLE_K
        or R > _ANGLE_MAX_ROT
        or tuple(z.shape[:3]) != (Bn, T, n)
        or hpre.shape != z.shape
        or tuple(h0.shape) != (Bn, n, k)
        or (has_scale and (u is None or tuple(u.shape) != (Bn, T, n)))
        or (has_decay and (gamma is None or tuple(gamma.shape) != (Bn, T, n)))
        or tuple(perm.shape) != (R, k)
    ):
        raise ScanFallback(
            f"gated angle scan (theta={tuple(theta.shape)}, z={tuple(z.shape)}, "
            f"hpre={tuple(hpre.shape)}, h0={tuple(h0.shape)}) outside the envelope: need "
            f"k in {sorted(_ANGLE_K)}, at most {_ANGLE_MAX_ROT} rounds and shapes agreeing on "
            "(B, T, n, R, k)"
        )
    sched, rounds = _classify_schedule(perm, sgn, p2p, k, R, half)
    if sched != 0:
        raise ScanFallback("gated angle scan: only the brick-wall schedule takes the fused heads")
    _same_device(theta, z, hpre, h0, *[t for t in (u, gamma) if t is not None])
    flags = (1 if has_scale else 0) | (2 if has_decay else 0)
    if T == 0:
        return z.new_empty(z.shape)
    return _funnel("angle-fused (gated heads)", _AngleGatedFn.apply, theta,
                   u if has_scale else None, gamma if has_decay else None, z, hpre, h0, rounds,
                   flags)


# ---------------------------------------------------------------------------
# DeltaMinGRU chunked-WY
# ---------------------------------------------------------------------------


def _delta_envelope_reason(*, is_cuda: bool, q_dtype, k_dtype, v_dtype, beta_dtype, h0_dtype,
                           d_k: int, d_v: int, chunk_size: int, nh: int) -> str | None:
    """Human-readable rejection reason, or ``None`` inside the envelope.

    Works on plain descriptors so every branch is reachable from a CPU test
    (reference ``src/mingru/triton_scans.py:335-389``); each violation yields a
    distinct string.  Q, K, V and beta may be float32, bfloat16 or float16 (the
    kernels read bf16 natively and compute in fp32; fp16 is upcast); H0 may be
    any of those.  float64 stays on the eager path.
    """
    if not is_cuda:
        return "DeltaMinGRU HIP kernel requires GPU tensors (got a non-GPU tensor)"
    for name, dt in (("Q", q_dtype), ("K", k_dtype), ("V", v_dtype), ("beta", beta_dtype),
                     ("H0", h0_dtype)):
        if dt not in _DELTA_DTYPES:
            return (f"DeltaMinGRU HIP kernel takes float32, bfloat16 or float16 inputs "
                    f"(got {name} dtype {dt})")
    if not 1 <= d_k <= _DELTA_MAX_DIM:
        return f"DeltaMinGRU HIP kernel needs 1 <= d_k <= {_DELTA_MAX_DIM} (got d_k={d_k})"
    if not 1 <= d_v <= _DELTA_MAX_DIM:
        return f"DeltaMinGRU HIP kernel needs 1 <= d_v <= {_DELTA_MAX_DIM} (got d_v={d_v})"
    if not 1 <= chunk_size <= _DELTA_MAX_CHUNK:
        return (f"DeltaMinGRU HIP kernel chunk_size must be in [1, {_DELTA_MAX_CHUNK}] "
                f"(got chunk_size={chunk_size})")
    if nh * chunk_size > _DELTA_MAX_MICROSTEPS:
        return (f"DeltaMinGRU HIP kernel requires nh * chunk_size <= {_DELTA_MAX_MICROSTEPS} "
                f"(got nh={nh}, chunk_size={chunk_size}, product={nh * chunk_size})")
    if nh > _DELTA_TILE_MICROSTEPS:
        return (f"DeltaMinGRU HIP kernel holds a token's micro-steps in one "
                f"{_DELTA_TILE_MICROSTEPS}-step tile, so nh must be <= {_DELTA_TILE_MICROSTEPS} "
                f"(got nh={nh})")
    return None


def _delta_tile_chunk(nh: int, chunk_size: int) -> int:
    """Tokens per kernel chunk: the requested chunk, capped so that one chunk holds at
    most 64 micro-steps (same result in exact arithmetic; see ``_DELTA_MAX_MICROSTEPS``)."""
    return max(1, min(int(chunk_size), _DELTA_TILE_MICROSTEPS // max(1, int(nh))))


def _delta_validate_envelope(Q, K, V, beta, H0, chunk_size: int) -> None:
    """Raise ``ScanFallback`` unless the kernel layouts are eligible
    (reference ``src/mingru/triton_scans.py:392-452``)."""
    if Q.ndim != 4 or K.ndim != 5 or V.ndim != 5 or beta.ndim != 4 or H0.ndim != 4:
        raise ScanFallback(
            "DeltaMinGRU HIP kernel needs 4-D Q (B, n_heads, T, d_k), 5-D K "
            "(B, n_heads, T, nh, d_k), 5-D V (B, n_heads, T, nh, d_v), 4-D beta "
            "(B, n_heads, T, nh) and 4-D H0 (B, n_heads, d_k, d_v); got ranks "
            f"Q={Q.ndim}, K={K.ndim}, V={V.ndim}, beta={beta.ndim}, H0={H0.ndim}"
        )
    Bn, nhd, T, d_k = Q.shape
    nh = K.shape[3]
    d_v = V.shape[4]
    if (
        tuple(K.shape[:3]) != (Bn, nhd, T)
        or K.shape[4] != d_k
        or tuple(V.shape[:3]) != (Bn, nhd, T)
        or V.shape[3] != nh
        or tuple(beta.shape) != (Bn, nhd, T, nh)
        or tuple(H0.shape) != (Bn, nhd, d_k, d_v)
    ):
        raise ScanFallback(
            "DeltaMinGRU HIP kernel shapes disagree: from Q=(B, n_heads, T, d_k)="
            f"{tuple(Q.shape)} expected K={(Bn, nhd, T, nh, d_k)}, V={(Bn, nhd, T, nh, d_v)}, "
            f"beta={(Bn, nhd, T, nh)}, H0={(Bn, nhd, d_k, d_v)}; got K={tuple(K.shape)}, "
            f"V={tuple(V.shape)}, beta={tuple(beta.shape)}, H0={tuple(H0.shape)}"
        )
    reason = _delta_envelope_reason(
        is_cuda=Q.is_cuda and K.is_cuda and V.is_cuda and beta.is_cuda and H0.is_cuda,
        q_dtype=Q.dtype, k_dtype=K.dtype, v_dtype=V.dtype, beta_dtype=beta.dtype,
        h0_dtype=H0.dtype, d_k=d_k, d_v=d_v, chunk_size=chunk_size, nh=nh,
    )
    if reason is not None:
        raise ScanFallback(reason)


def _delta_compute_dtype(*ts):
    """bf16 when Q, K, V and beta are all bf16 (read natively), else fp32."""
    return torch.bfloat16 if all(t.dtype == torch.bfloat16 for t in ts) else torch.float32


def _contig(t, dtype):
    t = t.to(dtype).contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


class _DeltaScanFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, Q, K, V, beta, H0, chunk_size):
        cdt = _delta_compute_dtype(Q, K, V, beta)
        q, k, v, bt = (_contig(t, cdt) for t in (Q, K, V, beta))
        h0 = _contig(H0, torch.float32)
        Bn, nhd, T, d_k = q.shape
        nh = k.shape[3]
        d_v = v.shape[4]
        dims = (Bn, nhd, T, nh, d_k, d_v, chunk_size)
        y = torch.empty(Bn, nhd, T, d_v, dtype=cdt, device=q.device)
        HT = torch.empty(Bn, nhd, d_k, d_v, dtype=torch.float32, device=q.device)
        Hb = torch.empty(max(_size("mg_delta_state_bytes", *dims), 16) // 4, dtype=torch.float32,
                         device=q.device)
        ws = _workspace(_size("mg_delta_workspace_bytes", *dims), q.device)
        _call("mg_delta_fwd", _ptr(q), _ptr(k), _ptr(v), _ptr(bt), _ptr(h0), _ptr(y), _ptr(HT),
              _ptr(Hb), *dims[:6], chunk_size, 1 if cdt == torch.bfloat16 else 0, _ptr(ws),
              ws.numel(), _stream(q))
        ctx.save_for_backward(q, k, v, bt, Hb)
        ctx.meta = (chunk_size, cdt, Q.dtype, K.dtype, V.dtype, beta.dtype, H0.dtype)
        return y.to(Q.dtype), HT.to(H0.dtype)

    @staticmethod
    @once_differentiable
    def backward(ctx, gy, gHT):
        q, k, v, bt, Hb = ctx.saved_tensors
        chunk_size, cdt, qdt, kdt, vdt, bdt, hdt = ctx.meta
        Bn, nhd, T, d_k = q.shape
        nh = k.shape[3]
        d_v = v.shape[4]
        dy = (torch.zeros(Bn, nhd, T, d_v, dtype=cdt, device=q.device) if gy is None
              else _contig(gy, cdt))
        dHT = (torch.zeros(Bn, nhd, d_k, d_v, dtype=torch.float32, device=q.device)
               if gHT is None else _contig(gHT, torch.float32))
        dQ, dK, dV, dbeta = (torch.empty_like(t) for t in (q, k, v, bt))
        dH0 = torch.empty(Bn, nhd, d_k, d_v, dtype=torch.float32, device=q.device)
        dims = (Bn, nhd, T, nh, d_k, d_v, chunk_size)
        ws = _workspace(_size("mg_delta_workspace_bytes", *dims), q.device)
        _call("mg_delta_bwd", _ptr(q), _ptr(k), _ptr(v), _ptr(bt), _ptr(Hb), _ptr(dy), _ptr(dHT),
              _ptr(dQ), _ptr(dK), _ptr(dV), _ptr(dbeta), _ptr(dH0), *dims[:6], chunk_size,
              1 if cdt == torch.bfloat16 else 0, _ptr(ws), ws.numel(), _stream(q))
        return dQ.to(qdt), dK.to(kdt), dV.to(vdt), dbeta.to(bdt), dH0.to(hdt), None


def delta_scan_impl(Q, K, V, beta, H0, *, chunk_size: int):
    """DeltaMinGRU chunked-WY forward on the kernel layouts; returns ``(y, H_T)``.

    Same contract as the reference entry point
    (``src/mingru/triton_scans.py:2403-2447``): ``Q`` ``(B, n_heads, T, d_k)``,
    ``K`` ``(B, n_heads, T, nh, d_k)``, ``V`` ``(B, n_heads, T, nh, d_v)``,
    ``beta`` ``(B, n_heads, T, nh)``, ``H0`` ``(B, n_heads, d_k, d_v)``; ``y``
    ``(B, n_heads, T, d_v)`` in Q's dtype and ``H_T`` in H0's dtype.
    Differentiable in all five tensors.
    """
    _delta_validate_envelope(Q, K, V, beta, H0, chunk_size)
    if Q.shape[2] == 0:
        return Q.new_zeros(Q.shape[:3] + (V.shape[-1],)), H0.clone()
    return _funnel("DeltaMinGRU chunked-WY", _DeltaScanFn.apply, Q, K, V, beta, H0,
                   _delta_tile_chunk(K.shape[3], chunk_size))


# ---------------------------------------------------------------------------
# DeltaMinGRU decay-gated chunked-WY
# ---------------------------------------------------------------------------


class _DeltaGatedScanFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, Q, K, V, beta, log_gamma, H0, chunk_size):
        # bf16 inputs read natively (bf16 MFMA, any nh); everything else in fp32.
        nh = K.shape[3]
        cdt = _delta_compute_dtype(Q, K, V, beta)
        q, k, v, bt = (_contig(t, cdt) for t in (Q, K, V, beta))
        lg, h0 = _contig(log_gamma, torch.float32), _contig(H0, torch.float32)
        Bn, nhd, T, d_k = q.shape
        d_v = v.shape[4]
        dims = (Bn, nhd, T, nh, d_k, d_v, chunk_size)
        y = torch.empty(Bn, nhd, T, d_v, dtype=cdt, device=q.device)
        HT = torch.empty(Bn, nhd, d_k, d_v, dtype=torch.float32, device=q.device)
        Hb = torch.empty(max(_size("mg_delta_state_bytes", *dims), 16) // 4, dtype=torch.float32,
                         device=q.device)
        ws = _workspace(_size("mg_delta_gated_workspace_bytes", *dims), q.device)
        tag = 1 if cdt == torch.bfloat16 else 0
        _call("mg_delta_gated_fwd", _ptr(q), _ptr(k), _ptr(v), _ptr(bt), _ptr(lg), _ptr(h0),
              _ptr(y), _ptr(HT), _ptr(Hb), *dims, tag, _ptr(ws), ws.numel(), _stream(q))
        ctx.save_for_backward(q, k, v, bt, lg, Hb)
        ctx.meta = (chunk_size, cdt, Q.dtype, K.dtype, V.dtype, beta.dtype, log_gamma.dtype,
                    H0.dtype)
        return y.to(Q.dtype), HT.to(H0.dtype)

    @staticmethod
    @once_differentiable
    def backward(ctx, gy, gHT):
        q, k, v, bt, lg, Hb = ctx.saved_tensors
        chunk_size, cdt, qdt, kdt, vdt, bdt, ldt, hdt = ctx.meta
        Bn, nhd, T, d_k = q.shape
        nh = k.shape[3]
        d_v = v.shape[4]
        dy = (torch.zeros(Bn, nhd, T, d_v, dtype=cdt, device=q.device) if gy is None
              else _contig(gy, cdt))
        dHT = (torch.zeros(Bn, nhd, d_k, d_v, dtype=torch.float32, device=q.device)
               if gHT is None else _contig(gHT, torch.float32))
        dQ, dK, dV, dbeta, dlg = (torch.empty_like(t) for t in (q, k, v, bt, lg))
        dH0 = torch.empty(Bn, nhd, d_k, d_v, dtype=torch.float32, device=q.device)
        dims = (Bn, nhd, T, nh, d_k, d_v, chunk_size)
        ws = _workspace(_size("mg_delta_gated_workspace_bytes", *dims), q.device)
        tag = 1 if cdt == torch.bfloat16 else 0
        _call("mg_delta_gated_bwd", _ptr(q), _ptr(k), _ptr(v), _ptr(bt), _ptr(lg), _ptr(Hb),
              _ptr(dy), _ptr(dHT), _ptr(dQ), _ptr(dK), _ptr(dV), _ptr(dbeta), _ptr(dlg),
              _ptr(dH0), *dims, tag, _ptr(ws), ws.numel(), _stream(q))
        return (dQ.to(qdt), dK.to(kdt), dV.to(vdt), dbeta.to(bdt), dlg.to(ldt), dH0.to(hdt),
                None)


def delta_gated_scan_impl(Q, K, V, beta, log_gamma, H0, *, chunk_size: int):
    """DeltaMinGRU decay-active chunked-WY forward; returns ``(y, H_T)``.

    No reference kernel: the reference runs this eagerly
    (``_forward_chunked_gated``, ``src/mingru/min_gru.py:3257-3448``).  Layouts
    as ``delta_scan_impl`` plus ``log_gamma`` ``(B, n_heads, T)``, the per-token
    log decay applied to the state before the token's micro-steps.  bf16 Q, K, V,
    beta run the bf16-MFMA kernels (fp32 state) for any ``nh``; other inputs run in
    fp32 (half inputs are upcast).  ``y`` comes back in Q's dtype and ``H_T`` in H0's.
    Differentiable in all six tensors.
    """
    _delta_validate_envelope(Q, K, V, beta, H0, chunk_size)
    if tuple(log_gamma.shape) != tuple(Q.shape[:3]):
        raise ScanFallback(
            f"DeltaMinGRU gated kernel needs log_gamma of shape (B, n_heads, T)="
            f"{tuple(Q.shape[:3])} (got {tuple(log_gamma.shape)})"
        )
    if log_gamma.dtype not in _DELTA_DTYPES or not log_gamma.is_cuda:
        raise ScanFallback(
            "DeltaMinGRU gated kernel needs a float32, bfloat16 or float16 GPU log_gamma "
            f"(got {log_gamma.dtype} on {log_gamma.device})"
        )
    if log_gamma.device != Q.device:
        raise ScanFallback("DeltaMinGRU gated kernel inputs live on different devices")
    if Q.shape[2] == 0:
        return Q.new_zeros(Q.shape[:3] + (V.shape[-1],)), H0.clone()
    return _funnel("DeltaMinGRU gated chunked-WY", _DeltaGatedScanFn.apply, Q, K, V, beta,
                   log_gamma, H0, _delta_tile_chunk(K.shape[3], chunk_size))


# ---------------------------------------------------------------------------
# streaming decode (one recurrent step; inference only)
# ---------------------------------------------------------------------------

GATE_STEP_KINDS = {"signed": 0, "signed_coupled": 1, "mingru": 2}


def _inference_only(what, *ts):
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ts):
        raise ScanFallback(f"{what} is inference-only (autograd is recording)")


def gate_step_impl(kind: str, p0, p1, p2, gamma, h_prev):
    """One step ``h = gamma * a * h_prev + b`` of a diagonal mixer; returns ``h``.

    No reference kernel; the arithmetic is the mixers' ``step()``
    (``src/mingru/min_gru.py:1399-1448`` for MinGRU, SignedMinGRU's
    ``_coeffs`` + ``step``).  ``kind`` is ``"signed"`` / ``"signed_coupled"``
    (``p0, p1, p2 = s, z, hpre``) or ``"mingru"`` (``p0, p1 = k, hpre``; ``p2``
    unused).  ``gamma`` (decay) may be ``None`` or broadcastable to ``h_prev``.
    """
    if kind not in GATE_STEP_KINDS:
        raise ScanFallback(f"unknown gate step kind {kind!r}")
    ins = [p0, p1] + ([] if kind == "mingru" else [p2])
    for t in ins:
        if t.shape != h_prev.shape:
            raise ScanFallback(
                f"gate step pre-activation shape {tuple(t.shape)} differs from h_prev "
                f"{tuple(h_prev.shape)}"
            )
    _same_device(h_prev, *ins)
    _inference_only("the gate step kernel", h_prev, gamma, *ins)
    out_dtype = h_prev.dtype
    f32 = _as_f32(*ins, h_prev)
    hp32 = f32[-1]
    g32 = None
    if gamma is not None:
        _same_device(h_prev, gamma)
        (g32,) = _as_f32(gamma.expand(h_prev.shape))
    h = torch.empty_like(hp32)
    q0, q1 = f32[0], f32[1]
    q2 = f32[2] if kind != "mingru" else None
    _call("mg_gate_step", GATE_STEP_KINDS[kind], _ptr(q0), _ptr(q1), _ptr(q2), _ptr(g32),
          _ptr(hp32), _ptr(h), h.numel(), _stream(h))
    return h if out_dtype == torch.float32 else h.to(out_dtype)


def delta_step_impl(H, q, K, V, beta, log_gamma):
    """One DeltaMinGRU step on the kernel layouts; returns ``(y, H_new)``.

    No reference kernel; the arithmetic is ``DeltaMinGRU.step``
    (``src/mingru/min_gru.py:3611-3688``): ``H <- exp(log_gamma) H`` (when given),
    then for each micro-step ``H <- H + beta k (v - H^T k)^T``, then ``y = H^T q``.
    ``H`` ``(B, n_heads, d_k, d_v)``, ``q`` ``(B, n_heads, d_k)``, ``K``
    ``(B, n_heads, nh, d_k)``, ``V`` ``(B, n_heads, nh, d_v)``, ``beta``
    ``(B, n_heads, nh)``, ``log_gamma`` ``(B, n_heads)`` or ``None``;
    ``y`` is ``(B, n_heads, d_v)``.  ``H`` is not modified.
    """
    if H.ndim != 4 or q.ndim != 3 or K.ndim != 4 or V.ndim != 4 or beta.ndim != 3:
        raise ScanFallback("DeltaMinGRU step kernel needs H (B,h,dk,dv), q (B,h,dk), "
                           "K (B,h,nh,dk), V (B,h,nh,dv), beta (B,h,nh)")
    Bn, nhd, dk, dv = H.shape
    nh = K.shape[2]
    if (tuple(q.shape) != (Bn, nhd, dk) or tuple(K.shape) != (Bn, nhd, nh, dk)
            or tuple(V.shape) != (Bn, nhd, nh, dv) or tuple(beta.shape) != (Bn, nhd, nh)
            or (log_gamma is not None and tuple(log_gamma.shape) != (Bn, nhd))):
        raise ScanFallback("DeltaMinGRU step kernel shapes disagree")
    if not (1 <= dk <= _DELTA_MAX_DIM and 1 <= dv <= _DELTA_MAX_DIM):
        raise ScanFallback(f"DeltaMinGRU step kernel needs d_k, d_v <= {_DELTA_MAX_DIM}")
    ts = [H, q, K, V, beta] + ([] if log_gamma is None else [log_gamma])
    _same_device(*ts)
    _inference_only("the DeltaMinGRU step kernel", *ts)
    if Bn * nhd == 0:
        return q.new_zeros(Bn, nhd, dv), H.clone()
    h32, q32, k32, v32, b32 = _as_f32(H, q, K, V, beta)
    lg32 = None if log_gamma is None else _as_f32(log_gamma)[0]
    y = torch.empty(Bn, nhd, dv, dtype=torch.float32, device=H.device)
    Hn = torch.empty_like(h32)
    _call("mg_delta_step", _ptr(h32), _ptr(q32), _ptr(k32), _ptr(v32), _ptr(b32), _ptr(lg32),
          _ptr(Hn), _ptr(y), Bn * nhd, nh, dk, dv, _stream(h32))
    return y.to(q.dtype), Hn.to(H.dtype)


SCAN_IMPLS: dict = {
    "parallel_scan_log": _parallel_scan_log_impl,
    "linear_scan": _linear_scan_impl,
    "matrix_scan": _matrix_scan_impl,
    "matrix_affine_scan": _matrix_affine_scan_impl,
}
