"""mingru_amd -- minGRU scan hot path, MI355X-native.

Public surface (same names and signatures as chris-santiago/minGRU,
``src/mingru/__init__.py:39-84``): the five mixers, ``MinGRUBlock``,
``MinGRUStack`` and the scan primitives ``parallel_scan_log``, ``linear_scan``,
``matrix_scan``, ``matrix_affine_scan``.

The GPU backend, :mod:`mingru_amd.hip_scans`, is never imported by
``import mingru_amd``: its public names resolve lazily (PEP 562) on first
access, and the ``MINGRU_SCAN`` seam imports it only for GPU tensors.
"""

from .min_gru import *  # noqa: F401,F403
from .min_gru import __all__ as _min_gru_all

__version__ = "0.2.1+mi355x"

_BACKEND_EXPORTS = (
    "available",
    "ScanFallback",
    "SCAN_IMPLS",
    "angle_scan_impl",
    "delta_scan_impl",
)

__all__ = [*_min_gru_all, "__version__"]


def __getattr__(name: str) -> object:
    if name in _BACKEND_EXPORTS or name == "hip_scans":
        import importlib

        backend = importlib.import_module(f"{__name__}.hip_scans")
        return backend if name == "hip_scans" else getattr(backend, name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")


def __dir__() -> list[str]:
    return sorted(__all__)
