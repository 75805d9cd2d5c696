"""The C-ABI library: loads on a machine without a GPU, exports every entry point
that ``include/*.h`` declares, and rejects invalid arguments on the host before
any device call (status 1).  No kernel is launched here."""

import ctypes
import glob
import os
import re

import pytest

from mingru_amd import _native
from mingru_amd import build as hip_build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NULL = ctypes.c_void_p(0)


def _declared():
    names = []
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names += re.findall(r"^\s*(?:int|size_t|int64_t)\s+(mg_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(hip_build.LIB_PATH):
        hip_build.build()
    return _native.load()


def test_header_declares_entry_points():
    names = _declared()
    assert len(names) >= 16
    for fam in ("linear_scan", "log_scan", "affine_scan", "angle_scan", "delta"):
        assert any(fam in n for n in names), fam


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in _declared() if getattr(lib, n, None) is None]
    assert not missing, f"declared in include/ but not exported: {missing}"


def test_ctypes_table_matches_header(lib):
    assert sorted(_native._SIGNATURES) == _declared()
    assert sorted(_native.exported_names()) == _declared()


def test_workspace_queries(lib):
    assert lib.mg_linear_scan_workspace_bytes(16, 4096, 1024) >= 256
    assert lib.mg_log_scan_workspace_bytes(4, 1024, 256) >= 256
    # log scan forward record: (s, e) per column at every 8-step boundary
    assert lib.mg_log_scan_state_bytes(4, 1024, 256) == 4 * 128 * 2 * 256 * 4
    assert lib.mg_log_scan_state_bytes(2, 13, 5) == 2 * 2 * 2 * 5 * 4
    assert lib.mg_log_scan_state_bytes(0, 13, 5) == 0
    assert lib.mg_affine_scan_workspace_bytes(16, 4096, 256, 2, 1) >= 256
    assert lib.mg_angle_scan_workspace_bytes(8, 2048, 64, 8) >= 256
    # angle chunk products: 8x8 floats per (block, 16-token chunk), then, past 16
    # chunks (the two-level walk), 8x8 floats per (block, group of 8 chunks)
    assert lib.mg_angle_scan_state_bytes(8, 2048, 64, 8) == (128 + 16) * 64 * 8 * 64 * 4
    assert lib.mg_angle_scan_state_bytes(2, 256, 3, 4) == 16 * 6 * 16 * 4
    assert lib.mg_angle_scan_state_bytes(2, 257, 3, 4) == (17 + 3) * 6 * 16 * 4
    # delta: six padded 64 x 64 fp32 matrices per (batch, head, chunk)
    assert lib.mg_delta_workspace_bytes(8, 8, 8192, 1, 64, 64, 64) == 6 * 64 * 128 * 64 * 64 * 4
    # saved state: two padded matrices per (batch, head, chunk) -- the chunk-entry
    # state and the chunk's inverse (I + L)^-1 kept for the backward
    assert lib.mg_delta_state_bytes(8, 8, 8192, 1, 64, 64, 64) == 2 * 64 * 128 * 64 * 64 * 4
    # outside the envelope: the minimum / zero answer, never a crash
    assert lib.mg_affine_scan_workspace_bytes(1, 8, 1, 32, 1) == 256
    assert lib.mg_affine_scan_workspace_bytes(1, 8, 1, 16, 3) == 256
    # 16x16 blocks: one wave per block, (P, LA, LB) backward slots of 12 tagged words
    # per lane for each 32-step chunk, an aggregate and an inclusive copy
    assert lib.mg_affine_scan_workspace_bytes(2, 64, 3, 16, 4) == 256 + 2 * (6 * 2 * 12 * 64 * 8)
    # 8x8 blocks: two planes per wave
    assert lib.mg_affine_scan_workspace_bytes(2, 64, 3, 8, 4) == 256 + 2 * (4 * 2 * 12 * 64 * 8)
    assert lib.mg_delta_state_bytes(1, 1, 8, 1, 65, 64, 8) == 0


def test_invalid_arguments_are_rejected_on_the_host(lib):
    one = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    assert lib.mg_linear_scan_fwd(NULL, one, one, one, 1, 4, 4, one, 4096, NULL) == 1
    assert lib.mg_linear_scan_fwd(one, one, one, one, 0, 4, 4, one, 4096, NULL) == 1
    assert lib.mg_log_scan_fwd(one, one, NULL, NULL, 1, 4, 4, one, 4096, NULL) == 1
    assert lib.mg_log_scan_bwd(one, one, one, NULL, NULL, one, one, 1, 4, 4, one, 4096,
                               NULL) == 1  # no upstream gradient
    assert lib.mg_scan_workspace_errors(NULL, None, NULL) == 1
    assert lib.mg_affine_scan_fwd(one, one, one, one, 1, 4, 4, 3, 1, one, 4096, NULL) == 1
    assert lib.mg_angle_scan_fwd(one, one, one, one, one, one, one, 1, 4, 4, 6, 0, 3, 0, one,
                                 4096, NULL) == 1
    assert lib.mg_angle_scan_fwd(one, one, one, one, one, one, NULL, 1, 4, 4, 8, 1, 28, 0, one,
                                 4096, NULL) == 1  # no chunk-product buffer
    assert lib.mg_angle_scan_bwd(*([one] * 5), NULL, *([one] * 6), 1, 4, 4, 8, 1, 28, 0, one,
                                 4096, NULL) == 1
    # delta: d_k above 64, nh * chunk above 64, unknown dtype tag
    assert lib.mg_delta_fwd(one, one, one, one, one, one, one, one, 1, 1, 8, 1, 65, 64, 8, 1,
                            one, 1 << 20, NULL) == 1
    assert lib.mg_delta_fwd(one, one, one, one, one, one, one, one, 1, 1, 8, 2, 64, 64, 33, 1,
                            one, 1 << 20, NULL) == 1
    assert lib.mg_delta_fwd(one, one, one, one, one, one, one, one, 1, 1, 8, 1, 64, 64, 8, 7,
                            one, 1 << 20, NULL) == 1
    assert lib.mg_delta_bwd(*([one] * 11), NULL, 1, 1, 8, 1, 64, 64, 8, 1, one, 1 << 20,
                            NULL) == 1


def test_size_queries_are_cached_per_arguments(lib, monkeypatch):
    """The wrappers' size queries answer from a per-arguments cache: same value as the
    C ABI, one call per distinct argument tuple, and the cache is bounded."""
    from mingru_amd import hip_scans

    monkeypatch.setattr(hip_scans, "_sizes", {})
    calls = []
    real = lib.mg_log_scan_workspace_bytes

    class Counting:
        def __getattr__(self, name):
            fn = getattr(lib, name)

            def wrapped(*args):
                calls.append((name, args))
                return fn(*args)
            return wrapped

    monkeypatch.setattr(hip_scans, "_lib", lambda: Counting())
    for _ in range(3):
        assert hip_scans._size("mg_log_scan_workspace_bytes", 4, 1024, 256) == \
            real(4, 1024, 256)
    assert len(calls) == 1
    assert hip_scans._size("mg_log_scan_workspace_bytes", 4, 1025, 256) == real(4, 1025, 256)
    assert len(calls) == 2
    for t in range(1, 4100):
        hip_scans._size("mg_log_scan_workspace_bytes", 1, t, 8)
    assert len(hip_scans._sizes) <= 4096
