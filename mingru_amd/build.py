"""Build recipe for the mingru_amd HIP library (``libmingru_hip.so``, gfx950).

Compiles every ``csrc/*.hip`` with ``hipcc --offload-arch=gfx950`` into one
shared library next to this file (``mingru_amd/_lib/``), which travels with
the source tree.  The library links against the HIP runtime that PyTorch
itself loads (``torch/lib/libamdhip64.so``), so device pointers and streams
handed over from torch belong to the same runtime instance.

Usage: ``python -m mingru_amd.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_lib")
LIB_NAME = "libmingru_hip.so"
LIB_PATH = os.path.join(OUT_DIR, LIB_NAME)
ARCH = os.environ.get("MINGRU_HIP_ARCH", "gfx950")

# Packed fp32 VALU ops are disabled: plain float code only.
HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    "-Wno-unused-command-line-argument",
]


# Per-source extra flags.  scan_elementwise.hip issues its header atomics from one
# thread; LLVM's atomic optimizer would turn each into a wave reduction that waits
# for the atomic's result at once, ahead of the chunk loads it should overlap.
EXTRA_FLAGS = {
    "scan_elementwise.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the HIP library cannot be built")
    return path


def _torch_lib_dir() -> str | None:
    try:
        import torch  # noqa: F401
    except ImportError:
        return None
    import torch

    d = os.path.join(os.path.dirname(torch.__file__), "lib")
    return d if os.path.exists(os.path.join(d, "libamdhip64.so")) else None


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile all kernels and link ``libmingru_hip.so``; returns its path."""
    os.makedirs(OUT_DIR, exist_ok=True)
    obj_dir = os.path.join(OUT_DIR, "obj")
    os.makedirs(obj_dir, exist_ok=True)
    hipcc = _hipcc()
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    procs = []
    objs = []
    for src in sources:
        obj = os.path.join(obj_dir, os.path.basename(src)[:-4] + ".o")
        objs.append(obj)
        extra = EXTRA_FLAGS.get(os.path.basename(src), [])
        cmd = [hipcc, *HIPCC_FLAGS, *extra, "-I", CSRC, "-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        text = "\n".join(
            line for line in out.decode(errors="replace").splitlines()
            if "packed-fp32-ops" not in line
        )
        if p.returncode != 0:
            failed.append((src, text))
        elif verbose and text.strip():
            print(text, flush=True)
    if failed:
        msg = "\n".join(f"--- {s}\n{t}" for s, t in failed)
        raise RuntimeError(f"HIP compilation failed:\n{msg}")
    tmp = LIB_PATH + ".tmp"
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    tdir = _torch_lib_dir()
    if tdir:
        # Resolve the HIP runtime to torch's copy at load time.
        link += [f"-L{tdir}", "-lamdhip64", f"-Wl,-rpath,{tdir}"]
    if verbose:
        print(" ".join(link), flush=True)
    res = subprocess.run(link, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if res.returncode != 0:
        raise RuntimeError("HIP link failed:\n" + res.stdout.decode(errors="replace"))
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
