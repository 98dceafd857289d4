"""Builds libdmuon_amd.so (gfx950) in-tree with hipcc.

    python -m dmuon_amd.csrc.build          # or: python dmuon_amd/csrc/build.py

Every call recompiles (the in-tree .so travels with the source tree to the GPU host).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
SOURCES = ["ns_gemm.hip", "ew_kernels.hip", "adamw.hip", "clip.hip", "abi.hip"]
LIB_NAME = "libdmuon_amd.so"
ARCH = "gfx950"

# -packed-fp32-ops: keep hipcc from emitting v_pk_{add,mul,fma}_f32 (unreliable on the target
# pool); the host pass prints a harmless "not a recognized feature" warning for it.
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # no a*b+c contraction: the momentum and weight updates round each op like the reference
    "-ffp-contract=off",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (need ROCm in /opt/rocm)")


def lib_path() -> Path:
    return HERE / LIB_NAME


def build(verbose: bool = False) -> Path:
    out = lib_path()
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), *FLAGS, "-I", str(ROOT / "include"), *[str(HERE / s) for s in SOURCES], "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (proc.stderr or "").splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    _check_launch_stubs(tmp)
    os.replace(tmp, out)
    return out


def _check_launch_stubs(so: Path) -> None:
    """clang can silently skip a kernel template's host launch stub (the library then fails
    to load with an undefined __device_stub__ symbol); catch that at build time."""
    nm = shutil.which("nm")
    if not nm:
        return
    proc = subprocess.run([nm, "-D", "--undefined-only", str(so)], capture_output=True, text=True)
    missing = [l.split()[-1] for l in proc.stdout.splitlines() if "__device_stub__" in l]
    if missing:
        so.unlink(missing_ok=True)
        raise RuntimeError("hipcc dropped kernel launch stubs: " + ", ".join(missing[:4]))


if __name__ == "__main__":
    p = build(verbose=True)
    print(f"built {p}")
