"""ctypes binding of libdmuon_amd.so (the C ABI declared in include/dmuon_amd.h).

There is no fallback: if the library is missing or fails to load, importing the compute
entry points raises. Build it with ``python -m dmuon_amd.csrc.build`` (``__graft_entry__.build``).
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional

_LIB_PATH = Path(__file__).resolve().parent / "csrc" / "libdmuon_amd.so"
_lib: Optional[ctypes.CDLL] = None

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2          # 16-bit product operands only

c_int, c_i64, c_f, c_d, c_vp = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_double, ctypes.c_void_p
c_fp = ctypes.POINTER(ctypes.c_float)
c_ip = ctypes.POINTER(ctypes.c_int)

NS_DIRECT = 0
NS_GRAM = 1

# DMUON_ABI_VERSION of include/dmuon_amd.h: the argument lists below are those of this
# version, and a library that reports another one is refused (its entry points would be
# called with the wrong arguments).
ABI_VERSION = 108

# name -> (restype, argtypes); mirrors include/dmuon_amd.h
_SIGNATURES = {
    "dmuon_last_error": (ctypes.c_char_p, []),
    "dmuon_abi_version": (c_int, []),
    "dmuon_profile_enable": (c_int, [c_int]),
    "dmuon_profile_collect": (c_int, [ctypes.POINTER(c_d), ctypes.POINTER(c_i64),
                                      ctypes.POINTER(c_d), ctypes.POINTER(c_d), c_int]),
    "dmuon_stream_copy": (c_int, [c_vp, c_vp, c_i64, c_vp]),
    "dmuon_syrk": (c_int, [c_int, c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp, c_i64, c_i64,
                           c_vp, c_i64, c_i64, c_int, c_int, c_int, c_f, c_f, c_f, c_vp, c_int,
                           c_vp, c_i64, c_vp]),
    "dmuon_syrk_workspace_size": (c_int, [c_int, c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp,
                                          c_i64, c_i64, c_vp, c_i64, c_i64, c_int, c_int, c_int,
                                          c_int, ctypes.POINTER(c_i64)]),
    "dmuon_ns_gemm": (c_int, [c_int, c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp, c_i64, c_i64,
                              c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_int, c_int, c_int,
                              c_f, c_f, c_vp, c_int, c_vp]),
    "dmuon_ns_gemm_final": (c_int, [c_int, c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp, c_i64,
                                    c_i64, c_int, c_int, c_int, c_f, c_f, c_vp, c_int, c_int,
                                    c_int, c_vp, c_int, c_vp, c_int, c_vp, c_int, c_f, c_f,
                                    c_int, c_vp]),
    "dmuon_syrk_bf16": (c_int, [c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp,
                                c_i64, c_i64, c_int, c_int, c_int, c_f, c_f, c_f, c_vp, c_int, c_vp]),
    "dmuon_ns_gemm_bf16": (c_int, [c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp, c_i64, c_i64,
                                   c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_int, c_int, c_int,
                                   c_f, c_f, c_vp, c_int, c_vp]),
    "dmuon_ns_gemm_final_bf16": (c_int, [c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp, c_i64,
                                         c_i64, c_int, c_int, c_int, c_f, c_f, c_vp, c_int, c_int,
                                         c_int, c_vp, c_int, c_vp, c_int, c_vp, c_int, c_f, c_f,
                                         c_int, c_vp]),
    "dmuon_muon_pre_partials": (c_int, [c_int, c_int]),
    "dmuon_muon_pre": (c_int, [c_vp, c_int, c_vp, c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp,
                               c_int, c_int, c_int, c_int, c_int, c_f, c_int, c_int, c_vp]),
    "dmuon_norm_finalize": (c_int, [c_vp, c_int, c_int, c_f, c_vp, c_vp, c_vp]),
    "dmuon_muon_update": (c_int, [c_vp, c_int, c_vp, c_int, c_i64, c_int, c_f, c_f, c_vp]),
    "dmuon_ns_plan": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int, ctypes.POINTER(c_int),
                              ctypes.POINTER(c_int), ctypes.POINTER(c_int), ctypes.POINTER(c_i64)]),
    "dmuon_muon_step_group": (c_int, [c_vp, c_int, c_vp, c_vp, c_vp, c_int, c_vp, c_int, c_int,
                                      c_int, c_int, c_int, c_d, c_d, c_d, c_int, c_int, c_fp,
                                      c_int, c_int, c_ip, c_int, c_f, c_vp, c_i64, c_int, c_vp]),
    "dmuon_muon_step_group_noalloc": (c_int, [c_vp, c_int, c_vp, c_vp, c_vp, c_int, c_vp, c_int,
                                              c_int, c_int, c_int, c_int, c_d, c_d, c_d, c_int,
                                              c_int, c_fp, c_int, c_int, c_ip, c_int, c_f, c_int,
                                              c_vp]),
    "dmuon_noalloc_init": (c_int, [ctypes.POINTER(c_vp), ctypes.POINTER(c_i64)]),
    "dmuon_muon_stage_group": (c_int, [c_vp, c_int, c_vp, c_vp, c_int, c_int, c_int, c_int, c_d,
                                       c_int, c_int, c_int, c_f, c_vp, c_i64, c_int, c_vp]),
    "dmuon_muon_apply_group": (c_int, [c_vp, c_int, c_vp, c_int, c_int, c_int, c_int, c_int, c_d,
                                       c_d, c_fp, c_int, c_int, c_ip, c_int, c_vp, c_i64, c_int,
                                       c_vp]),
    "dmuon_newton_schulz_group": (c_int, [c_vp, c_int, c_vp, c_int, c_int, c_int, c_int, c_int,
                                          c_fp, c_int, c_int, c_ip, c_int, c_f, c_vp, c_i64,
                                          c_int, c_vp]),
    "dmuon_adamw_multi": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_i64, c_int, c_int,
                                  c_int, c_int, c_f, c_f, c_f, c_f, c_f, c_f, c_f, c_f, c_vp]),
    "dmuon_segmented_l2_norm_sq": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_vp,
                                           c_vp]),
    "dmuon_segmented_scale": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_vp,
                                      c_vp]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)


def lib_path() -> Path:
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    """Loads (once) and returns the library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not _LIB_PATH.exists():
        raise RuntimeError(
            f"{_LIB_PATH} is missing: build the HIP kernels first "
            "(python -m dmuon_amd.csrc.build). dmuon_amd has no CPU fallback."
        )
    _lib = _bind(ctypes.CDLL(os.fspath(_LIB_PATH)), _LIB_PATH)
    return _lib


def _bind(handle, path) -> ctypes.CDLL:
    """Checks the library's ABI version, then sets every entry point's argument types."""
    version_fn = getattr(handle, "dmuon_abi_version", None)
    if version_fn is None:
        raise RuntimeError(f"{path} does not export dmuon_abi_version: not a dmuon_amd library")
    version_fn.restype = c_int
    version_fn.argtypes = []
    version = int(version_fn())
    if version != ABI_VERSION:
        raise RuntimeError(
            f"{path} reports ABI version {version}, this binding expects {ABI_VERSION}: the "
            "library is stale or from another checkout; rebuild it (python -m "
            "dmuon_amd.csrc.build)")
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    return handle


def check(rc: int) -> None:
    if rc != 0:
        msg = lib().dmuon_last_error().decode(errors="replace")
        raise RuntimeError(f"dmuon_amd: {msg}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))


PROFILE_CLASSES = ("pre", "norm", "syrk", "poly", "gemm", "final", "adamw", "clip")


def profile_enable(on: bool) -> None:
    check(lib().dmuon_profile_enable(1 if on else 0))


def profile_collect() -> dict:
    """Per kernel class: {"ms", "launches", "flops", "bytes"} since the last collect."""
    n = len(PROFILE_CLASSES)
    ms, cnt = (c_d * n)(), (c_i64 * n)()
    fl, by = (c_d * n)(), (c_d * n)()
    check(lib().dmuon_profile_collect(ms, cnt, fl, by, n))
    return {name: {"ms": ms[i], "launches": cnt[i], "flops": fl[i], "bytes": by[i]}
            for i, name in enumerate(PROFILE_CLASSES)}


def plan(rows: int, cols: int, batch: int, tile: int = 0, num_cus: int = 0,
         backend: int = NS_DIRECT):
    """(tile, m_pad, n_pad, workspace_bytes) for a group of same-shape matrices."""
    t, mp, np_, ws = c_int(), c_int(), c_int(), c_i64()
    check(lib().dmuon_ns_plan(rows, cols, batch, tile, num_cus, backend, ctypes.byref(t),
                              ctypes.byref(mp), ctypes.byref(np_), ctypes.byref(ws)))
    return t.value, mp.value, np_.value, ws.value


def restart_array(restarts) -> tuple:
    """(ctypes int array or None, count) for a restart-iteration list."""
    r = [int(i) for i in restarts]
    return ((c_int * len(r))(*r) if r else None), len(r)
