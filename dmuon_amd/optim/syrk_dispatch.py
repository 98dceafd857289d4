"""The symmetric-product seam of the reference (``dmuon/optim/syrk_dispatch.py:582-651``) on
the gfx950 HIP kernel.

``syrk_or_cublas(A, D, B=None, C=None, alpha=1.0, beta=1.0, diag_add=0.0)`` computes
``D = alpha * A @ B^T + beta * C + diag_add * I`` in place, as the reference does for
``gram_newton_schulz``'s fp16 operands (``newton_schulz.py:376-433``). The reference chooses
between a CuTeDSL / quack SYRK and cuBLAS per shape; here one kernel family serves every call:
upper-triangle tiles with the mirror written by the epilogue, fp32 accumulation, fp16 or bf16
operands (``dmuon_syrk``). Shapes the kernel cannot read in place (M not a multiple of the
tile, K not a multiple of 64, unaligned rows) run on zero-padded copies in a workspace this
module keeps per device and stream, which is where the reference would fall back to cuBLAS.

As in the reference, ``B`` other than ``A`` is allowed only when ``A @ B^T`` is symmetric (the
caller's responsibility: only one triangle is computed), a non-K-contiguous operand is copied
with a warning (``syrk_sm80.py:508-523``) and ``D`` must be contiguous (``:524``).
"""
from __future__ import annotations

import ctypes
import logging
from typing import Optional

import torch
from torch import Tensor

from dmuon_amd import _C
from dmuon_amd._scratch import StreamScratch

logger = logging.getLogger(__name__)

KERNEL_NAME = "hip_gfx950"
_OPERAND_CODES = {torch.float16: _C.DTYPE_F16, torch.bfloat16: _C.DTYPE_BF16}


# the padded path's operand copies, one buffer per (device, stream)
_SCRATCH = StreamScratch()


def _k_contiguous(t: Tensor, name: str) -> Tensor:
    if t.stride(-1) != 1:
        logger.warning(
            "syrk_or_cublas: %s is not K-contiguous (shape=%s, stride=%s); falling back to an "
            "implicit .contiguous() copy. Call .contiguous() on the input to avoid this.",
            name, tuple(t.shape), tuple(t.stride()))
        return t.contiguous()
    return t


def _batch_stride(t: Tensor) -> int:
    return int(t.stride(0)) if t.dim() == 3 else 0


def syrk_or_cublas(
    A: Tensor,
    D: Tensor,
    B: Optional[Tensor] = None,
    C: Optional[Tensor] = None,
    alpha: float = 1.0,
    beta: float = 1.0,
    diag_add: float = 0.0,
    tile: int = 0,
) -> None:
    """``D = alpha * A @ B^T + beta * C + diag_add * I`` (``syrk_dispatch.py:582-651``).

    ``A`` is ``(M, K)`` or a batch ``(L, M, K)`` of fp16 / bf16 GPU matrices; ``D`` (and ``C``)
    ``(M, M)`` / ``(L, M, M)`` of the same dtype. ``B=None`` means ``B = A``. ``tile`` (0 =
    automatic, 128 or 256) is a tuning knob with no reference counterpart."""
    if A.dim() not in (2, 3):
        raise ValueError(f"syrk_or_cublas: A must be 2-D (M, K) or 3-D (L, M, K), got {tuple(A.shape)}")
    if A.dtype not in _OPERAND_CODES:
        raise TypeError(f"syrk_or_cublas: A must be float16 or bfloat16, got {A.dtype} "
                        "(the HIP SYRK kernel has 16-bit operands only)")
    if not A.is_cuda:
        raise RuntimeError("syrk_or_cublas: A must be a GPU tensor (dmuon_amd has no CPU path)")
    M, K = int(A.shape[-2]), int(A.shape[-1])
    L = int(A.shape[0]) if A.dim() == 3 else 1
    mshape = (A.shape[0], M, M) if A.dim() == 3 else (M, M)
    for name, t, shape in (("D", D, mshape), ("B", B, A.shape), ("C", C, mshape)):
        if t is None:
            continue
        if tuple(t.shape) != tuple(shape):
            raise ValueError(f"syrk_or_cublas: {name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
        if t.dtype != A.dtype or t.device != A.device:
            raise ValueError(f"syrk_or_cublas: {name} must match A's dtype and device")
    if not D.is_contiguous():
        raise ValueError("syrk_or_cublas: output D must be contiguous")
    A = _k_contiguous(A, "A")
    if B is not None:
        if B.data_ptr() == A.data_ptr() and B.stride() == A.stride():
            B = None
        else:
            B = _k_contiguous(B, "B")
    if C is not None:
        C = _k_contiguous(C, "C")
    code = _OPERAND_CODES[A.dtype]
    args = (A.data_ptr(), A.stride(-2), _batch_stride(A),
            None if B is None else B.data_ptr(), 0 if B is None else B.stride(-2),
            0 if B is None else _batch_stride(B),
            None if C is None else C.data_ptr(), 0 if C is None else C.stride(-2),
            0 if C is None else _batch_stride(C),
            D.data_ptr(), D.stride(-2), _batch_stride(D), M, K, L)
    need = ctypes.c_int64()
    _C.call("dmuon_syrk_workspace_size", code, *args, int(tile), ctypes.byref(need))
    stream = torch.cuda.current_stream(A.device)
    ws = _SCRATCH.get(A.device, stream, need.value) if need.value > 0 else None
    _C.call("dmuon_syrk", code, *args, float(alpha), float(beta), float(diag_add), None,
            int(tile), None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(),
            stream.cuda_stream)


def get_ns_backend() -> str:
    """One-line description of the NS kernel (``syrk_dispatch.py:42-66``)."""
    return ("Gram-space NS with restarts / direct NS in SYRK form · kernel=hip_gfx950 "
            "(MI355X CDNA4, fp16 / bf16 MFMA 16x16x32)")


def get_backend_status() -> dict:
    """Diagnostic snapshot (``syrk_dispatch.py:69-84``)."""
    status = {
        "arch": "gfx950",
        "auto_choice": KERNEL_NAME,
        "library": str(_C.lib_path()),
        "library_built": _C.lib_path().exists(),
        "quack_available": False,
        "cute_sm80_available": False,
        "gpu_visible": torch.cuda.is_available(),
    }
    if status["library_built"]:
        status["abi_version"] = _C.lib().dmuon_abi_version()
    return status
