"""Newton-Schulz orthogonalisation on MI355X (host side of the HIP kernels in ``dmuon_amd/csrc``).

Public surface mirrors ``dmuon/optim/newton_schulz.py`` of X-Square-Robot/dmuon:
coefficient sets (``:45-75``), the :class:`NewtonSchulz` configuration object (``:81-219``),
``direct_newton_schulz`` (``:225-273``), ``newton_schulz`` (``:299-327``) and
``gram_newton_schulz`` (``:333-448``).

Two device algorithms, both on the fp16 MFMA NT kernels, for X = G / (||G||_F + eps) oriented
so that X has m = min(rows, cols) rows and n = max(rows, cols) columns:

``backend="direct"`` (``direct_newton_schulz``), per coefficient triple ``(a, b, c)``::

    A = X X^T            (SYRK: upper-triangle tiles, mirrored)
    P = b*A + c*A A^T    (the same SYRK kernel with C = A in the epilogue)
    X = a*X + P X        (GEMM against the transposed copy of X)

``backend="gram"`` (``gram_newton_schulz``, the reference's default), in fp16 as the reference
runs it: R = X X^T once, then per step only m x m products -- ``Z = c R R + b R``,
``P = Z + a I``, ``Q <- P Q`` (``Q = P`` after a start or restart) and, unless the next step is
the last or a restart, ``R <- P R P`` -- with ``X <- Q X; R = X X^T`` at each restart index and
``U = Q X`` at the end (``newton_schulz.py:364-448``). For n > m this needs fewer flops than the
direct form. bf16 is not accurate enough for this recurrence (R's small eigenvalues drown in
its rounding). Both backends stage X as fp16 of the normalised input times a power of two (the
reference computes both in fp16 too, ``newton_schulz.py:266,391``).

Results differ from the reference's fp16 pipeline by rounding (fp32 accumulation and fp32
epilogues here; exactly symmetric products).

There is no CPU path: CPU tensors raise.
"""
from __future__ import annotations

import ctypes
import logging
import math
from typing import Optional, Sequence

import torch
from torch import Tensor

from dmuon_amd import _C
from dmuon_amd._scratch import StreamScratch
from dmuon_amd.optim.syrk_dispatch import KERNEL_NAME, get_backend_status, get_ns_backend  # noqa: F401

logger = logging.getLogger(__name__)

# ---------------------------------------------------------------------------------------------
# Coefficient sets (values as in dmuon/optim/newton_schulz.py:45-75)
# ---------------------------------------------------------------------------------------------
#: @YouJiacheng's 5-step coefficients (newton_schulz.py:45-51)
YOU_COEFFICIENTS = [
    [4.0848, -6.8946, 2.9270],
    [3.9505, -6.3029, 2.6377],
    [3.7418, -5.5913, 2.3037],
    [2.8769, -3.1427, 1.2046],
    [2.8366, -3.0525, 1.2012],
]

# Polar Express (arXiv:2505.16932) with a 1.05 safety factor (newton_schulz.py:53-71)
_SAFETY_FACTOR = 1.05
_UNMODIFIED_POLAR_EXPRESS = [
    (8.28721201814563, -23.595886519098837, 17.300387312530933),
    (4.107059111542203, -2.9478499167379106, 0.5448431082926601),
    (3.9486908534822946, -2.908902115962949, 0.5518191394370137),
    (3.3184196573706015, -2.488488024314874, 0.51004894012372),
    (2.300652019954817, -1.6689039845747493, 0.4188073119525673),
]
POLAR_EXPRESS_COEFFICIENTS = [
    (a / _SAFETY_FACTOR, b / _SAFETY_FACTOR ** 3, c / _SAFETY_FACTOR ** 5)
    for (a, b, c) in _UNMODIFIED_POLAR_EXPRESS
]

#: Keller Jordan's constant quintic, the benchmark baseline of the reference
#: (benchmarks/bench_optimizer.py:41-60): five iterations of (3.4445, -4.7750, 2.0315).
KELLER_COEFFICIENTS = [(3.4445, -4.7750, 2.0315)] * 5

DEFAULT_COEFFICIENTS = POLAR_EXPRESS_COEFFICIENTS
DEFAULT_RESTART_ITERATIONS = [2]

_KERNEL_ALIASES = {"auto": KERNEL_NAME, "hip": KERNEL_NAME, KERNEL_NAME: KERNEL_NAME,
                   # the reference's bit-exact choice; the HIP kernels are deterministic
                   "cublas": KERNEL_NAME}
_UNAVAILABLE_KERNELS = {"quack": "Tri Dao quack (SM90+ CuTeDSL)",
                        "cute_sm80": "CuTeDSL SM80 SYRK"}


def _float_dtype_code(t: Tensor) -> int:
    if t.dtype == torch.float32:
        return _C.DTYPE_F32
    if t.dtype == torch.bfloat16:
        return _C.DTYPE_BF16
    raise TypeError(f"dmuon_amd: unsupported dtype {t.dtype} (float32 or bfloat16)")


def _require_gpu(t: Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(
            f"dmuon_amd: {what} must be a GPU tensor; this build runs only on the HIP kernels "
            "(no CPU path)")


def _coeff_array(coefficients: Sequence[Sequence[float]]):
    flat = [float(v) for triple in coefficients for v in triple]
    if len(flat) == 0 or len(flat) % 3:
        raise ValueError("coefficients must be a non-empty list of (a, b, c) triples")
    return (ctypes.c_float * len(flat))(*flat), len(flat) // 3


def _backend_code(backend: str) -> int:
    if backend == "direct":
        return _C.NS_DIRECT
    if backend == "gram":
        return _C.NS_GRAM
    raise ValueError(f"backend must be 'gram' or 'direct', got '{backend}'")


def _restarts(restart_iterations) -> list:
    if restart_iterations is None:
        return list(DEFAULT_RESTART_ITERATIONS)
    out = []
    for r in restart_iterations:
        if not isinstance(r, int):
            raise TypeError("restart_iterations must be a list of ints")
        out.append(r)
    return out


def _ptr_array(tensors: Sequence[Tensor], device: torch.device) -> Tensor:
    host = torch.tensor([t.data_ptr() for t in tensors], dtype=torch.int64, pin_memory=True)
    return host.to(device, non_blocking=True)


# NS scratch of the stand-alone functions, one buffer per (device, stream): calls on two
# streams of one device do not share it
_WORKSPACE = StreamScratch()


def newton_schulz_batched(
    Gs: Sequence[Tensor],
    coefficients: Sequence[Sequence[float]],
    eps: float = 1e-7,
    out: Optional[Sequence[Tensor]] = None,
    tile: int = 0,
    backend: str = "direct",
    restart_iterations: Sequence[int] = (),
) -> list[Tensor]:
    """NS of several same-shape, same-dtype 2-D GPU matrices in one grouped launch chain.

    ``backend`` "direct" or "gram" (with ``restart_iterations``), as described above."""
    if len(Gs) == 0:
        return []
    G0 = Gs[0]
    _require_gpu(G0, "G")
    if G0.dim() != 2:
        raise ValueError(f"Newton-Schulz needs 2-D matrices, got shape {tuple(G0.shape)}")
    for g in Gs:
        if g.shape != G0.shape or g.dtype != G0.dtype or g.device != G0.device:
            raise ValueError("newton_schulz_batched: matrices must share shape, dtype and device")
    work_dtype = G0.dtype if G0.dtype in (torch.float32, torch.bfloat16) else torch.float32
    ins = [g if (g.dtype == work_dtype and g.is_contiguous()) else g.to(work_dtype).contiguous()
           for g in Gs]
    if out is None:
        outs = [torch.empty_like(g, dtype=work_dtype, memory_format=torch.contiguous_format)
                for g in Gs]
    else:
        outs = list(out)
        for o in outs:
            if o.shape != G0.shape or not o.is_contiguous() or o.dtype != work_dtype:
                raise ValueError("out tensors must be contiguous with the input shape and dtype")
    rows, cols = G0.shape
    L = len(ins)
    coeff, T = _coeff_array(coefficients)
    code = _backend_code(backend)
    rst, n_rst = _C.restart_array(restart_iterations if code == _C.NS_GRAM else ())
    num_cus = torch.cuda.get_device_properties(G0.device).multi_processor_count
    t, _mp, _np, nbytes = _C.plan(rows, cols, L, tile, num_cus, code)
    cur = torch.cuda.current_stream(G0.device)
    ws = _WORKSPACE.get(G0.device, cur, nbytes)
    gp = _ptr_array(ins, G0.device)
    op = _ptr_array(outs, G0.device)
    stream = cur.cuda_stream
    _C.call("dmuon_newton_schulz_group", gp.data_ptr(), _float_dtype_code(ins[0]), op.data_ptr(),
            _float_dtype_code(outs[0]), rows, cols, L, 0, coeff, T, code, rst, n_rst, float(eps),
            ws.data_ptr(), ws.numel(), t, stream)
    if out is None and G0.dtype != work_dtype:
        return [o.to(G0.dtype) for o in outs]
    return outs


def direct_newton_schulz(
    G: Tensor,
    steps: int = 5,
    eps: float = 1e-7,
    coefficients: Optional[list[list[float]]] = None,
) -> Tensor:
    """Classic parameter-space NS (``newton_schulz.py:225-273``). ``steps`` is ignored, as in
    the reference: the iteration count is ``len(coefficients)``."""
    if coefficients is None:
        coefficients = DEFAULT_COEFFICIENTS
    return newton_schulz_batched([G], coefficients, eps)[0]


def gram_newton_schulz(
    G: Tensor,
    steps: int = 5,
    eps: float = 1e-7,
    coefficients: Optional[list[list[float]]] = None,
    restart_iterations: Optional[list[int]] = None,
    deterministic: bool = False,
) -> Tensor:
    """Gram-space NS (``newton_schulz.py:333-448``) on the HIP kernels.

    ``restart_iterations`` defaults to ``[2]``; ``deterministic`` is accepted for compatibility
    (the HIP kernels are deterministic).
    """
    if coefficients is None:
        coefficients = DEFAULT_COEFFICIENTS
    return newton_schulz_batched([G], coefficients, eps, backend="gram",
                                 restart_iterations=_restarts(restart_iterations))[0]


def newton_schulz(
    G: Tensor,
    steps: int = 5,
    eps: float = 1e-7,
    coefficients: Optional[list[list[float]]] = None,
    restart_iterations: Optional[list[int]] = None,
) -> Tensor:
    """Default public NS (``newton_schulz.py:299-327``): routes to :func:`gram_newton_schulz`."""
    return gram_newton_schulz(G, steps=steps, eps=eps, coefficients=coefficients,
                              restart_iterations=restart_iterations)


class NewtonSchulz:
    """Configurable Newton-Schulz backend (``newton_schulz.py:81-219``).

    Args mirror the reference: ``backend`` in {"gram", "direct"} (ValueError otherwise),
    ``kernel`` in {"auto", "hip", "hip_gfx950", "cublas"} -- every accepted value selects the
    HIP kernels; "quack" and "cute_sm80" name NVIDIA kernels and raise at construction, as the
    reference does for an unavailable kernel. ``coefficients=None`` uses the Polar-Express set;
    ``restart_iterations`` (gram only) defaults to ``[2]``; ``deterministic`` is accepted (the
    HIP path is bit-reproducible run to run).
    """

    def __init__(
        self,
        backend: str = "gram",
        kernel: str = "auto",
        coefficients: Optional[list[list[float]]] = None,
        restart_iterations: Optional[list[int]] = None,
        deterministic: bool = False,
    ):
        if backend not in ("gram", "direct"):
            raise ValueError(f"backend must be 'gram' or 'direct', got '{backend}'")
        if kernel in _UNAVAILABLE_KERNELS:
            raise ValueError(
                f"kernel={kernel!r} ({_UNAVAILABLE_KERNELS[kernel]}) is not available on MI355X; "
                f"use 'auto' (HIP gfx950 SYRK)")
        if kernel not in _KERNEL_ALIASES:
            valid = ", ".join(sorted(set(_KERNEL_ALIASES) | set(_UNAVAILABLE_KERNELS)))
            raise ValueError(f"kernel={kernel!r} is not a valid SYRK backend; choose one of: {valid}")
        if coefficients is not None:
            _coeff_array(coefficients)  # validates shape
        self.backend = backend
        self.kernel = _KERNEL_ALIASES[kernel]
        self.coefficients = coefficients
        self.restart_iterations = _restarts(restart_iterations)
        self.deterministic = True

    def resolved_coefficients(self) -> list:
        return list(DEFAULT_COEFFICIENTS if self.coefficients is None else self.coefficients)

    def local(self, G: Tensor, steps: int) -> Tensor:
        """NS of one full matrix (``newton_schulz.py:194-212``)."""
        return newton_schulz_batched([G], self.resolved_coefficients(), backend=self.backend,
                                     restart_iterations=self.restart_iterations)[0]

    def restart_codes(self) -> list:
        """The restart list the device algorithm receives (empty for the direct backend)."""
        return list(self.restart_iterations) if self.backend == "gram" else []

    def __repr__(self) -> str:
        coeff = "default" if self.coefficients is None else f"{len(self.coefficients)}-step custom"
        return f"NewtonSchulz(backend={self.backend!r}, kernel={self.kernel!r}, coefficients={coeff})"


def ns_useful_flops(rows: int, cols: int, steps: int = 5, backend: str = "direct",
                    restart_iterations: Sequence[int] = (2,)) -> float:
    """Useful NS FLOPs of one matrix (one triangle of each symmetric product, full GEMMs),
    m = min(rows, cols), n = max(rows, cols).

    direct: T*[m(m+1)n + m(m+1)m + 2 m^2 n].
    gram: (1 + r) m(m+1)n Gram products and r + 1 Q X products (2 m^2 n), r = the restarts
    inside (0, T); per step m(m+1)m for Z, 2 m^3 for Q <- P Q except right after a (re)start,
    and, unless the next step is the last or a restart, the R update P R P: m(m+1)m each for
    W = P R and W P. The Q update is a full product: 2 m^3."""
    m, n = min(rows, cols), max(rows, cols)
    sq, gram_mn, qx = m * (m + 1) * m, m * (m + 1) * n, 2.0 * m * m * n
    if backend == "direct":
        return float(steps) * (gram_mn + sq + qx)
    rs = {int(r) for r in restart_iterations if 0 < int(r) < steps}
    total = (1 + len(rs)) * (gram_mn + qx)
    for i in range(steps):
        total += sq
        if i != 0 and i not in rs:
            total += 2.0 * m * m * m
        if i + 1 < steps and (i + 1) not in rs:
            total += 2 * sq
    return float(total)


def muon_update_scale(rows: int, cols: int) -> float:
    """Shape-dependent update scale 0.2*sqrt(max(m, n)) (``muon.py:1731-1733``)."""
    return 0.2 * math.sqrt(max(rows, cols))
