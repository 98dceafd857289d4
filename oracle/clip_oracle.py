"""CPU oracle for segmented gradient clipping -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this module, and only as the checker; ``dmuon_amd`` never does.

Restates, in numpy, the reference's segment-local clipping (``dmuon/fast_clip.py:383-437``,
``clip_grad_norm_buckets_``, whose device half is ``dmuon/csrc/fast_clip_kernel.cu:34-107``):

    sq[s]    = sum over the bucket's grads of float(x)^2          (fp64 here: exact to the
                                                                    fp32 result's precision)
    norm[s]  = sqrt(sq[s])
    coef[s]  = min(max_norm / (norm[s] + 1e-6), 1)                  (1 if max_norm is None)
    x       <- dtype(float(x) * coef[s])                            (only when max_norm given)

and the global-norm strategy of ``dmuon/grad_clip.py:109-155`` / ``:268-321`` for p = 2:
per-tensor norms rounded to the gradient dtype (``torch._foreach_norm`` returns them in that
dtype), the total as the 2-norm of those, one coefficient for all tensors.

Pinning (tests/test_clip.py): the reference tests' known answers
(``tests/unit/test_fast_clip.py:37-61``: norms 5 / 12 / 17, coefficients 6/(12+1e-6) and
6/(17+1e-6)), numpy.linalg.norm, and a planted mistake (missing square root, coefficient not
clamped, epsilon on the wrong side) that must fail them.
"""
from __future__ import annotations

from typing import Optional, Sequence

import numpy as np

from .ns_oracle import round_bf16


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 values rounded to `dtype` ('fp32', 'fp16', 'bf16'), returned as float32."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "fp32":
        return x
    if dtype == "fp16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return round_bf16(x)
    raise ValueError(dtype)


def segment_sumsq(buckets: Sequence[Sequence[np.ndarray]]) -> np.ndarray:
    """Per-bucket sum of squares (fp64 accumulation of the float32 values)."""
    out = np.zeros(len(buckets), dtype=np.float64)
    for s, grads in enumerate(buckets):
        for g in grads:
            x = np.asarray(g, dtype=np.float32).astype(np.float64)
            out[s] += float(np.dot(x.ravel(), x.ravel()))
    return out


def clip_coefs(norms: np.ndarray, max_norm: Optional[float]) -> np.ndarray:
    norms = np.asarray(norms, dtype=np.float64)
    if max_norm is None:
        return np.ones_like(norms)
    with np.errstate(divide="ignore", invalid="ignore"):
        return np.minimum(float(max_norm) / (norms + 1e-6), 1.0)


def clip_buckets(buckets, dtypes, max_norm: Optional[float]):
    """Segment-local clip. buckets[s] is a list of float32 arrays holding values of
    dtypes[s][k]. Returns (norms, coefs, clipped buckets) with coefs as float32."""
    norms = np.sqrt(segment_sumsq(buckets))
    coefs = clip_coefs(norms, max_norm).astype(np.float32)
    out = []
    for s, grads in enumerate(buckets):
        if max_norm is None:
            out.append([np.asarray(g, dtype=np.float32).copy() for g in grads])
        else:
            out.append([scale(g, coefs[s], dt) for g, dt in zip(grads, dtypes[s])])
    return norms, coefs, out


def scale(g: np.ndarray, coef: float, dtype: str) -> np.ndarray:
    """x <- dtype(float(x) * coef): one fp32 product, rounded to the storage dtype."""
    return round_to(np.asarray(g, dtype=np.float32) * np.float32(coef), dtype)


def global_norm_p2(grads: Sequence[np.ndarray], dtypes: Sequence[str]) -> float:
    """grad_clip.py's total norm for p = 2: per-tensor 2-norms rounded to each gradient's
    dtype, then the 2-norm of those (as float32 values)."""
    per = []
    for g, dt in zip(grads, dtypes):
        x = np.asarray(g, dtype=np.float32).astype(np.float64)
        n32 = np.array([np.sqrt(np.dot(x.ravel(), x.ravel()))], dtype=np.float32)
        per.append(float(round_to(n32, dt).ravel()[0]))
    return float(np.sqrt(np.sum(np.square(np.asarray(per, dtype=np.float64)))))
