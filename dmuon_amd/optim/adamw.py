"""Fused decoupled AdamW on the HIP kernel ``dmuon_adamw_multi``.

``fused_adamw_`` updates one bucket of the reference's ``_adamw_update_batch``
(``dmuon/optim/muon.py:1857-1916``): tensors that share the post-increment step count, the
parameter dtype (which the ``exp_avg``/``exp_avg_sq`` state shares, ``zeros_like(param)``) and
the gradient dtype. The dozen ``torch._foreach`` passes of the reference become one pass over
HBM; the per-element arithmetic and its rounding points are the same (see ``adamw.hip``).
There is no CPU path: tensors must live on the GPU.
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch
from torch import Tensor

from .. import _C

_CODES = {torch.float32: _C.DTYPE_F32, torch.bfloat16: _C.DTYPE_BF16}


def adamw_scalars(step: int, lr: float, betas: tuple[float, float], weight_decay: float,
                  eps: float) -> dict:
    """The scalars of one step, derived in double exactly as the reference derives them."""
    beta1, beta2 = float(betas[0]), float(betas[1])
    bc1 = 1.0 - beta1 ** step
    bc2 = 1.0 - beta2 ** step
    return {
        "apply_wd": 1 if weight_decay > 0 else 0,
        "wd_scale": 1.0 - lr * weight_decay,
        "beta1": beta1, "alpha1": 1.0 - beta1,
        "beta2": beta2, "alpha2": 1.0 - beta2,
        "bc2_sqrt": bc2 ** 0.5,
        "eps": float(eps),
        "neg_step": -(lr / bc1),
    }


def fused_adamw_(params: Sequence[Tensor], grads: Sequence[Tensor], exp_avgs: Sequence[Tensor],
                 exp_avg_sqs: Sequence[Tensor], *, step: int, lr: float,
                 betas: tuple[float, float], weight_decay: float, eps: float,
                 publish: Optional[Sequence[Optional[Tensor]]] = None) -> None:
    """In-place AdamW step of one bucket (same step, param dtype and grad dtype).

    ``publish``: optional forward copies (one per param, or None) that receive the new param
    rounded to their dtype in the same pass -- the owner's master -> forward publish; all of
    them share one dtype. Raises ``ValueError`` for mismatched lists, shapes or dtypes and
    ``RuntimeError`` for tensors that are not on the GPU or not contiguous (gradients are made
    contiguous).
    """
    n = len(params)
    if not (len(grads) == len(exp_avgs) == len(exp_avg_sqs) == n):
        raise ValueError("fused_adamw_: params, grads, exp_avgs, exp_avg_sqs differ in length")
    if n == 0:
        return
    if step < 1:
        raise ValueError(f"fused_adamw_: step must be >= 1, got {step}")
    dev = params[0].device
    if dev.type != "cuda":
        raise RuntimeError("fused_adamw_: tensors must live on the GPU (HIP kernel only)")
    if torch.cuda.is_current_stream_capturing():
        # the bias correction follows the host step count and the job table is copied from a
        # temporary host buffer: a replay would repeat a stale step from freed memory
        raise RuntimeError("fused_adamw_ cannot be captured into a graph (host step count and "
                           "per-call job table); step AdamW-routed parameters eagerly")
    pdt, gdt = params[0].dtype, grads[0].dtype
    if pdt not in _CODES or gdt not in _CODES:
        raise ValueError(f"fused_adamw_: unsupported dtypes param {pdt}, grad {gdt}")
    gs = []
    for p, g, m, v in zip(params, grads, exp_avgs, exp_avg_sqs):
        for t in (p, g, m, v):
            if t.device != dev:
                raise RuntimeError("fused_adamw_: all tensors must be on one device")
        if p.dtype != pdt or m.dtype != pdt or v.dtype != pdt or g.dtype != gdt:
            raise ValueError("fused_adamw_: a bucket shares one param/state dtype and one grad "
                             "dtype")
        if not (p.numel() == g.numel() == m.numel() == v.numel()):
            raise ValueError("fused_adamw_: param, grad and state sizes differ")
        for t in (p, m, v):
            if not t.is_contiguous():
                raise RuntimeError("fused_adamw_: params and AdamW state must be contiguous")
        gs.append(g if g.is_contiguous() else g.contiguous())
    qdt = None
    if publish is not None:
        if len(publish) != n:
            raise ValueError("fused_adamw_: publish must list one tensor (or None) per param")
        for p, q in zip(params, publish):
            if q is None:
                continue
            if q.device != dev or q.dtype not in _CODES or not q.is_contiguous():
                raise ValueError("fused_adamw_: publish targets must be contiguous fp32/bf16 "
                                 "tensors on the params' device")
            if q.numel() != p.numel() or (qdt is not None and q.dtype != qdt):
                raise ValueError("fused_adamw_: publish targets must match the params in size "
                                 "and share one dtype")
            qdt = q.dtype
    offsets = [0]
    for p in params:
        offsets.append(offsets[-1] + p.numel())
    pubs = [0] * n if qdt is None else [0 if q is None else q.data_ptr() for q in publish]
    table = ([p.data_ptr() for p in params] + [g.data_ptr() for g in gs]
             + [m.data_ptr() for m in exp_avgs] + [v.data_ptr() for v in exp_avg_sqs] + pubs
             + offsets)
    dtab = torch.tensor(table, dtype=torch.int64, pin_memory=True).to(dev, non_blocking=True)
    base = dtab.data_ptr()
    s = adamw_scalars(step, lr, betas, weight_decay, eps)
    stream = torch.cuda.current_stream(dev).cuda_stream
    _C.call("dmuon_adamw_multi", base, base + 8 * n, base + 16 * n, base + 24 * n,
            None if qdt is None else base + 32 * n, base + 40 * n, n, offsets[-1], _CODES[pdt],
            _CODES[gdt], 0 if qdt is None else _CODES[qdt], s["apply_wd"], s["wd_scale"],
            s["beta1"], s["alpha1"], s["beta2"], s["alpha2"], s["bc2_sqrt"], s["eps"],
            s["neg_step"], stream)
