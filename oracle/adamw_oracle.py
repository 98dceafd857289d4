"""CPU oracle for the AdamW half of the Muon optimizer -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this module, and only as the checker; ``dmuon_amd`` never does.

``adamw_step`` restates, in numpy float32, one step of the reference's decoupled AdamW
(``dmuon/optim/muon.py:1857-1916``, ``_adamw_update_batch``) for one tensor whose
``exp_avg``/``exp_avg_sq`` state has the parameter's dtype (``zeros_like(param)``,
``muon.py:1887-1888``). Every ``torch._foreach`` call of the reference materialises a tensor in
that dtype, so the value is rounded to it after each one (``R`` below; identity for fp32):

    p = R(p * (1 - lr*wd))                         _foreach_mul_         muon.py:1902
    m = R(m * b1);  m = R(m + (1-b1) * g)          _foreach_mul_/add_    muon.py:1904-1905
    v = R(v * b2);  v = R(v + (1-b2) * (g*g))      _foreach_mul_/addcmul_ muon.py:1906-1907
    d = R(sqrt(v)); d = R(d / sqrt(bc2)); d = R(d + eps)                 muon.py:1913-1915
    p = R(p + (-lr/bc1) * (m / d))                 _foreach_addcdiv_     muon.py:1916

with ``bc1 = 1 - b1**step``, ``bc2 = 1 - b2**step`` and every scalar derived in double and
converted to float32, as a Python scalar reaching a foreach kernel is. Each multiply and add is
its own float32 rounding (numpy does not contract), sqrt and division are correctly rounded.

Pinning (tests/test_adamw.py): against the reference's own call sequence run through
``torch._foreach`` on CPU tensors (same ops, torch's CPU kernels), against
``torch.optim.AdamW(foreach=False)`` over several fp32 steps, and against the closed form of a
first step from zero state, ``p1 = p0 (1 - lr wd) - lr g / (|g| + eps)``; mutated copies
(bias correction dropped, betas swapped, decay applied after the update) fail those checks.
"""
from __future__ import annotations

import numpy as np

from .ns_oracle import round_bf16


def _rounder(dtype: str):
    if dtype == "bf16":
        return lambda x: round_bf16(np.asarray(x, dtype=np.float32))
    if dtype == "fp32":
        return lambda x: np.asarray(x, dtype=np.float32)
    raise ValueError(dtype)


def adamw_step(p, g, m, v, step: int, lr: float, betas=(0.9, 0.999), wd: float = 0.0,
               eps: float = 1e-8, dtype: str = "fp32"):
    """One AdamW step of one tensor; returns the new (p, m, v) as float32 arrays holding
    values of ``dtype`` (the storage dtype of p, m and v)."""
    R = _rounder(dtype)
    f32 = np.float32
    b1, b2 = float(betas[0]), float(betas[1])
    p = np.asarray(p, dtype=f32)
    g = np.asarray(g, dtype=f32)
    m = np.asarray(m, dtype=f32)
    v = np.asarray(v, dtype=f32)
    if wd > 0:
        p = R(p * f32(1.0 - lr * wd))
    m = R(m * f32(b1))
    m = R(m + f32(1.0 - b1) * g)
    v = R(v * f32(b2))
    v = R(v + f32(1.0 - b2) * (g * g))
    bc1 = 1.0 - b1 ** step
    bc2 = 1.0 - b2 ** step
    d = R(np.sqrt(v))
    d = R(d / f32(bc2 ** 0.5))
    d = R(d + f32(eps))
    p = R(p + f32(-(lr / bc1)) * (m / d))
    return p, m, v
