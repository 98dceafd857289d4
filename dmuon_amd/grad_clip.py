"""Gradient clipping of the Muon (dedicated, 2-D) gradients (reference: ``dmuon/grad_clip.py``).

``clip_grad_norm_(optimizer, max_norm)`` / ``Muon.clip_grad_norm_`` clip the owned Muon
gradients by one global p-norm coefficient and return ``MuonGradClipStats`` whose tensor
fields stay on the device. AdamW / non-dedicated gradients are not touched (use
``torch.nn.utils.clip_grad_norm_`` for those, as the reference says).

For p = 2 -- the default and the only order the reference's fast path handles -- the
per-tensor sums of squares and the final in-place scaling run on the HIP segmented-clip
kernels (one segment per tensor for the norms, one shared coefficient for the scale). The
reference takes the per-tensor norms with ``torch._foreach_norm``, which returns them in the
gradient's dtype; they are rounded the same way here before the total is formed, so the total
norm and coefficient follow the reference's arithmetic (up to the order of the fp32 sums).
Other orders (inf, p != 2) use the reference's torch reductions on the gradients' device.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Optional, Protocol, Union

import torch
import torch.distributed as dist

from .fast_clip import _job_table, _kernel_eligible, _load_fast_clip_extension, _resolve_chunk_size


@dataclass(frozen=True)
class MuonGradClipEntry:
    name: str
    grad: torch.Tensor
    shape: tuple
    is_tp_full_grad: bool = False


@dataclass(frozen=True)
class MuonGradClipStats:
    """``total_norm`` is the pre-clip norm; tensor fields are 0-dim device tensors."""

    total_norm: torch.Tensor
    max_norm: Optional[float]
    norm_type: float
    clip_coef: Union[torch.Tensor, float]
    clipped: Union[torch.Tensor, bool]
    param_count: int
    found_inf: torch.Tensor
    strategy: str = "global_norm"

    def as_dict(self) -> dict:
        return {"total_norm": self.total_norm, "max_norm": self.max_norm,
                "norm_type": self.norm_type, "clip_coef": self.clip_coef,
                "clipped": self.clipped, "param_count": self.param_count,
                "found_inf": self.found_inf, "strategy": self.strategy}


@dataclass(frozen=True)
class MuonGradClipContext:
    optimizer: Any
    entries: tuple
    max_norm: Optional[float]
    norm_type: float
    error_if_nonfinite: bool
    foreach: Optional[bool] = None


class MuonGradClipStrategy(Protocol):
    name: str

    def __call__(self, context: MuonGradClipContext) -> MuonGradClipStats:
        ...


class GlobalNormMuonClipStrategy:
    """All Muon gradients scaled by one global p-norm coefficient (``grad_clip.py:103-155``)."""

    name = "global_norm"

    @torch.no_grad()
    def __call__(self, context: MuonGradClipContext) -> MuonGradClipStats:
        entries = context.entries
        tensors = [e.grad for e in entries]
        device = _accumulator_device(context.optimizer, entries)
        ext = _load_fast_clip_extension()
        eligible = [t for t in tensors if ext is not None and _kernel_eligible(t, device)]
        table = (_job_table(eligible, list(range(len(eligible))), device, _resolve_chunk_size(None))
                 if eligible and context.norm_type == 2.0 else None)
        total = _total_norm(tensors, eligible, table, context.norm_type, device)
        if context.error_if_nonfinite and bool(torch.logical_or(total.isnan(), total.isinf())):
            raise RuntimeError(
                f"The total norm of order {context.norm_type} for DMuon Muon gradients is "
                "non-finite, so it cannot be clipped. To disable this error and scale the "
                "gradients by the non-finite norm anyway, set `error_if_nonfinite=False`.")
        max_norm = context.max_norm
        clip_coef: Union[torch.Tensor, float] = 1.0
        clipped: Union[torch.Tensor, bool] = False
        if max_norm is not None:
            if max_norm < 0:
                raise ValueError(f"max_norm must be non-negative, got {max_norm}")
            coef = float(max_norm) / (total + 1e-6)
            coef_c = torch.clamp(coef, max=1.0)
            _scale_all(tensors, eligible, table, coef_c, device)
            clip_coef = coef_c.detach()
            clipped = torch.isfinite(total.detach()) & (coef.detach() < 1.0)
        total = total.detach()
        return MuonGradClipStats(total_norm=total, max_norm=max_norm,
                                 norm_type=context.norm_type, clip_coef=clip_coef,
                                 clipped=clipped, param_count=len(entries),
                                 found_inf=~torch.isfinite(total), strategy=self.name)


def _total_norm(tensors, eligible, table, p, device) -> torch.Tensor:
    if not tensors:
        return torch.zeros((), device=device, dtype=torch.float32)
    eid = {id(t) for t in eligible}
    parts = []
    if table is not None:
        sq = torch.zeros(len(eligible), device=device, dtype=torch.float32)
        table.sumsq(sq)
        # per-tensor norms rounded to each gradient's dtype, as torch._foreach_norm returns them
        # (one rounding op per dtype present, not one per tensor)
        norms = torch.sqrt(sq)
        for dt, idx in table.dtype_groups():
            if dt == torch.float32:
                continue
            if idx is None:                   # every tensor has this dtype
                norms = norms.to(dt).float()
            else:
                norms[idx] = norms[idx].to(dt).float()
        parts.append(norms)
    others = [torch.linalg.vector_norm(t.detach(), p).to(device=device, dtype=torch.float32)
              for t in tensors if table is None or id(t) not in eid]
    if others:
        parts.append(torch.stack(others))
    local = torch.linalg.vector_norm(torch.cat(parts), p)
    if p == float("inf"):
        _all_reduce_if_needed(local, op=dist.ReduceOp.MAX)
        return local
    power = local.pow(p)
    _all_reduce_if_needed(power, op=dist.ReduceOp.SUM)
    return power.pow(1.0 / p)


def _scale_all(tensors, eligible, table, coef, device) -> None:
    eid = {id(t) for t in eligible}
    if table is not None:
        table.scale(coef.reshape(1).to(device=device, dtype=torch.float32),
                    segments=table.zero_segments)
    elif eligible:
        t0 = _job_table(eligible, [0] * len(eligible), device, _resolve_chunk_size(None))
        t0.scale(coef.reshape(1).to(device=device, dtype=torch.float32))
    for t in tensors:
        if id(t) not in eid:
            t.mul_(coef.to(t.device))


_STRATEGIES: dict = {GlobalNormMuonClipStrategy.name: GlobalNormMuonClipStrategy()}


def register_muon_grad_clip_strategy(name: str, strategy: MuonGradClipStrategy) -> None:
    if not name:
        raise ValueError("strategy name must be non-empty")
    _STRATEGIES[name] = strategy


def clip_grad_norm_(optimizer: Any, max_norm: Optional[float], *, norm_type: float = 2.0,
                    error_if_nonfinite: bool = False, foreach: Optional[bool] = None,
                    strategy: Union[str, MuonGradClipStrategy] = "global_norm"
                    ) -> MuonGradClipStats:
    """Clip the owned Muon gradients of a ``dmuon_amd.Muon`` (``grad_clip.py:171-200``)."""
    ensure = getattr(optimizer, "_ensure_grads_ready", None)
    if ensure is None or not hasattr(optimizer, "_dedicated_params"):
        raise TypeError("dmuon.clip_grad_norm_ expects a dmuon.Muon optimizer")
    ensure()
    return _clip_ready_muon_grad_norm_(optimizer, max_norm, norm_type=norm_type,
                                       error_if_nonfinite=error_if_nonfinite, foreach=foreach,
                                       strategy=strategy)


def _clip_ready_muon_grad_norm_(optimizer, max_norm, *, norm_type=2.0, error_if_nonfinite=False,
                                foreach=None, strategy="global_norm") -> MuonGradClipStats:
    if norm_type <= 0 and norm_type != float("inf"):
        raise ValueError(f"norm_type must be positive or inf, got {norm_type}")
    context = MuonGradClipContext(
        optimizer=optimizer, entries=tuple(_iter_muon_grad_entries(optimizer)),
        max_norm=None if max_norm is None else float(max_norm), norm_type=float(norm_type),
        error_if_nonfinite=error_if_nonfinite, foreach=foreach)
    stats = _resolve_strategy(strategy)(context)
    optimizer._last_muon_grad_clip_stats = stats
    return stats


def _resolve_strategy(strategy):
    if isinstance(strategy, str):
        try:
            return _STRATEGIES[strategy]
        except KeyError as exc:
            valid = ", ".join(sorted(_STRATEGIES))
            raise ValueError(f"unknown Muon grad clip strategy {strategy!r}; available: "
                             f"{valid}") from exc
    return strategy


def _iter_muon_grad_entries(optimizer: Any):
    """The owned Muon-routed gradients (``grad_clip.py:243-265``)."""
    muon_ids = set(getattr(optimizer, "_dp_to_muon_group_idx", {}).keys())
    for idx, dp in enumerate(getattr(optimizer, "_dedicated_params", [])):
        if muon_ids and id(dp) not in muon_ids:
            continue
        is_tp = bool(getattr(dp, "is_dtensor", False) and getattr(dp, "tp_group", None) is not None)
        if is_tp:
            if not bool(getattr(dp, "is_tp_owner", False)):
                continue
            grad = getattr(dp, "_tp_full_grad", None)
        else:
            grad = getattr(dp, "_reduced_grad", None)
        if grad is None:
            continue
        yield MuonGradClipEntry(name=str(getattr(dp, "param_name", f"dedicated_param_{idx}")),
                                grad=grad, shape=tuple(int(d) for d in grad.shape),
                                is_tp_full_grad=is_tp)


def _accumulator_device(optimizer: Any, entries) -> torch.device:
    if entries:
        return entries[0].grad.device
    dev = getattr(getattr(optimizer, "_comm_ctx", None), "device", None)
    if dev is not None:
        return torch.device(dev)
    if torch.cuda.is_available():
        return torch.device("cuda", torch.cuda.current_device())
    return torch.device("cpu")


def _all_reduce_if_needed(tensor: torch.Tensor, *, op) -> None:
    if dist.is_available() and dist.is_initialized():
        dist.all_reduce(tensor, op=op)
