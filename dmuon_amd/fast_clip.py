"""Segment-local gradient clipping on the HIP kernels (reference: ``dmuon/fast_clip.py``).

Every bucket (``GradClipBucket``) gets its own norm and coefficient::

    norm[s] = sqrt(sum over the bucket's grads of float(x)^2)
    coef[s] = min(max_norm / (norm[s] + 1e-6), 1)           (1 when max_norm is None)
    x      <- dtype(float(x) * coef[s])                     in place, when max_norm is given

The sums of squares and the scaling of every GPU-resident contiguous fp32/fp16/bf16 gradient
run in ``libdmuon_amd.so`` (``dmuon_segmented_l2_norm_sq`` / ``dmuon_segmented_scale``) over
one job table built once per call (a single pinned host buffer per integer width, copied
asynchronously). As in the reference (``fast_clip.py:154-163, 210-235``), the choice is per
tensor: a gradient the kernels cannot take (CPU-resident, non-contiguous, another dtype) is
handled with torch operations on its own device, which changes neither the result's meaning
nor the number of collectives. ``DMUON_FAST_CLIP=0`` turns the kernels off (reference
``fast_clip.py:96-129``); otherwise a missing library is an error, not a silent fallback.

Multi-rank reduction: the single ``all_reduce`` of the per-bucket squared norms of
``reduce=True`` buckets is kept (issued only when a process group is initialised), so the call
stays rank-uniform.
"""
from __future__ import annotations

import os
from collections import OrderedDict
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np
import torch
import torch.distributed as dist

from . import _C

_DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}   # fast_clip.py:31-35
_DEFAULT_CHUNK_SIZE = 262144


@dataclass(frozen=True)
class GradClipBucket:
    """One independently clipped gradient segment."""

    name: str
    grads: Sequence[torch.Tensor]
    reduce: bool = True


@dataclass(frozen=True)
class GradClipBucketStats:
    """Pre-clip norm and coefficient of one segment; tensor fields are 0-dim device tensors
    (the call itself never synchronises the host)."""

    name: str
    total_norm: torch.Tensor
    max_norm: Optional[float]
    clip_coef: torch.Tensor
    clipped: torch.Tensor
    param_count: int
    found_inf: torch.Tensor
    fastpath: bool

    def as_dict(self) -> dict:
        return {"name": self.name, "total_norm": self.total_norm, "max_norm": self.max_norm,
                "clip_coef": self.clip_coef, "clipped": self.clipped,
                "param_count": self.param_count, "found_inf": self.found_inf,
                "fastpath": self.fastpath}


@dataclass(frozen=True)
class SegmentedGradClipResult:
    total_norm: torch.Tensor
    bucket_stats: tuple
    fastpath: bool
    fallback_reason: Optional[str] = None

    @property
    def stats_by_name(self) -> dict:
        return {s.name: s for s in self.bucket_stats}


def _load_fast_clip_extension():
    """The kernel library, or ``None`` when ``DMUON_FAST_CLIP=0`` asks for torch math."""
    if os.environ.get("DMUON_FAST_CLIP", "1") == "0":
        return None
    return _C.lib()


def _resolve_chunk_size(chunk_size: Optional[int]) -> int:
    if chunk_size is not None:
        return max(1, int(chunk_size))
    raw = os.environ.get("DMUON_FAST_CLIP_CHUNK_SIZE")
    if raw is None:
        return _DEFAULT_CHUNK_SIZE
    try:
        return max(1, int(raw))
    except ValueError:
        return _DEFAULT_CHUNK_SIZE


def _resolve_device(buckets: Sequence[GradClipBucket]) -> torch.device:
    for b in buckets:
        for g in b.grads:
            if g is not None:
                return g.device
    if torch.cuda.is_available():
        return torch.device("cuda", torch.cuda.current_device())
    return torch.device("cpu")


def _kernel_eligible(g: torch.Tensor, device: torch.device) -> bool:
    return (device.type == "cuda" and g.device == device and not g.is_sparse
            and g.is_contiguous() and g.dtype in _DTYPE_CODES)


def _job_lists(numels, chunk: int):
    """Jobs of `chunk` elements over tensors of the given sizes, tensor by tensor: the tensor
    index and element offset of each job (the list ``fast_clip.py:190-196`` builds)."""
    numels = np.asarray(numels, dtype=np.int64)
    per = (numels + chunk - 1) // chunk                      # jobs per tensor
    job_t = np.repeat(np.arange(numels.size, dtype=np.int64), per)
    first = np.repeat(np.cumsum(per) - per, per)             # index of each tensor's first job
    return job_t, (np.arange(job_t.size, dtype=np.int64) - first) * chunk


class _JobTable:
    """Device-resident job table of the kernel-eligible tensors: int64 [ptrs | numels |
    job_offsets] and int32 [dtypes | segments | job_tensor_ids | zeros]."""

    def __init__(self, tensors, segments, device, chunk):
        n = len(tensors)
        numels = np.array([g.numel() for g in tensors], dtype=np.int64)
        job_t, job_off = _job_lists(numels, chunk)
        self.n, self.n_jobs, self.chunk = n, int(job_t.size), chunk
        i64 = np.concatenate([np.array([g.data_ptr() for g in tensors], dtype=np.int64), numels,
                              job_off])
        i32 = np.concatenate([np.array([_DTYPE_CODES[g.dtype] for g in tensors], dtype=np.int32),
                              np.asarray(segments, dtype=np.int32), job_t.astype(np.int32),
                              np.zeros(n, dtype=np.int32)])
        self._d64 = torch.from_numpy(i64).pin_memory().to(device, non_blocking=True)
        self._d32 = torch.from_numpy(i32).pin_memory().to(device, non_blocking=True)
        b64, b32 = self._d64.data_ptr(), self._d32.data_ptr()
        self.ptrs, self.numels, self.job_offsets = b64, b64 + 8 * n, b64 + 16 * n
        self.dtypes, self.segments = b32, b32 + 4 * n
        self.job_tensor_ids = b32 + 8 * n
        self.zero_segments = b32 + 8 * n + 4 * self.n_jobs
        self.device = device
        self._dtypes = [g.dtype for g in tensors]
        self._dtype_groups = None

    def dtype_groups(self):
        """(dtype, device index tensor of the table's tensors of that dtype, or None when all
        have it), built once per table: no host-to-device copy on later calls."""
        if self._dtype_groups is None:
            groups = []
            for dt in sorted(set(self._dtypes), key=str):
                sel = [i for i, d in enumerate(self._dtypes) if d == dt]
                idx = None if len(sel) == self.n else torch.tensor(sel).pin_memory().to(
                    self.device, non_blocking=True)
                groups.append((dt, idx))
            self._dtype_groups = groups
        return self._dtype_groups

    def _stream(self):
        return torch.cuda.current_stream(self.device).cuda_stream

    def sumsq(self, local_sq: torch.Tensor, segments=None) -> None:
        _C.call("dmuon_segmented_l2_norm_sq", self.ptrs, self.numels, self.dtypes,
                self.segments if segments is None else segments, self.job_tensor_ids,
                self.job_offsets, self.n_jobs, self.chunk, local_sq.data_ptr(), self._stream())

    def scale(self, coefs: torch.Tensor, segments=None) -> None:
        _C.call("dmuon_segmented_scale", self.ptrs, self.numels, self.dtypes,
                self.segments if segments is None else segments, self.job_tensor_ids,
                self.job_offsets, self.n_jobs, self.chunk, coefs.data_ptr(), self._stream())


# Tables keyed on everything they hold (addresses, sizes, dtypes, segments, chunk): gradients
# usually keep their storage from step to step, so later calls reuse the device table instead
# of rebuilding it on the host (for the c5 Muon gradients ~26.6k jobs, longer on the host than
# the two kernels take). A key that matches describes the same table, whatever tensors now sit
# at those addresses.
_TABLE_CACHE: "OrderedDict[tuple, _JobTable]" = OrderedDict()
_TABLE_CACHE_SIZE = 4


def _job_table(tensors, segments, device, chunk) -> _JobTable:
    key = (str(device), chunk, tuple(segments),
           tuple((g.data_ptr(), g.numel(), g.dtype) for g in tensors))
    table = _TABLE_CACHE.get(key)
    if table is None:
        table = _JobTable(tensors, segments, device, chunk)
        _TABLE_CACHE[key] = table
        while len(_TABLE_CACHE) > _TABLE_CACHE_SIZE:
            _TABLE_CACHE.popitem(last=False)
    else:
        _TABLE_CACHE.move_to_end(key)
    return table


def _split(buckets, device, ext):
    kt, ks, rest = [], [], []
    for s, b in enumerate(buckets):
        for g in b.grads:
            if g is None:
                continue
            if ext is not None and _kernel_eligible(g, device):
                kt.append(g)
                ks.append(s)
            else:
                rest.append((g, s))
    return kt, ks, rest


def _apply_segment_reductions(local_sq: torch.Tensor, reduce_flags, process_group=None):
    """The one rank-uniform collective over the reduce=True segments (fast_clip.py:313-339)."""
    if not (dist.is_available() and dist.is_initialized() and any(reduce_flags)):
        return local_sq
    mask = torch.tensor(reduce_flags, device=local_sq.device, dtype=torch.bool)
    red = torch.where(mask, local_sq, torch.zeros_like(local_sq))
    dist.all_reduce(red, op=dist.ReduceOp.SUM, group=process_group)
    return torch.where(mask, red, local_sq)


def _build_stats(buckets, total_norms, coefs, *, max_norm, fastpath):
    if not buckets:
        return tuple()
    total_norms, coefs = total_norms.detach(), coefs.detach()
    finite = torch.isfinite(total_norms)
    clipped = finite & (total_norms > float(max_norm)) if max_norm is not None \
        else torch.zeros_like(finite)
    found_inf = ~finite
    return tuple(
        GradClipBucketStats(name=b.name, total_norm=total_norms[i],
                            max_norm=None if max_norm is None else float(max_norm),
                            clip_coef=coefs[i], clipped=clipped[i],
                            param_count=sum(1 for g in b.grads if g is not None),
                            found_inf=found_inf[i], fastpath=fastpath)
        for i, b in enumerate(buckets))


@torch.no_grad()
def clip_grad_norm_buckets_(buckets: Sequence[GradClipBucket], max_norm: Optional[float], *,
                            process_group=None, chunk_size: Optional[int] = None
                            ) -> SegmentedGradClipResult:
    """Clip gradient buckets with segment-local semantics (``fast_clip.py:383-437``)."""
    device = _resolve_device(buckets)
    ext = _load_fast_clip_extension()
    chunk = _resolve_chunk_size(chunk_size)
    reduce_flags = [1 if b.reduce else 0 for b in buckets]
    kt, ks, rest = _split(buckets, device, ext)

    local_sq = torch.zeros(len(buckets), device=device, dtype=torch.float32)
    for g, s in rest:
        local_sq[s] += g.detach().float().pow(2).sum().to(device=device, dtype=torch.float32)
    table = _job_table(kt, ks, device, chunk) if kt else None
    if table is not None:
        table.sumsq(local_sq)

    global_sq = _apply_segment_reductions(local_sq, reduce_flags, process_group)
    total_norms = torch.sqrt(global_sq)
    if max_norm is None:
        coefs = torch.ones_like(total_norms)
    else:
        coefs = torch.clamp(float(max_norm) / (total_norms + 1e-6), max=1.0)
        for g, s in rest:
            g.mul_(coefs[s].to(device=g.device))
        if table is not None:
            table.scale(coefs)
    fastpath = ext is not None and device.type == "cuda"
    stats = _build_stats(buckets, total_norms, coefs, max_norm=max_norm, fastpath=fastpath)
    return SegmentedGradClipResult(
        torch.linalg.vector_norm(total_norms, 2.0), stats, fastpath=fastpath,
        fallback_reason=None if fastpath else
        ("disabled by DMUON_FAST_CLIP=0" if ext is None else "tensors not on a GPU"))


@torch.no_grad()
def try_clip_optimizer_grad_norm_buckets_(optimizer, *, regular_grads, adamw_grads,
                                          max_norm: float, process_group=None):
    """Regular / Muon / dedicated-AdamW clipping in one call (``fast_clip.py:440-489``);
    ``None`` when the kernels are switched off."""
    from .grad_clip import MuonGradClipStats, _iter_muon_grad_entries

    if _load_fast_clip_extension() is None:
        return None
    ensure = getattr(optimizer, "_ensure_grads_ready", None)
    if ensure is None:
        return None
    try:
        ensure(coalesce_wait=True)
    except TypeError:
        ensure()
    muon_grads = [e.grad for e in _iter_muon_grad_entries(optimizer)]
    result = clip_grad_norm_buckets_(
        (GradClipBucket("regular", regular_grads, reduce=False),
         GradClipBucket("muon", muon_grads, reduce=True),
         GradClipBucket("adamw", adamw_grads, reduce=True)),
        max_norm, process_group=process_group)
    ms = result.stats_by_name.get("muon")
    if ms is not None:
        optimizer._last_muon_grad_clip_stats = MuonGradClipStats(
            total_norm=ms.total_norm, max_norm=ms.max_norm, norm_type=2.0,
            clip_coef=ms.clip_coef, clipped=ms.clipped, param_count=ms.param_count,
            found_inf=ms.found_inf, strategy="segmented_cuda_fastpath")
    return result
