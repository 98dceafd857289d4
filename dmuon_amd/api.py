"""``dedicate_params`` / ``replicate`` at world_size=1 (reference: ``dmuon/api.py:392-751``,
``dmuon/_backends/ddp/replicate.py:87-282``).

With one rank every dedicated parameter is owned by rank 0, so the LPT owner partition, the
packed broadcast buffers and the forward/backward hooks of the reference reduce to marking the
parameters and attaching the world-1 data contract to the model.
"""
from __future__ import annotations

import logging
from typing import Callable, Optional

import torch
import torch.distributed as dist
from torch import nn

from dmuon_amd._backends.local import (
    DedicatedParam,
    DedicatedParamGroup,
    DedicatedState,
    LocalCommContext,
    ReplicatedGroup,
)

logger = logging.getLogger(__name__)


def _world_size(mesh) -> int:
    if mesh is not None and hasattr(mesh, "size"):
        return int(mesh.size())
    if dist.is_available() and dist.is_initialized():
        return dist.get_world_size()
    return 1


def dedicate_params(
    model: nn.Module,
    mesh=None,
    predicate: Optional[Callable[[str, nn.Parameter], bool]] = None,
    compute_dtype=None,
    reshard_after_forward: bool = True,
    replicate_mesh=None,
    **kwargs,
) -> dict[nn.Parameter, int]:
    """Marks parameters matching ``predicate(name, param)`` as dedicated (owned by rank 0).

    Returns the owner assignment ``{param: 0}``; logs a warning and returns ``{}`` when nothing
    matches (``api.py:576-578``). Raises ``NotImplementedError`` for a mesh or process group of
    more than one rank: this build implements the single-GPU owner path only.
    """
    if predicate is None:
        raise TypeError("dedicate_params() missing required argument: 'predicate'")
    ws = _world_size(mesh)
    if ws != 1 or (replicate_mesh is not None and _world_size(replicate_mesh) != 1):
        raise NotImplementedError(
            f"dmuon_amd implements the world_size=1 owner path only (got world size {ws})")
    assignment: dict[nn.Parameter, int] = {}
    dps: list[DedicatedParam] = []
    for name, p in model.named_parameters():
        if not p.requires_grad or not predicate(name, p):
            continue
        pdt, mdt = _resolve_policy(name, compute_dtype, kwargs.get("param_policy"))
        p._dedicated_owner_rank = (0, 0)      # the owner coordinate, as api.py tags it
        assignment[p] = 0
        dps.append(DedicatedParam(p, name, 0, param_dtype=pdt, master_dtype=mdt))
    if not assignment:
        logger.warning("dedicate_params: no parameters matched the predicate")
        return assignment
    group = DedicatedParamGroup(dps)
    model._dedicated_states = [DedicatedState(group)]
    model._dedicated_comm_ctx = LocalCommContext()
    return assignment


_DTYPE_NAMES = {"fp32": torch.float32, "float32": torch.float32, "bf16": torch.bfloat16,
                "bfloat16": torch.bfloat16, "fp16": torch.float16, "float16": torch.float16}


def _as_dtype(value) -> Optional[torch.dtype]:
    if value is None or isinstance(value, torch.dtype):
        return value
    key = str(value).strip().lower()
    if key in ("", "none", "null"):
        return None
    if key not in _DTYPE_NAMES:
        raise ValueError(f"unsupported dtype {value!r}")
    return _DTYPE_NAMES[key]


def _resolve_policy(name: str, compute_dtype, param_policy) -> tuple:
    """(param_dtype, master_dtype) of one dedicated parameter, as the reference resolves them
    (``policy.py:176-262``): ``compute_dtype`` is the legacy forward dtype, the policy's master
    dtype defaults to fp32, and ``param_policy = {"defaults": {...}, "overrides": [{"name" |
    "contains": ..., "set": {...}}]}`` may set ``param_dtype`` / ``master_dtype``."""
    pdt, mdt = _as_dtype(compute_dtype), torch.float32
    if param_policy:
        layers = [param_policy.get("defaults", {}) or {}]
        for ov in param_policy.get("overrides", ()) or ():
            if ("name" in ov and ov["name"] == name) or ("contains" in ov and ov["contains"] in name):
                layers.append(ov["set"])
        for layer in layers:
            if "param_dtype" in layer:
                pdt = _as_dtype(layer["param_dtype"])
            if "master_dtype" in layer:
                mdt = _as_dtype(layer["master_dtype"])
    return pdt, mdt


def replicate(model: nn.Module, mesh=None, **kwargs) -> nn.Module:
    """Registers every non-dedicated trainable parameter for AdamW (``replicate.py:87``)."""
    if _world_size(mesh) != 1:
        raise NotImplementedError("dmuon_amd implements the world_size=1 owner path only")
    params = [p for p in model.parameters()
              if p.requires_grad and not hasattr(p, "_dedicated_owner_rank")]
    model._replicated_group = ReplicatedGroup(params)
    return model


def iter_dedicated_states(model: nn.Module):
    return list(getattr(model, "_dedicated_states", []))
