"""world_size=1 data contract of the reference's dedicated-parameter runtime.

At one rank every dedicated parameter is owned locally, the grad reduce-to-owner is the
identity and the post-step publish has no peer, so the objects below keep only the fields the
optimizer reads and writes (reference: ``dmuon/_backends/fsdp2/param.py:116-628``,
``fsdp2/group.py:276-2177``, ``dmuon/_core/comm.py:24-110``):

* ``_owned_data``  -- the owner's master copy of the weight, in the master dtype of its policy
  (``fsdp2/param.py:263-271``; fp32 by default, ``policy.py:64-82``). When that dtype is the
  forward parameter's own, the master *is* the parameter storage and the update is in place;
  otherwise it is a separate tensor and every update is followed by the publish of
  ``round(master)`` into the parameter (the reference copies ``_owned_data`` into the packed
  forward buffer, ``fsdp2/group.py:766-781``) -- done by the update kernels themselves, in the
  same pass (``publish_target``).
* ``_reduced_grad`` -- the reduced gradient the Muon step consumes (``group.py:1348-1352``);
  here the parameter's ``.grad``, set by :func:`dmuon_amd.prepare_muon_grads` or read directly
  by the optimizer; cleared after the update (``muon.py:1746-1747``).
* ``is_owner``, ``owner_rank`` (the ``(shard, replicate)`` coordinate, ``(0, 0)``),
  ``owner_shard``, ``numel``, ``full_shape``, ``tp_group`` (always None: no tensor
  parallelism here).
"""
from __future__ import annotations

from typing import Optional, Tuple, Union

import torch
from torch import nn


OwnerRankLike = Union[int, Tuple[int, int]]
OwnerCoord = Tuple[int, int]


def normalize_owner_rank(owner_rank: OwnerRankLike) -> OwnerCoord:
    """An owner rank as the reference's ``(owner_shard, owner_replicate)`` coordinate
    (``_core/owner_rank.py:19-49``): an ``int`` is the 1-D form ``(int, 0)``; a pair passes
    through. ``bool`` and other types raise ``TypeError``, negative entries ``ValueError``."""
    if isinstance(owner_rank, tuple):
        if len(owner_rank) != 2:
            raise TypeError(f"owner_rank tuple must be (shard, replicate); got {owner_rank!r}")
        shard, rep = owner_rank
        if not (isinstance(shard, int) and isinstance(rep, int)) or isinstance(shard, bool) \
                or isinstance(rep, bool):
            raise TypeError(f"owner_rank tuple entries must be int; got {owner_rank!r}")
        if shard < 0 or rep < 0:
            raise ValueError(f"owner_rank must be non-negative; got {owner_rank!r}")
        return shard, rep
    if isinstance(owner_rank, bool) or not isinstance(owner_rank, int):
        raise TypeError(f"owner_rank must be int or Tuple[int, int]; got "
                        f"{type(owner_rank).__name__} {owner_rank!r}")
    if owner_rank < 0:
        raise ValueError(f"owner_rank must be non-negative; got {owner_rank!r}")
    return owner_rank, 0


class DedicatedParam:
    def __init__(self, param: nn.Parameter, name: str, owner_rank: OwnerRankLike = 0,
                 param_dtype: Optional[torch.dtype] = None,
                 master_dtype: Optional[torch.dtype] = None):
        self.param = param
        self._orig_param = param
        self.param_name = name
        coord = normalize_owner_rank(owner_rank)
        self.owner_rank: OwnerCoord = coord            # (owner_shard, owner_replicate)
        self.owner_shard: int = coord[0]
        self.is_owner = True
        self.full_shape = tuple(param.shape)
        self.numel: int = param.numel()                # fsdp2/param.py:214
        self.tp_group = None
        self.is_dtensor = False
        self.is_tp_owner = False
        self._reduced_grad: Optional[torch.Tensor] = None
        self._accumulated_grad: Optional[torch.Tensor] = None
        self._orig_dtype = param.dtype
        self._param_dtype = param_dtype
        self._master_dtype = master_dtype
        mdt = master_dtype or param.dtype
        fdt = param_dtype or param.dtype
        # master from the original values (before any cast of the forward parameter)
        self._master: Optional[torch.Tensor] = (
            None if mdt == fdt else param.data.detach().to(dtype=mdt).clone())
        if fdt != param.dtype:
            param.data = param.data.to(fdt)

    @property
    def _owned_data(self) -> torch.Tensor:
        return self.param.data if self._master is None else self._master

    def publish_target(self) -> Optional[torch.Tensor]:
        """The forward tensor that receives round(master) after an update, or None when the
        master is the parameter itself."""
        return None if self._master is None else self.param.data

    def current_grad(self) -> Optional[torch.Tensor]:
        g = self._reduced_grad
        return self.param.grad if g is None else g

    def uses_sharded_muon_forward(self) -> bool:
        return False

    def __repr__(self) -> str:
        return f"DedicatedParam({self.param_name}, shape={self.full_shape}, owner={self.owner_rank})"


class DedicatedParamGroup:
    def __init__(self, params: list[DedicatedParam]):
        self.params = params
        self.replicate_group = None

    # reduce / publish hooks are identities at world_size=1 (group.py:1727-1729, :1792-1794)
    def wait_for_reduce(self) -> None:
        for dp in self.params:
            if dp._reduced_grad is None and dp.param.grad is not None:
                dp._reduced_grad = dp.param.grad

    def replicate_broadcast_async(self) -> None:
        return None


class DedicatedState:
    def __init__(self, group: DedicatedParamGroup):
        self.group = group


class ReplicatedGroup:
    """Non-dedicated parameters updated by AdamW (``ddp/replicate.py:87-282`` at one rank)."""

    def __init__(self, params: list[nn.Parameter]):
        self.params = params


class LocalCommContext:
    """Stand-in for ``DedicatedCommContext`` (``_core/comm.py:24-110``) at world_size=1: no
    collectives, no side streams; everything runs on the caller's current stream."""

    def __init__(self) -> None:
        self.world_size = 1
        self.rank = 0
        self.replicate_group = None
        self.forward_prefetch_depth = 1
        self.sharded_adamw_unshard_separate_stream_enabled = False
