"""Grad-readiness and publish helpers (reference: ``dmuon/utils.py``), at world_size=1.

``prepare_muon_grads`` materialises ``_reduced_grad`` from ``.grad`` (the reduce-to-owner is
the identity on one rank); ``wait_all_reduces`` and ``broadcast_all_updates`` have no peer to
wait for or publish to and return immediately.
"""
from __future__ import annotations

from torch import nn

from dmuon_amd._backends.local import normalize_owner_rank
from dmuon_amd.api import iter_dedicated_states


def get_comm_ctx(model: nn.Module):
    return getattr(model, "_dedicated_comm_ctx", None)


def get_dedicated_params(model: nn.Module) -> list:
    out = []
    for st in iter_dedicated_states(model):
        out.extend(st.group.params)
    return out


def get_owned_params(model: nn.Module, rank=0) -> list:
    """``utils.py:51-60``: the dedicated params owned by ``rank`` -- a shard ``int`` (1-D form)
    or a ``(shard, replicate)`` pair, matched against each param's owner coordinate. At
    world_size=1 every dedicated param is owned by ``(0, 0)``."""
    coord = normalize_owner_rank(rank)
    return [dp for dp in get_dedicated_params(model) if dp.owner_rank == coord]


def prepare_muon_grads(model: nn.Module, *, use_reduce_stream: bool = False,
                       coalesce_wait: bool = False) -> None:
    """``utils.py:178-204``: make every owned dedicated param's reduced grad available. The
    reduce-stream and coalesced-wait options of the reference order a side-stream reduce
    against the current stream; at world_size=1 there is no reduce, so both are accepted and
    change nothing."""
    for st in iter_dedicated_states(model):
        st.group.wait_for_reduce()


def wait_all_reduces(model: nn.Module) -> None:
    prepare_muon_grads(model)


def broadcast_all_updates(model: nn.Module) -> None:
    """``utils.py:358-371``: no replicate peers at world_size=1."""
    return None


def broadcast_all_updates_async(model: nn.Module) -> None:
    return None


def wait_all_replicate_broadcasts(model: nn.Module) -> None:
    return None


def wait_all_post_step_broadcasts(model: nn.Module) -> None:
    return None
