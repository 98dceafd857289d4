"""Grad-readiness and publish helpers (reference: ``dmuon/utils.py``), at world_size=1.

``prepare_muon_grads`` materialises ``_reduced_grad`` from ``.grad`` (the reduce-to-owner is
the identity on one rank); ``wait_all_reduces`` and ``broadcast_all_updates`` have no peer to
wait for or publish to and return immediately.
"""
from __future__ import annotations

from torch import nn

from dmuon_amd.api import iter_dedicated_states


def get_comm_ctx(model: nn.Module):
    return getattr(model, "_dedicated_comm_ctx", None)


def get_dedicated_params(model: nn.Module) -> list:
    out = []
    for st in iter_dedicated_states(model):
        out.extend(st.group.params)
    return out


def get_owned_params(model: nn.Module) -> list:
    return [dp for dp in get_dedicated_params(model) if dp.is_owner]


def prepare_muon_grads(model: nn.Module) -> None:
    """``utils.py:178-204``: make every owned dedicated param's reduced grad available."""
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
