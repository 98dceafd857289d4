"""dmuon_amd -- MI355X-native owner-rank Muon update, a drop-in for the ``dmuon`` API at
world_size=1 (``import dmuon_amd as dmuon``).

Exports the names of X-Square-Robot/dmuon's ``dmuon/__init__.py:80-122`` that concern the
owner-rank update path. The compute runs in ``dmuon_amd/csrc/libdmuon_amd.so`` (HIP, gfx950);
there is no CPU fallback.
"""
from .api import dedicate_params, replicate
from .fast_clip import (
    GradClipBucket,
    GradClipBucketStats,
    SegmentedGradClipResult,
    clip_grad_norm_buckets_,
    try_clip_optimizer_grad_norm_buckets_,
)
from .grad_clip import MuonGradClipStats, clip_grad_norm_, register_muon_grad_clip_strategy
from .optim import (
    KELLER_COEFFICIENTS,
    POLAR_EXPRESS_COEFFICIENTS,
    YOU_COEFFICIENTS,
    Muon,
    NewtonSchulz,
    direct_newton_schulz,
    fused_adamw_,
    get_backend_status,
    get_ns_backend,
    gram_newton_schulz,
    newton_schulz,
    newton_schulz_batched,
)
from .utils import (
    broadcast_all_updates,
    broadcast_all_updates_async,
    get_comm_ctx,
    get_dedicated_params,
    get_owned_params,
    prepare_muon_grads,
    wait_all_post_step_broadcasts,
    wait_all_reduces,
    wait_all_replicate_broadcasts,
)

__all__ = [
    "dedicate_params", "replicate", "Muon", "NewtonSchulz", "newton_schulz",
    "gram_newton_schulz", "direct_newton_schulz", "newton_schulz_batched", "fused_adamw_",
    "get_backend_status",
    "get_ns_backend", "get_comm_ctx", "get_dedicated_params", "get_owned_params",
    "prepare_muon_grads", "wait_all_reduces", "wait_all_replicate_broadcasts",
    "wait_all_post_step_broadcasts", "broadcast_all_updates", "broadcast_all_updates_async",
    "YOU_COEFFICIENTS", "POLAR_EXPRESS_COEFFICIENTS", "KELLER_COEFFICIENTS",
    "clip_grad_norm_", "clip_grad_norm_buckets_", "try_clip_optimizer_grad_norm_buckets_",
    "register_muon_grad_clip_strategy", "MuonGradClipStats", "GradClipBucket",
    "GradClipBucketStats", "SegmentedGradClipResult",
]
