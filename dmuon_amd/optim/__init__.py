from .adamw import fused_adamw_
from .muon import Muon
from .newton_schulz import (
    DEFAULT_COEFFICIENTS,
    DEFAULT_RESTART_ITERATIONS,
    KELLER_COEFFICIENTS,
    POLAR_EXPRESS_COEFFICIENTS,
    YOU_COEFFICIENTS,
    NewtonSchulz,
    direct_newton_schulz,
    get_backend_status,
    get_ns_backend,
    gram_newton_schulz,
    newton_schulz,
    newton_schulz_batched,
)
from .syrk_dispatch import syrk_or_cublas

__all__ = [
    "Muon", "fused_adamw_", "NewtonSchulz", "newton_schulz", "gram_newton_schulz", "direct_newton_schulz",
    "newton_schulz_batched", "get_ns_backend", "get_backend_status", "YOU_COEFFICIENTS",
    "POLAR_EXPRESS_COEFFICIENTS", "KELLER_COEFFICIENTS", "DEFAULT_COEFFICIENTS",
    "DEFAULT_RESTART_ITERATIONS", "syrk_or_cublas",
]
