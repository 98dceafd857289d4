"""``import dmuon`` for code written against X-Square-Robot/dmuon's owner-rank Muon path.

The MI355X implementation lives in ``dmuon_amd``; this package exposes it under the
reference's name: every public name of ``dmuon_amd`` (the subset of the reference's
``dmuon/__init__.py:80-122`` that concerns the owner-rank update), and the submodules a
reference user imports (``dmuon.optim``, ``dmuon.optim.newton_schulz``,
``dmuon.optim.syrk_dispatch``, ``dmuon.optim.muon``, ``dmuon.utils``, ``dmuon.fast_clip``,
``dmuon.grad_clip``, ``dmuon.api``) as the very same module objects, so classes, caches and
the loaded HIP library are shared whichever name is used.
"""
import importlib
import sys

import dmuon_amd
from dmuon_amd import *  # noqa: F401,F403
from dmuon_amd import __all__  # noqa: F401

_SUBMODULES = (
    "api", "utils", "fast_clip", "grad_clip", "optim", "optim.muon", "optim.newton_schulz",
    "optim.syrk_dispatch", "optim.adamw", "_backends", "_backends.local",
    "_backends.local.param",
)
for _name in _SUBMODULES:
    sys.modules[f"{__name__}.{_name}"] = importlib.import_module(f"dmuon_amd.{_name}")
api = dmuon_amd.api
utils = dmuon_amd.utils
fast_clip = dmuon_amd.fast_clip
grad_clip = dmuon_amd.grad_clip
optim = dmuon_amd.optim
del _name
