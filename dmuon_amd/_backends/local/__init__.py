from .param import (DedicatedParam, DedicatedParamGroup, DedicatedState, LocalCommContext,
                    ReplicatedGroup, normalize_owner_rank)

__all__ = ["DedicatedParam", "DedicatedParamGroup", "DedicatedState", "LocalCommContext",
           "ReplicatedGroup", "normalize_owner_rank"]
