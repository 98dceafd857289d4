from .param import DedicatedParam, DedicatedParamGroup, DedicatedState, LocalCommContext, ReplicatedGroup

__all__ = ["DedicatedParam", "DedicatedParamGroup", "DedicatedState", "LocalCommContext",
           "ReplicatedGroup"]
