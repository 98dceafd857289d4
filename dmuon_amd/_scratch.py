"""Device scratch buffers kept per (device, stream) for the C-ABI calls that need a workspace.

Kernels on one stream run in submission order, so successive calls on that stream reuse its
buffer safely. A buffer shared between streams would let a call on one stream overwrite
scratch that a call on another is still reading, so each stream has its own. Each buffer is
allocated with its stream current: when a larger one replaces it, or the least recently used
entry is dropped, torch's caching allocator hands the old memory out again only in that
stream's order.

The key is the stream handle. torch's pool streams (``torch.cuda.Stream()``,
``current_stream()``) are never destroyed, so a handle names one hardware queue for the life
of the process. A caller that destroys a stream of its own (``ExternalStream``) must
synchronise it first, as with any memory its kernels still use. At most ``max_streams``
buffers are kept per device; the least recently used one is released beyond that, so
short-lived side streams do not pin memory for the life of the process.
"""
from __future__ import annotations

from collections import OrderedDict

import torch
from torch import Tensor


class StreamScratch:
    def __init__(self, max_streams: int = 8) -> None:
        self.max_streams = int(max_streams)
        self._bufs: "OrderedDict[tuple, Tensor]" = OrderedDict()

    def get(self, device: torch.device, stream: "torch.cuda.Stream", nbytes: int) -> Tensor:
        """A uint8 device buffer of at least ``nbytes`` bytes for work enqueued on ``stream``."""
        key = (torch.device(device), int(stream.cuda_stream))
        buf = self._bufs.get(key)
        if buf is not None and buf.numel() >= nbytes:
            self._bufs.move_to_end(key)
            return buf
        self._bufs.pop(key, None)
        with torch.cuda.stream(stream):
            buf = torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)
        self._bufs[key] = buf
        self._evict(key[0])
        return buf

    def _evict(self, device: torch.device) -> None:
        keys = [k for k in self._bufs if k[0] == device]
        for k in keys[:max(0, len(keys) - self.max_streams)]:
            del self._bufs[k]

    def streams(self, device: torch.device) -> list:
        """Stream handles that hold a buffer on ``device``, least recently used first."""
        return [k[1] for k in self._bufs if k[0] == torch.device(device)]

    def clear(self) -> None:
        self._bufs.clear()
