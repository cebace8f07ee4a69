"""Device workspaces for the split reductions of the kernels.

A workspace is a zero-initialised byte buffer on one device.  The kernels hand their
counter slots back to zero, so a workspace stays valid for any number of calls issued in
stream order.  One shared workspace per device serves every call on one stream; calls on
other streams that may overlap should pass their own (``Workspace(device)``).

Growing a workspace allocates, so it is refused while a graph is being captured: warm up
(run each shape once) before capture, as the reference's graph bench does.  A buffer that is
outgrown is kept alive (never freed) rather than released: graphs captured before the growth
still point at it, and since every kernel leaves its counters at zero, they stay valid.
"""
from __future__ import annotations

import threading

import torch


class Workspace:
    def __init__(self, device, nbytes: int = 0):
        self.device = torch.device(device)
        self._buf = None
        self._retired = []  # outgrown buffers, still referenced by graphs captured earlier
        self._lock = threading.Lock()
        if nbytes:
            self.ensure(nbytes)

    @property
    def nbytes(self) -> int:
        return 0 if self._buf is None else self._buf.numel()

    def ensure(self, nbytes: int) -> "tuple[int, int]":
        """Return (pointer, size) of a zeroed buffer of at least nbytes bytes."""
        if nbytes <= 0:
            return (0, 0)
        if self._buf is None or self._buf.numel() < nbytes:
            with self._lock:
                if self._buf is None or self._buf.numel() < nbytes:
                    if torch.cuda.is_current_stream_capturing():
                        raise RuntimeError(
                            f"specq workspace must grow to {nbytes} bytes during graph capture; "
                            "run the same call once before capturing")
                    size = max(nbytes, 2 * (self._buf.numel() if self._buf is not None else 0), 1 << 20)
                    if self._buf is not None:
                        self._retired.append(self._buf)
                    # Ordered after the work already queued on the current stream.
                    self._buf = torch.zeros(size, dtype=torch.uint8, device=self.device)
        return (self._buf.data_ptr(), self._buf.numel())


_shared: dict = {}
_shared_lock = threading.Lock()


def shared(device) -> Workspace:
    dev = torch.device(device)
    key = (dev.type, dev.index if dev.index is not None else torch.cuda.current_device())
    ws = _shared.get(key)
    if ws is None:
        with _shared_lock:
            ws = _shared.get(key)
            if ws is None:
                ws = _shared[key] = Workspace(torch.device(dev.type, key[1]))
    return ws
