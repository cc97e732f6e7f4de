"""Scratch buffers of the operators, reused across calls.

One buffer per (device, stream, tag): calls issued on different streams never
share scratch memory, and calls on one stream are ordered by that stream.  A
buffer is allocated on first need (from the calling stream, so the caching
allocator ties it to that stream) and grown when a larger call arrives.  An
outgrown buffer is never handed back to the allocator: a HIP graph captured
before the growth still holds its address and keeps writing it on every
replay, so it stays alive (and unused by anything else) until the process
ends.  Growth is geometric, so at most a few buffers per key are retired.
"""
import threading

import torch

_lock = threading.Lock()
_buffers = {}
_retired = []


def _key(device, tag, stream):
    index = device.index if device.index is not None else torch.cuda.current_device()
    if stream is None:
        stream = torch.cuda.current_stream(index)
    return index, stream.cuda_stream, tag


def workspace(device, nbytes, tag="default", stream=None):
    """(pointer, size) of a device buffer of at least nbytes for calls on
    `stream` (default: the device's current stream), or (0, 0)."""
    if nbytes <= 0:
        return 0, 0
    key = _key(device, tag, stream)
    with _lock:
        buf = _buffers.get(key)
        if buf is None or buf.numel() < nbytes:
            size = int(nbytes) if buf is None else max(int(nbytes), buf.numel() + buf.numel() // 2)
            new = torch.empty(size, dtype=torch.uint8, device=device)
            if buf is not None:
                _retired.append(buf)
            _buffers[key] = buf = new
        return buf.data_ptr(), buf.numel()


def buffers():
    """Live buffers: {(device index, stream handle, tag): bytes}."""
    with _lock:
        return {k: v.numel() for k, v in _buffers.items()}


def retired_bytes():
    with _lock:
        return sum(b.numel() for b in _retired)
