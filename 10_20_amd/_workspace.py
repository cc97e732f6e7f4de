"""Per-device scratch buffers reused across calls (allocated on first need,
grown when a larger call arrives, never shrunk)."""
import threading

import torch

_lock = threading.Lock()
_buffers = {}


def workspace(device, nbytes, tag="default"):
    """(pointer, size) of a device buffer of at least nbytes, or (0, 0).
    One buffer per (device, tag); calls that use one tag must not overlap."""
    if nbytes <= 0:
        return 0, 0
    key = (device.type, device.index if device.index is not None else torch.cuda.current_device(), tag)
    with _lock:
        buf = _buffers.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(int(nbytes), dtype=torch.uint8, device=device)
            _buffers[key] = buf
        return buf.data_ptr(), buf.numel()


def release_all():
    with _lock:
        _buffers.clear()
