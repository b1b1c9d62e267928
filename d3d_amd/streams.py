"""HIP streams with a hardware queue of their own.

HIP maps a process's streams onto a small set of hardware queues
(GPU_MAX_HW_QUEUES, 4 by default); two streams that land on one queue run
their work one after the other.  The engine's verify and draft streams must
overlap, so they are created with hipExtStreamCreateWithCUMask: a stream
with a CU mask gets a dedicated hardware queue.  The mask enables every CU
(no partitioning) and the streams keep the default priority.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

_hip: Optional[ctypes.CDLL] = None


def _runtime() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipExtStreamCreateWithCUMask.restype = ctypes.c_int
        _hip.hipExtStreamCreateWithCUMask.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint32,
                                                      ctypes.POINTER(ctypes.c_uint32)]
    return _hip


def dedicated_stream(device) -> torch.cuda.ExternalStream:
    """A default-priority stream on its own hardware queue, covering all CUs.

    The stream lives until the process ends (graphs replayed on it may
    outlive any one owner).
    """
    device = torch.device(device)
    n = torch.cuda.get_device_properties(device).multi_processor_count
    words = (n + 31) // 32
    mask = (ctypes.c_uint32 * words)(*([0xFFFFFFFF] * words))
    if n % 32:
        mask[words - 1] = (1 << (n % 32)) - 1
    handle = ctypes.c_void_p()
    with torch.cuda.device(device):
        status = _runtime().hipExtStreamCreateWithCUMask(ctypes.byref(handle), words, mask)
    if status != 0:
        raise RuntimeError(f"hipExtStreamCreateWithCUMask failed with HIP error {status}")
    return torch.cuda.ExternalStream(handle.value, device=device)
