"""HIP streams with a hardware queue of their own, and the process-exit teardown.

HIP maps a process's streams onto a small set of hardware queues
(GPU_MAX_HW_QUEUES, 4 by default); two streams that land on one queue run
their work one after the other.  The engine's verify and draft streams must
overlap, so they are created with hipExtStreamCreateWithCUMask: a stream
with a CU mask gets a dedicated hardware queue.  The mask enables every CU
(no partitioning) and the streams keep the default priority.

Hardware queues are a scarce, per-device resource: past the number the
scheduler keeps mapped, a process's queues are time-sliced.  So there is
one dedicated stream per (device, role) for the life of the process, shared
by every Runner of that role (an engine's target and its draft take
different roles); engines built one after another reuse the same two
queues instead of adding two each.  Runners of one role driven from several
threads at once therefore serialise on their shared stream.

Teardown: HIP objects this package creates -- the dedicated streams and the
HIP graphs captured by model.BlockStep, with their workspaces -- are
released by an interpreter-exit hook, in order (drain the devices that hold
them, drop the graphs and their memory, drop the per-stream workspaces,
destroy the streams), while the HIP runtime and any attached tool are still
fully up, instead of being left to the runtime's own static destruction.
The hook is private: the streams it destroys are shared by every live
Runner, so it runs only when nothing can launch on them again.
"""
from __future__ import annotations

import atexit
import ctypes
import weakref
from typing import Dict, List, Optional, Tuple

import torch

_hip: Optional[ctypes.CDLL] = None
_streams: List[int] = []            # raw handles of the dedicated streams
_pool: Dict[Tuple[int, str], torch.cuda.ExternalStream] = {}  # (device, role) -> stream
_graph_owners: "weakref.WeakSet" = weakref.WeakSet()
_hook_registered = False


def register_graph_owner(owner) -> None:
    """An object with a ``release()`` that drops its captured graphs and
    their memory; called at interpreter exit before the streams go."""
    _ensure_hook()
    _graph_owners.add(owner)


def _ensure_hook() -> None:
    global _hook_registered
    if not _hook_registered:
        atexit.register(_teardown)
        _hook_registered = True


def _used_devices() -> List[int]:
    """Devices that hold a dedicated stream or a captured graph's owner."""
    devs = {d for d, _ in _pool}
    for owner in list(_graph_owners):
        dev = getattr(owner, "device", None)
        if dev is not None:
            devs.add(torch.device(dev).index or 0)
    return sorted(devs)


def _teardown() -> None:
    """Interpreter-exit hook (idempotent): release captured graphs, drop the
    workspaces cached for the dedicated streams and destroy the streams.
    Only the devices this package put streams or graphs on are drained, so
    no context is opened on another GPU."""
    try:
        if not torch.cuda.is_initialized():
            return
        devices = _used_devices()
        for d in devices:
            torch.cuda.synchronize(d)
    except Exception:
        return
    for owner in list(_graph_owners):
        try:
            owner.release()
        except Exception:
            pass
    _graph_owners.clear()
    try:
        for d in devices:
            torch.cuda.synchronize(d)
    except Exception:
        pass
    _pool.clear()
    if _streams:
        from . import _lib
        doomed = set(_streams)
        for k in [k for k in _lib._workspaces if k[1] in doomed]:
            del _lib._workspaces[k]
        hip = _runtime()
        while _streams:
            handle = _streams.pop()
            hip.hipStreamDestroy(ctypes.c_void_p(handle))


def _runtime() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipExtStreamCreateWithCUMask.restype = ctypes.c_int
        _hip.hipExtStreamCreateWithCUMask.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint32,
                                                      ctypes.POINTER(ctypes.c_uint32)]
        _hip.hipStreamDestroy.restype = ctypes.c_int
        _hip.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    return _hip


def dedicated_stream(device, role: str = "default") -> torch.cuda.ExternalStream:
    """The default-priority stream with a hardware queue of its own for
    (device, role), covering all CUs: created on the first request and
    returned to every later one for the same pair.

    The stream lives until the process ends (graphs replayed on it may
    outlive any one owner); the exit hook destroys it.
    """
    device = torch.device(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, role)
    stream = _pool.get(key)
    if stream is not None:
        return stream
    n = torch.cuda.get_device_properties(index).multi_processor_count
    words = (n + 31) // 32
    mask = (ctypes.c_uint32 * words)(*([0xFFFFFFFF] * words))
    if n % 32:
        mask[words - 1] = (1 << (n % 32)) - 1
    handle = ctypes.c_void_p()
    with torch.cuda.device(index):
        status = _runtime().hipExtStreamCreateWithCUMask(ctypes.byref(handle), words, mask)
    if status != 0:
        raise RuntimeError(f"hipExtStreamCreateWithCUMask failed with HIP error {status}")
    _ensure_hook()
    _streams.append(handle.value)
    stream = torch.cuda.ExternalStream(handle.value, device=torch.device("cuda", index))
    _pool[key] = stream
    return stream
