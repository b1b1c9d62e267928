"""ctypes binding of ``libd3d_hip.so``, the gfx950 kernels behind d3d_amd.

The library is the product path: if it is missing, or a tensor is not on a
HIP device, the calls below raise instead of falling back to CPU code.
Build it with ``python -m d3d_amd.build``.
"""
from __future__ import annotations

import ctypes
import gc
from pathlib import Path
from typing import Optional

import torch

LIB_PATH = Path(__file__).resolve().with_name("libd3d_hip.so")

D3D_DTYPE_F32 = 0
D3D_DTYPE_BF16 = 1
D3D_INPUT_LOGITS = 0
D3D_INPUT_PROBS = 1
D3D_ACCEPT_NOALLOC_SCRATCH_BYTES = 4 << 20
D3D_CONF_MAX_SOFTMAX = 0
D3D_CONF_ONE_HOT = 1
D3D_TOKEN_EMPTY_DISTRIBUTION = -1
D3D_TOKEN_BAD_DRAFT = -2
D3D_TOKEN_TIMEOUT = -3

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/d3d_hip.h.
SIGNATURES = {
    "d3d_status_string": (ctypes.c_char_p, [_I]),
    "d3d_version": (_I, []),
    "d3d_accept_workspace_bytes": (_SZ, [_I, _I, _I64]),
    "d3d_accept_fused": (
        _I,
        [_P, _P, _I, _I, _P, _P, _P, _F, _I, _I, _I64, _P, _P, _P, _P, _P, _P, _SZ, _P],
    ),
    "d3d_accept_fused_noalloc": (
        _I,
        [_P, _P, _I, _I, _P, _P, _P, _F, _I, _I, _I64, _P, _P, _P, _P, _P, _P],
    ),
    "d3d_accept_fused_sparse": (
        _I,
        [_P, _I, _I, _P, _P, _P, _I, _P, _P, _F, _I, _I, _I64, _P, _P, _P, _P, _P, _P, _SZ, _P],
    ),
    "d3d_attn_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I, _I, _I]),
    "d3d_verify_attn_paged": (
        _I,
        [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _P, _SZ, _P],
    ),
    "d3d_draft_block_attn": (
        _I,
        [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _P, _SZ, _P],
    ),
    "d3d_packed_block_attn": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _P, _SZ, _P],
    ),
    "d3d_kv_append": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I64, _P]),
    "d3d_confidence_workspace_bytes": (_SZ, [_I, _I, _I64]),
    "d3d_confidence_topk_unmask": (
        _I,
        [_P, _I, _P, _I64, _I, _F, _I, _I, _F, _I, _I, _I64, _P, _P, _P, _SZ, _P],
    ),
    "d3d_select_transfer": (_I, [_P, _I64, _I, _I, _F, _P, _P, _P, _I, _I, _P]),
    "d3d_topk_workspace_bytes": (_SZ, [_I, _I64, _I]),
    "d3d_topk_rows": (_I, [_P, _I, _I, _I64, _I, _I, _P, _P, _P, _SZ, _P]),
    "d3d_block_inputs": (_I, [_P, _I, _I, _P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _P]),
    "d3d_lmhead_workspace_bytes": (_SZ, [_I, _I64, _I]),
    "d3d_lmhead_topk": (_I, [_P, _P, _I, _I, _I64, _I, _I, _P, _P, _P, _SZ, _P]),
    "d3d_sample_workspace_bytes": (_SZ, [_I, _I64]),
    "d3d_sample_rows": (_I, [_P, _I, _I, _I64, _F, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "d3d_softmax_rows": (_I, [_P, _I, _I, _I64, _F, _P, _P, _P, _P, _P, _SZ, _P]),
    "d3d_row_filter": (_I, [_P, _I, _I, _I64, _F, _I, _F, _P, _P, _P]),
    "d3d_support_workspace_bytes": (_SZ, [_I, _I]),
    "d3d_sample_support_wide": (_I, [_P, _I, _I, _I64, _F, _I, _F, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "d3d_sample_support": (_I, [_P, _P, _I, _I, _F, _F, _P, _P, _P, _P, _P]),
    "d3d_add_rmsnorm": (_I, [_P, _P, _P, _P, _I, _I, _F, _P]),
    "d3d_qk_rope_append": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I64, _P],
    ),
    "d3d_silu_mul": (_I, [_P, _P, _I, _I, _P]),
    "d3d_gemm_rows64": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "d3d_gemm_rows64_splits": (_I, [_I, _I]),
    "d3d_gemm_rows64_silu_mul": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "d3d_add_rmsnorm_parts": (_I, [_P, _I, _P, _P, _P, _I, _I, _F, _P]),
    "d3d_qk_rope_append_parts": (
        _I,
        [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I64, _P],
    ),
}

_lib: Optional[ctypes.CDLL] = None


def load() -> ctypes.CDLL:
    """Load libd3d_hip.so once and declare every exported signature."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built: run `python -m d3d_amd.build` (hipcc, gfx950)"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    """Raise for a non-zero status: ValueError for argument errors, RuntimeError for HIP errors."""
    if status == 0:
        return
    msg = load().d3d_status_string(status).decode()
    if status < 0:
        raise ValueError(f"{what}: {msg} (status {status})")
    raise RuntimeError(f"{what}: HIP error {status}: {msg}")


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def require_device(*tensors: Optional[torch.Tensor]) -> torch.device:
    """All given tensors must live on one HIP device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "d3d_amd kernels run on a HIP device only; got a tensor on "
                f"{t.device} (there is no CPU path)"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise RuntimeError("no device tensor given")
    return dev


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


_workspaces: dict = {}
_capture_owner: Optional[list] = None


class collection_paused:
    """Python's cyclic garbage collector stays off inside (its previous
    state is restored on exit; nesting is fine).

    Graph captures run under it.  A collection that an allocation starts in
    the middle of a capture runs the finalizers of whatever unreachable
    objects exist -- an earlier step's graph, events, pinned buffers -- and
    their HIP calls are not allowed while a stream captures; an error raised
    in a finalizer aborts the process.  torch.cuda.graph no longer collects
    before it begins a capture, so the garbage is left for a collection
    after the capture instead."""

    def __enter__(self):
        self.was_enabled = gc.isenabled()
        gc.disable()
        return self

    def __exit__(self, *exc):
        if self.was_enabled:
            gc.enable()
        return False


class capture_workspaces:
    """Context for HIP graph capture: workspaces requested inside it are
    allocated afresh and appended to ``owner``, which must live as long as the
    captured graph (the graph's kernels keep their addresses).  No garbage
    collection runs inside it (``collection_paused``)."""

    def __init__(self, owner: list):
        self.owner = owner

    def __enter__(self):
        global _capture_owner
        self.paused = collection_paused().__enter__()
        self.prev, _capture_owner = _capture_owner, self.owner
        return self.owner

    def __exit__(self, *exc):
        global _capture_owner
        _capture_owner = self.prev
        self.paused.__exit__(*exc)
        return False


def workspace(device: torch.device, key: str, nbytes: int) -> torch.Tensor:
    """Workspace cached per (device, current stream, key).

    One workspace per stream keeps calls on concurrent streams from sharing
    scratch memory; calls on one stream are ordered, so reuse is safe.
    During a graph capture the cache is bypassed: every captured graph gets
    its own workspace, owned by the capture_workspaces owner list.
    """
    if torch.cuda.is_current_stream_capturing():
        if _capture_owner is None:
            raise RuntimeError("d3d_amd kernels captured into a graph need a workspace owner "
                               "(wrap the capture in d3d_amd._lib.capture_workspaces)")
        ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        _capture_owner.append(ws)
        return ws
    sp = stream_ptr(device)
    k = (device.index, sp, key)
    ws = _workspaces.get(k)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
        _workspaces[k] = ws
    return ws


def dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return D3D_DTYPE_F32
    if t.dtype == torch.bfloat16:
        return D3D_DTYPE_BF16
    raise ValueError(f"unsupported dtype {t.dtype}: expected float32 or bfloat16")
