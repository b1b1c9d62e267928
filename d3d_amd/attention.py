"""Paged block attention and KV append on the gfx950 kernels.

Mirrors the calls the reference's attention dispatch makes
(serving/vendor/ssd/layers/attention.py:16-53):

* ``kv_append``                  -- ``k_cache.view(-1, Hkv, D)[slot_mapping] = k``
                                    (and v), :21-22
* ``flash_attn_with_kvcache``    -- same name, arguments and return value as
                                    the flash-attn call at :38-41 (target
                                    block-verify, bottom-right causal);
                                    ``causal=False`` gives the draft block
* ``draft_block_attn``           -- the draft branch :42-52 under the recovery
                                    mask of serving/engine.py:41-42: every
                                    block query sees the prefix and the whole
                                    block

All tensors live on one HIP device; there is no CPU path.
"""
from __future__ import annotations

import math
from typing import Sequence, Optional

import torch

from . import _lib


def _check_cache(k_cache: torch.Tensor, v_cache: torch.Tensor):
    if k_cache.ndim != 4 or k_cache.shape != v_cache.shape:
        raise ValueError("expected k_cache/v_cache [num_pages, page_size, Hkv, D] of equal shape")
    if k_cache.dtype != torch.bfloat16 or v_cache.dtype != torch.bfloat16:
        raise ValueError("KV caches must be bfloat16")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("KV caches must be contiguous")
    for t in (k_cache, v_cache):
        if t.data_ptr() % 16:
            raise ValueError("KV caches must be 16-byte aligned")


def kv_append(k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
              slot_mapping: torch.Tensor) -> None:
    """Scatter new keys/values into the paged cache by flat slot index.

    ``k``/``v`` [N, Hkv, D] (or [N, Hkv*D]) bf16, ``slot_mapping`` [N] int;
    slot = page_id * page_size + offset (serving/backend.py:123-124).
    Negative slots are skipped.
    """
    dev = _lib.require_device(k, v, k_cache, v_cache, slot_mapping)
    _check_cache(k_cache, v_cache)
    P, ps, Hkv, D = k_cache.shape
    n = slot_mapping.numel()
    k = k.reshape(n, Hkv, D).to(torch.bfloat16).contiguous()
    v = v.reshape(n, Hkv, D).to(torch.bfloat16).contiguous()
    slots = slot_mapping.reshape(n).to(torch.int64).contiguous()
    lib = _lib.load()
    st = lib.d3d_kv_append(k.data_ptr(), v.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                           slots.data_ptr(), n, Hkv, D, P * ps, _lib.stream_ptr(dev))
    _lib.check(st, "d3d_kv_append")


def _attn(fn_name: str, q, k_cache, v_cache, cache_seqlens, block_table, softmax_scale, max_seqlen_k, out,
          vis=None):
    dev = _lib.require_device(q, k_cache, v_cache, cache_seqlens, block_table, vis)
    _check_cache(k_cache, v_cache)
    if q.ndim != 4:
        raise ValueError("expected q [B, Q, Hq, D]")
    B, Q, Hq, D = q.shape
    P, ps, Hkv, Dk = k_cache.shape
    if Dk != D or Hq % Hkv:
        raise ValueError("q and cache head shapes are incompatible")
    if block_table.ndim != 2 or block_table.shape[0] != B:
        raise ValueError("expected block_table [B, max_pages]")
    max_pages = block_table.shape[1]
    if max_seqlen_k is None:
        max_seqlen_k = max_pages * ps  # an upper bound that needs no host read
    if max_seqlen_k > max_pages * ps:
        raise ValueError("max_seqlen_k exceeds the block table's capacity")
    q = q.to(torch.bfloat16).contiguous()
    bt = block_table.to(torch.int32).contiguous()
    lens = cache_seqlens.to(torch.int32).reshape(B).contiguous()
    if out is None:
        out = torch.empty(B, Q, Hq, D, dtype=torch.bfloat16, device=dev)
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(D)
    lib = _lib.load()
    nbytes = lib.d3d_attn_workspace_bytes(B, Q, Hq, Hkv, D, ps, int(max_seqlen_k))
    ws = _lib.workspace(dev, "attn", nbytes)
    vis_args = () if vis is None else (vis.data_ptr(),)
    st = getattr(lib, fn_name)(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), bt.data_ptr(), lens.data_ptr(), *vis_args,
        out.data_ptr(), B, Q, Hq, Hkv, D, ps, max_pages, P, float(scale), int(max_seqlen_k),
        ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev))
    _lib.check(st, fn_name)
    return out


def flash_attn_with_kvcache(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                            cache_seqlens: torch.Tensor, block_table: torch.Tensor, *,
                            causal: bool = True, softmax_scale: Optional[float] = None,
                            max_seqlen_k: Optional[int] = None,
                            out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Paged attention of a block of Q queries per request; returns [B, Q, Hq, D] bf16.

    With ``causal=True`` query i sees keys j <= cache_seqlens[b] - Q + i (the
    flash-attn convention used at serving/vendor/ssd/layers/attention.py:38-41);
    with ``causal=False`` every query sees every key j < cache_seqlens[b].
    ``max_seqlen_k`` (optional) bounds cache_seqlens and sizes the context
    split; it defaults to the block table's capacity.
    """
    name = "d3d_verify_attn_paged" if causal else "d3d_draft_block_attn"
    return _attn(name, q, k_cache, v_cache, cache_seqlens, block_table, softmax_scale, max_seqlen_k, out)


def draft_block_attn(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     context_lens: torch.Tensor, block_table: torch.Tensor, *,
                     softmax_scale: Optional[float] = None, max_seqlen_k: Optional[int] = None,
                     out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Draft block attention: prefix plus a bidirectional block (recovery mask)."""
    return _attn("d3d_draft_block_attn", q, k_cache, v_cache, context_lens, block_table,
                 softmax_scale, max_seqlen_k, out)


def packed_visibility(K: int, accepted: Sequence[int]) -> torch.Tensor:
    """Per-query visibility [Q, 3] int32 of a packed draft block (CPU tensor).

    Rows 0..K-1 are the pending block, causal over prefix + block
    (serving/engine.py:45); branch j (rows K + jK ..) has ``accepted[j]``
    accepted pending tokens and sees the prefix, those tokens and its own K
    positions bidirectionally (serving/engine.py:46-50).  Q = K (1 + len(accepted)).
    """
    rows = [(i + 1, 0, 0) for i in range(K)]
    for j, n in enumerate(accepted):
        if not 0 <= n <= K:
            raise ValueError("accepted counts must lie in [0, K]")
        off = K + j * K
        rows.extend((n, off, off + K) for _ in range(K))
    return torch.tensor(rows, dtype=torch.int32)


def packed_block_attn(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, context_lens: torch.Tensor,
                      block_table: torch.Tensor, q_visibility: torch.Tensor, *,
                      softmax_scale: Optional[float] = None, max_seqlen_k: Optional[int] = None,
                      out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Packed multi-branch draft attention over a paged cache.

    ``q`` [B, Q, Hq, D]; ``context_lens`` = prefix + Q (the packed block's
    keys are appended after the prefix); ``q_visibility`` [Q, 3] int32 on
    the device: query i sees keys t < prefix + v[i, 0] and
    prefix + v[i, 1] <= t < prefix + v[i, 2] (see :func:`packed_visibility`).
    """
    if q_visibility.shape != (q.shape[1], 3) or q_visibility.dtype != torch.int32:
        raise ValueError("q_visibility must be int32 [Q, 3]")
    return _attn("d3d_packed_block_attn", q, k_cache, v_cache, context_lens, block_table, softmax_scale,
                 max_seqlen_k, out, vis=q_visibility.contiguous())
