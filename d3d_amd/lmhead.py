"""Fused LM head + top-k on gfx950: logits of a few hidden rows reduced to
top-k ids (and values) without writing the [T, V] logits.

Reference behaviour (D3D repository):

* serving/backend.py:84-93 -- ``Runner._run``: ``logits = lm_head(h)``,
  ``greedy = logits.argmax(-1)``, ``top = logits.topk(anchor_num + 1)``.
* single/eval_sync.py:713-717 and :763-768 -- the draft's argmax and
  ``torch.topk(log_softmax(logits), k)`` anchors.

The kernel streams the weight once per 64 hidden rows, so it pays off up to
64 rows (verify and recovery blocks of four requests); longer row sets are
better served by a GEMM followed by ``draft.topk_tokens``.
"""
from __future__ import annotations

import torch

from . import _lib

MAX_K = 8
ROWS_PER_PASS = 64


def lmhead_topk(hidden: torch.Tensor, weight: torch.Tensor, k: int, with_values: bool = False,
                log_softmax: bool = False):
    """Top-k ids [..., k] int64 of ``hidden @ weight.T`` (bf16 logits).

    ``hidden`` [..., H] and ``weight`` [V, H] are bf16 on one HIP device, H a
    multiple of 32.  Descending value, equal values by ascending id, so
    ``ids[..., 0]`` is torch's argmax.  With ``with_values`` also returns the
    values [..., k] fp32: the bf16 logits, or their log-softmax over the
    whole row with ``log_softmax``.
    """
    dev = _lib.require_device(hidden, weight)
    if hidden.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("lmhead_topk expects bf16 hidden rows and weight")
    if weight.ndim != 2 or hidden.shape[-1] != weight.shape[1]:
        raise ValueError(f"hidden [..., H] and weight [V, H] disagree: {tuple(hidden.shape)} vs {tuple(weight.shape)}")
    if not 1 <= k <= MAX_K or k > weight.shape[0]:
        raise ValueError(f"k must be in [1, {MAX_K}] and at most V")
    x = hidden.contiguous()
    w = weight.contiguous()
    H = w.shape[1]
    V = w.shape[0]
    T = x.numel() // H
    ids = torch.empty(*x.shape[:-1], k, dtype=torch.int64, device=dev)
    vals = torch.empty(*x.shape[:-1], k, dtype=torch.float32, device=dev) if with_values else None
    lib = _lib.load()
    ws = _lib.workspace(dev, "lmhead", lib.d3d_lmhead_workspace_bytes(max(T, 1), V, k))
    st = lib.d3d_lmhead_topk(x.data_ptr(), w.data_ptr(), T, H, V, int(k), int(bool(log_softmax)), ids.data_ptr(),
                             _lib.ptr(vals), ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev))
    _lib.check(st, "d3d_lmhead_topk")
    return (ids, vals) if with_values else ids
