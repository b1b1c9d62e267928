"""Diffusion-draft block step on the gfx950 kernels.

Mirrors single/eval_sync.py:

* ``get_num_transfer_tokens``  -- :440-444, the per-step unmask schedule
* ``confidence_topk_unmask``   -- :447-465 (_select_transfer, low-confidence
                                  remasking) with the greedy confidence of
                                  :713-717, one kernel launch per iteration
* ``d3d_draft_block``          -- :482-592, the denoise loop (greedy), with
                                  the block attending to the paged prefix and
                                  to itself bidirectionally (store_kv=False:
                                  the block's K/V are rewritten each step)

Selection is per request (the reference applies row 0's indices to every
row, :461-464) and ties in confidence go to the lowest position.
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import torch

from . import _lib
from .model import BlockStep, PagedKV, Qwen3PagedModel, Sequence, block_inputs, reserve

MASK_ID = 151669


def get_num_transfer_tokens(num_masks: int, steps: int) -> List[int]:
    """single/eval_sync.py:440-444: an even split, the remainder going first."""
    steps = max(1, int(steps))
    base, extra = divmod(int(num_masks), steps)
    return [base + (1 if i < extra else 0) for i in range(steps)]


def confidence_topk_unmask(logits: torch.Tensor, block: torch.Tensor, mask_id: int, k: int,
                           temperature: float = 0.0) -> Tuple[torch.Tensor, torch.Tensor]:
    """Unmask the k most confident masked positions of each request, in place.

    ``logits`` [B, Q, V] (fp32 or bf16), ``block`` [B, Q] int64 on the same
    device.  Returns (x0 [B, Q] int64, conf [B, Q] fp32) for every position.
    """
    dev = _lib.require_device(logits, block)
    if logits.ndim != 3 or block.shape != logits.shape[:2] or block.dtype != torch.int64:
        raise ValueError("expected logits [B,Q,V] and an int64 block [B,Q]")
    if not block.is_contiguous():
        raise ValueError("block must be contiguous (it is updated in place)")
    B, Q, V = logits.shape
    lg = logits if logits.dtype in (torch.float32, torch.bfloat16) else logits.float()
    lg = lg.contiguous()
    x0 = torch.empty(B, Q, dtype=torch.int64, device=dev)
    conf = torch.empty(B, Q, dtype=torch.float32, device=dev)
    lib = _lib.load()
    nbytes = lib.d3d_confidence_workspace_bytes(B, Q, V)
    ws = _lib.workspace(dev, "confidence", nbytes)
    st = lib.d3d_confidence_topk_unmask(lg.data_ptr(), _lib.dtype_code(lg), block.data_ptr(), int(mask_id),
                                        int(k), float(temperature), B, Q, V, x0.data_ptr(), conf.data_ptr(),
                                        ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev))
    _lib.check(st, "d3d_confidence_topk_unmask")
    return x0, conf


def topk_tokens(logits: torch.Tensor, k: int, with_values: bool = False):
    """Top-k token ids [..., k] int64 of logits [..., V] (fp32 or bf16), one launch pair.

    Descending value, equal values by ascending id: ``ids[..., 0]`` is the
    argmax (torch's first maximum).  serving/backend.py:84-93 (greedy and
    ``logits.topk(k).indices``).  With ``with_values`` also returns the
    values [..., k] fp32.
    """
    dev = _lib.require_device(logits)
    lg = logits if logits.dtype in (torch.float32, torch.bfloat16) else logits.float()
    lg = lg.contiguous()
    V = lg.shape[-1]
    N = lg.numel() // V
    ids = torch.empty(*lg.shape[:-1], k, dtype=torch.int64, device=dev)
    vals = torch.empty(*lg.shape[:-1], k, dtype=torch.float32, device=dev) if with_values else None
    lib = _lib.load()
    ws = _lib.workspace(dev, "topk", lib.d3d_topk_workspace_bytes(max(N, 1), V, k))
    st = lib.d3d_topk_rows(lg.data_ptr(), _lib.dtype_code(lg), N, V, int(k), ids.data_ptr(), _lib.ptr(vals),
                           ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev))
    _lib.check(st, "d3d_topk_rows")
    return (ids, vals) if with_values else ids


def draft_block_forward(drafter: Qwen3PagedModel, kv: PagedKV, seqs: List[Sequence], ids: torch.Tensor,
                        name: str = "draft", starts: Optional[List[int]] = None) -> torch.Tensor:
    """Logits [B, Q, V] of a block at positions starts[b].. (prefix + bidirectional block)."""
    B, Q = ids.shape
    starts = [s.prefix for s in seqs] if starts is None else starts
    for s, st in zip(seqs, starts):
        reserve(kv, s, name, st + Q)
    tables, slots, lens, logical, max_ctx = block_inputs(kv, seqs, name, starts, Q, drafter.device)
    hidden = drafter(ids, logical, kv, tables, lens, slots, causal=False, max_context=max_ctx)
    return drafter.logits(hidden)


def d3d_draft_block(drafter: Qwen3PagedModel, kv: PagedKV, seqs: List[Sequence], block: torch.Tensor,
                    denoising_steps: int, *, mask_id: int = MASK_ID, temperature: float = 0.0,
                    name: str = "draft", graphs: Optional[dict] = None, width: Optional[int] = None) -> torch.Tensor:
    """Denoise a block [B, Q] whose masked positions hold ``mask_id``.

    single/eval_sync.py:482-592 with greedy low-confidence remasking: each
    step runs the draft over the block, then unmasks the scheduled number of
    most confident masked positions; the last step fills every remaining
    mask.  ``num_masks`` is taken from request 0, as the reference's
    schedule is (:503-508).

    With a ``graphs`` dict each (forward + unmask) step is replayed from a
    HIP graph cached there per (B, Q, k, table width); ``width`` fixes the
    page-table width (default: the current longest table).
    """
    cur = block.clone().contiguous()
    num_masks = int((cur[0] == mask_id).sum().item())
    if num_masks == 0:
        return cur
    schedule = get_num_transfer_tokens(num_masks, denoising_steps)
    B, Q = cur.shape
    starts = [s.prefix for s in seqs]
    for s in seqs:
        reserve(kv, s, name, s.prefix + Q)
    tables, slots, lens, logical, _ = block_inputs(kv, seqs, name, starts, Q, drafter.device, width)
    W = tables.shape[1]
    for step, k in enumerate(schedule):
        if step == len(schedule) - 1:
            k = Q  # the last step unmasks everything left (:549-550)
        if graphs is None:
            hidden = drafter(cur, logical, kv, tables, lens, slots, causal=False, max_context=W * kv.page_size)
            confidence_topk_unmask(drafter.logits(hidden), cur, mask_id, k, temperature)
            continue
        key = (B, Q, k, W, temperature)
        step_fn = graphs.get(key)
        if step_fn is None:
            def post(hidden, ids, k=k):
                confidence_topk_unmask(drafter.logits(hidden), ids, mask_id, k, temperature)
                return ids
            step_fn = graphs[key] = BlockStep(drafter, kv, B, Q, W, causal=False, post=post)
        cur.copy_(step_fn(cur, logical, tables, slots, lens))
    return cur
