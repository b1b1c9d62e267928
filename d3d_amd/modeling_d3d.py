"""The draft model's call surface over a paged KV cache.

Mirrors models/d3d/modeling_d3d.py:

* ``D3DForCausalLM.__call__(input_ids, attention_mask, position_ids,
  past_key_values, use_cache, store_kv, logits_to_keep)`` -- :855-934 with
  the attention of D3DAttention.forward, :263-368: q/k RMSNorm, RoPE with
  cos/sin in the activation dtype, the new tokens' K/V stored in the cache
  (``store_kv=True``) or used for this call only (``store_kv=False``, the
  concatenation at :293-306), then attention under ``attention_mask``;
  returns an object with ``.logits`` [B, logits_to_keep or q, V] and
  ``.past_key_values``.
* ``PagedCache`` -- what the reference's transformers DynamicCache provides
  to the draft loop (``get_seq_length``, ``crop``, ``len``), holding each
  request's K/V in pages of the model's pool instead of growing tensors.

Attention masks are [B or 1, 1, q, kv_len] bool (True = visible), integer
(non-zero = visible) or additive float (0 = visible, large negative =
hidden), as normalize_sdpa_attention_mask (:203-218) accepts.  The kernels
take a per-query visibility descriptor -- keys t < A, plus lo <= t < hi --
so every mask row must be such a union of two intervals, the same for every
request; the reference's masks (_full_mask, _draft_attention_mask,
_fused_draft_mask, Engine._mask) all are.  Anything else raises ValueError.
``attention_mask=None`` lets every query see every key, as SDPA does without
a mask.
"""
from __future__ import annotations

from types import SimpleNamespace
from typing import List, Optional, Union

import torch

from .model import (D3D_1P7B, ModelShape, PagedKV, Qwen3PagedModel, Sequence, block_inputs, release, reserve,
                    trim)


def mask_to_visibility(mask: Optional[torch.Tensor], q: int, kv_len: int) -> torch.Tensor:
    """[q, 3] int32 descriptor (A, lo, hi) -- absolute key indices -- of a
    [.., q, kv_len'] mask (kv_len' >= kv_len; columns past kv_len ignored, as
    normalize_sdpa_attention_mask trims them).  Reads the mask on the host."""
    if mask is None:
        return torch.tensor([[kv_len, 0, 0]] * q, dtype=torch.int32)
    m = mask.detach()
    if m.shape[-2] != q or m.shape[-1] < kv_len:
        raise ValueError(f"attention mask of shape {tuple(m.shape)} does not cover {q} queries x {kv_len} keys")
    m = m[..., :kv_len]
    if m.dtype == torch.bool:
        vis = m
    elif torch.is_floating_point(m):
        hidden = m <= -1e4
        if not bool(((m == 0) | hidden).all()):
            raise ValueError("additive float masks must hold 0 (visible) or large negative (hidden) values")
        vis = ~hidden
    else:
        vis = m != 0
    vis = vis.reshape(-1, q, kv_len).cpu()
    if not bool((vis == vis[:1]).all()):
        raise ValueError("attention masks that differ between requests are not supported")
    row = vis[0].to(torch.int64)
    idx = torch.arange(kv_len)
    # A: length of the leading visible run; lo / hi: the next visible run.
    first_hidden = torch.where(row == 0, idx, kv_len).min(-1).values
    after = idx[None, :] >= first_hidden[:, None]
    lo = torch.where((row == 1) & after, idx, kv_len).min(-1).values
    beyond = idx[None, :] >= lo[:, None]
    hi = torch.where((row == 0) & beyond, idx, kv_len).min(-1).values
    rebuilt = (idx[None, :] < first_hidden[:, None]) | ((idx[None, :] >= lo[:, None]) & (idx[None, :] < hi[:, None]))
    if not torch.equal(rebuilt, row.bool()):
        raise ValueError("attention mask rows must be a visible prefix plus at most one more visible range")
    return torch.stack([first_hidden, lo, hi], -1).to(torch.int32)


class PagedCache:
    """Per-request K/V of the draft in pages of its pool (the DynamicCache role).

    ``get_seq_length()`` is the stored length (equal for every request of
    the batch); ``crop(n)`` drops the tokens past ``n`` and returns their
    pages to the pool; ``release()`` frees every page.
    """

    def __init__(self, model: "D3DForCausalLM", batch: int = 1):
        self.model = model
        self.seqs: List[Sequence] = [model._new_sequence() for _ in range(batch)]
        for s in self.seqs:
            s.prefix = 0

    def __len__(self) -> int:
        return self.model.model.shape.layers

    @property
    def batch(self) -> int:
        return len(self.seqs)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.seqs[0].prefix

    def crop(self, length: int) -> None:
        length = max(0, int(length))
        for s in self.seqs:
            if s.prefix > length:
                s.prefix = length
            trim(self.model.kv, s, self.model.name, length)

    def release(self) -> None:
        for s in self.seqs:
            if self.model.name in s.pages:
                release(self.model.kv, s, self.model.name)
            s.prefix = 0


class D3DForCausalLM:
    """Random-initialised bf16 D3D draft (Qwen3 backbone) with the reference's call surface.

    ``shape`` defaults to the D3D-1.7B draft (28 layers, hidden 2048, 16/8
    heads, MLP 6144, V 151,936); ``pages`` x ``page_size`` tokens of K/V
    are shared by every PagedCache of this model.
    """

    name = "draft"

    def __init__(self, shape: ModelShape = D3D_1P7B, device="cuda:0", *, pages: int = 4096, page_size: int = 16,
                 seed: int = 0, model: Optional[Qwen3PagedModel] = None, kv: Optional[PagedKV] = None):
        self.device = torch.device(device)
        self.model = model if model is not None else Qwen3PagedModel(shape, self.device, draft=True, seed=seed)
        self.config = SimpleNamespace(vocab_size=self.model.shape.vocab, num_hidden_layers=self.model.shape.layers,
                                      hidden_size=self.model.shape.hidden)
        self.kv = kv if kv is not None else PagedKV(self.model.shape, pages, page_size, self.device)
        self._next_id = 0

    def _new_sequence(self) -> Sequence:
        self._next_id += 1
        return Sequence(-self._next_id, [])

    def new_cache(self, batch: int = 1) -> PagedCache:
        return PagedCache(self, batch)

    def prefill(self, cache: PagedCache, input_ids: torch.Tensor) -> None:
        """Store K/V of a causal prefix (the reference's prefill with store_kv=True)."""
        q = input_ids.shape[1]
        past = cache.get_seq_length()
        vis = torch.tensor([[past + i + 1, 0, 0] for i in range(q)], dtype=torch.int32)
        self.forward_vis(input_ids, vis, None, cache, store_kv=True, logits_to_keep=1)

    def forward_vis(self, input_ids: torch.Tensor, vis: torch.Tensor, position_ids: Optional[torch.Tensor],
                    cache: PagedCache, *, store_kv: bool, logits_to_keep: Union[int, torch.Tensor] = 0,
                    past: Optional[int] = None):
        """Forward with an absolute visibility descriptor [q, 3] (A, lo, hi).

        The new tokens' K/V go to positions ``past`` .. past + q - 1 of each
        request (default: the stored length); ``store_kv`` then sets the
        stored length to past + q.
        """
        dev = self.device
        ids = torch.as_tensor(input_ids, dtype=torch.int64, device=dev)
        if ids.ndim != 2 or ids.shape[0] != cache.batch:
            raise ValueError(f"input_ids must be [{cache.batch}, q] for this cache")
        B, q = ids.shape
        if past is None:
            past = cache.get_seq_length()
            if any(s.prefix != past for s in cache.seqs):
                raise ValueError("every request of a cache must hold the same number of tokens")
        kv_len = past + q
        for s in cache.seqs:
            reserve(self.kv, s, self.name, kv_len)
        tables, slots, lens, logical, max_ctx = block_inputs(self.kv, cache.seqs, self.name, [past] * B, q, dev)
        pos = logical if position_ids is None else torch.as_tensor(position_ids, device=dev).to(torch.int64)
        pos = pos.expand(B, q).contiguous()
        # The kernels count A, lo, hi from the block start (context - q).
        rel = vis.to(torch.int32).clone()
        rel[:, 0] -= past
        rel[:, 1] -= past
        rel[:, 2] -= past
        hidden = self.model(ids, pos, self.kv, tables, lens, slots, causal=False, max_context=max_ctx,
                            q_vis=rel.to(dev, non_blocking=True))
        if store_kv:
            for s in cache.seqs:
                s.prefix = kv_len
        if isinstance(logits_to_keep, int):
            hidden = hidden[:, -logits_to_keep:] if logits_to_keep > 0 else hidden
        else:
            hidden = hidden[:, logits_to_keep]
        return SimpleNamespace(logits=self.model.logits(hidden), past_key_values=cache)

    def __call__(self, input_ids: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
                 position_ids: Optional[torch.Tensor] = None, past_key_values: Optional[PagedCache] = None,
                 use_cache: Optional[bool] = None, store_kv: bool = False,
                 logits_to_keep: Union[int, torch.Tensor] = 0, **_unused):
        """models/d3d/modeling_d3d.py:855-934 over the paged cache.

        Without ``past_key_values`` the call runs on a temporary cache that is
        released afterwards.  ``store_kv=True`` keeps the new tokens' K/V
        (DynamicCache.update); ``store_kv=False`` uses them for this call
        only.  ``position_ids`` default to past .. past + q - 1.
        """
        ids = torch.as_tensor(input_ids, dtype=torch.int64, device=self.device)
        q = ids.shape[1]
        temp = past_key_values is None
        cache = self.new_cache(ids.shape[0]) if temp else past_key_values
        try:
            past = cache.get_seq_length()
            vis = mask_to_visibility(attention_mask, q, past + q)
            out = self.forward_vis(ids, vis, position_ids, cache, store_kv=store_kv and not temp,
                                   logits_to_keep=logits_to_keep)
        finally:
            if temp:
                cache.release()
        if temp:
            out.past_key_values = None
        return out
