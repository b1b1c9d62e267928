"""ORACLE -- test infrastructure only.

fp64 numpy restatement of the paged attention the reference runs:

* block-verify: flash_attn_with_kvcache(..., causal=True) at
  serving/vendor/ssd/layers/attention.py:38-41 -- query i of a block of Q
  sees keys j <= ctx - Q + i (bottom-right aligned causal mask);
* draft block: the draft branch at :42-52 with the recovery mask of
  serving/engine.py:41-42 -- every block query sees keys j < ctx;
* GQA: head h reads KV head h // (Hq / Hkv) (repeat_interleave at :47-48,
  repeat_kv at models/d3d/modeling_d3d.py:190-200);
* packed multi-branch draft: the bool mask Engine._mask builds from branch
  specs (serving/engine.py:35-52), restated by ``engine_mask``;
* keys are gathered through the page table: token t of request b lives in
  page block_table[b, t // page_size] at offset t % page_size
  (serving/backend.py:123-124).
"""
from __future__ import annotations

import numpy as np


def gather_kv(cache: np.ndarray, block_table: np.ndarray, b: int, ctx: int) -> np.ndarray:
    """Logical [ctx, Hkv, D] keys (or values) of request b."""
    P, ps, Hkv, D = cache.shape
    t = np.arange(ctx)
    pages = block_table[b, t // ps]
    return cache[pages, t % ps]


def engine_mask(prefix: int, Q: int, S: int, K: int, specs=None) -> np.ndarray:
    """[Q, S] bool mask of Engine._mask (serving/engine.py:35-52) for one request.

    ``specs`` None is the recovery mask (every query sees cols < prefix + Q);
    otherwise rows 0..K-1 see the prefix and the pending block causally, and
    branch j (rows K + jK ..) with ``specs[j] = (accepted, anchor)`` sees
    cols < prefix + accepted and its own K columns.
    """
    cols = np.arange(S)[None, :]
    local = cols - prefix
    if specs is None:
        return np.broadcast_to(cols < prefix + Q, (Q, S)).copy()
    mask = np.zeros((Q, S), bool)
    rows = np.arange(K)[:, None]
    mask[:K] = (cols < prefix) | ((local >= 0) & (local <= rows))
    for j, (accepted, _anchor) in enumerate(specs):
        off = K + j * K
        mask[off:off + K] = (cols < prefix + accepted) | ((local >= off) & (local < off + K))
    return mask


def paged_attention(q, k_cache, v_cache, block_table, context_lens, scale, causal=True, masks=None):
    """q [B,Q,Hq,D]; caches [P,ps,Hkv,D]; returns fp64 [B,Q,Hq,D].

    ``masks`` (optional): per request a [Q, >= ctx] bool mask of visible keys,
    overriding ``causal``.  Rows that see no key give zeros.
    """
    q = np.asarray(q, np.float64)
    kc = np.asarray(k_cache, np.float64)
    vc = np.asarray(v_cache, np.float64)
    bt = np.asarray(block_table)
    B, Q, Hq, D = q.shape
    Hkv = kc.shape[2]
    G = Hq // Hkv
    out = np.zeros((B, Q, Hq, D))
    for b in range(B):
        ctx = int(context_lens[b])
        K = gather_kv(kc, bt, b, ctx)
        V = gather_kv(vc, bt, b, ctx)
        j = np.arange(ctx)[None, :]
        i = np.arange(Q)[:, None]
        if masks is not None:
            visible = np.asarray(masks[b])[:, :ctx]
        else:
            visible = (j <= ctx - Q + i) if causal else np.ones((Q, ctx), bool)
        any_row = visible.any(axis=1, keepdims=True)
        for h in range(Hq):
            s = q[b, :, h, :] @ K[:, h // G, :].T * scale
            s = np.where(visible, s, -np.inf)
            s -= np.where(any_row, s.max(axis=1, keepdims=True), 0.0)
            p = np.exp(s)
            p /= np.where(any_row, p.sum(axis=1, keepdims=True), 1.0)
            out[b, :, h, :] = p @ V[:, h // G, :]
    return out
