"""Synthetic inputs for the per-step speculative hot path.

Each builder draws from a seeded ``torch.Generator`` with the distributions
of the workloads this package is measured on:

* acceptance: target logits ~ N(0, 2^2) over [B, K+1, V]; draft logits =
  target[:, :K] + N(0, 0.5^2); draft tokens sampled from softmax(draft / T)
  by inverse CDF (argmax at T <= 1e-5); uniforms ~ U(0, 1) passed explicitly.
* paged attention: q, k, v ~ N(0, 1) / sqrt(d) in bf16, pages of
  ``page_size`` tokens, page tables drawn as a seeded permutation of the pool.

Builders run on the CPU generator (``device="cpu"``, reproducible across
machines) or directly on a device generator for large benchmark inputs.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional

import torch

VOCAB = 151936
MASK_ID = 151669
EOS_IDS = (151643, 151645)


@dataclass
class AcceptInputs:
    target: torch.Tensor  # [B, K+1, V] fp32 logits
    draft: torch.Tensor  # [B, K, V] fp32 logits
    tokens: torch.Tensor  # [B, K] int64
    uniforms: torch.Tensor  # [B, K] fp32
    resample_u: torch.Tensor  # [B] fp32


def accept_inputs(seed: int, B: int = 1, K: int = 15, V: int = VOCAB, temperature: float = 1.0,
                  device: str = "cpu", target_std: float = 2.0, noise_std: float = 0.5) -> AcceptInputs:
    g = torch.Generator(device=device).manual_seed(seed)
    target = torch.randn(B, K + 1, V, generator=g, device=device) * target_std
    draft = target[:, :K] + torch.randn(B, K, V, generator=g, device=device) * noise_std
    tok_u = torch.rand(B, K, generator=g, device=device)
    uniforms = torch.rand(B, K, generator=g, device=device)
    resample_u = torch.rand(B, generator=g, device=device)
    if temperature <= 1e-5:
        tokens = draft.argmax(dim=-1)
    else:
        probs = torch.softmax(draft / temperature, dim=-1)
        cdf = probs.double().cumsum(dim=-1)
        tokens = torch.searchsorted(cdf, (tok_u.double() * cdf[..., -1])[..., None], right=True)[..., 0]
        tokens = tokens.clamp_(max=V - 1)
    return AcceptInputs(target.contiguous(), draft.contiguous(), tokens.long(), uniforms, resample_u)


@dataclass
class SparseAcceptInputs:
    target: torch.Tensor  # [B, K+1, V] fp32 logits
    tokens: torch.Tensor  # [B, K] int64
    q_ids: torch.Tensor  # [B, K, S] int64 support ids
    q_probs: torch.Tensor  # [B, K, S] fp32 support probabilities
    uniforms: torch.Tensor  # [B, K] fp32
    resample_u: torch.Tensor  # [B] fp32


def sparse_accept_inputs(seed: int, B: int = 1, K: int = 15, V: int = VOCAB, S: int = 64,
                         temperature: float = 1.0, target_std: float = 2.0,
                         noise_std: float = 0.5) -> SparseAcceptInputs:
    """Sparse proposals as single/eval_sync.py:341-367 forms them: the
    top-S draft logits at ``temperature``, softmax over that support, and
    the draft token drawn from it (inverse CDF over a seeded uniform)."""
    base = accept_inputs(seed, B, K, V, temperature=1.0, target_std=target_std, noise_std=noise_std)
    g = torch.Generator().manual_seed(seed + 7919)
    vals, ids = torch.topk(base.draft / max(temperature, 1e-5), k=S, dim=-1)
    probs = torch.softmax(vals, dim=-1)
    cdf = probs.double().cumsum(-1)
    u = torch.rand(B, K, generator=g)
    local = torch.searchsorted(cdf, (u.double() * cdf[..., -1])[..., None], right=True).clamp_(max=S - 1)
    tokens = ids.gather(-1, local)[..., 0]
    return SparseAcceptInputs(base.target, tokens.long(), ids.long(), probs.float(), base.uniforms,
                              base.resample_u)


@dataclass
class PagedKV:
    k_cache: torch.Tensor  # [num_pages, page_size, Hkv, D] bf16
    v_cache: torch.Tensor
    block_table: torch.Tensor  # [B, max_pages] int32
    context_lens: torch.Tensor  # [B] int32 (prefix + Q)
    page_size: int


def paged_kv(seed: int, context_lens: List[int], Hkv: int = 8, D: int = 128, page_size: int = 16,
             num_pages: Optional[int] = None, device: str = "cpu",
             dtype: torch.dtype = torch.bfloat16) -> PagedKV:
    """A shuffled page pool holding ``context_lens[b]`` tokens per request.

    The pool has ``max(num_pages, sum of pages needed)`` pages rounded up to a
    multiple of 256; each request gets a disjoint slice of a seeded random
    permutation of the page ids.  Unused table entries are 0.
    """
    g = torch.Generator(device="cpu").manual_seed(seed)
    need = [math.ceil(c / page_size) for c in context_lens]
    total = max(sum(need), num_pages or 0, 1)
    total = ((total + 255) // 256) * 256
    perm = torch.randperm(total, generator=g)
    max_pages = max(max(need), 1)
    table = torch.zeros(len(context_lens), max_pages, dtype=torch.int32)
    off = 0
    for b, n in enumerate(need):
        table[b, :n] = perm[off:off + n].int()
        off += n
    gd = torch.Generator(device=device).manual_seed(seed + 1)
    scale = 1.0 / math.sqrt(D)
    k = (torch.randn(total, page_size, Hkv, D, generator=gd, device=device) * scale).to(dtype)
    v = (torch.randn(total, page_size, Hkv, D, generator=gd, device=device) * scale).to(dtype)
    return PagedKV(k, v, table.to(device), torch.tensor(context_lens, dtype=torch.int32, device=device),
                   page_size)


def queries(seed: int, B: int, Q: int, Hq: int = 32, D: int = 128, device: str = "cpu",
            dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    g = torch.Generator(device=device).manual_seed(seed)
    return (torch.randn(B, Q, Hq, D, generator=g, device=device) / math.sqrt(D)).to(dtype)


def concurrent_context_lens(seed: int, B: int = 8, lo: int = 512, hi: int = 8192) -> List[int]:
    """Per-request context lengths ~ U[lo, hi] (inclusive), seeded."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (B,), generator=g).tolist()
