"""ORACLE -- test infrastructure only.

fp32 torch-CPU restatement of the reference acceptance path, op for op:

* ``sampling_probs``     single/eval_sync.py:287-305 (top-k/top-p off)
* ``verify_block``       single/speculative_sampling.py:15-76, with the
                         uniforms passed in instead of ``torch.rand_like``
                         (:55) and ``torch.multinomial`` (:71) replaced by the
                         inverse CDF ``first t with cumsum(dist)_t > v*sum``
* ``verify_block_sparse`` single/speculative_sampling.py:79-143, same changes
* ``greedy``             single/eval_sync.py:1223-1234
* ``paged_attention_sdpa`` the reference's draft-branch pattern
                         (serving/vendor/ssd/layers/attention.py:42-52):
                         gather pages, repeat_interleave the KV heads, SDPA
                         with an explicit mask -- in fp32, with the causal
                         block mask of flash_attn_with_kvcache for verify

It rounds the way the reference's own tensor ops round on CPU, so together
with the fp64 C oracle it brackets the kernel's fp32 results.  It also is the
CPU baseline that bench.py times (kind "port").
"""
from __future__ import annotations

import torch


def sampling_probs(logits: torch.Tensor, temperature: float) -> torch.Tensor:
    if temperature is None or temperature <= 1e-5:
        probs = torch.zeros_like(logits, dtype=torch.float32)
        probs.scatter_(-1, logits.argmax(dim=-1, keepdim=True), 1.0)
        return probs
    return torch.softmax(logits.float() / float(temperature), dim=-1)


def _draw(dist: torch.Tensor, v: float) -> int:
    cdf = torch.cumsum(dist.double(), dim=0)
    total = float(cdf[-1])
    if not total > 0:
        return -1
    hit = torch.nonzero(cdf > v * total)
    if hit.numel():
        return int(hit[0, 0])
    pos = torch.nonzero(dist > 0)
    return int(pos[-1, 0]) if pos.numel() else -1


def verify_block(draft_tokens, target_probs, draft_probs, uniforms, resample_u):
    """Returns (accepted_count, token, all_accepted, accept_mask) for B == 1."""
    p = target_probs.float()
    p = p / p.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    q = draft_probs.float()
    q = q / q.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    draft_len = draft_tokens.shape[1]
    token_ids = draft_tokens[0].long()
    positions = torch.arange(draft_len)
    p_token = p[0, positions, token_ids]
    q_token = q[0, positions, token_ids]
    acceptance_probability = torch.minimum(torch.ones_like(p_token), p_token / q_token.clamp_min(1e-12))
    accepted = uniforms.reshape(-1).float() <= acceptance_probability
    rejected = (~accepted).nonzero(as_tuple=True)[0]
    if rejected.numel() == 0:
        count, dist, all_acc = draft_len, p[0, draft_len], True
    else:
        count = int(rejected[0].item())
        residual = torch.clamp(p[0, count] - q[0, count], min=0.0)
        mass = residual.sum()
        dist = p[0, count] if float(mass.item()) <= 1e-12 else residual / mass
        all_acc = False
    return count, _draw(dist, float(resample_u)), all_acc, accepted


def verify_block_sparse(draft_tokens, target_probs, q_ids, q_probs, uniforms, resample_u):
    p = target_probs.float()
    p = p / p.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    qp = q_probs.float()
    qp = qp / qp.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    qi = q_ids.long()
    draft_len = draft_tokens.shape[1]
    token_ids = draft_tokens[0].long()
    positions = torch.arange(draft_len)
    p_token = p[0, positions, token_ids]
    q_token = (qp[0] * (qi[0] == token_ids.unsqueeze(-1))).sum(dim=-1)
    acceptance_probability = torch.minimum(torch.ones_like(p_token), p_token / q_token.clamp_min(1e-12))
    accepted = uniforms.reshape(-1).float() <= acceptance_probability
    rejected = (~accepted).nonzero(as_tuple=True)[0]
    if rejected.numel() == 0:
        count, dist, all_acc = draft_len, p[0, draft_len], True
    else:
        count = int(rejected[0].item())
        dist = p[0, count].clone()
        dist.scatter_add_(0, qi[0, count], -qp[0, count])
        dist.clamp_min_(0.0)
        mass = dist.sum()
        dist = p[0, count] if float(mass.item()) <= 1e-12 else dist / mass
        all_acc = False
    return count, _draw(dist, float(resample_u)), all_acc, accepted


def greedy(target_logits: torch.Tensor, block: torch.Tensor):
    """(accepted_tail, correction_token, posterior) per request."""
    posterior = target_logits.argmax(dim=-1)
    matches = block[:, 1:] == posterior[:, :-1]
    accepted_tail = matches.long().cumprod(dim=1).sum(dim=1)
    correction = posterior.gather(1, accepted_tail[:, None])[:, 0]
    return accepted_tail, correction, posterior


def paged_attention_sdpa(q, k_cache, v_cache, block_table, context_lens, scale, causal=True):
    """fp32 torch-CPU paged attention; q [B,Q,Hq,D], caches [P,ps,Hkv,D]."""
    B, Q, Hq, D = q.shape
    P, ps, Hkv, _ = k_cache.shape
    outs = []
    for b in range(B):
        ctx = int(context_lens[b])
        t = torch.arange(ctx)
        slots = block_table[b].long()[t // ps] * ps + t % ps
        keys = k_cache.reshape(-1, Hkv, D)[slots].float().transpose(0, 1)
        vals = v_cache.reshape(-1, Hkv, D)[slots].float().transpose(0, 1)
        keys = keys.repeat_interleave(Hq // Hkv, 0)
        vals = vals.repeat_interleave(Hq // Hkv, 0)
        queries = q[b].float().transpose(0, 1)
        if causal:
            mask = torch.arange(ctx)[None, :] <= (ctx - Q + torch.arange(Q))[:, None]
        else:
            mask = torch.ones(Q, ctx, dtype=torch.bool)
        o = torch.nn.functional.scaled_dot_product_attention(queries, keys, vals, attn_mask=mask, scale=scale)
        outs.append(o.transpose(0, 1))
    return torch.stack(outs)
