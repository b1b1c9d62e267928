"""Target verify step: forward over the draft block, then acceptance.

Mirrors the verifier process's "verify" command, single/eval_async_packed.py:
115-199, batched over requests:

* the block (anchor + draft tokens) runs through the target at positions
  prefix.. with causal attention within the block; its K/V land in the
  paged cache after the committed prefix (the reference crops its cache to
  kv_len first, :121; here the committed prefix bounds every read);
* T <= 1e-5: greedy acceptance -- posterior = argmax of every row,
  accepted = leading draft tokens equal to the posterior before them,
  correction = posterior[accepted] (:168-174);
* T > 1e-5: rejection sampling against the sparse proposal
  (verify_speculative_block_sparse, :152-167) or a dense proposal given as
  the draft logits rows, in one fused kernel that also applies the target
  temperature softmax (_sampling_probs, :134-139);
* a block of one token (no draft tail) draws the correction from the last
  row (:143-150).

Tokens that cannot be drawn come back from the kernels as negative statuses
(an out-of-range draft token, a distribution without mass).  The reference's
gather and torch.multinomial raise there, so ``verify_step`` checks the
correction tokens by default and raises the same errors; ``check=False``
keeps the step free of host synchronisation and leaves the statuses in
``correction_token`` for the caller (``correction_token >= 0`` marks the
valid requests).
"""
from __future__ import annotations

from typing import List, NamedTuple, Optional

import torch

from . import speculative_sampling as ss
from .draft import sample_tokens
from .model import PagedKV, Qwen3PagedModel, Sequence, block_inputs, reserve


class VerifyResult(NamedTuple):
    posterior: torch.Tensor        # [B, Q] int64, argmax of every target row
    accepted_tail: torch.Tensor    # [B] int32, accepted draft tokens (0..Q-1)
    correction_token: torch.Tensor  # [B] int64
    logits: Optional[torch.Tensor]  # [B, Q, V] target logits when asked for


def verify_step(target: Qwen3PagedModel, kv: PagedKV, seqs: List[Sequence], blocks: torch.Tensor, *,
                temperature: float = 0.0, draft_token_ids: Optional[torch.Tensor] = None,
                draft_token_probs: Optional[torch.Tensor] = None, draft_logits: Optional[torch.Tensor] = None,
                uniforms: Optional[torch.Tensor] = None, resample_uniform: Optional[torch.Tensor] = None,
                generator: Optional[torch.Generator] = None, name: str = "target", width: Optional[int] = None,
                return_logits: bool = False, check: bool = True) -> VerifyResult:
    """Verify B blocks [B, Q] against the target.  With ``check`` (the
    default) one host synchronisation reads the correction tokens and raises
    ValueError / RuntimeError for a request that carries a status instead."""
    B, Q = blocks.shape
    dev = target.device
    blocks = blocks.to(dev, torch.int64).contiguous()
    if check and bool(((blocks < 0) | (blocks >= target.shape.vocab)).any()):
        # The embedding lookup of the forward must not see such an id.
        raise ValueError("draft token id outside the vocabulary")
    for s in seqs:
        reserve(kv, s, name, s.prefix + Q)
    tables, slots, lens, logical, max_ctx = block_inputs(kv, seqs, name, [s.prefix for s in seqs], Q, dev, width)
    hidden = target(blocks, logical, kv, tables, lens, slots, causal=True, max_context=max_ctx)
    logits = target.logits(hidden)
    greedy = not temperature > 1e-5
    if Q == 1:
        posterior = logits.argmax(-1)
        if greedy:
            corr = posterior[:, 0]
        else:
            corr = sample_tokens(logits[:, -1], temperature, uniforms=resample_uniform, generator=generator)
        acc = torch.zeros(B, dtype=torch.int32, device=dev)
        if check:
            for b, token in enumerate(corr.tolist()):
                if token < 0:
                    ss._raise_for_token(token, b if B > 1 else None)
        return VerifyResult(posterior, acc, corr, logits if return_logits else None)
    tail = blocks[:, 1:]
    if greedy:
        out = ss.greedy_accept(logits, blocks)
    elif draft_token_ids is not None and draft_token_probs is not None:
        out = ss.accept_fused_sparse(logits, tail, draft_token_ids, draft_token_probs, temperature=temperature,
                                     uniforms=uniforms, resample_uniform=resample_uniform, input_kind="logits",
                                     generator=generator)
    elif draft_logits is not None:
        out = ss.accept_fused(logits, draft_logits, tail, temperature=temperature, uniforms=uniforms,
                              resample_uniform=resample_uniform, input_kind="logits", generator=generator)
    else:
        raise RuntimeError("temperature > 0 verification requires sparse draft q")
    if check:
        out.check()
    return VerifyResult(out.posterior, out.accepted, out.out_token, logits if return_logits else None)
