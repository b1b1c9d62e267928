"""Diffusion-draft block step on the gfx950 kernels.

Mirrors single/eval_sync.py:

* ``sample_tokens`` / ``sample_with_prob`` -- :308-338, proposal draws
                                  (argmax at T <= 1e-5, else the inverse
                                  CDF of softmax(logits / T) at a uniform)
* ``sample_with_sparse_probs`` -- :341-367, top-S support and a draw from it
* ``select_transfer``          -- :447-465 with caller-given tokens and
                                  confidences (the sampled path)

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


def _uniforms(shape, dev, uniforms, generator):
    if uniforms is None:
        uniforms = torch.rand(shape, device=dev, generator=generator)
    return uniforms.to(device=dev, dtype=torch.float32).reshape(shape).contiguous()


def sample_with_prob(logits: torch.Tensor, temperature: float = 0.0, *, uniforms: Optional[torch.Tensor] = None,
                     generator: Optional[torch.Generator] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """(tokens [...], probs [...]) of logits [..., V]: single/eval_sync.py:324-338.

    T <= 1e-5: the argmax with probability 1.  Otherwise the token is the
    inverse-CDF draw of softmax(logits / T) at ``uniforms`` (one per row,
    drawn with torch.rand when omitted) and probs its probability.
    """
    dev = _lib.require_device(logits)
    lg = logits if logits.dtype in (torch.float32, torch.bfloat16) else logits.float()
    lg = lg.contiguous()
    V = lg.shape[-1]
    N = lg.numel() // V
    greedy = not temperature > 1e-5
    u = None if greedy else _uniforms(lg.shape[:-1], dev, uniforms, generator)
    tok = torch.empty(lg.shape[:-1], dtype=torch.int64, device=dev)
    prob = torch.empty(lg.shape[:-1], dtype=torch.float32, device=dev)
    lib = _lib.load()
    ws = _lib.workspace(dev, "sample", lib.d3d_sample_workspace_bytes(max(N, 1), V))
    st = lib.d3d_sample_rows(lg.data_ptr(), _lib.dtype_code(lg), N, V, float(temperature), _lib.ptr(u),
                             tok.data_ptr(), prob.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev))
    _lib.check(st, "d3d_sample_rows")
    return tok, prob


def sample_tokens(logits: torch.Tensor, temperature: float = 0.0, *, uniforms: Optional[torch.Tensor] = None,
                  generator: Optional[torch.Generator] = None) -> torch.Tensor:
    """single/eval_sync.py:308-321: the tokens of :func:`sample_with_prob`."""
    return sample_with_prob(logits, temperature, uniforms=uniforms, generator=generator)[0]


def sample_with_sparse_probs(logits: torch.Tensor, temperature: float, top_k: int, *,
                             uniforms: Optional[torch.Tensor] = None, generator: Optional[torch.Generator] = None):
    """(tokens, support ids [..., S], support probs [..., S]): single/eval_sync.py:341-367.

    T <= 1e-5: the argmax as a support of one with probability 1.  Otherwise
    the support is the S = top_k largest logits (descending, ties by lower
    id; 1 <= S <= 64), its probabilities softmax(logits / T) over the
    support, and the token the inverse-CDF draw from them.
    """
    dev = _lib.require_device(logits)
    if not temperature > 1e-5:
        tok = topk_tokens(logits, 1)
        return tok[..., 0], tok, torch.ones(tok.shape, dtype=torch.float32, device=dev)
    S = int(top_k)
    if not 1 <= S <= min(64, logits.shape[-1]):
        raise ValueError("sparse proposals need 1 <= top_k <= 64 support entries")
    ids, vals = topk_tokens(logits, S, with_values=True)
    N = ids.numel() // S
    u = _uniforms(logits.shape[:-1], dev, uniforms, generator)
    tok = torch.empty(logits.shape[:-1], dtype=torch.int64, device=dev)
    probs = torch.empty(ids.shape, dtype=torch.float32, device=dev)
    st = _lib.load().d3d_sample_support(vals.data_ptr(), ids.data_ptr(), N, S, float(temperature), u.data_ptr(),
                                        tok.data_ptr(), probs.data_ptr(), None, _lib.stream_ptr(dev))
    _lib.check(st, "d3d_sample_support")
    return tok, ids, probs


def select_transfer(block: torch.Tensor, mask_id: int, k: int, x0: torch.Tensor,
                    conf: torch.Tensor) -> torch.Tensor:
    """Unmask the k most confident masked positions of each request in place.

    single/eval_sync.py:447-465 with caller-given x0 [B, Q] and confidences
    [B, Q] (ties: lowest position); returns the unmasked positions [B, Q]
    bool.  Selection is per request.
    """
    dev = _lib.require_device(block, x0, conf)
    if block.ndim != 2 or block.dtype != torch.int64 or not block.is_contiguous():
        raise ValueError("block must be a contiguous int64 [B, Q] tensor (updated in place)")
    B, Q = block.shape
    x0 = x0.to(torch.int64).reshape(B, Q).contiguous()
    conf = conf.to(torch.float32).reshape(B, Q).contiguous()
    sel = torch.empty(B, Q, dtype=torch.uint8, device=dev)
    st = _lib.load().d3d_select_transfer(block.data_ptr(), int(mask_id), int(k), x0.data_ptr(), conf.data_ptr(),
                                         sel.data_ptr(), B, Q, _lib.stream_ptr(dev))
    _lib.check(st, "d3d_select_transfer")
    return sel.bool()


def topk_tokens(logits: torch.Tensor, k: int, with_values: bool = False, log_softmax: bool = False):
    """Top-k token ids [..., k] int64 of logits [..., V] (fp32 or bf16), one launch pair.

    Descending value, equal values by ascending id: ``ids[..., 0]`` is the
    argmax (torch's first maximum).  serving/backend.py:84-93 (greedy and
    ``logits.topk(k).indices``).  With ``with_values`` also returns the
    values [..., k] fp32 -- as log-probabilities with ``log_softmax``
    (single/eval_sync.py:763-768).
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
    st = lib.d3d_topk_rows(lg.data_ptr(), _lib.dtype_code(lg), N, V, int(k), int(bool(log_softmax)),
                           ids.data_ptr(), _lib.ptr(vals), ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev))
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


def _denoise(drafter: Qwen3PagedModel, kv: PagedKV, seqs: List[Sequence], cur: torch.Tensor, schedule: List[int],
             *, mask_id: int, temperature: float, top_k: int, name: str, graphs: Optional[dict],
             width: Optional[int], uniforms: Optional[torch.Tensor], generator: Optional[torch.Generator],
             return_proposal: Optional[str], first_forward=None):
    """The denoise loop of single/eval_sync.py:511-589, in place on ``cur``.

    ``first_forward`` (optional) computes step 0's logits instead of the
    plain block forward (the fused commit of the pending tokens).  Returns
    (proposal, logits of the last step or None when replayed from graphs).
    """
    stochastic = temperature > 1e-5
    B, Q = cur.shape
    starts = [s.prefix for s in seqs]
    for s in seqs:
        reserve(kv, s, name, s.prefix + Q)
    tables, slots, lens, logical, _ = block_inputs(kv, seqs, name, starts, Q, drafter.device, width)
    W = tables.shape[1]
    if stochastic:
        u_all = uniforms if uniforms is not None else torch.rand(len(schedule), B, Q, device=cur.device,
                                                                 generator=generator)
        u_all = u_all.to(device=cur.device, dtype=torch.float32).reshape(len(schedule), B, Q)
    proposal = logits = None
    for step, k in enumerate(schedule):
        if step == len(schedule) - 1:
            k = Q  # the last step unmasks everything left (:549-550)
        if not stochastic and graphs is not None and not (step == 0 and first_forward is not None):
            key = (B, Q, k, W, temperature)
            step_fn = graphs.get(key)
            if step_fn is None:
                def post(hidden, ids, k=k):
                    confidence_topk_unmask(drafter.logits(hidden), ids, mask_id, k, temperature)
                    return ids
                step_fn = graphs[key] = BlockStep(drafter, kv, B, Q, W, causal=False, post=post)
            cur.copy_(step_fn(cur, logical, tables, slots, lens))
            logits = None
            continue
        if step == 0 and first_forward is not None:
            logits = first_forward(cur)
        else:
            hidden = drafter(cur, logical, kv, tables, lens, slots, causal=False, max_context=W * kv.page_size)
            logits = drafter.logits(hidden)
        if not stochastic:
            confidence_topk_unmask(logits, cur, mask_id, k, temperature)
            continue
        if return_proposal == "sparse":
            x0, ids, probs = sample_with_sparse_probs(logits, temperature, top_k, uniforms=u_all[step])
            conf = probs.gather(-1, (ids == x0[..., None]).long().argmax(-1, keepdim=True))[..., 0]
        else:
            x0, conf = sample_with_prob(logits, temperature, uniforms=u_all[step])
        sel = select_transfer(cur, mask_id, k, x0, conf)
        if return_proposal == "logits":
            proposal = logits.clone() if proposal is None else torch.where(sel[..., None], logits, proposal)
        elif return_proposal == "sparse":
            if proposal is None:
                proposal = (torch.zeros_like(ids), torch.zeros_like(probs))
            proposal = (torch.where(sel[..., None], ids, proposal[0]), torch.where(sel[..., None], probs, proposal[1]))
    return proposal, logits


def d3d_draft_block(drafter: Qwen3PagedModel, kv: PagedKV, seqs: List[Sequence], block: torch.Tensor,
                    denoising_steps: int, *, mask_id: int = MASK_ID, temperature: float = 0.0, top_k: int = 0,
                    name: str = "draft", graphs: Optional[dict] = None, width: Optional[int] = None,
                    uniforms: Optional[torch.Tensor] = None, generator: Optional[torch.Generator] = None,
                    return_proposal: Optional[str] = None):
    """Denoise a block [B, Q] whose masked positions hold ``mask_id``.

    single/eval_sync.py:482-592 with low-confidence remasking: each step
    runs the draft over the block, then unmasks the scheduled number of most
    confident masked positions; the last step fills every remaining mask.
    ``num_masks`` is taken from request 0, as the reference's schedule is
    (:503-508).

    T <= 1e-5: x0 is the argmax and the confidence its softmax probability
    (one fused kernel per step).  T > 1e-5: x0 is drawn from softmax(logits
    / T) (dense) or from the top-``top_k`` support (``return_proposal=
    "sparse"``) at ``uniforms`` [steps, B, Q] (torch.rand when omitted), and
    the confidence is the drawn token's probability (:560-576).

    ``return_proposal`` (T > 1e-5): ``"logits"`` also returns the draft
    logits row of every position at the step it was unmasked -- the proposal
    q = softmax(row / T) that the reference keeps as proposal_probs
    (:577-584), consumed by the acceptance kernel directly -- and
    ``"sparse"`` returns (support ids [B, Q, S], support probs [B, Q, S])
    (:585-589).

    With a ``graphs`` dict (greedy mode) each (forward + unmask) step is
    replayed from a HIP graph cached there per (B, Q, k, table width);
    ``width`` fixes the page-table width (default: the current longest table).
    """
    if return_proposal not in (None, "logits", "sparse"):
        raise ValueError("return_proposal must be None, 'logits' or 'sparse'")
    cur = block.clone().contiguous()
    num_masks = int((cur[0] == mask_id).sum().item())
    if num_masks == 0:
        return (cur, None) if return_proposal else cur
    schedule = get_num_transfer_tokens(num_masks, denoising_steps)
    proposal, _ = _denoise(drafter, kv, seqs, cur, schedule, mask_id=mask_id, temperature=temperature, top_k=top_k,
                           name=name, graphs=graphs, width=width, uniforms=uniforms, generator=generator,
                           return_proposal=return_proposal)
    if return_proposal:
        return cur, proposal
    return cur


def d3d_draft_block_fused_commit(drafter: Qwen3PagedModel, kv: PagedKV, seqs: List[Sequence], block: torch.Tensor,
                                 pending: Optional[torch.Tensor], denoising_steps: int, *, mask_id: int = MASK_ID,
                                 temperature: float = 0.0, top_k: int = 0,
                                 attention_mask_mode: str = "block_causal", return_topk: int = 0,
                                 return_proposal: Optional[str] = None, uniforms: Optional[torch.Tensor] = None,
                                 generator: Optional[torch.Generator] = None, name: str = "draft",
                                 width: Optional[int] = None):
    """Anchor-conditioned draft step that also commits the pending tokens' K/V.

    single/eval_sync.py:596-775.  ``pending`` [B, n] holds the committed
    tokens whose draft K/V are not written yet; each ``seqs[b].prefix``
    counts them (the reference's prefix_len = draft_kv_len + n).  The first
    denoise step runs one forward over [pending; block] at positions
    draft_kv_len.. with the fused mask of :251-275 (pending rows see the
    cache and the pending tokens -- all of them in "block_causal" mode,
    causally in "causal" mode -- and block rows see everything); the pending
    tokens' K/V stay in the cache.  Later steps are the plain block forward.

    Returns ``cur`` alone, or ``(cur, metrics)`` when ``return_topk`` > 0, or
    ``(cur, metrics, proposal)`` with ``return_proposal``; metrics holds
    ``top_tokens`` / ``top_logprobs`` [B, Q, return_topk] of the last step's
    log_softmax (:763-768), None when the block had no mask.
    """
    if attention_mask_mode not in ("block_causal", "causal"):
        raise ValueError(f"unsupported attention_mask_mode={attention_mask_mode!r}")
    if return_proposal not in (None, "logits", "sparse"):
        raise ValueError("return_proposal must be None, 'logits' or 'sparse'")
    cur = block.clone().contiguous()
    B, Q = cur.shape
    dev = cur.device
    n = 0 if pending is None else int(pending.shape[1])
    if n and (pending.shape[0] != B or any(s.prefix < n for s in seqs)):
        raise ValueError("pending must be [B, n] with n <= every request's committed prefix")

    def commit_forward(ids_block: torch.Tensor) -> torch.Tensor:
        """Forward over [pending; block] at draft_kv_len..; logits of the block rows."""
        kv_lens = [s.prefix - n for s in seqs]
        for s, k0 in zip(seqs, kv_lens):
            reserve(kv, s, name, k0 + n + Q)
        tables, slots, lens, logical, _ = block_inputs(kv, seqs, name, kv_lens, n + Q, dev, width)
        rows = [(i + 1 if attention_mask_mode == "causal" else n, 0, 0) for i in range(n)]
        rows += [(n + Q, 0, 0)] * Q
        vis = torch.tensor(rows, dtype=torch.int32).to(dev, non_blocking=True)
        ids = torch.cat([pending.to(dev, torch.int64), ids_block], dim=1)
        hidden = drafter(ids, logical, kv, tables, lens, slots, causal=False,
                         max_context=tables.shape[1] * kv.page_size, q_vis=vis)
        return drafter.logits(hidden[:, n:])

    num_masks = int((cur == mask_id).sum().item())
    metrics = {"top_tokens": None, "top_logprobs": None}
    proposal = None
    if num_masks == 0:
        if n:
            commit_forward(cur)
    else:
        schedule = get_num_transfer_tokens(num_masks, denoising_steps)
        proposal, final = _denoise(drafter, kv, seqs, cur, schedule, mask_id=mask_id, temperature=temperature,
                                   top_k=top_k, name=name, graphs=None, width=width, uniforms=uniforms,
                                   generator=generator, return_proposal=return_proposal,
                                   first_forward=commit_forward if n else None)
        if return_topk > 0 and final is not None:
            k = min(int(return_topk), final.shape[-1])
            ids, lp = topk_tokens(final, k, with_values=True, log_softmax=True)
            metrics = {"top_tokens": ids, "top_logprobs": lp}
    if return_proposal:
        return cur, metrics, proposal
    if return_topk > 0:
        return cur, metrics
    return cur
