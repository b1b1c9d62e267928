"""Diffusion-draft block step on the gfx950 kernels.

Mirrors single/eval_sync.py:

* ``sampling_probs``           -- :287-305 (_sampling_probs), the dense
                                  proposal distribution: one-hot at T <= 1e-5,
                                  else softmax(logits / T) with the top-k
                                  filter (ties with the k-th value kept) and
                                  the top-p (nucleus) filter
* ``sample_tokens`` / ``sample_with_prob`` -- :308-338, proposal draws
                                  (argmax at T <= 1e-5, else the inverse CDF
                                  of the filtered softmax at a uniform)
* ``sample_with_sparse_probs`` -- :341-367, top-S support (any S, sorted
                                  descending), nucleus filter and a draw
* ``select_transfer``          -- :447-465 (_select_transfer) with
                                  caller-given tokens and confidences,
                                  "low_confidence" and "dynamic" remasking
* ``get_num_transfer_tokens``  -- :440-444, the per-step unmask schedule
* ``confidence_topk_unmask``   -- the greedy step of :511-576 in one kernel
                                  launch: argmax, confidence and selection
* ``d3d_draft_block``          -- :482-592 with the reference's parameters
* ``d3d_draft_block_fused_commit`` -- :596-775 with the reference's parameters
* ``draft_block_step``         -- the batched denoise loop over a paged cache
                                  (the engine's and the benchmarks' form),
                                  optionally replayed from HIP graphs

Greedy confidence: the reference draws greedy tokens through
_sample_with_prob, whose one-hot distribution gives every position
confidence 1.0 (:287-291, :323-338), so its top-k among masked positions
falls to the lowest positions (the index order in which torch's CUDA top-k
gathers tied values).  That is ``confidence="sampled"``, the default.
``confidence="max_softmax"`` ranks by the argmax token's softmax
probability instead -- the reference's metrics confidence (:713-717) and
SGLang's LowConfidence.  Selection is per request (the reference applies
row 0's indices to every row, :461-464) and ties in confidence go to the
lowest position.
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import torch

from . import _lib
from .model import BlockStep, PagedKV, Qwen3PagedModel, Sequence, block_inputs, reserve

MASK_ID = 151669
_REMASKING = ("low_confidence", "dynamic", "low_confidence_dynamic")


def get_num_transfer_tokens(num_masks: int, steps: int) -> List[int]:
    """single/eval_sync.py:440-444: an even split, the remainder going first."""
    steps = max(1, int(steps))
    base, extra = divmod(int(num_masks), steps)
    return [base + (1 if i < extra else 0) for i in range(steps)]


def _remasking(remasking: Optional[str], threshold: Optional[float]) -> Tuple[bool, float]:
    """(dynamic, threshold) of a remasking name (single/eval_sync.py:453)."""
    name = remasking or "low_confidence"
    if name not in _REMASKING:
        raise ValueError(f"unsupported remasking={remasking!r}: expected one of {_REMASKING}")
    dynamic = "dynamic" in name
    if dynamic:
        if threshold is None or not threshold == threshold:
            raise ValueError("dynamic remasking needs a numeric threshold")
        return True, float(threshold)
    return False, 0.0


def confidence_topk_unmask(logits: torch.Tensor, block: torch.Tensor, mask_id: int, k: int,
                           temperature: float = 0.0, *, confidence: str = "max_softmax",
                           remasking: str = "low_confidence",
                           threshold: Optional[float] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Unmask the k most confident masked positions of each request, in place.

    ``logits`` [B, Q, V] (fp32 or bf16), ``block`` [B, Q] int64 on the same
    device.  ``confidence`` "max_softmax" (the argmax token's softmax
    probability) or "sampled" (1.0: the greedy draw's one-hot probability;
    T <= 1e-5 only).  Returns (x0 [B, Q] int64, conf [B, Q] fp32) for every
    position.
    """
    dev = _lib.require_device(logits, block)
    if logits.ndim != 3 or block.shape != logits.shape[:2] or block.dtype != torch.int64:
        raise ValueError("expected logits [B,Q,V] and an int64 block [B,Q]")
    if not block.is_contiguous():
        raise ValueError("block must be contiguous (it is updated in place)")
    if confidence not in ("max_softmax", "sampled"):
        raise ValueError("confidence must be 'max_softmax' or 'sampled'")
    dynamic, thr = _remasking(remasking, threshold)
    mode = _lib.D3D_CONF_MAX_SOFTMAX if confidence == "max_softmax" else _lib.D3D_CONF_ONE_HOT
    B, Q, V = logits.shape
    lg = logits if logits.dtype in (torch.float32, torch.bfloat16) else logits.float()
    lg = lg.contiguous()
    x0 = torch.empty(B, Q, dtype=torch.int64, device=dev)
    conf = torch.empty(B, Q, dtype=torch.float32, device=dev)
    lib = _lib.load()
    nbytes = lib.d3d_confidence_workspace_bytes(B, Q, V)
    ws = _lib.workspace(dev, "confidence", nbytes)
    st = lib.d3d_confidence_topk_unmask(lg.data_ptr(), _lib.dtype_code(lg), block.data_ptr(), int(mask_id),
                                        int(k), float(temperature), mode, int(dynamic), thr, B, Q, V,
                                        x0.data_ptr(), conf.data_ptr(), ws.data_ptr(), ws.numel(),
                                        _lib.stream_ptr(dev))
    _lib.check(st, "d3d_confidence_topk_unmask")
    return x0, conf


def _uniforms(shape, dev, uniforms, generator):
    if uniforms is None:
        uniforms = torch.rand(shape, device=dev, generator=generator)
    return uniforms.to(device=dev, dtype=torch.float32).reshape(shape).contiguous()


def _filters(logits: torch.Tensor, temperature: float, top_k: int, top_p: Optional[float]):
    """The top-k / top-p filter of _sampling_probs (single/eval_sync.py:
    292-303) for rows [N, V]: (kth, None, None) with kth the per-row k-th
    largest logit for a top-k filter alone of at most 64 entries (one top-k
    launch pair), (None, zfloor, zlimit) from d3d_row_filter for top-p or a
    wider top-k, (None, None, None) when both are off."""
    V = logits.shape[-1]
    k = int(top_k) if top_k and top_k > 0 else 0
    if k >= V:
        k = 0
    p = 1.0 if top_p is None else float(top_p)
    if not 0.0 < p <= 1.0:
        raise ValueError("top_p must lie in (0, 1]")
    if p >= 1.0 and k == 0:
        return None, None, None
    if p >= 1.0 and k <= 64:
        _, vals = topk_tokens(logits, k, with_values=True)
        return vals[..., k - 1].reshape(-1).contiguous(), None, None
    N = logits.numel() // V
    dev = logits.device
    zf = torch.empty(N, dtype=torch.float32, device=dev)
    lim = torch.empty(N, dtype=torch.int32, device=dev)
    st = _lib.load().d3d_row_filter(logits.data_ptr(), _lib.dtype_code(logits), N, V, float(temperature), k, p,
                                    zf.data_ptr(), lim.data_ptr(), _lib.stream_ptr(dev))
    _lib.check(st, "d3d_row_filter")
    return None, zf, lim


def sample_with_prob(logits: torch.Tensor, temperature: float = 0.0, top_k: int = 0, top_p: float = 1.0, *,
                     uniforms: Optional[torch.Tensor] = None,
                     generator: Optional[torch.Generator] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """(tokens [...], probs [...]) of logits [..., V]: single/eval_sync.py:324-338.

    T <= 1e-5: the argmax with probability 1.  Otherwise the token is the
    inverse-CDF draw of softmax(logits / T) over the entries the top-k and
    top-p filters keep (both as in :func:`sampling_probs`) at ``uniforms``
    (one per row, drawn with torch.rand when omitted) and probs its
    probability.
    """
    dev = _lib.require_device(logits)
    lg = logits if logits.dtype in (torch.float32, torch.bfloat16) else logits.float()
    lg = lg.contiguous()
    V = lg.shape[-1]
    N = lg.numel() // V
    greedy = not temperature > 1e-5
    u = None if greedy else _uniforms(lg.shape[:-1], dev, uniforms, generator)
    kth, zf, lim = (None, None, None) if greedy else _filters(lg, temperature, top_k, top_p)
    tok = torch.empty(lg.shape[:-1], dtype=torch.int64, device=dev)
    prob = torch.empty(lg.shape[:-1], dtype=torch.float32, device=dev)
    lib = _lib.load()
    ws = _lib.workspace(dev, "sample", lib.d3d_sample_workspace_bytes(max(N, 1), V))
    st = lib.d3d_sample_rows(lg.data_ptr(), _lib.dtype_code(lg), N, V, float(temperature), _lib.ptr(kth),
                             _lib.ptr(zf), _lib.ptr(lim), _lib.ptr(u), tok.data_ptr(), prob.data_ptr(),
                             ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev))
    _lib.check(st, "d3d_sample_rows")
    return tok, prob


def sample_tokens(logits: torch.Tensor, temperature: float = 0.0, top_k: int = 0, top_p: float = 1.0, *,
                  uniforms: Optional[torch.Tensor] = None,
                  generator: Optional[torch.Generator] = None) -> torch.Tensor:
    """single/eval_sync.py:308-321: the tokens of :func:`sample_with_prob`."""
    return sample_with_prob(logits, temperature, top_k, top_p, uniforms=uniforms, generator=generator)[0]


def sampling_probs(logits: torch.Tensor, temperature: float = 0.0, top_k: int = 0,
                   top_p: float = 1.0) -> torch.Tensor:
    """single/eval_sync.py:287-305: dense probabilities [..., V] fp32.

    One-hot at the first argmax for T <= 1e-5.  Otherwise softmax over z =
    logits / T restricted to the entries the filters keep: ``top_k`` > 0 the
    entries at or above the k-th largest z (ties kept), then ``top_p`` < 1
    the shortest prefix of those in descending order (ties by ascending id)
    whose softmax mass exceeds top_p, the entry that crosses it included."""
    dev = _lib.require_device(logits)
    lg = logits if logits.dtype in (torch.float32, torch.bfloat16) else logits.float()
    lg = lg.contiguous()
    V = lg.shape[-1]
    N = lg.numel() // V
    greedy = not temperature > 1e-5
    kth, zf, lim = (None, None, None) if greedy else _filters(lg, temperature, top_k, top_p)
    out = torch.empty(lg.shape, dtype=torch.float32, device=dev)
    lib = _lib.load()
    ws = _lib.workspace(dev, "sample", lib.d3d_sample_workspace_bytes(max(N, 1), V))
    st = lib.d3d_softmax_rows(lg.data_ptr(), _lib.dtype_code(lg), N, V, float(temperature), _lib.ptr(kth),
                              _lib.ptr(zf), _lib.ptr(lim), out.data_ptr(), ws.data_ptr(), ws.numel(),
                              _lib.stream_ptr(dev))
    _lib.check(st, "d3d_softmax_rows")
    return out


def sample_with_sparse_probs(logits: torch.Tensor, temperature: float, top_k: int, top_p: float = 1.0, *,
                             uniforms: Optional[torch.Tensor] = None, generator: Optional[torch.Generator] = None):
    """(tokens, support ids [..., S], support probs [..., S]): single/eval_sync.py:341-367.

    T <= 1e-5: the argmax as a support of one with probability 1.  Otherwise
    the support is the S = top_k largest z = logits / T (top_k = 0: the
    whole vocabulary) in descending order, ties by ascending id; its
    probabilities are softmax(z) over the support after the nucleus filter
    (``top_p`` < 1: entry s > 0 is dropped when the mass of entries 0..s-1
    exceeds top_p), and the token is the inverse-CDF draw from them in
    support order.  Supports of up to 64 entries take the top-k kernel and
    one wave per row; wider ones the sorted-support path.
    """
    dev = _lib.require_device(logits)
    if not temperature > 1e-5:
        tok = topk_tokens(logits, 1)
        return tok[..., 0], tok, torch.ones(tok.shape, dtype=torch.float32, device=dev)
    if not (top_p is None or 0.0 < top_p <= 1.0):
        raise ValueError("top_p must lie in (0, 1]")
    p = float(1.0 if top_p is None else top_p)
    V = logits.shape[-1]
    S = int(top_k) if int(top_k) > 0 else V
    S = min(S, V)
    lg = logits if logits.dtype in (torch.float32, torch.bfloat16) else logits.float()
    lg = lg.contiguous()
    N = lg.numel() // V
    u = _uniforms(lg.shape[:-1], dev, uniforms, generator)
    tok = torch.empty(lg.shape[:-1], dtype=torch.int64, device=dev)
    probs = torch.empty(*lg.shape[:-1], S, dtype=torch.float32, device=dev)
    if S > 64:
        ids = torch.empty(*lg.shape[:-1], S, dtype=torch.int64, device=dev)
        lib = _lib.load()
        nbytes = lib.d3d_support_workspace_bytes(max(N, 1), S)
        if nbytes == 0:
            raise RuntimeError("d3d_support_workspace_bytes failed")
        ws = _lib.workspace(dev, "support", nbytes)
        st = lib.d3d_sample_support_wide(lg.data_ptr(), _lib.dtype_code(lg), N, V, float(temperature), S, p,
                                         u.data_ptr(), tok.data_ptr(), ids.data_ptr(), probs.data_ptr(), None,
                                         ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev))
        _lib.check(st, "d3d_sample_support_wide")
        return tok, ids, probs
    ids, vals = topk_tokens(lg, S, with_values=True)
    st = _lib.load().d3d_sample_support(vals.data_ptr(), ids.data_ptr(), N, S, float(temperature), p,
                                        u.data_ptr(), tok.data_ptr(), probs.data_ptr(), None, _lib.stream_ptr(dev))
    _lib.check(st, "d3d_sample_support")
    return tok, ids, probs


def select_transfer(block: torch.Tensor, mask_id: int, k: int, x0: torch.Tensor, conf: torch.Tensor, *,
                    remasking: str = "low_confidence", threshold: Optional[float] = None) -> torch.Tensor:
    """Unmask the k most confident masked positions of each request in place.

    single/eval_sync.py:447-465 with caller-given x0 [B, Q] and confidences
    [B, Q] (ties: lowest position); "dynamic" remasking takes only the masked
    positions whose confidence reaches ``threshold`` (at most k of them)
    when there are any.  Returns the unmasked positions [B, Q] bool.
    Selection is per request.
    """
    dev = _lib.require_device(block, x0, conf)
    if block.ndim != 2 or block.dtype != torch.int64 or not block.is_contiguous():
        raise ValueError("block must be a contiguous int64 [B, Q] tensor (updated in place)")
    dynamic, thr = _remasking(remasking, threshold)
    B, Q = block.shape
    x0 = x0.to(torch.int64).reshape(B, Q).contiguous()
    conf = conf.to(torch.float32).reshape(B, Q).contiguous()
    sel = torch.empty(B, Q, dtype=torch.uint8, device=dev)
    st = _lib.load().d3d_select_transfer(block.data_ptr(), int(mask_id), int(k), int(dynamic), thr, x0.data_ptr(),
                                         conf.data_ptr(), sel.data_ptr(), B, Q, _lib.stream_ptr(dev))
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


def _mask_count(cur: torch.Tensor, mask_id: int) -> int:
    """Masked positions per request; every request must hold the same number
    (one schedule serves the batch, as in the reference's B = 1 loop)."""
    counts = (cur == mask_id).sum(-1).tolist()
    if len(set(counts)) > 1:
        raise ValueError("every request of a draft batch must hold the same number of masked positions")
    return int(counts[0]) if counts else 0


def _denoise(drafter: Qwen3PagedModel, kv: PagedKV, seqs: List[Sequence], cur: torch.Tensor, schedule: List[int],
             *, mask_id: int, temperature: float, top_k: int, top_p: float, remasking: str,
             threshold: Optional[float], confidence: str, name: str, graphs: Optional[dict],
             width: Optional[int], uniforms: Optional[torch.Tensor], generator: Optional[torch.Generator],
             proposal: Optional[str], first_forward=None, metrics_last: bool = False):
    """The denoise loop of single/eval_sync.py:511-589 (and :673-757), in place on ``cur``.

    ``first_forward`` (optional) computes step 0's logits instead of the
    plain block forward (the fused commit of the pending tokens).
    ``proposal``: None, "probs" (dense proposal_probs [B, Q, V]), "logits"
    (the logits row of each position at the step it was unmasked) or
    "sparse" ((ids, probs) [B, Q, S]).  ``metrics_last``: the last step
    takes the max-softmax confidence (:708-717).  Returns (proposal, logits
    of the last step -- None when replayed from graphs).
    """
    stochastic = temperature > 1e-5
    dynamic, _ = _remasking(remasking, threshold)
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
    out = None
    logits = None
    remaining = _mask_count(cur, mask_id)
    for step, k in enumerate(schedule):
        # The loop stops once no mask is left (:512-514).  Without dynamic
        # remasking the schedule says when; with it, the block is read.
        if dynamic and step > 0:
            remaining = int((cur == mask_id).sum().item())
        if remaining == 0:
            break
        last = step == len(schedule) - 1
        if last:
            k = Q  # the last step unmasks everything left (:549-550)
        conf_mode = "max_softmax" if (last and metrics_last) else confidence
        replay = (not stochastic and graphs is not None and not (step == 0 and first_forward is not None))
        if replay:
            key = (B, Q, k, W, temperature, conf_mode, remasking, threshold)
            step_fn = graphs.get(key)
            if step_fn is None:
                def post(hidden, ids, k=k, conf_mode=conf_mode):
                    confidence_topk_unmask(drafter.logits(hidden), ids, mask_id, k, temperature,
                                           confidence=conf_mode, remasking=remasking, threshold=threshold)
                    return ids
                step_fn = graphs[key] = BlockStep(drafter, kv, B, Q, W, causal=False, post=post)
            cur.copy_(step_fn(cur, logical, tables, slots, lens))
            logits = None
        else:
            if step == 0 and first_forward is not None:
                logits = first_forward(cur)
            else:
                hidden = drafter(cur, logical, kv, tables, lens, slots, causal=False, max_context=W * kv.page_size)
                logits = drafter.logits(hidden)
            if not stochastic:
                confidence_topk_unmask(logits, cur, mask_id, k, temperature, confidence=conf_mode,
                                       remasking=remasking, threshold=threshold)
            else:
                if proposal == "sparse":
                    x0, ids, probs = sample_with_sparse_probs(logits, temperature, top_k, top_p,
                                                              uniforms=u_all[step])
                    conf = probs.gather(-1, (ids == x0[..., None]).long().argmax(-1, keepdim=True))[..., 0]
                else:
                    x0, conf = sample_with_prob(logits, temperature, top_k, top_p, uniforms=u_all[step])
                sel = select_transfer(cur, mask_id, k, x0, conf, remasking=remasking, threshold=threshold)
                if proposal == "logits":
                    out = logits.clone() if out is None else torch.where(sel[..., None], logits, out)
                elif proposal == "probs":
                    step_probs = sampling_probs(logits, temperature, top_k, top_p)
                    out = torch.where(sel[..., None], step_probs, torch.zeros_like(step_probs) if out is None else out)
                elif proposal == "sparse":
                    if out is None:
                        out = (torch.zeros_like(ids), torch.zeros_like(probs))
                    out = (torch.where(sel[..., None], ids, out[0]), torch.where(sel[..., None], probs, out[1]))
        if not dynamic:
            remaining -= min(k, remaining)
    return out, logits


def draft_block_step(drafter: Qwen3PagedModel, kv: PagedKV, seqs: List[Sequence], block: torch.Tensor,
                     denoising_steps: int, *, mask_id: int = MASK_ID, temperature: float = 0.0, top_k: int = 0,
                     top_p: float = 1.0, remasking: str = "low_confidence", threshold: Optional[float] = None,
                     confidence: str = "sampled", name: str = "draft", graphs: Optional[dict] = None,
                     width: Optional[int] = None, uniforms: Optional[torch.Tensor] = None,
                     generator: Optional[torch.Generator] = None, return_proposal: Optional[str] = None):
    """Denoise a block [B, Q] of B requests whose masked positions hold ``mask_id``.

    single/eval_sync.py:482-592 over a paged cache: each step runs the draft
    over the block at positions ``seqs[b].prefix``.. (the prefix and the
    whole block visible, store_kv=False: the block's K/V are rewritten each
    step), then unmasks the scheduled number of most confident masked
    positions; the last step fills every remaining mask.  Every request must
    hold the same number of masks (one schedule).

    T <= 1e-5: x0 is the argmax and the confidence per ``confidence`` (one
    fused kernel per step).  T > 1e-5: x0 is drawn from the top-k filtered
    softmax(logits / T) (dense) or from the top-``top_k`` support
    (``return_proposal="sparse"``) at ``uniforms`` [steps, B, Q]
    (torch.rand when omitted), and the confidence is the drawn token's
    probability (:560-576).

    ``return_proposal`` (T > 1e-5): ``"probs"`` returns the dense proposal
    [B, Q, V] the reference keeps as proposal_probs (:566-570, :577-584);
    ``"logits"`` the draft logits row of every position at the step it was
    unmasked, which the fused acceptance kernel consumes directly (q =
    softmax(row / T), top_k = 0 only); ``"sparse"`` (support ids [B, Q, S],
    support probs [B, Q, S]) (:585-589).

    With a ``graphs`` dict (greedy mode) each (forward + unmask) step is
    replayed from a HIP graph cached there per (B, Q, k, table width);
    ``width`` fixes the page-table width (default: the current longest table).
    """
    if return_proposal not in (None, "logits", "probs", "sparse"):
        raise ValueError("return_proposal must be None, 'logits', 'probs' or 'sparse'")
    if return_proposal == "logits" and ((top_k and top_k > 0) or (top_p is not None and top_p < 1.0)):
        raise ValueError("a logits proposal cannot carry the top-k / top-p filters: use 'probs' or 'sparse'")
    cur = block.clone().contiguous()
    num_masks = _mask_count(cur, mask_id)
    if num_masks == 0:
        return (cur, None) if return_proposal else cur
    schedule = get_num_transfer_tokens(num_masks, denoising_steps)
    stochastic = temperature > 1e-5
    proposal, _ = _denoise(drafter, kv, seqs, cur, schedule, mask_id=mask_id, temperature=temperature, top_k=top_k,
                           top_p=top_p, remasking=remasking, threshold=threshold, confidence=confidence, name=name,
                           graphs=graphs, width=width, uniforms=uniforms, generator=generator,
                           proposal=return_proposal if stochastic else None)
    if return_proposal:
        return cur, proposal
    return cur


# -- the reference's call surfaces --------------------------------------------
def _pos(start: int, end: int, device):
    return torch.arange(start, end, device=device).unsqueeze(0)


def _prefix_visibility(prefix_len: int, attention_mask_mode: str, block_size: int) -> torch.Tensor:
    """Absolute visibility [prefix_len, 3] of the prefix rows of
    _draft_attention_mask (single/eval_sync.py:208-239): block-causal rows
    see every prefix block up to their own; causal rows see keys <= row."""
    rows = []
    if attention_mask_mode == "block_causal":
        bs = max(1, int(block_size))
        for i in range(prefix_len):
            rows.append((min((i // bs + 1) * bs, prefix_len), 0, 0))
    elif attention_mask_mode == "causal":
        rows = [(i + 1, 0, 0) for i in range(prefix_len)]
    else:
        raise ValueError(f"unsupported attention_mask_mode={attention_mask_mode!r}")
    return torch.tensor(rows, dtype=torch.int32).reshape(prefix_len, 3)


def _draft_cache(drafter, past_key_values, prefix_len: int, batch: int):
    from .modeling_d3d import D3DForCausalLM, PagedCache
    if not isinstance(drafter, D3DForCausalLM):
        raise TypeError("drafter must be a d3d_amd.modeling_d3d.D3DForCausalLM")
    if past_key_values is not None:
        if not isinstance(past_key_values, PagedCache):
            raise TypeError("past_key_values must be a PagedCache of this drafter")
        if past_key_values.batch != batch:
            raise ValueError("block and past_key_values hold different batch sizes")
        if past_key_values.get_seq_length() != int(prefix_len):
            raise ValueError(f"past_key_values holds {past_key_values.get_seq_length()} tokens, "
                             f"prefix_len is {prefix_len}")
    return PagedCache


def d3d_draft_block(drafter, block, prefix_len: int, denoising_steps: int, remasking: str, threshold: float,
                    temperature: float, top_k: int, top_p: float, mask_id: int, prefix_ids=None,
                    past_key_values=None, attention_mask_mode: str = "block_causal", block_size: int = 32,
                    return_proposal_probs: bool = False, return_sparse_proposal: bool = False, *,
                    confidence: str = "sampled", uniforms: Optional[torch.Tensor] = None,
                    generator: Optional[torch.Generator] = None):
    """single/eval_sync.py:482-592 with the reference's parameters.

    ``drafter`` is a :class:`d3d_amd.modeling_d3d.D3DForCausalLM`.  The block
    [B, Q] attends to ``past_key_values`` (a PagedCache holding prefix_len
    tokens, store_kv=False), or to ``prefix_ids`` [B, P] under
    ``_draft_attention_mask`` (the prefix's K/V depend only on the prefix,
    which never sees the block in either mask mode, so they are computed
    once on a temporary cache rather than at every step), or to itself
    alone; positions start at prefix_len (P with prefix_ids, 0 alone).

    Returns ``cur``, or ``(cur, proposal_probs [B, Q, V])`` /
    ``(cur, (ids, probs))`` as the reference does (None proposal at T <=
    1e-5).  Extensions: ``confidence`` (see the module notes), ``uniforms``
    [steps, B, Q] and ``generator`` in place of torch.multinomial's stream.
    """
    PagedCache = _draft_cache(drafter, past_key_values, prefix_len, block.shape[0])
    dynamic, _ = _remasking(remasking, threshold)
    cur = block.to(drafter.device).clone().contiguous()
    B, Q = cur.shape
    num_masks = _mask_count(cur, mask_id)
    if num_masks == 0:
        if return_proposal_probs or return_sparse_proposal:
            return cur, None
        return cur
    temp = None
    if past_key_values is not None:
        cache = past_key_values
    else:
        temp = cache = drafter.new_cache(B)
        if prefix_ids is not None:
            pids = torch.as_tensor(prefix_ids, dtype=torch.int64, device=drafter.device)
            vis = _prefix_visibility(pids.shape[1], attention_mask_mode, block_size)
            drafter.forward_vis(pids, vis, None, cache, store_kv=True, logits_to_keep=1)
    try:
        stochastic = temperature > 1e-5
        proposal = None
        if stochastic:
            proposal = "sparse" if return_sparse_proposal else ("probs" if return_proposal_probs else None)
        schedule = get_num_transfer_tokens(num_masks, denoising_steps)
        out, _ = _denoise(drafter.model, drafter.kv, cache.seqs, cur, schedule, mask_id=mask_id,
                          temperature=temperature, top_k=top_k, top_p=top_p, remasking=remasking,
                          threshold=threshold, confidence=confidence, name=drafter.name, graphs=None, width=None,
                          uniforms=uniforms, generator=generator, proposal=proposal)
    finally:
        if temp is not None:
            temp.release()
        else:
            # The block's K/V were written past the stored prefix: drop them.
            cache.crop(cache.get_seq_length())
    if return_sparse_proposal:
        return cur, out
    if return_proposal_probs:
        return cur, out
    return cur


def d3d_draft_block_fused_commit(drafter, block, *, draft_kv, draft_kv_len: int, pending_commit, prefix_len: int,
                                 denoising_steps: int, remasking: str, threshold: float, temperature: float,
                                 top_k: int, top_p: float, mask_id: int, attention_mask_mode: str = "block_causal",
                                 return_metrics: bool = False, return_topk: int = 0,
                                 return_proposal_probs: bool = False, return_sparse_proposal: bool = False,
                                 confidence: str = "sampled", uniforms: Optional[torch.Tensor] = None,
                                 generator: Optional[torch.Generator] = None):
    """single/eval_sync.py:596-775 with the reference's parameters.

    ``draft_kv`` (a PagedCache holding draft_kv_len tokens) gains the
    ``pending_commit`` [B, n] tokens' K/V: the first denoise step runs one
    forward over [pending; block] at positions draft_kv_len.. under
    _fused_draft_mask (:251-275) with store_kv=True, then the cache is
    cropped to prefix_len = draft_kv_len + n; later steps are the plain
    block forward at prefix_len.. .  With ``return_topk`` > 0 (or
    ``return_metrics``) the last step's confidence is the max-softmax one
    (:708-717) and metrics hold ``top_tokens`` / ``top_logprobs`` [B, Q, k]
    of the last step's log_softmax (:763-768).  Return values as the
    reference's.
    """
    _draft_cache(drafter, draft_kv, draft_kv_len, block.shape[0])
    dynamic, _ = _remasking(remasking, threshold)
    if attention_mask_mode not in ("block_causal", "causal"):
        raise ValueError(f"unsupported attention_mask_mode={attention_mask_mode!r}")
    cur = block.to(drafter.device).clone().contiguous()
    B, Q = cur.shape
    dev = cur.device
    pending_len = int(pending_commit.shape[1]) if pending_commit is not None else 0
    if pending_len != int(prefix_len) - int(draft_kv_len):
        raise RuntimeError(
            f"draft pending length mismatch: pending={pending_len}, "
            f"prefix_len={prefix_len}, draft_kv_len={draft_kv_len}"
        )
    n = pending_len

    def commit_forward(ids_block: torch.Tensor) -> torch.Tensor:
        """[pending; block] at draft_kv_len..: the pending tokens' K/V stay in
        the cache (the stored length becomes prefix_len), the block's are
        scratch; returns the block rows' logits."""
        k0 = int(draft_kv_len)
        rows = [(k0 + (i + 1 if attention_mask_mode == "causal" else n), 0, 0) for i in range(n)]
        rows += [(k0 + n + Q, 0, 0)] * Q
        vis = torch.tensor(rows, dtype=torch.int32)
        ids = torch.cat([pending_commit.to(dev, torch.int64), ids_block], dim=1)
        out = drafter.forward_vis(ids, vis, None, draft_kv, store_kv=False, logits_to_keep=Q, past=k0)
        for s in draft_kv.seqs:
            s.prefix = int(prefix_len)
        return out.logits

    num_masks = _mask_count(cur, mask_id)
    metrics = {"top_tokens": None, "top_logprobs": None}
    want_metrics = return_metrics or int(return_topk) > 0
    out = None
    try:
        if num_masks == 0:
            if n:
                commit_forward(cur)
        else:
            stochastic = temperature > 1e-5
            proposal = None
            if stochastic:
                proposal = "sparse" if return_sparse_proposal else ("probs" if return_proposal_probs else None)
            schedule = get_num_transfer_tokens(num_masks, denoising_steps)
            # Every step's block sits at prefix_len..; the first one also
            # writes the pending tokens' K/V at draft_kv_len.. .
            for s in draft_kv.seqs:
                s.prefix = int(prefix_len)
            out, final = _denoise(drafter.model, drafter.kv, draft_kv.seqs, cur, schedule, mask_id=mask_id,
                                  temperature=temperature, top_k=top_k, top_p=top_p, remasking=remasking,
                                  threshold=threshold, confidence=confidence, name=drafter.name, graphs=None,
                                  width=None, uniforms=uniforms, generator=generator, proposal=proposal,
                                  first_forward=commit_forward if n else None, metrics_last=want_metrics)
            if int(return_topk) > 0 and final is not None:
                k = min(int(return_topk), final.shape[-1])
                ids, lp = topk_tokens(final, k, with_values=True, log_softmax=True)
                metrics = {"top_tokens": ids, "top_logprobs": lp}
    finally:
        # The block's scratch K/V past the committed prefix are dropped.
        draft_kv.crop(prefix_len)
    if want_metrics or return_proposal_probs or return_sparse_proposal:
        if return_sparse_proposal or return_proposal_probs:
            return cur, metrics, out
        return cur, metrics
    return cur
