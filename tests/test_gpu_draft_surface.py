"""The draft-side call surfaces, called as the reference calls them (GPU).

* d3d_draft_block(drafter, block, prefix_len, denoising_steps, remasking,
  threshold, temperature, top_k, top_p, mask_id, prefix_ids=None,
  past_key_values=None, ...) -- single/eval_sync.py:482-592;
* d3d_draft_block_fused_commit(drafter, block, *, draft_kv, draft_kv_len,
  pending_commit, prefix_len, ...) -- :596-775;
* D3DForCausalLM(input_ids, attention_mask, position_ids, past_key_values,
  use_cache, store_kv, logits_to_keep) -- models/d3d/modeling_d3d.py:855-934.

Each loop is checked against the same loop written out step by step the
way the reference writes it: the drafter called with the reference's masks
(_full_mask, _draft_attention_mask, _fused_draft_mask, restated below from
single/eval_sync.py:194-275), greedy tokens, and the selection of the
reference's greedy steps (confidence 1.0 for every position, so the lowest
masked positions are unmasked first).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from d3d_amd import draft as dr
from d3d_amd import speculative_sampling as ss
from d3d_amd.model import ModelShape
from d3d_amd.modeling_d3d import D3DForCausalLM, mask_to_visibility
from oracle import model_ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TINY = ModelShape(layers=2, hidden=256, heads=8, kv_heads=2, head_dim=128, mlp=512, vocab=1000)
MASK = TINY.vocab - 1


# -- the reference's mask helpers (single/eval_sync.py:194-275) ---------------
def _pos(start, end):
    return torch.arange(start, end, device=DEV).unsqueeze(0)


def _full_mask(q, kv):
    return torch.ones((1, 1, q, kv), dtype=torch.bool, device=DEV)


def _causal_mask(q, kv, query_start=0):
    qp = torch.arange(query_start, query_start + q, device=DEV)
    kp = torch.arange(kv, device=DEV)
    return (kp.unsqueeze(0) <= qp.unsqueeze(1)).unsqueeze(0).unsqueeze(0)


def _draft_attention_mask(prefix_len, block_len, mode, block_size):
    total = prefix_len + block_len
    if mode == "block_causal":
        ids = torch.zeros(total, dtype=torch.int32, device=DEV)
        nb = (prefix_len + block_size - 1) // block_size
        for i in range(nb):
            ids[i * block_size:min((i + 1) * block_size, prefix_len)] = i
        ids[prefix_len:] = nb
        return (ids[:, None] >= ids[None, :]).unsqueeze(0).unsqueeze(0)
    mask = torch.zeros((1, 1, total, total), dtype=torch.bool, device=DEV)
    if prefix_len > 0:
        mask[:, :, :prefix_len, :prefix_len] = _causal_mask(prefix_len, prefix_len)
    mask[:, :, prefix_len:, :] = True
    return mask


def _fused_draft_mask(pending_len, block_len, past_len, mode):
    q = pending_len + block_len
    kv = past_len + q
    mask = torch.ones((1, 1, q, kv), dtype=torch.bool, device=DEV)
    if mode == "causal":
        if pending_len > 0:
            mask[:, :, :pending_len, :] = _causal_mask(pending_len, kv, query_start=past_len)
        return mask
    if pending_len > 0 and block_len > 0:
        mask[:, :, :pending_len, past_len + pending_len:] = False
    return mask


def _select_lowest(cur, x0, k):
    """The reference's greedy selection: every confidence 1.0, the lowest
    k masked positions of each request take x0."""
    for b in range(cur.shape[0]):
        masked = torch.nonzero(cur[b] == MASK)[:, 0].tolist()[:k]
        cur[b, masked] = x0[b, masked]


def _drafter(seed):
    d = D3DForCausalLM(TINY, DEV, pages=96, seed=seed)
    d.model.lm_head.mul_(20.0)  # decisive logits
    return d


def test_d3d_draft_block_with_cache_reference_call():
    drafter = _drafter(21)
    g = torch.Generator().manual_seed(0)
    prefix = torch.randint(0, MASK, (1, 40), generator=g).to(DEV)
    block = torch.full((1, 16), MASK, dtype=torch.int64, device=DEV)
    block[0, 0] = 7
    cache = drafter.new_cache(1)
    drafter.prefill(cache, prefix)
    free_before = len(drafter.kv.pool.free)
    # positional, as single/eval_sync.py's callers pass them
    got = dr.d3d_draft_block(drafter, block, 40, 4, "low_confidence", 0.9, 0.0, 0, 1.0, MASK,
                             past_key_values=cache)
    assert cache.get_seq_length() == 40 and len(drafter.kv.pool.free) == free_before
    cur = block.clone()
    sched = dr.get_num_transfer_tokens(15, 4)
    for step, k in enumerate(sched):
        logits = drafter(cur, attention_mask=_full_mask(16, 56), position_ids=_pos(40, 56), past_key_values=cache,
                         use_cache=True, store_kv=False, logits_to_keep=16).logits
        if step == len(sched) - 1:
            k = int((cur == MASK).sum())
        _select_lowest(cur, logits.argmax(-1), k)
    assert torch.equal(got, cur) and not (got == MASK).any()
    cache.release()


@pytest.mark.parametrize("mode,bs", [("block_causal", 8), ("causal", 32)])
def test_d3d_draft_block_prefix_ids(mode, bs):
    """prefix_ids path, one denoising step, against the drafter called over
    [prefix; block] with _draft_attention_mask and against the fp32
    restatement, on positions whose top-2 margin is decisive."""
    drafter = _drafter(22)
    g = torch.Generator().manual_seed(1)
    P = 37
    prefix = torch.randint(0, MASK, (1, P), generator=g).to(DEV)
    block = torch.full((1, 16), MASK, dtype=torch.int64, device=DEV)
    block[0, 0] = 11
    got = dr.d3d_draft_block(drafter, block, P, 1, "low_confidence", 0.9, 0.0, 0, 1.0, MASK, prefix_ids=prefix,
                             attention_mask_mode=mode, block_size=bs)
    assert len(drafter.kv.pool.free) == drafter.kv.num_pages
    ids = torch.cat([prefix, block], 1)
    logits = drafter(ids, attention_mask=_draft_attention_mask(P, 16, mode, bs), position_ids=_pos(0, P + 16),
                     use_cache=False, logits_to_keep=16).logits[0]
    W = model_ref.weights_fp32(drafter.model)
    ref = model_ref.forward(W, TINY, ids[0].cpu(), torch.arange(P + 16),
                            _draft_attention_mask(P, 16, mode, bs)[0, 0].cpu())[P:]
    top2 = ref.topk(2, -1).values
    sure = (top2[:, 0] - top2[:, 1]) > 0.05 * ref.std(-1)
    sure[0] = False  # the anchor stays
    assert sure.sum() >= 6
    assert torch.equal(got[0].cpu()[sure], logits.argmax(-1).cpu()[sure])
    assert torch.equal(got[0].cpu()[sure], ref.argmax(-1)[sure])
    assert got[0, 0].item() == 11


def test_d3d_draft_block_alone():
    """Neither prefix nor cache: the block attends to itself at positions 0.."""
    drafter = _drafter(23)
    block = torch.full((2, 16), MASK, dtype=torch.int64, device=DEV)
    block[:, 0] = torch.tensor([3, 9], device=DEV)
    got = dr.d3d_draft_block(drafter, block, 0, 2, "low_confidence", 0.9, 0.0, 0, 1.0, MASK)
    cur = block.clone()
    for step, k in enumerate(dr.get_num_transfer_tokens(15, 2)):
        logits = drafter(cur, attention_mask=_full_mask(16, 16), position_ids=_pos(0, 16), use_cache=False,
                         logits_to_keep=16).logits
        _select_lowest(cur, logits.argmax(-1), 16 if step == 1 else k)
    assert torch.equal(got, cur)
    assert len(drafter.kv.pool.free) == drafter.kv.num_pages


@pytest.mark.parametrize("mode", ["block_causal", "causal"])
def test_fused_commit_batch2_four_steps(mode):
    """B = 2, denoising_steps = 4: each request keeps its own 15-mask
    schedule [4, 4, 4, 3] (not a schedule over the whole batch), against the
    loop of single/eval_sync.py:596-775 written out with the drafter."""
    drafter = _drafter(24)
    g = torch.Generator().manual_seed(2)
    prompts = torch.randint(0, MASK, (2, 32), generator=g).to(DEV)
    pending = torch.randint(0, MASK, (2, 5), generator=g).to(DEV)
    block = torch.full((2, 16), MASK, dtype=torch.int64, device=DEV)
    block[:, 0] = torch.tensor([5, 6], device=DEV)
    caches = []
    for _ in range(2):
        c = drafter.new_cache(2)
        drafter.prefill(c, prompts)
        caches.append(c)
    got = dr.d3d_draft_block_fused_commit(
        drafter, block, draft_kv=caches[0], draft_kv_len=32, pending_commit=pending, prefix_len=37,
        denoising_steps=4, remasking="low_confidence", threshold=0.9, temperature=0.0, top_k=0, top_p=1.0,
        mask_id=MASK, attention_mask_mode=mode)
    cache = caches[1]
    cur = block.clone()
    sched = dr.get_num_transfer_tokens(15, 4)
    assert sched == [4, 4, 4, 3]
    counts = []
    for step, k in enumerate(sched):
        if step == 0:
            logits = drafter(torch.cat([pending, cur], 1), attention_mask=_fused_draft_mask(5, 16, 32, mode),
                             position_ids=_pos(32, 53), past_key_values=cache, use_cache=True, store_kv=True,
                             logits_to_keep=16).logits
            cache.crop(37)
        else:
            logits = drafter(cur, attention_mask=_full_mask(16, 53), position_ids=_pos(37, 53), past_key_values=cache,
                             use_cache=True, store_kv=False, logits_to_keep=16).logits
        if step == len(sched) - 1:
            k = 16
        _select_lowest(cur, logits.argmax(-1), k)
        counts.append(int((cur[0] == MASK).sum()))
    assert counts == [11, 7, 3, 0]
    assert torch.equal(got, cur)
    assert caches[0].get_seq_length() == 37
    for c in caches:
        c.release()
    assert len(drafter.kv.pool.free) == drafter.kv.num_pages


def test_fused_commit_length_mismatch_raises():
    drafter = _drafter(25)
    cache = drafter.new_cache(1)
    block = torch.full((1, 16), MASK, dtype=torch.int64, device=DEV)
    with pytest.raises(RuntimeError, match="draft pending length mismatch"):
        dr.d3d_draft_block_fused_commit(drafter, block, draft_kv=cache, draft_kv_len=0,
                                        pending_commit=torch.zeros(1, 3, dtype=torch.int64, device=DEV),
                                        prefix_len=5, denoising_steps=1, remasking="low_confidence",
                                        threshold=0.9, temperature=0.0, top_k=0, top_p=1.0, mask_id=MASK)


def test_unsupported_parameters_raise():
    drafter = _drafter(26)
    block = torch.full((1, 16), MASK, dtype=torch.int64, device=DEV)
    with pytest.raises(ValueError):
        dr.d3d_draft_block(drafter, block, 0, 2, "random", 0.9, 1.0, 0, 1.0, MASK, return_proposal_probs=True)


@pytest.mark.parametrize("top_k,top_p", [(0, 0.9), (100, 1.0), (100, 0.8)])
def test_filtered_proposals_through_the_block_step(top_k, top_p):
    """top-p and top-k above 64 (single/eval_sync.py:292-303) through the
    reference's d3d_draft_block call: every position is unmasked, each
    proposal row is a distribution, the drawn token carries probability
    under it, and the filters cut the support (top_k: at least k entries, more
    with ties; top_p: fewer than the whole vocabulary)."""
    drafter = _drafter(27)
    block = torch.full((1, 16), MASK, dtype=torch.int64, device=DEV)
    torch.manual_seed(3)
    out, probs = dr.d3d_draft_block(drafter, block, 0, 2, "low_confidence", 0.9, 1.0, top_k, top_p, MASK,
                                    return_proposal_probs=True)
    assert not bool((out == MASK).any())
    p = probs[0].float()
    np.testing.assert_allclose(p.sum(-1).cpu().numpy(), 1.0, rtol=1e-4)
    picked = p.gather(-1, out[0][:, None])[:, 0]
    assert bool((picked > 0).all())
    support = (p > 0).sum(-1)
    if top_k and top_p >= 1.0:
        assert int(support.min()) >= top_k  # ties with the k-th value only add entries
    assert int(support.max()) < p.shape[-1]


def test_dynamic_remasking_one_hot_equals_low_confidence():
    """At T = 0 every confidence is 1.0 >= threshold, so "dynamic" takes the
    scheduled k like low_confidence (single/eval_sync.py:453-462)."""
    drafter = _drafter(27)
    g = torch.Generator().manual_seed(3)
    prefix = torch.randint(0, MASK, (1, 20), generator=g).to(DEV)
    block = torch.full((1, 16), MASK, dtype=torch.int64, device=DEV)
    cache = drafter.new_cache(1)
    drafter.prefill(cache, prefix)
    a = dr.d3d_draft_block(drafter, block, 20, 4, "low_confidence", 0.9, 0.0, 0, 1.0, MASK, past_key_values=cache)
    b = dr.d3d_draft_block(drafter, block, 20, 4, "low_confidence_dynamic", 0.9, 0.0, 0, 1.0, MASK,
                           past_key_values=cache)
    assert torch.equal(a, b)
    cache.release()


def test_sampled_dense_proposal_top_k_feeds_verification():
    """T = 1 with top_k = 8 and return_proposal_probs: each position's
    proposal row is the top-8 filtered softmax of the step that unmasked
    it, the drawn token lies in its support, and the rows feed
    verify_speculative_block."""
    drafter = _drafter(28)
    g = torch.Generator().manual_seed(4)
    prefix = torch.randint(0, MASK, (1, 24), generator=g).to(DEV)
    block = torch.full((1, 16), MASK, dtype=torch.int64, device=DEV)
    block[0, 0] = 17
    cache = drafter.new_cache(1)
    drafter.prefill(cache, prefix)
    u = torch.rand(2, 1, 16, generator=g).to(DEV)
    cur, probs = dr.d3d_draft_block(drafter, block, 24, 2, "low_confidence", 0.9, 1.0, 8, 1.0, MASK,
                                    past_key_values=cache, return_proposal_probs=True, uniforms=u)
    assert probs.shape == (1, 16, TINY.vocab)
    rows = probs[0, 1:]
    np.testing.assert_allclose(rows.sum(-1).cpu().numpy(), 1.0, rtol=1e-5)
    assert ((rows > 0).sum(-1) >= 8).all()  # ties with the 8th value are kept
    drawn = cur[0, 1:]
    assert (rows.gather(-1, drawn[:, None]) > 0).all()
    assert probs[0, 0].abs().sum() == 0  # the anchor is never unmasked
    target = torch.softmax(torch.randn(1, 16, TINY.vocab, generator=g), -1).to(DEV)
    res = ss.verify_speculative_block(drawn[None], target, rows[None].contiguous(),
                                      uniforms=torch.rand(1, 15, generator=g).to(DEV),
                                      resample_uniform=torch.rand(1, generator=g).to(DEV))
    assert 0 <= res.accepted_draft_tokens <= 15
    cache.release()


def test_sparse_proposal_top_p_matches_oracle():
    """T = 0.8, top_k = 16, top_p = 0.7 through the sparse path: the support
    probabilities equal the oracle's nucleus-filtered softmax of the same
    logits."""
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(6, 5000, generator=g) * 2).float()
    u = torch.rand(6, generator=g)
    tok, ids, probs = dr.sample_with_sparse_probs(x.to(DEV), 0.8, 16, 0.7, uniforms=u.to(DEV))
    rt, rids, rprobs, margin = oracle.sample_sparse(x.numpy(), 0.8, 16, u.numpy(), top_p=0.7)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    np.testing.assert_allclose(probs.cpu().numpy(), rprobs, rtol=2e-5, atol=1e-7)
    ok = margin > 1e-6
    np.testing.assert_array_equal(tok.cpu().numpy()[ok], rt[ok])


def test_forward_store_kv_and_masks():
    """store_kv=True advances the cache; False leaves it; a mask that is not
    a prefix plus one range raises."""
    drafter = _drafter(29)
    cache = drafter.new_cache(1)
    ids = torch.arange(10, device=DEV)[None]
    drafter(ids, attention_mask=_causal_mask(10, 10), past_key_values=cache, use_cache=True, store_kv=True)
    assert cache.get_seq_length() == 10
    drafter(ids[:, :4], attention_mask=_full_mask(4, 14), past_key_values=cache, use_cache=True, store_kv=False)
    assert cache.get_seq_length() == 10
    bad = torch.zeros(1, 1, 4, 14, dtype=torch.bool, device=DEV)
    bad[..., 0] = bad[..., 3] = bad[..., 7] = True
    with pytest.raises(ValueError):
        drafter(ids[:, :4], attention_mask=bad, past_key_values=cache, use_cache=True, store_kv=False)
    # additive float masks: 0 visible, large negative hidden
    fm = torch.where(_full_mask(4, 14), 0.0, torch.finfo(torch.float32).min)
    a = drafter(ids[:, :4], attention_mask=fm, past_key_values=cache, store_kv=False).logits
    b = drafter(ids[:, :4], attention_mask=_full_mask(4, 14), past_key_values=cache, store_kv=False).logits
    assert torch.equal(a, b)
    assert mask_to_visibility(_full_mask(4, 14), 4, 14).tolist() == [[14, 14, 14]] * 4
    cache.release()
