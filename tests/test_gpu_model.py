"""Paged model forwards and the denoise loop against the fp32 CPU restatement (GPU).

The models are bf16 with fp32 accumulation; logits are compared to the fp32
restatement with max abs error <= 5e-2 relative to the logit scale and
relative Frobenius error <= 3e-2.  Greedy tokens must agree wherever the
restatement's top-2 margin exceeds 5 % of its logit standard deviation.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from d3d_amd import draft as dr
from d3d_amd.model import ModelShape, PagedKV, Qwen3PagedModel, Sequence, block_inputs, prefill
from oracle import model_ref

pytestmark = pytest.mark.gpu

TINY = ModelShape(layers=2, hidden=256, heads=8, kv_heads=2, head_dim=128, mlp=512, vocab=1000)


def _close(got, ref):
    got = got.float().cpu()
    scale = ref.abs().max()
    rel = (got - ref).norm() / ref.norm()
    assert (got - ref).abs().max() <= 5e-2 * scale, float((got - ref).abs().max() / scale)
    assert rel <= 3e-2, float(rel)


def _greedy_agree(got, ref):
    """Greedy tokens agree wherever the top-2 margin exceeds 5 % of the logit spread."""
    top2 = ref.topk(2, -1).values
    sure = (top2[..., 0] - top2[..., 1]) > 0.05 * ref.std(-1)
    assert sure.float().mean() >= 0.5
    assert torch.equal(got.float().cpu().argmax(-1)[sure], ref.argmax(-1)[sure])


@pytest.mark.parametrize("draft_mode", [False, True])
def test_prefill_then_block_matches_restatement(draft_mode):
    dev = torch.device("cuda:0")
    model = Qwen3PagedModel(TINY, dev, draft=draft_mode, seed=3, init_std=0.05)
    model.lm_head.mul_(20.0)  # decisive logits: top-2 margins far above rounding
    kv = PagedKV(TINY, 64, 16, dev)
    g = torch.Generator().manual_seed(0)
    prompts = torch.randint(0, TINY.vocab, (2, 48), generator=g)
    seqs = [Sequence(i, p.tolist()) for i, p in enumerate(prompts)]
    prefill(model, kv, seqs, "m")
    blk = torch.randint(0, TINY.vocab, (2, 16), generator=g)
    from d3d_amd.model import reserve
    for s in seqs:
        reserve(kv, s, "m", s.prefix + 16)
    tables, slots, lens, logical, mx = block_inputs(kv, seqs, "m", [s.prefix for s in seqs], 16, dev)
    hid = model(blk.to(dev), logical, kv, tables, lens, slots, causal=not draft_mode, max_context=mx)
    got = model.logits(hid)
    W = model_ref.weights_fp32(model)
    for b in range(2):
        ids = torch.cat([prompts[b], blk[b]])
        mask = model_ref.causal_then_block(48, 16, bidirectional=draft_mode)
        ref = model_ref.forward(W, TINY, ids, torch.arange(64), mask)[48:]
        _close(got[b], ref)
        _greedy_agree(got[b], ref)


def test_denoise_loop_matches_restatement():
    """Four greedy denoise steps over a 16-mask block after a 32-token prefix.

    Each step's logits are checked against the restatement given the same
    block state, and its confidences, greedy tokens and unmasked set against
    the softmax of those logits (where the k-th and (k+1)-th masked
    confidences differ by more than 1e-4).
    The loop itself must reproduce the step-by-step result bit for bit.
    """
    dev = torch.device("cuda:0")
    model = Qwen3PagedModel(TINY, dev, draft=True, seed=5, init_std=0.05)
    model.lm_head.mul_(20.0)
    kv = PagedKV(TINY, 64, 16, dev)
    g = torch.Generator().manual_seed(1)
    prompts = torch.randint(0, TINY.vocab - 1, (2, 32), generator=g)
    seqs = [Sequence(i, p.tolist()) for i, p in enumerate(prompts)]
    prefill(model, kv, seqs, "draft")
    mask_id = TINY.vocab - 1
    W = model_ref.weights_fp32(model)
    cur = torch.full((2, 16), mask_id, dtype=torch.int64, device=dev)
    checked = 0
    for step, k in enumerate(dr.get_num_transfer_tokens(16, 4)):
        before = cur.cpu().clone()
        logits = dr.draft_block_forward(model, kv, seqs, cur, "draft")
        k = 16 if step == 3 else k
        x0, conf = dr.confidence_topk_unmask(logits, cur, mask_id, k)
        x0, conf, after = x0.cpu(), conf.cpu(), cur.cpu()
        for b in range(2):
            # The forward: logits against the restatement on the same block state.
            ids = torch.cat([prompts[b], before[b]])
            ref = model_ref.forward(W, TINY, ids, torch.arange(48), model_ref.causal_then_block(32, 16, True))[32:]
            _close(logits[b], ref)
            _greedy_agree(logits[b], ref)
            # The unmask: confidence and selection from these logits.
            p = torch.softmax(logits[b].float().cpu(), -1)
            rx0, rconf = p.argmax(-1), p.max(-1).values
            assert torch.equal(x0[b], rx0)
            np.testing.assert_allclose(conf[b].numpy(), rconf.numpy(), rtol=1e-5)
            masked = torch.nonzero(before[b] == mask_id)[:, 0].tolist()
            order = sorted(masked, key=lambda i: (-float(rconf[i]), i))
            kk = min(k, len(order))
            gap_ok = kk == len(order) or float(rconf[order[kk - 1]] - rconf[order[kk]]) > 1e-4
            if gap_ok:
                chosen = sorted(i for i in masked if after[b, i] != mask_id)
                assert chosen == sorted(order[:kk])
                checked += 1
    assert checked >= 4
    # The loop gives the same block as the steps above.
    again = dr.draft_block_step(model, kv, seqs, torch.full((2, 16), mask_id, dtype=torch.int64, device=dev), 4,
                                mask_id=mask_id, confidence="max_softmax")
    assert torch.equal(again, cur)


@pytest.mark.parametrize("confidence", ["max_softmax", "sampled"])
def test_denoise_graph_replay_matches_eager(confidence):
    dev = torch.device("cuda:0")
    model = Qwen3PagedModel(TINY, dev, draft=True, seed=9, init_std=0.05)
    model.lm_head.mul_(20.0)
    kv = PagedKV(TINY, 64, 16, dev)
    g = torch.Generator().manual_seed(2)
    seqs = [Sequence(i, torch.randint(0, TINY.vocab - 1, (32,), generator=g).tolist()) for i in range(2)]
    prefill(model, kv, seqs, "draft")
    mask_id = TINY.vocab - 1
    block = torch.full((2, 16), mask_id, dtype=torch.int64, device=dev)
    eager = dr.draft_block_step(model, kv, seqs, block, 4, mask_id=mask_id, confidence=confidence)
    graphs = {}
    for _ in range(3):  # capture, then replays with eager work in between
        got = dr.draft_block_step(model, kv, seqs, block, 4, mask_id=mask_id, confidence=confidence, graphs=graphs)
        torch.cuda.synchronize()
        assert torch.equal(got, eager)
        assert torch.equal(dr.draft_block_step(model, kv, seqs, block, 4, mask_id=mask_id, confidence=confidence),
                           eager)


@pytest.mark.parametrize("mode", ["block_causal", "causal"])
def test_fused_commit_matches_restatement(mode):
    """single/eval_sync.py:596-775 called with the reference's parameters:
    pending tokens committed to the draft cache in the same forward as the
    anchor block (mask of :251-275), top-2 log-probabilities of the last
    step, then a later block that reads the committed K/V."""
    from d3d_amd.modeling_d3d import D3DForCausalLM
    dev = torch.device("cuda:0")
    model = Qwen3PagedModel(TINY, dev, draft=True, seed=13, init_std=0.05)
    drafter = D3DForCausalLM(TINY, dev, pages=64, model=model)
    model.lm_head.mul_(20.0)
    g = torch.Generator().manual_seed(6)
    mask_id = TINY.vocab - 1
    prompts = torch.randint(0, mask_id, (2, 32), generator=g)
    pending = torch.randint(0, mask_id, (2, 5), generator=g)
    cache = drafter.new_cache(2)
    drafter.prefill(cache, prompts.to(dev))
    assert cache.get_seq_length() == 32
    block = torch.full((2, 16), mask_id, dtype=torch.int64)
    block[:, 0] = torch.tensor([3, 4])
    cur, metrics = dr.d3d_draft_block_fused_commit(
        drafter, block.to(dev), draft_kv=cache, draft_kv_len=32, pending_commit=pending.to(dev), prefix_len=37,
        denoising_steps=1, remasking="low_confidence", threshold=0.9, temperature=0.0, top_k=0, top_p=1.0,
        mask_id=mask_id, attention_mask_mode=mode, return_topk=2)
    assert cache.get_seq_length() == 37
    W = model_ref.weights_fp32(model)
    T = 32 + 5 + 16
    for b in range(2):
        ids = torch.cat([prompts[b], pending[b], block[b]])
        mask = torch.ones(T, T).tril().bool()
        if mode == "block_causal":
            mask[32:37, :37] = True  # pending rows see every pending token
        mask[37:, :] = True  # block rows see everything
        ref = model_ref.forward(W, TINY, ids, torch.arange(T), mask)[37:]
        lp = torch.log_softmax(ref, -1)
        top2 = ref.topk(3, -1)
        sure = (top2.values[:, 1] - top2.values[:, 2]) > 0.05 * ref.std(-1)
        sure &= (top2.values[:, 0] - top2.values[:, 1]) > 0.05 * ref.std(-1)
        assert sure.float().mean() >= 0.25  # both top-2 gaps decisive
        got_ids = metrics["top_tokens"][b].cpu()
        assert torch.equal(got_ids[sure], top2.indices[sure, :2])
        got_lp = metrics["top_logprobs"][b].cpu()
        ref_lp = lp.gather(-1, got_ids)
        assert float((got_lp - ref_lp).abs().max()) <= 5e-2 * float(ref.abs().max())
        # one step: every mask takes the greedy token, the anchor stays
        assert cur[b, 0].item() == block[b, 0].item()
        assert torch.equal(cur[b, 1:].cpu()[sure[1:]], ref.argmax(-1)[1:][sure[1:]])
    # A later block reads the committed pending K/V (the draft model's call
    # surface, store_kv=False, with the reference's _full_mask).
    nxt = torch.randint(0, mask_id, (2, 16), generator=g)
    out = drafter(nxt.to(dev), attention_mask=torch.ones(1, 1, 16, 37 + 16, dtype=torch.bool, device=dev),
                  position_ids=torch.arange(37, 53, device=dev)[None], past_key_values=cache, use_cache=True,
                  store_kv=False, logits_to_keep=16)
    assert cache.get_seq_length() == 37
    for b in range(2):
        ids = torch.cat([prompts[b], pending[b], nxt[b]])
        mask = torch.ones(T, T).tril().bool()
        if mode == "block_causal":
            mask[32:37, :37] = True
        mask[37:, :] = True
        ref = model_ref.forward(W, TINY, ids, torch.arange(T), mask)[37:]
        _close(out.logits[b], ref)
    cache.release()
    assert len(drafter.kv.pool.free) == drafter.kv.num_pages
