"""Configurations 3 and 4 at their full sizes, by properties (GPU).

* Config 3, the diffusion-draft block step: the Qwen3-1.7B-shaped draft
  (28 layers, hidden 2048, 16/8 heads, MLP 6144, V 151,936, random bf16
  weights), batch 4, a 1024-token prefix, one block of 16 masks, 4
  iterations of top-4 by max-softmax confidence (single/eval_sync.py:482-592,
  the confidence of :713-717).  Every iteration unmasks exactly 4 positions
  per request; no mask is left; each unmasked token is that iteration's
  argmax; its confidence is at least every still-masked position's; and the
  batched, graph-replayed loop reproduces the iterations run one by one.
* Config 4, the engine: the Qwen3-8B-shaped target (36 layers, hidden 4096,
  32/8 heads, MLP 12288) and the config-3 draft on two streams, batch 4,
  512-token prompts, 32 new tokens: the output equals target-only greedy
  decoding on the same HIP target (generate_ar), up to a first divergence
  that must be a near tie: both diverging tokens' logits lie within a
  quarter of the logits' standard deviation of the maximum, recomputed on a
  third path
  (a prefill of the common prefix).  The block-verify, one-token and
  prefill paths round differently through 36 bf16 layers, and the top of
  151,936 random-model logits holds several candidates a few bf16 ulps
  apart (measured: the one-token path's pick 0.12 standard deviations, 5
  bf16 ulps, below the maximum); a logic error -- a wrong accepted count,
  anchor or K/V -- gives a token with an ordinary logit, about 4.5
  standard deviations below the maximum.  No page leaks (generate asserts
  it).
"""
from __future__ import annotations

import pytest
import torch

from d3d_amd import draft as dr
from d3d_amd.model import D3D_1P7B, QWEN3_8B, PagedKV, Qwen3PagedModel, Sequence, prefill

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def test_config3_draft_block_step_full_size():
    model = Qwen3PagedModel(D3D_1P7B, DEV, draft=True, seed=11)
    kv = PagedKV(D3D_1P7B, 512, 16, DEV)
    g = torch.Generator().manual_seed(5)
    prompts = torch.randint(0, 151936, (4, 1024), generator=g)
    seqs = [Sequence(i, p.tolist()) for i, p in enumerate(prompts)]
    prefill(model, kv, seqs, "draft")
    block = torch.full((4, 16), dr.MASK_ID, dtype=torch.int64, device=DEV)
    cur = block.clone()
    sched = dr.get_num_transfer_tokens(16, 4)
    assert sched == [4, 4, 4, 4]
    for step, k in enumerate(sched):
        before = cur.clone()
        logits = dr.draft_block_forward(model, kv, seqs, cur)
        x0, conf = dr.confidence_topk_unmask(logits, cur, dr.MASK_ID, k, confidence="max_softmax")
        lg = logits.float()
        top2 = lg.topk(2, -1).values
        decisive = (top2[..., 0] - top2[..., 1]) > 0
        assert torch.equal(x0[decisive], lg.argmax(-1)[decisive])
        for b in range(4):
            was = before[b] == dr.MASK_ID
            now = cur[b] == dr.MASK_ID
            picked = was & ~now
            assert int(picked.sum()) == 4, (step, b)
            assert torch.equal(cur[b][picked], x0[b][picked])
            assert torch.equal(cur[b][~picked], before[b][~picked])
            if now.any():
                assert float(conf[b][picked].min()) >= float(conf[b][now].max())
    assert not (cur == dr.MASK_ID).any()
    graphs = {}
    for _ in range(2):  # capture, then replay
        again = dr.draft_block_step(model, kv, seqs, block, 4, confidence="max_softmax", graphs=graphs)
        assert torch.equal(again, cur)
    del model, kv, graphs
    torch.cuda.empty_cache()


def test_config4_engine_full_size_is_lossless():
    from d3d_amd.engine import Engine, generate_ar
    eng = Engine(QWEN3_8B, D3D_1P7B, anchor_num=1, pages=32, seed=42)
    g = torch.Generator().manual_seed(9)
    prompts = torch.randint(0, 151936, (4, 512), generator=g).tolist()
    new = 32
    res = eng.generate(prompts, 4, max_new_tokens=new, ignore_eos=True)
    assert [len(o["tokens"]) for o in res["outputs"]] == [new] * 4
    assert res["steps"] >= 2 and res["overlap_fraction"] > 0.5
    ar = generate_ar(eng.target, prompts, 4, new, ignore_eos=True)
    for p, a, s in zip(prompts, (o["tokens"] for o in ar["outputs"]), (o["tokens"] for o in res["outputs"])):
        if a == s:
            continue
        i = next(j for j in range(new) if a[j] != s[j])
        seq = Sequence(99, p + a[:i])
        logits = eng.target.model.logits(prefill(eng.target.model, eng.target.kv, [seq], "probe"))[0].float()
        mx, sd = float(logits.max()), float(logits.std())
        gaps = [mx - float(logits[t]) for t in (a[i], s[i])]
        assert max(gaps) <= 0.25 * sd, f"divergence at position {i}: gaps {gaps} to the max, std {sd}"
        from d3d_amd.model import release
        release(eng.target.kv, seq, "probe")
    del eng
    torch.cuda.empty_cache()
