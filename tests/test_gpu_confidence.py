"""Parity of the confidence / top-k unmask kernel with the oracle (GPU).

x0 (argmax) and the unmasked block are bit-exact; confidences agree with the
fp64 oracle to 1e-5 relative.  Cases whose k-th and (k+1)-th masked
confidences are closer than 1e-4 relative (order decided by rounding) are
excluded, and at least 80 % of requests must remain.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from d3d_amd import draft

pytestmark = pytest.mark.gpu
MASK = 151669


def _case(seed, B, Q, V, n_masked, scale=3.0):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(B, Q, V, generator=g) * scale
    block = torch.randint(0, min(V, MASK), (B, Q), generator=g)
    for b in range(B):
        idx = torch.randperm(Q, generator=g)[:n_masked]
        block[b, idx] = MASK
    return logits, block


def _certified(conf, block, k):
    keep = []
    for b in range(block.shape[0]):
        m = np.flatnonzero(block[b] == MASK)
        c = np.sort(conf[b][m])[::-1]
        kk = min(k, len(m))
        ok = kk == 0 or kk == len(m) or (c[kk - 1] - c[kk]) > 1e-4 * c[kk - 1]
        keep.append(ok)
    return np.array(keep)


@pytest.mark.parametrize("V", [1000, 4099, 151936])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("k,T", [(4, 0.0), (2, 0.7), (16, 0.0)])
def test_confidence_topk_vs_oracle(V, dtype, k, T):
    logits, block = _case(V + k, 4, 16, V, 12)
    dev = torch.device("cuda:0")
    lg = logits.to(dtype)
    blk = block.to(dev)
    x0, conf = draft.confidence_topk_unmask(lg.to(dev), blk, MASK, k, T)
    torch.cuda.synchronize()
    ref_blk, ref_x0, ref_conf = oracle.confidence_topk(lg.float().numpy(), block.numpy(), MASK, k, T)
    np.testing.assert_array_equal(x0.cpu().numpy(), ref_x0)
    np.testing.assert_allclose(conf.cpu().numpy(), ref_conf, rtol=1e-5)
    ok = _certified(ref_conf, block.numpy(), k)
    assert ok.mean() >= 0.8
    np.testing.assert_array_equal(blk.cpu().numpy()[ok], ref_blk[ok])


def test_denoise_schedule_fills_block_in_four_steps():
    """Config-3 shape of the schedule: 16 masks, 4 steps of top-4."""
    assert draft.get_num_transfer_tokens(16, 4) == [4, 4, 4, 4]
    dev = torch.device("cuda:0")
    logits, _ = _case(1, 4, 16, 5000, 0)
    blk = torch.full((4, 16), MASK, dtype=torch.int64, device=dev)
    for step in range(4):
        draft.confidence_topk_unmask(logits.to(dev), blk, MASK, 4)
        assert int((blk == MASK).sum()) == 4 * 4 * (3 - step)
    assert torch.equal(blk.cpu(), logits.argmax(-1))


def test_positions_without_masks_are_untouched():
    dev = torch.device("cuda:0")
    logits, block = _case(2, 3, 16, 777, 0)
    blk = block.to(dev)
    x0, _ = draft.confidence_topk_unmask(logits.to(dev), blk, MASK, 16)
    assert torch.equal(blk.cpu(), block)
    assert torch.equal(x0.cpu(), logits.argmax(-1))


@pytest.mark.parametrize("T", [0.0, 0.7])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_exact_ties_go_to_lower_id_and_position(T, dtype):
    """Equal maxima in a row give the lowest id as x0; positions with equal
    confidences are unmasked lowest position first.  Tied rows are
    identical, so their confidences are equal bit for bit."""
    V, Q = 4099, 16
    g = torch.Generator().manual_seed(41)
    logits = torch.randn(2, Q, V, generator=g)
    peaked = torch.randn(V, generator=g)
    peaked[[77, 5, 4098]] = 12.0
    for p in (9, 3, 12, 7):
        logits[0, p] = peaked
    logits[1, :] = peaked  # every position ties
    block = torch.full((2, Q), MASK, dtype=torch.int64)
    dev = torch.device("cuda:0")
    lg = logits.to(dtype)
    blk = block.to(dev)
    x0, conf = draft.confidence_topk_unmask(lg.to(dev), blk, MASK, 2, T)
    torch.cuda.synchronize()
    ref_blk, ref_x0, _ = oracle.confidence_topk(lg.float().numpy(), block.numpy(), MASK, 2, T)
    x0, blk, conf = x0.cpu().numpy(), blk.cpu().numpy(), conf.cpu().numpy()
    np.testing.assert_array_equal(x0, ref_x0)
    assert all(x0[0, p] == 5 for p in (3, 7, 9, 12)) and (x0[1] == 5).all()
    assert len({conf[0, p] for p in (3, 7, 9, 12)}) == 1 and len(set(conf[1])) == 1
    np.testing.assert_array_equal(blk, ref_blk)
    assert list(np.flatnonzero(blk[0] != MASK)) == [3, 7]
    assert list(np.flatnonzero(blk[1] != MASK)) == [0, 1]


@pytest.mark.parametrize("V", [1000, 151936])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_one_hot_confidence_takes_lowest_masked_positions(V, dtype):
    """The reference's greedy low_confidence step: every confidence is 1.0
    (single/eval_sync.py:287-291, :323-338), so the k lowest masked
    positions of each request take their argmax."""
    logits, block = _case(V + 5, 4, 16, V, 11)
    dev = torch.device("cuda:0")
    lg = logits.to(dtype)
    blk = block.to(dev)
    x0, conf = draft.confidence_topk_unmask(lg.to(dev), blk, MASK, 4, 0.0, confidence="sampled")
    torch.cuda.synchronize()
    ref_blk, ref_x0, ref_conf = oracle.confidence_topk(lg.float().numpy(), block.numpy(), MASK, 4, 0.0,
                                                       one_hot=True)
    assert (conf.cpu().numpy() == 1.0).all() and (ref_conf == 1.0).all()
    np.testing.assert_array_equal(x0.cpu().numpy(), ref_x0)
    np.testing.assert_array_equal(blk.cpu().numpy(), ref_blk)
    for b in range(4):
        masked = np.flatnonzero(block[b].numpy() == MASK)
        assert (blk.cpu().numpy()[b][masked[:4]] != MASK).all() and (blk.cpu().numpy()[b][masked[4:]] == MASK).all()


@pytest.mark.parametrize("threshold", [0.05, 0.3, 0.9, 2.0])
@pytest.mark.parametrize("confidence", ["max_softmax", "sampled"])
def test_dynamic_remasking_vs_oracle(threshold, confidence):
    """single/eval_sync.py:453-462: the masked positions whose confidence
    reaches the threshold (at most k), or the plain top-k when none does;
    requests are selected independently."""
    V = 4099
    g = torch.Generator().manual_seed(int(threshold * 100))
    logits = torch.randn(6, 16, V, generator=g) * torch.linspace(0.5, 9.0, 16)[None, :, None]
    block = torch.full((6, 16), MASK, dtype=torch.int64)
    block[:, ::5] = 3
    dev = torch.device("cuda:0")
    blk = block.to(dev)
    x0, conf = draft.confidence_topk_unmask(logits.to(dev), blk, MASK, 5, 0.0, confidence=confidence,
                                            remasking="low_confidence_dynamic", threshold=threshold)
    torch.cuda.synchronize()
    ref_blk, ref_x0, ref_conf = oracle.confidence_topk(logits.numpy(), block.numpy(), MASK, 5, 0.0,
                                                       one_hot=confidence == "sampled", dynamic=True,
                                                       threshold=threshold)
    np.testing.assert_array_equal(x0.cpu().numpy(), ref_x0)
    # rows whose confidences sit within rounding of the threshold or of each other are left out
    c = ref_conf
    near = (np.abs(c - threshold) < 1e-5 * np.maximum(c, 1e-30)).any(-1)
    if confidence == "sampled":
        ok = ~near  # every confidence is exactly 1.0: ties by position, nothing to certify
    else:
        ok = ~near & _certified(ref_conf, block.numpy(), 5)
    assert ok.mean() >= 0.5
    np.testing.assert_array_equal(blk.cpu().numpy()[ok], ref_blk[ok])


def test_select_transfer_dynamic_vs_oracle():
    g = torch.Generator().manual_seed(8)
    B, Q = 5, 24
    block = torch.where(torch.rand(B, Q, generator=g) < 0.7, MASK, 4)
    x0 = torch.randint(0, 100, (B, Q), generator=g)
    conf = torch.round(torch.rand(B, Q, generator=g) * 10) / 10  # many ties
    dev = torch.device("cuda:0")
    for thr in (0.0, 0.65, 0.95, 1.5):
        blk = block.clone().to(dev)
        sel = draft.select_transfer(blk, MASK, 6, x0.to(dev), conf.to(dev), remasking="dynamic", threshold=thr)
        ref_blk, ref_sel = oracle.select_transfer(block.numpy(), MASK, 6, x0.numpy(), conf.numpy(), dynamic=True,
                                                  threshold=thr)
        np.testing.assert_array_equal(blk.cpu().numpy(), ref_blk)
        np.testing.assert_array_equal(sel.cpu().numpy(), ref_sel)
