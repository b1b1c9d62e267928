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
