"""Parity of the paged attention kernels and KV append with the oracle (GPU).

Tolerance (bf16 inputs and output, fp32 accumulation), against the fp64
oracle on the same bf16 inputs: max abs error <= 2e-2 and relative
Frobenius error <= 1e-2.  KV append is bit-exact.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from d3d_amd import attention as att
from d3d_amd import workloads
from oracle import attention as oa

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
REL = 1e-2


def _check(got, ref):
    got = got.float().cpu().numpy().astype(np.float64)
    err = np.abs(got - ref)
    rel = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert err.max() <= MAX_ABS, f"max abs err {err.max():.3e}"
    assert rel <= REL, f"relative err {rel:.3e}"
    return err.max(), rel


def _run(lens, Q, Hq, Hkv, ps, causal, seed=0, num_pages=None, max_seqlen_k=None):
    dev = torch.device("cuda:0")
    kv = workloads.paged_kv(seed, lens, Hkv=Hkv, D=128, page_size=ps, num_pages=num_pages, device="cpu")
    q = workloads.queries(seed + 7, len(lens), Q, Hq=Hq, D=128)
    out = att.flash_attn_with_kvcache(q.to(dev), kv.k_cache.to(dev), kv.v_cache.to(dev),
                                      kv.context_lens.to(dev), kv.block_table.to(dev), causal=causal,
                                      max_seqlen_k=max_seqlen_k)
    torch.cuda.synchronize()
    ref = oa.paged_attention(q.float().numpy(), kv.k_cache.float().numpy(), kv.v_cache.float().numpy(),
                             kv.block_table.numpy(), kv.context_lens.numpy(), 1.0 / math.sqrt(128),
                             causal=causal)
    return out, ref


def test_verify_block_qwen3_8b_prefix_2048():
    """Batch 1, 32/8 heads, d 128, K=16 causal block over a 2048-token prefix, 16-token pages."""
    out, ref = _run([2048 + 16], 16, 32, 8, 16, True, num_pages=256)
    _check(out, ref)


def test_verify_concurrent_batch8_shuffled_pages():
    lens = [c + 16 for c in workloads.concurrent_context_lens(2024, B=8)]
    out, ref = _run(lens, 16, 32, 8, 16, True, seed=3)
    _check(out, ref)


def test_verify_reference_page_size_256():
    out, ref = _run([1000 + 16, 300 + 16], 16, 32, 8, 256, True, seed=4)
    _check(out, ref)


def test_draft_block_bidirectional_qwen3_1p7b():
    """Batch 4, 16/8 heads, block of 16 seeing a 1024-token prefix and itself."""
    out, ref = _run([1024 + 16] * 4, 16, 16, 8, 16, False, seed=5)
    _check(out, ref)


@pytest.mark.parametrize(
    "lens,Q,Hq,Hkv,ps,causal",
    [
        ([77], 5, 32, 8, 16, True),      # ragged context, padded MFMA rows
        ([16], 16, 32, 8, 16, True),     # block alone, no prefix
        ([1], 1, 8, 1, 16, True),        # single key, single query, 8 query heads
        ([130, 64, 65], 1, 64, 8, 16, True),  # decode-shaped, 8 heads per group
        ([500], 16, 8, 8, 32, False),    # MHA group of 1
        ([9000], 16, 32, 8, 16, True),   # long context, many splits
    ],
)
def test_shapes_and_edges(lens, Q, Hq, Hkv, ps, causal):
    out, ref = _run(lens, Q, Hq, Hkv, ps, causal, seed=len(lens) + Q)
    _check(out, ref)


_RNG = np.random.default_rng(31)


# Split layouts at their edges: one long request (many splits), 32 requests
# with 4 query tiles each, 64 requests on 1-token pages (non-uniform page
# fetch, one page id per key), 24-token pages (1536-key split alignment) and
# more than 64 requests (fixed per-request split slots).
@pytest.mark.parametrize(
    "lens,Q,Hq,Hkv,ps",
    [
        ([20016], 16, 32, 8, 16),
        (list(_RNG.integers(1, 601, 32)), 64, 32, 8, 16),
        (list(_RNG.integers(2950, 3101, 64)), 1, 4, 1, 1),
        ([5016, 7016, 116], 16, 32, 8, 24),
        (list(_RNG.integers(1, 201, 70)), 1, 8, 1, 16),
    ],
    ids=["long-b1", "b32-four-query-tiles", "b64-one-token-pages", "pages-24", "b70"],
)
def test_split_layout_edges(lens, Q, Hq, Hkv, ps):
    lens = [int(x) for x in lens]
    out, ref = _run(lens, Q, Hq, Hkv, ps, True, seed=len(lens) + ps)
    _check(out, ref)


def test_tight_max_seqlen_k_matches_default_bound():
    lens = [700, 1300]
    a, ref = _run(lens, 16, 32, 8, 16, True, seed=9)
    b, _ = _run(lens, 16, 32, 8, 16, True, seed=9, max_seqlen_k=1300)
    _check(a, ref)
    _check(b, ref)


def test_page_ids_outside_pool_read_as_zero():
    dev = torch.device("cuda:0")
    kv = workloads.paged_kv(11, [64], Hkv=8, D=128, page_size=16)
    kv.block_table[0, 2] = kv.k_cache.shape[0] + 5  # outside the pool
    q = workloads.queries(12, 1, 16, Hq=32)
    out = att.flash_attn_with_kvcache(q.to(dev), kv.k_cache.to(dev), kv.v_cache.to(dev),
                                      kv.context_lens.to(dev), kv.block_table.to(dev))
    kc = kv.k_cache.float().numpy()
    vc = kv.v_cache.float().numpy()
    kc = np.concatenate([kc, np.zeros((6,) + kc.shape[1:])])
    vc = np.concatenate([vc, np.zeros((6,) + vc.shape[1:])])
    ref = oa.paged_attention(q.float().numpy(), kc, vc, kv.block_table.numpy(), [64], 1 / math.sqrt(128))
    _check(out, ref)


def test_kv_append_bit_exact_and_skips_negative_slots():
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(0)
    P, ps, Hkv, D = 40, 16, 8, 128
    kc = torch.randn(P, ps, Hkv, D, generator=g).to(torch.bfloat16).to(dev)
    vc = torch.randn(P, ps, Hkv, D, generator=g).to(torch.bfloat16).to(dev)
    n = 48
    slots = torch.randperm(P * ps, generator=g)[:n]
    slots[5] = -1
    k = torch.randn(n, Hkv, D, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(n, Hkv, D, generator=g).to(torch.bfloat16).to(dev)
    ek, ev = kc.clone(), vc.clone()
    keep = slots >= 0
    ek.view(-1, Hkv, D)[slots[keep].to(dev)] = k[keep.to(dev)]
    ev.view(-1, Hkv, D)[slots[keep].to(dev)] = v[keep.to(dev)]
    att.kv_append(k, v, kc, vc, slots.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(kc, ek) and torch.equal(vc, ev)


# -- query tiling and the packed multi-branch draft block -------------------
@pytest.mark.parametrize("lens,Q,Hq,causal", [([700, 129], 64, 32, True), ([300], 100, 16, False),
                                              ([2000 + 40], 40, 32, True)])
def test_query_tiling_beyond_128_rows(lens, Q, Hq, causal):
    """Blocks with (Hq/Hkv) * Q > 128 rows are tiled over workgroups."""
    out, ref = _run(lens, Q, Hq, 8, 16, causal, seed=21)
    _check(out, ref)


def _packed_specs(K: int, A: int):
    """Branch specs of Engine._predict (serving/engine.py:98-105): A anchors for
    each accepted count 1..K-1, then the all-accepted branch."""
    specs = [(n, 1000 + n * A + a) for n in range(1, K) for a in range(A)]
    return specs + [(K, None)]


@pytest.mark.parametrize("A,Hq,prefixes,ps", [(1, 16, [1024, 517, 33, 2048], 16), (3, 16, [200, 95], 16),
                                              (1, 32, [640, 1], 16), (1, 16, [300, 700], 256)])
def test_packed_block_matches_engine_mask(A, Hq, prefixes, ps):
    """Packed draft attention against the fp64 oracle under Engine._mask."""
    K = 16
    specs = _packed_specs(K, A)
    Q = K * (1 + len(specs))
    lens = [p + Q for p in prefixes]
    dev = torch.device("cuda:0")
    kv = workloads.paged_kv(31, lens, Hkv=8, D=128, page_size=ps, device="cpu")
    q = workloads.queries(37, len(lens), Q, Hq=Hq, D=128)
    vis = att.packed_visibility(K, [n for n, _ in specs])
    out = att.packed_block_attn(q.to(dev), kv.k_cache.to(dev), kv.v_cache.to(dev), kv.context_lens.to(dev),
                                kv.block_table.to(dev), vis.to(dev))
    torch.cuda.synchronize()
    masks = [oa.engine_mask(p, Q, p + Q, K, specs) for p in prefixes]
    ref = oa.paged_attention(q.float().numpy(), kv.k_cache.float().numpy(), kv.v_cache.float().numpy(),
                             kv.block_table.numpy(), kv.context_lens.numpy(), 1.0 / math.sqrt(128), masks=masks)
    _check(out, ref)


def test_packed_recovery_descriptor_equals_bidirectional_block():
    """A visibility of {Q, 0, 0} on every row is the recovery mask (d3d_draft_block_attn)."""
    dev = torch.device("cuda:0")
    lens = [1024 + 16, 77 + 16]
    kv = workloads.paged_kv(5, lens, Hkv=8, D=128, page_size=16, device="cpu")
    q = workloads.queries(6, 2, 16, Hq=16, D=128).to(dev)
    args = (kv.k_cache.to(dev), kv.v_cache.to(dev), kv.context_lens.to(dev), kv.block_table.to(dev))
    vis = torch.tensor([[16, 0, 0]] * 16, dtype=torch.int32, device=dev)
    a = att.packed_block_attn(q, *args, vis)
    b = att.draft_block_attn(q, *args)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
