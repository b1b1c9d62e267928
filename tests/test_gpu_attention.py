"""Parity of the paged attention kernels and KV append with the oracle (GPU).

Tolerance (bf16 inputs and output, fp32 accumulation), against the fp64
oracle on the same bf16 inputs: max abs error <= 2e-2, max abs error <=
2e-2 of the output's own scale (max |ref|), and relative Frobenius error <=
1e-2.  The scale-relative bound matters: with q, k ~ N(0, 1/128) the softmax
is nearly uniform and every output is below 6e-3, so an absolute 2e-2 alone
would pass an all-zero output.  Peaked-score cases (score std >= 3, planted
dominant keys in the first and in the last split, a late maximum that
forces a rescale) exercise the running-max rescale, the split (m, l) merge
and the combine weighting.  KV append is bit-exact.
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


def _check(got, ref, absolute=True):
    """``absolute=False`` drops the absolute 2e-2 bound, which is meant for
    unit-scale activations, for outputs scaled far above it."""
    got = got.float().cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all(), "non-finite output"
    err = np.abs(got - ref)
    scale = max(np.abs(ref).max(), 1e-30)
    rel = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    if absolute:
        assert err.max() <= MAX_ABS, f"max abs err {err.max():.3e}"
    assert err.max() <= MAX_ABS * scale, f"max abs err {err.max():.3e} against output scale {scale:.3e}"
    assert rel <= REL, f"relative err {rel:.3e}"
    return err.max(), rel


def _run(lens, Q, Hq, Hkv, ps, causal, seed=0, num_pages=None, max_seqlen_k=None, edit=None):
    """Paged inputs for ``lens``; ``edit(q, kv)`` may rewrite q, kv.k_cache and
    kv.v_cache (CPU bf16 tensors) in place before the call."""
    dev = torch.device("cuda:0")
    kv = workloads.paged_kv(seed, lens, Hkv=Hkv, D=128, page_size=ps, num_pages=num_pages, device="cpu")
    q = workloads.queries(seed + 7, len(lens), Q, Hq=Hq, D=128)
    if edit is not None:
        edit(q, kv)
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
        ([3000], 16, 32, 8, 16, True),   # 24 two-tile splits: the 24-slot combine
        ([4000], 16, 32, 8, 16, True),   # 32 two-tile splits: the 32-slot combine
        ([1416] * 4, 16, 16, 8, 16, False),  # draft shape, 23 one-tile splits: 24 slots
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
                                              (1, 32, [640, 1], 16), (1, 16, [300, 700], 256),
                                              (1, 16, [900], 16), (3, 16, [1500], 16)])
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


@pytest.mark.parametrize("prefixes,ps", [([560, 1024, 33, 2048], 16), ([600, 5], 16), ([300, 700], 256)])
def test_packed_tile_skipping_is_exact(prefixes, ps):
    """A query tile skips the key tiles none of its rows sees.  Making one row
    in every 16 see every key forces those tiles in; every other row's output
    must not change by a single bit (a fully masked tile adds exactly
    nothing to a row's running max, sum and output)."""
    K = 16
    specs = _packed_specs(K, 1)
    Q = K * (1 + len(specs))
    lens = [p + Q for p in prefixes]
    dev = torch.device("cuda:0")
    kv = workloads.paged_kv(41, lens, Hkv=8, D=128, page_size=ps, device="cpu")
    q = workloads.queries(43, len(lens), Q, Hq=16, D=128).to(dev)
    args = (kv.k_cache.to(dev), kv.v_cache.to(dev), kv.context_lens.to(dev), kv.block_table.to(dev))
    vis = att.packed_visibility(K, [n for n, _ in specs])
    witness = vis.clone()
    rows = list(range(0, Q, 16))
    witness[rows] = torch.tensor([Q, 0, 0], dtype=torch.int32)
    a = att.packed_block_attn(q, *args, vis.to(dev))
    b = att.packed_block_attn(q, *args, witness.to(dev))
    torch.cuda.synchronize()
    keep = [i for i in range(Q) if i % 16]
    assert torch.equal(a[:, keep], b[:, keep])
    assert not torch.equal(a[:, rows], b[:, rows])  # the witnesses did see more


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


# -- peaked scores, planted keys, large and tiny values ---------------------
def _slot_of(kv, b, t):
    """(page, in-page slot) of request b's logical token t."""
    ps = kv.page_size
    return int(kv.block_table[b, t // ps]), t % ps


def _plant(q, kv, b, t, strength):
    """Make key t of request b dominant for every query of every KV head:
    its key is ``strength`` times the mean unit query direction of the head
    group, so each row's score at t exceeds the others by a wide margin."""
    B, Q, Hq, D = q.shape
    Hkv = kv.k_cache.shape[2]
    G = Hq // Hkv
    pg, sl = _slot_of(kv, b, t)
    qf = q[b].float()
    for h in range(Hkv):
        grp = qf[:, h * G:(h + 1) * G].reshape(-1, D)
        u = grp / grp.norm(dim=-1, keepdim=True)
        d = u.mean(0)
        kv.k_cache[pg, sl, h] = (strength * d / d.norm()).to(torch.bfloat16)


@pytest.mark.parametrize(
    "lens,Q,Hq,causal,plant",
    [
        ([2048 + 16], 16, 32, True, "first"),      # batch-1 verify shape, 17 splits
        ([2048 + 16], 16, 32, True, "last"),
        ([2048 + 16], 16, 32, True, "late-max"),  # moderate early peak, larger late one
        ([1024 + 16] * 4, 16, 16, False, "first"),  # batch-4 draft shape
        ([1024 + 16] * 4, 16, 16, False, "late-max"),
        ([6202, 873, 5365, 1619], 16, 32, True, "last"),  # batch-8-like mixed contexts
    ],
)
def test_peaked_scores(lens, Q, Hq, causal, plant):
    """q scaled by 40 (score std about 3.5) plus planted dominant keys."""
    def edit(q, kv):
        q.mul_(40.0)
        for b, ctx in enumerate(lens):
            last = ctx - Q - 1 if causal else ctx - 1  # visible to every query of the block
            if plant == "first":
                _plant(q, kv, b, 3, 60.0)
            elif plant == "last":
                _plant(q, kv, b, max(last, 0), 60.0)
            else:
                _plant(q, kv, b, 5, 25.0)
                _plant(q, kv, b, max(last, 0), 80.0)
    out, ref = _run(lens, Q, Hq, 8, 16, causal, seed=41, edit=edit)
    _check(out, ref)


@pytest.mark.parametrize("vscale", [2.0e5, 1.0e-6], ids=["large-v", "tiny-v"])
@pytest.mark.parametrize("lens,Q,Hq,causal", [([2048 + 16], 16, 32, True), ([1024 + 16] * 4, 16, 16, False),
                                              ([9000], 16, 32, True)])
def test_value_magnitudes(lens, Q, Hq, causal, vscale):
    """|V| far above fp16's 65504 and far below its normal range: the split
    partials are stored in fp16 with a per-row power-of-two scale.  Peaked
    scores (q x 40) make each split's O / l close to single values of V, so
    the large case exceeds 65504 in the partials."""
    def edit(q, kv):
        q.mul_(40.0)
        kv.v_cache.copy_((kv.v_cache.float() * (vscale * math.sqrt(128))).to(torch.bfloat16))
    out, ref = _run(lens, Q, Hq, 8, 16, causal, seed=43, edit=edit)
    _check(out, ref, absolute=False)


@pytest.mark.parametrize(
    "lens,Q,Hq,causal",
    [([3000], 16, 32, True), ([4000], 16, 32, True), ([4096], 16, 32, True),
     ([1400] * 4, 16, 16, False), ([1500, 1300, 1536, 1281], 16, 16, False)],
    ids=["b1-24-slots", "b1-32-slots", "b1-32-full", "b4-draft-22-slots", "b4-draft-mixed"],
)
def test_combine_slot_forms(lens, Q, Hq, causal):
    """Contexts whose split counts select the 24- and 32-slot combine forms,
    with peaked scores so the split weighting decides the output."""
    def edit(q, kv):
        q.mul_(30.0)
    out, ref = _run(lens, Q, Hq, 8, 16, causal, seed=47, edit=edit)
    _check(out, ref)
