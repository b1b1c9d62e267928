"""Pins the paged-attention oracle (CPU only).

The reference's attention is flash-attn (CUDA only, not importable here), so
the oracle is pinned against torch's scaled_dot_product_attention on the CPU
-- the library routine the reference's draft branch calls -- with the
reference's masks and GQA expansion, plus closed forms and a page-table
gather check.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oa


def _contiguous_problem(seed, B, Q, Hq, Hkv, D, lens, ps):
    rng = np.random.default_rng(seed)
    pages = [int(np.ceil(c / ps)) for c in lens]
    P = sum(pages) + 3
    kc = rng.standard_normal((P, ps, Hkv, D))
    vc = rng.standard_normal((P, ps, Hkv, D))
    perm = rng.permutation(P)
    bt = np.zeros((B, max(pages)), np.int64)
    off = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[off:off + n]
        off += n
    q = rng.standard_normal((B, Q, Hq, D))
    return q, kc, vc, bt


@pytest.mark.parametrize("causal", [True, False])
def test_matches_torch_sdpa_with_reference_masks(causal):
    B, Q, Hq, Hkv, D, ps = 2, 5, 8, 2, 16, 4
    lens = [23, 9]
    q, kc, vc, bt = _contiguous_problem(0, B, Q, Hq, Hkv, D, lens, ps)
    scale = D ** -0.5
    got = oa.paged_attention(q, kc, vc, bt, lens, scale, causal=causal)
    for b, ctx in enumerate(lens):
        K = torch.from_numpy(oa.gather_kv(kc, bt, b, ctx)).permute(1, 0, 2)[None]
        V = torch.from_numpy(oa.gather_kv(vc, bt, b, ctx)).permute(1, 0, 2)[None]
        K = K.repeat_interleave(Hq // Hkv, dim=1)
        V = V.repeat_interleave(Hq // Hkv, dim=1)
        qq = torch.from_numpy(q[b]).permute(1, 0, 2)[None]
        cols = torch.arange(ctx)[None, :]
        rows = torch.arange(Q)[:, None]
        mask = cols <= ctx - Q + rows if causal else torch.ones(Q, ctx, dtype=torch.bool)
        ref = F.scaled_dot_product_attention(qq, K, V, attn_mask=mask, scale=scale)
        np.testing.assert_allclose(got[b], ref[0].permute(1, 0, 2).numpy(), rtol=1e-10, atol=1e-12)


def test_gather_follows_page_table():
    ps, Hkv, D = 4, 1, 2
    kc = np.arange(3 * ps * Hkv * D, dtype=float).reshape(3, ps, Hkv, D)
    bt = np.array([[2, 0]])
    got = oa.gather_kv(kc, bt, 0, 6)
    np.testing.assert_array_equal(got[:4], kc[2])
    np.testing.assert_array_equal(got[4:], kc[0, :2])


def test_closed_forms():
    B, Q, Hq, Hkv, D, ps = 1, 3, 2, 1, 4, 2
    ctx = 6
    kc = np.zeros((3, ps, Hkv, D))  # all keys equal -> uniform weights
    rng = np.random.default_rng(1)
    vc = rng.standard_normal((3, ps, Hkv, D))
    bt = np.array([[0, 1, 2]])
    q = rng.standard_normal((B, Q, Hq, D))
    out = oa.paged_attention(q, kc, vc, bt, [ctx], 0.5, causal=True)
    V = oa.gather_kv(vc, bt, 0, ctx)[:, 0]
    for i in range(Q):
        np.testing.assert_allclose(out[0, i, 0], V[: ctx - Q + i + 1].mean(0), rtol=1e-12)
    out = oa.paged_attention(q, kc, vc, bt, [ctx], 0.5, causal=False)
    np.testing.assert_allclose(out[0, :, 1], np.broadcast_to(V.mean(0), (Q, D)), rtol=1e-12)
    # a block alone (ctx == Q): query 0 sees only key 0
    out = oa.paged_attention(q, rng.standard_normal((3, ps, Hkv, D)), vc, bt, [Q], 0.5, causal=True)
    np.testing.assert_allclose(out[0, 0, :], np.broadcast_to(V[0], (Hq, D)), rtol=1e-12)


def test_fp32_torch_restatement_matches_fp64_oracle():
    from oracle import torch_ref
    from d3d_amd import workloads
    kv = workloads.paged_kv(3, [100, 37], Hkv=2, D=128, page_size=16)
    q = workloads.queries(4, 2, 5, Hq=4)
    for causal in (True, False):
        a = torch_ref.paged_attention_sdpa(q, kv.k_cache, kv.v_cache, kv.block_table, kv.context_lens,
                                           128 ** -0.5, causal=causal)
        b = oa.paged_attention(q.float().numpy(), kv.k_cache.float().numpy(), kv.v_cache.float().numpy(),
                               kv.block_table.numpy(), kv.context_lens.numpy(), 128 ** -0.5, causal=causal)
        np.testing.assert_allclose(a.numpy(), b, atol=2e-6)


def test_packed_visibility_restates_engine_mask():
    """d3d_amd.attention.packed_visibility, expanded to a bool mask, equals
    the oracle's restatement of Engine._mask (serving/engine.py:35-52)."""
    import numpy as np
    from d3d_amd.attention import packed_visibility
    from oracle.attention import engine_mask
    K = 16
    for A in (1, 2, 3):
        specs = [(n, 7) for n in range(1, K) for _ in range(A)] + [(K, None)]
        Q = K * (1 + len(specs))
        vis = packed_visibility(K, [n for n, _ in specs]).numpy()
        for prefix in (0, 5, 1024):
            S = prefix + Q
            t = np.arange(S)[None, :]
            got = (t < prefix + vis[:, :1]) | ((t >= prefix + vis[:, 1:2]) & (t < prefix + vis[:, 2:3]))
            np.testing.assert_array_equal(got, engine_mask(prefix, Q, S, K, specs))


def test_engine_mask_closed_form():
    """engine_mask pinned by counts and intervals written from
    serving/engine.py:35-52 directly (not from packed_visibility):

    * recovery: every row sees exactly the columns [0, prefix + Q);
    * pending rows i < K: [0, prefix + i + 1) -- the prefix and the pending
      block causally;
    * branch j with (accepted n, anchor) at rows K + jK .. K + jK + K - 1:
      [0, prefix + n) plus its own block [prefix + K + jK, prefix + K + jK + K),
      so prefix + n + K columns, and nothing of any other branch.
    """
    engine_mask = oa.engine_mask
    K = 16
    for prefix in (0, 3, 257):
        Q, S = K, prefix + K + 5
        m = engine_mask(prefix, Q, S, K)
        assert (m.sum(1) == prefix + Q).all()
        assert m[:, :prefix + Q].all() and not m[:, prefix + Q:].any()
        for A in (1, 3):
            specs = [(n, 100 + a) for n in range(1, K) for a in range(A)] + [(K, None)]
            Q = K * (1 + len(specs))
            S = prefix + Q
            m = engine_mask(prefix, Q, S, K, specs)
            for i in range(K):
                row = np.zeros(S, bool)
                row[:prefix + i + 1] = True
                np.testing.assert_array_equal(m[i], row)
            for j, (n, _a) in enumerate(specs):
                off = K + j * K
                for r in range(off, off + K):
                    row = np.zeros(S, bool)
                    row[:prefix + n] = True
                    row[prefix + off:prefix + off + K] = True
                    np.testing.assert_array_equal(m[r], row)
                    assert m[r].sum() == prefix + n + K
            # Branch blocks never see each other's columns.
            own = np.zeros((Q, S), bool)
            for j in range(len(specs)):
                off = K + j * K
                own[off:off + K, prefix + off:prefix + off + K] = True
            other_blocks = np.zeros(S, bool)
            other_blocks[prefix + K:] = True
            assert not (m[K:] & other_blocks[None, :] & ~own[K:]).any()
