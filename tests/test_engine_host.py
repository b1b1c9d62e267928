"""Host-side logic of the engine step (CPU): branch specs, acceptance lists,
the packed mask builder and constructor validation."""
from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from d3d_amd.engine import Engine, _Mask, branch_specs
from d3d_amd.modeling_d3d import mask_to_visibility


def _reference_specs(K, A, current, top):
    """serving/engine.py:98-105 (non-shallow branches), restated."""
    branches = []
    for accepted in range(1, K):
        anchors = [v for v in top[accepted] if v != current[accepted]][:A]
        assert len(anchors) == A
        branches.extend((accepted, a) for a in anchors)
    branches.append((K, None))
    return branches


@pytest.mark.parametrize("A", [1, 2, 3])
def test_branch_specs_follow_engine_predict(A):
    rng = random.Random(A)
    K = 16
    for _ in range(50):
        top = [rng.sample(range(40), A + 1) for _ in range(K)]
        # current agrees with the draft's greedy token at some positions only
        current = [t[0] if rng.random() < 0.5 else rng.randrange(40) for t in top]
        assert branch_specs(K, A, current, top) == _reference_specs(K, A, current, top)
    assert len(branch_specs(K, A, current, top)) == A * (K - 1) + 1


def test_shallow_branches():
    """serving/engine.py:98-104 with shallow=True: only n = 1, fan-out
    miss_anchors, no all-accepted branch."""
    top = [[7, 8, 9, 10]] * 4
    current = [1, 8, 2, 3]
    assert branch_specs(4, 1, current, top, shallow=True, fanout=3) == [(1, 7), (1, 9), (1, 10)]


def test_branch_specs_need_enough_alternatives():
    with pytest.raises(RuntimeError):
        branch_specs(3, 2, [1, 2, 3], [[1, 2, 3], [2, 2, 2], [5, 6, 7]])


def test_accepted_lists_follow_engine_accepted():
    """Engine._accepted keeps serving/engine.py:138-145's list semantics."""
    assert Engine._accepted([[5, 1, 2, 9]], [[1, 2, 7, 8]]) == [(3, 7)]
    assert Engine._accepted([[5, 1, 2]], [[1, 2, 4]]) == [(3, 4)]
    assert Engine._accepted([[5, 0, 0]], [[1, 2, 4]]) == [(1, 1)]


@pytest.mark.parametrize("A", [1, 3])
def test_mask_builder_visibility_equals_its_mask(A):
    """_Mask's bool mask (serving/engine.py:35-52) and its descriptor agree,
    for the recovery mask and the packed mask, at several prefixes."""
    K = 16
    specs = [(n, 100 + a) for n in range(1, K) for a in range(A)] + [(K, None)]
    Q = K * (1 + len(specs))
    for builder, q in ((_Mask(K), K), (_Mask(K, [specs, specs]), Q)):
        starts = torch.tensor([0, 37])
        S = 37 + q
        mask = builder(starts, q, S)
        vis = builder.visibility(q)
        for b, p in enumerate(starts.tolist()):
            got = mask_to_visibility(mask[b:b + 1, ..., :p + q], q, p + q)
            rel = vis + torch.tensor([p, p, p], dtype=torch.int32)
            # empty second ranges may be written as any lo == hi
            empty = got[:, 1] == got[:, 2]
            assert torch.equal(got[:, 0], rel[:, 0])
            assert torch.equal(got[~empty, 1:], rel[~empty, 1:])
            assert ((rel[empty, 1] == rel[empty, 2]) | (rel[empty, 2] <= rel[empty, 0])).all()


def test_mask_to_visibility_rejects_other_shapes():
    m = torch.zeros(1, 1, 2, 10, dtype=torch.bool)
    m[0, 0, 0, [0, 1, 4, 8]] = True  # three runs
    with pytest.raises(ValueError):
        mask_to_visibility(m, 2, 10)
    m2 = torch.ones(2, 1, 2, 10, dtype=torch.bool)
    m2[1, 0, 0, 9] = False  # differs between requests
    with pytest.raises(ValueError):
        mask_to_visibility(m2, 2, 10)
    assert mask_to_visibility(None, 3, 7).tolist() == [[7, 0, 0]] * 3


@pytest.mark.parametrize("kw", [dict(backup="slow"), dict(anchor_num=0), dict(fast_miss_anchors=-1),
                                dict(draft_microbatch=0)])
def test_engine_rejects_bad_arguments_before_allocating(kw):
    with pytest.raises(ValueError):
        Engine("Qwen/Qwen3-8B", "fudan-generative-ai/D3D-1.7B-8B", **kw)


def test_split_product_rejects_a_leading_dimension_other_than_splits():
    from d3d_amd.layers import SplitProduct
    ok = SplitProduct(torch.zeros(3, 4, 8), 3)
    assert ok.shape == (4, 8)
    for parts, splits in ((torch.zeros(2, 4, 8), 3), (torch.zeros(4, 8), 1), (torch.zeros(0, 4, 8), 0)):
        with pytest.raises(ValueError, match="split partials must be"):
            SplitProduct(parts, splits)


def test_page_table_updates_keep_the_mirror_equal_to_the_host_lists():
    """DevicePageTables.updates/apply (the entries block_inputs rewrites in
    one copy) on a CPU pool: after every reserve / trim / re-reserve of the
    engine's step pattern (a 272-token packed block reserved, the tail
    trimmed, reserved again) each row holds the host page list, then -1."""
    from d3d_amd.model import DevicePageTables, PagePool, Sequence, reserve, trim

    class _KV:  # the two members reserve/trim use
        page_size = 16
        pool = PagePool(256)

    kv = _KV()
    kv.tables = DevicePageTables(256, "cpu", rows=2)  # grows past two rows
    rng = random.Random(5)
    seqs = [Sequence(i, [0] * (20 + 9 * i)) for i in range(5)]

    def check():
        upds = [u for u in (kv.tables.updates(s, "d") for s in seqs) if u is not None]
        if upds:
            flat = torch.from_numpy(np.concatenate([u[0] for u in upds]).astype(np.int32))
            vals = torch.from_numpy(np.concatenate([u[1] for u in upds]).astype(np.int32))
            kv.tables.apply(flat, vals)
        for s in seqs:
            row = kv.tables.pool[s.rows["d"]].tolist()
            n = len(s.pages["d"])
            assert row[:n] == s.pages["d"] and all(v == -1 for v in row[n:])
        assert all(kv.tables.updates(s, "d") is None for s in seqs)  # nothing left to write

    for step in range(12):
        for s in seqs:
            reserve(kv, s, "d", s.prefix + 272)
        check()
        for s in seqs:
            s.prefix += rng.randint(1, 16)
            trim(kv, s, "d", s.prefix)
        if step % 3 == 2:
            check()  # trims alone: -1 over the released entries
        for s in seqs:
            reserve(kv, s, "d", s.prefix + 16)
        check()
