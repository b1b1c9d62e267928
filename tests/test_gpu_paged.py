"""Device paged-KV block inputs (GPU) against the integer restatement in
oracle/paged.py (serving/backend.py:73-76, :123-124); bit-exact."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from d3d_amd import _lib
from d3d_amd.attention import kv_append
from d3d_amd.model import D3D_1P7B, PagedKV, Sequence, block_inputs, release, reserve, trim
from oracle import paged

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _kernel(pool: np.ndarray, rows, starts, Q, width, page_size):
    lib = _lib.load()
    B = len(rows)
    pool_d = torch.from_numpy(pool).to(DEV)
    rows_d = torch.tensor(rows, dtype=torch.int32, device=DEV)
    starts_d = torch.tensor(starts, dtype=torch.int32, device=DEV)
    tab = torch.empty(B, width, dtype=torch.int32, device=DEV)
    slots = torch.empty(B, Q, dtype=torch.int64, device=DEV)
    pos = torch.empty(B, Q, dtype=torch.int64, device=DEV)
    lens = torch.empty(B, dtype=torch.int32, device=DEV)
    st = lib.d3d_block_inputs(pool_d.data_ptr(), pool.shape[0], pool.shape[1], rows_d.data_ptr(), starts_d.data_ptr(),
                              B, Q, width, page_size, tab.data_ptr(), slots.data_ptr(), pos.data_ptr(),
                              lens.data_ptr(), _lib.stream_ptr(DEV))
    _lib.check(st, "d3d_block_inputs")
    return tab.cpu().numpy(), slots.cpu().numpy(), pos.cpu().numpy(), lens.cpu().numpy()


@pytest.mark.parametrize("page_size", [1, 16, 24, 64])
@pytest.mark.parametrize("Q", [1, 16, 272])
def test_block_inputs_kernel_matches_restatement(page_size, Q):
    rng = np.random.default_rng(page_size * 1000 + Q)
    R, W = 12, 40
    lists = [list(rng.permutation(500)[: rng.integers(1, W)]) for _ in range(R)]
    pool = np.full((R, W), -1, np.int32)
    for r, l in enumerate(lists):
        pool[r, : len(l)] = l
    rows = list(rng.permutation(R)[:7])
    starts = [int(rng.integers(0, len(lists[r]) * page_size + 5)) for r in rows]
    width = 30
    got = _kernel(pool, rows, starts, Q, width, page_size)
    want = paged.block_inputs([lists[r] for r in rows], starts, Q, page_size, width)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)


def test_rows_outside_the_pool_read_as_empty():
    pool = np.arange(12, dtype=np.int32).reshape(3, 4)
    tab, slots, _, lens = _kernel(pool, [5, -1], [0, 3], 4, 4, 2)
    assert not tab.any() and (slots == -1).all()
    assert list(lens) == [4, 7]


def _host_inputs(kv, seqs, name, starts, Q, width):
    return paged.block_inputs([s.pages[name] for s in seqs], starts, Q, kv.page_size, width)


def test_device_mirror_follows_reserve_trim_release():
    kv = PagedKV(D3D_1P7B, 64, 16, DEV)
    seqs = [Sequence(i, list(range(10 + 7 * i))) for i in range(5)]
    for s in seqs:
        reserve(kv, s, "draft", s.prefix + 16)
    width = 8
    for step in range(6):
        starts = [s.prefix for s in seqs]
        tab, slots, lens, pos, max_ctx = block_inputs(kv, seqs, "draft", starts, 16, DEV, width)
        want = _host_inputs(kv, seqs, "draft", starts, 16, width)
        np.testing.assert_array_equal(tab.cpu().numpy(), want[0])
        np.testing.assert_array_equal(slots.view(len(seqs), 16).cpu().numpy(), want[1])
        np.testing.assert_array_equal(pos.cpu().numpy(), want[2])
        np.testing.assert_array_equal(lens.cpu().numpy(), want[3])
        assert max_ctx == width * 16
        # commit a few tokens, trim the rejected tail, let one sequence finish
        for j, s in enumerate(seqs):
            s.prefix += (step + j) % 5
            trim(kv, s, "draft", s.prefix)
            reserve(kv, s, "draft", s.prefix + 16)
        if step == 2:
            release(kv, seqs[1], "draft")
            seqs.pop(1)
            new = Sequence(9, list(range(33)))
            reserve(kv, new, "draft", new.prefix + 16)
            seqs.append(new)


def test_kv_round_trip_through_device_slots():
    """K/V appended at the kernel's slots read back through its tables."""
    kv = PagedKV(D3D_1P7B, 32, 16, DEV)
    seqs = [Sequence(i, list(range(5 + 9 * i))) for i in range(3)]
    for s in seqs:
        reserve(kv, s, "draft", s.prefix + 16)
    tab, slots, lens, pos, _ = block_inputs(kv, seqs, "draft", [s.prefix for s in seqs], 16, DEV, 4)
    Hkv, D = D3D_1P7B.kv_heads, D3D_1P7B.head_dim
    g = torch.Generator().manual_seed(1)
    k = torch.randn(3 * 16, Hkv, D, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(3 * 16, Hkv, D, generator=g).to(torch.bfloat16).to(DEV)
    kv_append(k, v, kv.k[0], kv.v[0], slots)
    torch.cuda.synchronize()
    kc = kv.k[0].cpu()
    for b, s in enumerate(seqs):
        for i in range(16):
            t = s.prefix + i
            page = int(tab[b, t // 16])
            assert torch.equal(kc[page, t % 16], k[b * 16 + i].cpu())
