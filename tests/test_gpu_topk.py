"""Top-k token ids of logits rows (GPU) against a CPU sort.

Order: descending value, equal values by ascending id; NaN never selected.
Bit-exact: the ids and values must equal the CPU selection on the same
(fp32 or bf16-rounded) inputs.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from d3d_amd.draft import topk_tokens

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _ref(x: torch.Tensor, k: int):
    a = x.float().numpy().reshape(-1, x.shape[-1])
    out = np.empty((a.shape[0], k), np.int64)
    for r, row in enumerate(a):
        idx = np.arange(row.size)
        ok = ~np.isnan(row)
        order = np.lexsort((idx[ok], -row[ok]))  # primary -value, secondary id
        out[r] = idx[ok][order[:k]]
    return out.reshape(*x.shape[:-1], k)


@pytest.mark.parametrize("V", [151936, 4099, 4096, 100])
@pytest.mark.parametrize("k", [1, 2, 4, 16, 64])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_topk_matches_cpu_sort(V, k, dtype):
    g = torch.Generator().manual_seed(V + k)
    x = (torch.randn(3, 7, V, generator=g) * 3).to(dtype)
    ids, vals = topk_tokens(x.to(DEV), k, with_values=True)
    torch.cuda.synchronize()
    ref = _ref(x, k)
    np.testing.assert_array_equal(ids.cpu().numpy(), ref)
    np.testing.assert_array_equal(vals.cpu().numpy(), np.take_along_axis(x.float().numpy(), ref, -1))
    assert torch.equal(ids[..., 0].cpu(), x.float().argmax(-1))


@pytest.mark.parametrize("k", [2, 16])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_many_rows_match_cpu_sort(k, dtype):
    """128 rows of 151936 (the 1088-row predict's shape, fewer rows)."""
    g = torch.Generator().manual_seed(128 + k)
    x = (torch.randn(128, 151936, generator=g) * 3).to(dtype)
    ids, vals = topk_tokens(x.to(DEV), k, with_values=True)
    torch.cuda.synchronize()
    ref = _ref(x, k)
    np.testing.assert_array_equal(ids.cpu().numpy(), ref)
    np.testing.assert_array_equal(vals.cpu().numpy(), np.take_along_axis(x.float().numpy(), ref, -1))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_ties_go_to_the_lowest_id(dtype):
    V = 9000
    x = torch.zeros(4, V)
    x[0, [17, 4095, 4096, 8999]] = 5.0     # equal maxima across chunks
    x[1] = 1.0                              # constant row
    x[2, ::3] = 2.0
    x[3, 8000:] = -1.0
    x = x.to(dtype)
    ids = topk_tokens(x.to(DEV), 5).cpu().numpy()
    np.testing.assert_array_equal(ids, _ref(x, 5))
    assert list(ids[0, :4]) == [17, 4095, 4096, 8999]
    assert list(ids[1]) == [0, 1, 2, 3, 4]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_nan_and_infinities(dtype):
    V = 5000
    x = torch.randn(2, V, generator=torch.Generator().manual_seed(1))
    x[0, 10] = float("nan")
    x[0, 11] = float("inf")
    x[1, :] = float("-inf")
    x[1, 4999] = float("nan")
    x = x.to(dtype)
    ids = topk_tokens(x.to(DEV), 3).cpu().numpy()
    assert ids[0, 0] == 11 and 10 not in ids[0]
    np.testing.assert_array_equal(ids[1], [0, 1, 2])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_signed_zeros_tie_and_keep_their_sign(dtype):
    """-0 and +0 are equal values (ties by id); the returned values keep
    their sign bits; -inf entries are selectable, NaN never."""
    V = 9000
    x = torch.full((3, V), -1.0)
    x[0, [5, 4100, 30]] = torch.tensor([-0.0, 0.0, -0.0])
    x[1, :] = float("-inf")
    x[1, [7, 8001]] = float("nan")
    x[2, :] = -0.0
    x[2, 3] = 0.0
    x = x.to(dtype)
    ids, vals = topk_tokens(x.to(DEV), 4, with_values=True)
    torch.cuda.synchronize()
    ids, vals = ids.cpu().numpy(), vals.cpu().numpy()
    np.testing.assert_array_equal(ids, _ref(x, 4))
    assert list(ids[0, :3]) == [5, 30, 4100] and list(ids[1]) == [0, 1, 2, 3]
    np.testing.assert_array_equal(np.signbit(vals[0, :3]), [True, True, False])
    np.testing.assert_array_equal(np.signbit(vals[2]), [True, True, True, False])
    assert list(ids[2]) == [0, 1, 2, 3]


def test_k_equals_vocabulary():
    x = torch.randn(5, 8, generator=torch.Generator().manual_seed(2))
    ids = topk_tokens(x.to(DEV), 8).cpu().numpy()
    np.testing.assert_array_equal(ids, _ref(x, 8))


def test_invalid_k_is_rejected():
    with pytest.raises(ValueError):
        topk_tokens(torch.zeros(2, 10, device=DEV), 17)
