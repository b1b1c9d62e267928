"""Top-k log-probabilities (GPU): torch.topk(log_softmax(x), k) of the anchor
draft, single/eval_sync.py:763-768, against fp64 log_softmax."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from d3d_amd.draft import topk_tokens

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("V,k", [(151936, 4), (5000, 2), (64, 8)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_topk_log_softmax_values(V, k, dtype):
    x = (torch.randn(6, V, generator=torch.Generator().manual_seed(V)) * 4).to(dtype)
    ids, lp = topk_tokens(x.to("cuda:0"), k, with_values=True, log_softmax=True)
    ref = torch.log_softmax(x.double(), -1)
    # Descending value, equal values by ascending id (bf16 rows hold many
    # exact ties): a stable sort of -x.
    want = np.argsort(-x.float().numpy(), axis=-1, kind="stable")[:, :k]
    np.testing.assert_array_equal(ids.cpu().numpy(), want)
    np.testing.assert_allclose(lp.cpu().numpy(), ref.gather(-1, ids.cpu()).numpy(), atol=2e-5, rtol=0)


def test_log_softmax_values_many_rows():
    """128 rows of 151936, bf16."""
    x = (torch.randn(128, 151936, generator=torch.Generator().manual_seed(9)) * 4).to(torch.bfloat16)
    ids, lp = topk_tokens(x.to("cuda:0"), 2, with_values=True, log_softmax=True)
    ref = torch.log_softmax(x.double(), -1)
    np.testing.assert_allclose(lp.cpu().numpy(), ref.gather(-1, ids.cpu()).numpy(), atol=2e-5, rtol=0)
    assert torch.equal(ids[:, 0].cpu(), x.float().argmax(-1))
