"""Fused LM head + top-k (GPU) against an fp32 GEMM reference.

The reference logits are hidden @ weight.T in fp32 (torch, on the device),
rounded to bf16 as the reference's bf16 linear layer returns them; the top-k
order is descending bf16 value, equal values by ascending id.

Parity bar: the kernel accumulates the same bf16 products in fp32 in another
order, so a logit within about 1e-5 (relative) of a bf16 rounding boundary
may round the other way.  A row is certified when every logit within two
bf16 ulps of its k-th largest keeps its bf16 value under a 3e-5 relative
perturbation; on certified rows ids and values must equal the reference
exactly, and on every row each returned value must be within one bf16 ulp
of the reference value at the same rank.
"""
from __future__ import annotations

import pytest
import torch

from d3d_amd.draft import topk_tokens
from d3d_amd.lmhead import lmhead_topk

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _inputs(seed: int, T: int, H: int, V: int):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = (torch.randn(V, H, generator=g) / H ** 0.5).to(torch.bfloat16)
    return x.to(DEV), w.to(DEV)


def _reference(x: torch.Tensor, w: torch.Tensor):
    lf = torch.matmul(x.float(), w.float().t().contiguous())     # fp32 logits
    lb = lf.to(torch.bfloat16).float()                           # bf16-rounded
    return lf, lb


def _ref_topk(lb: torch.Tensor, k: int):
    order = torch.sort(-lb, dim=-1, stable=True).indices         # ties: ascending id
    return order[:, :k]


def _ulp(v: torch.Tensor) -> torch.Tensor:
    # bf16 keeps 8 significant bits: one ulp is 2^(exponent - 7).
    e = torch.floor(torch.log2(v.abs().clamp_min(1e-30)))
    return torch.pow(2.0, e - 7)


def _certified(lf: torch.Tensor, lb: torch.Tensor, k: int) -> torch.Tensor:
    kth = torch.sort(lb, dim=-1, descending=True).values[:, k - 1:k]
    near = lb >= kth - 2 * _ulp(kth)
    up = (lf * (1 + 3e-5)).to(torch.bfloat16).float()
    dn = (lf * (1 - 3e-5)).to(torch.bfloat16).float()
    stable = (up == lb) & (dn == lb)
    return (~near | stable).all(dim=-1)


@pytest.mark.parametrize("T,H,V", [(64, 2048, 151936), (16, 4096, 151936), (1, 2048, 151936),
                                   (65, 128, 4099), (5, 64, 333), (3, 32, 1)])
@pytest.mark.parametrize("k", [1, 2, 4, 8])
def test_lmhead_topk_matches_fp32_gemm(T, H, V, k):
    if k > V:
        pytest.skip("k larger than the vocabulary")
    x, w = _inputs(T * 7 + H + V + k, T, H, V)
    ids, vals = lmhead_topk(x, w, k, with_values=True)
    lf, lb = _reference(x, w)
    ref = _ref_topk(lb, k)
    ref_vals = torch.gather(lb, 1, ref)
    cert = _certified(lf, lb, k)
    assert cert.float().mean().item() >= 0.8, "too few certified rows to judge"
    assert torch.equal(ids[cert], ref[cert])
    assert torch.equal(vals[cert], ref_vals[cert])
    # every row: the returned values are the bf16 logits of the returned ids
    # (within one ulp) and within one ulp of the reference at the same rank
    got_ref = torch.gather(lb, 1, ids)
    assert ((vals - got_ref).abs() <= _ulp(got_ref)).all()
    assert ((vals - ref_vals).abs() <= _ulp(ref_vals)).all()
    # descending values, and equal values by ascending id
    assert (vals[:, 1:] <= vals[:, :-1]).all()
    tie = vals[:, 1:] == vals[:, :-1]
    assert (ids[:, 1:][tie] > ids[:, :-1][tie]).all()


@pytest.mark.parametrize("H,V", [(2048, 151936), (256, 5000)])
def test_lmhead_log_softmax_values(H, V):
    x, w = _inputs(11, 64, H, V)
    ids, lp = lmhead_topk(x, w, 4, with_values=True, log_softmax=True)
    lf, lb = _reference(x, w)
    ref_lp = torch.log_softmax(lb, dim=-1)
    cert = _certified(lf, lb, 4)
    assert torch.equal(ids[cert], _ref_topk(lb, 4)[cert])
    assert torch.allclose(lp, torch.gather(ref_lp, 1, ids), atol=1e-3, rtol=0)


def test_fused_path_equals_gemm_then_topk_on_certified_rows():
    """The engine's unfused path (bf16 GEMM, then topk_tokens) and the fused
    kernel pick the same anchors wherever the bf16 logits are unambiguous."""
    x, w = _inputs(5, 64, 2048, 151936)
    fused = lmhead_topk(x, w, 2)
    logits = torch.nn.functional.linear(x, w)                    # bf16, the engine's path
    unfused = topk_tokens(logits, 2)
    lf, lb = _reference(x, w)
    # Both paths accumulate in fp32 (in different orders); where the logits
    # near the top round stably, both equal the fp32 reference's choice.
    cert = _certified(lf, lb, 2)
    assert cert.float().mean().item() >= 0.8
    assert torch.equal(fused[cert], unfused[cert])


def test_batched_leading_dims():
    x, w = _inputs(3, 4 * 16, 256, 3000)
    ids = lmhead_topk(x.view(4, 16, 256), w, 3)
    assert ids.shape == (4, 16, 3)
    assert torch.equal(ids.view(64, 3), lmhead_topk(x, w, 3))


def test_invalid_arguments_are_rejected():
    x, w = _inputs(1, 4, 64, 100)
    with pytest.raises(ValueError):
        lmhead_topk(x, w, 9)
    with pytest.raises(ValueError):
        lmhead_topk(x.float(), w, 1)
    with pytest.raises(ValueError):
        lmhead_topk(x[:, :48].contiguous(), w[:, :48].contiguous(), 1)  # H not a multiple of 32
