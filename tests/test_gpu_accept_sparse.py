"""Parity of the sparse-proposal acceptance kernel with the oracle (GPU).

single/speculative_sampling.py:79-143 (verify_speculative_block_sparse),
batched.  Integer outputs must be bit-exact wherever the fp64 oracle
certifies the decision margins (|u - a| > 1e-5 and the inverse-CDF crossing
more than 1e-6 * W from both bar edges).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from d3d_amd import speculative_sampling as ss
from d3d_amd import workloads

pytestmark = pytest.mark.gpu

U_MARGIN = 1e-5
CDF_MARGIN = 1e-6
DEV = torch.device("cuda:0")


def _run(inp: workloads.SparseAcceptInputs, temperature=1.0, dtype=torch.float32, kind="logits", target=None):
    t = (inp.target if target is None else target).to(DEV, dtype)
    out = ss.accept_fused_sparse(t, inp.tokens.to(DEV), inp.q_ids.to(DEV), inp.q_probs.to(DEV),
                                 temperature=temperature, uniforms=inp.uniforms.to(DEV),
                                 resample_uniform=inp.resample_u.to(DEV), input_kind=kind)
    torch.cuda.synchronize()
    return {k: getattr(out, k).cpu().numpy() for k in out._fields}, t.float().cpu()


def _oracle(inp, t, kind, T=1.0):
    return oracle.accept_sparse(t.numpy(), inp.tokens.numpy(), inp.q_ids.numpy(), inp.q_probs.numpy(),
                                inp.uniforms.numpy(), inp.resample_u.numpy(), kind=kind, temperature=T)


def _check(got, ref, min_certified):
    ok = (ref["u_margin"] > U_MARGIN) & (ref["cdf_margin"] > CDF_MARGIN)
    assert ok.mean() >= min_certified, f"only {ok.mean():.2f} of cases certified"
    idx = np.flatnonzero(ok)
    for k in ("accepted", "out_token"):
        np.testing.assert_array_equal(got[k][idx], ref[k][idx])
    np.testing.assert_array_equal(got["all_accepted"][idx], ref["all_accepted"][idx].astype(bool))
    np.testing.assert_array_equal(got["accept_mask"][idx], ref["accept_mask"][idx].astype(bool))


@pytest.mark.parametrize("V,B,S", [(1000, 8, 8), (4099, 4, 64), (151936, 8, 64), (151936, 4, 1), (70001, 3, 1024)])
@pytest.mark.parametrize("T", [1.0, 0.7])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sparse_logits_vs_oracle(V, B, S, T, dtype):
    inp = workloads.sparse_accept_inputs(200 + V % 89 + S, B=B, K=15, V=V, S=S, temperature=T)
    got, t = _run(inp, T, dtype)
    ref = _oracle(inp, t, oracle.KIND_LOGITS, T)
    _check(got, ref, 0.6)
    np.testing.assert_array_equal(got["posterior"], t.numpy().argmax(-1))


@pytest.mark.parametrize("V", [512, 151936])
def test_sparse_probs_input_vs_oracle(V):
    inp = workloads.sparse_accept_inputs(31, B=6, K=15, V=V, S=64)
    tp = torch.softmax(inp.target, -1) * 2.5  # unnormalised probabilities
    got, t = _run(inp, kind="probs", target=tp)
    _check(got, _oracle(inp, t, oracle.KIND_PROBS), 0.66)


def test_config0_sparse_fixture_seeds():
    """Batch-1 sparse acceptance at V=151936, S=64, T=1 on 32 seeds."""
    certified = 0
    for seed in range(32):
        inp = workloads.sparse_accept_inputs(seed, B=1, K=15, S=64)
        got, t = _run(inp)
        ref = _oracle(inp, t, oracle.KIND_LOGITS)
        if ref["u_margin"][0] > U_MARGIN and ref["cdf_margin"][0] > CDF_MARGIN:
            certified += 1
            assert got["accepted"][0] == ref["accepted"][0], seed
            assert got["out_token"][0] == ref["out_token"][0], seed
    assert certified >= 26


def test_duplicate_and_out_of_range_support_ids():
    """Duplicates accumulate (scatter_add) and ids outside [0, V) carry no mass."""
    V, S = 2048, 16
    inp = workloads.sparse_accept_inputs(5, B=4, K=7, V=V, S=S)
    ids = inp.q_ids.clone()
    ids[:, :, 3] = ids[:, :, 0]  # duplicate of the top id
    ids[:, :, 5] = ids[:, :, 1]
    ids[:, :, 9] = -1
    ids[:, :, 10] = V
    ids[:, :, 11] = V + 12345
    inp.q_ids = ids
    inp.uniforms[:] = 0.97  # many rejections: exercise the residual path
    got, t = _run(inp)
    ref = _oracle(inp, t, oracle.KIND_LOGITS)
    _check(got, ref, 0.75)
    assert (got["accepted"] < 7).any()


def test_full_support_matches_dense_acceptance():
    """S = V with ids 0..V-1 is the dense proposal: the sparse entry point
    reaches the dense oracle's decisions wherever those are certified."""
    V, K, B = 640, 5, 8
    d = workloads.accept_inputs(17, B=B, K=K, V=V)
    q = torch.softmax(d.draft, -1)
    p = torch.softmax(d.target, -1)
    sp = workloads.SparseAcceptInputs(d.target, d.tokens, torch.arange(V).expand(B, K, V).contiguous(), q,
                                      d.uniforms, d.resample_u)
    got, _ = _run(sp, kind="probs", target=p)
    ref = oracle.accept_dense(p.numpy(), q.numpy(), d.tokens.numpy(), d.uniforms.numpy(), d.resample_u.numpy(),
                              kind=oracle.KIND_PROBS)
    _check(got, ref, 0.75)


def test_greedy_mode_ignores_proposals():
    inp = workloads.sparse_accept_inputs(3, B=3, K=15, V=4096, S=8)
    got, t = _run(inp, temperature=0.0)
    ref = oracle.accept_greedy(t.numpy(), inp.tokens.numpy())
    np.testing.assert_array_equal(got["accepted"], ref["accepted"])
    np.testing.assert_array_equal(got["out_token"], ref["out_token"])


def test_verify_speculative_block_sparse_reference_surface():
    for seed in range(9, 40):  # first seed whose decisions the oracle certifies
        inp = workloads.sparse_accept_inputs(seed, B=1, K=15, S=64)
        ref = _oracle(inp, torch.softmax(inp.target, -1), oracle.KIND_PROBS)
        if ref["u_margin"][0] > U_MARGIN and ref["cdf_margin"][0] > CDF_MARGIN:
            break
    p = torch.softmax(inp.target, -1).to(DEV)
    res = ss.verify_speculative_block_sparse(inp.tokens.to(DEV), p, inp.q_ids.to(DEV), inp.q_probs.to(DEV),
                                             uniforms=inp.uniforms.to(DEV),
                                             resample_uniform=inp.resample_u.to(DEV))
    ref = _oracle(inp, p.cpu(), oracle.KIND_PROBS)
    assert ref["u_margin"][0] > U_MARGIN and ref["cdf_margin"][0] > CDF_MARGIN
    assert res.accepted_draft_tokens == ref["accepted"][0]
    assert int(res.correction_token[0]) == ref["out_token"][0]
    assert res.all_accepted == bool(ref["all_accepted"][0])
    res2 = ss.verify_speculative_block_sparse(inp.tokens.to(DEV), p, inp.q_ids.to(DEV), inp.q_probs.to(DEV))
    assert 0 <= res2.accepted_draft_tokens <= 15
    with pytest.raises(ValueError, match="batch size 1"):
        ss.verify_speculative_block_sparse(inp.tokens.repeat(2, 1).to(DEV), p.repeat(2, 1, 1),
                                           inp.q_ids.repeat(2, 1, 1).to(DEV), inp.q_probs.repeat(2, 1, 1).to(DEV))
    with pytest.raises(ValueError, match="identical shapes"):
        ss.verify_speculative_block_sparse(inp.tokens.to(DEV), p, inp.q_ids.to(DEV), inp.q_probs[..., :3].to(DEV))
    with pytest.raises(ValueError, match=r"\[B,K,S\]"):
        ss.verify_speculative_block_sparse(inp.tokens.to(DEV), p, inp.q_ids[0].to(DEV), inp.q_probs.to(DEV))


def test_support_size_limit():
    inp = workloads.sparse_accept_inputs(1, B=1, K=2, V=4096, S=1025)
    with pytest.raises(ValueError):
        _run(inp)
