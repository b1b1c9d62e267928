"""Draft proposal sampling and caller-given top-k unmask (GPU) against the oracle.

single/eval_sync.py:287-367 (proposal draws) and :447-465 (_select_transfer).
torch.multinomial is replaced by the inverse CDF at a given uniform, so
tokens are compared bit-exactly wherever the fp64 oracle certifies the CDF
crossing to lie more than 1e-6 * W from both bar edges; probabilities agree
with the fp64 values to 2e-6 relative.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from d3d_amd import draft as dr
from d3d_amd.model import ModelShape, PagedKV, Qwen3PagedModel, Sequence, prefill

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
CDF_MARGIN = 1e-6


def _logits(seed, N, V, dtype, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(N, V, generator=g) * scale).to(dtype)


@pytest.mark.parametrize("V", [1000, 4099, 151936])
@pytest.mark.parametrize("T", [1.0, 0.7])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sample_with_prob_vs_oracle(V, T, dtype):
    N = 24
    x = _logits(V + int(T * 10), N, V, dtype)
    u = torch.rand(N, generator=torch.Generator().manual_seed(V))
    tok, prob = dr.sample_with_prob(x.to(DEV), T, uniforms=u.to(DEV))
    torch.cuda.synchronize()
    rt, rp, margin = oracle.sample_with_prob(x.float().numpy(), T, u.numpy())
    ok = margin > CDF_MARGIN
    assert ok.mean() >= 0.7  # bars of a 151936-entry softmax are ~1e-5 wide
    np.testing.assert_array_equal(tok.cpu().numpy()[ok], rt[ok])
    np.testing.assert_allclose(prob.cpu().numpy()[ok], rp[ok], rtol=2e-6, atol=1e-9)


def test_greedy_sampling_is_argmax_with_probability_one():
    x = _logits(3, 10, 5000, torch.bfloat16)
    tok, prob = dr.sample_with_prob(x.to(DEV), 0.0)
    assert torch.equal(tok.cpu(), x.float().argmax(-1))
    assert torch.equal(prob.cpu(), torch.ones(10))
    assert torch.equal(dr.sample_tokens(x.to(DEV), 0.0).cpu(), tok.cpu())


def test_inverse_cdf_edges():
    """u = 0 takes the first token with positive weight; a one-hot row always its token."""
    V = 300
    x = torch.full((3, V), -float("inf"))
    x[0, 7] = 0.0
    x[0, 200] = 0.0
    x[1, 123] = 5.0
    x[2, :] = 0.0
    u = torch.tensor([0.0, 0.9999, 0.5])
    tok, prob = dr.sample_with_prob(x.to(DEV), 1.0, uniforms=u.to(DEV))
    tok, prob = tok.cpu().tolist(), prob.cpu().tolist()
    assert tok[0] == 7 and abs(prob[0] - 0.5) < 1e-7
    assert tok[1] == 123 and prob[1] == 1.0
    assert tok[2] == 150 and abs(prob[2] - 1.0 / V) < 1e-9


@pytest.mark.parametrize("V,S", [(151936, 64), (4099, 8), (1000, 1)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sparse_support_vs_oracle(V, S, dtype):
    N, T = 20, 0.8
    x = _logits(S + V, N, V, dtype)
    u = torch.rand(N, generator=torch.Generator().manual_seed(S))
    tok, ids, probs = dr.sample_with_sparse_probs(x.to(DEV), T, S, uniforms=u.to(DEV))
    torch.cuda.synchronize()
    rt, rids, rprobs, margin = oracle.sample_sparse(x.float().numpy(), T, S, u.numpy())
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    np.testing.assert_allclose(probs.cpu().numpy(), rprobs, rtol=2e-6, atol=1e-8)
    ok = margin > CDF_MARGIN
    assert ok.mean() >= 0.7  # bars of a 151936-entry softmax are ~1e-5 wide
    np.testing.assert_array_equal(tok.cpu().numpy()[ok], rt[ok])


def test_sparse_greedy_is_a_support_of_one():
    x = _logits(1, 4, 3000, torch.float32)
    tok, ids, probs = dr.sample_with_sparse_probs(x.to(DEV), 0.0, 64)
    assert torch.equal(tok.cpu(), x.argmax(-1)) and ids.shape == (4, 1)
    assert torch.equal(probs.cpu(), torch.ones(4, 1))


def _select_ref(block, mask_id, k, x0, conf):
    block = block.clone()
    sel = torch.zeros_like(block, dtype=torch.bool)
    for b in range(block.shape[0]):
        idx = [i for i in range(block.shape[1]) if block[b, i] == mask_id]
        idx.sort(key=lambda i: (-float(conf[b, i]), i))
        for i in idx[:k]:
            block[b, i] = x0[b, i]
            sel[b, i] = True
    return block, sel


@pytest.mark.parametrize("Q,k", [(16, 4), (16, 16), (33, 5), (1024, 100)])
def test_select_transfer_matches_ranking(Q, k):
    g = torch.Generator().manual_seed(Q + k)
    B, M = 3, 99
    block = torch.randint(0, 50, (B, Q), generator=g)
    block[torch.rand(B, Q, generator=g) < 0.6] = M
    x0 = torch.randint(0, 50, (B, Q), generator=g)
    conf = torch.rand(B, Q, generator=g)
    conf[:, ::4] = 0.5  # ties go to the lower position
    blk = block.clone().to(DEV)
    sel = dr.select_transfer(blk, M, k, x0.to(DEV), conf.to(DEV))
    ref_block, ref_sel = _select_ref(block, M, k, x0, conf)
    assert torch.equal(blk.cpu(), ref_block) and torch.equal(sel.cpu(), ref_sel)


TINY = ModelShape(layers=2, hidden=256, heads=8, kv_heads=2, head_dim=128, mlp=512, vocab=1000)


@pytest.mark.parametrize("proposal,top_k", [("logits", 0), ("probs", 16), ("sparse", 16)])
def test_stochastic_denoise_loop_plumbing(proposal, top_k):
    """The sampled denoise loop equals its steps run one by one: the forward,
    the draw at that step's uniforms (top-k filtered when top_k > 0), the
    top-k unmask, the last step filling every mask, and proposals recorded
    at the step a position is unmasked."""
    model = Qwen3PagedModel(TINY, DEV, draft=True, seed=5, init_std=0.05)
    T, steps, S = 0.9, 4, 16
    g = torch.Generator().manual_seed(1)
    prompts = torch.randint(0, 998, (2, 32), generator=g)
    block = torch.full((2, 16), 999, dtype=torch.int64)
    block[:, 0] = torch.tensor([5, 6])
    u = torch.rand(steps, 2, 16, generator=g)

    def fresh():
        kv = PagedKV(TINY, 64, 16, DEV)
        seqs = [Sequence(i, p.tolist()) for i, p in enumerate(prompts)]
        prefill(model, kv, seqs, "d")
        return kv, seqs

    kv, seqs = fresh()
    got, prop = dr.draft_block_step(model, kv, seqs, block.to(DEV), steps, mask_id=999, temperature=T,
                                    top_k=top_k, name="d", uniforms=u.to(DEV), return_proposal=proposal)
    kv, seqs = fresh()
    cur = block.clone().to(DEV)
    sched = dr.get_num_transfer_tokens(15, steps)
    rows = {}
    for step, k in enumerate(sched):
        k = 16 if step == len(sched) - 1 else k
        logits = dr.draft_block_forward(model, kv, seqs, cur, name="d")
        if proposal == "sparse":
            x0, ids, probs = dr.sample_with_sparse_probs(logits, T, S, uniforms=u[step].to(DEV))
            conf = probs.gather(-1, (ids == x0[..., None]).long().argmax(-1, keepdim=True))[..., 0]
        else:
            x0, conf = dr.sample_with_prob(logits, T, top_k, uniforms=u[step].to(DEV))
        sel = dr.select_transfer(cur, 999, k, x0, conf)
        for b, i in sel.nonzero().tolist():
            if proposal == "logits":
                rows[(b, i)] = logits[b, i].clone()
            elif proposal == "probs":
                rows[(b, i)] = dr.sampling_probs(logits, T, top_k)[b, i].clone()
            else:
                rows[(b, i)] = (ids[b, i].clone(), probs[b, i].clone())
    assert torch.equal(got, cur) and not (got == 999).any()
    for (b, i), r in rows.items():
        if proposal == "sparse":
            assert torch.equal(prop[0][b, i], r[0]) and torch.equal(prop[1][b, i], r[1])
        else:
            assert torch.equal(prop[b, i], r)
    assert len(rows) == 30


@pytest.mark.parametrize("V,top_k", [(1000, 5), (151936, 64), (151936, 1)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_top_k_filtered_sampling_vs_oracle(V, top_k, dtype):
    """_sampling_probs' top-k filter (single/eval_sync.py:292-295): only
    entries at or above the k-th largest scaled logit carry probability
    (bf16 rows hold ties with the k-th value, all kept); draws and their
    probabilities match the fp64 oracle on certified rows."""
    N, T = 24, 0.8
    x = _logits(V + top_k, N, V, dtype)
    u = torch.rand(N, generator=torch.Generator().manual_seed(top_k))
    tok, prob = dr.sample_with_prob(x.to(DEV), T, top_k, uniforms=u.to(DEV))
    dense = dr.sampling_probs(x.to(DEV), T, top_k)
    torch.cuda.synchronize()
    rt, rp, margin = oracle.sample_with_prob(x.float().numpy(), T, u.numpy(), top_k=top_k)
    rd = oracle.softmax_rows(x.float().numpy(), T, top_k)
    np.testing.assert_array_equal(dense.cpu().numpy() > 0, rd > 0)
    np.testing.assert_allclose(dense.cpu().numpy(), rd, rtol=2e-5, atol=1e-8)
    ok = margin > CDF_MARGIN
    assert ok.mean() >= 0.8
    np.testing.assert_array_equal(tok.cpu().numpy()[ok], rt[ok])
    np.testing.assert_allclose(prob.cpu().numpy()[ok], rp[ok], rtol=2e-5, atol=1e-9)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_dense_probs_vs_oracle(dtype):
    x = _logits(77, 6, 151936, dtype)
    for T in (1.0, 0.6, 0.0):
        got = dr.sampling_probs(x.to(DEV), T)
        ref = oracle.softmax_rows(x.float().numpy(), T)
        np.testing.assert_allclose(got.cpu().numpy(), ref, rtol=2e-5, atol=1e-9)


TOP_P_MARGIN = 1e-6  # |C_j - top_p| the kernels' fp32 masses cannot decide the other way


@pytest.mark.parametrize("V,top_k,top_p", [(151936, 0, 0.9), (151936, 0, 0.5), (151936, 1000, 0.8),
                                           (5000, 100, 0.3), (151936, 70, 1.0), (5000, 4999, 1.0)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_top_p_and_wide_top_k_vs_oracle(V, top_k, top_p, dtype):
    """_sampling_probs' top-p filter and top-k filters wider than 64
    (single/eval_sync.py:292-303): the kept set equals the oracle's exactly
    (bf16 rows put many ties at the cut: the lowest ids stay), the dense
    probabilities agree, and draws match on certified rows."""
    N, T = 12, 0.8
    x = _logits(V + top_k + int(100 * top_p), N, V, dtype)
    u = torch.rand(N, generator=torch.Generator().manual_seed(top_k + 5))
    dense = dr.sampling_probs(x.to(DEV), T, top_k, top_p)
    tok, prob = dr.sample_with_prob(x.to(DEV), T, top_k, top_p, uniforms=u.to(DEV))
    torch.cuda.synchronize()
    xf = x.float().numpy()
    rd = oracle.softmax_rows(xf, T, top_k, top_p)
    fm = oracle.filter_margins(xf, T, top_k, top_p)
    ok_f = fm > TOP_P_MARGIN
    assert ok_f.mean() >= 0.5
    got = dense.cpu().numpy()
    np.testing.assert_array_equal((got > 0)[ok_f], (rd > 0)[ok_f])
    np.testing.assert_allclose(got[ok_f], rd[ok_f], rtol=2e-5, atol=1e-8)
    rt, rp, margin = oracle.sample_with_prob(xf, T, u.numpy(), top_k=top_k, top_p=top_p)
    ok = ok_f & (margin > CDF_MARGIN)
    assert ok.mean() >= 0.4
    np.testing.assert_array_equal(tok.cpu().numpy()[ok], rt[ok])
    np.testing.assert_allclose(prob.cpu().numpy()[ok], rp[ok], rtol=2e-5, atol=1e-9)


def test_row_filter_tie_run_at_the_cut():
    """Known answer: five equal logits after a leading one; top_p cuts inside
    the run, so exactly the lowest ids of the run stay."""
    x = torch.full((1, 300), -30.0)
    x[0, 250] = 2.0
    for i in (10, 20, 30, 40, 50):
        x[0, i] = 1.0
    p = np.exp(np.array([2.0] + [1.0] * 5) - 2.0)
    p /= p.sum()
    c = np.cumsum(p)
    top_p = float((c[2] + c[3]) / 2)  # ids 250, 10, 20, 30 stay
    dense = dr.sampling_probs(x.to(DEV), 1.0, 0, top_p).cpu()
    assert torch.nonzero(dense[0] > 0)[:, 0].tolist() == [10, 20, 30, 250]


@pytest.mark.parametrize("V,S,top_p", [(151936, 65, 1.0), (151936, 1000, 0.9), (5000, 4999, 1.0), (5000, 0, 0.7),
                                       (151936, 0, 1.0)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_wide_sparse_support_vs_oracle(V, S, top_p, dtype):
    """_sample_with_sparse_probs with supports above 64 entries and top_k = 0
    (the whole vocabulary; single/eval_sync.py:341-367): ids in descending
    order of logits / T (ties by ascending id) bit-exact, probabilities after
    the nucleus filter, draws on certified rows."""
    N, T = 6, 0.8
    x = _logits(V + S + 3, N, V, dtype)
    u = torch.rand(N, generator=torch.Generator().manual_seed(S + 11))
    tok, ids, probs = dr.sample_with_sparse_probs(x.to(DEV), T, S, top_p, uniforms=u.to(DEV))
    torch.cuda.synchronize()
    SS = S if S > 0 else V
    assert ids.shape == (N, SS) and probs.shape == (N, SS)
    rt, rids, rprobs, margin = oracle.sample_sparse(x.float().numpy(), T, SS, u.numpy(), top_p=top_p)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    ok = margin > CDF_MARGIN  # includes the nucleus cut's margin
    assert ok.mean() >= 0.5
    np.testing.assert_allclose(probs.cpu().numpy()[ok], rprobs[ok], rtol=2e-5, atol=1e-9)
    np.testing.assert_array_equal(tok.cpu().numpy()[ok], rt[ok])
