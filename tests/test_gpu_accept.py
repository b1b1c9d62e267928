"""Parity of the fused acceptance kernel with the oracle (GPU).

Integer outputs (accept mask, accepted length, correction/bonus token,
posterior) must be bit-exact.  Stochastic cases are compared where the fp64
oracle certifies the decision margins (|u - a| > 1e-5 at every position and
the inverse-CDF crossing more than 1e-6 * W from both bar edges), so the
result cannot depend on fp32 summation order; the fraction of certified
cases is asserted to stay high.
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


def _dev():
    return torch.device("cuda:0")


def _run(inp: workloads.AcceptInputs, temperature: float, dtype=torch.float32, kind="logits"):
    dev = _dev()
    t = inp.target.to(dev, dtype)
    d = inp.draft.to(dev, dtype)
    out = ss.accept_fused(t, d, inp.tokens.to(dev), temperature=temperature,
                          uniforms=inp.uniforms.to(dev), resample_uniform=inp.resample_u.to(dev),
                          input_kind=kind)
    torch.cuda.synchronize()
    return {k: getattr(out, k).cpu().numpy() for k in out._fields}, t.float().cpu(), d.float().cpu()


def _check_stochastic(got, ref, min_certified=0.8):
    ok = (ref["u_margin"] > U_MARGIN) & (ref["cdf_margin"] > CDF_MARGIN)
    assert ok.mean() >= min_certified, f"only {ok.mean():.2f} of cases certified"
    idx = np.flatnonzero(ok)
    np.testing.assert_array_equal(got["accepted"][idx], ref["accepted"][idx])
    np.testing.assert_array_equal(got["out_token"][idx], ref["out_token"][idx])
    np.testing.assert_array_equal(got["all_accepted"][idx], ref["all_accepted"][idx].astype(bool))
    np.testing.assert_array_equal(got["accept_mask"][idx], ref["accept_mask"][idx].astype(bool))
    return idx


@pytest.mark.parametrize("V", [1000, 4096, 4099, 10007, 151936])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_greedy_bit_exact(V, dtype):
    inp = workloads.accept_inputs(11, B=4, K=15, V=V, temperature=0.0)
    # make request 1 accept a prefix and request 2 accept everything
    post = inp.target.to(dtype).float().argmax(-1)
    inp.tokens[1, :6] = post[1, :6]
    inp.tokens[2] = post[2, :15]
    got, t, _ = _run(inp, 0.0, dtype)
    ref = oracle.accept_greedy(t.numpy(), inp.tokens.numpy())
    np.testing.assert_array_equal(got["posterior"], ref["posterior"])
    np.testing.assert_array_equal(got["accepted"], ref["accepted"])
    np.testing.assert_array_equal(got["out_token"], ref["out_token"])
    np.testing.assert_array_equal(got["accept_mask"], ref["accept_mask"].astype(bool))
    np.testing.assert_array_equal(got["all_accepted"], ref["all_accepted"].astype(bool))
    assert got["accepted"][2] == 15 and got["accepted"][1] >= 6


@pytest.mark.parametrize("V,B,K", [(1000, 8, 15), (4099, 4, 7), (32768, 2, 15), (151936, 8, 15)])
@pytest.mark.parametrize("T", [1.0, 0.6])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_stochastic_logits_vs_oracle(V, B, K, T, dtype):
    inp = workloads.accept_inputs(100 + V % 97 + B, B=B, K=K, V=V, temperature=T)
    got, t, d = _run(inp, T, dtype)
    ref = oracle.accept_dense(t.numpy(), d.numpy(), inp.tokens.numpy(), inp.uniforms.numpy(),
                              inp.resample_u.numpy(), kind=oracle.KIND_LOGITS, temperature=T)
    _check_stochastic(got, ref, min_certified=0.75)
    # posterior is the argmax of every target row in every mode
    np.testing.assert_array_equal(got["posterior"], t.numpy().argmax(-1))


@pytest.mark.parametrize("B,dtype", [(8, torch.float32), (1, torch.bfloat16)])
def test_stochastic_decision_without_posterior_is_unchanged(B, dtype):
    """posterior=False skips the argmax reduction of the stochastic modes:
    the decision (mask, length, token) is the same, bit for bit, and the
    posterior is not returned; greedy acceptance still returns it."""
    dev = _dev()
    inp = workloads.accept_inputs(41 + B, B=B, K=15, V=151936, temperature=1.0)
    t, d = inp.target.to(dev, dtype), inp.draft.to(dev, dtype)
    args = (t, d, inp.tokens.to(dev))
    kw = dict(temperature=1.0, uniforms=inp.uniforms.to(dev), resample_uniform=inp.resample_u.to(dev))
    full = ss.accept_fused(*args, **kw)
    bare = ss.accept_fused(*args, posterior=False, **kw)
    assert bare.posterior is None
    for key in ("accepted", "accept_mask", "out_token", "all_accepted"):
        assert torch.equal(getattr(full, key), getattr(bare, key)), key
    greedy = ss.accept_fused(t, None, inp.tokens.to(dev), temperature=0.0, posterior=False)
    assert torch.equal(greedy.posterior.cpu(), t.float().cpu().argmax(-1))


@pytest.mark.parametrize("V", [64, 4096, 151936])
def test_stochastic_probs_input_vs_oracle(V):
    inp = workloads.accept_inputs(7, B=6, K=15, V=V)
    tp = torch.softmax(inp.target, -1) * 3.0  # unnormalised probabilities
    dp = torch.softmax(inp.draft, -1)
    inp2 = workloads.AcceptInputs(tp, dp, inp.tokens, inp.uniforms, inp.resample_u)
    got, t, d = _run(inp2, 1.0, kind="probs")
    ref = oracle.accept_dense(t.numpy(), d.numpy(), inp.tokens.numpy(), inp.uniforms.numpy(),
                              inp.resample_u.numpy(), kind=oracle.KIND_PROBS)
    _check_stochastic(got, ref, min_certified=0.66)


def test_config0_fixture_seeds_bit_exact():
    """Batch-1 acceptance at V=151936 (T=1) on 32 seeds, each request alone."""
    certified = 0
    for seed in range(32):
        inp = workloads.accept_inputs(seed, B=1, K=15)
        got, t, d = _run(inp, 1.0)
        ref = oracle.accept_dense(t.numpy(), d.numpy(), inp.tokens.numpy(), inp.uniforms.numpy(),
                                  inp.resample_u.numpy(), kind=oracle.KIND_LOGITS, temperature=1.0)
        if ref["u_margin"][0] > U_MARGIN and ref["cdf_margin"][0] > CDF_MARGIN:
            certified += 1
            assert got["accepted"][0] == ref["accepted"][0], seed
            assert got["out_token"][0] == ref["out_token"][0], seed
            np.testing.assert_array_equal(got["accept_mask"][0], ref["accept_mask"][0].astype(bool))
    assert certified >= 28


def test_equal_distributions_accept_all_and_draw_bonus_row():
    V = 5000
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 4, V, generator=g)
    x[:, 3] = -30.0
    x[0, 3, 1234] = 30.0  # bonus row of request 0 is (numerically) one-hot
    inp = workloads.AcceptInputs(x, x[:, :3].clone(), torch.randint(0, V, (2, 3), generator=g),
                                 torch.rand(2, 3, generator=g), torch.rand(2, generator=g))
    got, _, _ = _run(inp, 1.0)
    assert list(got["accepted"]) == [3, 3] and got["all_accepted"].all()
    assert got["out_token"][0] == 1234


def test_bad_draft_token_is_reported_not_read():
    """Stochastic modes index p and q by the draft token: an out-of-range
    token reports the request (-2).  Greedy acceptance only compares the
    token with the argmax (single/eval_sync.py:1223-1234): a mismatch."""
    inp = workloads.accept_inputs(5, B=3, K=4, V=512)
    inp.tokens[1, 2] = 512
    inp.tokens[2, 0] = -1
    got, _, _ = _run(inp, 1.0)
    assert got["out_token"][1] == -2 and got["out_token"][2] == -2
    assert got["out_token"][0] >= 0
    got, t, _ = _run(inp, 0.0)
    ref = oracle.accept_greedy(t.numpy(), inp.tokens.numpy())
    for key in ("accepted", "out_token", "posterior"):
        np.testing.assert_array_equal(got[key], ref[key])
    np.testing.assert_array_equal(got["accept_mask"], ref["accept_mask"].astype(bool))
    assert got["accepted"][2] == 0 and not got["accept_mask"][1][2]


def test_empty_distribution_sentinel():
    V = 300
    t = torch.zeros(1, 2, V)
    d = torch.full((1, 1, V), 1.0 / V)
    inp = workloads.AcceptInputs(t, d, torch.tensor([[7]]), torch.tensor([[0.5]]), torch.tensor([0.5]))
    got, _, _ = _run(inp, 1.0, kind="probs")
    assert got["accepted"][0] == 0 and got["out_token"][0] == -1


def test_u_equal_a_boundary_accepts_on_device():
    V = 4
    t = torch.tensor([[[0.25, 0.75, 0, 0], [0.25, 0.75, 0, 0]]])
    d = torch.tensor([[[0.5, 0.5, 0, 0]]])
    for u, expect in ((0.5, 1), (float(np.nextafter(np.float32(0.5), np.float32(1))), 0)):
        inp = workloads.AcceptInputs(t, d, torch.tensor([[0]]), torch.tensor([[u]]), torch.tensor([0.1]))
        got, _, _ = _run(inp, 1.0, kind="probs")
        assert got["accepted"][0] == expect
        if not expect:
            assert got["out_token"][0] == 1


@pytest.mark.parametrize("K,V", [(1, 8195), (127, 8195), (127, 1000), (15, 1), (3, 4096)])
@pytest.mark.parametrize("T", [0.0, 1.0])
def test_block_length_and_vocabulary_extremes(K, V, T):
    """K = 1 and K = 127 (the maximum: 255 rows merged per request), a
    one-entry vocabulary and a vocabulary of exactly one chunk, greedy and
    T = 1, against the oracle."""
    inp = workloads.accept_inputs(K * 31 + V % 17, B=3, K=K, V=V, temperature=T)
    got, t, d = _run(inp, T)
    if T == 0.0:
        ref = oracle.accept_greedy(t.numpy(), inp.tokens.numpy())
        np.testing.assert_array_equal(got["posterior"], ref["posterior"])
        np.testing.assert_array_equal(got["accepted"], ref["accepted"])
        np.testing.assert_array_equal(got["out_token"], ref["out_token"])
        np.testing.assert_array_equal(got["accept_mask"], ref["accept_mask"].astype(bool))
    else:
        ref = oracle.accept_dense(t.numpy(), d.numpy(), inp.tokens.numpy(), inp.uniforms.numpy(),
                                  inp.resample_u.numpy(), kind=oracle.KIND_LOGITS, temperature=T)
        _check_stochastic(got, ref, min_certified=0.3 if V == 1 else 0.6)
    if V == 1:  # every token is 0 and every draft accepted; the bonus draw is token 0
        assert (got["accepted"] == K).all() and (got["out_token"] == 0).all()


@pytest.mark.parametrize("T", [0.0, 1.0])
def test_workspace_reuse_across_calls_and_shapes(T):
    """One cached workspace serves calls of different sizes in turn (the
    stats launch resets the hand-off records each call): every call agrees
    with the oracle."""
    for B, V in ((8, 151936), (1, 4096), (3, 70000), (8, 151936), (2, 1000)):
        inp = workloads.accept_inputs(B * 7 + V % 13, B=B, K=15, V=V, temperature=T)
        got, t, d = _run(inp, T)
        if T == 0.0:
            ref = oracle.accept_greedy(t.numpy(), inp.tokens.numpy())
            np.testing.assert_array_equal(got["posterior"], ref["posterior"])
            np.testing.assert_array_equal(got["out_token"], ref["out_token"])
        else:
            ref = oracle.accept_dense(t.numpy(), d.numpy(), inp.tokens.numpy(), inp.uniforms.numpy(),
                                      inp.resample_u.numpy(), kind=oracle.KIND_LOGITS, temperature=T)
            _check_stochastic(got, ref, min_certified=0.5)


def test_verify_speculative_block_reference_surface():
    inp = workloads.accept_inputs(9, B=1, K=15)
    dev = _dev()
    p = torch.softmax(inp.target, -1).to(dev)
    q = torch.softmax(inp.draft, -1).to(dev)
    res = ss.verify_speculative_block(inp.tokens.to(dev), p, q, uniforms=inp.uniforms.to(dev),
                                      resample_uniform=inp.resample_u.to(dev))
    ref = oracle.accept_dense(p.cpu().numpy(), q.cpu().numpy(), inp.tokens.numpy(), inp.uniforms.numpy(),
                              inp.resample_u.numpy(), kind=oracle.KIND_PROBS)
    assert ref["u_margin"][0] > U_MARGIN and ref["cdf_margin"][0] > CDF_MARGIN
    assert res.accepted_draft_tokens == ref["accepted"][0]
    assert int(res.correction_token[0]) == ref["out_token"][0]
    assert res.all_accepted == bool(ref["all_accepted"][0])
    assert res.correction_token.shape == (1,) and res.correction_token.dtype == torch.int64
    # reference-style call without uniforms still works
    res2 = ss.verify_speculative_block(inp.tokens.to(dev), p, q)
    assert 0 <= res2.accepted_draft_tokens <= 15
    with pytest.raises(ValueError, match="batch size 1"):
        ss.verify_speculative_block(inp.tokens.repeat(2, 1).to(dev), p.repeat(2, 1, 1), q.repeat(2, 1, 1))


def test_cpu_tensors_are_rejected_loudly():
    inp = workloads.accept_inputs(1, B=1, K=3, V=64)
    with pytest.raises(RuntimeError, match="HIP device"):
        ss.accept_fused(inp.target, inp.draft, inp.tokens, uniforms=inp.uniforms,
                        resample_uniform=inp.resample_u)


def test_graph_replays_match_eager_calls():
    """The acceptance captured in a HIP graph (its workspace owned by the
    graph) gives, on every replay over new inputs copied into the static
    buffers, the eager call's outputs."""
    from d3d_amd import _lib
    dev = _dev()
    B, K, V = 4, 15, 151936
    sets = [workloads.accept_inputs(300 + i, B=B, K=K, V=V, device="cuda") for i in range(4)]
    t = sets[0].target.clone()
    d = sets[0].draft.clone()
    tok = sets[0].tokens.clone()
    u = sets[0].uniforms.clone()
    ru = sets[0].resample_u.clone()

    def body():
        return ss.accept_fused(t, d, tok, temperature=1.0, uniforms=u, resample_uniform=ru)

    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        body()
    torch.cuda.current_stream(dev).wait_stream(side)
    owner: list = []
    g = torch.cuda.CUDAGraph()
    with _lib.capture_workspaces(owner), torch.cuda.graph(g):
        out = body()
    assert owner, "the captured acceptance asked for no workspace"
    for rep in range(8):
        src = sets[rep % len(sets)]
        for dst, x in ((t, src.target), (d, src.draft), (tok, src.tokens), (u, src.uniforms),
                       (ru, src.resample_u)):
            dst.copy_(x)
        g.replay()
        torch.cuda.synchronize()
        got = [x.clone() for x in out]
        want = ss.accept_fused(src.target, src.draft, src.tokens, temperature=1.0, uniforms=src.uniforms,
                               resample_uniform=src.resample_u)
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b), rep
    del g


def test_status_tokens_are_flagged_and_raise_on_check():
    """A draft token outside the vocabulary (-2) and a request without
    probability mass (-1) come back as statuses, flagged by ``valid`` on the
    device, agreeing with the oracle, and ``check()`` raises the reference's
    errors for them; a clean call checks through."""
    from d3d_amd import _lib
    dev = _dev()
    V = 4096
    inp = workloads.accept_inputs(21, B=3, K=15, V=V)
    tokens = inp.tokens.clone()
    tokens[1, 4] = V + 5
    kw = dict(uniforms=inp.uniforms.to(dev), resample_uniform=inp.resample_u.to(dev))
    out = ss.accept_fused(inp.target.to(dev), inp.draft.to(dev), tokens.to(dev), **kw)
    assert out.valid.cpu().tolist() == [True, False, True]
    assert int(out.out_token[1]) == _lib.D3D_TOKEN_BAD_DRAFT
    ref = oracle.accept_dense(inp.target.numpy(), inp.draft.numpy(), tokens.numpy(), inp.uniforms.numpy(),
                              inp.resample_u.numpy(), kind=oracle.KIND_LOGITS, temperature=1.0)
    assert int(ref["out_token"][1]) == _lib.D3D_TOKEN_BAD_DRAFT
    with pytest.raises(ValueError, match="request 1: draft token id outside the vocabulary"):
        out.check()

    p = torch.softmax(inp.target, -1)
    q = torch.softmax(inp.draft, -1)
    p[2] = 0.0  # request 2 has no target mass at all
    out = ss.accept_fused(p.to(dev), q.to(dev), inp.tokens.to(dev), input_kind="probs", **kw)
    assert out.valid.cpu().tolist() == [True, True, False]
    ref = oracle.accept_dense(p.numpy(), q.numpy(), inp.tokens.numpy(), inp.uniforms.numpy(),
                              inp.resample_u.numpy(), kind=oracle.KIND_PROBS)
    assert int(out.out_token[2]) == int(ref["out_token"][2]) == _lib.D3D_TOKEN_EMPTY_DISTRIBUTION
    with pytest.raises(RuntimeError, match="request 2: invalid multinomial distribution"):
        out.check()

    out = ss.accept_fused(inp.target.to(dev), inp.draft.to(dev), inp.tokens.to(dev), **kw)
    assert out.check() is out and bool(out.valid.all())

    # Greedy acceptance only compares tokens with the argmax: the same
    # out-of-range token is a mismatch, decided as the oracle decides it.
    out = ss.accept_fused(inp.target.to(dev), None, tokens.to(dev), temperature=0.0)
    ref = oracle.accept_greedy(inp.target.numpy(), tokens.numpy())
    assert out.check() is out
    np.testing.assert_array_equal(out.accepted.cpu().numpy(), ref["accepted"])
    np.testing.assert_array_equal(out.out_token.cpu().numpy(), ref["out_token"])
    np.testing.assert_array_equal(out.accept_mask.cpu().numpy(), ref["accept_mask"].astype(bool))


def test_sparse_status_tokens_raise_on_check():
    from d3d_amd import _lib
    dev = _dev()
    inp = workloads.sparse_accept_inputs(22, B=2, K=15, V=4096, S=16)
    tokens = inp.tokens.clone()
    tokens[0, 0] = -7
    out = ss.accept_fused_sparse(torch.softmax(inp.target, -1).to(dev), tokens.to(dev), inp.q_ids.to(dev),
                                 inp.q_probs.to(dev), uniforms=inp.uniforms.to(dev),
                                 resample_uniform=inp.resample_u.to(dev))
    assert int(out.out_token[0]) == _lib.D3D_TOKEN_BAD_DRAFT and bool(out.valid[1])
    with pytest.raises(ValueError, match="request 0: draft token id outside the vocabulary"):
        out.check()
