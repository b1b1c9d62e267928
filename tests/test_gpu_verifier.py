"""Target verify step (GPU): forward + acceptance against the oracle.

single/eval_async_packed.py:115-199.  The target logits are checked against
the fp32 restatement (model tolerance); the acceptance is checked against
the fp64 oracle on the same logits: bit-exact for greedy, bit-exact where
the oracle certifies the margins for the sampled modes.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from d3d_amd import verifier
from d3d_amd.model import ModelShape, PagedKV, Qwen3PagedModel, Sequence, prefill
from oracle import model_ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TINY = ModelShape(layers=2, hidden=256, heads=8, kv_heads=2, head_dim=128, mlp=512, vocab=1000)


def _setup(seed, B=3):
    model = Qwen3PagedModel(TINY, DEV, draft=False, seed=seed, init_std=0.05)
    model.lm_head.mul_(8.0)
    kv = PagedKV(TINY, 64, 16, DEV)
    g = torch.Generator().manual_seed(seed)
    prompts = torch.randint(0, 1000, (B, 32), generator=g)
    seqs = [Sequence(i, p.tolist()) for i, p in enumerate(prompts)]
    prefill(model, kv, seqs, "target")
    return model, kv, seqs, prompts, g


def test_greedy_verify_step():
    model, kv, seqs, prompts, g = _setup(1)
    blocks = torch.randint(0, 1000, (3, 16), generator=g)
    res = verifier.verify_step(model, kv, seqs, blocks.to(DEV), return_logits=True)
    lg = res.logits.float().cpu()
    W = model_ref.weights_fp32(model)
    for b in range(3):
        ids = torch.cat([prompts[b], blocks[b]])
        ref = model_ref.forward(W, TINY, ids, torch.arange(48), torch.ones(48, 48).tril().bool())[32:]
        assert float((lg[b] - ref).abs().max()) <= 5e-2 * float(ref.abs().max())
    ref = oracle.accept_greedy(lg.numpy(), blocks[:, 1:].numpy())
    np.testing.assert_array_equal(res.posterior.cpu().numpy(), ref["posterior"])
    np.testing.assert_array_equal(res.accepted_tail.cpu().numpy(), ref["accepted"])
    np.testing.assert_array_equal(res.correction_token.cpu().numpy(), ref["out_token"])


def test_greedy_accepts_the_targets_own_tokens():
    """A block whose tail is the target's greedy continuation is fully accepted."""
    model, kv, seqs, prompts, g = _setup(2, B=1)
    block = torch.randint(0, 1000, (1, 16), generator=g)
    res = verifier.verify_step(model, kv, seqs, block.to(DEV))
    post = res.posterior.cpu()
    # Feed the posterior back: block[i + 1] = posterior[i] for every i.
    for _ in range(16):
        block[0, 1:] = post[0, :-1]
        res = verifier.verify_step(model, kv, seqs, block.to(DEV))
        if torch.equal(res.posterior.cpu(), post):
            break
        post = res.posterior.cpu()
    assert int(res.accepted_tail[0]) == 15 and int(res.correction_token[0]) == int(post[0, 15])


@pytest.mark.parametrize("kind", ["sparse", "dense"])
def test_sampled_verify_step(kind):
    model, kv, seqs, prompts, g = _setup(3, B=6)
    T, S, V = 0.9, 16, 1000
    blocks = torch.randint(0, V, (6, 16), generator=g)
    dl = (torch.randn(6, 15, V, generator=g) * 3).bfloat16().float()  # the model's logits dtype
    q_ids = torch.topk(dl, S, -1).indices
    q_probs = torch.softmax(torch.topk(dl, S, -1).values / T, -1)
    blocks[:, 1:] = q_ids[:, :, 0]  # draft tokens from the proposal support
    u = torch.rand(6, 15, generator=g)
    ru = torch.rand(6, generator=g)
    kw = dict(temperature=T, uniforms=u.to(DEV), resample_uniform=ru.to(DEV), return_logits=True)
    if kind == "sparse":
        res = verifier.verify_step(model, kv, seqs, blocks.to(DEV), draft_token_ids=q_ids.to(DEV),
                                   draft_token_probs=q_probs.to(DEV), **kw)
    else:
        res = verifier.verify_step(model, kv, seqs, blocks.to(DEV), draft_logits=dl.to(DEV), **kw)
    lg = res.logits.float().cpu().numpy()
    if kind == "sparse":
        ref = oracle.accept_sparse(lg, blocks[:, 1:].numpy(), q_ids.numpy(), q_probs.numpy(), u.numpy(),
                                   ru.numpy(), kind=oracle.KIND_LOGITS, temperature=T)
    else:
        ref = oracle.accept_dense(lg, dl.numpy(), blocks[:, 1:].numpy(), u.numpy(), ru.numpy(),
                                  kind=oracle.KIND_LOGITS, temperature=T)
    ok = (ref["u_margin"] > 1e-5) & (ref["cdf_margin"] > 1e-6)
    assert ok.mean() >= 0.5
    np.testing.assert_array_equal(res.accepted_tail.cpu().numpy()[ok], ref["accepted"][ok])
    np.testing.assert_array_equal(res.correction_token.cpu().numpy()[ok], ref["out_token"][ok])
    np.testing.assert_array_equal(res.posterior.cpu().numpy(), lg.argmax(-1))


def test_sampled_verify_needs_a_proposal():
    model, kv, seqs, prompts, g = _setup(4, B=1)
    with pytest.raises(RuntimeError, match="requires sparse draft q"):
        verifier.verify_step(model, kv, seqs, torch.zeros(1, 16, dtype=torch.int64, device=DEV), temperature=1.0)


def test_verify_step_rejects_out_of_vocabulary_draft_tokens():
    """The check runs before the forward: the embedding never sees the id."""
    model, kv, seqs, prompts, g = _setup(5, B=2)
    blocks = torch.randint(0, 1000, (2, 16), generator=g)
    blocks[1, 7] = 1000 + 3
    with pytest.raises(ValueError, match="draft token id outside the vocabulary"):
        verifier.verify_step(model, kv, seqs, blocks.to(DEV), temperature=0.9,
                             draft_logits=torch.zeros(2, 15, 1000, device=DEV))


def test_verify_step_raises_for_acceptance_statuses(monkeypatch):
    """verify_step reads the acceptance's statuses: an empty distribution
    (-1) raises the reference's multinomial error; with check=False the
    status is handed back in correction_token."""
    from d3d_amd import _lib
    from d3d_amd import speculative_sampling as ss
    real = ss.accept_fused

    def with_status(*a, **k):
        out = real(*a, **k)
        out.out_token[1] = _lib.D3D_TOKEN_EMPTY_DISTRIBUTION
        return out

    monkeypatch.setattr(ss, "accept_fused", with_status)
    model, kv, seqs, prompts, g = _setup(6, B=3)
    blocks = torch.randint(0, 1000, (3, 16), generator=g).to(DEV)
    dl = torch.randn(3, 15, 1000, generator=g).to(DEV)
    with pytest.raises(RuntimeError, match="request 1: invalid multinomial distribution"):
        verifier.verify_step(model, kv, seqs, blocks, temperature=0.9, draft_logits=dl)
    res = verifier.verify_step(model, kv, seqs, blocks, temperature=0.9, draft_logits=dl, check=False)
    assert int(res.correction_token[1]) == _lib.D3D_TOKEN_EMPTY_DISTRIBUTION
    assert bool((res.correction_token[[0, 2]] >= 0).all())
