"""End-to-end greedy speculative loop (GPU), called as serving/bench.py calls it.

Greedy speculative decoding is lossless: whatever the draft proposes, each
committed token is the target's greedy token given the tokens before it.
Checks:

* teacher forcing against the fp32 CPU restatement of the target: every
  token is the restatement's argmax wherever its top-2 logit margin
  exceeds 5 % of the logit standard deviation (closer margins are near ties
  that bf16 rounding may decide either way), on at least half the
  positions;
* equality with target-only greedy decoding on the same HIP model
  (generate_ar, serving/baseline_concurrency.py), up to a first divergence
  that must sit at such a near tie;
* the reference's Engine surface: positional ``concurrency``, admission
  capped at it, ragged prompts, EOS stops, the ``fast`` / ``fast_legacy``
  backups, ``_predict``'s outcome dictionary and ``_verify`` against
  ``_accepted`` on the target's posterior; no page leaks.
"""
from __future__ import annotations

import pytest
import torch

from d3d_amd.engine import Engine, generate_ar
from d3d_amd.model import ModelShape
from oracle import model_ref

pytestmark = pytest.mark.gpu

TARGET = ModelShape(layers=2, hidden=256, heads=8, kv_heads=2, head_dim=128, mlp=512, vocab=1000)
DRAFT = ModelShape(layers=1, hidden=256, heads=4, kv_heads=2, head_dim=128, mlp=256, vocab=1000)


def _engine(seed, **kw):
    eng = Engine(TARGET, DRAFT, pages=16, seed=seed, mask_id=999, **kw)
    for r in (eng.target, eng.draft):
        r.model.lm_head.mul_(20.0)  # logits with std ~6: top-2 margins far above rounding
    return eng


def _near_tie(W, prompt, tokens, i):
    """Is the target's top-2 margin at generated position i a near tie?"""
    ids = list(prompt) + list(tokens[:i])
    T = len(ids)
    logits = model_ref.forward(W, TARGET, torch.tensor(ids), torch.arange(T), torch.ones(T, T).tril().bool())[-1]
    top2 = logits.topk(2).values
    return float(top2[0] - top2[1]) <= 0.05 * float(logits.std())


def _same_up_to_near_tie(W, prompts, a, b):
    for p, x, y in zip(prompts, a, b):
        if x == y:
            continue
        i = next(j for j in range(min(len(x), len(y))) if x[j] != y[j])
        assert _near_tie(W, p, x, i), f"outputs diverge at a decisive position {i}"


def test_engine_output_is_target_greedy_decoding():
    eng = _engine(7)
    g = torch.Generator().manual_seed(3)
    prompts = torch.randint(0, 999, (2, 32), generator=g).tolist()
    new = 40
    res = eng.generate(prompts, 2, max_new_tokens=new, ignore_eos=True)
    assert [len(o["tokens"]) for o in res["outputs"]] == [new, new]
    assert res["steps"] >= 1 and 0.0 <= res["overlap_fraction"] <= 1.0
    assert res["target_active_sequences"] == 0 and res["target_free_pages"] == eng.target.kv.num_pages
    W = model_ref.weights_fp32(eng.target.model)
    for o, p in zip(res["outputs"], prompts):
        ids = list(p)
        decisive = 0
        for t in o["tokens"]:
            T = len(ids)
            logits = model_ref.forward(W, TARGET, torch.tensor(ids), torch.arange(T),
                                       torch.ones(T, T).tril().bool())[-1]
            top2 = logits.topk(2).values
            if float(top2[0] - top2[1]) > 0.05 * float(logits.std()):
                assert t == int(logits.argmax()), f"token {T - len(p)} differs from greedy decoding"
                decisive += 1
            ids.append(t)  # teacher forcing with the engine's own tokens
        assert decisive >= new // 2
    ar = generate_ar(eng.target, prompts, 2, new, ignore_eos=True)
    _same_up_to_near_tie(W, prompts, [o["tokens"] for o in ar["outputs"]], [o["tokens"] for o in res["outputs"]])


def test_graph_replay_matches_eager_engine():
    """Every step replayed from HIP graphs gives the eager run's tokens."""
    outs = []
    for graphs in (False, True):
        eng = _engine(11, use_graphs=graphs)
        g = torch.Generator().manual_seed(4)
        prompts = torch.randint(0, 999, (3, 48), generator=g).tolist()
        res = eng.generate(prompts, 3, max_new_tokens=30, ignore_eos=True)
        outs.append([o["tokens"] for o in res["outputs"]])
        # a second run on the same engine replays the cached graphs again
        res2 = eng.generate(prompts, 3, max_new_tokens=30, ignore_eos=True)
        assert [o["tokens"] for o in res2["outputs"]] == outs[-1]
    assert outs[0] == outs[1]


def test_admission_ragged_prompts_and_eos():
    """Five prompts of lengths 1..45 at concurrency 2: no more than two run
    at once, every prompt is served in index order of the outputs; an EOS
    id stops a request right after it (inclusive) and the rest keep going."""
    eng = _engine(13)
    g = torch.Generator().manual_seed(5)
    lens = [1, 17, 45, 16, 30]
    prompts = [torch.randint(0, 999, (n,), generator=g).tolist() for n in lens]
    res = eng.generate(prompts, 2, max_new_tokens=24, ignore_eos=True)
    assert res["max_active"] <= 2 and max(res["decode_batch_sizes"]) <= 2
    assert [o["index"] for o in res["outputs"]] == list(range(5))
    assert all(len(o["tokens"]) == 24 for o in res["outputs"])
    W = model_ref.weights_fp32(eng.target.model)
    ar = generate_ar(eng.target, prompts, 2, 24, ignore_eos=True)
    _same_up_to_near_tie(W, prompts, [o["tokens"] for o in ar["outputs"]], [o["tokens"] for o in res["outputs"]])
    first = res["outputs"][2]["tokens"]
    stop = first[5]
    j = first.index(stop)  # the first occurrence ends the request
    res2 = eng.generate(prompts, 2, max_new_tokens=24, ignore_eos=False, eos=(stop,))
    out2 = res2["outputs"][2]["tokens"]
    assert out2 == first[:j + 1]
    for o in res2["outputs"]:
        assert stop not in o["tokens"][:-1]


@pytest.mark.parametrize("backup", ["fast", "fast_legacy"])
def test_fast_backups_stay_lossless(backup):
    """Random backup blocks change what is verified, not what is committed."""
    g = torch.Generator().manual_seed(6)
    prompts = torch.randint(0, 999, (3, 20), generator=g).tolist()
    ref = _engine(17)
    want = ref.generate(prompts, 3, max_new_tokens=20, ignore_eos=True)
    eng = _engine(17, backup=backup, fast_miss_anchors=2 if backup == "fast" else 0)
    got = eng.generate(prompts, 3, max_new_tokens=20, ignore_eos=True)
    assert got["backup"] == backup
    assert sum(o["fast_backups"] for o in got["outputs"]) >= 1
    W = model_ref.weights_fp32(eng.target.model)
    _same_up_to_near_tie(W, prompts, [o["tokens"] for o in want["outputs"]], [o["tokens"] for o in got["outputs"]])


def test_all_accepted_blocks_continue_from_the_hit_branch():
    """With both LM heads zeroed every logit is 0 and every greedy token is
    id 0 (the first maximum): the target accepts every drafted token, the
    packed prediction's all-accepted branch matches the verify, and
    generate continues from that branch's block (a hit) instead of a
    recovery forward.  The output is still the target's greedy decoding."""
    eng = _engine(31)
    for r in (eng.target, eng.draft):
        r.model.lm_head.zero_()
    prompts = torch.randint(0, 999, (3, 20), generator=torch.Generator().manual_seed(3)).tolist()
    res = eng.generate(prompts, 3, max_new_tokens=40, ignore_eos=True)
    assert all(o["tokens"] == [0] * 40 for o in res["outputs"])
    assert all(o["hits"] >= 1 for o in res["outputs"])
    ar = generate_ar(eng.target, prompts, 3, 40, ignore_eos=True)
    assert [o["tokens"] for o in ar["outputs"]] == [o["tokens"] for o in res["outputs"]]


def test_a_dropped_engine_frees_its_graphs_by_reference_counting():
    """Runners and their captured steps form no reference cycle: dropping
    an engine frees its graphs at once, with the cyclic collector off, so no
    collection pass meets them later in the middle of another capture."""
    import gc
    import weakref
    eng = _engine(19)
    prompts = torch.randint(0, 999, (2, 20), generator=torch.Generator().manual_seed(8)).tolist()
    eng.generate(prompts, 2, max_new_tokens=8, ignore_eos=True)
    steps = [st for r in (eng.target, eng.draft) for st in r._steps.values()]
    assert steps and all(st.graph is not None for st in steps)
    refs = [weakref.ref(o) for o in (eng, eng.target, eng.draft, *steps)]
    torch.cuda.synchronize()
    was_enabled = gc.isenabled()
    gc.disable()
    try:
        del steps, eng
        assert [r() is None for r in refs] == [True] * len(refs)
    finally:
        if was_enabled:
            gc.enable()


def test_engines_share_one_dedicated_stream_per_role():
    """Engines built one after another reuse the process's two dedicated
    streams (one hardware queue each) instead of adding two per engine, and
    interleaved use of two engines on the shared streams gives each the
    outputs it gives alone."""
    a, b = _engine(41), _engine(43)
    assert a.target.stream.cuda_stream == b.target.stream.cuda_stream
    assert a.draft.stream.cuda_stream == b.draft.stream.cuda_stream
    assert a.target.stream.cuda_stream != a.draft.stream.cuda_stream
    prompts = torch.randint(0, 999, (2, 24), generator=torch.Generator().manual_seed(5)).tolist()
    first = [o["tokens"] for o in a.generate(prompts, 2, max_new_tokens=12, ignore_eos=True)["outputs"]]
    other = [o["tokens"] for o in b.generate(prompts, 2, max_new_tokens=12, ignore_eos=True)["outputs"]]
    again = [o["tokens"] for o in a.generate(prompts, 2, max_new_tokens=12, ignore_eos=True)["outputs"]]
    alone = [o["tokens"] for o in _engine(43).generate(prompts, 2, max_new_tokens=12, ignore_eos=True)["outputs"]]
    assert again == first and other == alone


def test_predict_and_verify_surfaces():
    """_predict returns {seq_id: {(n, anchor or None): (block, top)}} with A
    branches per accepted count and the all-accepted one; _verify equals
    _accepted on the target's greedy posterior."""
    from d3d_amd.model import Sequence
    eng = _engine(19, anchor_num=2)
    g = torch.Generator().manual_seed(7)
    seqs = []
    for i, n in enumerate((20, 33)):
        s = Sequence(i, torch.randint(0, 999, (n,), generator=g).tolist())
        s.prefix = n
        s.needs_fast_seed = False
        s.recoveries = 0
        seqs.append(s)
    anchors = eng.target.prefill(seqs)
    eng.draft.prefill(seqs)
    for s, a in zip(seqs, anchors):
        s.anchor = a
    eng._recover(seqs)
    assert all(len(s.current) == 16 and s.current[0] == s.anchor and len(s.top) == 16 for s in seqs)
    pred = eng._predict(seqs)
    for s in seqs:
        keys = list(pred[s.seq_id])
        assert len(keys) == 2 * 15 + 1 and keys[-1] == (16, None)
        for (n, a), (block, top) in pred[s.seq_id].items():
            assert len(block) == 16 and len(top) == 16 and len(top[0]) == 3
            if a is not None:
                assert block[0] == a and a != s.current[n]
    blocks = [list(s.current) for s in seqs]
    got = eng._verify(seqs, blocks)
    posterior = eng.target.forward(seqs, blocks).cpu().tolist()
    assert got == Engine._accepted(blocks, posterior)
    for s in seqs:
        eng.target.release(s)
        eng.draft.release(s)
    assert eng.target.free_pages == eng.target.kv.num_pages and eng.draft.free_pages == eng.draft.kv.num_pages


@pytest.mark.parametrize("lens,every", [((21, 34, 27), 1), ((21, 34, 27, 40, 18, 25), 2)])
def test_lazy_hit_branches_equal_the_full_prediction(lens, every):
    """The engine keeps the packed prediction's hidden states and turns only
    the branches the verify hits into tokens (_predict_hits): for every
    branch key of every request, those tokens equal _predict's (every
    branch through the LM head at once) -- block with the anchor in its
    first slot, and top-(A+1).  Six requests make two prediction groups of
    the four-request micro-batch, with hits in only some of the requests."""
    from d3d_amd.model import Sequence
    eng = _engine(29, anchor_num=2)
    g = torch.Generator().manual_seed(13)
    seqs = []
    for i, n in enumerate(lens):
        s = Sequence(i, torch.randint(0, 999, (n,), generator=g).tolist())
        s.prefix = n
        s.needs_fast_seed = False
        s.recoveries = s.hits = 0
        seqs.append(s)
    anchors = eng.target.prefill(seqs)
    eng.draft.prefill(seqs)
    for s, a in zip(seqs, anchors):
        s.anchor = a
    eng._recover(seqs)
    saved = [(list(s.current), [list(t) for t in s.top]) for s in seqs]
    full = eng._predict(seqs)
    pending = eng._predict_submit(seqs, lazy=True)
    specs = {s.seq_id: e[1][b] for e in pending for b, s in enumerate(e[0])}
    checked = 0
    if len(lens) > eng.micro:
        assert len(pending) == 2
    for j in range(2 * 15 + 1):  # every branch position, one key per hit request each round
        hitting = [i for i in range(len(seqs)) if (i + j) % every == 0]
        hits = []
        for i in hitting:
            s = seqs[i]
            key = specs[s.seq_id][j]
            hits.append((s, key, key[1] if key[1] is not None else 123))
        out = eng._predict_hits(pending, hits)
        eng._apply_hits(hits, out)
        for i, (s, key, anchor) in zip(hitting, hits):
            cur, top = saved[i]
            block, want_top = full[s.seq_id][key]
            want = list(block)
            want[0] = anchor
            assert s.current == want and s.top == want_top, (s.seq_id, key)
            s.current, s.top = list(cur), [list(t) for t in top]
            checked += 1
        for i in set(range(len(seqs))) - set(hitting):  # a request that missed keeps its block
            assert (seqs[i].current, seqs[i].top) == saved[i]
    assert checked == sum(1 for j in range(31) for i in range(len(seqs)) if (i + j) % every == 0)
    for s in seqs:
        eng.target.release(s)
        eng.draft.release(s)


def test_prepared_block_inputs_are_used_only_while_they_hold():
    """Runner.prepare fills a step's block inputs ahead of its forward: a
    verify and a packed prediction on prepared inputs equal the same calls
    without them, and after a prefix moves (or a table is trimmed) the
    forward prepares again instead of using the stale inputs."""
    from d3d_amd.model import Sequence
    eng = _engine(23)
    g = torch.Generator().manual_seed(11)
    seqs = []
    for i, n in enumerate((19, 40, 26)):
        s = Sequence(i, torch.randint(0, 999, (n,), generator=g).tolist())
        s.prefix = n
        s.needs_fast_seed = False
        s.recoveries = 0
        seqs.append(s)
    anchors = eng.target.prefill(seqs)
    eng.draft.prefill(seqs)
    for s, a in zip(seqs, anchors):
        s.anchor = a
    eng._recover(seqs)
    blocks = [list(s.current) for s in seqs]

    def verify():
        out = eng.target.verify(seqs, blocks)
        eng.target.stream.synchronize()
        return out.tolist()

    def predict():
        return eng._predict(seqs)

    plain_v, plain_p = verify(), predict()
    eng._prepare_next(seqs)
    assert verify() == plain_v and predict() == plain_p
    # stale: the prefixes move after the preparation (the engine's trim and
    # next reserve happen in between), so both forwards prepare again
    eng._prepare_next(seqs)
    for s in seqs:
        s.prefix += 1
        eng.target.trim(s, s.prefix)
        eng.draft.trim(s, s.prefix)
    moved_v, moved_p = verify(), predict()
    eng._prepare_next(seqs)
    assert verify() == moved_v and predict() == moved_p
    assert moved_v != plain_v or moved_p != plain_p
    for s in seqs:
        eng.target.release(s)
        eng.draft.release(s)
    assert eng.target.free_pages == eng.target.kv.num_pages and eng.draft.free_pages == eng.draft.kv.num_pages


def test_generic_mask_builder_equals_descriptor():
    """Runner.forward compiles a plain mask callable (the reference's
    Engine._mask closure) to the same per-query visibility the engine's
    builder carries."""
    from d3d_amd.model import Sequence
    eng = _engine(23, anchor_num=1)
    g = torch.Generator().manual_seed(8)
    seqs = []
    for i in range(2):
        s = Sequence(i, torch.randint(0, 999, (40,), generator=g).tolist())
        seqs.append(s)
    eng.draft.prefill(seqs)
    K = 16
    specs = [[(n, 5) for n in range(1, K)] + [(K, None)]] * 2
    Q = K * (1 + len(specs[0]))
    ids = torch.randint(0, 999, (2, Q), generator=g)
    builder = eng._mask(specs)
    a_top, a_g = eng.draft.forward(seqs, ids, mask_builder=builder, topk=2)

    def plain(starts, Q_, S):
        return builder(starts, Q_, S)

    b_top, b_g = eng.draft.forward(seqs, ids, mask_builder=plain, topk=2)
    assert torch.equal(a_top, b_top) and torch.equal(a_g, b_g)


@pytest.mark.parametrize("side,entry", [("target", "d3d_accept_fused"), ("draft", "d3d_topk_rows")])
def test_failed_launch_on_either_stream_raises(side, entry):
    """A launch that fails on the verify (target) or the draft stream -- the
    library call reports a HIP error on the third call -- surfaces from
    generate as RuntimeError naming the side, after both streams drain
    (the in-process form of serving/target_process.py:82-96)."""
    from d3d_amd import _lib
    eng = _engine(29, use_graphs=False)
    lib = _lib.load()
    real = getattr(lib, entry)
    calls = {"n": 0}

    def failing(*args):
        calls["n"] += 1
        return 98 if calls["n"] == 3 else real(*args)  # 98: hipErrorInvalidDeviceFunction

    setattr(lib, entry, failing)
    try:
        prompts = torch.randint(0, 999, (2, 20), generator=torch.Generator().manual_seed(9)).tolist()
        with pytest.raises(RuntimeError, match=f"{side} step failed"):
            eng.generate(prompts, 2, max_new_tokens=10, ignore_eos=True)
    finally:
        setattr(lib, entry, real)
    torch.cuda.synchronize()
    # The library is usable again afterwards.
    ok = _engine(29, use_graphs=False).generate([[1, 2, 3]], 1, max_new_tokens=4, ignore_eos=True)
    assert len(ok["outputs"][0]["tokens"]) == 4
