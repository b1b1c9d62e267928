"""Greedy speculative engine with the target and the draft on one GPU.

Mirrors serving/engine.py:14-227 (the concurrent greedy engine) with the
same constructor, methods and result dictionary:

* ``Engine(target, draft, block_size=16, anchor_num=3, draft_microbatch=4,
  pages=512, backup="neural", seed=42, fast_miss_anchors=0,
  draft_pages=None)`` -- :15-31;
* ``_mask(specs)`` -- :35-52, the draft's recovery / packed mask builder
  (it also carries the per-query visibility descriptor the kernels read);
* ``_recover(seqs)`` -- :54-62, anchor + masks from the committed prefix;
* ``_fast_backup(seqs)`` -- :64-71, random blocks for the "fast" backups;
* ``_predict(seqs)`` -- :73-131, the packed multi-branch prediction:
  ``{seq_id: {(n, anchor or None): (block, top)}}``;
* ``_verify(seqs, blocks)`` / ``_accepted`` -- :133-145;
* ``generate(prompts, concurrency, max_new_tokens=256, ignore_eos=False,
  eos=(151643, 151645))`` -- :147-227, admission capped at
  ``concurrency``, prefill in groups of 4, EOS and length stops, page
  release and the leak checks.

Keywords past the reference's (``device``, ``page_size``, ``mask_id``,
``use_graphs``, ``tuned_gemms``) choose the device, the KV page size, the
draft's mask id, whether steps replay HIP graphs, and whether the step's
library GEMMs use the solution choices in gemm_tuned_gfx950.csv
(``tuned_gemms=True``, off by default: gemm_tuning.enable turns on
TunableOp, a process-wide torch switch, and ``close()`` turns it back; a
no-op where the file's library versions or GPU do not match).

The reference runs the target in another process on another GPU
(serving/target_process.py) and exchanges token lists over a pipe; here
both models are co-resident, each Runner on its own HIP stream (its own
hardware queue), so the target's verify and the draft's packed prediction
overlap, and the exchange is a pair of stream events plus small pinned
device-to-host copies.  The packed prediction keeps its final hidden
states; once the verify result is known only the branches it hits (one per
request at most) go through the draft's LM head and top-k, queued on the
target's stream beside the recovery forward (which needs the prediction's
K/V, not its tokens).  ``_predict`` still returns every branch.  Verify fuses the greedy acceptance kernel after
the target forward (commit length and anchor come back, not the posterior
list); its results equal Engine._accepted on the posterior.
"""
from __future__ import annotations

import time
from functools import lru_cache
from typing import Dict, List, Optional, Sequence as Seq, Tuple

import numpy as np
import torch

from . import gemm_tuning
from .attention import packed_visibility
from .backend import MASK_ID, Runner, SamplingParams
from .model import Sequence

EOS_IDS = (151643, 151645)


def branch_specs(K: int, A: int, current: List[int], top: List[List[int]], shallow: bool = False,
                 fanout: Optional[int] = None) -> List[Tuple[int, Optional[int]]]:
    """Engine._predict's branches for one request (serving/engine.py:96-105):
    for each accepted count n in 1..K-1 (only n = 1 when ``shallow``) the
    first ``fanout`` (default A) tokens of the draft's top list at position n
    that differ from current[n], then -- unless shallow -- the all-accepted
    branch (K, None)."""
    fanout = A if fanout is None else fanout
    out: List[Tuple[int, Optional[int]]] = []
    for n in (range(1, 2) if shallow else range(1, K)):
        anchors = [v for v in top[n] if v != current[n]][:fanout]
        if len(anchors) != fanout:
            raise RuntimeError("draft top-k holds fewer alternative anchors than the fan-out")
        out.extend((n, a) for a in anchors)
    if not shallow:
        out.append((K, None))
    return out


@lru_cache(maxsize=64)
def _packed_visibility(K: int, accepted: Tuple[int, ...]) -> torch.Tensor:
    """packed_visibility for one branch layout, built once (the engine
    repeats a handful of layouts every step); callers only read it."""
    return packed_visibility(K, accepted)


class _Mask:
    """Engine._mask's builder (serving/engine.py:35-52).

    Called as ``builder(starts, Q, S)`` it returns the reference's
    [B, 1, Q, S] bool mask; ``visibility(Q)`` gives the same mask as the
    per-query descriptor [Q, 3] the packed attention kernel reads.
    """

    def __init__(self, K: int, specs=None):
        self.K, self.specs = K, specs

    def _accepted(self) -> Optional[List[int]]:
        if self.specs is None:
            return None
        counts = [n for n, _ in self.specs[0]]
        if any([n for n, _ in sp] != counts for sp in self.specs):
            raise ValueError("packed branch layouts differ between requests of one microbatch")
        return counts

    def visibility(self, Q: int) -> torch.Tensor:
        acc = self._accepted()
        if acc is None:
            return torch.tensor([[Q, 0, 0]] * Q, dtype=torch.int32)
        vis = _packed_visibility(self.K, tuple(acc))
        if vis.shape[0] != Q:
            raise ValueError("packed block length does not match the branch specs")
        return vis

    def __call__(self, starts: torch.Tensor, Q: int, S: int) -> torch.Tensor:
        dev = starts.device
        cols = torch.arange(S, device=dev)[None, None, :].expand(len(starts), -1, -1)
        pref = starts[:, None, None]
        local = cols - pref
        if self.specs is None:
            mask = (cols < pref + Q).expand(-1, Q, -1).clone()
        else:
            K = self.K
            mask = torch.zeros(len(starts), Q, S, dtype=torch.bool, device=dev)
            rows = torch.arange(K, device=dev)[None, :, None]
            mask[:, :K] = (cols < pref) | ((local >= 0) & (local <= rows))
            for b, branches in enumerate(self.specs):
                for j, (accepted, _anchor) in enumerate(branches):
                    off = K + j * K
                    mask[b, off:off + K] = (cols[b] < pref[b] + accepted) | ((local[b] >= off) & (local[b] < off + K))
        return mask[:, None]


class Engine:
    def __init__(self, target, draft, block_size: int = 16, anchor_num: int = 3, draft_microbatch: int = 4,
                 pages: int = 512, backup: str = "neural", seed: int = 42, fast_miss_anchors: int = 0,
                 draft_pages: Optional[int] = None, *, device: str = "cuda:0", page_size: int = 16,
                 mask_id: int = MASK_ID, use_graphs: bool = True, tuned_gemms: bool = False):
        if backup not in ("neural", "fast", "fast_legacy"):
            raise ValueError(backup)
        if anchor_num < 1:
            raise ValueError("anchor_num must be positive")
        if fast_miss_anchors < 0:
            raise ValueError("fast_miss_anchors must be nonnegative")
        if draft_microbatch < 1:
            raise ValueError("draft_microbatch must be positive")
        # generate sizes every page table for at least this many tokens per
        # request (prompt + output), so that the graphs one call captures
        # (keyed by table width) serve a later, longer call too.
        self.min_table_tokens = 0
        self.fast_miss_anchors = fast_miss_anchors
        self.backup, self.seed = backup, seed
        self.K, self.A, self.micro = block_size, anchor_num, draft_microbatch
        self.mask_id = mask_id
        self.device = torch.device(device)
        # tuned_gemms: the step's library GEMMs (packed-predict projections,
        # LM heads, the 64-row target qkv and gate-ups) on the shipped
        # TunableOp choices.  TunableOp is a process-wide torch switch that
        # would also reach the caller's own GEMMs of those shapes, so it is
        # opt-in, and close() puts the switches back as they were.
        self._tunable_saved = gemm_tuning.state() if tuned_gemms else None
        self.tuned_gemms = gemm_tuning.enable() if tuned_gemms else False
        self.target = Runner(target, self.device, pages=pages, page_size=page_size, seed=seed,
                             use_graphs=use_graphs)
        self.draft = Runner(draft, self.device, draft=True, pages=pages if draft_pages is None else draft_pages,
                            page_size=page_size, seed=seed + 1, use_graphs=use_graphs)
        if self.target.shape.vocab != self.draft.shape.vocab:
            raise ValueError("target and draft vocabularies must match")
        if not 0 <= mask_id < self.draft.shape.vocab:
            raise ValueError(f"mask id {mask_id} outside the draft vocabulary")

    def close(self) -> None:
        """Wait for both streams; undo the TunableOp switch ``tuned_gemms``
        turned on."""
        torch.cuda.synchronize(self.device)
        if self._tunable_saved is not None:
            gemm_tuning.restore(self._tunable_saved)
            self._tunable_saved = None
            self.tuned_gemms = False

    # -- failure propagation ---------------------------------------------------
    def _drain(self) -> None:
        """Wait for both streams, ignoring their errors (a failed step is
        being reported already)."""
        for r in (self.target, self.draft):
            try:
                r.stream.synchronize()
            except Exception:
                pass

    def _side(self, side: str, fn, *args, **kw):
        """Run one side's call; a failure there (a launch or argument error,
        or a host error around it) drains both streams and surfaces as a
        RuntimeError naming the side, as the reference's target worker
        errors do (serving/target_process.py:82-96)."""
        try:
            return fn(*args, **kw)
        except Exception as exc:
            self._drain()
            raise RuntimeError(f"{side} step failed: {exc}") from exc

    def _mask(self, specs=None) -> _Mask:
        return _Mask(self.K, specs)

    # -- draft side ------------------------------------------------------------
    def _recover_submit(self, seqs: List[Sequence], topk: int):
        """Recovery forwards (serving/engine.py:54-62) on the draft stream:
        per microbatch the device (top, greedy) of anchor + K-1 masks."""
        out = []
        for off in range(0, len(seqs), self.micro):
            group = seqs[off:off + self.micro]
            ids = torch.full((len(group), self.K), self.mask_id, dtype=torch.long)
            ids[:, 0] = torch.tensor([s.anchor for s in group])
            top, greedy = self.draft.forward(group, ids, mask_builder=self._mask(), topk=topk, host=True)
            out.append((group, top, greedy))
        return out

    def _recover(self, seqs: List[Sequence]) -> None:
        """serving/engine.py:54-62: s.current = [anchor, draft greedy ...], s.top = top-(A+1)."""
        out = self._recover_submit(seqs, self.A + 1)
        self.draft.stream.synchronize()
        self._apply_recovered(out)

    @staticmethod
    def _apply_recovered(out) -> None:
        """Adopt finished recovery forwards (their host copies complete)."""
        for group, top, greedy in out:
            for s, blk, t in zip(group, greedy.tolist(), top.tolist()):
                blk[0] = s.anchor
                s.current, s.top = blk, t
                s.recoveries += 1

    def _prepare_next(self, seqs: List[Sequence]) -> None:
        """Page tables, slots and context lengths of the next step's verify
        and packed prediction, filled while this step's recovery runs (the
        prefixes are final once the verify result is applied).  The packed
        layout (accepted count per branch) does not depend on the tokens.
        Skipped where the next prediction seeds fast backups (other
        layouts); a layout that does not match is prepared again."""
        K, A = self.K, self.A
        self.target.prepare(seqs, K)
        if self.backup == "fast" and any(s.needs_fast_seed for s in seqs):
            return
        layout = [(n, None) for n in range(1, K) for _ in range(A)] + [(K, None)]
        Q = K + len(layout) * K
        for off in range(0, len(seqs), self.micro):
            group = seqs[off:off + self.micro]
            self.draft.prepare(group, Q, mask_builder=self._mask([layout] * len(group)), deferred=True)

    def _fast_backup(self, seqs: List[Sequence]) -> None:
        """serving/engine.py:64-71: a random block after the anchor (greedy
        verification needs token ids only); the draft's masked prediction is
        built later, in _predict."""
        V = self.draft.shape.vocab
        for s in seqs:
            cur = torch.randint(V, (self.K,), generator=self.backup_rng).tolist()
            cur[0] = s.anchor
            s.current = cur
            s.needs_fast_seed = True
            s.fast_backups += 1

    def _predict_submit(self, seqs: List[Sequence], lazy: bool = False):
        """serving/engine.py:73-131 up to the packed forwards, which run on
        the draft stream; returns what _predict_collect (every branch's
        tokens) or, with ``lazy``, _predict_hits needs: then no branch is
        turned into tokens yet, only the hidden states are kept."""
        K, A = self.K, self.A
        missing = [s for s in seqs if s.needs_fast_seed]
        missing_ids = {s.seq_id for s in missing}
        miss_anchors = (self.fast_miss_anchors or A) if self.backup == "fast" else A
        if missing:
            for group, top, _ in self._recover_submit(missing, max(A, miss_anchors) + 1):
                self.draft.stream.synchronize()
                for s, t in zip(group, top.tolist()):
                    s.top = t
                    s.needs_fast_seed = False
                    s.fast_seeds += 1
        if self.backup == "fast":
            partitions = [([s for s in seqs if s.seq_id not in missing_ids], False), (missing, True)]
        else:
            partitions = [(seqs, False)]
        groups = [(part[off:off + self.micro], shallow)
                  for part, shallow in partitions for off in range(0, len(part), self.micro)]
        pending = []
        ar = np.arange(K, dtype=np.int64)
        for group, shallow in groups:
            specs = [branch_specs(K, A, s.current, s.top, shallow, miss_anchors if shallow else A) for s in group]
            nb = len(specs[0])
            Q = K + nb * K
            # Row b: the current block at prefix..prefix+K-1, then branch j
            # (n accepted, anchor a) at prefix+n.. with a in its first slot.
            ids = np.full((len(group), Q), self.mask_id, dtype=np.int64)
            pos = np.empty((len(group), Q), dtype=np.int64)
            for b, s in enumerate(group):
                ns = np.array([n for n, _ in specs[b]], dtype=np.int64)
                ids[b, :K] = s.current
                pos[b, :K] = s.prefix + ar
                pos[b, K:] = (s.prefix + ns[:, None] + ar[None, :]).reshape(-1)
                for j, (_, a) in enumerate(specs[b]):
                    if a is not None:
                        ids[b, K + j * K] = a
            hidden, ready = self.draft.forward_hidden(group, torch.from_numpy(ids), positions=torch.from_numpy(pos),
                                                      mask_builder=self._mask(specs))
            if lazy:
                pending.append((group, specs, hidden, ready))
                continue
            # Every branch's tokens: the LM head and top-(A+1) of all rows,
            # queued on the target stream behind the verify.
            B_, Q_, H_ = hidden.shape
            top, greedy, done = self.draft.topk_post(hidden.reshape(B_ * Q_, H_), A + 1, self.target.stream, (ready,))
            pending.append((group, specs, top.view(B_, Q_, A + 1), greedy.view(B_, Q_), done))
        return pending

    def _predict_hits(self, pending, hits):
        """The tokens of the predicted branches that matched the verify
        (``hits``: (sequence, branch key, anchor)), from the lazily kept
        hidden states of _predict_submit(..., lazy=True): the LM head and
        top-(A+1) of those K rows per hit only, queued on the target stream
        behind the verify.  Returns (top, greedy, done, rows) for
        _apply_hits, or None without hits."""
        if not hits:
            return None
        K = self.K
        where = {s.seq_id: (e, b) for e in pending for b, s in enumerate(e[0])}
        rows, after = [], []
        for s, key, _ in hits:
            (group, specs, hidden, ready), b = where[s.seq_id]
            start = K + specs[b].index(key) * K
            rows.append((hidden, b, start))
            if ready not in after:
                after.append(ready)
        with torch.cuda.stream(self.target.stream):
            for ev in after:
                self.target.stream.wait_event(ev)
            x = torch.cat([h[b, st:st + K] for h, b, st in rows])
        top, greedy, done = self.draft.topk_post(x, self.A + 1, self.target.stream)
        return top, greedy, done

    def _apply_hits(self, hits, out) -> None:
        """s.current, s.top of each hit from _predict_hits' tokens."""
        if out is None:
            return
        top, greedy, done = out
        done.synchronize()
        K = self.K
        top_l, greedy_l = top.tolist(), greedy.tolist()
        for i, (s, key, anchor) in enumerate(hits):
            s.current = greedy_l[i * K:(i + 1) * K]
            s.current[0] = anchor
            s.top = top_l[i * K:(i + 1) * K]
            s.hits += 1

    def _predict_collect(self, pending) -> Dict[int, Dict]:
        """The packed predictions as host lists, once their top-k copies
        (on the target stream) have completed."""
        for entry in pending:
            entry[4].synchronize()
        K = self.K
        results: Dict[int, Dict] = {}
        for group, specs, top, greedy, _ in pending:
            top_l, greedy_l = top.tolist(), greedy.tolist()
            for b, s in enumerate(group):
                outcomes = {}
                for j, key in enumerate(specs[b]):
                    start = K + j * K
                    block = greedy_l[b][start:start + K]
                    if key[1] is not None:
                        block[0] = key[1]
                    outcomes[key] = (block, top_l[b][start:start + K])
                results[s.seq_id] = outcomes
        return results

    def _predict(self, seqs: List[Sequence]) -> Dict[int, Dict]:
        """serving/engine.py:73-131: {seq_id: {(n, anchor or None): (block, top)}}."""
        return self._predict_collect(self._predict_submit(seqs))

    # -- target side -----------------------------------------------------------
    def _verify(self, seqs: List[Sequence], blocks: List[List[int]]) -> List[Tuple[int, int]]:
        """serving/engine.py:133-136: (commit length, next anchor) per request."""
        res = self.target.verify(seqs, blocks)
        self.target.stream.synchronize()
        nl, al = res.tolist()
        return list(zip(nl, al))

    @staticmethod
    def _accepted(blocks: List[List[int]], posterior: List[List[int]]) -> List[Tuple[int, int]]:
        """serving/engine.py:138-145: (commit length, next anchor) per request."""
        out = []
        for block, p in zip(blocks, posterior):
            accepted = 1
            while accepted < len(block) and block[accepted] == p[accepted - 1]:
                accepted += 1
            out.append((accepted, p[accepted - 1]))
        return out

    # -- the loop ----------------------------------------------------------------
    @torch.inference_mode()
    def generate(self, prompts: Seq[Seq[int]], concurrency: int, max_new_tokens: int = 256,
                 ignore_eos: bool = False, eos: Tuple[int, ...] = EOS_IDS) -> Dict:
        if concurrency < 1 or max_new_tokens < 1:
            raise ValueError("positive concurrency and output length required")
        K = self.K
        vocab = self.target.shape.vocab
        prompts = [list(p) for p in prompts]
        if any(len(p) < 1 for p in prompts):
            raise ValueError("every prompt needs at least one token")
        if any(not 0 <= t < vocab for p in prompts for t in p):
            raise ValueError("prompt token id outside the vocabulary")
        dev = self.device
        self.backup_rng = torch.Generator().manual_seed(self.seed)
        # One page-table width for the run, so the captured graphs serve
        # every step: the longest prompt, the output, one packed block.
        ps = self.target.page_size
        A_max = max(self.A, self.fast_miss_anchors)
        Qp = K * (1 + A_max * (K - 1) + 1)
        need = max(max(len(p) for p in prompts) + max_new_tokens, self.min_table_tokens)
        width = -(-(need + Qp + K) // ps)
        self.target.width = self.draft.width = width
        waiting = iter(enumerate(prompts))
        running: List[Sequence] = []
        admitted_all: List[Sequence] = []
        outputs: List[Dict] = []
        exhausted = False
        torch.cuda.synchronize(dev)
        torch.cuda.reset_peak_memory_stats(dev)
        origin = torch.cuda.Event(enable_timing=True)
        origin.record(torch.cuda.current_stream(dev))
        started = time.perf_counter()
        max_active, batch_sizes = 0, []
        miss_rounds = miss_requests = 0
        steps = 0
        decode_s = 0.0  # wall time of the decode steps (admission and prefill excluded)
        verify_ms, draft_ms, overlap_ms, timeline = [], [], [], []
        while running or not exhausted:
            admitted = []
            while len(running) + len(admitted) < concurrency and not exhausted:
                try:
                    idx, ids = next(waiting)
                except StopIteration:
                    exhausted = True
                    break
                s = Sequence(idx, ids)
                s.sampling_params = SamplingParams(temperature=0, max_new_tokens=max_new_tokens)
                s.index = idx
                s.prefix = len(ids)
                s.generated, s.accepts = [], []
                s.born = time.perf_counter()
                s.hits = s.recoveries = s.fast_backups = s.fast_seeds = 0
                s.needs_fast_seed = False
                admitted.append(s)
                admitted_all.append(s)
            if admitted:
                # Prefill runs concurrently on the two streams, in groups of 4.
                for off in range(0, len(admitted), 4):
                    group = admitted[off:off + 4]
                    self._side("draft", self.draft.prefill_async, group)
                    anchors = self._side("target", self.target.prefill, group)
                    ready = []
                    for s, a in zip(group, anchors):
                        s.anchor = a
                        if not ignore_eos and a in eos:
                            s.generated = [a]
                            self._finish(s, outputs)
                        else:
                            ready.append(s)
                    self._side("draft", self._recover, ready)
                    running.extend(ready)
            if not running:
                continue
            max_active = max(max_active, len(running))
            batch_sizes.append(len(running))
            t_step = time.perf_counter()
            ev = {k: torch.cuda.Event(enable_timing=True) for k in ("vs", "ve", "ps", "pe", "rs", "re")}
            blocks = [list(s.current) for s in running]
            # Target verify on its stream ...
            ev["vs"].record(self.target.stream)
            res = self._side("target", self.target.verify, running, blocks)
            ev["ve"].record(self.target.stream)
            # ... while the draft predicts every outcome on its own.
            ev["ps"].record(self.draft.stream)
            pending = self._side("draft", self._predict_submit, running, True)
            ev["pe"].record(self.draft.stream)
            # The verify result decides the step; only the branches it hits
            # are then turned into tokens (their LM head on the target
            # stream, beside the recovery forwards).
            self._side("target", ev["ve"].synchronize)
            accepted = list(zip(*res.tolist()))
            predicted = {s.seq_id: set(e[1][b]) for e in pending for b, s in enumerate(e[0])}
            steps += 1
            remaining, recover, hits = [], [], []
            for s, block, (n, anchor) in zip(running, blocks, accepted):
                n, anchor = int(n), int(anchor)
                emitted = block[:n][: max_new_tokens - len(s.generated)]
                stop = False
                if not ignore_eos:
                    for j, t in enumerate(emitted):
                        if t in eos:
                            emitted, stop = emitted[: j + 1], True
                            break
                s.generated.extend(emitted)
                s.accepts.append(n)
                s.prefix += n
                s.anchor = anchor
                if stop or len(s.generated) >= max_new_tokens:
                    self._finish(s, outputs)
                    continue
                if not ignore_eos and anchor in eos:
                    s.generated.append(anchor)
                    self._finish(s, outputs)
                    continue
                key = (n, None if n == K else anchor)
                if key in predicted[s.seq_id]:
                    hits.append((s, key, anchor))
                else:
                    recover.append(s)
                self.target.trim(s, s.prefix)
                self.draft.trim(s, s.prefix)
                remaining.append(s)
            running = remaining
            miss_rounds += bool(recover)
            miss_requests += len(recover)
            hit_tokens = self._side("draft", self._predict_hits, pending, hits)
            ev["rs"].record(self.draft.stream)
            recovered = []
            if self.backup in ("fast", "fast_legacy"):
                self._fast_backup(recover)
            elif recover:
                recovered = self._side("draft", self._recover_submit, recover, self.A + 1)
            ev["re"].record(self.draft.stream)
            if running and (exhausted or len(running) >= concurrency):
                self._side("draft", self._prepare_next, running)
            self._side("draft", self._apply_hits, hits, hit_tokens)
            self._side("draft", self.draft.stream.synchronize)
            self._apply_recovered(recovered)
            decode_s += time.perf_counter() - t_step
            vs, ve = origin.elapsed_time(ev["vs"]), origin.elapsed_time(ev["ve"])
            ps_, pe = origin.elapsed_time(ev["ps"]), origin.elapsed_time(ev["pe"])
            if len(timeline) < 8:
                timeline.append(tuple(round(origin.elapsed_time(ev[k]), 3) for k in ("vs", "ve", "ps", "pe", "rs", "re")))
            verify_ms.append(ve - vs)
            draft_ms.append((pe - ps_) + ev["rs"].elapsed_time(ev["re"]))
            overlap_ms.append(max(0.0, min(ve, pe) - max(vs, ps_)))
        torch.cuda.synchronize(dev)
        elapsed = time.perf_counter() - started
        active = [s for s in admitted_all if "target" in s.pages]
        assert not active, "Target sequences leaked"
        assert self.draft.free_pages == self.draft.kv.num_pages, "Draft pages leaked"
        assert self.target.free_pages == self.target.kv.num_pages, "Target pages leaked"
        outputs.sort(key=lambda o: o["index"])
        total = sum(len(o["tokens"]) for o in outputs)
        peak = torch.cuda.max_memory_allocated(dev) / 1e9
        return dict(outputs=outputs, elapsed_s=elapsed, output_tokens=total, tps=total / elapsed,
                    max_active=max_active, decode_batch_sizes=batch_sizes, backup=self.backup,
                    miss_rounds=miss_rounds, miss_requests=miss_requests,
                    peak_allocated_gb=[peak, peak], target_active_sequences=len(active),
                    target_free_pages=self.target.free_pages,
                    steps=steps, decode_s=decode_s, steps_per_s=steps / max(decode_s, 1e-9),
                    verify_ms=sum(verify_ms) / max(len(verify_ms), 1),
                    draft_ms=sum(draft_ms) / max(len(draft_ms), 1),
                    overlap_fraction=sum(overlap_ms) / max(sum(verify_ms), 1e-9),
                    timeline=timeline)

    def _finish(self, s: Sequence, outputs: List[Dict]) -> None:
        outputs.append(dict(index=s.index, tokens=s.generated, latency_s=time.perf_counter() - s.born,
                            accepts=s.accepts, hits=s.hits, recoveries=s.recoveries,
                            fast_backups=s.fast_backups, fast_seeds=s.fast_seeds))
        self.target.release(s)
        self.draft.release(s)


@torch.inference_mode()
def generate_ar(worker: Runner, prompts: Seq[Seq[int]], concurrency: int, limit: int, eos=EOS_IDS,
                ignore_eos: bool = False) -> Dict:
    """Target-only greedy decoding with bounded admission and EOS refill.

    serving/baseline_concurrency.py:33-90 (the reference's autoregressive
    baseline) on a target Runner: prefill in groups of 4, then one token per
    running request per forward.  Its tokens are what a lossless greedy
    speculative engine must reproduce.
    """
    if concurrency < 1 or limit < 1 or not prompts:
        raise ValueError("Nonempty prompts and positive concurrency/token limit required")
    eos = set(eos)
    started = time.perf_counter()
    waiting = iter(enumerate(prompts))
    running: List[Sequence] = []
    outputs: List[Dict] = []
    batches: List[int] = []
    exhausted = False
    max_active = 0

    def emit(seq: Sequence, token: int) -> bool:
        seq.generated.append(token)
        hit_eos = (not ignore_eos) and token in eos
        if hit_eos or len(seq.generated) >= limit:
            outputs.append(dict(index=seq.index, tokens=seq.generated, latency_s=time.perf_counter() - seq.born,
                                finish_reason="eos" if hit_eos else "length"))
            worker.release(seq)
            return True
        return False

    while running or not exhausted:
        admitted = []
        while len(running) + len(admitted) < concurrency and not exhausted:
            try:
                index, ids = next(waiting)
            except StopIteration:
                exhausted = True
                break
            seq = Sequence(index, list(ids))
            seq.index, seq.prefix = index, len(ids)
            seq.generated, seq.born = [], time.perf_counter()
            admitted.append(seq)
        max_active = max(max_active, len(running) + len(admitted))
        for offset in range(0, len(admitted), 4):
            group = admitted[offset:offset + 4]
            for seq, token in zip(group, worker.prefill(group)):
                if not emit(seq, token):
                    running.append(seq)
        if running:
            batches.append(len(running))
            nxt = worker.forward(running, [[seq.generated[-1]] for seq in running], host=True)
            worker.stream.synchronize()
            remaining = []
            for seq, tokens in zip(running, nxt.tolist()):
                seq.prefix += 1
                if not emit(seq, int(tokens[0])):
                    remaining.append(seq)
            running = remaining
    torch.cuda.synchronize(worker.device)
    elapsed = time.perf_counter() - started
    outputs.sort(key=lambda o: o["index"])
    total = sum(len(o["tokens"]) for o in outputs)
    return dict(outputs=outputs, elapsed_s=elapsed, output_tokens=total, tps=total / elapsed,
                mean_output_tokens=total / len(outputs), max_active=max_active, decode_batch_sizes=batches)
