"""Greedy speculative engine with the target and the draft on one GPU.

Mirrors serving/engine.py:14-227 (the concurrent greedy engine): every step
the target verifies each running request's block (anchor + 15 draft tokens)
while the draft, on a second HIP stream, runs the packed multi-branch
prediction (serving/engine.py:73-131): one forward over the pending block
(causal: this commits the pending tokens' draft K/V) and one branch block
per (accepted count n, anchor) outcome plus the all-accepted outcome.  A
request whose outcome (n, anchor) was predicted takes that branch's block;
the others are recovered by a draft forward from the new anchor
(serving/engine.py:54-62).  The reference runs the target in another
process on another GPU and exchanges token lists over a pipe
(serving/target_process.py); here both models are co-resident and the
exchange is a pair of stream events plus small device-to-host copies.

Differences from the reference, on purpose:

* acceptance is the fused greedy kernel on the target logits (no argmax
  list round trip): commit length = accepted + 1, anchor = correction
  token, exactly Engine._accepted (serving/engine.py:138-145);
* the draft's greedy tokens and top-(A+1) anchors come from one top-k
  kernel over the logits (serving/backend.py:84-93);
* the packed mask is a per-query visibility descriptor read by the
  attention kernel instead of a materialised [B, 1, Q, S] bool tensor.
"""
from __future__ import annotations

import time
from typing import Dict, List, Optional, Sequence as Seq, Tuple

import torch

from .attention import packed_visibility
from .draft import MASK_ID, topk_tokens
from . import speculative_sampling as ss
from .streams import dedicated_stream
from .model import (D3D_1P7B, QWEN3_8B, BlockStep, ModelShape, PagedKV, Qwen3PagedModel, Sequence, block_inputs,
                    prefill, release, reserve, trim)

EOS_IDS = (151643, 151645)


def _to_host(t: torch.Tensor) -> torch.Tensor:
    """Stream-ordered copy into pinned host memory (a pageable destination
    would make the copy block the host until the stream drains)."""
    buf = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
    buf.copy_(t, non_blocking=True)
    return buf


def branch_specs(K: int, A: int, current: List[int], top: List[List[int]]) -> List[Tuple[int, Optional[int]]]:
    """Engine._predict's branches (serving/engine.py:98-105): for each accepted
    count n in 1..K-1 the first A draft top-(A+1) tokens at position n that
    differ from current[n], then the all-accepted branch (K, None)."""
    out: List[Tuple[int, Optional[int]]] = []
    for n in range(1, K):
        anchors = [v for v in top[n] if v != current[n]][:A]
        if len(anchors) != A:
            raise RuntimeError("draft top-k holds fewer than A alternative anchors")
        out.extend((n, a) for a in anchors)
    out.append((K, None))
    return out


class Engine:
    def __init__(self, target_shape: ModelShape = QWEN3_8B, draft_shape: ModelShape = D3D_1P7B, *,
                 block_size: int = 16, anchor_num: int = 1, page_size: int = 16, pages: int = 4096,
                 device: str = "cuda:0", seed: int = 42, mask_id: int = MASK_ID, use_graphs: bool = True):
        if target_shape.vocab != draft_shape.vocab:
            raise ValueError("target and draft vocabularies must match")
        if not 0 <= mask_id < draft_shape.vocab:
            raise ValueError(f"mask id {mask_id} outside the draft vocabulary")
        if anchor_num < 1:
            raise ValueError("anchor_num must be positive")
        self.K, self.A = block_size, anchor_num
        self.mask_id = mask_id
        self.use_graphs = use_graphs
        self._cache: Dict = {}
        self.device = torch.device(device)
        self.target = Qwen3PagedModel(target_shape, self.device, draft=False, seed=seed)
        self.draft = Qwen3PagedModel(draft_shape, self.device, draft=True, seed=seed + 1)
        self.tkv = PagedKV(target_shape, pages, page_size, self.device)
        self.dkv = PagedKV(draft_shape, pages, page_size, self.device)
        # Packed prediction: the pending block + A anchors per accepted count 1..K-1 + all accepted.
        self.nbranch = self.A * (self.K - 1) + 1
        self.Qp = self.K * (1 + self.nbranch)
        # Two streams at the default priority, each on its own hardware
        # queue, so that verify and draft overlap.
        self.ts = dedicated_stream(self.device)
        self.ds = dedicated_stream(self.device)

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

    # -- graph-replayed block steps --------------------------------------------
    def _steps(self, B: int, width: int):
        """(verify, recovery, packed prediction) block steps for B requests, cached."""
        key = (B, width)
        if key not in self._cache:
            K, k = self.K, self.A + 1

            def verify_post(hidden, ids):
                out = ss.greedy_accept(self.target.logits(hidden), ids)
                return out.accepted, out.out_token

            def recover_post(hidden, ids):
                top = topk_tokens(self.draft.logits(hidden), k)
                block = top[..., 0].clone()
                block[:, 0] = ids[:, 0]
                return block, top

            def predict_post(hidden, ids):
                return topk_tokens(self.draft.logits(hidden), k)

            names = [n for n, _ in branch_specs(K, self.A, [0] * K, [list(range(1, k + 1))] * K)]
            self._cache[key] = (
                BlockStep(self.target, self.tkv, B, K, width, causal=True, post=verify_post,
                          use_graph=self.use_graphs),
                BlockStep(self.draft, self.dkv, B, K, width, causal=False, post=recover_post,
                          use_graph=self.use_graphs),
                BlockStep(self.draft, self.dkv, B, self.Qp, width, causal=False, post=predict_post,
                          use_graph=self.use_graphs, q_vis=packed_visibility(K, names)),
            )
        return self._cache[key]

    def _recover(self, seqs: List[Sequence], anchors: List[int], width: int):
        """serving/engine.py:54-62: anchor + K-1 masks from the committed prefix;
        returns (block [B, K], top [B, K, A+1]) on the device."""
        ids = torch.full((len(seqs), self.K), self.mask_id, dtype=torch.int64)
        ids[:, 0] = torch.tensor(anchors)
        for s in seqs:
            reserve(self.dkv, s, "draft", s.prefix + self.K)
        tables, slots, lens, logical, _ = block_inputs(self.dkv, seqs, "draft", [s.prefix for s in seqs], self.K,
                                                       self.device, width)
        block, top = self._steps(len(seqs), width)[1](ids.to(self.device, non_blocking=True), logical, tables,
                                                     slots, lens)
        return block.clone(), top.clone()

    def _predict(self, seqs: List[Sequence], current: List[List[int]], top: List[List[List[int]]], width: int):
        """serving/engine.py:73-131, one packed forward: returns the branch
        specs per request and the device top-(A+1) [B, Qp, A+1] of every
        packed position (index 0 is the greedy token)."""
        K, Qp = self.K, self.Qp
        B = len(seqs)
        specs = [branch_specs(K, self.A, current[b], top[b]) for b in range(B)]
        ids = torch.full((B, Qp), self.mask_id, dtype=torch.int64)
        pos = torch.empty((B, Qp), dtype=torch.int64)
        for b, s in enumerate(seqs):
            ids[b, :K] = torch.tensor(current[b])
            pos[b, :K] = torch.arange(s.prefix, s.prefix + K)
            for j, (n, a) in enumerate(specs[b]):
                start = K + j * K
                if a is not None:
                    ids[b, start] = a
                pos[b, start:start + K] = torch.arange(s.prefix + n, s.prefix + n + K)
        for s in seqs:
            reserve(self.dkv, s, "draft", s.prefix + Qp)
        tables, slots, lens, _, _ = block_inputs(self.dkv, seqs, "draft", [s.prefix for s in seqs], Qp,
                                                 self.device, width)
        dev = self.device
        out = self._steps(B, width)[2](ids.to(dev, non_blocking=True), pos.to(dev, non_blocking=True), tables,
                                       slots, lens)
        return specs, out.clone()

    # -- main loop -----------------------------------------------------------
    @torch.inference_mode()
    def generate(self, prompts: Seq[Seq[int]], max_new_tokens: int = 256, ignore_eos: bool = False,
                 eos: Tuple[int, ...] = EOS_IDS) -> Dict:
        if max_new_tokens < 1:
            raise ValueError("positive output length required")
        dev = self.device
        vocab = self.target.shape.vocab
        if any(not 0 <= t < vocab for p in prompts for t in p):
            raise ValueError("prompt token id outside the vocabulary")
        seqs = [Sequence(i, p) for i, p in enumerate(prompts)]
        for s in seqs:
            s.generated, s.accepts, s.hits, s.recoveries = [], [], 0, 0
        # One page-table width for the whole run: the attention's context
        # bound and the captured graphs stay fixed while contexts grow.
        K = self.K
        ps = self.tkv.page_size
        width = -(-(max(len(p) for p in prompts) + max_new_tokens + self.Qp + K) // ps)
        origin = torch.cuda.Event(enable_timing=True)
        origin.record(torch.cuda.current_stream(dev))
        started = time.perf_counter()

        # Prefill both models concurrently; the target's last position gives the anchor.
        with torch.cuda.stream(self.ts):
            h = prefill(self.target, self.tkv, seqs, "target")
            anchor_t = self.target.logits(h).argmax(-1)
        with torch.cuda.stream(self.ds):
            prefill(self.draft, self.dkv, seqs, "draft")
        self.ts.synchronize()
        anchors = anchor_t.cpu().tolist()
        with torch.cuda.stream(self.ds):
            block, top = self._recover(seqs, anchors, width)
        self.ds.synchronize()
        for s, blk, t in zip(seqs, block.cpu().tolist(), top.cpu().tolist()):
            s.current, s.top = blk, t
        running = list(seqs)
        steps = 0
        verify_ms, draft_ms, overlap_ms = [], [], []
        timeline = []  # (verify start, end, predict start, end, recovery start, end) ms, first steps
        outputs = []
        while running:
            ev = {k: torch.cuda.Event(enable_timing=True) for k in ("vs", "ve", "ps", "pe", "rs", "re")}
            blocks = [s.current for s in running]
            # -- target verify on ts ------------------------------------------
            with torch.cuda.stream(self.ts):
                ev["vs"].record(self.ts)
                for s in running:
                    reserve(self.tkv, s, "target", s.prefix + K)
                tables, slots, lens, logical, _ = block_inputs(self.tkv, running, "target",
                                                               [s.prefix for s in running], K, dev, width)
                cur = torch.tensor(blocks, dtype=torch.int64).to(dev, non_blocking=True)
                accepted, out_token = self._steps(len(running), width)[0](cur, logical, tables, slots, lens)
                res = _to_host(torch.stack([accepted.long(), out_token]))
                ev["ve"].record(self.ts)
            # -- packed multi-branch draft prediction on ds ---------------------
            with torch.cuda.stream(self.ds):
                ev["ps"].record(self.ds)
                specs, ptop = self._predict(running, blocks, [s.top for s in running], width)
                ptop_host = _to_host(ptop)
                ev["pe"].record(self.ds)
            ev["ve"].synchronize()
            ev["pe"].synchronize()
            n_acc, tokens = res.tolist()
            ptop_l = ptop_host.tolist()
            steps += 1
            remaining, recover, rec_anchor = [], [], []
            for i, s in enumerate(running):
                n = int(n_acc[i]) + 1
                anchor = int(tokens[i])
                emitted = blocks[i][:n][: max_new_tokens - len(s.generated)]
                stop = False
                if not ignore_eos:
                    for j, t in enumerate(emitted):
                        if t in eos:
                            emitted, stop = emitted[: j + 1], True
                            break
                s.generated.extend(emitted)
                s.accepts.append(n)
                s.prefix += n
                if stop or len(s.generated) >= max_new_tokens:
                    outputs.append(s)
                    continue
                if not ignore_eos and anchor in eos:
                    s.generated.append(anchor)
                    outputs.append(s)
                    continue
                trim(self.tkv, s, "target", s.prefix)
                remaining.append(s)
                key = (n, None if n == K else anchor)
                j = specs[i].index(key) if key in specs[i] else -1
                if j >= 0:
                    rows = ptop_l[i][K + j * K: K + (j + 1) * K]
                    s.current = [r[0] for r in rows]
                    s.current[0] = anchor
                    s.top = rows
                    s.hits += 1
                else:
                    s.recoveries += 1
                    recover.append(s)
                    rec_anchor.append(anchor)
            for s in outputs:
                if "target" in s.pages:
                    release(self.tkv, s, "target")
                if "draft" in s.pages:
                    release(self.dkv, s, "draft")
            if not remaining:
                break
            # -- misses: recovery from the new anchor ---------------------------
            with torch.cuda.stream(self.ds):
                ev["rs"].record(self.ds)
                if recover:
                    block, top = self._recover(recover, rec_anchor, width)
                    block_host, top_host = _to_host(block), _to_host(top)
                ev["re"].record(self.ds)
            ev["re"].synchronize()
            if recover:
                for s, blk, t in zip(recover, block_host.tolist(), top_host.tolist()):
                    s.current, s.top = blk, t
            for s in remaining:
                trim(self.dkv, s, "draft", s.prefix)
            vs = origin.elapsed_time(ev["vs"])
            ve = origin.elapsed_time(ev["ve"])
            ps_ = origin.elapsed_time(ev["ps"])
            pe = origin.elapsed_time(ev["pe"])
            if len(timeline) < 8:
                timeline.append(tuple(round(origin.elapsed_time(ev[k]), 3) for k in ("vs", "ve", "ps", "pe", "rs", "re")))
            verify_ms.append(ve - vs)
            draft_ms.append((pe - ps_) + ev["rs"].elapsed_time(ev["re"]))
            overlap_ms.append(max(0.0, min(ve, pe) - max(vs, ps_)))
            running = remaining
        torch.cuda.synchronize(dev)
        elapsed = time.perf_counter() - started
        outputs.sort(key=lambda s: s.seq_id)
        total = sum(len(s.generated) for s in outputs)
        assert len(self.tkv.pool.free) == self.tkv.num_pages, "target pages leaked"
        assert len(self.dkv.pool.free) == self.dkv.num_pages, "draft pages leaked"
        return dict(
            outputs=[dict(index=s.seq_id, tokens=s.generated, accepts=s.accepts, hits=s.hits,
                          recoveries=s.recoveries) for s in outputs],
            elapsed_s=elapsed, output_tokens=total, tps=total / elapsed, steps=steps,
            steps_per_s=steps / elapsed,
            verify_ms=sum(verify_ms) / max(len(verify_ms), 1),
            draft_ms=sum(draft_ms) / max(len(draft_ms), 1),
            overlap_fraction=sum(overlap_ms) / max(sum(verify_ms), 1e-9),
            timeline=timeline,
        )
