"""Greedy speculative engine with the target and the draft on one GPU.

Mirrors serving/engine.py:14-227 (the concurrent greedy engine): every step
the target verifies each running request's block (anchor + 15 draft tokens)
while the draft, on a second HIP stream, prepares the next block for the
"all accepted" outcome; requests whose outcome misses that prediction are
recovered by a draft forward from the new anchor.  The reference runs the
target in another process on another GPU and exchanges token lists over a
pipe (serving/target_process.py); here both models are co-resident and the
exchange is a pair of stream events plus one small device-to-host copy of
the acceptance results per step.

Differences from the reference, on purpose:

* acceptance is the fused greedy kernel on the target logits (no argmax
  list round trip): commit length = accepted + 1, anchor = correction
  token, exactly Engine._accepted (serving/engine.py:138-145);
* the prediction covers one outcome, all 16 accepted (key (16, None) of
  serving/engine.py:73-131); the multi-branch packed prediction with a
  structured mask is not built yet, so other outcomes take the recovery
  path (serving/engine.py:54-62), as misses do in the reference;
* the draft fills a block in one forward (greedy per position), as the
  reference's Runner does (serving/backend.py:84-93).
"""
from __future__ import annotations

import time
from typing import Dict, List, Sequence as Seq, Tuple

import torch

from . import speculative_sampling as ss
from .draft import MASK_ID, confidence_topk_unmask
from .model import (D3D_1P7B, QWEN3_8B, BlockStep, ModelShape, PagedKV, Qwen3PagedModel, Sequence, block_inputs,
                    prefill, release, reserve, trim)

EOS_IDS = (151643, 151645)


class Engine:
    def __init__(self, target_shape: ModelShape = QWEN3_8B, draft_shape: ModelShape = D3D_1P7B, *,
                 block_size: int = 16, page_size: int = 16, pages: int = 4096, device: str = "cuda:0",
                 seed: int = 42, mask_id: int = MASK_ID, use_graphs: bool = True):
        if target_shape.vocab != draft_shape.vocab:
            raise ValueError("target and draft vocabularies must match")
        if not 0 <= mask_id < draft_shape.vocab:
            raise ValueError(f"mask id {mask_id} outside the draft vocabulary")
        self.K = block_size
        self.mask_id = mask_id
        self.use_graphs = use_graphs
        self._cache: Dict = {}
        self.device = torch.device(device)
        self.target = Qwen3PagedModel(target_shape, self.device, draft=False, seed=seed)
        self.draft = Qwen3PagedModel(draft_shape, self.device, draft=True, seed=seed + 1)
        self.tkv = PagedKV(target_shape, pages, page_size, self.device)
        self.dkv = PagedKV(draft_shape, pages, page_size, self.device)
        # Two streams at the default priority: verify and draft overlap.
        self.ts = torch.cuda.Stream(self.device)
        self.ds = torch.cuda.Stream(self.device)

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
        """(verify, draft commit, draft fill) block steps for B requests, cached."""
        key = (B, width)
        if key not in self._cache:
            K, mid = self.K, self.mask_id

            def verify_post(hidden, ids):
                out = ss.greedy_accept(self.target.logits(hidden), ids)
                return out.accepted, out.out_token

            def fill_post(hidden, ids):
                confidence_topk_unmask(self.draft.logits(hidden), ids, mid, K)
                return ids

            self._cache[key] = (
                BlockStep(self.target, self.tkv, B, K, width, causal=True, post=verify_post,
                          use_graph=self.use_graphs),
                BlockStep(self.draft, self.dkv, B, K, width, causal=True, post=None, use_graph=self.use_graphs),
                BlockStep(self.draft, self.dkv, B, K, width, causal=False, post=fill_post,
                          use_graph=self.use_graphs),
            )
        return self._cache[key]

    def _fill(self, seqs: List[Sequence], ids: torch.Tensor, starts: List[int], width: int) -> torch.Tensor:
        """One draft forward of a block; masked positions take the greedy token."""
        for s, st in zip(seqs, starts):
            reserve(self.dkv, s, "draft", st + self.K)
        tables, slots, lens, logical, _ = block_inputs(self.dkv, seqs, "draft", starts, self.K, self.device, width)
        return self._steps(len(seqs), width)[2](ids, logical, tables, slots, lens).clone()

    def _recover(self, seqs: List[Sequence], anchors: List[int], width: int) -> torch.Tensor:
        """serving/engine.py:54-62: anchor + 15 masks from the committed prefix."""
        ids = torch.full((len(seqs), self.K), self.mask_id, dtype=torch.int64)
        ids[:, 0] = torch.tensor(anchors)
        return self._fill(seqs, ids.to(self.device, non_blocking=True), [s.prefix for s in seqs], width)

    def _predict_full(self, seqs: List[Sequence], blocks: torch.Tensor, width: int) -> torch.Tensor:
        """Writes the pending block's draft K/V (causal) and drafts the block after it."""
        starts = [s.prefix for s in seqs]
        for s in seqs:
            reserve(self.dkv, s, "draft", s.prefix + 2 * self.K)
        tables, slots, lens, logical, _ = block_inputs(self.dkv, seqs, "draft", starts, self.K, self.device, width)
        self._steps(len(seqs), width)[1](blocks, logical, tables, slots, lens)
        ids = torch.full((len(seqs), self.K), self.mask_id, dtype=torch.int64, device=self.device)
        return self._fill(seqs, ids, [s.prefix + self.K for s in seqs], width)

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
        ps = self.tkv.page_size
        width = -(-(max(len(p) for p in prompts) + max_new_tokens + 2 * self.K) // ps)
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
            current = self._recover(seqs, anchors, width)
        running = list(seqs)
        steps = 0
        verify_ms, draft_ms, overlap_ms = [], [], []
        outputs = []
        while running:
            ev = {k: torch.cuda.Event(enable_timing=True) for k in ("vs", "ve", "ps", "pe", "rs", "re")}
            # -- target verify on ts ------------------------------------------
            self.ts.wait_stream(self.ds)
            current.record_stream(self.ts)
            with torch.cuda.stream(self.ts):
                ev["vs"].record(self.ts)
                for s in running:
                    reserve(self.tkv, s, "target", s.prefix + self.K)
                tables, slots, lens, logical, _ = block_inputs(self.tkv, running, "target",
                                                               [s.prefix for s in running], self.K, dev, width)
                accepted, out_token = self._steps(len(running), width)[0](current, logical, tables, slots, lens)
                res = torch.stack([accepted.long(), out_token]).to("cpu", non_blocking=True)
                blocks_host = current.to("cpu", non_blocking=True)
                ev["ve"].record(self.ts)
            # -- draft prediction of the all-accepted outcome on ds -------------
            with torch.cuda.stream(self.ds):
                ev["ps"].record(self.ds)
                predicted = self._predict_full(running, current, width)
                ev["pe"].record(self.ds)
            ev["ve"].synchronize()
            n_acc, tokens = res.tolist()
            blocks = blocks_host.tolist()
            steps += 1
            remaining, recover, rec_anchor, hit_rows = [], [], [], []
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
                if n == self.K:
                    s.hits += 1
                    hit_rows.append((len(remaining) - 1, i, anchor))
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
            # -- next blocks: hits reuse the prediction, misses recover ---------
            with torch.cuda.stream(self.ds):
                ev["rs"].record(self.ds)
                nxt = torch.empty(len(remaining), self.K, dtype=torch.int64, device=dev)
                if hit_rows:
                    dst = torch.tensor([r for r, _, _ in hit_rows], device=dev)
                    src = torch.tensor([i for _, i, _ in hit_rows], device=dev)
                    nxt[dst] = predicted[src]
                    nxt[dst, 0] = torch.tensor([a for _, _, a in hit_rows], device=dev)
                if recover:
                    rec = self._recover(recover, rec_anchor, width)
                    idx = torch.tensor([remaining.index(s) for s in recover], device=dev)
                    nxt[idx] = rec
                ev["re"].record(self.ds)
            for s in remaining:
                trim(self.dkv, s, "draft", s.prefix)
            ev["re"].synchronize()
            vs = origin.elapsed_time(ev["vs"])
            ve = origin.elapsed_time(ev["ve"])
            ps_ = origin.elapsed_time(ev["ps"])
            pe = origin.elapsed_time(ev["pe"])
            verify_ms.append(ve - vs)
            draft_ms.append((pe - ps_) + ev["rs"].elapsed_time(ev["re"]))
            overlap_ms.append(max(0.0, min(ve, pe) - max(vs, ps_)))
            current = nxt
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
        )
