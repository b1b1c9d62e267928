"""Paged model runner with the reference's call surface.

Mirrors serving/backend.py:

* ``Runner(path, device, *, draft=False, pages=512)`` -- :24-53: one model
  (target or draft) with its paged K/V cache and page pool on one device;
  ``path`` names a model shape (there is no checkpoint loading: weights are
  random-initialised bf16), see :func:`resolve_shape`;
* ``reserve`` / ``release`` / ``trim`` / ``_tables`` -- :55-76, the page
  bookkeeping (device-resident tables here, see model.DevicePageTables);
* ``prefill(seqs)`` -- :98-112: the prompts' K/V and the greedy token after
  each prompt (the target's first anchor);
* ``forward(seqs, tokens, *, positions=None, mask_builder=None, topk=0)`` --
  :114-136: a block of Q tokens per request after its committed prefix;
  the target attends causally within the block, the draft under
  ``mask_builder``'s mask (Engine._mask); returns greedy [B, Q] or
  (top [B, Q, k], greedy [B, Q]);
* ``verify(seqs, tokens)`` -- the target forward with the greedy acceptance
  kernel fused after it (what Engine._verify does with the forward's greedy
  list, serving/engine.py:133-145), returning (accepted + 1, anchor) per
  request without a host list of the posterior.

All work runs on the runner's own HIP stream (``self.stream``, a dedicated
hardware queue) so that a target runner and a draft runner on one GPU
overlap; block forwards are replayed from HIP graphs per (batch, block
length, table width, mask) once seen.  Masks: a builder from
``Engine._mask`` carries its per-query visibility descriptor; any other
callable is evaluated and compiled to the descriptor (see
modeling_d3d.mask_to_visibility), which must then hold for every request.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Union

import numpy as np
import torch

from .draft import topk_tokens
from .model import (D3D_1P7B, QWEN3_8B, BlockStep, ModelShape, PagedKV, Qwen3PagedModel, Sequence, block_inputs,
                    prefill, release, reserve, trim)
from .modeling_d3d import mask_to_visibility
from . import speculative_sampling as ss
from .streams import dedicated_stream

PAGE = 256          # the reference's page size; ``pages`` counts pages of this size


def _to_host(t: torch.Tensor) -> torch.Tensor:
    """Copy into pinned host memory queued on the current stream (a pageable
    destination would block the host until the stream drains)."""
    buf = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
    buf.copy_(t, non_blocking=True)
    return buf


def _host_ids(x):
    """Token ids or positions [B, Q] as a host array (device tensors pass through)."""
    if isinstance(x, torch.Tensor):
        return x if x.is_cuda else x.to(torch.int64).numpy()
    arr = np.asarray(x, dtype=np.int64)
    if arr.ndim != 2:
        raise ValueError(f"expected [B, Q] token ids, got shape {arr.shape}")
    return arr


MASK_ID = 151669

# Model names the reference's command lines use (serving/bench.py:26-27),
# mapped to their shapes.
_SHAPES: Dict[str, ModelShape] = {
    "Qwen/Qwen3-8B": QWEN3_8B,
    "qwen3-8b": QWEN3_8B,
    "fudan-generative-ai/D3D-1.7B-8B": D3D_1P7B,
    "d3d-1.7b": D3D_1P7B,
}


def resolve_shape(path: Union[str, ModelShape]) -> ModelShape:
    """The model shape a Runner builds: a ModelShape, or a known model name."""
    if isinstance(path, ModelShape):
        return path
    if isinstance(path, str) and path in _SHAPES:
        return _SHAPES[path]
    raise ValueError(f"unknown model {path!r}: pass a ModelShape or one of {sorted(_SHAPES)}")


class SamplingParams:
    """serving/vendor/ssd/sampling_params.py's fields the engine sets."""

    def __init__(self, temperature: float = 0.0, max_new_tokens: int = 256):
        self.temperature = temperature
        self.max_new_tokens = max_new_tokens


class Runner:
    def __init__(self, path, device="cuda:0", *, draft: bool = False, pages: int = 512, page_size: int = 16,
                 seed: Optional[int] = None, use_graphs: bool = True):
        self.device = torch.device(device)
        self.draft = draft
        shape = resolve_shape(path)
        self.shape = shape
        self.config = type("Config", (), dict(vocab_size=shape.vocab, num_key_value_heads=shape.kv_heads,
                                              head_dim=shape.head_dim, hidden_size=shape.hidden,
                                              num_hidden_layers=shape.layers))()
        self.name = "draft" if draft else "target"
        self.page_size = page_size
        # ``pages`` is the reference's capacity in 256-token pages.
        num_pages = max(1, pages * PAGE // page_size)
        self.model = Qwen3PagedModel(shape, self.device, draft=draft, seed=(1 if draft else 0) if seed is None
                                     else seed)
        self.kv = PagedKV(shape, num_pages, page_size, self.device)
        self.pool = self.kv.pool
        self.stream = dedicated_stream(self.device, "draft" if draft else "target")
        self.use_graphs = use_graphs
        self._steps: Dict = {}
        self.width: Optional[int] = None  # fixed page-table width (graph replays), None = longest table

    # -- page bookkeeping (serving/backend.py:55-76) ---------------------------
    def table(self, seq: Sequence) -> List[int]:
        return seq.pages.setdefault(self.name, [])

    def reserve(self, seq: Sequence, length: int) -> None:
        reserve(self.kv, seq, self.name, length)

    # The device page-table pool is updated on the runner's stream, the
    # stream every block forward reads it on.
    def release(self, seq: Sequence) -> None:
        if self.name in seq.pages:
            with torch.cuda.stream(self.stream):
                release(self.kv, seq, self.name)

    def trim(self, seq: Sequence, length: int) -> None:
        # Host bookkeeping only: the device table rows are rewritten by the
        # next block_inputs on this runner's stream.
        trim(self.kv, seq, self.name, length)

    def _tables(self, seqs: List[Sequence]) -> torch.Tensor:
        width = max(len(self.table(s)) for s in seqs)
        return torch.tensor([self.table(s) + [0] * (width - len(self.table(s))) for s in seqs],
                            dtype=torch.int32, device=self.device)

    @property
    def free_pages(self) -> int:
        return len(self.pool.free)

    # -- forwards ----------------------------------------------------------------
    @torch.inference_mode()
    def prefill(self, seqs: List[Sequence]) -> List[int]:
        """K/V of every prompt; the greedy next token after each prompt."""
        nxt = self.prefill_async(seqs, tokens=True)
        self.stream.synchronize()
        return nxt.tolist()

    @torch.inference_mode()
    def prefill_async(self, seqs: List[Sequence], tokens: bool = False) -> Optional[torch.Tensor]:
        """The prompts' K/V on the runner's stream, no host wait; with
        ``tokens`` a pinned host tensor of the greedy next tokens, valid
        once the stream has drained."""
        with torch.cuda.stream(self.stream):
            hidden = prefill(self.model, self.kv, seqs, self.name)
            if not tokens:
                return None
            return _to_host(self.model.logits(hidden).argmax(-1))

    def _prepare(self, seqs: List[Sequence], Q: int, kind: str, vis: Optional[torch.Tensor], k: int) -> BlockStep:
        """Reserve the block's pages and write its page tables, slots,
        context lengths and positions straight into the step's static
        buffers (on the runner's stream); returns the step.  A step that
        ``prepare`` already filled for the same requests, prefixes and page
        lists is returned as it is."""
        for s in seqs:
            self.reserve(s, s.prefix + Q)
        width = self.width if self.width is not None else max(len(self.table(s)) for s in seqs)
        step = self._step(kind, len(seqs), Q, width, vis, k)
        key = tuple((s.seq_id, s.prefix, tuple(self.table(s))) for s in seqs)
        if step.prepared == key:
            step.prepared = None
            return step
        step.prepared = None
        block_inputs(self.kv, seqs, self.name, [s.prefix for s in seqs], Q, self.device, width, out=step.inputs())
        return step

    def prepare(self, seqs: List[Sequence], Q: int, *, mask_builder=None, topk: int = 0,
                deferred: bool = False) -> None:
        """Fill the page tables, slots and context lengths of the next block
        forward over ``seqs`` (Q tokens at their prefixes) ahead of it, on
        the runner's stream, so that the forward itself only copies its
        token ids and replays.  The next ``forward`` / ``verify`` (or, with
        ``deferred``, ``forward_hidden``) with the same requests, prefixes,
        page lists and block shape uses them; anything else prepares again."""
        with torch.cuda.stream(self.stream):
            if self.draft:
                vis = self._visibility(seqs, Q, mask_builder)
                step = self._prepare(seqs, Q, "hidden" if deferred else "forward", vis, 0 if deferred else topk)
            else:
                step = self._prepare(seqs, Q, "verify", None, 0)
            step.prepared = tuple((s.seq_id, s.prefix, tuple(self.table(s))) for s in seqs)

    def _step(self, kind: str, B: int, Q: int, width: int, vis: Optional[torch.Tensor], k: int):
        key = (kind, B, Q, width, k, None if vis is None else (tuple(vis.shape), vis.numpy().tobytes()))
        step = self._steps.get(key)
        if step is None:
            # The post functions hold the model, not the runner: a step that
            # referred back to the runner holding it would make every dropped
            # runner, with its captured graphs, garbage that only a cyclic
            # collection frees, at a moment nobody chooses.
            model = self.model
            if kind == "verify":
                def post(hidden, ids):
                    out = ss.greedy_accept(model.logits(hidden), ids)
                    return out.accepted, out.out_token
            elif kind == "hidden":
                def post(hidden, ids):
                    return hidden
            else:
                def post(hidden, ids):
                    top = topk_tokens(model.logits(hidden), max(k, 1))
                    return top, top[..., 0]
            step = BlockStep(self.model, self.kv, B, Q, width, causal=not self.draft, post=post,
                             use_graph=self.use_graphs, q_vis=vis)
            self._steps[key] = step
        return step

    @torch.inference_mode()
    def forward(self, seqs: List[Sequence], tokens, *, positions=None, mask_builder=None, topk: int = 0,
                host: bool = False):
        """serving/backend.py:114-136 on the runner's stream (no host sync).

        With ``host`` the results are pinned host tensors whose copies are
        queued on the runner's stream (valid once it has drained)."""
        with torch.cuda.stream(self.stream):
            ids = _host_ids(tokens)
            B, Q = ids.shape
            vis = self._visibility(seqs, Q, mask_builder) if self.draft else None
            step = self._prepare(seqs, Q, "forward", vis, topk)
            top, greedy = step.run(ids, None if positions is None else _host_ids(positions))
            copy = _to_host if host else torch.clone
            if topk:
                return copy(top[..., :topk].contiguous()), copy(greedy)
            return copy(greedy)

    @torch.inference_mode()
    def forward_hidden(self, seqs: List[Sequence], tokens, *, positions=None, mask_builder=None):
        """The block forward of ``forward`` without its LM head: returns the
        final hidden states [B, Q, hidden] (a captured step's output, valid
        until the next forward of that shape) and an event recorded on this
        runner's stream after them.  ``topk_post`` turns any of its rows into
        tokens later, on any stream."""
        with torch.cuda.stream(self.stream):
            ids = _host_ids(tokens)
            B, Q = ids.shape
            vis = self._visibility(seqs, Q, mask_builder) if self.draft else None
            step = self._prepare(seqs, Q, "hidden", vis, 0)
            hidden = step.run(ids, None if positions is None else _host_ids(positions))
            ready = torch.cuda.Event()
            ready.record(self.stream)
        return hidden, ready

    @torch.inference_mode()
    def topk_post(self, rows: torch.Tensor, topk: int, stream: torch.cuda.Stream, after=()):
        """LM head + top-``topk`` of hidden rows [R, hidden] on ``stream``,
        once the events ``after`` have completed: pinned host (top [R, topk],
        greedy [R]) and the event after their copies."""
        if topk < 1:
            raise ValueError("topk_post needs topk >= 1")
        with torch.cuda.stream(stream):
            for ev in after:
                stream.wait_event(ev)
            top = topk_tokens(self.model.logits(rows), topk)
            out = _to_host(top[..., :topk].contiguous()), _to_host(top[..., 0])
            done = torch.cuda.Event()
            done.record(stream)
        return out[0], out[1], done

    @torch.inference_mode()
    def verify(self, seqs: List[Sequence], tokens) -> torch.Tensor:
        """Target forward over the blocks + greedy acceptance on the device.

        Returns a pinned host tensor [2, B] int64 -- commit length (accepted
        + 1) and next anchor per request -- whose copy is queued on the
        runner's stream (valid once it has drained)."""
        if self.draft:
            raise RuntimeError("verify runs on the target runner")
        with torch.cuda.stream(self.stream):
            ids = _host_ids(tokens)
            B, Q = ids.shape
            accepted, out_token = self._prepare(seqs, Q, "verify", None, 0).run(ids)
            return _to_host(torch.stack([accepted.long() + 1, out_token]))

    def _visibility(self, seqs: List[Sequence], Q: int, mask_builder) -> torch.Tensor:
        """Per-query visibility [Q, 3] (relative to the block start) of the draft mask."""
        if mask_builder is None:
            return torch.tensor([[Q, 0, 0]] * Q, dtype=torch.int32)  # recovery: prefix + whole block
        desc = getattr(mask_builder, "visibility", None)
        if desc is not None:
            vis = desc(Q)
            if vis.shape != (Q, 3):
                raise ValueError("mask builder visibility must be [Q, 3]")
            return vis.to(torch.int32)
        # A generic builder: evaluate its [B, 1, Q, S] mask, compile it per
        # request (each relative to its own prefix) and require one result.
        starts = torch.tensor([s.prefix for s in seqs], device=self.device)
        S = max(s.prefix for s in seqs) + Q
        mask = mask_builder(starts, Q, S)
        out = None
        for b, s in enumerate(seqs):
            v = mask_to_visibility(mask[b:b + 1, ..., :s.prefix + Q], Q, s.prefix + Q)
            v = v - torch.tensor([s.prefix, s.prefix, s.prefix], dtype=torch.int32)
            if out is None:
                out = v
            elif not torch.equal(out, v):
                raise ValueError("the mask differs between requests beyond their prefixes")
        return out
