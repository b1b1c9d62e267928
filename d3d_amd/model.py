"""Qwen3-shaped paged models for the verify (target) and draft forwards.

Host code in PyTorch-ROCm (GEMMs on hipBLASLt); attention, the norms,
RoPE with the KV append, SiLU-mul and the speculative reductions run on the
gfx950 kernels.  Weights are
random-initialised bf16 (there are no checkpoints on this path's benchmarks).

Reference structure followed:

* target -- serving/vendor/ssd/models/qwen3.py:14-325: fused QKV and
  gate-up projections, per-head q/k RMSNorm (RMSHeadNorm), rotary
  embedding computed in fp32 from a cos/sin cache
  (serving/vendor/ssd/layers/rotary_embedding.py:6-16, :19-60), fused
  residual add + RMSNorm (serving/vendor/ssd/layers/layernorm.py:53-98),
  SiLU-and-mul MLP, untied LM head;
* draft -- models/d3d/modeling_d3d.py: the same backbone with q/k RMSNorm
  and HF-style RoPE whose cos/sin are cast to the activation dtype
  (:164-187, :470-516), attention through the paged draft branch
  (serving/d3d_adapter.py:20-51).

Block attention: the target attends causally within the 16-token block
(flash_attn_with_kvcache, serving/vendor/ssd/layers/attention.py:38-41); the
draft block sees the prefix and the whole block (recovery mask,
serving/engine.py:41-42).  Prompt prefill reuses the block kernel: each
prompt is cut into 16-token slices aligned to its end, and each slice runs as
its own request whose context ends at the slice, which is exactly causal
attention over the prompt (any prompt length).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np
import torch
import torch.nn.functional as F

from . import _lib
from . import attention as att
from . import layers as ly


@dataclass(frozen=True)
class ModelShape:
    layers: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    mlp: int
    vocab: int = 151936
    rope_theta: float = 1_000_000.0
    eps: float = 1e-6

    @property
    def params(self) -> int:
        h, d = self.hidden, self.head_dim
        per_layer = (h * (self.heads + 2 * self.kv_heads) * d + self.heads * d * h + 3 * h * self.mlp
                     + 2 * h + 2 * d)
        return 2 * self.vocab * h + self.layers * per_layer + h


# Qwen3-8B-shaped target and Qwen3-1.7B-shaped D3D draft (2,031,739,904
# parameters with an untied LM head).
QWEN3_8B = ModelShape(layers=36, hidden=4096, heads=32, kv_heads=8, head_dim=128, mlp=12288)
D3D_1P7B = ModelShape(layers=28, hidden=2048, heads=16, kv_heads=8, head_dim=128, mlp=6144)


class PagePool:
    """Page allocator over a fixed pool (serving/vendor/ssd/engine/block_manager.py:65-88)."""

    def __init__(self, num_pages: int):
        self.num_pages = num_pages
        self.free: List[int] = list(range(num_pages))

    def alloc(self, n: int) -> List[int]:
        if n > len(self.free):
            raise RuntimeError(f"page pool exhausted: need {n}, have {len(self.free)}")
        out, self.free = self.free[:n], self.free[n:]
        return out

    def release(self, pages: Sequence[int]) -> None:
        self.free.extend(pages)


class DevicePageTables:
    """Device mirror of the sequences' page lists (serving/backend.py:55-76).

    A [rows, num_pages] int32 pool on the device holds one row of page ids
    per (sequence, model) table; only the ids appended since the last sync
    cross to the device (a pinned copy), and ``block_inputs`` reads the
    per-step tables, slots, positions and context lengths out of the pool
    with one kernel (``d3d_block_inputs``) instead of rebuilding them from
    host lists.  Rows freed by ``release`` are reused.
    """

    def __init__(self, num_pages: int, device, rows: int = 64):
        self.width = num_pages
        self.device = torch.device(device)
        # -1 marks entries past a sequence's page list.
        self.pool = torch.full((rows, num_pages), -1, dtype=torch.int32, device=self.device)
        self.free_rows: List[int] = list(range(rows))

    def row(self, seq: "Sequence", name: str) -> int:
        """The pool row of seq's table ``name``, assigned on first use."""
        row = seq.rows.get(name)
        if row is None:
            if not self.free_rows:
                old = self.pool
                self.pool = torch.full((2 * old.shape[0], self.width), -1, dtype=torch.int32, device=self.device)
                self.pool[: old.shape[0]].copy_(old)
                self.free_rows = list(range(old.shape[0], 2 * old.shape[0]))
            row = self.free_rows.pop(0)
            seq.rows[name] = row
            seq.synced[name] = [0, 0]
        return row

    def updates(self, seq: "Sequence", name: str) -> tuple:
        """The pool entries to rewrite for seq's table ``name``: (flat
        indices, values) of the page ids appended since the last sync and
        of the -1 marks over the ids a trim removed.  The caller applies
        them (``apply``) before the table is next read on the device."""
        row = self.row(seq, name)
        pages = seq.pages.get(name, [])
        state = seq.synced[name]  # [entries equal to the host list, entries written]
        valid, written = state
        n = len(pages)
        state[0] = state[1] = n
        if n > valid:
            cols = np.arange(valid, max(n, written), dtype=np.int64)
            vals = np.full(len(cols), -1, dtype=np.int64)
            vals[: n - valid] = pages[valid:]
        elif written > n:
            cols = np.arange(n, written, dtype=np.int64)
            vals = np.full(len(cols), -1, dtype=np.int64)
        else:
            return None
        return row * self.width + cols, vals

    def apply(self, flat: torch.Tensor, vals: torch.Tensor) -> None:
        """pool.flat[flat[i]] = vals[i] on the current stream (device int32 tensors)."""
        if self.pool.numel() >= 2 ** 31:
            raise ValueError("page-table pool too large for int32 entry indices")
        self.pool.view(-1).index_put_((flat.long(),), vals)

    def sync(self, seq: "Sequence", name: str) -> None:
        """Copy the page ids appended since the last sync; mark the ids a trim removed -1."""
        upd = self.updates(seq, name)
        if upd is not None:
            h = torch.from_numpy(np.stack(upd).astype(np.int32)).pin_memory()
            d = h.to(self.device, non_blocking=True)
            self.apply(d[0], d[1])

    def drop(self, seq: "Sequence", name: str) -> None:
        row = seq.rows.pop(name, None)
        if row is not None:
            written = seq.synced.pop(name, [0, 0])[1]
            if written:
                self.pool[row, :written].fill_(-1)
            self.free_rows.append(row)


class PagedKV:
    """Per-layer K/V caches [num_pages, page_size, Hkv, D] bf16 (serving/backend.py:46-48)."""

    def __init__(self, shape: ModelShape, num_pages: int, page_size: int, device):
        self.page_size = page_size
        self.num_pages = num_pages
        self.k = [torch.zeros(num_pages, page_size, shape.kv_heads, shape.head_dim, dtype=torch.bfloat16,
                              device=device) for _ in range(shape.layers)]
        self.v = [torch.zeros_like(t) for t in self.k]
        self.pool = PagePool(num_pages)
        self.tables = DevicePageTables(num_pages, device)


class Qwen3PagedModel(torch.nn.Module):
    """Random-initialised bf16 Qwen3-shaped model over a paged KV cache."""

    def __init__(self, shape: ModelShape, device, *, draft: bool, seed: int = 0, init_std: float = 0.02):
        super().__init__()
        self.shape, self.draft, self.device = shape, draft, torch.device(device)
        # Blocks of at most 64 tokens run their projections through
        # layers.project (the weight-streaming HIP GEMM where it is faster
        # than hipBLASLt) unless this is off.
        self.rows64_gemm = True
        g = torch.Generator(device=self.device).manual_seed(seed)
        h, d, Hq, Hkv = shape.hidden, shape.head_dim, shape.heads, shape.kv_heads

        def w(*dims):
            return (torch.randn(*dims, generator=g, device=self.device) * init_std).to(torch.bfloat16)

        def ones(n):
            return torch.ones(n, dtype=torch.bfloat16, device=self.device)

        self.embed = w(shape.vocab, h)
        self.layers = []
        for _ in range(shape.layers):
            self.layers.append(dict(
                qkv=w((Hq + 2 * Hkv) * d, h), o=w(h, Hq * d), gate_up=w(2 * shape.mlp, h),
                down=w(h, shape.mlp), ln1=ones(h), ln2=ones(h), qn=ones(d), kn=ones(d)))
        self.norm = ones(h)
        self.lm_head = w(shape.vocab, h)
        half = d // 2
        self.inv_freq = 1.0 / (shape.rope_theta ** (torch.arange(0, half, device=self.device,
                                                                   dtype=torch.float32) * 2 / d))

    def forward(self, ids: torch.Tensor, positions: torch.Tensor, kv: PagedKV, block_tables: torch.Tensor,
                context_lens: torch.Tensor, slot_mapping: torch.Tensor, *, causal: bool,
                max_context: int, q_vis: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Hidden states [B, Q, hidden] of a block of Q tokens per request.

        The block's K/V are appended at ``slot_mapping`` before attention;
        ``context_lens`` counts the prefix plus the block.  With ``q_vis``
        ([Q, 3] int32, device) the block is a packed multi-branch draft block
        and attention follows that per-query visibility; otherwise it is
        causal (verify) or bidirectional (draft recovery) within the block.  Per layer: fused
        add + RMSNorm, QKV GEMM, fused q/k norm + RoPE + KV append, paged
        attention, O GEMM, fused add + RMSNorm, gate-up GEMM, fused SiLU-mul,
        down GEMM (the decoder layer of serving/vendor/ssd/models/qwen3.py).
        Blocks of at most 64 tokens run the projections on the
        weight-streaming HIP GEMM where layers.project / gate_up_silu pick it
        (when ``rows64_gemm``: the QKV, O and down GEMMs, whose K-split
        partials the next fused kernel sums, and the draft's gate-up with the
        SiLU-mul fused in); the target's gate-up and larger blocks use
        F.linear.
        """
        B, Q = ids.shape
        s = self.shape
        Hq, Hkv, d = s.heads, s.kv_heads, s.head_dim
        pos = positions.reshape(-1)
        residual = F.embedding(ids.reshape(-1), self.embed)  # updated in place below
        hs = torch.empty_like(residual)
        x = None
        proj = ly.project if self.rows64_gemm else F.linear
        for li, L in enumerate(self.layers):
            ly.add_rmsnorm(x, residual, L["ln1"], s.eps, out=hs)
            qkv = proj(hs, L["qkv"])
            q = ly.qk_rope_append(qkv, pos, L["qn"], L["kn"], self.inv_freq, kv.k[li], kv.v[li], slot_mapping,
                                  Hq, Hkv, s.eps, draft_rope=self.draft)
            if q_vis is None:
                o = att.flash_attn_with_kvcache(q.view(B, Q, Hq, d), kv.k[li], kv.v[li], context_lens,
                                                block_tables, causal=causal, max_seqlen_k=max_context)
            else:
                o = att.packed_block_attn(q.view(B, Q, Hq, d), kv.k[li], kv.v[li], context_lens, block_tables,
                                          q_vis, max_seqlen_k=max_context)
            x = proj(o.reshape(B * Q, Hq * d), L["o"])
            ly.add_rmsnorm(x, residual, L["ln2"], s.eps, out=hs)
            act = ly.gate_up_silu(hs, L["gate_up"]) if self.rows64_gemm else ly.silu_mul(F.linear(hs, L["gate_up"]))
            x = proj(act, L["down"])
        out = ly.add_rmsnorm(x, residual, self.norm, s.eps)
        return out.reshape(B, Q, s.hidden)

    def logits(self, hidden: torch.Tensor) -> torch.Tensor:
        return F.linear(hidden, self.lm_head)


# -- page bookkeeping (serving/backend.py:55-76, :123-124) --------------------
class Sequence:
    """One request: token ids, committed prefix length and its page table."""

    def __init__(self, seq_id: int, token_ids: List[int]):
        self.seq_id = seq_id
        self.token_ids = list(token_ids)
        self.prefix = len(token_ids)
        self.pages: dict = {}  # model name -> list of page ids
        self.rows: dict = {}    # model name -> row of its device page-table pool
        self.synced: dict = {}  # model name -> [ids equal on the device, ids written there]


def reserve(kv: PagedKV, seq: Sequence, name: str, length: int) -> None:
    table = seq.pages.setdefault(name, [])
    missing = -(-length // kv.page_size) - len(table)
    if missing > 0:
        table.extend(kv.pool.alloc(missing))


def trim(kv: PagedKV, seq: Sequence, name: str, length: int) -> None:
    table = seq.pages.setdefault(name, [])
    keep = -(-length // kv.page_size)
    if len(table) > keep:
        kv.pool.release(table[keep:])
        del table[keep:]
        if name in seq.synced:  # the device row holds the trimmed ids past keep
            seq.synced[name][0] = min(seq.synced[name][0], keep)


def release(kv: PagedKV, seq: Sequence, name: str) -> None:
    kv.tables.drop(seq, name)
    kv.pool.release(seq.pages.pop(name, []))


def block_inputs(kv: PagedKV, seqs: List[Sequence], name: str, starts: List[int], Q: int, device,
                 width: Optional[int] = None, out: Optional[tuple] = None):
    """Page tables, slots and context lengths for a block of Q tokens at starts[b].

    ``width`` fixes the page-table width (and so the attention's context
    bound, width * page_size); by default it is the longest table.  The
    tables come from the device mirror: per step only the request rows and
    starts cross to the device, and one kernel gathers the tables and
    computes the slot mapping (serving/backend.py:73-76, :123-124).
    ``out`` = (tables [B, width] int32, slots [B*Q] int64, logical [B, Q]
    int64, lens [B] int32) receives the results in place (a block step's
    static buffers) instead of new tensors.
    """
    width = max(len(s.pages[name]) for s in seqs) if width is None else width
    if any(len(s.pages[name]) > width for s in seqs):
        raise ValueError("a page table is wider than the fixed width")
    from . import _lib
    dev = torch.device(device)
    T = kv.tables
    B = len(seqs)
    # One pinned buffer, one copy: the request rows and starts, then the
    # page-table entries to rewrite (appended pages, -1 over trimmed ones)
    # of every request.
    rows = [T.row(s, name) for s in seqs]
    upds = [u for u in (T.updates(s, name) for s in seqs) if u is not None]
    n = sum(len(u[0]) for u in upds)
    host = torch.empty(2 * B + 2 * n, dtype=torch.int32, pin_memory=True)
    hn = host.numpy()
    hn[:B] = rows
    hn[B:2 * B] = [int(x) for x in starts]
    if n:
        hn[2 * B:2 * B + n] = np.concatenate([u[0] for u in upds])
        hn[2 * B + n:] = np.concatenate([u[1] for u in upds])
    dh = host.to(dev, non_blocking=True)
    if n:
        T.apply(dh[2 * B:2 * B + n], dh[2 * B + n:])
    ri = dh[:2 * B].view(2, B)
    if out is None:
        tables = torch.empty(B, width, dtype=torch.int32, device=dev)
        slots = torch.empty(B * Q, dtype=torch.int64, device=dev)
        logical = torch.empty(B, Q, dtype=torch.int64, device=dev)
        lens = torch.empty(B, dtype=torch.int32, device=dev)
    else:
        tables, slots, logical, lens = out
        if (tuple(tables.shape) != (B, width) or tables.dtype != torch.int32 or slots.numel() != B * Q
                or slots.dtype != torch.int64 or tuple(logical.shape) != (B, Q) or logical.dtype != torch.int64
                or tuple(lens.shape) != (B,) or lens.dtype != torch.int32
                or not all(t.is_contiguous() and t.device == dev for t in out)):
            raise ValueError("block_inputs out buffers do not match the block")
    st = _lib.load().d3d_block_inputs(T.pool.data_ptr(), T.pool.shape[0], T.width, ri[0].data_ptr(),
                                      ri[1].data_ptr(), B, int(Q), int(width), kv.page_size, tables.data_ptr(),
                                      slots.data_ptr(), logical.data_ptr(), lens.data_ptr(), _lib.stream_ptr(dev))
    _lib.check(st, "d3d_block_inputs")
    return tables, slots, lens, logical, width * kv.page_size


_WARMUP: dict = {}


def _warmup_stream(device) -> torch.cuda.Stream:
    """One side stream per device for pre-capture warm-ups."""
    key = torch.device(device).index
    if key not in _WARMUP:
        _WARMUP[key] = torch.cuda.Stream(device)
    return _WARMUP[key]


class BlockStep:
    """A block forward plus a post-processing function over static device
    buffers, replayed from a HIP graph after the first call.

    The forward issues some 60 small operations per layer; replaying them
    as one graph removes the per-launch host cost.  Inputs are copied into
    the static buffers before each replay; the KV cache, page tables and
    context lengths are read from device memory by the kernels, so one
    capture serves every step with the same (B, Q, table width).  Outputs
    live in the graph's memory pool and are overwritten by the next replay.
    """

    def __init__(self, model: "Qwen3PagedModel", kv: PagedKV, B: int, Q: int, width: int, causal: bool,
                 post=None, use_graph: bool = True, q_vis: Optional[torch.Tensor] = None):
        dev = model.device
        self.device = dev
        self.model, self.kv, self.causal, self.post, self.use_graph = model, kv, causal, post, use_graph
        self.q_vis = None if q_vis is None else q_vis.to(dev, torch.int32).contiguous()
        self.ids = torch.zeros(B, Q, dtype=torch.int64, device=dev)
        self.pos = torch.zeros(B, Q, dtype=torch.int64, device=dev)
        self.tables = torch.zeros(B, width, dtype=torch.int32, device=dev)
        self.slots = torch.zeros(B * Q, dtype=torch.int64, device=dev)
        self.lens = torch.ones(B, dtype=torch.int32, device=dev)
        self.max_ctx = width * kv.page_size
        self.graph = None
        self.out = None
        self.workspaces: list = []
        self.prepared = None  # the requests whose block inputs the static buffers hold
        from .streams import register_graph_owner
        register_graph_owner(self)

    def release(self) -> None:
        """Drop the captured graph, its outputs and its workspaces (the next
        call captures again)."""
        self.graph = None
        self.out = None
        self.workspaces.clear()

    def _body(self):
        hidden = self.model(self.ids, self.pos, self.kv, self.tables, self.lens, self.slots, causal=self.causal,
                            max_context=self.max_ctx, q_vis=self.q_vis)
        return self.post(hidden, self.ids) if self.post is not None else None

    def _load(self, ids, pos, tables, slots, lens):
        self.ids.copy_(ids, non_blocking=True)
        self.pos.copy_(pos, non_blocking=True)
        self.tables.copy_(tables, non_blocking=True)
        self.slots.copy_(slots, non_blocking=True)
        self.lens.copy_(lens, non_blocking=True)

    def __call__(self, ids, pos, tables, slots, lens):
        # Always under inference mode: torch keeps per-generator graph state
        # tensors that a first capture creates, and a later capture outside
        # the mode they were created in cannot update them in place.
        with torch.inference_mode():
            return self._call(ids, pos, tables, slots, lens)

    def _call(self, ids, pos, tables, slots, lens):
        self._load(ids, pos, tables, slots, lens)
        return self._replay()

    def inputs(self) -> tuple:
        """The static (tables, slots, positions, lens) buffers, in
        ``block_inputs``'s ``out`` order."""
        return self.tables, self.slots, self.pos, self.lens

    def run(self, ids, pos=None):
        """Replay on token ids (and positions) given as host arrays, after
        ``block_inputs(..., out=self.inputs())`` has filled the page tables,
        slots, context lengths and default positions on the stream.  The
        host arrays cross in one pinned copy each."""
        with torch.inference_mode():
            _stage(self.ids, ids)
            if pos is not None:
                _stage(self.pos, pos)
            return self._replay()

    def _replay(self):
        if not self.use_graph:
            return self._body()
        if self.graph is None:
            bufs = (self.ids, self.pos, self.tables, self.slots, self.lens)
            saved = [t.clone() for t in bufs]
            cur = torch.cuda.current_stream(self.model.device)
            side = _warmup_stream(self.model.device)
            side.wait_stream(cur)
            with torch.cuda.stream(side):  # warm-up outside the capture
                self._body()
            cur.wait_stream(side)
            g = torch.cuda.CUDAGraph()
            # Workspaces used by the captured kernels belong to this step.
            with _lib.capture_workspaces(self.workspaces), torch.cuda.graph(g):
                self.out = self._body()
            self.graph = g
            # The warm-up may have updated the static inputs in place.
            for t, v in zip(bufs, saved):
                t.copy_(v)
        self.graph.replay()
        return self.out


def _stage(dst: torch.Tensor, src) -> None:
    """dst (device, int64) <- src (host list, numpy array or tensor) through
    a pinned buffer, queued on the current stream."""
    if isinstance(src, torch.Tensor) and src.is_cuda:
        dst.copy_(src.reshape(dst.shape), non_blocking=True)
        return
    arr = src.numpy() if isinstance(src, torch.Tensor) else np.asarray(src)
    if arr.size != dst.numel():
        raise ValueError(f"expected {tuple(dst.shape)} values, got {arr.shape}")
    h = torch.empty(dst.shape, dtype=torch.int64, pin_memory=True)
    h.numpy()[...] = arr.reshape(dst.shape)
    dst.copy_(h, non_blocking=True)


def prefill(model: Qwen3PagedModel, kv: PagedKV, seqs: List[Sequence], name: str, block: int = 16) -> torch.Tensor:
    """Writes the prompts' K/V and returns the last prompt position's hidden state [B, hidden].

    The prefill of serving/backend.py:98-112 for prompts of any lengths >= 1
    on the block kernel: prompt b of n tokens is cut into J = ceil(n / block)
    slices aligned to its end; slice j starts at n - block (J - j) and runs
    as a request of ``block`` queries whose context is start + block, so
    query i sees positions <= start + i (causal attention over the prompt).
    Rows of the first slice before position 0 are padding: their slot is -1
    (no K/V written) and they see no key.
    """
    dev = model.device
    lens = [len(s.token_ids) for s in seqs]
    if min(lens) < 1:
        raise ValueError("prefill needs prompts of at least one token")
    for s, n in zip(seqs, lens):
        reserve(kv, s, name, n)
    rows, starts, ids, last = [], [], [], []
    for s, n in zip(seqs, lens):
        J = -(-n // block)
        toks = s.token_ids
        for j in range(J):
            st = n - block * (J - j)
            rows.append(s)
            starts.append(st)
            ids.append([toks[p] if p >= 0 else 0 for p in range(st, st + block)])
        last.append(len(rows) - 1)
    ids_t = torch.tensor(ids, dtype=torch.int64).to(dev, non_blocking=True)
    tables, slots, ctx, logical, max_ctx = block_inputs(kv, rows, name, starts, block, dev)
    hidden = model(ids_t, logical, kv, tables, ctx, slots, causal=True, max_context=max_ctx)
    return hidden[torch.tensor(last, device=dev), -1]
