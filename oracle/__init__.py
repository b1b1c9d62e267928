"""ORACLE -- test infrastructure only.

CPU restatements of D3D's per-step hot path, against which the tests compare
the gfx950 kernels.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package; the product
(``d3d_amd``) never does.

* ``accept_oracle.c`` (built into ``liboracle.so`` by ``oracle/Makefile``):
  fp64 acceptance, greedy acceptance, inverse CDF, confidence/top-k unmask.
* ``attention.py``: fp64 numpy paged attention (causal verify and
  bidirectional draft block) over a logical gather of the pages.
* ``torch_ref.py``: fp32 torch-CPU line-by-line restatement of
  ``single/speculative_sampling.py`` with explicit uniforms (the CPU
  baseline and a second, independently rounded check).
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

KIND_LOGITS = 0
KIND_PROBS = 1

_lib = None


def build() -> Path:
    """Compile liboracle.so with gcc (via oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "-B", "liboracle.so"], check=True)
    return LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(LIB_PATH))
        P, I, L, D = ctypes.c_void_p, ctypes.c_int, ctypes.c_long, ctypes.c_double
        lib.oracle_argmax_f32.restype = L
        lib.oracle_argmax_f32.argtypes = [P, L]
        lib.oracle_row_probs.restype = None
        lib.oracle_row_probs.argtypes = [P, L, I, D, P]
        lib.oracle_inverse_cdf.restype = L
        lib.oracle_inverse_cdf.argtypes = [P, L, D, P]
        lib.oracle_accept_dense.restype = None
        lib.oracle_accept_dense.argtypes = [P, P, I, D, P, P, P, I, I, L, P, P, P, P, P, P]
        lib.oracle_accept_sparse.restype = None
        lib.oracle_accept_sparse.argtypes = [P, I, D, P, P, P, I, P, P, I, I, L, P, P, P, P, P, P]
        lib.oracle_accept_greedy.restype = None
        lib.oracle_accept_greedy.argtypes = [P, P, I, I, L, P, P, P, P, P]
        lib.oracle_confidence_topk.restype = None
        lib.oracle_confidence_topk.argtypes = [P, P, ctypes.c_int64, I, D, I, I, D, I, I, L, P, P]
        lib.oracle_select_transfer.restype = None
        lib.oracle_select_transfer.argtypes = [P, ctypes.c_int64, I, I, D, P, P, P, I]
        _lib = lib
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _i64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int64))


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def argmax(x) -> int:
    x = _f32(x)
    return int(_load().oracle_argmax_f32(_p(x), x.size))


def row_probs(x, kind: int = KIND_LOGITS, temperature: float = 1.0) -> np.ndarray:
    x = _f32(x)
    p = np.empty(x.size, dtype=np.float64)
    _load().oracle_row_probs(_p(x), x.size, kind, float(temperature), _p(p))
    return p


def inverse_cdf(w, v: float):
    """(token, margin) of the inverse-CDF draw over unnormalised fp64 weights."""
    w = np.ascontiguousarray(np.asarray(w, dtype=np.float64))
    m = np.zeros(1, dtype=np.float64)
    t = _load().oracle_inverse_cdf(_p(w), w.size, float(v), _p(m))
    return int(t), float(m[0])


def accept_dense(target, draft, tokens, uniforms, resample_u, *, kind=KIND_LOGITS, temperature=1.0):
    """fp64 dense acceptance; arrays [B,K+1,V], [B,K,V], [B,K], [B,K], [B]."""
    t, d = _f32(target), _f32(draft)
    tok, u, ru = _i64(tokens), _f32(uniforms), _f32(resample_u)
    B, K1, V = t.shape
    K = K1 - 1
    out = dict(
        accept_mask=np.zeros((B, K), np.uint8), accepted=np.zeros(B, np.int32),
        out_token=np.zeros(B, np.int64), all_accepted=np.zeros(B, np.uint8),
        u_margin=np.zeros(B, np.float64), cdf_margin=np.zeros(B, np.float64),
    )
    _load().oracle_accept_dense(
        _p(t), _p(d), kind, float(temperature), _p(tok), _p(u), _p(ru), B, K, V,
        _p(out["accept_mask"]), _p(out["accepted"]), _p(out["out_token"]),
        _p(out["all_accepted"]), _p(out["u_margin"]), _p(out["cdf_margin"]),
    )
    return out


def accept_sparse(target, tokens, q_ids, q_probs, uniforms, resample_u, *, kind=KIND_PROBS, temperature=1.0):
    """fp64 sparse-proposal acceptance; q_ids/q_probs [B,K,S]."""
    t, tok, qi, qp = _f32(target), _i64(tokens), _i64(q_ids), _f32(q_probs)
    u, ru = _f32(uniforms), _f32(resample_u)
    B, K1, V = t.shape
    K, S = K1 - 1, qi.shape[2]
    out = dict(
        accept_mask=np.zeros((B, K), np.uint8), accepted=np.zeros(B, np.int32),
        out_token=np.zeros(B, np.int64), all_accepted=np.zeros(B, np.uint8),
        u_margin=np.zeros(B, np.float64), cdf_margin=np.zeros(B, np.float64),
    )
    _load().oracle_accept_sparse(
        _p(t), kind, float(temperature), _p(tok), _p(qi), _p(qp), S, _p(u), _p(ru), B, K, V,
        _p(out["accept_mask"]), _p(out["accepted"]), _p(out["out_token"]),
        _p(out["all_accepted"]), _p(out["u_margin"]), _p(out["cdf_margin"]),
    )
    return out


def accept_greedy(target, tokens):
    """Greedy acceptance; target [B,K+1,V], tokens [B,K]."""
    t, tok = _f32(target), _i64(tokens)
    B, K1, V = t.shape
    K = K1 - 1
    out = dict(
        posterior=np.zeros((B, K1), np.int64), accept_mask=np.zeros((B, K), np.uint8),
        accepted=np.zeros(B, np.int32), out_token=np.zeros(B, np.int64),
        all_accepted=np.zeros(B, np.uint8),
    )
    _load().oracle_accept_greedy(
        _p(t), _p(tok), B, K, V, _p(out["posterior"]), _p(out["accept_mask"]),
        _p(out["accepted"]), _p(out["out_token"]), _p(out["all_accepted"]),
    )
    return out


def confidence_topk(logits, block, mask_id: int, k: int, temperature: float = 0.0, *, one_hot: bool = False,
                    dynamic: bool = False, threshold: float = 0.0):
    """One unmask iteration; returns (new_block, x0, conf)."""
    x = _f32(logits)
    blk = _i64(block).copy()
    B, Q, V = x.shape
    x0 = np.zeros((B, Q), np.int64)
    conf = np.zeros((B, Q), np.float32)
    _load().oracle_confidence_topk(_p(x), _p(blk), int(mask_id), int(k), float(temperature), int(one_hot),
                                   int(dynamic), float(threshold), B, Q, V, _p(x0), _p(conf))
    return blk, x0, conf


def select_transfer(block, mask_id: int, k: int, x0, conf, *, dynamic: bool = False, threshold: float = 0.0):
    """_select_transfer per request with given x0 / conf [B, Q]; returns
    (new_block, selected [B, Q] bool)."""
    blk = _i64(block).copy()
    B, Q = blk.shape
    x0 = _i64(x0).reshape(B, Q)
    cf = _f32(conf).reshape(B, Q)
    sel = np.zeros((B, Q), np.uint8)
    for b in range(B):
        _load().oracle_select_transfer(_p(blk[b]), int(mask_id), int(k), int(dynamic), float(threshold),
                                       _p(x0[b]), _p(cf[b]), _p(sel[b]), Q)
    return blk, sel.astype(bool)


def num_transfer_tokens(num_masks: int, steps: int):
    """single/eval_sync.py:440-444: even split, remainder to the first steps."""
    steps = max(1, int(steps))
    base, extra = divmod(int(num_masks), steps)
    return [base + (1 if i < extra else 0) for i in range(steps)]


def topk_keep(x, temperature: float, top_k: int) -> np.ndarray:
    """The top-k filter of _sampling_probs (single/eval_sync.py:292-295) on
    one fp32 row: z = x / T in fp32 (the reference's logits.float() / T),
    kth = the k-th largest z counting repeats (torch.topk(...).values[-1]),
    keep z >= kth (ties with the k-th value are kept)."""
    z = _f32(x) / np.float32(temperature)
    if not top_k or top_k <= 0:
        return np.ones(z.shape, bool)
    kth = np.sort(z)[::-1][min(int(top_k), z.size) - 1]
    return z >= kth


def filter_keep(x, temperature: float, top_k: int = 0, top_p: float = 1.0):
    """The entries _sampling_probs keeps (single/eval_sync.py:292-303) on one
    fp32 row, and the top-p decision margin.

    z = x / T in fp32 (the reference's logits.float() / T).  Top-k keeps z >=
    the k-th largest z (ties kept).  Top-p (< 1) orders the kept entries by z
    descending -- ties by ascending id, the order of a stable sort -- takes
    their fp64 softmax and its running sum c, and keeps entry j iff j == 0 or
    c[j - 1] <= top_p (so the entry that first exceeds top_p stays).
    Returns (keep [V] bool, margin): margin = min_j |c[j] - top_p| over the
    sorted entries (inf when top-p is off), so a fixture whose margin exceeds
    the kernels' rounding cannot be decided differently by them."""
    x = _f32(x)
    keep = topk_keep(x, temperature, top_k)
    margin = np.inf
    if top_p is not None and top_p < 1.0:
        z = x / np.float32(temperature)
        idx = np.flatnonzero(keep)
        order = idx[np.lexsort((idx, -z[idx].astype(np.float64)))]
        zz = z[order].astype(np.float64)
        e = np.exp(zz - zz.max())
        c = np.cumsum(e / e.sum())
        margin = float(np.min(np.abs(c - top_p)))
        before = np.concatenate([[0.0], c[:-1]])
        drop = order[(before > top_p) & (np.arange(order.size) > 0)]
        keep = keep.copy()
        keep[drop] = False
    return keep, margin


def softmax_rows(logits, temperature: float, top_k: int = 0, top_p: float = 1.0) -> np.ndarray:
    """_sampling_probs (single/eval_sync.py:287-305), fp64: one-hot at the
    first argmax for T <= 1e-5, else softmax(x / T) over the entries
    filter_keep keeps, 0 elsewhere.  [N, V] -> [N, V]."""
    x = _f32(logits).reshape(-1, np.asarray(logits).shape[-1])
    out = np.zeros(x.shape, np.float64)
    for n in range(x.shape[0]):
        if temperature <= 1e-5:
            out[n, argmax(x[n])] = 1.0
            continue
        keep, _ = filter_keep(x[n], temperature, top_k, top_p)
        z = x[n].astype(np.float64) / temperature
        e = np.where(keep, np.exp(z - z[keep].max()), 0.0)
        out[n] = e / e.sum()
    return out


def filter_margins(logits, temperature: float, top_k: int = 0, top_p: float = 1.0) -> np.ndarray:
    """filter_keep's top-p margin of every row of [N, V]."""
    x = _f32(logits).reshape(-1, np.asarray(logits).shape[-1])
    return np.array([filter_keep(r, temperature, top_k, top_p)[1] for r in x])


def sample_with_prob(logits, temperature: float, uniforms, top_k: int = 0, top_p: float = 1.0):
    """single/eval_sync.py:324-338 (_sample_with_prob over _sampling_probs),
    with torch.multinomial replaced by the inverse CDF of each row's fp64
    softmax at u[n] (over the top-k kept entries when top_k > 0).  Returns
    (tokens, probs, margins) per row of [N, V]; T <= 1e-5 gives the argmax
    with probability 1 (margin inf)."""
    x = _f32(logits).reshape(-1, np.asarray(logits).shape[-1])
    u = np.asarray(uniforms, np.float64).reshape(-1)
    N = x.shape[0]
    tok = np.zeros(N, np.int64)
    prob = np.zeros(N, np.float64)
    margin = np.full(N, np.inf)
    for n in range(N):
        filtered = top_k or (top_p is not None and top_p < 1.0)
        p = softmax_rows(x[n][None], temperature, top_k, top_p)[0] if filtered else row_probs(x[n], KIND_LOGITS,
                                                                                                 temperature)
        if temperature <= 1e-5:
            tok[n] = int(np.argmax(p))
        else:
            tok[n], margin[n] = inverse_cdf(p, u[n])
        prob[n] = p[tok[n]]
    return tok, prob, margin


def sample_sparse(logits, temperature: float, S: int, uniforms, top_p: float = 1.0):
    """single/eval_sync.py:341-367 (_sample_with_sparse_probs), fp64: the S
    largest entries of z = logits / T (z in fp32, the reference's
    logits.float() / T; descending, ties by lower id), softmax over them, the
    nucleus filter (entry s > 0 dropped when the inclusive mass of entries
    0..s-1 exceeds top_p, then renormalised), inverse-CDF draw at u[n].
    Returns (tokens, ids [N,S], probs [N,S], margins); the margin is the
    draw's, and with top_p < 1 also the nucleus cut's (min |C_s - top_p|)."""
    x = _f32(logits).reshape(-1, np.asarray(logits).shape[-1])
    u = np.asarray(uniforms, np.float64).reshape(-1)
    N, V = x.shape
    ids = np.zeros((N, S), np.int64)
    probs = np.zeros((N, S), np.float64)
    tok = np.zeros(N, np.int64)
    margin = np.zeros(N)
    for n in range(N):
        z32 = x[n] / np.float32(temperature)
        order = np.lexsort((np.arange(V), -z32.astype(np.float64)))[:S]
        zs = z32[order].astype(np.float64)
        e = np.exp(zs - zs.max())
        ids[n] = order
        probs[n] = e / e.sum()
        cut = np.inf
        if top_p < 1.0:
            c = np.cumsum(probs[n])
            cut = float(np.min(np.abs(c - top_p)))
            before = np.concatenate([[0.0], c[:-1]])
            e = np.where(before > top_p, 0.0, e)
            probs[n] = e / e.sum()
        local, margin[n] = inverse_cdf(probs[n], u[n])
        margin[n] = min(margin[n], cut)
        tok[n] = order[local]
    return tok, ids, probs, margin
