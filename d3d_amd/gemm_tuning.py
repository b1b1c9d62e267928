"""Library-GEMM solution choices for the engine's fixed projection shapes.

The projections that stay on the BLAS libraries (F.linear: the 1088-row
packed-predict projections and LM head, the 64-row target qkv and gate-up
and both LM heads) run whatever solution hipBLASLt's heuristic returns for
the shape.  PyTorch's TunableOp times every hipBLASLt and rocBLAS solution
of a shape (the heuristic's default among them) on rotating HBM-resident
operands and keeps the fastest; ``tune`` does that for the engine's step
shapes and writes the results file, ``enable`` makes torch use the file's
choices (tuning itself stays off, so no shape is timed at run time and
shapes the file does not list keep the default solution).  The packed
predict's qkv and down projections and the verify's gate-up are the
exception: the two forwards run side by side, and the file lists these on
the library default, which slows the other stream less than their
fastest-alone choices (``corun_default_shapes``).

The choice changes the solution, not the operation: outputs stay within the
usual bf16 GEMM rounding of one another, not bit-equal across solutions.

Run on the GPU the engine serves on (the file's validator lines pin the
torch, HIP, hipBLASLt and rocBLAS versions and the gfx arch; ``enable``
ignores a file that does not match)::

    python -m d3d_amd.gemm_tuning [--out PATH] [--duration MS]
"""
from __future__ import annotations

import argparse
import os
import sys
import tempfile
import time
import warnings
from pathlib import Path
from typing import Iterable, List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

RESULTS = Path(__file__).with_name("gemm_tuned_gfx950.csv")
_enabled: Optional[Path] = None


def step_gemm_shapes(target, draft, block: int = 16, batches: Iterable[int] = (1, 2, 3, 4),
                     anchors: Iterable[int] = (1, 3)) -> List[Tuple[int, int, int]]:
    """(M, N, K) of every library GEMM of an engine step, for the given
    batch sizes and anchor counts: the target's verify and the draft's
    recovery over ``block`` rows per request (the projections that
    layers.project leaves to hipBLASLt, plus the LM heads), and the draft's
    packed predict over ``block * (2 + A * (block - 1))`` rows per request
    (every projection and the LM head).  Sorted, without repeats."""
    from .layers import ROWS64, rows64_splits

    def projections(s):
        q, kv = s.heads * s.head_dim, s.kv_heads * s.head_dim
        return [(q + 2 * kv, s.hidden), (s.hidden, q), (2 * s.mlp, s.hidden), (s.hidden, s.mlp),
                (s.vocab, s.hidden)]

    out = set()
    for b in batches:
        M = block * b
        for s in (target, draft):
            for N, K in projections(s):
                if N == s.vocab or M > ROWS64 or not rows64_splits(N, K):
                    out.add((M, N, K))
        for A in anchors:
            Mp = b * block * (2 + A * (block - 1))
            out.update((Mp, N, K) for N, K in projections(draft))
    return sorted(out)


def corun_default_shapes(target, draft, block: int = 16, batches: Iterable[int] = (1, 2, 3, 4),
                         anchors: Iterable[int] = (1, 3)) -> List[Tuple[int, int, int]]:
    """The shapes that keep the library heuristic's default solution
    ("Default" in the results file) instead of the fastest one alone: the
    packed predict's qkv and down projections and the verify's gate-up.

    The packed predict and the verify run side by side on the two streams,
    and these fastest-alone choices slow the other stream more than they
    gain.  Beside a loop of the tuned 1088-row qkv, the target's o
    projection takes 20.3 us a call against 16.4 beside the default (10.1
    alone).  Engine loop (B=4, A=1, 96 new tokens, twelve runs each,
    alternating processes on one box): 86.2-86.9 steps/s with every shape
    tuned, 88.0-88.8 with the predict qkv and down on the default; then,
    on another box, 89.4-90.1 against 90.2-90.8 with the verify's gate-up
    on the default as well."""
    out = set()
    q, kv = draft.heads * draft.head_dim, draft.kv_heads * draft.head_dim
    for b in batches:
        out.add((b * block, 2 * target.mlp, target.hidden))
        for A in anchors:
            Mp = b * block * (2 + A * (block - 1))
            out.update({(Mp, q + 2 * kv, draft.hidden), (Mp, draft.hidden, draft.mlp)})
    return sorted(out)


def enable(path: Path = RESULTS) -> bool:
    """Use the solution choices in ``path`` for every matching torch GEMM of
    this process (TunableOp on, tuning off).  Returns False, leaving torch's
    defaults, when there is no GPU, no file, or the file was made with other
    library versions or another GPU."""
    global _enabled
    path = Path(path)
    if not torch.cuda.is_available() or not path.is_file():
        return False
    tun = torch.cuda.tunable
    if _enabled == path and tun.is_enabled() and not tun.tuning_is_enabled():
        return True
    tun.enable(True)
    tun.tuning_enable(False)
    try:
        ok = bool(tun.read_file(str(path)))
    except Exception as exc:  # a malformed or foreign file
        warnings.warn(f"GEMM tuning results {path} not loaded: {exc}")
        ok = False
    if not ok:
        tun.enable(False)
        return False
    _enabled = path
    return True


def state() -> Tuple[bool, bool, Optional[Path]]:
    """TunableOp's process-wide switches (enabled, tuning enabled) and the
    results file ``enable`` loaded, for :func:`restore`."""
    if not torch.cuda.is_available():
        return (False, False, None)
    tun = torch.cuda.tunable
    return (bool(tun.is_enabled()), bool(tun.tuning_is_enabled()), _enabled)


def restore(saved: Tuple[bool, bool, Optional[Path]]) -> None:
    """Put TunableOp's switches back as :func:`state` recorded them.  The
    solution choices ``enable`` read stay in torch's table but are used only
    while TunableOp is on."""
    global _enabled
    if not torch.cuda.is_available():
        return
    on, tuning, path = saved
    tun = torch.cuda.tunable
    tun.enable(on)
    tun.tuning_enable(tuning)
    _enabled = path if on else None


def disable() -> None:
    """Back to the libraries' default solutions."""
    global _enabled
    if torch.cuda.is_available():
        torch.cuda.tunable.enable(False)
    _enabled = None


def _time_default(M: int, N: int, K: int, calls: int = 50) -> float:
    """Milliseconds per F.linear call on the library's default solution
    (TunableOp off)."""
    dev = torch.device("cuda:0")
    tun = torch.cuda.tunable
    was = tun.is_enabled()
    tun.enable(False)
    try:
        g = torch.Generator(device=dev).manual_seed(1)
        x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        w = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        for _ in range(5):
            F.linear(x, w)
        torch.cuda.synchronize(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(calls):
            F.linear(x, w)
        e1.record()
        torch.cuda.synchronize(dev)
        return e0.elapsed_time(e1) / calls
    finally:
        tun.enable(was)


def write_defaults(path: Path, shapes: Sequence[Tuple[int, int, int]], log=print) -> None:
    """Set ``shapes`` to the library default in the results file at
    ``path`` (replacing their lines, or adding them), each with its
    milliseconds per call timed on one operand set (cache-warm, unlike the
    tuner's rotating operands; the figure is informational)."""
    lines = [l for l in Path(path).read_text().splitlines() if l.strip()]
    keys = {f"tn_{N}_{M}_{K}_ld_{K}_{K}_{N}": (M, N, K) for M, N, K in shapes}
    kept = [l for l in lines if l.startswith("Validator,") or l.split(",")[1] not in keys]
    res = [l for l in kept if not l.startswith("Validator,")]
    for key, (M, N, K) in keys.items():
        ms = _time_default(M, N, K)
        res.append(f"GemmTunableOp_BFloat16_TN,{key},Default,{ms}")
        log(f"default M={M} N={N} K={K}: {ms * 1e3:.1f} us")
    val = [l for l in kept if l.startswith("Validator,")]
    res.sort(key=lambda l: l.split(",")[1])
    Path(path).write_text("\n".join(val + res) + "\n")


def tune(shapes: Sequence[Tuple[int, int, int]], out: Path = RESULTS, duration_ms: int = 150,
         rotating_mb: int = 512, log=print, keep_default: Sequence[Tuple[int, int, int]] = ()) -> None:
    """Tune F.linear(x [M, K], w [N, K]) in bf16 for each shape and write the
    validators and results to ``out``; shapes in ``keep_default`` are not
    tuned but written as the library default (``write_defaults``)."""
    keep = set(keep_default)
    shapes = [s for s in shapes if s not in keep]
    dev = torch.device("cuda:0")
    tun = torch.cuda.tunable
    tun.enable(True)
    tun.tuning_enable(True)
    tun.set_max_tuning_duration(duration_ms)
    tun.set_rotating_buffer_size(rotating_mb)
    # TunableOp also writes its own copy at process exit: keep that out of the
    # package directory.
    tun.set_filename(os.path.join(tempfile.gettempdir(), f"d3d_tunableop_{os.getpid()}.csv"))
    g = torch.Generator(device=dev).manual_seed(0)
    for M, N, K in shapes:
        x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        w = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        t0 = time.perf_counter()
        F.linear(x, w)
        torch.cuda.synchronize(dev)
        log(f"tuned M={M} N={N} K={K} in {time.perf_counter() - t0:.1f} s")
        del x, w
        torch.cuda.empty_cache()
    tun.tuning_enable(False)
    lines = [f"Validator,{k},{v}" for k, v in tun.get_validators()]
    lines += [f"{op},{params},{kernel},{ms}" for op, params, kernel, ms in sorted(tun.get_results())]
    Path(out).write_text("\n".join(lines) + "\n")
    if keep:
        write_defaults(out, sorted(keep), log=log)
    log(f"wrote {out}")


def main(argv=None) -> int:
    from .model import D3D_1P7B, QWEN3_8B
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--out", type=Path, default=RESULTS)
    ap.add_argument("--duration", type=int, default=150, help="tuning milliseconds per shape and solution set")
    ap.add_argument("--defaults-only", action="store_true",
                    help="only rewrite the library-default lines of an existing results file")
    args = ap.parse_args(argv)
    log = lambda s: print(s, flush=True)
    keep = corun_default_shapes(QWEN3_8B, D3D_1P7B)
    if args.defaults_only:
        write_defaults(args.out, keep, log=log)
        return 0
    shapes = step_gemm_shapes(QWEN3_8B, D3D_1P7B)
    print(f"{len(shapes)} shapes", flush=True)
    tune(shapes, args.out, args.duration, log=log, keep_default=keep)
    return 0


if __name__ == "__main__":
    sys.exit(main())
