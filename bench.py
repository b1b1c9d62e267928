"""Benchmark of the per-step speculative hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

One step is one pass of the hot path over one batch of synthetic input with
inputs resident in HBM: the fused acceptance of a batch-1 block of 16 target
rows and 15 draft rows over the 151,936-entry vocabulary (fp32 logits,
temperature 1).  Prints ONE JSON line.

The roofline entry is for the fused acceptance call (stats + resample
kernels, one launch each): algorithmic bytes = (16 + 15) rows x V x 4 B =
18,840,064 B per call, divided by the call's average duration from HIP events
recorded on the launch stream around the timed steps.

The CPU baseline times the fp32 torch-CPU restatement of the reference
acceptance (softmax of both logit blocks, then single/speculative_sampling.py
arithmetic) on a bounded number of calls of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

HBM_PEAK_GBPS = 8000.0


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    return ap.parse_args()


class AcceptStep:
    """Pre-bound fused-acceptance call (no Python-side allocation per step)."""

    def __init__(self, inp, temperature: float, dev):
        from d3d_amd import _lib
        self.lib = _lib.load()
        self.t = inp.target.to(dev).contiguous()
        self.d = inp.draft.to(dev).contiguous()
        self.tok = inp.tokens.to(dev)
        self.u = inp.uniforms.to(dev)
        self.ru = inp.resample_u.to(dev)
        B, K1, V = self.t.shape
        K = K1 - 1
        self.shape = (B, K, V)
        self.acc = torch.empty(B, dtype=torch.int32, device=dev)
        self.mask = torch.empty(B, K, dtype=torch.uint8, device=dev)
        self.tokout = torch.empty(B, dtype=torch.int64, device=dev)
        self.alla = torch.empty(B, dtype=torch.uint8, device=dev)
        self.post = torch.empty(B, K1, dtype=torch.int64, device=dev)
        n = self.lib.d3d_accept_workspace_bytes(B, K, V)
        self.ws = torch.zeros(n, dtype=torch.uint8, device=dev)
        self.stream = torch.cuda.current_stream(dev).cuda_stream
        self.args = (
            self.t.data_ptr(), self.d.data_ptr(), _lib.D3D_DTYPE_F32, _lib.D3D_INPUT_LOGITS,
            self.tok.data_ptr(), self.u.data_ptr(), self.ru.data_ptr(), float(temperature), B, K, V,
            self.acc.data_ptr(), self.mask.data_ptr(), self.tokout.data_ptr(), self.alla.data_ptr(),
            self.post.data_ptr(), self.ws.data_ptr(), n, self.stream,
        )
        self.greedy = temperature <= 1e-5
        self._check = _lib.check

    def __call__(self):
        st = self.lib.d3d_accept_fused(*self.args)
        if st:
            self._check(st, "d3d_accept_fused")

    def algorithmic_bytes(self) -> int:
        B, K, V = self.shape
        rows = B * (K + 1) + (0 if self.greedy else B * K)
        return rows * V * 4


def time_calls(fn, steps: int, warmup: int, dev) -> float:
    """Average milliseconds per call from events on the launch stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize(dev)
    s = torch.cuda.current_stream(dev)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(s)
    for _ in range(steps):
        fn()
    end.record(s)
    torch.cuda.synchronize(dev)
    return start.elapsed_time(end) / steps


def cpu_baseline(seconds: float):
    """fp32 torch-CPU restatement of the reference acceptance, batch 1, T = 1."""
    from d3d_amd import workloads
    from oracle import torch_ref
    inp = workloads.accept_inputs(1234, B=1, K=15)
    threads = torch.get_num_threads()

    def once():
        p = torch_ref.sampling_probs(inp.target, 1.0)
        q = torch_ref.sampling_probs(inp.draft, 1.0)
        torch_ref.verify_block(inp.tokens, p, q, inp.uniforms, float(inp.resample_u[0]))

    for _ in range(2):
        once()
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        once()
        n += 1
    us = (time.perf_counter() - t0) / n * 1e6
    return {
        "value": round(us, 1), "unit": "us/call", "cores": threads, "kind": "port",
        "sample": f"{n} calls of batch-1 T=1 acceptance (16+15 rows x 151936 fp32 logits), "
                  f"torch CPU fp32 restatement, {threads} threads",
    }


def main():
    args = _parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); "
              "multi-GPU runs are not part of this build", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    from d3d_amd import workloads

    inp = workloads.accept_inputs(1234, B=1, K=15, device="cuda")
    step = AcceptStep(inp, 1.0, dev)
    ms = time_calls(step, args.steps, args.warmup, dev)
    nbytes = step.algorithmic_bytes()
    gbps = nbytes / (ms * 1e-3) / 1e9

    # Secondary figures (not the headline): greedy acceptance, batch-8 acceptance.
    g_inp = workloads.accept_inputs(1234, B=1, K=15, temperature=0.0, device="cuda")
    g_step = AcceptStep(g_inp, 0.0, dev)
    g_ms = time_calls(g_step, args.steps, args.warmup, dev)
    b8_inp = workloads.accept_inputs(1234, B=8, K=15, device="cuda")
    b8_step = AcceptStep(b8_inp, 1.0, dev)
    b8_ms = time_calls(b8_step, args.steps, args.warmup, dev)

    out = {
        "metric": "accept-kernel us & HBM GB/s; verify-attn TFLOP/s; draft+verify steps/s at 1 GPU",
        "value": round(1e3 / ms, 1),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "fused acceptance, batch 1, 16 target + 15 draft rows, vocab 151936, "
                        "fp32 logits N(0,4), draft = target + N(0,0.25), T=1, seeded uniforms",
            "global_batch": 1,
            "draft_block": 16,
            "vocab": 151936,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "traffic": None,
        },
        "accept_us": round(ms * 1e3, 2),
        "accept_greedy_us": round(g_ms * 1e3, 2),
        "accept_greedy_gbps": round(g_step.algorithmic_bytes() / (g_ms * 1e-3) / 1e9, 1),
        "accept_b8_us": round(b8_ms * 1e3, 2),
        "accept_b8_gbps": round(b8_step.algorithmic_bytes() / (b8_ms * 1e-3) / 1e9, 1),
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
