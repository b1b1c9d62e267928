"""Benchmark of the per-step speculative hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

One step is one pass of the hot path over one batch of synthetic input with
inputs resident in HBM: block-verify attention of a batch-1 block of 16
queries (Qwen3-8B GQA: 32 query / 8 KV heads, d 128, bf16) over a 2048-token
prefix in a paged cache, then the fused acceptance of 16 target and 15 draft
fp32 logit rows over the 151,936-entry vocabulary at temperature 1.  Prints
ONE JSON line.

The roofline entry is for whichever of the two calls takes longer:
acceptance algorithmic bytes = (16 + 15) rows x V x 4 B = 18,840,064 B;
attention algorithmic bytes = K and V rows of 2064 tokens x 8 heads x 256 B
+ q and o + page table = 8,716,804 B; each divided by the call's average
duration from HIP events recorded on the launch stream.

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

# HBM bytes per call measured with rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE
# (two passes of `bench.py --no-cpu-baseline --no-models --calibrate-copy`),
# each counter scaled by what it reads for a plain 64 MiB device copy in the
# same process: FETCH_SIZE x 1.99921, WRITE_SIZE x 1.0.  They are measured
# figures, not computed here; a kernel change needs a new counter pass.
TRAFFIC_ACCEPT_B1 = 20_703_291      # stats + decide + resample, 1.099 x algorithmic
TRAFFIC_VERIFY_ATTN_B1 = 13_678_652  # split + combine, 1.569 x algorithmic (fp16 partials)


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-models", action="store_true",
                    help="skip the draft-block (1.7B) and end-to-end (8B + 1.7B) model runs")
    ap.add_argument("--e2e-new-tokens", type=int, default=512)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run a plain 64 MiB device copy 5 times (the reference kernel for "
                         "scaling FETCH_SIZE / WRITE_SIZE counters)")
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


class AttnStep:
    """Pre-bound paged attention call (verify: causal block; draft: bidirectional)."""

    def __init__(self, lens, Q, Hq, Hkv, page_size, causal: bool, dev, seed=0, num_pages=None):
        import math
        from d3d_amd import _lib, workloads
        self.lib = _lib.load()
        kv = workloads.paged_kv(seed, lens, Hkv=Hkv, D=128, page_size=page_size, num_pages=num_pages,
                                device="cuda")
        self.kv = kv
        self.q = workloads.queries(seed + 7, len(lens), Q, Hq=Hq, device="cuda")
        B = len(lens)
        self.out = torch.empty_like(self.q)
        P = kv.k_cache.shape[0]
        max_pages = kv.block_table.shape[1]
        max_ctx = max(lens)
        n = self.lib.d3d_attn_workspace_bytes(B, Q, Hq, Hkv, 128, page_size, max_ctx)
        self.ws = torch.zeros(max(n, 256), dtype=torch.uint8, device=dev)
        self.fn = self.lib.d3d_verify_attn_paged if causal else self.lib.d3d_draft_block_attn
        self.args = (self.q.data_ptr(), kv.k_cache.data_ptr(), kv.v_cache.data_ptr(),
                     kv.block_table.data_ptr(), kv.context_lens.data_ptr(), self.out.data_ptr(),
                     B, Q, Hq, Hkv, 128, page_size, max_pages, P, 1.0 / math.sqrt(128), max_ctx,
                     self.ws.data_ptr(), self.ws.numel(), torch.cuda.current_stream(dev).cuda_stream)
        self._check = _lib.check
        # Algorithmic work: every visible key/value row once, q in, o out, the page table.
        kv_bytes = sum(c * Hkv * 128 * 2 * 2 for c in lens)
        self.bytes = kv_bytes + 2 * B * Q * Hq * 128 * 2 + sum(-(-c // page_size) * 4 for c in lens)
        flops = 0
        for c in lens:
            seen = sum(min(c, c - Q + i + 1) for i in range(Q)) if causal else Q * c
            flops += 4 * Hq * 128 * seen
        self.flops = flops

    def __call__(self):
        st = self.fn(*self.args)
        if st:
            self._check(st, "paged attention")


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


def draft_block_bench(dev, reps: int = 20):
    """Diffusion-draft block step at Qwen3-1.7B draft shapes (random bf16 weights):
    batch 4, 1024-token prefix, one block of 16 masks, 4 iterations of top-4."""
    from d3d_amd import draft as dr
    from d3d_amd.model import D3D_1P7B, PagedKV, Qwen3PagedModel, Sequence, prefill
    model = Qwen3PagedModel(D3D_1P7B, dev, draft=True, seed=11)
    kv = PagedKV(D3D_1P7B, 512, 16, dev)
    g = torch.Generator().manual_seed(5)
    seqs = [Sequence(i, torch.randint(0, 151936, (1024,), generator=g).tolist()) for i in range(4)]
    prefill(model, kv, seqs, "draft")
    block = torch.full((4, 16), dr.MASK_ID, dtype=torch.int64, device=dev)
    graphs = {}  # each (forward + unmask) iteration replayed from a HIP graph
    dr.d3d_draft_block(model, kv, seqs, block, 4, graphs=graphs)
    torch.cuda.synchronize(dev)
    ms = time_calls(lambda: dr.d3d_draft_block(model, kv, seqs, block, 4, graphs=graphs), reps, 1, dev)
    del model, kv
    torch.cuda.empty_cache()
    return ms


def lmhead_bench(dev, steps: int, warmup: int):
    """Fused LM head + top-2 (the draft recovery block: 64 hidden rows, H 2048,
    V 151936, random bf16 weights) against the unfused bf16 GEMM + top-k."""
    from d3d_amd.draft import topk_tokens
    from d3d_amd.lmhead import lmhead_topk
    g = torch.Generator().manual_seed(3)
    T, H, V = 64, 2048, 151936
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(V, H, generator=g) / H ** 0.5).to(torch.bfloat16).to(dev)
    fused = time_calls(lambda: lmhead_topk(x, w, 2), steps, warmup, dev)
    unfused = time_calls(lambda: topk_tokens(torch.nn.functional.linear(x, w), 2), steps, warmup, dev)
    nbytes = V * H * 2 + T * H * 2
    del x, w
    torch.cuda.empty_cache()
    return fused, unfused, nbytes


def e2e_bench(dev, new_tokens: int):
    """Qwen3-8B-shaped target + Qwen3-1.7B-shaped draft co-resident, two streams:
    batch 4, prompts of 512 random ids, greedy, 16-token blocks, 16-token pages."""
    from d3d_amd.engine import Engine
    eng = Engine(seed=42)
    g = torch.Generator().manual_seed(9)
    prompts = torch.randint(0, 151936, (4, 512), generator=g).tolist()
    eng.generate([p[:64] for p in prompts], max_new_tokens=8, ignore_eos=True)  # warm-up
    res = eng.generate(prompts, max_new_tokens=new_tokens, ignore_eos=True)
    del eng
    torch.cuda.empty_cache()
    return res


def cpu_baseline(seconds: float):
    """fp32 torch-CPU restatement of the same step: paged attention + acceptance."""
    import math
    from d3d_amd import workloads
    from oracle import torch_ref
    kv = workloads.paged_kv(1234, [2048 + 16], Hkv=8, D=128, page_size=16, num_pages=256)
    q = workloads.queries(1234 + 7, 1, 16, Hq=32)
    inp = workloads.accept_inputs(1234, B=1, K=15)
    threads = torch.get_num_threads()

    def once():
        torch_ref.paged_attention_sdpa(q, kv.k_cache, kv.v_cache, kv.block_table, kv.context_lens,
                                       1.0 / math.sqrt(128), causal=True)
        p = torch_ref.sampling_probs(inp.target, 1.0)
        pq = torch_ref.sampling_probs(inp.draft, 1.0)
        torch_ref.verify_block(inp.tokens, p, pq, inp.uniforms, float(inp.resample_u[0]))

    for _ in range(2):
        once()
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        once()
        n += 1
    us = (time.perf_counter() - t0) / n * 1e6
    return {
        "value": round(1e6 / us, 1), "unit": "steps/s", "us_per_step": round(us, 1), "cores": threads,
        "kind": "port",
        "sample": f"{n} steps of the same workload (fp32 SDPA over the gathered 2064-token paged "
                  f"prefix + batch-1 T=1 acceptance), torch CPU fp32 restatement, {threads} threads",
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

    if args.calibrate_copy:
        src = torch.ones(64 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize(dev)
        del src, dst

    # Headline step: block-verify attention (batch 1, Qwen3-8B GQA 32/8, d 128, K=16
    # causal block over a 2048-token prefix in 16-token pages of a shuffled
    # 256-page pool) followed by fused acceptance (16 target + 15 draft fp32
    # rows over vocab 151936, T = 1).
    attn = AttnStep([2048 + 16], 16, 32, 8, 16, True, dev, seed=1234, num_pages=256)
    inp = workloads.accept_inputs(1234, B=1, K=15, device="cuda")
    acc = AcceptStep(inp, 1.0, dev)

    def step():
        attn()
        acc()

    ms = time_calls(step, args.steps, args.warmup, dev)
    attn_ms = time_calls(attn, args.steps, args.warmup, dev)
    acc_ms = time_calls(acc, args.steps, args.warmup, dev)
    acc_gbps = acc.algorithmic_bytes() / (acc_ms * 1e-3) / 1e9
    attn_gbps = attn.bytes / (attn_ms * 1e-3) / 1e9
    attn_tflops = attn.flops / (attn_ms * 1e-3) / 1e12
    # The dominant kernel is the acceptance call when it takes longer.
    if acc_ms >= attn_ms:
        roof = {"bound": "hbm", "achieved": round(acc_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(acc_gbps / HBM_PEAK_GBPS, 4), "traffic": TRAFFIC_ACCEPT_B1, "kernel": "fused acceptance"}
    else:
        roof = {"bound": "hbm", "achieved": round(attn_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(attn_gbps / HBM_PEAK_GBPS, 4), "traffic": TRAFFIC_VERIFY_ATTN_B1, "kernel": "verify attention"}

    # Secondary figures: greedy acceptance, batch-8 acceptance, batch-8
    # concurrent verify attention, batch-4 draft block attention.
    g_step = AcceptStep(workloads.accept_inputs(1234, B=1, K=15, temperature=0.0, device="cuda"), 0.0, dev)
    g_ms = time_calls(g_step, args.steps, args.warmup, dev)
    b8_step = AcceptStep(workloads.accept_inputs(1234, B=8, K=15, device="cuda"), 1.0, dev)
    b8_ms = time_calls(b8_step, args.steps, args.warmup, dev)
    lens8 = [c + 16 for c in workloads.concurrent_context_lens(2024, B=8)]
    v8 = AttnStep(lens8, 16, 32, 8, 16, True, dev, seed=2024)
    v8_ms = time_calls(v8, args.steps, args.warmup, dev)
    dr = AttnStep([1024 + 16] * 4, 16, 16, 8, 16, False, dev, seed=77)
    dr_ms = time_calls(dr, args.steps, args.warmup, dev)

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
        "dtype": "bf16 attention, f32 acceptance",
        "data": "synthetic",
        "config": {
            "workload": "block-verify attention (batch 1, 32/8 heads, d 128, 16-query causal block, "
                        "2048-token prefix, 16-token pages, shuffled 256-page pool, bf16) + fused "
                        "acceptance (16 target + 15 draft fp32 rows, vocab 151936, T=1, seeded uniforms)",
            "global_batch": 1,
            "draft_block": 16,
            "prefix": 2048,
            "vocab": 151936,
        },
        "roofline": roof,
        "verify_attn_us": round(attn_ms * 1e3, 2),
        "verify_attn_gbps": round(attn_gbps, 1),
        "verify_attn_tflops": round(attn_tflops, 2),
        "accept_us": round(acc_ms * 1e3, 2),
        "accept_gbps": round(acc_gbps, 1),
        "accept_greedy_us": round(g_ms * 1e3, 2),
        "accept_greedy_gbps": round(g_step.algorithmic_bytes() / (g_ms * 1e-3) / 1e9, 1),
        "accept_b8_us": round(b8_ms * 1e3, 2),
        "accept_b8_gbps": round(b8_step.algorithmic_bytes() / (b8_ms * 1e-3) / 1e9, 1),
        "verify_attn_b8_us": round(v8_ms * 1e3, 2),
        "verify_attn_b8_gbps": round(v8.bytes / (v8_ms * 1e-3) / 1e9, 1),
        "verify_attn_b8_tflops": round(v8.flops / (v8_ms * 1e-3) / 1e12, 2),
        "draft_attn_b4_us": round(dr_ms * 1e3, 2),
        "draft_attn_b4_gbps": round(dr.bytes / (dr_ms * 1e-3) / 1e9, 1),
    }
    lm_ms, lm_unfused_ms, lm_bytes = lmhead_bench(dev, min(args.steps, 100), min(args.warmup, 10))
    out["lmhead_top2_t64_us"] = round(lm_ms * 1e3, 2)
    out["lmhead_top2_t64_gbps"] = round(lm_bytes / (lm_ms * 1e-3) / 1e9, 1)
    out["lmhead_gemm_then_topk_t64_us"] = round(lm_unfused_ms * 1e3, 2)
    if not args.no_models:
        out["draft_block_step_ms"] = round(draft_block_bench(dev), 3)
        res = e2e_bench(dev, args.e2e_new_tokens)
        out["e2e"] = {
            "steps_per_s": round(res["steps_per_s"], 2),
            "tokens_per_s": round(res["tps"], 1),
            "verify_ms": round(res["verify_ms"], 3),
            "draft_ms": round(res["draft_ms"], 3),
            "overlap_fraction": round(res["overlap_fraction"], 3),
            "timeline_ms": res["timeline"][:3],
            "steps": res["steps"],
            "new_tokens": args.e2e_new_tokens,
            "batch": 4,
            "note": "random weights: drafts almost never match, so each step commits 1 token",
        }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
