// Top-k token ids of logits rows for the draft's anchor proposals.
//
// Reference behaviour (D3D repository):
//   serving/backend.py:84-93  Runner._run: per 256-row chunk of hidden
//       states, logits = lm_head(h); greedy = logits.argmax(-1);
//       top = logits.topk(k).indices (k = anchor_num + 1), used by
//       Engine._recover / Engine._predict (serving/engine.py:54-131) to pick
//       the anchor tokens of the packed branches
//
// Order: descending value, equal values by ascending index, so top[0] is
// torch.argmax's first maximum.  NaN entries are never selected.  With
// log_softmax the values are returned as log-probabilities x - logsumexp(x)
// (single/eval_sync.py:763-768, torch.topk of log_softmax: the same ids).
//
// Two kernels: (1) grid (chunks, rows): each workgroup takes k rounds of a
// workgroup argmax over its 4096-entry chunk (each thread holds 16 entries
// in registers and excludes the ones already taken) and writes k (value,
// index) candidates; (2) one workgroup per row merges the chunk candidates
// the same way.  Streaming the logits once is the HBM-bound part.  Four
// chunks per workgroup (64 entries per thread) measured 166 -> 340 us at
// 1088 bf16 rows of 151936: the per-round rescans of the registers are
// VALU-bound, and fewer workgroups hide less of it.  For bf16 rows each
// entry is one sortable integer key (value, position in the chunk, sign of
// zero), so a round is 16 integer maxes, an unsigned-max butterfly and one
// barrier: 161.8 -> 136.3 us at that shape against the (value, index)
// compares with a taken mask and two-barrier argmax that fp32 rows keep.
#include "d3d_common.hpp"
#include "rowstats.hpp"
#include "../../include/d3d_hip.h"

#include <limits.h>

namespace d3d {
namespace topk {

using namespace rows;

constexpr int kMaxK = 64;
// bf16 rows: vocabulary chunks per workgroup (16 entries each per thread).
// Two measured 135.6 -> 153.3 us at 1088 rows of 151936 (77 VGPRs, fewer
// waves per SIMD, half the workgroups).
constexpr int kBf16Chunks = 1;
template <int DT>
constexpr int chunks_per_wg() { return DT == kBF16 ? kBf16Chunks : 1; }
constexpr int kMaxCand = 8192;  // chunk candidates per row merged in LDS

struct Cand {
    float v;
    int i;
};

struct Params {
    const void* logits;  // [N, V]
    int N, V, C, k;
    Cand* cand;       // [N][C][k]
    float2* lse;      // [N][C] chunk (max, sum exp(x - max)) when log-probabilities are asked for
    int64_t* ids;     // [N, k]
    float* vals;      // [N, k] (may be null)
};

// Round 0's winner is the chunk max: the chunk's share of logsumexp,
// (max, sum exp(x - max)) over the live entries.
template <int DT, int LT>
__device__ __forceinline__ void chunk_lse(const Params& P, const float (&x)[LT], int first, float wv, int n, int c,
                                          float* sv) {
    constexpr int E = Vec<DT>::E;
    float se = 0.f;
    if (wv != -INFINITY) {
#pragma unroll
        for (int l = 0; l < LT; ++l)
            if (tile_index<DT>(first, NT * E, l) < P.V) se += expf(x[l] - wv);
    }
    se = block_sum<NT>(se, sv);
    if (threadIdx.x == 0) P.lse[(size_t)n * P.C + c] = make_float2(wv, se);
}

template <int DT, bool VEC>
__global__ __launch_bounds__(NT) void topk_chunk_kernel(Params P) {
    constexpr int E = Vec<DT>::E;
    const int c = blockIdx.x, n = blockIdx.y;
    __shared__ float sv[NT / kWave];
    __shared__ int si[NT / kWave];
    const void* row = row_ptr<DT>(P.logits, n, P.V);
    constexpr int LT = L * chunks_per_wg<DT>();  // entries per thread
    constexpr int span = kChunk * chunks_per_wg<DT>();
    const int first = c * span + threadIdx.x * E;
    float x[LT];
    load_tile<DT, VEC, true, LT>(row, P.V, first, NT * E, -INFINITY, x);
    if constexpr (DT == kBF16) {
        // Each entry is one sortable key: its order-preserving 16-bit value
        // (-0 ordered as +0), then span - 1 - its position in the span,
        // then a -0 flag.  Keys are unique within the chunk, and the
        // largest is the larger value, among equal values the lower index
        // (the flag never decides, as the positions differ first).  So a
        // round is an unsigned max: LT per thread, a DPP butterfly per wave,
        // one LDS slot per wave and round, one barrier.  Key 0 marks NaN,
        // entries past the row and entries taken; -inf keeps a positive key,
        // as its (value, index) pair is selectable.
        constexpr int kPosBits = 13;
        static_assert(span <= (1 << kPosBits), "position field of the key");
        __shared__ uint32_t swin[kMaxK][NT / kWave];
        const int base = c * span, w = threadIdx.x / kWave;
        uint32_t key[LT];
#pragma unroll
        for (int l = 0; l < LT; ++l) {
            const int e = tile_index<DT>(first, NT * E, l);
            const uint32_t u = __float_as_uint(x[l]) >> 16;
            const uint32_t nz = u == 0x8000u;
            const uint32_t v = nz ? 0u : u;
            const bool nan = (v & 0x7f80u) == 0x7f80u && (v & 0x7fu);
            const uint32_t ord = (v & 0x8000u) ? (~v & 0xffffu) : (v | 0x8000u);
            key[l] = (nan || e >= P.V) ? 0u : (ord << (kPosBits + 1)) | ((uint32_t)(span - 1 - (e - base)) << 1) | nz;
        }
        for (int r = 0; r < P.k; ++r) {
            uint32_t win = key[0];
#pragma unroll
            for (int l = 1; l < LT; ++l) win = max(win, key[l]);
            win = max(win, xor_partner_desc<32>(win));
            win = max(win, xor_partner_desc<16>(win));
            win = max(win, xor_partner_desc<8>(win));
            win = max(win, xor_partner_desc<4>(win));
            win = max(win, xor_partner_desc<2>(win));
            win = max(win, xor_partner_desc<1>(win));
            if ((threadIdx.x & (kWave - 1)) == 0) swin[r][w] = win;
            __syncthreads();
            win = swin[r][0];
#pragma unroll
            for (int k = 1; k < NT / kWave; ++k) win = max(win, swin[r][k]);
#pragma unroll
            for (int l = 0; l < LT; ++l)
                if (key[l] == win) key[l] = 0;  // the winner, in its owner's registers
            float wv = -INFINITY;
            int wi = INT_MAX;
            if (win) {
                const uint32_t ord = win >> (kPosBits + 1);
                const uint32_t u = ((ord & 0x8000u) ? (ord & 0x7fffu) : (~ord & 0xffffu)) | ((win & 1u) << 15);
                wv = __uint_as_float(u << 16);
                wi = base + span - 1 - (int)((win >> 1) & ((1u << kPosBits) - 1));
            }
            if (threadIdx.x == 0) P.cand[((size_t)n * P.C + c) * P.k + r] = Cand{wv, wi};
            if (r == 0 && P.lse) chunk_lse<DT>(P, x, first, wv, n, c, sv);
        }
        return;
    }
    static_assert(LT <= 32, "one mask bit per entry");
    uint32_t taken = 0;  // bit l: entry l already selected
    for (int r = 0; r < P.k; ++r) {
        float bv = -INFINITY;
        int bi = INT_MAX;
#pragma unroll
        for (int l = 0; l < LT; ++l) {
            const int e = tile_index<DT>(first, NT * E, l);
            if (!((taken >> l) & 1u) && e < P.V) argmax_merge(bv, bi, x[l], e);
        }
        float wv = bv;
        int wi = bi;
        block_argmax<NT>(wv, wi, sv, si);
        // The owner of the winning entry excludes it from later rounds.
#pragma unroll
        for (int l = 0; l < LT; ++l)
            if (tile_index<DT>(first, NT * E, l) == wi) taken |= 1u << l;
        if (threadIdx.x == 0) P.cand[((size_t)n * P.C + c) * P.k + r] = Cand{wv, wi};
        if (r == 0 && P.lse) chunk_lse<DT>(P, x, first, wv, n, c, sv);
    }
}

__global__ __launch_bounds__(NT) void topk_merge_kernel(Params P) {
    const int n = blockIdx.x;
    __shared__ Cand lds[kMaxCand];
    __shared__ float sv[NT / kWave];
    __shared__ int si[NT / kWave];
    const int total = P.C * P.k;
    for (int e = threadIdx.x; e < total; e += NT) lds[e] = P.cand[(size_t)n * total + e];
    float logz = 0.f;
    if (P.lse) {
        // logsumexp over the chunk records, in a fixed order.
        float mx = -INFINITY;
        for (int c = threadIdx.x; c < P.C; c += NT) mx = fmaxf(mx, P.lse[(size_t)n * P.C + c].x);
        mx = block_max<NT>(mx, sv);
        float se = 0.f;
        for (int c = threadIdx.x; c < P.C; c += NT) {
            const float2 t = P.lse[(size_t)n * P.C + c];
            if (t.x != -INFINITY) se += t.y * expf(t.x - mx);
        }
        se = block_sum<NT>(se, sv);
        logz = mx + logf(se);
    }
    __syncthreads();
    for (int r = 0; r < P.k; ++r) {
        float bv = -INFINITY;
        int bi = INT_MAX, bp = -1;
        for (int e = threadIdx.x; e < total; e += NT) {
            const Cand cd = lds[e];
            if (cd.i == INT_MAX) continue;  // taken, or a chunk with fewer than k entries
            const float v0 = bv;
            const int i0 = bi;
            argmax_merge(bv, bi, cd.v, cd.i);
            if (bv != v0 || bi != i0) bp = e;
        }
        float wv = bv;
        int wi = bi;
        block_argmax<NT>(wv, wi, sv, si);
        if (threadIdx.x == 0) {
            P.ids[(size_t)n * P.k + r] = wi == INT_MAX ? -1 : wi;
            if (P.vals) P.vals[(size_t)n * P.k + r] = P.lse ? wv - logz : wv;
        }
        // Token ids are unique among candidates: the holder marks its entry.
        if (bp >= 0 && bi == wi && wi != INT_MAX) lds[bp].i = INT_MAX;
        __syncthreads();
    }
}


// ---------------------------------------------------------------- fused LM head
// Logits of up to kLmRows hidden rows against a kLmCols-row slice of the LM
// head weight, computed with v_mfma_f32_16x16x32_bf16 and reduced inside the
// workgroup to the slice's top-KK (value, id) candidates and (max,
// sum exp(x - max)) per hidden row, in the chunk-record format of
// topk_chunk_kernel; topk_merge_kernel then merges the slices.  The logits
// never reach HBM.
//
// Reference behaviour (D3D repository): serving/backend.py:84-93
// (Runner._run: logits = lm_head(h) per 256-row chunk, greedy =
// logits.argmax(-1), top = logits.topk(anchor_num + 1)); single/eval_sync.py
// :713-717 and :763-768 (argmax and log_softmax top-k of the draft logits).
// Every logit is rounded to bf16 before it is compared or exponentiated, as
// the reference's bf16 linear layer returns bf16 logits.
//
// Both operands are K-contiguous rows: lane l holds hidden row 16rb + l%16
// and weight row 16cb + l%16 at K offsets 32s + 8(l/16) .. +7, which are the
// A and B operand layouts of the MFMA, so no transpose is needed.  Wave w
// owns kLmCB 16-row blocks of the weight slice for all 64 hidden rows (four
// 16-row blocks).  Three K steps of operands are in flight while one is
// multiplied.  A slice of 320 weight rows gives 475 workgroups for the
// 151,936-entry vocabulary: one round at two workgroups per CU (the
// accumulators and operand buffers take two waves' worth of registers per
// SIMD), so no short second round streams alone.  With at most 64 hidden
// rows the weight is read once: HBM-bound, V x H x 2 bytes per launch.
constexpr int kLmRows = 64;
constexpr int kLmCB = 5;                  // 16-row weight blocks per wave
constexpr int kLmCols = 4 * 16 * kLmCB;   // weight rows per workgroup
constexpr int kLmMaxK = 8;
constexpr int kLmStride = kLmCols + 8;    // bf16 entries per LDS row (16-byte pad)
constexpr int kLmPer = kLmCols / 4;       // slice columns per epilogue thread

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

struct LmParams {
    const uint16_t* x;  // [T, H] bf16 hidden rows
    const uint16_t* w;  // [V, H] bf16 weight rows
    int T, H, V, k, C;
    Cand* cand;   // [T][C][k]
    float2* lse;  // [T][C] (max, sum exp(x - max)); always written
};

// (cv, ci) enters the sorted list (value descending, id ascending) if it
// beats an entry; the last entry falls off.
template <int KK>
__device__ __forceinline__ void list_insert(float (&tv)[KK], int (&ti)[KK], float cv, int ci) {
#pragma unroll
    for (int p = 0; p < KK; ++p) {
        const bool better = cv > tv[p] || (cv == tv[p] && ci < ti[p]);
        if (better) {
            const float fv = tv[p];
            const int fi = ti[p];
            tv[p] = cv;
            ti[p] = ci;
            cv = fv;
            ci = fi;
        }
    }
}

// Epilogue shared by the LM-head kernels: the tile's bf16 logits go through
// LDS (s_log, kLmRows x kLmStride entries) to four threads per hidden row,
// which keep the row's top-KK and (max, sum exp(x - max)) over the slice.
template <int KK>
__device__ __forceinline__ void lmhead_epilogue(const LmParams& P, const f32x4 (&acc)[4][kLmCB], int slice, int row0,
                                                uint16_t* s_log) {
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    const int c16 = lane & 15, g4 = lane >> 4;
    // bf16 logits of the tile into LDS: accumulator (rb, cb) element r of
    // lane l is hidden row 16rb + 4(l/16) + r, slice column 16(kLmCB w + cb) + l%16.
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int cb = 0; cb < kLmCB; ++cb)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                s_log[(16 * rb + 4 * g4 + r) * kLmStride + 16 * (kLmCB * w + cb) + c16] =
                    f32_to_bf16_bits(acc[rb][cb][r]);
    __syncthreads();

    // Four threads per hidden row, kLmPer consecutive slice columns each:
    // max and top-KK in one pass, sum exp(x - max) in a second.
    const int row = threadIdx.x >> 2, q = threadIdx.x & 3;
    const int vbase = slice * kLmCols + kLmPer * q;
    const int nvalid = min(kLmPer, P.V - vbase);  // may be <= 0 in the last slice
    const uint16_t* src = &s_log[row * kLmStride + kLmPer * q];
    float tv[KK];
    int ti[KK];
#pragma unroll
    for (int p = 0; p < KK; ++p) {
        tv[p] = -INFINITY;
        ti[p] = INT_MAX;
    }
    float mx = -INFINITY;
    for (int j8 = 0; j8 < kLmPer; j8 += 8) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(src + j8);
        const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int h = 0; h < 8; ++h) {
            const int j = j8 + h;
            const float xj = bf16_bits_to_f32(h & 1 ? wd[h >> 1] >> 16 : wd[h >> 1] & 0xffffu);
            if (j < nvalid) {
                mx = fmaxf(mx, xj);
                // Ids rise with j, so an equal value never displaces an earlier one.
                if (xj > tv[KK - 1]) list_insert<KK>(tv, ti, xj, vbase + j);
            }
        }
    }
    // Merge the four threads of the row (lanes 4i .. 4i+3): butterfly over
    // xor 1 and xor 2; both partners end with the same list (ids are unique).
#pragma unroll
    for (int o = 1; o <= 2; o <<= 1) {
        float ov[KK];
        int oi[KK];
#pragma unroll
        for (int p = 0; p < KK; ++p) {
            ov[p] = __shfl_xor(tv[p], o, kWave);
            oi[p] = __shfl_xor(ti[p], o, kWave);
        }
#pragma unroll
        for (int p = 0; p < KK; ++p) list_insert<KK>(tv, ti, ov[p], oi[p]);
        mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
    }
    float se = 0.f;
    if (mx != -INFINITY) {
        for (int j8 = 0; j8 < kLmPer; j8 += 8) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(src + j8);
            const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int h = 0; h < 8; ++h) {
                const float xj = bf16_bits_to_f32(h & 1 ? wd[h >> 1] >> 16 : wd[h >> 1] & 0xffffu);
                if (j8 + h < nvalid) se += expf(xj - mx);
            }
        }
    }
    se += __shfl_xor(se, 1, kWave);
    se += __shfl_xor(se, 2, kWave);
    const int grow = row0 + row;
    if (q == 0 && grow < P.T) {
        Cand* dst = P.cand + ((size_t)grow * P.C + slice) * P.k;
#pragma unroll
        for (int p = 0; p < KK; ++p)
            if (p < P.k) dst[p] = Cand{tv[p], ti[p]};
        P.lse[(size_t)grow * P.C + slice] = make_float2(mx, se);
    }
}

template <int KK>
__global__ __launch_bounds__(NT, 2) void lmhead_partial_kernel(LmParams P) {
    const int slice = blockIdx.x, row0 = blockIdx.y * kLmRows;
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    const int c16 = lane & 15, g4 = lane >> 4;
    const int vw = slice * kLmCols + 16 * kLmCB * w;  // this wave's first weight row

    // Operand row pointers; rows past T or V read a valid row and are dropped.
    const uint16_t* xa[4];
    const uint16_t* wb[kLmCB];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
        const int r = min(row0 + 16 * rb + c16, P.T - 1);
        xa[rb] = P.x + (size_t)r * P.H + 8 * g4;
    }
#pragma unroll
    for (int cb = 0; cb < kLmCB; ++cb) {
        const int v = min(vw + 16 * cb + c16, P.V - 1);
        wb[cb] = P.w + (size_t)v * P.H + 8 * g4;
    }
    f32x4 acc[4][kLmCB];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int cb = 0; cb < kLmCB; ++cb) acc[rb][cb] = {0.f, 0.f, 0.f, 0.f};

    auto load = [&](u32x4 (&a)[4], u32x4 (&b)[kLmCB], int s) {
#pragma unroll
        for (int cb = 0; cb < kLmCB; ++cb) b[cb] = *reinterpret_cast<const u32x4*>(wb[cb] + 32 * s);
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) a[rb] = *reinterpret_cast<const u32x4*>(xa[rb] + 32 * s);
    };
    auto mma = [&](const u32x4 (&a)[4], const u32x4 (&b)[kLmCB]) {
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int cb = 0; cb < kLmCB; ++cb)
                acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[rb]),
                                                                      __builtin_bit_cast(bf16x8, b[cb]), acc[rb][cb],
                                                                      0, 0, 0);
    };
    // K steps of 32: the first S3 (a multiple of 3) run through a
    // three-buffer pipeline whose loop body has no conditional loads (with
    // conditional loads the compiler waits for every outstanding load at the
    // top of each iteration); the remaining 0-2 steps run unpipelined.
    const int S = P.H / 32, S3 = S - S % 3;
    u32x4 a0[4], b0[kLmCB], a1[4], b1[kLmCB], a2[4], b2[kLmCB];
    if (S3 > 0) {
        load(a0, b0, 0);
        load(a1, b1, 1);
        load(a2, b2, 2);
        // The scheduling barriers keep each load right behind the MFMAs it
        // follows (left alone, the scheduler sinks all loads to the end).
        for (int s = 0; s < S3 - 3; s += 3) {
            mma(a0, b0);
            __builtin_amdgcn_sched_barrier(0);
            load(a0, b0, s + 3);
            __builtin_amdgcn_sched_barrier(0);
            mma(a1, b1);
            __builtin_amdgcn_sched_barrier(0);
            load(a1, b1, s + 4);
            __builtin_amdgcn_sched_barrier(0);
            mma(a2, b2);
            __builtin_amdgcn_sched_barrier(0);
            load(a2, b2, s + 5);
            __builtin_amdgcn_sched_barrier(0);
        }
        mma(a0, b0);
        mma(a1, b1);
        mma(a2, b2);
    }
    for (int s = S3; s < S; ++s) {
        load(a0, b0, s);
        mma(a0, b0);
    }

    __shared__ __attribute__((aligned(16))) uint16_t s_log[kLmRows * kLmStride];
    lmhead_epilogue<KK>(P, acc, slice, row0, s_log);
}

// Variant for H a multiple of 256: the hidden rows are staged in LDS 256 K
// at a time (a 32 KiB chunk, two buffers), loaded once per workgroup
// instead of once per wave, so the vector memory pipe carries the weight
// stream almost alone (per-wave hidden-row loads measured about a quarter of
// the stream's throughput).  The weight loads run four K steps ahead in
// registers; their step index is clamped to the last step (a few redundant
// in-bounds loads at the end) and the next chunk's index to the last chunk,
// so the loop body has no conditional loads (with conditional loads the
// compiler waits for every outstanding load at the top of each iteration).
constexpr int kXC = 8;                                  // K steps of 32 per chunk
constexpr int kXStride = 32 * kXC + 8;                  // bf16 entries per chunk row (16-byte pad)
constexpr int kXBuf = kLmRows * kXStride;               // entries per chunk buffer
constexpr int kLmSmem = 2 * kXBuf * 2 > kLmRows * kLmStride * 2 ? 2 * kXBuf * 2 : kLmRows * kLmStride * 2;

template <int KK>
__global__ __launch_bounds__(NT, 2) void lmhead_partial_xlds_kernel(LmParams P) {
    __shared__ __attribute__((aligned(16))) char smem[kLmSmem];
    uint16_t* sx = reinterpret_cast<uint16_t*>(smem);  // [2][kLmRows][kXStride]; the epilogue reuses it
    const int slice = blockIdx.x, row0 = blockIdx.y * kLmRows;
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    const int c16 = lane & 15, g4 = lane >> 4;
    const int vw = slice * kLmCols + 16 * kLmCB * w;
    const int S = P.H / 32, nch = S / kXC;

    const uint16_t* wb[kLmCB];
#pragma unroll
    for (int cb = 0; cb < kLmCB; ++cb) {
        const int v = min(vw + 16 * cb + c16, P.V - 1);
        wb[cb] = P.w + (size_t)v * P.H + 8 * g4;
    }
    f32x4 acc[4][kLmCB];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int cb = 0; cb < kLmCB; ++cb) acc[rb][cb] = {0.f, 0.f, 0.f, 0.f};

    // Chunk c of the hidden rows: 64 rows x 512 bytes = 2048 16-byte pieces,
    // 8 per thread; rows past T repeat row T - 1.
    u32x4 xr[8];
    auto xload = [&](int c) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int piece = (int)threadIdx.x + NT * i, row = piece >> 5, col = piece & 31;
            const int r = min(row0 + row, P.T - 1);
            xr[i] = *reinterpret_cast<const u32x4*>(P.x + (size_t)r * P.H + 256 * c + 8 * col);
        }
    };
    auto xstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int piece = (int)threadIdx.x + NT * i, row = piece >> 5, col = piece & 31;
            *reinterpret_cast<u32x4*>(sx + buf * kXBuf + row * kXStride + 8 * col) = xr[i];
        }
    };
    u32x4 b[4][kLmCB];
    auto wload = [&](u32x4 (&bb)[kLmCB], int st) {
        st = min(st, S - 1);
#pragma unroll
        for (int cb = 0; cb < kLmCB; ++cb) bb[cb] = *reinterpret_cast<const u32x4*>(wb[cb] + 32 * st);
    };
    auto step = [&](const u32x4 (&bb)[kLmCB], const uint16_t* xs, int sp) {
        u32x4 a[4];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
            a[rb] = *reinterpret_cast<const u32x4*>(xs + (16 * rb + c16) * kXStride + 32 * sp + 8 * g4);
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int cb = 0; cb < kLmCB; ++cb)
                acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[rb]),
                                                                      __builtin_bit_cast(bf16x8, bb[cb]), acc[rb][cb],
                                                                      0, 0, 0);
    };

    xload(0);
#pragma unroll
    for (int i = 0; i < 4; ++i) wload(b[i], i);
    xstore(0);
    xload(min(1, nch - 1));
    __syncthreads();
    for (int c = 0; c < nch; ++c) {
        const uint16_t* xs = sx + (c & 1) * kXBuf;
#pragma unroll
        for (int sp = 0; sp < kXC; ++sp) {
            step(b[sp & 3], xs, sp);
            __builtin_amdgcn_sched_barrier(0);
            wload(b[sp & 3], c * kXC + sp + 4);
            __builtin_amdgcn_sched_barrier(0);
        }
        // The other buffer was last read in chunk c - 1, before the previous
        // barrier.  At the last chunk this stores a repeat of it, unread.
        xstore((c + 1) & 1);
        xload(min(c + 2, nch - 1));
        __syncthreads();
    }
    lmhead_epilogue<KK>(P, acc, slice, row0, reinterpret_cast<uint16_t*>(smem));
}

}  // namespace topk
}  // namespace d3d

using namespace d3d;

static size_t cand_bytes(int N, int64_t V, int k) {
    const size_t C = (size_t)((V + rows::kChunk - 1) / rows::kChunk);
    return ((size_t)N * C * k * sizeof(topk::Cand) + 255) & ~(size_t)255;
}

extern "C" size_t d3d_topk_workspace_bytes(int N, int64_t V, int k) {
    if (N < 1 || V < 1 || k < 1) return 0;
    const size_t C = (size_t)((V + rows::kChunk - 1) / rows::kChunk);
    return cand_bytes(N, V, k) + (((size_t)N * C * sizeof(float2) + 255) & ~(size_t)255);
}

extern "C" int d3d_topk_rows(const void* logits, int dtype, int N, int64_t V, int k, int log_softmax,
                             int64_t* ids_out, float* vals_out, void* workspace, size_t workspace_bytes,
                             void* stream) {
    using namespace topk;
    if (N < 0 || V < 1 || V > INT_MAX / 2 || k < 1 || k > kMaxK || k > V) return D3D_E_SHAPE;
    if (dtype != D3D_DTYPE_F32 && dtype != D3D_DTYPE_BF16) return D3D_E_DTYPE;
    if (N == 0) return D3D_OK;
    if (N > 65535) return D3D_E_SHAPE;
    if (!logits || !ids_out || !workspace) return D3D_E_NULL;
    Params P;
    P.logits = logits;
    P.N = N;
    P.V = (int)V;
    const int span = rows::kChunk * (dtype == D3D_DTYPE_BF16 ? kBf16Chunks : 1);
    P.C = (int)((V + span - 1) / span);
    P.k = k;
    if ((int64_t)P.C * k > kMaxCand) return D3D_E_SHAPE;
    if (workspace_bytes < d3d_topk_workspace_bytes(N, V, k)) return D3D_E_WORKSPACE;
    P.cand = static_cast<Cand*>(workspace);
    P.lse = (log_softmax && vals_out)
                ? reinterpret_cast<float2*>(static_cast<char*>(workspace) + cand_bytes(N, V, k))
                : nullptr;
    P.ids = ids_out;
    P.vals = vals_out;
    const size_t esize = dtype == D3D_DTYPE_F32 ? 4 : 2;
    const bool vec = ((uintptr_t)logits % 16 == 0) && ((size_t)V * esize) % 16 == 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 g1(P.C, N);
    if (dtype == D3D_DTYPE_F32) {
        if (vec)
            hipLaunchKernelGGL((topk_chunk_kernel<kF32, true>), g1, dim3(rows::NT), 0, s, P);
        else
            hipLaunchKernelGGL((topk_chunk_kernel<kF32, false>), g1, dim3(rows::NT), 0, s, P);
    } else {
        if (vec)
            hipLaunchKernelGGL((topk_chunk_kernel<kBF16, true>), g1, dim3(rows::NT), 0, s, P);
        else
            hipLaunchKernelGGL((topk_chunk_kernel<kBF16, false>), g1, dim3(rows::NT), 0, s, P);
    }
    hipLaunchKernelGGL(topk_merge_kernel, dim3(N), dim3(rows::NT), 0, s, P);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? D3D_OK : (int)err;
}

static size_t lm_slices(int64_t V) { return (size_t)((V + topk::kLmCols - 1) / topk::kLmCols); }

extern "C" size_t d3d_lmhead_workspace_bytes(int T, int64_t V, int k) {
    if (T < 1 || V < 1 || k < 1) return 0;
    const size_t C = lm_slices(V);
    return (((size_t)T * C * k * sizeof(topk::Cand) + 255) & ~(size_t)255) +
           (((size_t)T * C * sizeof(float2) + 255) & ~(size_t)255);
}

extern "C" int d3d_lmhead_topk(const void* hidden, const void* weight, int T, int H, int64_t V, int k,
                               int log_softmax, int64_t* ids_out, float* vals_out, void* workspace,
                               size_t workspace_bytes, void* stream) {
    using namespace topk;
    if (T < 0 || H < 32 || H % 32 || V < 1 || V > INT_MAX / 2 || k < 1 || k > kLmMaxK || k > V)
        return D3D_E_SHAPE;
    if (T == 0) return D3D_OK;
    if (T > 65535 * kLmRows || (int64_t)T > 65535) return D3D_E_SHAPE;  // merge grid: one workgroup per row
    if (!hidden || !weight || !ids_out || !workspace) return D3D_E_NULL;
    if ((uintptr_t)hidden % 16 || (uintptr_t)weight % 16) return D3D_E_UNSUPPORTED;
    const int C = (int)lm_slices(V);
    if ((int64_t)C * k > kMaxCand) return D3D_E_SHAPE;
    if (workspace_bytes < d3d_lmhead_workspace_bytes(T, V, k)) return D3D_E_WORKSPACE;
    LmParams L;
    L.x = static_cast<const uint16_t*>(hidden);
    L.w = static_cast<const uint16_t*>(weight);
    L.T = T;
    L.H = H;
    L.V = (int)V;
    L.k = k;
    L.C = C;
    L.cand = static_cast<Cand*>(workspace);
    L.lse = reinterpret_cast<float2*>(static_cast<char*>(workspace) +
                                      (((size_t)T * C * k * sizeof(Cand) + 255) & ~(size_t)255));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 g1(C, (T + kLmRows - 1) / kLmRows);
    // H a multiple of 256: hidden rows staged in LDS; otherwise per-wave loads.
    const bool xlds = H % (32 * kXC) == 0;
    const int kk = k == 1 ? 1 : (k == 2 ? 2 : (k <= 4 ? 4 : 8));
    switch (kk * 2 + (xlds ? 1 : 0)) {
        case 2: hipLaunchKernelGGL(lmhead_partial_kernel<1>, g1, dim3(rows::NT), 0, s, L); break;
        case 3: hipLaunchKernelGGL(lmhead_partial_xlds_kernel<1>, g1, dim3(rows::NT), 0, s, L); break;
        case 4: hipLaunchKernelGGL(lmhead_partial_kernel<2>, g1, dim3(rows::NT), 0, s, L); break;
        case 5: hipLaunchKernelGGL(lmhead_partial_xlds_kernel<2>, g1, dim3(rows::NT), 0, s, L); break;
        case 8: hipLaunchKernelGGL(lmhead_partial_kernel<4>, g1, dim3(rows::NT), 0, s, L); break;
        case 9: hipLaunchKernelGGL(lmhead_partial_xlds_kernel<4>, g1, dim3(rows::NT), 0, s, L); break;
        case 16: hipLaunchKernelGGL(lmhead_partial_kernel<8>, g1, dim3(rows::NT), 0, s, L); break;
        default: hipLaunchKernelGGL(lmhead_partial_xlds_kernel<8>, g1, dim3(rows::NT), 0, s, L); break;
    }
    Params P;
    P.logits = nullptr;
    P.N = T;
    P.V = (int)V;
    P.C = C;
    P.k = k;
    P.cand = L.cand;
    P.lse = (log_softmax && vals_out) ? L.lse : nullptr;
    P.ids = ids_out;
    P.vals = vals_out;
    hipLaunchKernelGGL(topk_merge_kernel, dim3(T), dim3(rows::NT), 0, s, P);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? D3D_OK : (int)err;
}
