// Fused speculative acceptance for gfx950.
//
// Two stream-ordered launches:
//
//   1. stats   grid (C, rows, B).  Workgroup (c, r, b) streams chunk c of row
//              r of request b once (target rows 0..K, then draft rows 0..K-1;
//              greedy mode and sparse proposals read target rows only) and
//              reduces it to (max z, sum exp(z - max z), max x, argmax) with
//              z = x / T, or to a plain sum for probability inputs.  One chunk
//              per workgroup and no cross-workgroup traffic: the HBM-bound
//              pass runs at the rate of a plain streaming read.
//   2. finish  grid B * C (greedy: B).  Every workgroup of request b merges
//              the request's chunk records (a few KiB, from L2) into row
//              statistics, evaluates u_i <= min(1, p_i / max(q_i, 1e-12)) at
//              every position and finds the first reject n, each computing
//              the same bits; the request's last workgroup writes the
//              decision outputs.  Workgroup q then reduces part q (4096
//              entries) of the selected row pair to the sums of the residual
//              max(p - q, 0) and of p, publishes them as a tagged record and
//              collects every other part's record (one wave, polling).  Each
//              workgroup then runs the same part-level inverse CDF; the one
//              whose part holds the crossing of u * W scans its entries, still
//              in registers, and writes the token.
//
// The part records are the only cross-workgroup hand-off: each is written
// as two agent-scope atomic 8-byte stores, every word carrying a nonzero tag
// next to its value, and polled with agent-scope atomic loads until every
// tag is set (the stats launch of the same call clears them, so the
// workspace needs no initial contents).  No fence, counter or L2 write-back
// sits on the path.  A workgroup waits only for the other workgroups of its
// own request, and only after publishing its own record; workgroups are
// dispatched in index order, so the lowest unfinished request always has
// all of its workgroups dispatched, its waits end, and so on by induction.  Each wait is bounded
// regardless: on expiry the token stays D3D_TOKEN_TIMEOUT.
//
// Reference semantics (D3D repository):
//   single/eval_sync.py:287-305           temperature softmax / greedy one-hot
//   single/speculative_sampling.py:37-76  normalise, accept test (<=), first
//                                         reject, bonus row, residual with the
//                                         mass <= 1e-12 fallback, resample
//   single/eval_sync.py:1223-1234         greedy leading-match acceptance
//
// Sparse proposals (single/speculative_sampling.py:79-143): the draft side is
// a support of S (id, probability) pairs per position instead of a dense row.
// Phase 1 then reads target rows only (and computes the support mass and q
// at each draft token); the residual of the reject row subtracts the
// normalised support from p entry by entry, in support order (scatter_add),
// before the clamp at zero.  Ids outside [0, V) carry no mass.
//
// Every reduction runs in one fixed order for a given (V, dtype), so outputs
// are deterministic.  The stochastic draw replaces torch.multinomial with an
// inverse CDF over the unnormalised weights driven by resample_u:
// token = first t with C_t > u * W, else the last t with positive weight.
#include "d3d_common.hpp"

#include <mutex>
#include "rowstats.hpp"
#include "../../include/d3d_hip.h"

#include <limits.h>

namespace d3d {
namespace accept {

using namespace rows;

constexpr int kMaxK = 127;       // K+1 target rows + K draft rows <= 255
constexpr int kMaxS = 1024;      // sparse support entries per position
constexpr int kPart = 4096;      // residual part: entries per workgroup
constexpr int kRun = kPart / NT; // contiguous entries per thread in a part
constexpr int kMaxParts = kMaxStatLds;  // V <= kMaxStatLds * kChunk
static_assert(kPart == kChunk, "part q is cleared by the stats workgroup of chunk q");
// Polls of a part record before a waiting workgroup gives up (with
// s_sleep 2 between polls, well over 100 ms).
constexpr int kSpinLimit = 1 << 20;

// Part record: two 8-byte words, each a float and a tag that is nonzero
// once written (tag = last positive index + 2).
struct PartRec {
    float r;  // sum of residual weights max(p - q, 0) over the part
    int tr;   // last index with positive residual + 2
    float p;  // sum of target probabilities over the part
    int tp;   // last index with positive probability + 2
};

struct Params {
    const void* target;
    const void* draft;
    const int64_t* tokens;
    const float* uniforms;
    const float* resample_u;
    float T;
    int B;
    int K;
    int V;
    int C;    // chunks (= parts) per row
    int Rm;   // rows merged per request: K + 1 (greedy, sparse) or 2K + 1
    RowStat* stats;  // [B][R][C], R = 2K+1 (target rows 0..K, draft rows K+1..2K)
    float* xtok;     // [B][R]: value of row r at its draft token (rows != K);
                     // sparse proposals: q at draft token i in slot K+1+i
    float* zsp;      // [B][K]: sparse support mass max(sum_s q_s, 1e-12)
    PartRec* parts;  // [B][C], cleared by the stats launch
    const int64_t* q_ids;  // sparse proposals [B][K][S], else null
    const float* q_probs;  // [B][K][S]
    int S;
    int32_t* accepted;
    uint8_t* mask;
    int64_t* out_token;
    uint8_t* all_accepted;
    int64_t* posterior;
};

// 8-byte agent-scope atomic store / load: coherent across XCDs without an
// L2 write-back.
__device__ __forceinline__ void store_word(void* dst, float v, int tag) {
    const uint64_t w = (uint64_t)__float_as_uint(v) | ((uint64_t)(uint32_t)tag << 32);
    __hip_atomic_store(static_cast<uint64_t*>(dst), w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t load_word(const void* src) {
    return __hip_atomic_load(static_cast<const uint64_t*>(src), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Sparse support mass Z = max(sum_s q_s, 1e-12) of position i and the
// normalised mass on token tok (sum over matching ids of q_s / Z), one wave
// per call.
__device__ __forceinline__ void sparse_q_at(const Params& P, int b, int i, int64_t tok, float& Z, float& qt) {
    const int lane = threadIdx.x & (kWave - 1);
    const size_t row = ((size_t)b * P.K + i) * P.S;
    float z = 0.f;
    for (int s = lane; s < P.S; s += kWave) z += P.q_probs[row + s];
    Z = fmaxf(wave_sum(z), 1e-12f);
    float m = 0.f;
    for (int s = lane; s < P.S; s += kWave)
        if (P.q_ids[row + s] == tok) m += P.q_probs[row + s] / Z;
    qt = wave_sum(m);
}

// ---------------------------------------------------------------- phase 1
template <int DT, bool VEC, Mode M>
__global__ __launch_bounds__(NT) void accept_stats_kernel(Params P) {
    constexpr int E = Vec<DT>::E;
    const int c = blockIdx.x, r = blockIdx.y, b = blockIdx.z;
    const int K = P.K, V = P.V, C = P.C, R = 2 * K + 1;
    __shared__ float rf[NT / kWave];
    __shared__ int ri[NT / kWave];

    const void* row = r <= K ? row_ptr<DT>(P.target, (size_t)b * (K + 1) + r, V)
                             : row_ptr<DT>(P.draft, (size_t)b * K + (r - K - 1), V);
    // Draft token scored by this row (target row i and draft row i: token i).
    const int ti = r < K ? r : r - K - 1;
    int64_t tok = -1;
    if (M != kGreedy && r != K && threadIdx.x == 0) tok = P.tokens[(size_t)b * K + ti];
    const int first = c * kChunk + threadIdx.x * E;
    float x[L];
    load_tile<DT, VEC, true, L>(row, V, first, NT * E, fill_value<M>(), x);
    // Argmax of the target rows: the greedy decision, and the posterior
    // output when the caller asks for it (it costs the stats pass about 1 us
    // at batch 8; the stochastic decision does not need it).
    const bool want_arg = r <= K && (M == kGreedy || P.posterior != nullptr);
    const RowStat st = P.T == 1.0f ? chunk_stats<DT, M, true>(x, first, P.T, want_arg, rf, ri)
                                   : chunk_stats<DT, M, false>(x, first, P.T, want_arg, rf, ri);
    if (threadIdx.x == 0) {
        P.stats[((size_t)b * R + r) * C + c] = st;
        // The workgroup whose chunk holds the token records its value once.
        if (M != kGreedy && tok >= (int64_t)c * kChunk && tok < (int64_t)(c + 1) * kChunk && tok < V)
            P.xtok[(size_t)b * R + r] = load_one<DT>(row, (int)tok);
        // Part record c of this request starts untagged, and the output
        // token at the timeout sentinel, for the finish launch (stream
        // order makes the stores visible to it).
        if (M != kGreedy && r == 0) {
            P.parts[(size_t)b * C + c] = PartRec{0.f, 0, 0.f, 0};
            if (c == 0) P.out_token[b] = D3D_TOKEN_TIMEOUT;
        }
    }
    // Sparse proposals: chunk 0 of target row i also reduces position i's
    // support (one wave): its mass and q at draft token i.
    if (M != kGreedy && P.S > 0 && c == 0 && r < K && threadIdx.x < kWave) {
        float Z, qt;
        sparse_q_at(P, b, r, P.tokens[(size_t)b * K + r], Z, qt);
        if (threadIdx.x == 0) {
            P.xtok[(size_t)b * R + K + 1 + r] = qt;
            P.zsp[(size_t)b * K + r] = Z;
        }
    }
}

// ---------------------------------------------------------------- sparse
// Residual weights of a sparse proposal over entries [lo, lo + span): buf
// holds p at local index e - lo on entry and p - sum(q_s / Z) (support
// order, unclamped) at every support id on exit.  Block-wide; every thread
// must call it.
__device__ __forceinline__ void sparse_subtract(const Params& P, int b, int n, float Z, int lo, int span,
                                                float* buf, int* s_id, float* s_q) {
    const size_t row = ((size_t)b * P.K + n) * P.S;
    for (int s = threadIdx.x; s < P.S; s += NT) {
        const int64_t id = P.q_ids[row + s];
        s_id[s] = (id >= lo && id < (int64_t)lo + span && id < P.V) ? (int)(id - lo) : -1;
        s_q[s] = P.q_probs[row + s] / Z;
    }
    __syncthreads();
    for (int s = threadIdx.x; s < P.S; s += NT) {
        const int li = s_id[s];
        if (li < 0) continue;
        bool first = true;
        for (int t = 0; t < s && first; ++t) first = s_id[t] != li;
        if (!first) continue;  // the first occurrence applies every duplicate, in order
        float v = buf[li];
        for (int t = s; t < P.S; ++t)
            if (s_id[t] == li) v -= s_q[t];
        buf[li] = v;
    }
    __syncthreads();
}

// ---------------------------------------------------------------- phase 2
// The decision of request b, computed with the same bits by each of its
// workgroups.
struct Decision {
    int n;     // first rejected position (K when all accepted)
    bool bad;  // a draft token outside [0, V)
    float Mt, It;  // selected target row: max z and 1 / normaliser
    float Mq, Iq;  // selected draft row (dense proposals)
    float Zq;      // support mass of the selected position (sparse proposals)
};

// Merges the request's chunk records, evaluates the accept test at every
// position and finds the first reject; the writer also stores the decision
// outputs (and, in greedy mode or on a bad draft, the output token).
template <int DT, Mode M, bool UNIT_T, bool SP>
__device__ __forceinline__ Decision decide(const Params& P, int b, bool writer) {
    __shared__ float sM[2 * kMaxK + 1], sS[2 * kMaxK + 1];
    __shared__ int sArg[kMaxK + 1];
    __shared__ RowStat lds[kMaxStatLds];
    __shared__ uint64_t s_bits[4];
    const int K = P.K, V = P.V, R = 2 * K + 1;
    const int tid = threadIdx.x;
    // Per-position inputs first: their loads overlap the record merge.
    int64_t tok = 0;
    float u = 0.f, xt = 0.f, xq = 0.f;
    if (tid < K) {
        tok = P.tokens[(size_t)b * K + tid];
        if (M != kGreedy) {
            u = P.uniforms[(size_t)b * K + tid];
            xt = P.xtok[(size_t)b * R + tid];
            xq = P.xtok[(size_t)b * R + K + 1 + tid];  // draft row value, or sparse q
        }
    }
    merge_row_stats<M>(P.stats + (size_t)b * R * P.C, P.Rm, P.C, K + 1, sM, sS, sArg, lds);
    bool acc = false, badp = false;
    if (tid < K) {
        badp = tok < 0 || tok >= V;
        if constexpr (M == kGreedy) {
            acc = !badp && tok == (int64_t)sArg[tid];
        } else {
            if (!badp) {
                const float pt = prob_of<M, UNIT_T>(xt, sM[tid], inv_sum<M>(sS[tid]), P.T);
                const float qt = SP ? xq : prob_of<M, UNIT_T>(xq, sM[K + 1 + tid], inv_sum<M>(sS[K + 1 + tid]), P.T);
                const float a = fminf(1.0f, pt / fmaxf(qt, 1e-12f));
                acc = u <= a;
            }
        }
    }
    {
        const uint64_t rej = __ballot(tid < K && !acc);
        // Greedy acceptance only compares a token with the argmax, so an
        // out-of-range token is a plain mismatch there; the other modes
        // index p and q by it and report the request instead.
        const uint64_t bb = __ballot(M != kGreedy && badp);
        const int wv = tid / kWave;
        if ((tid & (kWave - 1)) == 0 && wv < 2) {
            s_bits[wv] = rej;
            s_bits[2 + wv] = bb;
        }
    }
    __syncthreads();
    Decision d;
    d.n = s_bits[0] ? __builtin_ctzll(s_bits[0]) : (s_bits[1] ? 64 + __builtin_ctzll(s_bits[1]) : K);
    d.bad = (s_bits[2] | s_bits[3]) != 0;
    const int n = d.n;
    if (writer) {
        for (int p = tid; p < K; p += NT) P.mask[(size_t)b * K + p] = acc;
        if (P.posterior)
            for (int r = tid; r <= K; r += NT) P.posterior[(size_t)b * (K + 1) + r] = sArg[r];
        if (tid == 0) {
            P.accepted[b] = d.bad ? 0 : n;
            P.all_accepted[b] = !d.bad && n == K;
            if (M == kGreedy || d.bad)
                P.out_token[b] = d.bad ? (int64_t)D3D_TOKEN_BAD_DRAFT : (int64_t)sArg[n];
        }
    }
    d.Mt = sM[n];
    d.It = inv_sum<M>(sS[n]);
    d.Mq = 0.f;
    d.Iq = 0.f;
    d.Zq = 1.f;
    if (M != kGreedy && n < K) {
        if (SP) {
            d.Zq = P.zsp[(size_t)b * K + n];
        } else {
            d.Mq = sM[K + 1 + n];
            d.Iq = inv_sum<M>(sS[K + 1 + n]);
        }
    }
    return d;
}

// Entries e0 .. e0 + kRun - 1 of a row (fill past V).
template <int DT, bool VEC, Mode M>
__device__ __forceinline__ void load_run(const void* row, int V, int e0, float (&x)[kRun]) {
    constexpr int E = Vec<DT>::E;
    if (VEC && e0 + kRun <= V) {
#pragma unroll
        for (int j = 0; j < kRun / E; ++j) {
            if constexpr (DT == kF32) {
                const f32x4 v = reinterpret_cast<const f32x4*>(static_cast<const float*>(row) + e0)[j];
                x[j * 4 + 0] = v.x;
                x[j * 4 + 1] = v.y;
                x[j * 4 + 2] = v.z;
                x[j * 4 + 3] = v.w;
            } else {
                const u32x4 v = reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(row) + e0)[j];
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    x[j * 8 + 2 * h] = bf16_bits_to_f32(w[h] & 0xffffu);
                    x[j * 8 + 2 * h + 1] = bf16_bits_to_f32(w[h] >> 16);
                }
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < kRun; ++k) x[k] = e0 + k < V ? load_one<DT>(row, e0 + k) : fill_value<M>();
    }
}

// Weights of this thread's run of part q: wr = the residual max(p - q, 0)
// (zero when every position was accepted), wp = p.  Sparse proposals
// subtract the support through an LDS copy of the part.  Block-wide.
template <int DT, bool VEC, Mode M, bool UNIT_T, bool SP>
__device__ __forceinline__ void part_weights(const Params& P, int b, const Decision& d, int q, float (&wr)[kRun],
                                             float (&wp)[kRun]) {
    const int K = P.K, V = P.V;
    const bool res = d.n < K;
    const int e0 = q * kPart + (int)threadIdx.x * kRun;
    float xt[kRun];
    load_run<DT, VEC, M>(row_ptr<DT>(P.target, (size_t)b * (K + 1) + d.n, V), V, e0, xt);
#pragma unroll
    for (int k = 0; k < kRun; ++k) wp[k] = prob_of<M, UNIT_T>(xt[k], d.Mt, d.It, P.T);
    if constexpr (SP) {
        __shared__ float buf[kPart];
        __shared__ int s_id[kMaxS];
        __shared__ float s_q[kMaxS];
#pragma unroll
        for (int k = 0; k < kRun; ++k) buf[threadIdx.x * kRun + k] = wp[k];
        if (res) sparse_subtract(P, b, d.n, d.Zq, q * kPart, kPart, buf, s_id, s_q);
        else __syncthreads();
#pragma unroll
        for (int k = 0; k < kRun; ++k) wr[k] = res ? fmaxf(buf[threadIdx.x * kRun + k], 0.f) : 0.f;
        __syncthreads();  // buf is reused by the next call
    } else {
        if (res) {
            float xq[kRun];
            load_run<DT, VEC, M>(row_ptr<DT>(P.draft, (size_t)b * K + d.n, V), V, e0, xq);
#pragma unroll
            for (int k = 0; k < kRun; ++k) wr[k] = fmaxf(wp[k] - prob_of<M, UNIT_T>(xq[k], d.Mq, d.Iq, P.T), 0.f);
        } else {
#pragma unroll
            for (int k = 0; k < kRun; ++k) wr[k] = 0.f;
        }
    }
}

// Sums of the weights over the workgroup's part, their last positive
// indices, and each thread's exclusive prefix of its run sums within the
// part (thread order), for the residual (r) and target (p) weights: wave
// scans on the VALU, one barrier.  The part sums are the totals of the same
// scan, so a crossing located by the part sums is met again by the entry
// scan of the part.
struct PartSums {
    float r, p;
    int lr, lp;
};

__device__ __forceinline__ PartSums block_part_scan(float tr, float tp, int lr, int lp, float4* s4, float& xr,
                                                    float& xp) {
    const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
    const float ir = wave_incl_scan(tr, lane), ip = wave_incl_scan(tp, lane);
    const float er = up_f<1>(ir), ep = up_f<1>(ip);  // lane - 1's inclusive value
    lr = wave_max_int(lr);
    lp = wave_max_int(lp);
    if (lane == kWave - 1) s4[wv] = make_float4(ir, ip, __int_as_float(lr), __int_as_float(lp));
    __syncthreads();
    PartSums o{0.f, 0.f, -1, -1};
    float offr = 0.f, offp = 0.f;
#pragma unroll
    for (int k = 0; k < NT / kWave; ++k) {
        const float4 t = s4[k];
        if (k == wv) {
            offr = o.r;
            offp = o.p;
        }
        o.r += t.x;
        o.p += t.y;
        o.lr = max(o.lr, __float_as_int(t.z));
        o.lp = max(o.lp, __float_as_int(t.w));
    }
    xr = lane ? offr + er : offr;
    xp = lane ? offp + ep : offp;
    return o;
}

// Lowest `found` and highest `last` over the workgroup, one barrier.
__device__ __forceinline__ void block_min_max(int& found, int& last, int2* s2) {
    found = wave_min_int(found);
    last = wave_max_int(last);
    if ((threadIdx.x & (kWave - 1)) == 0) s2[threadIdx.x / kWave] = make_int2(found, last);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < NT / kWave; ++k) {
        found = min(found, s2[k].x);
        last = max(last, s2[k].y);
    }
}

// What wave 0 of every part workgroup derives from all part records.
struct Crossing {
    int late;   // a record did not arrive within the bound
    int cs;     // part where the inverse CDF crosses u * W (INT_MAX: none)
    int use_r;  // residual weights (else p)
    int last;   // last positive index over the row (fallback token)
    float W, target, base;  // total, u * W, weight of the parts before cs
};

// Wave 0: collects every part's sums (its own from registers, the others
// by polling their tagged records), then the part-level inverse CDF in
// part order.  Every workgroup of the request computes the same bits.
__device__ __forceinline__ Crossing find_crossing(const Params& P, int b, int q, const Decision& d,
                                                  const PartSums& own, float* s_r, float* s_p) {
    const int C = P.C, lane = threadIdx.x & (kWave - 1);
    float WR = 0.f, WP = 0.f;
    int LR = -1, LP = -1, late = 0;
    for (int q0 = 0; q0 < C; q0 += kWave) {
        const int qq = q0 + lane;
        float r = 0.f, p = 0.f;
        int lr = -1, lp = -1;
        if (qq == q) {
            r = own.r;
            p = own.p;
            lr = own.lr;
            lp = own.lp;
        } else if (qq < C) {
            const PartRec* rec = P.parts + (size_t)b * C + qq;
            uint64_t w0 = load_word(&rec->r), w1 = load_word(&rec->p);
            for (int it = 0; ((w0 >> 32) == 0 || (w1 >> 32) == 0) && it < kSpinLimit; ++it) {
                __builtin_amdgcn_s_sleep(2);
                if ((w0 >> 32) == 0) w0 = load_word(&rec->r);
                if ((w1 >> 32) == 0) w1 = load_word(&rec->p);
            }
            late |= (w0 >> 32) == 0 || (w1 >> 32) == 0;
            r = __uint_as_float((uint32_t)w0);
            p = __uint_as_float((uint32_t)w1);
            lr = (int)(w0 >> 32) - 2;
            lp = (int)(w1 >> 32) - 2;
        }
        if (qq < C) {
            s_r[qq] = r;
            s_p[qq] = p;
        }
        WR += wave_sum(r);
        WP += wave_sum(p);
        LR = max(LR, wave_max_int(lr));
        LP = max(LP, wave_max_int(lp));
    }
    Crossing x;
    x.late = wave_max_int(late);
    x.use_r = d.n < P.K && WR > 1e-12f;
    x.W = x.use_r ? WR : WP;
    x.last = x.use_r ? LR : LP;
    x.target = P.resample_u[b] * x.W;
    x.cs = INT_MAX;
    x.base = 0.f;
    if (x.late || !(x.W > 0.f)) return x;
    float carry = 0.f;
    for (int q0 = 0; q0 < C && x.cs == INT_MAX; q0 += kWave) {
        const int qq = q0 + lane;
        const float w = qq < C ? (x.use_r ? s_r[qq] : s_p[qq]) : 0.f;  // written by this lane
        const float incl = carry + wave_incl_scan(w, lane);
        const uint64_t hit = __ballot(qq < C && incl > x.target);
        if (hit) {
            const int f = __builtin_ctzll(hit);
            x.cs = q0 + f;
            x.base = __shfl(incl - w, f);
        }
        carry = __shfl(incl, kWave - 1);
    }
    return x;
}

template <int DT, bool VEC, Mode M, bool UNIT_T, bool SP>
__global__ __launch_bounds__(NT) void accept_finish_kernel(Params P) {
    const int per = M == kGreedy ? 1 : P.C;
    const int b = blockIdx.x / per, q = blockIdx.x - b * per;
    const bool writer = q == per - 1;
    const Decision d = decide<DT, M, UNIT_T, SP>(P, b, writer);
    if constexpr (M != kGreedy) {
        if (d.bad) return;
        __shared__ float4 s4[NT / kWave];
        __shared__ int2 s2[NT / kWave];
        __shared__ float s_r[kMaxParts], s_p[kMaxParts];
        __shared__ Crossing s_x;
        float wr[kRun], wp[kRun];
        part_weights<DT, VEC, M, UNIT_T, SP>(P, b, d, q, wr, wp);
        const int e0 = q * kPart + (int)threadIdx.x * kRun;
        float tr = 0.f, tp = 0.f;
        int lr = -1, lp = -1;
#pragma unroll
        for (int k = 0; k < kRun; ++k) {
            tr += wr[k];
            tp += wp[k];
            if (wr[k] > 0.f) lr = e0 + k;
            if (wp[k] > 0.f) lp = e0 + k;
        }
        float xr, xp;
        const PartSums own = block_part_scan(tr, tp, lr, lp, s4, xr, xp);
        if (threadIdx.x == 0) {
            PartRec* rec = P.parts + (size_t)b * P.C + q;
            store_word(&rec->r, own.r, own.lr + 2);
            store_word(&rec->p, own.p, own.lp + 2);
        }
        if (threadIdx.x < kWave) {
            const Crossing x = find_crossing(P, b, q, d, own, s_r, s_p);
            if (threadIdx.x == 0) s_x = x;
        }
        __syncthreads();
        const Crossing x = s_x;
        // out_token holds D3D_TOKEN_TIMEOUT from the stats launch until a
        // workgroup that saw every record writes the token.
        if (x.late) return;
        if (!(x.W > 0.f) || x.cs == INT_MAX) {
            if (writer && threadIdx.x == 0)
                P.out_token[b] = x.W > 0.f ? (int64_t)x.last : (int64_t)D3D_TOKEN_EMPTY_DISTRIBUTION;
            return;
        }
        if (x.cs != q) return;
        // This part holds the crossing: scan its entries in index order.
        float run = x.base + (x.use_r ? xr : xp);
        int found = INT_MAX, lastpos = -1;
#pragma unroll
        for (int k = 0; k < kRun; ++k) {
            const float w = x.use_r ? wr[k] : wp[k];
            run += w;
            if (w > 0.f) {
                lastpos = e0 + k;
                if (found == INT_MAX && run > x.target) found = e0 + k;
            }
        }
        block_min_max(found, lastpos, s2);
        if (threadIdx.x == 0) P.out_token[b] = found != INT_MAX ? found : lastpos;
    }
}

struct Layout {
    size_t stats, xtok, zsp, parts, total;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static int num_chunks(int64_t V) { return (int)((V + kChunk - 1) / kChunk); }

static Layout layout(int B, int K, int64_t V) {
    Layout l;
    const size_t C = (size_t)num_chunks(V), R = 2 * (size_t)K + 1;
    l.stats = 0;
    l.xtok = align256((size_t)B * R * C * sizeof(RowStat));
    l.zsp = l.xtok + align256((size_t)B * R * sizeof(float));
    l.parts = l.zsp + align256((size_t)B * K * sizeof(float));
    l.total = l.parts + align256((size_t)B * C * sizeof(PartRec));
    return l;
}

template <int DT, bool VEC, bool SP, Mode M, bool UNIT_T>
static void launch_mode(const Params& P, hipStream_t stream) {
    const dim3 grid_stats(P.C, P.Rm, P.B);
    hipLaunchKernelGGL((accept_stats_kernel<DT, VEC, M>), grid_stats, dim3(NT), 0, stream, P);
    const int per = M == kGreedy ? 1 : P.C;
    hipLaunchKernelGGL((accept_finish_kernel<DT, VEC, M, UNIT_T, SP>), dim3(P.B * per), dim3(NT), 0, stream, P);
}

template <int DT, bool VEC, bool SP>
static hipError_t launch(const Params& P, Mode mode, hipStream_t stream) {
    switch (mode) {
        case kGreedy:
            launch_mode<DT, VEC, SP, kGreedy, true>(P, stream);
            break;
        case kLogits:
            if (P.T == 1.0f)
                launch_mode<DT, VEC, SP, kLogits, true>(P, stream);
            else
                launch_mode<DT, VEC, SP, kLogits, false>(P, stream);
            break;
        default:
            launch_mode<DT, VEC, SP, kProbs, true>(P, stream);
            break;
    }
    return hipGetLastError();
}

// Shared by the dense and sparse entry points: validation, workspace carving
// and dispatch.
static int run(const void* target, const void* draft, const int64_t* q_ids, const float* q_probs, int S,
               int dtype, int input_kind, const int64_t* draft_tokens, const float* uniforms,
               const float* resample_u, float temperature, int B, int K, int64_t V, int32_t* accepted,
               uint8_t* accept_mask, int64_t* out_token, uint8_t* all_accepted, int64_t* posterior,
               void* workspace, size_t workspace_bytes, void* stream) {
    const bool sparse = q_ids != nullptr || q_probs != nullptr || S != 0;
    if (B < 1 || B > 65535 || K < 1 || K > kMaxK || V < 1 || V > (int64_t)kMaxStatLds * kChunk)
        return D3D_E_SHAPE;
    if (sparse && (S < 1 || S > kMaxS)) return D3D_E_SHAPE;
    if (dtype != D3D_DTYPE_F32 && dtype != D3D_DTYPE_BF16) return D3D_E_DTYPE;
    if (input_kind != D3D_INPUT_LOGITS && input_kind != D3D_INPUT_PROBS) return D3D_E_UNSUPPORTED;
    const bool greedy = input_kind == D3D_INPUT_LOGITS && !(temperature > 1e-5f);
    if (!target || !draft_tokens || !accepted || !accept_mask || !out_token || !all_accepted || !workspace)
        return D3D_E_NULL;
    if (!greedy && (!uniforms || !resample_u)) return D3D_E_NULL;
    if (!greedy && (sparse ? (!q_ids || !q_probs) : !draft)) return D3D_E_NULL;
    const Layout lay = layout(B, K, V);
    if (workspace_bytes < lay.total) return D3D_E_WORKSPACE;

    char* ws = static_cast<char*>(workspace);
    Params P;
    P.target = target;
    P.draft = (greedy || sparse) ? nullptr : draft;
    P.tokens = draft_tokens;
    P.uniforms = uniforms;
    P.resample_u = resample_u;
    P.T = input_kind == D3D_INPUT_LOGITS ? temperature : 1.0f;
    P.B = B;
    P.K = K;
    P.V = (int)V;
    P.C = num_chunks(V);
    P.Rm = (greedy || sparse) ? K + 1 : 2 * K + 1;
    P.stats = reinterpret_cast<RowStat*>(ws + lay.stats);
    P.xtok = reinterpret_cast<float*>(ws + lay.xtok);
    P.zsp = reinterpret_cast<float*>(ws + lay.zsp);
    P.parts = reinterpret_cast<PartRec*>(ws + lay.parts);
    P.q_ids = sparse ? q_ids : nullptr;
    P.q_probs = sparse ? q_probs : nullptr;
    P.S = sparse ? S : 0;
    P.accepted = accepted;
    P.mask = accept_mask;
    P.out_token = out_token;
    P.all_accepted = all_accepted;
    P.posterior = posterior;

    const size_t esize = dtype == D3D_DTYPE_F32 ? 4 : 2;
    const bool vec = ((uintptr_t)target % 16 == 0) && (greedy || sparse || (uintptr_t)draft % 16 == 0) &&
                     ((size_t)V * esize) % 16 == 0;
    const Mode mode = greedy ? kGreedy : (input_kind == D3D_INPUT_PROBS ? kProbs : kLogits);
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t err;
    if (dtype == D3D_DTYPE_F32) {
        if (sparse)
            err = vec ? launch<kF32, true, true>(P, mode, s) : launch<kF32, false, true>(P, mode, s);
        else
            err = vec ? launch<kF32, true, false>(P, mode, s) : launch<kF32, false, false>(P, mode, s);
    } else {
        if (sparse)
            err = vec ? launch<kBF16, true, true>(P, mode, s) : launch<kBF16, false, true>(P, mode, s);
        else
            err = vec ? launch<kBF16, true, false>(P, mode, s) : launch<kBF16, false, false>(P, mode, s);
    }
    return err == hipSuccess ? D3D_OK : (int)err;
}

}  // namespace accept
}  // namespace d3d

// Scratch of d3d_accept_fused_noalloc: one copy per GPU, held until the
// process ends.  In host code the name is a stand-in for the symbol, not a
// device address: the address comes from hipGetSymbolAddress, per device.
static __device__ __align__(256) unsigned char scratch[D3D_ACCEPT_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the device that owns `stream` (the current
// device for the null stream), looked up once per device with that device
// current.
int scratch_address(void* stream, void** out) {
    int dev = 0;
    hipError_t e = stream ? hipStreamGetDevice(static_cast<hipStream_t>(stream), &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxScratchDevices) return D3D_E_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        int cur = 0;
        e = hipGetDevice(&cur);
        if (e != hipSuccess) return (int)e;
        if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return (int)e;
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) {
            const hipError_t r = hipSetDevice(cur);
            if (e == hipSuccess) e = r;
        }
        if (e != hipSuccess) return (int)e;
        if (!p) return D3D_E_NULL;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return D3D_OK;
}

}  // namespace

using namespace d3d;

extern "C" size_t d3d_accept_workspace_bytes(int B, int K, int64_t V) {
    if (B < 1 || K < 1 || V < 1) return 0;
    return accept::layout(B, K, V).total;
}

extern "C" int d3d_accept_fused(const void* target, const void* draft, int dtype, int input_kind,
                                const int64_t* draft_tokens, const float* uniforms,
                                const float* resample_u, float temperature, int B, int K, int64_t V,
                                int32_t* accepted, uint8_t* accept_mask, int64_t* out_token,
                                uint8_t* all_accepted, int64_t* posterior, void* workspace,
                                size_t workspace_bytes, void* stream) {
    return accept::run(target, draft, nullptr, nullptr, 0, dtype, input_kind, draft_tokens, uniforms, resample_u,
                       temperature, B, K, V, accepted, accept_mask, out_token, all_accepted, posterior, workspace,
                       workspace_bytes, stream);
}

extern "C" int d3d_accept_fused_sparse(const void* target, int dtype, int input_kind,
                                       const int64_t* draft_tokens, const int64_t* q_ids, const float* q_probs,
                                       int S, const float* uniforms, const float* resample_u, float temperature,
                                       int B, int K, int64_t V, int32_t* accepted, uint8_t* accept_mask,
                                       int64_t* out_token, uint8_t* all_accepted, int64_t* posterior,
                                       void* workspace, size_t workspace_bytes, void* stream) {
    if (S < 1) return D3D_E_SHAPE;
    return accept::run(target, nullptr, q_ids, q_probs, S, dtype, input_kind, draft_tokens, uniforms, resample_u,
                       temperature, B, K, V, accepted, accept_mask, out_token, all_accepted, posterior, workspace,
                       workspace_bytes, stream);
}

extern "C" int d3d_accept_fused_noalloc(const void* target, const void* draft, int dtype, int input_kind,
                                        const int64_t* draft_tokens, const float* uniforms,
                                        const float* resample_u, float temperature, int B, int K, int64_t V,
                                        int32_t* accepted, uint8_t* accept_mask, int64_t* out_token,
                                        uint8_t* all_accepted, int64_t* posterior, void* stream) {
    if (B < 1 || K < 1 || V < 1) return D3D_E_SHAPE;
    // Sizes whose workspace would not fit the static scratch are refused
    // before anything is launched.
    if (accept::layout(B, K, V).total > (size_t)D3D_ACCEPT_NOALLOC_SCRATCH_BYTES) return D3D_E_WORKSPACE;
    void* ws = nullptr;
    const int st = scratch_address(stream, &ws);
    if (st != D3D_OK) return st;
    return accept::run(target, draft, nullptr, nullptr, 0, dtype, input_kind, draft_tokens, uniforms, resample_u,
                       temperature, B, K, V, accepted, accept_mask, out_token, all_accepted, posterior, ws,
                       (size_t)D3D_ACCEPT_NOALLOC_SCRATCH_BYTES, stream);
}
