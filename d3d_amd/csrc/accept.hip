// Fused speculative acceptance for gfx950.
//
// Three stream-ordered phases, no atomics and no cross-workgroup waits:
//
//   1. stats     grid (C, rows, B).  Workgroup (c, r, b) streams chunk c of
//                row r of request b once (target rows 0..K, then draft rows
//                0..K-1; greedy mode reads target rows only) and reduces it to
//                (max z, sum exp(z - max z), max x, argmax) with z = x / T, or
//                to a plain sum for probability inputs.
//   2. decide    grid (C, B).  Every workgroup of request b merges the chunk
//                statistics of all rows in one fixed order (so all of them
//                reach the same bits), evaluates u_i <= min(1, p_i / max(q_i,
//                1e-12)) at every position and finds the first reject.
//                Workgroup 0 writes the outputs; in stochastic modes every
//                workgroup then reduces chunk c of the selected row pair
//                (residual max(p - q, 0), and p) to chunk sums.
//   3. resample  grid (B), stochastic modes only.  Locates the chunk in which
//                the inverse CDF crosses u * W and scans it entry by entry.
//
// The phases replace per-workgroup completion counters: on MI355X a
// device-scope release per workgroup (L2 write-back across XCDs) and
// same-address atomics serialise, and cost far more than two extra launches
// (folding phase 3 into phase 2 with a last-workgroup counter measured
// 17 -> 22 us at one request and 43 -> 60 us at eight).
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
// Phase 1 then reads target rows only; phase 2 computes q at the draft token
// as the normalised support mass on that id, and the residual of the reject
// row subtracts the normalised support from p entry by entry, in support
// order (scatter_add), before the clamp at zero.  Ids outside [0, V) carry
// no mass.
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
// Phases 2 and 3 are latency-bound, so their chunks hold nv2 16-byte vectors
// per thread (nv2 in 1..kMaxNv2), chosen per launch: few requests get fine
// chunks (more workgroups, shorter per-thread chains), many requests get
// coarse ones (fewer redundant row merges).
constexpr int kMaxNv2 = 4;
constexpr int kMaxS = 1024;  // sparse support entries per position

struct Decision {
    int n;  // first rejected position (K when all accepted)
    int flags;
    float Mt, St, Mq, Sq;  // row statistics of the selected target/draft rows
                           // (sparse proposals: Sq = support mass of the reject row)
    int pad0, pad1;
};

struct ResStat {
    float r;     // sum of residual weights over the chunk
    float p;     // sum of target probabilities over the chunk
    int last_r;  // last index with positive residual (-1 if none)
    int last_p;  // last index with positive probability (-1 if none)
};

enum : int { kFlagInvalid = 1 };

struct Params {
    const void* target;
    const void* draft;
    const int64_t* tokens;
    const float* uniforms;
    const float* resample_u;
    float T;
    int K;
    int V;
    int C;   // phase-1 chunks per row
    int C2;  // phase-2/3 sub-chunks per row (NT 16-byte vectors each)
    int nv2; // sub-chunks per phase-2 workgroup
    RowStat* stats;  // [B][R][C], R = 2K+1 (target rows 0..K, draft rows K+1..2K)
    Decision* dec;   // [B]
    ResStat* rstats; // [B][C]
    float* xtok;     // [B][R]: value of row r at its draft token (rows != K)
    const int64_t* q_ids;  // sparse proposals [B][K][S], else null
    const float* q_probs;  // [B][K][S]
    int S;
    int32_t* accepted;
    uint8_t* mask;
    int64_t* out_token;
    uint8_t* all_accepted;
    int64_t* posterior;
};

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
    const bool want_arg = r <= K;  // posterior needs target rows only
    const RowStat st = P.T == 1.0f ? chunk_stats<DT, M, true>(x, first, P.T, want_arg, rf, ri)
                                   : chunk_stats<DT, M, false>(x, first, P.T, want_arg, rf, ri);
    if (threadIdx.x == 0) {
        P.stats[((size_t)b * R + r) * C + c] = st;
        // The workgroup whose chunk holds the token records its value once.
        if (M != kGreedy && tok >= (int64_t)c * kChunk && tok < (int64_t)(c + 1) * kChunk && tok < V)
            P.xtok[(size_t)b * R + r] = load_one<DT>(row, (int)tok);
    }
}

// ---------------------------------------------------------------- sparse
// Support mass Z = max(sum_s q_s, 1e-12) of position i and the normalised
// mass on token tok (sum over matching ids of q_s / Z), one wave per call.
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
// Row statistics of request b: sM/sS per row (target rows 0..K, draft rows
// K+1..2K) and sArg for target rows.
template <Mode M, bool SP>
__device__ __forceinline__ void merge_rows(const Params& P, int b, float* sM, float* sS, int* sArg,
                                           RowStat* lds) {
    const int K = P.K, C = P.C, R = 2 * K + 1;
    merge_row_stats<M>(P.stats + (size_t)b * R * C, (M == kGreedy || SP) ? K + 1 : R, C, K + 1, sM, sS, sArg,
                       lds);
}

// One descending butterfly step of the residual chunk sums (sub-chunks
// j < nv2): sums of r and p, last positive index of each.
template <int O>
__device__ __forceinline__ void res_step(float (&rs)[kMaxNv2], float (&ps)[kMaxNv2], int (&lr)[kMaxNv2],
                                         int (&lp)[kMaxNv2], int nv2) {
#pragma unroll
    for (int j = 0; j < kMaxNv2; ++j) {
        if (j >= nv2) break;
        rs[j] += xor_desc<O>(rs[j]);
        ps[j] += xor_desc<O>(ps[j]);
        lr[j] = max(lr[j], xor_desc<O>(lr[j]));
        lp[j] = max(lp[j], xor_desc<O>(lp[j]));
    }
}

template <int DT, bool VEC, Mode M, bool UNIT_T, bool SP>
__device__ __forceinline__ void decide_body(const Params& P, int c, int b, RowStat* lds, float* sM, float* sS,
                                            int* sArg, uint64_t* s_bits, float* rf, int* ri) {
    __shared__ float sQt[SP ? kMaxK : 1], sZ[SP ? kMaxK : 1];
    constexpr int E = Vec<DT>::E;
    const int K = P.K, V = P.V;
    const int tid = threadIdx.x;

    // Independent loads first: tokens, uniforms and token values.
    int64_t tok = 0;
    float u = 0.f, xt = 0.f, xq = 0.f;
    if (tid < K) {
        tok = P.tokens[(size_t)b * K + tid];
        if (M != kGreedy) {
            u = P.uniforms[(size_t)b * K + tid];
            xt = P.xtok[(size_t)b * (2 * K + 1) + tid];
            if (!SP) xq = P.xtok[(size_t)b * (2 * K + 1) + K + 1 + tid];
        }
    }
    if constexpr (SP) {
        // q at the draft token of every position, one wave per position.
        for (int i = tid / kWave; i < K; i += NT / kWave) {
            float Z, qt;
            sparse_q_at(P, b, i, P.tokens[(size_t)b * K + i], Z, qt);
            if ((tid & (kWave - 1)) == 0) {
                sZ[i] = Z;
                sQt[i] = qt;
            }
        }
    }
    merge_rows<M, SP>(P, b, sM, sS, sArg, lds);
    if constexpr (SP) __syncthreads();

    // Per-position decisions, then the first reject and the bad-token flag
    // from wave ballots (positions 0..K-1 live in waves 0 and 1).
    bool acc = false, badp = false;
    if (tid < K) {
        badp = tok < 0 || tok >= V;
        if constexpr (M == kGreedy) {
            acc = !badp && tok == (int64_t)sArg[tid];
        } else {
            if (!badp) {
                const float pt = prob_of<M, UNIT_T>(xt, sM[tid], inv_sum<M>(sS[tid]), P.T);
                const float qt = SP ? sQt[tid]
                                    : prob_of<M, UNIT_T>(xq, sM[K + 1 + tid], inv_sum<M>(sS[K + 1 + tid]), P.T);
                const float a = fminf(1.0f, pt / fmaxf(qt, 1e-12f));
                acc = u <= a;
            }
        }
    }
    {
        const uint64_t rej = __ballot(tid < K && !acc);
        const uint64_t bb = __ballot(badp);
        const int wv = tid / kWave;
        if ((tid & (kWave - 1)) == 0 && wv < 2) {
            s_bits[wv] = rej;
            s_bits[2 + wv] = bb;
        }
    }
    __syncthreads();
    const int n = s_bits[0] ? __builtin_ctzll(s_bits[0]) : (s_bits[1] ? 64 + __builtin_ctzll(s_bits[1]) : K);
    const bool bad = (s_bits[2] | s_bits[3]) != 0;
    if (c == 0) {
        for (int p = tid; p < K; p += NT) P.mask[(size_t)b * K + p] = acc;
        if (P.posterior)
            for (int r = tid; r <= K; r += NT) P.posterior[(size_t)b * (K + 1) + r] = sArg[r];
        if (tid == 0) {
            P.accepted[b] = bad ? 0 : n;
            P.all_accepted[b] = !bad && n == K;
            if (M == kGreedy || bad)
                P.out_token[b] = bad ? (int64_t)D3D_TOKEN_BAD_DRAFT : (int64_t)sArg[n];
            if (M != kGreedy) {
                Decision d;
                d.n = n;
                d.flags = bad ? kFlagInvalid : 0;
                d.Mt = sM[n];
                d.St = sS[n];
                d.Mq = (n < K && !SP) ? sM[K + 1 + n] : 0.f;
                d.Sq = n < K ? (SP ? sZ[n] : sS[K + 1 + n]) : 0.f;
                d.pad0 = d.pad1 = 0;
                P.dec[b] = d;
            }
        }
    }
    if constexpr (M != kGreedy) {
        if (bad) return;
        // Chunk sums of the selected row pair (reject row, or bonus row).
        const bool res = n < K;
        const void* trow = row_ptr<DT>(P.target, (size_t)b * (K + 1) + n, V);
        const bool dres = res && !SP;  // dense draft row to read
        const void* drow = dres ? row_ptr<DT>(P.draft, (size_t)b * K + n, V) : nullptr;
        const float Mt = sM[n], It = inv_sum<M>(sS[n]);
        const float Mq = dres ? sM[K + 1 + n] : 0.f, Iq = dres ? inv_sum<M>(sS[K + 1 + n]) : 0.f;
        // Workgroup c covers sub-chunks c*nv2 .. c*nv2+nv2-1; sub-chunk j is
        // vector j of every thread (NT*E consecutive entries) and gets its own
        // record, so phase 3 always scans one vector per thread.
        constexpr int LM = kMaxNv2 * E;
        const int nv2 = P.nv2;
        const int first = c * (NT * E * nv2) + tid * E;
        float xt[LM], xq[LM];
        load_tile_n<DT, VEC, LM>(trow, V, first, NT * E, nv2, fill_value<M>(), xt);
        if (dres) load_tile_n<DT, VEC, LM>(drow, V, first, NT * E, nv2, fill_value<M>(), xq);
        if constexpr (SP) {
            // xq <- p - q (unclamped) through the workgroup's LDS copy of p.
            __shared__ float buf[NT * kMaxNv2 * E];
            __shared__ int s_id[kMaxS];
            __shared__ float s_q[kMaxS];
            const int lo = c * (NT * E * nv2);
#pragma unroll
            for (int j = 0; j < kMaxNv2; ++j)
#pragma unroll
                for (int k = 0; k < E; ++k)
                    if (j < nv2) buf[j * NT * E + tid * E + k] = prob_of<M, UNIT_T>(xt[j * E + k], Mt, It, P.T);
            if (res) sparse_subtract(P, b, n, sZ[n], lo, NT * E * nv2, buf, s_id, s_q);
#pragma unroll
            for (int j = 0; j < kMaxNv2; ++j)
#pragma unroll
                for (int k = 0; k < E; ++k)
                    if (j < nv2) xq[j * E + k] = buf[j * NT * E + tid * E + k];
        }
        float rs[kMaxNv2], ps[kMaxNv2];
        int lr[kMaxNv2], lp[kMaxNv2];
#pragma unroll
        for (int j = 0; j < kMaxNv2; ++j) {
            rs[j] = ps[j] = 0.f;
            lr[j] = lp[j] = -1;
            if (j >= nv2) continue;
#pragma unroll
            for (int k = 0; k < E; ++k) {
                const int l = j * E + k;
                const int e = first + j * NT * E + k;
                const float p = prob_of<M, UNIT_T>(xt[l], Mt, It, P.T);
                ps[j] += p;
                if (p > 0.f) lp[j] = e;
                if (res) {
                    const float r = SP ? fmaxf(xq[l], 0.f) : fmaxf(p - prob_of<M, UNIT_T>(xq[l], Mq, Iq, P.T), 0.f);
                    rs[j] += r;
                    if (r > 0.f) lr[j] = e;
                }
            }
        }
        // One combined workgroup reduction for the nv2 sub-chunks.
        res_step<32>(rs, ps, lr, lp, nv2);
        res_step<16>(rs, ps, lr, lp, nv2);
        res_step<8>(rs, ps, lr, lp, nv2);
        res_step<4>(rs, ps, lr, lp, nv2);
        res_step<2>(rs, ps, lr, lp, nv2);
        res_step<1>(rs, ps, lr, lp, nv2);
        __shared__ ResStat s_red[NT / kWave][kMaxNv2];
        const int lane = tid & (kWave - 1), wv = tid / kWave;
        if (lane == 0)
#pragma unroll
            for (int j = 0; j < kMaxNv2; ++j) s_red[wv][j] = ResStat{rs[j], ps[j], lr[j], lp[j]};
        __syncthreads();
        if (tid < nv2 && c * nv2 + tid < P.C2) {
            ResStat st = s_red[0][tid];
            for (int w = 1; w < NT / kWave; ++w) {
                const ResStat t = s_red[w][tid];
                st.r += t.r;
                st.p += t.p;
                st.last_r = max(st.last_r, t.last_r);
                st.last_p = max(st.last_p, t.last_p);
            }
            P.rstats[(size_t)b * P.C2 + c * nv2 + tid] = st;
        }
    }
}

template <int DT, bool VEC, Mode M, bool SP>
__global__ __launch_bounds__(NT) void accept_decide_kernel(Params P) {
    __shared__ RowStat lds[kMaxStatLds];
    __shared__ float sM[2 * kMaxK + 2], sS[2 * kMaxK + 2];
    __shared__ int sArg[kMaxK + 1];
    __shared__ uint64_t s_bits[4];
    __shared__ float rf[NT / kWave];
    __shared__ int ri[NT / kWave];
    if (P.T == 1.0f)
        decide_body<DT, VEC, M, true, SP>(P, blockIdx.x, blockIdx.y, lds, sM, sS, sArg, s_bits, rf, ri);
    else
        decide_body<DT, VEC, M, false, SP>(P, blockIdx.x, blockIdx.y, lds, sM, sS, sArg, s_bits, rf, ri);
}

// ---------------------------------------------------------------- phase 3
template <int DT, bool VEC, Mode M, bool UNIT_T, bool SP>
__device__ __forceinline__ void resample_body(const Params& P, int b, float* s_wave, float* s_f, int* s_i,
                                              int* ri) {
    constexpr int E = Vec<DT>::E;
    const int K = P.K, V = P.V, C = P.C2;
    const int tid = threadIdx.x;
    // All independent loads are issued before the first use.
    const Decision d = P.dec[b];
    const float v = P.resample_u[b];
    ResStat mine0;  // this thread's chunk record of the first pass, reused below
    mine0.r = mine0.p = 0.f;
    mine0.last_r = mine0.last_p = -1;
    if (tid < C) mine0 = P.rstats[(size_t)b * C + tid];
    if (d.flags & kFlagInvalid) return;
    const bool res = d.n < K;
    const float It = inv_sum<M>(d.St), Iq = (res && !SP) ? inv_sum<M>(d.Sq) : 0.f;

    // Chunk-level inverse CDF: inclusive scan of chunk sums in chunk order,
    // the crossing chunk is the first whose inclusive sum exceeds v * W.
    // The weights are the residual unless its mass is <= 1e-12.
    float WR = 0.f, WP = 0.f;
    int LR = -1, LP = -1;
    int cs = INT_MAX;
    float base = 0.f;
    bool use_r;
    float W, target;
    if (C <= NT) {
        // One record per thread: both scans, both maxima and the crossing
        // in two workgroup exchanges.
        __shared__ float s_tot[2][NT / kWave];
        __shared__ int s_max[2][NT / kWave];
        __shared__ int s_first[NT / kWave];
        __shared__ float s_base[NT / kWave];
        const int lane = tid & (kWave - 1), wv = tid / kWave;
        float ir = wave_incl_scan(mine0.r, lane), ip = wave_incl_scan(mine0.p, lane);
        const int mr = wave_max_int(mine0.last_r), mp = wave_max_int(mine0.last_p);
        if (lane == kWave - 1) {
            s_tot[0][wv] = ir;
            s_tot[1][wv] = ip;
        }
        if (lane == 0) {
            s_max[0][wv] = mr;
            s_max[1][wv] = mp;
        }
        __syncthreads();
        // Same arithmetic as block_incl_scan: wave scan + earlier waves' totals.
        float orr = 0.f, orp = 0.f;
        for (int k = 0; k < NT / kWave; ++k) {
            if (k < wv) {
                orr += s_tot[0][k];
                orp += s_tot[1][k];
            }
            LR = max(LR, s_max[0][k]);
            LP = max(LP, s_max[1][k]);
        }
        {
            float offr = 0.f, offp = 0.f;
            for (int k = 0; k < NT / kWave - 1; ++k) {
                offr += s_tot[0][k];
                offp += s_tot[1][k];
            }
            WR = s_tot[0][NT / kWave - 1] + offr;  // the scan's last element
            WP = s_tot[1][NT / kWave - 1] + offp;
        }
        ir += orr;
        ip += orp;
        use_r = res && WR > 1e-12f;
        W = use_r ? WR : WP;
        target = v * W;
        const float incl = use_r ? ir : ip, w = use_r ? mine0.r : mine0.p;
        const uint64_t bal = __ballot(tid < C && incl > target);
        if (bal && lane == __builtin_ctzll(bal)) {
            s_first[wv] = tid;
            s_base[wv] = incl - w;
        }
        if (!bal && lane == 0) s_first[wv] = INT_MAX;
        __syncthreads();
        for (int k = 0; k < NT / kWave; ++k)
            if (s_first[k] != INT_MAX) {
                cs = s_first[k];
                base = s_base[k];
                break;
            }
        if (!(W > 0.f)) {
            if (tid == 0) P.out_token[b] = D3D_TOKEN_EMPTY_DISTRIBUTION;
            return;
        }
    } else {
    for (int c0 = 0; c0 < C; c0 += NT) {
        float r = 0.f, p = 0.f;
        if (c0 + tid < C) {
            const ResStat t = c0 == 0 ? mine0 : P.rstats[(size_t)b * C + c0 + tid];
            r = t.r;
            p = t.p;
            LR = max(LR, t.last_r);
            LP = max(LP, t.last_p);
        }
        const float ir = block_incl_scan(r, s_wave);
        const float ip = block_incl_scan(p, s_wave);
        if (tid == NT - 1) {
            s_f[0] = ir;
            s_f[1] = ip;
        }
        __syncthreads();
        WR += s_f[0];
        WP += s_f[1];
        __syncthreads();
    }
    LR = block_max_int(LR, ri);
    LP = block_max_int(LP, ri);
    use_r = res && WR > 1e-12f;
    W = use_r ? WR : WP;
    target = v * W;
    if (!(W > 0.f)) {
        if (tid == 0) P.out_token[b] = D3D_TOKEN_EMPTY_DISTRIBUTION;
        return;
    }
    float carry = 0.f;
    for (int c0 = 0; c0 < C && cs == INT_MAX; c0 += NT) {
        float w = 0.f;
        if (c0 + tid < C) {
            const ResStat t = c0 == 0 ? mine0 : P.rstats[(size_t)b * C + c0 + tid];
            w = use_r ? t.r : t.p;
        }
        const float incl = carry + block_incl_scan(w, s_wave);
        const int mine = (c0 + tid < C && incl > target) ? c0 + tid : INT_MAX;
        const int first = block_min_int(mine, ri);
        if (first != INT_MAX && first == c0 + tid) s_f[2] = incl - w;
        if (tid == NT - 1) s_f[3] = incl;
        __syncthreads();
        if (first != INT_MAX) {
            cs = first;
            base = s_f[2];
        }
        carry = s_f[3];
        __syncthreads();
    }
    }
    int token;
    if (cs == INT_MAX) {
        token = use_r ? LR : LP;
    } else {
        // Contiguous ownership: thread tid holds entries first..first+L-1.
        // Sub-chunk cs: thread tid owns entries first..first+E-1.
        const int first = cs * (NT * E) + tid * E;
        float xt[E], xq[E];
        load_tile<DT, VEC, false, E>(row_ptr<DT>(P.target, (size_t)b * (K + 1) + d.n, V), V, first, E,
                                     fill_value<M>(), xt);
        if (res && !SP)
            load_tile<DT, VEC, false, E>(row_ptr<DT>(P.draft, (size_t)b * K + d.n, V), V, first, E,
                                         fill_value<M>(), xq);
        float w[E];
        if constexpr (SP) {
            __shared__ float buf[NT * E];
            __shared__ int s_id[kMaxS];
            __shared__ float s_q[kMaxS];
#pragma unroll
            for (int l = 0; l < E; ++l) buf[tid * E + l] = prob_of<M, UNIT_T>(xt[l], d.Mt, It, P.T);
            if (use_r) sparse_subtract(P, b, d.n, d.Sq, cs * (NT * E), NT * E, buf, s_id, s_q);
            else __syncthreads();
#pragma unroll
            for (int l = 0; l < E; ++l) w[l] = use_r ? fmaxf(buf[tid * E + l], 0.f) : buf[tid * E + l];
        }
        float tsum = 0.f;
#pragma unroll
        for (int l = 0; l < E; ++l) {
            if constexpr (!SP) {
                const float p = prob_of<M, UNIT_T>(xt[l], d.Mt, It, P.T);
                w[l] = use_r ? fmaxf(p - prob_of<M, UNIT_T>(xq[l], d.Mq, Iq, P.T), 0.f) : p;
            }
            tsum += w[l];
        }
        const float incl = block_incl_scan(tsum, s_wave);
        float run = base + (incl - tsum);
        int found = INT_MAX, lastpos = -1;
#pragma unroll
        for (int l = 0; l < E; ++l) {
            run += w[l];
            if (w[l] > 0.f) {
                lastpos = first + l;
                if (found == INT_MAX && run > target) found = first + l;
            }
        }
        found = block_min_int(found, ri);
        lastpos = block_max_int(lastpos, ri);
        token = found != INT_MAX ? found : lastpos;
    }
    if (tid == 0) P.out_token[b] = token;
}

template <int DT, bool VEC, Mode M, bool SP>
__global__ __launch_bounds__(NT) void accept_resample_kernel(Params P) {
    __shared__ float s_wave[NT / kWave];
    __shared__ float s_f[4];
    __shared__ int s_i[2];
    __shared__ int ri[NT / kWave];
    if (P.T == 1.0f)
        resample_body<DT, VEC, M, true, SP>(P, blockIdx.x, s_wave, s_f, s_i, ri);
    else
        resample_body<DT, VEC, M, false, SP>(P, blockIdx.x, s_wave, s_f, s_i, ri);
}

struct Layout {
    size_t stats, dec, rstats, xtok, total;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static int num_chunks(int64_t V) { return (int)((V + kChunk - 1) / kChunk); }
// Vectors per thread in phase-2/3 chunks: aim for >= ~128 workgroups per
// launch with as few redundant row merges as possible.
static int pick_nv2(int B) { return B >= 4 ? 4 : (B >= 2 ? 2 : 1); }
static int num_subchunks(int64_t V, int dtype) {
    const int ch = NT * (dtype == D3D_DTYPE_F32 ? 4 : 8);
    return (int)((V + ch - 1) / ch);
}

static Layout layout(int B, int K, int64_t V) {
    Layout l;
    const size_t C = (size_t)num_chunks(V), R = 2 * (size_t)K + 1;
    const size_t C2 = (size_t)num_subchunks(V, D3D_DTYPE_F32);  // the larger count of the two dtypes
    l.stats = 0;
    l.dec = align256((size_t)B * R * C * sizeof(RowStat));
    l.rstats = l.dec + align256((size_t)B * sizeof(Decision));
    l.xtok = l.rstats + align256((size_t)B * C2 * sizeof(ResStat));
    l.total = l.xtok + align256((size_t)B * R * sizeof(float));
    return l;
}

template <int DT, bool VEC, bool SP>
static hipError_t launch(const Params& P, Mode mode, int B, hipStream_t stream) {
    const dim3 block(NT);
    const dim3 grid_dec(mode == kGreedy ? 1 : (P.C2 + P.nv2 - 1) / P.nv2, B);
    // Target rows 0..K, then (dense proposals) draft rows.
    const dim3 grid_stats(P.C, (mode == kGreedy || SP) ? P.K + 1 : 2 * P.K + 1, B);
    switch (mode) {
        case kGreedy:
            hipLaunchKernelGGL((accept_stats_kernel<DT, VEC, kGreedy>), grid_stats, block, 0, stream, P);
            hipLaunchKernelGGL((accept_decide_kernel<DT, VEC, kGreedy, false>), grid_dec, block, 0, stream, P);
            return hipGetLastError();
        case kLogits:
            hipLaunchKernelGGL((accept_stats_kernel<DT, VEC, kLogits>), grid_stats, block, 0, stream, P);
            hipLaunchKernelGGL((accept_decide_kernel<DT, VEC, kLogits, SP>), grid_dec, block, 0, stream, P);
            hipLaunchKernelGGL((accept_resample_kernel<DT, VEC, kLogits, SP>), dim3(B), block, 0, stream, P);
            return hipGetLastError();
        default:
            hipLaunchKernelGGL((accept_stats_kernel<DT, VEC, kProbs>), grid_stats, block, 0, stream, P);
            hipLaunchKernelGGL((accept_decide_kernel<DT, VEC, kProbs, SP>), grid_dec, block, 0, stream, P);
            hipLaunchKernelGGL((accept_resample_kernel<DT, VEC, kProbs, SP>), dim3(B), block, 0, stream, P);
            return hipGetLastError();
    }
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
    P.K = K;
    P.V = (int)V;
    P.C = num_chunks(V);
    P.nv2 = pick_nv2(B);
    P.C2 = num_subchunks(V, dtype);
    P.stats = reinterpret_cast<RowStat*>(ws + lay.stats);
    P.dec = reinterpret_cast<Decision*>(ws + lay.dec);
    P.rstats = reinterpret_cast<ResStat*>(ws + lay.rstats);
    P.xtok = reinterpret_cast<float*>(ws + lay.xtok);
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
            err = vec ? launch<kF32, true, true>(P, mode, B, s) : launch<kF32, false, true>(P, mode, B, s);
        else
            err = vec ? launch<kF32, true, false>(P, mode, B, s) : launch<kF32, false, false>(P, mode, B, s);
    } else {
        if (sparse)
            err = vec ? launch<kBF16, true, true>(P, mode, B, s) : launch<kBF16, false, true>(P, mode, B, s);
        else
            err = vec ? launch<kBF16, true, false>(P, mode, B, s) : launch<kBF16, false, false>(P, mode, B, s);
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
