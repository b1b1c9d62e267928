// Draft proposal sampling: one token per logits row, with its probability.
//
// Reference behaviour (D3D repository):
//   single/eval_sync.py:287-305  _sampling_probs: T <= 1e-5 is one-hot at
//       the argmax, else softmax(logits / T); top-k keeps the entries at or
//       above the k-th largest scaled logit (ties kept, :293-295); top-p
//       (:296-303) and wide top-k come as the per-row filter of
//       d3d_row_filter (filter.hip)
//   single/eval_sync.py:308-338  _sample_tokens / _sample_with_prob: the
//       argmax (probability 1) or a multinomial draw and its probability
//   single/eval_sync.py:341-367  _sample_with_sparse_probs: top-S support of
//       logits / T, the nucleus (top-p) filter over the sorted support,
//       softmax over the support, a draw from it
//
// torch.multinomial is replaced by the inverse CDF driven by one uniform u
// per row: token = first t with C_t > u * W over the weights, else the last
// t with positive weight (the acceptance kernels' rule).
//
// Dense rows: (1) chunk statistics (max z, sum exp(z - max z)) of every
// 4096-entry chunk, streamed once; (2) one workgroup per row scans the chunk
// masses s_c * exp(m_c - M) in chunk order, finds the chunk where the CDF
// crosses u * W and scans that chunk entry by entry (weights exp(z - m_c),
// the target rescaled to the chunk).  Sparse rows: top-S values and ids come
// from d3d_topk_rows; one wave per row forms softmax(v / T) over the
// support and draws from it.
#include "d3d_common.hpp"
#include "rowstats.hpp"
#include "../../include/d3d_hip.h"

#include <limits.h>

namespace d3d {
namespace sample {

using namespace rows;

constexpr int kMaxSupport = 64;

struct Params {
    const void* logits;  // [N, V]
    int N, V, C;
    float T;
    const float* kth;   // [N] top-k floor (raw logit), or null
    const float* zf;    // [N] filter floor on z = x / T, or null
    const int32_t* zlim;  // [N] ids kept at z == zf[n]: e <= zlim[n]
    const float* u;     // [N]
    RowStat* stats;     // [N][C]
    int64_t* tok;       // [N]
    float* prob;        // [N] (may be null)
    float* probs_out;   // [N, V] dense probabilities (d3d_softmax_rows)
};

// Top-k filter of _sampling_probs (single/eval_sync.py:293-295): entries
// whose scaled logit x / T lies below the row's k-th largest scaled logit
// kth / T become -inf (probability 0).  The division matches the
// reference's logits.float() / T, so ties with the k-th value are kept.
template <bool UNIT_T, int LT>
__device__ __forceinline__ void apply_floor(const Params& P, int n, float (&x)[LT]) {
    if (!P.kth) return;
    const float fl = UNIT_T ? P.kth[n] : P.kth[n] / P.T;
#pragma unroll
    for (int j = 0; j < LT; ++j) {
        const float z = UNIT_T ? x[j] : x[j] / P.T;
        x[j] = z < fl ? -INFINITY : x[j];
    }
}

// Row filter of d3d_row_filter (top-k and top-p of _sampling_probs,
// single/eval_sync.py:292-303): entry e with z = x / T is kept iff
// z > zf[n], or z == zf[n] and e <= zlim[n]; the others become -inf.  x[j*E +
// k] holds entry first + j * stride + k.
template <int DT, bool UNIT_T, int LT>
__device__ __forceinline__ void apply_filter(const Params& P, int n, int first, int stride, float (&x)[LT]) {
    if (!P.zf) return;
    constexpr int E = Vec<DT>::E;
    const float f = P.zf[n];
    const int lim = P.zlim[n];
#pragma unroll
    for (int j = 0; j < LT; ++j) {
        const int e = first + (j / E) * stride + (j % E);
        const float z = UNIT_T ? x[j] : x[j] / P.T;
        x[j] = (z > f || (z == f && e <= lim)) ? x[j] : -INFINITY;
    }
}

template <int DT, bool VEC, Mode M, bool UNIT_T>
__global__ __launch_bounds__(NT) void sample_stats_kernel(Params P) {
    constexpr int E = Vec<DT>::E;
    const int c = blockIdx.x, n = blockIdx.y;
    __shared__ float rf[NT / kWave];
    __shared__ int ri[NT / kWave];
    const void* row = row_ptr<DT>(P.logits, n, P.V);
    const int first = c * kChunk + threadIdx.x * E;
    float x[L];
    load_tile<DT, VEC, true, L>(row, P.V, first, NT * E, -INFINITY, x);
    if constexpr (M != kGreedy) {
        apply_floor<UNIT_T>(P, n, x);
        apply_filter<DT, UNIT_T>(P, n, first, NT * E, x);
    }
    const RowStat st = chunk_stats<DT, M, UNIT_T>(x, first, P.T, M == kGreedy, rf, ri);
    if (threadIdx.x == 0) P.stats[(size_t)n * P.C + c] = st;
}

template <int DT, bool VEC, Mode M, bool UNIT_T>
__global__ __launch_bounds__(NT) void sample_pick_kernel(Params P) {
    constexpr int E = Vec<DT>::E;
    const int n = blockIdx.x, tid = threadIdx.x;
    const int C = P.C;
    __shared__ RowStat lds[kMaxStatLds];
    __shared__ float s_wave[NT / kWave];
    __shared__ float rf[NT / kWave];
    __shared__ int ri[NT / kWave];
    __shared__ float s_f[2];
    const RowStat* src = P.stats + (size_t)n * C;
    for (int c = tid; c < C; c += NT) lds[c] = src[c];
    __syncthreads();
    const void* row = row_ptr<DT>(P.logits, n, P.V);

    if constexpr (M == kGreedy) {
        float bv = -INFINITY;
        int bi = INT_MAX;
        for (int c = tid; c < C; c += NT) argmax_merge(bv, bi, lds[c].xmax, lds[c].arg);
        block_argmax<NT>(bv, bi, rf, ri);
        if (tid == 0) {
            P.tok[n] = bi;
            if (P.prob) P.prob[n] = 1.0f;
        }
        return;
    } else {
        float mx = -INFINITY;
        for (int c = tid; c < C; c += NT) mx = fmaxf(mx, lds[c].m);
        const float Mrow = block_max<NT>(mx, rf);
        auto mass = [&](int c) {
            const RowStat t = lds[c];
            return t.m == -INFINITY ? 0.f : t.s * expf(t.m - Mrow);
        };
        // Pass 1: total mass W in chunk order; the last chunk with mass.
        float carry = 0.f;
        int last_c = -1;
        for (int c0 = 0; c0 < C; c0 += NT) {
            const float w = c0 + tid < C ? mass(c0 + tid) : 0.f;
            if (w > 0.f) last_c = c0 + tid;
            const float incl = block_incl_scan(w, s_wave);
            if (tid == NT - 1) s_f[0] = incl;
            __syncthreads();
            carry += s_f[0];
            __syncthreads();
        }
        last_c = block_max_int(last_c, ri);
        const float W = carry;
        const float target = P.u[n] * W;
        // Pass 2: the first chunk whose inclusive mass exceeds u * W.
        int cs = INT_MAX;
        float base = 0.f;
        carry = 0.f;
        for (int c0 = 0; c0 < C && cs == INT_MAX; c0 += NT) {
            const float w = c0 + tid < C ? mass(c0 + tid) : 0.f;
            const float incl = carry + block_incl_scan(w, s_wave);
            const int mine = (c0 + tid < C && incl > target) ? c0 + tid : INT_MAX;
            const int first = block_min_int(mine, ri);
            if (first != INT_MAX && first == c0 + tid) s_f[0] = incl - w;
            if (tid == NT - 1) s_f[1] = incl;
            __syncthreads();
            if (first != INT_MAX) {
                cs = first;
                base = s_f[0];
            }
            carry = s_f[1];
            __syncthreads();
        }
        const bool crossed = cs != INT_MAX;
        const int c = crossed ? cs : last_c;
        int token = -1;
        if (c >= 0) {
            // Entries of chunk c in index order: vector j of every thread.
            const RowStat st = lds[c];
            const float scale = expf(st.m - Mrow);
            const float tl = crossed ? (target - base) / scale : INFINITY;
            const int first = c * kChunk + tid * E;
            float x[L];
            load_tile<DT, VEC, false, L>(row, P.V, first, NT * E, -INFINITY, x);
            apply_floor<UNIT_T>(P, n, x);
            apply_filter<DT, UNIT_T>(P, n, first, NT * E, x);
            float run = 0.f;
            int found = INT_MAX, lastpos = -1;
#pragma unroll
            for (int j = 0; j < L / E; ++j) {
                float w[E], ts = 0.f;
#pragma unroll
                for (int k = 0; k < E; ++k) {
                    const float z = UNIT_T ? x[j * E + k] : x[j * E + k] / P.T;
                    w[k] = st.m == -INFINITY ? 0.f : expf(z - st.m);
                    ts += w[k];
                }
                const float incl = block_incl_scan(ts, s_wave);
                float r = run + (incl - ts);
#pragma unroll
                for (int k = 0; k < E; ++k) {
                    r += w[k];
                    if (w[k] > 0.f) {
                        const int e = first + j * NT * E + k;
                        lastpos = e;
                        if (found == INT_MAX && r > tl) found = e;
                    }
                }
                if (tid == NT - 1) s_f[0] = incl;
                __syncthreads();
                run += s_f[0];
                __syncthreads();
            }
            found = block_min_int(found, ri);
            lastpos = block_max_int(lastpos, ri);
            token = found != INT_MAX ? found : lastpos;
        }
        if (tid == 0) {
            P.tok[n] = token < 0 ? (int64_t)D3D_TOKEN_EMPTY_DISTRIBUTION : token;
            if (P.prob) {
                float p = 0.f;
                if (token >= 0) {
                    const float z = UNIT_T ? load_one<DT>(row, token) : load_one<DT>(row, token) / P.T;
                    p = expf(z - Mrow) / W;
                }
                P.prob[n] = p;
            }
        }
    }
}

// Sparse support: vals/ids [N][S] (top-S logits in descending order), one
// wave per row: probs = softmax(vals / T) over the support, then the draw.
__device__ __forceinline__ float wave_incl_scan(float v, int lane) {
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const float t = __shfl_up(v, o, kWave);
        if (lane >= o) v += t;
    }
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

__global__ __launch_bounds__(NT) void support_sample_kernel(const float* __restrict__ vals,
                                                            const int64_t* __restrict__ ids, int N, int S, float T,
                                                            float top_p, const float* __restrict__ u, int64_t* tok,
                                                            float* probs, float* tok_prob) {
    const int lane = threadIdx.x & (kWave - 1);
    const int n = blockIdx.x * (NT / kWave) + threadIdx.x / kWave;
    if (n >= N) return;
    const bool live = lane < S;
    const float z = live ? vals[(size_t)n * S + lane] / T : -INFINITY;
    float m = z;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, kWave));
    float e = (live && z != -INFINITY) ? expf(z - m) : 0.f;
    float Z = wave_sum(e);
    float p = Z > 0.f ? e / Z : 0.f;
    if (top_p < 1.0f) {
        // Nucleus filter over the descending support (:356-361): entry s > 0
        // goes when the inclusive mass of entries 0..s-1 exceeds top_p; the
        // kept logits are renormalised (dropped ones become exactly 0).
        const float incl = wave_incl_scan(p, lane);
        const float before = __shfl_up(incl, 1, kWave);
        const bool drop = lane > 0 && before > top_p;
        e = drop ? 0.f : e;
        Z = wave_sum(e);
        p = Z > 0.f ? e / Z : 0.f;
    }
    if (live) probs[(size_t)n * S + lane] = p;
    // Inclusive scan of p in support order, total W.
    const float c = wave_incl_scan(p, lane);
    const float W = __shfl(c, kWave - 1, kWave);
    const float target = u[n] * W;
    const uint64_t hit = __ballot(live && c > target && p > 0.f);
    const uint64_t pos = __ballot(live && p > 0.f);
    int pick = -1;
    if (hit) pick = __builtin_ctzll(hit);
    else if (pos) pick = 63 - __builtin_clzll(pos);
    const float pp = __shfl(p, pick >= 0 ? pick : 0, kWave);  // every lane takes part
    if (lane == 0) {
        tok[n] = pick >= 0 ? ids[(size_t)n * S + pick] : (int64_t)D3D_TOKEN_EMPTY_DISTRIBUTION;
        if (tok_prob) tok_prob[n] = pick >= 0 ? pp : 0.f;
    }
}

template <int DT, bool VEC, Mode M, bool UNIT_T>
static void launch(const Params& P, hipStream_t s) {
    hipLaunchKernelGGL((sample_stats_kernel<DT, VEC, M, UNIT_T>), dim3(P.C, P.N), dim3(NT), 0, s, P);
    hipLaunchKernelGGL((sample_pick_kernel<DT, VEC, M, UNIT_T>), dim3(P.N), dim3(NT), 0, s, P);
}

template <int DT, bool VEC>
static void dispatch(const Params& P, bool greedy, hipStream_t s) {
    if (greedy)
        launch<DT, VEC, kGreedy, true>(P, s);
    else if (P.T == 1.0f)
        launch<DT, VEC, kLogits, true>(P, s);
    else
        launch<DT, VEC, kLogits, false>(P, s);
}

// Dense probabilities: workgroup (chunk, row) merges the row's chunk
// records in chunk order (every workgroup of the row gets the same M and W)
// and writes p = exp(z - M) / W for its chunk, 0 for entries below the
// top-k floor; greedy rows get the one-hot row at the argmax.
template <int DT, bool VEC, Mode M, bool UNIT_T>
__global__ __launch_bounds__(NT) void softmax_write_kernel(Params P) {
    constexpr int E = Vec<DT>::E;
    const int c = blockIdx.x, n = blockIdx.y, tid = threadIdx.x;
    __shared__ float s_row[2];
    __shared__ int s_arg;
    const RowStat* src = P.stats + (size_t)n * P.C;
    if (tid == 0) {
        if constexpr (M == kGreedy) {
            float bv = -INFINITY;
            int bi = INT_MAX;
            for (int i = 0; i < P.C; ++i) argmax_merge(bv, bi, src[i].xmax, src[i].arg);
            s_arg = bi;
        } else {
            float mx = -INFINITY;
            for (int i = 0; i < P.C; ++i) mx = fmaxf(mx, src[i].m);
            float w = 0.f;
            for (int i = 0; i < P.C; ++i) w += src[i].m == -INFINITY ? 0.f : src[i].s * expf(src[i].m - mx);
            s_row[0] = mx;
            s_row[1] = w > 0.f ? 1.0f / w : 0.f;
        }
    }
    __syncthreads();
    float* out = P.probs_out + (size_t)n * P.V;
    const int first = c * kChunk + tid * E;
    if constexpr (M == kGreedy) {
        const int arg = s_arg;
#pragma unroll
        for (int j = 0; j < L / E; ++j)
#pragma unroll
            for (int k = 0; k < E; ++k) {
                const int e = first + j * NT * E + k;
                if (e < P.V) out[e] = e == arg ? 1.0f : 0.0f;
            }
    } else {
        const void* row = row_ptr<DT>(P.logits, n, P.V);
        float x[L];
        load_tile<DT, VEC, true, L>(row, P.V, first, NT * E, -INFINITY, x);
        apply_floor<UNIT_T>(P, n, x);
        apply_filter<DT, UNIT_T>(P, n, first, NT * E, x);
        const float Mrow = s_row[0], inv = s_row[1];
#pragma unroll
        for (int j = 0; j < L / E; ++j)
#pragma unroll
            for (int k = 0; k < E; ++k) {
                const int e = first + j * NT * E + k;
                const float z = UNIT_T ? x[j * E + k] : x[j * E + k] / P.T;
                if (e < P.V) out[e] = z == -INFINITY ? 0.f : expf(z - Mrow) * inv;
            }
    }
}

template <int DT, bool VEC, Mode M, bool UNIT_T>
static void launch_probs(const Params& P, hipStream_t s) {
    hipLaunchKernelGGL((sample_stats_kernel<DT, VEC, M, UNIT_T>), dim3(P.C, P.N), dim3(NT), 0, s, P);
    hipLaunchKernelGGL((softmax_write_kernel<DT, VEC, M, UNIT_T>), dim3(P.C, P.N), dim3(NT), 0, s, P);
}

template <int DT, bool VEC>
static void dispatch_probs(const Params& P, bool greedy, hipStream_t s) {
    if (greedy)
        launch_probs<DT, VEC, kGreedy, true>(P, s);
    else if (P.T == 1.0f)
        launch_probs<DT, VEC, kLogits, true>(P, s);
    else
        launch_probs<DT, VEC, kLogits, false>(P, s);
}

}  // namespace sample
}  // namespace d3d

using namespace d3d;

extern "C" size_t d3d_sample_workspace_bytes(int N, int64_t V) {
    if (N < 1 || V < 1) return 0;
    const size_t C = (size_t)((V + rows::kChunk - 1) / rows::kChunk);
    return ((size_t)N * C * sizeof(rows::RowStat) + 255) & ~(size_t)255;
}

extern "C" int d3d_sample_rows(const void* logits, int dtype, int N, int64_t V, float temperature,
                               const float* kth, const float* zfloor, const int32_t* zlimit, const float* uniforms,
                               int64_t* tokens_out, float* probs_out, void* workspace, size_t workspace_bytes,
                               void* stream) {
    using namespace sample;
    if (N < 0 || N > 65535 || V < 1 || V > (int64_t)rows::kMaxStatLds * rows::kChunk) return D3D_E_SHAPE;
    if (dtype != D3D_DTYPE_F32 && dtype != D3D_DTYPE_BF16) return D3D_E_DTYPE;
    if (N == 0) return D3D_OK;
    const bool greedy = !(temperature > 1e-5f);
    if (!logits || !tokens_out || !workspace || (!greedy && !uniforms)) return D3D_E_NULL;
    if (workspace_bytes < d3d_sample_workspace_bytes(N, V)) return D3D_E_WORKSPACE;
    Params P;
    P.logits = logits;
    P.N = N;
    P.V = (int)V;
    P.C = (int)((V + rows::kChunk - 1) / rows::kChunk);
    P.T = greedy ? 1.0f : temperature;
    P.kth = greedy ? nullptr : kth;
    if (!greedy && (zfloor == nullptr) != (zlimit == nullptr)) return D3D_E_NULL;
    P.zf = greedy ? nullptr : zfloor;
    P.zlim = greedy ? nullptr : zlimit;
    P.u = uniforms;
    P.stats = static_cast<rows::RowStat*>(workspace);
    P.tok = tokens_out;
    P.prob = probs_out;
    const size_t esize = dtype == D3D_DTYPE_F32 ? 4 : 2;
    const bool vec = ((uintptr_t)logits % 16 == 0) && ((size_t)V * esize) % 16 == 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == D3D_DTYPE_F32) {
        if (vec) dispatch<kF32, true>(P, greedy, s);
        else dispatch<kF32, false>(P, greedy, s);
    } else {
        if (vec) dispatch<kBF16, true>(P, greedy, s);
        else dispatch<kBF16, false>(P, greedy, s);
    }
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? D3D_OK : (int)err;
}

extern "C" int d3d_softmax_rows(const void* logits, int dtype, int N, int64_t V, float temperature,
                                const float* kth, const float* zfloor, const int32_t* zlimit, float* probs_out,
                                void* workspace, size_t workspace_bytes, void* stream) {
    using namespace sample;
    if (N < 0 || N > 65535 || V < 1 || V > (int64_t)rows::kMaxStatLds * rows::kChunk) return D3D_E_SHAPE;
    if (dtype != D3D_DTYPE_F32 && dtype != D3D_DTYPE_BF16) return D3D_E_DTYPE;
    if (N == 0) return D3D_OK;
    if (!logits || !probs_out || !workspace) return D3D_E_NULL;
    if (workspace_bytes < d3d_sample_workspace_bytes(N, V)) return D3D_E_WORKSPACE;
    const bool greedy = !(temperature > 1e-5f);
    Params P;
    P.logits = logits;
    P.N = N;
    P.V = (int)V;
    P.C = (int)((V + rows::kChunk - 1) / rows::kChunk);
    P.T = greedy ? 1.0f : temperature;
    P.kth = greedy ? nullptr : kth;
    if (!greedy && (zfloor == nullptr) != (zlimit == nullptr)) return D3D_E_NULL;
    P.zf = greedy ? nullptr : zfloor;
    P.zlim = greedy ? nullptr : zlimit;
    P.u = nullptr;
    P.stats = static_cast<rows::RowStat*>(workspace);
    P.tok = nullptr;
    P.prob = nullptr;
    P.probs_out = probs_out;
    const size_t esize = dtype == D3D_DTYPE_F32 ? 4 : 2;
    const bool vec = ((uintptr_t)logits % 16 == 0) && ((size_t)V * esize) % 16 == 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == D3D_DTYPE_F32) {
        if (vec) dispatch_probs<kF32, true>(P, greedy, s);
        else dispatch_probs<kF32, false>(P, greedy, s);
    } else {
        if (vec) dispatch_probs<kBF16, true>(P, greedy, s);
        else dispatch_probs<kBF16, false>(P, greedy, s);
    }
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? D3D_OK : (int)err;
}

extern "C" int d3d_sample_support(const float* support_vals, const int64_t* support_ids, int N, int S,
                                  float temperature, float top_p, const float* uniforms, int64_t* tokens_out,
                                  float* support_probs_out, float* token_probs_out, void* stream) {
    using namespace sample;
    if (N < 0 || S < 1 || S > kMaxSupport) return D3D_E_SHAPE;
    if (!(temperature > 1e-5f)) return D3D_E_UNSUPPORTED;
    if (!(top_p > 0.f && top_p <= 1.f)) return D3D_E_VALUE;
    if (N == 0) return D3D_OK;
    if (!support_vals || !support_ids || !uniforms || !tokens_out || !support_probs_out) return D3D_E_NULL;
    const int per = rows::NT / kWave;
    hipLaunchKernelGGL(support_sample_kernel, dim3((N + per - 1) / per), dim3(rows::NT), 0,
                       static_cast<hipStream_t>(stream), support_vals, support_ids, N, S, temperature, top_p,
                       uniforms, tokens_out, support_probs_out, token_probs_out);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? D3D_OK : (int)err;
}
