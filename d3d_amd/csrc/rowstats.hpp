// Row statistics over a large vocabulary, shared by the acceptance and the
// confidence/top-k kernels: 16-byte tile loads of fp32 or bf16 rows, per
// chunk (max z, sum exp(z - max z), max x, argmax) reductions, and a
// fixed-order merge of chunk records into row statistics.
#pragma once

#include "d3d_common.hpp"

#include <limits.h>

namespace d3d {
namespace rows {

constexpr int NT = 256;            // threads per workgroup (4 waves)
constexpr int kChunk = 4096;       // vocabulary entries per chunk
constexpr int L = kChunk / NT;     // entries per thread per chunk
constexpr int kMaxStatLds = 2048;  // RowStat entries staged in LDS per batch (32 KiB)

struct __attribute__((aligned(16))) RowStat {
    float m;     // max of z over the chunk (logits), 0 (probs)
    float s;     // sum exp(z - m) (logits) or sum x (probs)
    float xmax;  // max raw value
    int arg;     // first index of xmax
};

enum Mode : int { kGreedy = 0, kLogits = 1, kProbs = 2 };

template <int DT>
struct Vec;
template <>
struct Vec<kF32> {
    static constexpr int E = 4;
    static constexpr size_t bytes = 4;
};
template <>
struct Vec<kBF16> {
    static constexpr int E = 8;
    static constexpr size_t bytes = 2;
};

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int DT>
__device__ __forceinline__ const void* row_ptr(const void* base, size_t row, int V) {
    return static_cast<const char*>(base) + row * (size_t)V * Vec<DT>::bytes;
}

template <int DT>
__device__ __forceinline__ float load_one(const void* row, int e) {
    if constexpr (DT == kF32) {
        return static_cast<const float*>(row)[e];
    } else {
        return bf16_bits_to_f32(static_cast<const uint16_t*>(row)[e]);
    }
}

// Loads L entries of one row into x[]: x[j*E + k] holds entry
// first + j*stride + k.  Entries at or beyond V read as FILL (-inf for logits,
// 0 for probabilities), which leaves every reduction unchanged, so the
// arithmetic loops carry no bounds checks.  STREAM marks a single-use read
// (non-temporal hint).
template <int DT, bool VEC, bool STREAM, int LT>
__device__ __forceinline__ void load_tile(const void* row, int V, int first, int stride, float fill,
                                          float (&x)[LT]) {
    constexpr int E = Vec<DT>::E;
#pragma unroll
    for (int j = 0; j < LT / E; ++j) {
        const int e0 = first + j * stride;
        if (VEC && e0 + E <= V) {
            if constexpr (DT == kF32) {
                const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(row) + e0);
                const f32x4 v = STREAM ? __builtin_nontemporal_load(p) : *p;
                x[j * E + 0] = v.x;
                x[j * E + 1] = v.y;
                x[j * E + 2] = v.z;
                x[j * E + 3] = v.w;
            } else {
                const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(row) + e0);
                const u32x4 v = STREAM ? __builtin_nontemporal_load(p) : *p;
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    x[j * E + 2 * h] = bf16_bits_to_f32(w[h] & 0xffffu);
                    x[j * E + 2 * h + 1] = bf16_bits_to_f32(w[h] >> 16);
                }
            }
        } else {
#pragma unroll
            for (int k = 0; k < E; ++k) {
                const int e = e0 + k;
                x[j * E + k] = e < V ? load_one<DT>(row, e) : fill;
            }
        }
    }
}

// As load_tile, for the first nv (runtime, <= LT/E) vectors only.
template <int DT, bool VEC, int LT>
__device__ __forceinline__ void load_tile_n(const void* row, int V, int first, int stride, int nv, float fill,
                                            float (&x)[LT]) {
    constexpr int E = Vec<DT>::E;
#pragma unroll
    for (int j = 0; j < LT / E; ++j) {
        if (j >= nv) break;
        const int e0 = first + j * stride;
        if (VEC && e0 + E <= V) {
            if constexpr (DT == kF32) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(static_cast<const float*>(row) + e0);
                x[j * E + 0] = v.x;
                x[j * E + 1] = v.y;
                x[j * E + 2] = v.z;
                x[j * E + 3] = v.w;
            } else {
                const u32x4 v = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(row) + e0);
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    x[j * E + 2 * h] = bf16_bits_to_f32(w[h] & 0xffffu);
                    x[j * E + 2 * h + 1] = bf16_bits_to_f32(w[h] >> 16);
                }
            }
        } else {
#pragma unroll
            for (int k = 0; k < E; ++k) {
                const int e = e0 + k;
                x[j * E + k] = e < V ? load_one<DT>(row, e) : fill;
            }
        }
    }
}

template <int DT>
__device__ __forceinline__ int tile_index(int first, int stride, int l) {
    constexpr int E = Vec<DT>::E;
    return first + (l / E) * stride + (l % E);
}

template <Mode M>
__device__ __forceinline__ constexpr float fill_value() {
    return M == kProbs ? 0.f : -INFINITY;
}

// Probability of one entry given its row statistics: softmax(x / T) entry
// exp(x / T - M) / S for logits, x / max(S, 1e-12) for probabilities.
// inv_s is 1 / S (logits) or 1 / max(S, 1e-12) (probabilities).
template <Mode M, bool UNIT_T>
__device__ __forceinline__ float prob_of(float x, float rowM, float inv_s, float T) {
    if constexpr (M == kProbs) {
        return x * inv_s;
    } else {
        return expf((UNIT_T ? x : x / T) - rowM) * inv_s;
    }
}

template <Mode M>
__device__ __forceinline__ float inv_sum(float S) {
    return M == kProbs ? 1.0f / fmaxf(S, 1e-12f) : 1.0f / S;
}

__device__ __forceinline__ int wave_max_int(int v) {
    v = max(v, xor_desc<32>(v));
    v = max(v, xor_desc<16>(v));
    v = max(v, xor_desc<8>(v));
    v = max(v, xor_desc<4>(v));
    v = max(v, xor_desc<2>(v));
    return max(v, xor_desc<1>(v));
}

__device__ __forceinline__ int wave_min_int(int v) {
    v = min(v, xor_desc<32>(v));
    v = min(v, xor_desc<16>(v));
    v = min(v, xor_desc<8>(v));
    v = min(v, xor_desc<4>(v));
    v = min(v, xor_desc<2>(v));
    return min(v, xor_desc<1>(v));
}

// One ascending step (lane groups of 2 * O) of the row merge: max, argmax.
template <int O>
__device__ __forceinline__ void merge_step_asc(float& m, float& xm, int& am) {
    m = fmaxf(m, xor_asc<O>(m));
    const float x2 = xor_asc<O>(xm);
    const int a2 = xor_asc<O>(am);
    argmax_merge(xm, am, x2, a2);
}

__device__ __forceinline__ int block_max_int(int v, int* scratch) {
    v = wave_max_int(v);
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0) scratch[threadIdx.x / kWave] = v;
    __syncthreads();
    int r = scratch[0];
#pragma unroll
    for (int k = 1; k < NT / kWave; ++k) r = max(r, scratch[k]);
    return r;
}

__device__ __forceinline__ int block_min_int(int v, int* scratch) {
    v = wave_min_int(v);
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0) scratch[threadIdx.x / kWave] = v;
    __syncthreads();
    int r = scratch[0];
#pragma unroll
    for (int k = 1; k < NT / kWave; ++k) r = min(r, scratch[k]);
    return r;
}

template <int DT, Mode M, bool UNIT_T>
__device__ __forceinline__ RowStat chunk_stats(const float (&x)[L], int first, float T, bool want_arg,
                                               float* rf, int* ri) {
    constexpr int E = Vec<DT>::E;
    float bv = x[0];
    int bi = first;
    if (want_arg) {
        // Entries are visited in increasing index order, so ">" keeps the first max.
#pragma unroll
        for (int l = 1; l < L; ++l) {
            if (x[l] > bv) {
                bv = x[l];
                bi = tile_index<DT>(first, NT * E, l);
            }
        }
        block_argmax<NT>(bv, bi, rf, ri);
    } else {
#pragma unroll
        for (int l = 1; l < L; ++l) bv = fmaxf(bv, x[l]);
        bv = block_max<NT>(bv, rf);
        bi = INT_MAX;
    }
    RowStat st;
    st.xmax = bv;
    st.arg = bi;
    st.m = 0.f;
    st.s = 0.f;
    if constexpr (M == kProbs) {
        float s = 0.f;
#pragma unroll
        for (int l = 0; l < L; ++l) s += x[l];
        st.s = block_sum<NT>(s, rf);
    } else if constexpr (M == kLogits) {
        // max z equals (max x) / T: division by T > 0 is monotone.
        const float m = UNIT_T ? bv : bv / T;
        float s = 0.f;
        if (m != -INFINITY) {
#pragma unroll
            for (int l = 0; l < L; ++l) s += expf((UNIT_T ? x[l] : x[l] / T) - m);
        }
        st.m = m;
        st.s = block_sum<NT>(s, rf);
    }
    return st;
}

constexpr int kLanesPerRow = 8;
constexpr int kRowsPerPass = NT / kLanesPerRow;

// Merges a [rows][C] array of chunk records (global) into per-row statistics
// in LDS: sM/sS for every row, sArg for rows < arg_rows.  Records are
// staged in LDS; 8 lanes per row then take every 8th chunk: first the row
// max (and argmax) by a fold and a 3-step butterfly, then
// sum_c s_c * exp(m_c - M) with independent exponentials, folded and
// butterflied the same way.  Every caller gets the same bits for the same
// records.
template <Mode M>
__device__ __forceinline__ void merge_row_stats(const RowStat* stats, int rows, int C, int arg_rows, float* sM,
                                                float* sS, int* sArg, RowStat* lds) {
    const int g = threadIdx.x % kLanesPerRow;
    // Up to kRowsPerPass rows of up to kLanesPerRow * kDirect records: each
    // lane loads its records straight into registers (all at once, from
    // clamped addresses) instead of staging them in LDS, and folds them in
    // the same order as the staged path below, so the results are the same
    // bits.
    constexpr int kDirect = 8;
    if (rows <= kRowsPerPass && C <= kLanesPerRow * kDirect) {
        const int rr = threadIdx.x / kLanesPerRow;
        const bool live = rr < rows;
        const int last = rows * C - 1;
        RowStat t[kDirect];
#pragma unroll
        for (int j = 0; j < kDirect; ++j)
            t[j] = stats[min(rr * C + g + j * kLanesPerRow, last)];
        float m = -INFINITY, xm = -INFINITY;
        int am = INT_MAX;
#pragma unroll
        for (int j = 0; j < kDirect; ++j) {
            if (live && g + j * kLanesPerRow < C) {
                m = fmaxf(m, t[j].m);
                argmax_merge(xm, am, t[j].xmax, t[j].arg);
            }
        }
        static_assert(kLanesPerRow == 8, "three ascending merge steps");
        merge_step_asc<1>(m, xm, am);
        merge_step_asc<2>(m, xm, am);
        merge_step_asc<4>(m, xm, am);
        float sum = 0.f;
        if (M != kGreedy) {
#pragma unroll
            for (int j = 0; j < kDirect; ++j) {
                if (live && g + j * kLanesPerRow < C) {
                    if constexpr (M == kProbs) {
                        sum += t[j].s;
                    } else {
                        if (t[j].m != -INFINITY) sum += t[j].s * expf(t[j].m - m);
                    }
                }
            }
        }
        sum += xor_asc<1>(sum);
        sum += xor_asc<2>(sum);
        sum += xor_asc<4>(sum);
        __syncthreads();  // earlier readers of sM / sS / sArg are done
        if (live && g == 0) {
            sM[rr] = m;
            sS[rr] = sum;
            if (rr < arg_rows) sArg[rr] = am;
        }
        __syncthreads();
        return;
    }
    const int batch_rows = min(rows, kMaxStatLds / C);  // >= 1: C <= kMaxStatLds
    for (int r0 = 0; r0 < rows; r0 += batch_rows) {
        const int nr = min(batch_rows, rows - r0);
        const RowStat* src = stats + (size_t)r0 * C;
        __syncthreads();
        // Up to kStage 16-byte records per thread in flight at once (loads
        // past the end re-read the last record and are not stored).
        constexpr int kStage = 8;
        const int n = nr * C;
        const u32x4* s4 = reinterpret_cast<const u32x4*>(src);
        u32x4* l4 = reinterpret_cast<u32x4*>(lds);
        for (int e0 = 0; e0 < n; e0 += NT * kStage) {
            u32x4 t[kStage];
#pragma unroll
            for (int j = 0; j < kStage; ++j) t[j] = s4[min(e0 + j * NT + (int)threadIdx.x, n - 1)];
#pragma unroll
            for (int j = 0; j < kStage; ++j) {
                const int e = e0 + j * NT + threadIdx.x;
                if (e < n) l4[e] = t[j];
            }
        }
        __syncthreads();
        for (int rr0 = 0; rr0 < nr; rr0 += kRowsPerPass) {
            const int rr = rr0 + threadIdx.x / kLanesPerRow;
            const bool live = rr < nr;
            float m = -INFINITY, xm = -INFINITY;
            int am = INT_MAX;
            if (live) {
#pragma unroll 4
                for (int k = g; k < C; k += kLanesPerRow) {
                    const RowStat t = lds[rr * C + k];
                    m = fmaxf(m, t.m);
                    argmax_merge(xm, am, t.xmax, t.arg);
                }
            }
            static_assert(kLanesPerRow == 8, "three ascending merge steps");
            merge_step_asc<1>(m, xm, am);
            merge_step_asc<2>(m, xm, am);
            merge_step_asc<4>(m, xm, am);
            float s = 0.f;
            if (live && M != kGreedy) {
#pragma unroll 4
                for (int k = g; k < C; k += kLanesPerRow) {
                    const RowStat t = lds[rr * C + k];
                    if constexpr (M == kProbs) {
                        s += t.s;
                    } else {
                        if (t.m != -INFINITY) s += t.s * expf(t.m - m);
                    }
                }
            }
            s += xor_asc<1>(s);
            s += xor_asc<2>(s);
            s += xor_asc<4>(s);
            if (live && g == 0) {
                sM[r0 + rr] = m;
                sS[r0 + rr] = s;
                if (r0 + rr < arg_rows) sArg[r0 + rr] = am;
            }
        }
    }
    __syncthreads();
}

// Inclusive scan over the workgroup in thread order (fixed order).
__device__ __forceinline__ float block_incl_scan(float v, float* s_wave) {
    const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
    v = wave_incl_scan(v, lane);
    __syncthreads();
    if (lane == kWave - 1) s_wave[wv] = v;
    __syncthreads();
    float off = 0.f;
    for (int k = 0; k < wv; ++k) off += s_wave[k];
    return v + off;
}

}  // namespace rows
}  // namespace d3d
