// Shared device helpers for the gfx950 kernels of libd3d_hip.
//
// Everything here is wave64-specific: reductions are butterflies over the 64
// lanes of a wavefront followed by a fixed-order combine of the per-wave
// partials in LDS, so every reduction has one summation order for a given
// launch shape and results are reproducible run to run.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace d3d {

constexpr int kWave = 64;

enum Dtype : int { kF32 = 0, kBF16 = 1 };

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (finite inputs; NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Butterfly partners on the VALU (gfx950), without an LDS permute: the value
// __shfl_xor(v, D) would return, for a full, convergent wave, under the
// stated precondition on earlier steps.
//   D = 32, 16  v_permlane32_swap / v_permlane16_swap: swap(v, v) returns
//               halves {lo, lo} / {hi, hi} (rows {0,0,2,2} / {1,1,3,3});
//               the partner is the one of the pair that is not this lane's.
//   D = 8       DPP row_ror:8 (lane i <- i + 8 mod 16).
//   D = 2, 1    DPP quad_perm [2,3,0,1] / [1,0,3,2].
//   Descending order (32, 16, 8, 4, 2, 1), D = 4: row_ror:4, exact because
//               the 8-step left lanes 8 apart equal.
//   Ascending order (1, 2, 4, 8, ...), D = 4: row_half_mirror (lane j <-
//               7 - j in each 8-lane half), exact because quads are uniform;
//               D = 8: row_mirror (j <- 15 - j), exact because 8-lane halves
//               are uniform.
template <int D>
__device__ __forceinline__ uint32_t lane_swap32(uint32_t v) {
    if constexpr (D == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (threadIdx.x & 32) ? r[0] : r[1];
    } else {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (threadIdx.x & 16) ? r[0] : r[1];
    }
}

template <int D>
__device__ __forceinline__ uint32_t xor_partner_desc(uint32_t v) {
    if constexpr (D >= 16) return lane_swap32<D>(v);
    else if constexpr (D == 8) return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x128, 0xf, 0xf, false);
    else if constexpr (D == 4) return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x124, 0xf, 0xf, false);
    else if constexpr (D == 2) return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4e, 0xf, 0xf, false);
    else return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xb1, 0xf, 0xf, false);
}

template <int D>
__device__ __forceinline__ uint32_t xor_partner_asc(uint32_t v) {
    if constexpr (D >= 16) return lane_swap32<D>(v);
    else if constexpr (D == 8) return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x140, 0xf, 0xf, false);
    else if constexpr (D == 4) return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x141, 0xf, 0xf, false);
    else if constexpr (D == 2) return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4e, 0xf, 0xf, false);
    else return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xb1, 0xf, 0xf, false);
}

// The value __shfl_up(v, O) returns to lanes l >= O (lane l - O), on the
// VALU: DPP wave_shr:1 (lane l <- l - 1 across rows) applied O times for
// O <= 8; for 16, rows 1 and 3 take rows 0 and 2 from v_permlane16_swap and
// row 2 takes row 1 from v_permlane32_swap of that swap's other half; for
// 32, v_permlane32_swap.  Lanes below O get unspecified values.
template <int O>
__device__ __forceinline__ uint32_t up_partner(uint32_t v) {
    if constexpr (O <= 8) {
#pragma unroll
        for (int k = 0; k < O; ++k) v = (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x138, 0xf, 0xf, false);
        return v;
    } else if constexpr (O == 16) {
        const auto r16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);  // {0,0,2,2}, {1,1,3,3}
        const auto r32 = __builtin_amdgcn_permlane32_swap(r16[1], r16[1], false, false);  // {1,1,1,1}, ...
        return ((threadIdx.x & 63) >> 4) == 2 ? r32[0] : r16[0];
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return r[0];
    }
}

template <int O>
__device__ __forceinline__ float up_f(float v) {
    return __uint_as_float(up_partner<O>(__float_as_uint(v)));
}

// Inclusive wave scan in the Hillis-Steele order (distances 1, 2, ..., 32),
// bit-identical to the __shfl_up loop.
__device__ __forceinline__ float wave_incl_scan(float v, int lane) {
    float t;
    t = up_f<1>(v);
    if (lane >= 1) v += t;
    t = up_f<2>(v);
    if (lane >= 2) v += t;
    t = up_f<4>(v);
    if (lane >= 4) v += t;
    t = up_f<8>(v);
    if (lane >= 8) v += t;
    t = up_f<16>(v);
    if (lane >= 16) v += t;
    t = up_f<32>(v);
    if (lane >= 32) v += t;
    return v;
}

template <int D>
__device__ __forceinline__ float xor_desc(float v) {
    return __uint_as_float(xor_partner_desc<D>(__float_as_uint(v)));
}
template <int D>
__device__ __forceinline__ int xor_desc(int v) {
    return (int)xor_partner_desc<D>((uint32_t)v);
}
template <int D>
__device__ __forceinline__ float xor_asc(float v) {
    return __uint_as_float(xor_partner_asc<D>(__float_as_uint(v)));
}
template <int D>
__device__ __forceinline__ int xor_asc(int v) {
    return (int)xor_partner_asc<D>((uint32_t)v);
}

// Full-wave reductions: the descending butterfly 32, 16, ..., 1 on the
// VALU, bit-identical to the __shfl_xor loop with the same operation order.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, xor_desc<32>(v));
    v = fmaxf(v, xor_desc<16>(v));
    v = fmaxf(v, xor_desc<8>(v));
    v = fmaxf(v, xor_desc<4>(v));
    v = fmaxf(v, xor_desc<2>(v));
    return fmaxf(v, xor_desc<1>(v));
}

__device__ __forceinline__ float wave_sum(float v) {
    v += xor_desc<32>(v);
    v += xor_desc<16>(v);
    v += xor_desc<8>(v);
    v += xor_desc<4>(v);
    v += xor_desc<2>(v);
    return v + xor_desc<1>(v);
}

// (value, index) argmax with torch's tie rule: larger value wins, equal values
// keep the lower index.
__device__ __forceinline__ void argmax_merge(float& v, int& i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

template <int O>
__device__ __forceinline__ void argmax_step_desc(float& v, int& i) {
    const float v2 = xor_desc<O>(v);
    const int i2 = xor_desc<O>(i);
    argmax_merge(v, i, v2, i2);
}

__device__ __forceinline__ void wave_argmax(float& v, int& i) {
    argmax_step_desc<32>(v, i);
    argmax_step_desc<16>(v, i);
    argmax_step_desc<8>(v, i);
    argmax_step_desc<4>(v, i);
    argmax_step_desc<2>(v, i);
    argmax_step_desc<1>(v, i);
}

// Workgroup reductions for blockDim.x == NT (a multiple of 64).  `scratch`
// holds at least NT/64 entries; the call contains two barriers.
template <int NT>
__device__ __forceinline__ float block_max(float v, float* scratch) {
    v = wave_max(v);
    const int w = threadIdx.x / kWave;
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0) scratch[w] = v;
    __syncthreads();
    float r = scratch[0];
#pragma unroll
    for (int k = 1; k < NT / kWave; ++k) r = fmaxf(r, scratch[k]);
    return r;
}

template <int NT>
__device__ __forceinline__ float block_sum(float v, float* scratch) {
    v = wave_sum(v);
    const int w = threadIdx.x / kWave;
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0) scratch[w] = v;
    __syncthreads();
    float r = scratch[0];
#pragma unroll
    for (int k = 1; k < NT / kWave; ++k) r += scratch[k];
    return r;
}

template <int NT>
__device__ __forceinline__ void block_argmax(float& v, int& i, float* sv, int* si) {
    wave_argmax(v, i);
    const int w = threadIdx.x / kWave;
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0) {
        sv[w] = v;
        si[w] = i;
    }
    __syncthreads();
    v = sv[0];
    i = si[0];
#pragma unroll
    for (int k = 1; k < NT / kWave; ++k) argmax_merge(v, i, sv[k], si[k]);
}

}  // namespace d3d
