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

template <typename T>
__device__ __forceinline__ T wave_shfl_xor(T v, int mask) {
    return __shfl_xor(v, mask, kWave);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, wave_shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += wave_shfl_xor(v, o);
    return v;
}

// (value, index) argmax with torch's tie rule: larger value wins, equal values
// keep the lower index.
__device__ __forceinline__ void argmax_merge(float& v, int& i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float v2 = wave_shfl_xor(v, o);
        int i2 = wave_shfl_xor(i, o);
        argmax_merge(v, i, v2, i2);
    }
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

// Agent-scope release/acquire used by the "last workgroup finishes" pattern.
// Workgroups of one launch sit on different XCDs with separate L2s, so the
// counter increment is an acq_rel atomic at agent scope: it writes back this
// workgroup's results before the increment and invalidates stale lines after.
__device__ __forceinline__ unsigned atomic_inc_agent(unsigned* p) {
    return __hip_atomic_fetch_add(p, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void store_relaxed_agent(unsigned* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void fence_acquire_agent() {
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

}  // namespace d3d
