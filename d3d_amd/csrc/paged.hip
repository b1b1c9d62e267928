// Paged-KV block inputs on the device: the per-step page tables, slot
// mapping, positions and context lengths of a block of Q tokens per request,
// read from a device-resident page-table pool instead of built from host
// lists every step.
//
// Reference behaviour (D3D repository):
//   serving/backend.py:73-76    Runner._tables: per-sequence page lists padded
//                               with 0 to the longest list
//   serving/backend.py:123-124  slot = table[pos // PAGE] * PAGE + pos % PAGE
//                               for pos = start .. start + Q - 1
//   serving/backend.py:114-136  context_lens = start + Q (the block's keys are
//                               appended before attention)
//
// Pool entries past a sequence's page list hold -1: the gathered table
// shows them as 0 (the reference's padding) and their positions get slot -1.
// One workgroup per request: threads stride over the table width (gather of
// the request's pool row) and over the Q positions.
#include "d3d_common.hpp"
#include "../../include/d3d_hip.h"

namespace d3d {
namespace paged {

constexpr int NT = 256;

__global__ __launch_bounds__(NT) void block_inputs_kernel(const int32_t* pool, int pool_width, int pool_rows,
                                                          const int32_t* rows, const int32_t* starts, int Q,
                                                          int width, int page_size, int32_t* tables,
                                                          int64_t* slots, int64_t* positions, int32_t* lens) {
    const int b = blockIdx.x;
    const int row = rows[b];
    const bool row_ok = row >= 0 && row < pool_rows;
    const int32_t* src = pool + (size_t)(row_ok ? row : 0) * pool_width;
    for (int j = threadIdx.x; j < width; j += NT)
        tables[(size_t)b * width + j] = (row_ok && j < pool_width && src[j] >= 0) ? src[j] : 0;
    const int start = starts[b];
    for (int i = threadIdx.x; i < Q; i += NT) {
        const int64_t pos = (int64_t)start + i;
        const int64_t pi = pos / page_size;
        int64_t slot = -1;  // no page: the KV append skips the token
        if (row_ok && pos >= 0 && pi < width && pi < pool_width) {
            const int32_t page = src[pi];
            if (page >= 0) slot = (int64_t)page * page_size + pos % page_size;
        }
        slots[(size_t)b * Q + i] = slot;
        if (positions) positions[(size_t)b * Q + i] = pos;
    }
    if (threadIdx.x == 0 && lens) lens[b] = start + Q;
}

}  // namespace paged
}  // namespace d3d

using namespace d3d;

extern "C" int d3d_block_inputs(const int32_t* page_pool, int pool_rows, int pool_width, const int32_t* rows,
                                const int32_t* starts, int B, int Q, int width, int page_size,
                                int32_t* tables_out, int64_t* slots_out, int64_t* positions_out,
                                int32_t* context_lens_out, void* stream) {
    if (B < 0 || B > 65535 || Q < 1 || width < 1 || page_size < 1 || pool_rows < 1 || pool_width < 1)
        return D3D_E_SHAPE;
    if (B == 0) return D3D_OK;
    if (!page_pool || !rows || !starts || !tables_out || !slots_out) return D3D_E_NULL;
    hipLaunchKernelGGL(paged::block_inputs_kernel, dim3(B), dim3(paged::NT), 0, static_cast<hipStream_t>(stream),
                       page_pool, pool_width, pool_rows, rows, starts, Q, width, page_size, tables_out, slots_out,
                       positions_out, context_lens_out);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? D3D_OK : (int)err;
}
