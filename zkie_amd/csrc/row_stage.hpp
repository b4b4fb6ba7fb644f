// Block-wide staging of matrix rows into LDS.
//
// A kernel that gives each lane one row of W u64 (W * 8 = 64 or 128 bytes)
// and lets the lane read its own row touches a different cache line in every
// lane of a load instruction; with many waves per CU the lines are evicted
// before the lane reads their second half, and HBM serves each row twice.
// Copying the block's rows first with 16-byte loads that cover consecutive
// bytes reads every line once. The LDS row stride W + 1 (odd) puts the lanes'
// later reads of element c of their rows on different banks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace zk {

// Workgroup size of the kernels that stage rows (one row per thread).
constexpr uint32_t kStageThreads = 256;

// Rows [first, first + nrows) of a row-major matrix of W u64 per row (W even,
// mat 16-byte aligned) into tile[r * (W + 1) + c]; ends with a barrier.
template <int W>
__device__ __forceinline__ void stage_rows(const uint64_t* __restrict__ mat, uint64_t first,
                                           uint32_t nrows, uint64_t* tile)
{
    static_assert(W % 2 == 0, "16-byte loads");
    const ulonglong2* src = reinterpret_cast<const ulonglong2*>(mat + first * W);
    if (blockDim.x == kStageThreads && nrows == kStageThreads) {
        // A full tile: every load of the thread is issued before the first
        // LDS store waits for one, so W / 2 loads per lane are in flight.
        constexpr uint32_t N = W / 2;
        ulonglong2 v[N];
#pragma unroll
        for (uint32_t i = 0; i < N; i++) v[i] = src[threadIdx.x + i * kStageThreads];
#pragma unroll
        for (uint32_t i = 0; i < N; i++) {
            const uint32_t e = threadIdx.x + i * kStageThreads;
            const uint32_t r = (2 * e) / W, c = (2 * e) % W;
            tile[r * (W + 1) + c] = v[i].x;
            tile[r * (W + 1) + c + 1] = v[i].y;
        }
        __syncthreads();
        return;
    }
    for (uint32_t e = threadIdx.x; e < nrows * (W / 2); e += blockDim.x) {
        const ulonglong2 v = src[e];
        const uint32_t r = (2 * e) / W, c = (2 * e) % W;
        tile[r * (W + 1) + c] = v.x;
        tile[r * (W + 1) + c + 1] = v.y;
    }
    __syncthreads();
}

}  // namespace zk
