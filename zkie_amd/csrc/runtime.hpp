// Host-side runtime shared by the kernels' entry points: status codes,
// launch checks, the grow-only per-device workspace and the kernel timers.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/zkie_hip.h"

namespace zk {

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

#define ZK_TRY(expr)                                   \
    do {                                               \
        hipError_t zk_e_ = (expr);                     \
        if (zk_e_ != hipSuccess) return (int)zk_e_;    \
    } while (0)

#define ZK_LAUNCHED()                                  \
    do {                                               \
        hipError_t zk_e_ = hipGetLastError();          \
        if (zk_e_ != hipSuccess) return (int)zk_e_;    \
    } while (0)

// Grow-only device scratch, one per (device, slot); the same role as the
// reference's CudaBuffer arenas (cuda_buffer.rs:7-57). Returns nullptr on
// allocation failure. Not thread-safe across host threads sharing a device.
enum WorkspaceSlot { WS_NTT = 0, WS_MERKLE = 1, WS_MISC = 2, WS_FOLD = 3, WS_COUNT = 4 };
void* workspace(WorkspaceSlot slot, size_t bytes);

// Kernel timers: when profiling is on, every instrumented launch records a
// HIP event pair on the launch stream; totals are read back on query.
struct ProfMark {
    int id = -1;
};
ProfMark prof_begin(const char* kernel, hipStream_t s);
void prof_end(ProfMark m, hipStream_t s);

// Current device ordinal (for per-device caches).
int current_device();

}  // namespace zk
