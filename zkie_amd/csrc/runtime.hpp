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

// A grid of at least `blocks` workgroups of `threads` work-items. A dispatch
// holds its size in work-items as a 32-bit number per dimension, so past
// 2^32 work-items the grid becomes rows of 2^16 workgroups; the last row can
// overshoot, so kernels launched this way check their index against their
// size, and read their workgroup index with flat_block().
inline dim3 grid_of(uint64_t blocks, uint32_t threads)
{
    if (blocks * threads < (1ull << 32)) return dim3((unsigned)blocks, 1, 1);
    return dim3(65536u, (unsigned)((blocks + 65535) / 65536), 1);
}

__device__ __forceinline__ uint64_t flat_block() { return blockIdx.x + (uint64_t)blockIdx.y * gridDim.x; }

// Grow-only device scratch, one buffer per (device, slot); the same role as
// the reference's CudaBuffer arenas (cuda_buffer.rs:7-57), which the
// reference serialises behind a Mutex (cuda_buffer.rs:59).
//
// A Scratch lease owns its slot from construction to destruction: it holds
// the slot's host lock while the caller enqueues work that uses the buffer,
// makes the caller's stream wait for the GPU work of the previous lease (an
// event recorded when that lease ended, on whatever stream it used), and
// records its own end on its stream when destroyed. Calls on different
// streams, or from different host threads, therefore never use one buffer
// at the same time on the GPU, and none of them blocks the host. Nested
// leases are taken in the order WS_FOLD, WS_MISC, WS_NTT.
enum WorkspaceSlot { WS_NTT = 0, WS_MISC = 1, WS_FOLD = 2, WS_COUNT = 3 };

struct ScratchSlot;

class Scratch {
public:
    Scratch(WorkspaceSlot slot, size_t bytes, hipStream_t s);
    ~Scratch();
    Scratch(const Scratch&) = delete;
    Scratch& operator=(const Scratch&) = delete;
    // The buffer (at least `bytes` long), or nullptr when status() != 0.
    void* get() const { return ptr_; }
    // 0, a hipError_t, ZKIE_ERR_ALLOC or ZKIE_ERR_NO_DEVICE.
    int status() const { return rc_; }

private:
    ScratchSlot* slot_ = nullptr;
    hipStream_t s_;
    void* ptr_ = nullptr;
    int rc_ = 0;
};

// Kernel timers: when profiling is on, every instrumented launch records a
// HIP event pair on the launch stream; totals are read back on query. A mark
// owns its event pair until prof_end hands it to the pending list, so a
// concurrent drain never touches a pair whose end is not recorded yet.
struct ProfMark {
    int kernel = -1;
    hipEvent_t a = nullptr, b = nullptr;
};
ProfMark prof_begin(const char* kernel, hipStream_t s);
void prof_end(ProfMark m, hipStream_t s);

// Current device ordinal (for per-device caches).
int current_device();

// Work buffers of an LDE supplied by the caller instead of leased from the
// library's scratch: `ntt` holds the intermediate of a multi-pass transform
// (ntt_words u64), `coset` the 2 x 2^16 powers of a coset shift.
struct LdeWorkspace {
    uint64_t* ntt = nullptr;
    uint64_t ntt_words = 0;
    uint64_t* coset = nullptr;
};

struct PassArgs;

// A replacement for the last pass of a multi-pass LDE (the fused last pass
// and leaf hash of the commitment): fn launches it for the pass arguments a
// on stream s, or returns ZKIE_PASS_NOT_TAKEN to leave it to the plain pass.
constexpr int ZKIE_PASS_NOT_TAKEN = 1;
struct LastPassHook {
    int (*fn)(const PassArgs& a, hipStream_t s, void* ctx);
    void* ctx;
};

// zkie_lde_batch with the work buffers of `ws`, or leased ones when ws is
// null; `hook` (may be null) is offered the last pass. Only the first
// in_rows (1 <= in_rows <= h) rows of d_in are read: the rows from in_rows to
// h are zero coefficients. in_rows < h needs log_blowup >= 1.
int lde_run_rows(const uint64_t* d_in, uint64_t h, uint64_t in_rows, uint64_t w, uint32_t log_blowup,
                 uint64_t shift, uint64_t* d_out, hipStream_t s, const LdeWorkspace* ws,
                 const LastPassHook* hook);

inline int lde_run(const uint64_t* d_in, uint64_t h, uint64_t w, uint32_t log_blowup, uint64_t shift,
                   uint64_t* d_out, hipStream_t s, const LdeWorkspace* ws, const LastPassHook* hook)
{
    return lde_run_rows(d_in, h, h, w, log_blowup, shift, d_out, s, ws, hook);
}

}  // namespace zk
