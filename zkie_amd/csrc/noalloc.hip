// zkie_lde_batch for callers that cannot allocate device memory (code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// The LDE's two work buffers (the intermediate of a multi-pass transform and
// the powers of a coset shift) live in one file-scope device array of fixed
// size instead of the library's grow-only scratch. The array is part of the
// code object: each device that loads the library holds its own copy, at its
// own address, until the process ends. Host code never passes the array's
// name to a kernel (on the host it names a stand-in, not device memory): the
// first call on a device, with that device current, looks up that device's
// address with hipGetSymbolAddress and keeps it, and every launch takes that
// address. The same first call also fills the twiddle tables, which live in a
// device array of the library as well.
//
// Nothing in the array has to start at zero: a transform writes the whole
// intermediate before reading it, and the coset powers are formed in full
// before the scaling reads them. Every call on one device shares that
// device's array, so calls that overlap on one device (several streams, or
// several host threads, without ordering between them) race on it.
#include <mutex>

#include "ntt_plan.hpp"
#include "runtime.hpp"

namespace zk {
namespace {

constexpr int kMaxDevices = 64;
// An n x w codeword of at most 2^23 u64 (64 MiB), e.g. 2^19 rows of 16.
constexpr uint64_t kNttWords = 1ull << 23;
constexpr uint64_t kCosetWords = 2 * kBigLen;  // 2 x 2^16 powers of the shift (1 MiB)

static __device__ __align__(256) uint64_t scratch[kCosetWords + kNttWords];

std::mutex g_mu;
uint64_t* g_scratch[kMaxDevices];  // per device: the device address of `scratch`

int scratch_address(uint64_t** out)
{
    std::lock_guard<std::mutex> g(g_mu);
    const int dev = current_device();
    if (dev < 0 || dev >= kMaxDevices) return ZKIE_ERR_NO_DEVICE;
    if (!g_scratch[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!ptr) return ZKIE_ERR_NO_DEVICE;
        g_scratch[dev] = (uint64_t*)ptr;
    }
    *out = g_scratch[dev];
    return ZKIE_OK;
}

}  // namespace
}  // namespace zk

using namespace zk;

extern "C" int zkie_lde_batch_noalloc(const uint64_t* d_in, uint64_t h, uint64_t w, uint32_t log_blowup,
                                      uint64_t shift, uint64_t* d_out, void* stream)
{
    if (h == 0 || (h & (h - 1)) != 0 || !d_in || !d_out || log_blowup > 32) return ZKIE_ERR_INVALID;
    if (w == 0) return ZKIE_OK;
    uint32_t lgh = 0;
    while ((1ull << lgh) < h) lgh++;
    if (lgh + log_blowup > 32) return ZKIE_ERR_INVALID;
    const uint64_t n = h << log_blowup;
    if (w > kNttWords || n > kNttWords / w) return ZKIE_ERR_SCRATCH_LIMIT;
    uint64_t* base = nullptr;
    const int rc = scratch_address(&base);
    if (rc) return rc;
    LdeWorkspace ws;
    ws.coset = base;
    ws.ntt = base + kCosetWords;
    ws.ntt_words = kNttWords;
    return lde_run(d_in, h, w, log_blowup, shift, d_out, as_stream(stream), &ws, nullptr);
}
