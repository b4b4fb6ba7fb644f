// Device memory, workspace, kernel timers and device queries.
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "runtime.hpp"

namespace zk {

int current_device()
{
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess) return 0;
    return d;
}

namespace {

constexpr int kMaxDevices = 64;

}  // namespace

struct ScratchSlot {
    std::mutex mu;              // held for the whole of a lease
    void* ptr = nullptr;
    size_t bytes = 0;
    hipEvent_t done = nullptr;  // recorded on the last lease's stream when it ended
    bool pending = false;       // `done` marks GPU work that may still use ptr
};

namespace {

ScratchSlot g_slots[kMaxDevices][WS_COUNT];

struct ProfRecord {
    int kernel;
    hipEvent_t a, b;
};

struct ProfState {
    std::mutex mu;
    bool on = false;
    std::vector<std::string> names;
    std::unordered_map<std::string, int> ids;
    std::vector<ProfRecord> pending;
    std::vector<uint64_t> launches;
    std::vector<double> total_ms;
};

ProfState& prof()
{
    static ProfState s;
    return s;
}

int prof_id(ProfState& P, const char* kernel)
{
    auto it = P.ids.find(kernel);
    if (it != P.ids.end()) return it->second;
    int id = (int)P.names.size();
    P.names.emplace_back(kernel);
    P.ids.emplace(kernel, id);
    P.launches.push_back(0);
    P.total_ms.push_back(0.0);
    return id;
}

// Drain recorded event pairs into the totals (events are complete after a
// device synchronisation).
void prof_drain(ProfState& P)
{
    for (auto& r : P.pending) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, r.a, r.b) == hipSuccess) {
            P.launches[r.kernel] += 1;
            P.total_ms[r.kernel] += ms;
        }
        (void)hipEventDestroy(r.a);
        (void)hipEventDestroy(r.b);
    }
    P.pending.clear();
}

}  // namespace

Scratch::Scratch(WorkspaceSlot slot, size_t bytes, hipStream_t s) : s_(s)
{
    const int dev = current_device();
    if (dev < 0 || dev >= kMaxDevices || slot < 0 || slot >= WS_COUNT) {
        rc_ = ZKIE_ERR_NO_DEVICE;
        return;
    }
    ScratchSlot& w = g_slots[dev][slot];
    w.mu.lock();
    slot_ = &w;
    if (!w.ptr || w.bytes < bytes) {
        if (w.ptr) {
            // Queued kernels of earlier leases may still use the old buffer.
            const hipError_t e = hipDeviceSynchronize();
            if (e != hipSuccess) {
                rc_ = (int)e;
                return;
            }
            (void)hipFree(w.ptr);
            w.ptr = nullptr;
            w.bytes = 0;
        }
        w.pending = false;  // a fresh buffer has no users yet
        if (hipMalloc(&w.ptr, bytes ? bytes : 8) != hipSuccess) {
            w.ptr = nullptr;
            rc_ = ZKIE_ERR_ALLOC;
            return;
        }
        w.bytes = bytes;
    }
    if (w.pending) {
        // Also on the previous lease's own stream: a destroyed stream's handle
        // can come back for a new stream while the old work still runs.
        const hipError_t e = hipStreamWaitEvent(s, w.done, 0);
        if (e != hipSuccess) {
            rc_ = (int)e;
            return;
        }
    }
    ptr_ = w.ptr;
}

Scratch::~Scratch()
{
    if (!slot_) return;
    ScratchSlot& w = *slot_;
    if (ptr_) {
        bool recorded = false;
        if (!w.done) (void)hipEventCreateWithFlags(&w.done, hipEventDisableTiming);
        if (w.done) recorded = hipEventRecord(w.done, s_) == hipSuccess;
        // Without an event to order the next lease, wait for this one here.
        if (!recorded) (void)hipStreamSynchronize(s_);
        w.pending = recorded;
    }
    w.mu.unlock();
}

ProfMark prof_begin(const char* kernel, hipStream_t s)
{
    ProfState& P = prof();
    ProfMark m;
    {
        std::lock_guard<std::mutex> g(P.mu);
        if (!P.on) return m;
        m.kernel = prof_id(P, kernel);
    }
    if (hipEventCreate(&m.a) != hipSuccess) {
        m.kernel = -1;
        return m;
    }
    if (hipEventCreate(&m.b) != hipSuccess) {
        (void)hipEventDestroy(m.a);
        m.kernel = -1;
        return m;
    }
    (void)hipEventRecord(m.a, s);
    return m;
}

void prof_end(ProfMark m, hipStream_t s)
{
    if (m.kernel < 0) return;
    (void)hipEventRecord(m.b, s);
    ProfState& P = prof();
    std::lock_guard<std::mutex> g(P.mu);
    P.pending.push_back(ProfRecord{m.kernel, m.a, m.b});
}

}  // namespace zk

using namespace zk;

extern "C" {

int zkie_device_count(void)
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int zkie_dev_alloc(void** d_ptr, size_t bytes)
{
    if (!d_ptr) return ZKIE_ERR_INVALID;
    *d_ptr = nullptr;
    if (bytes == 0) return ZKIE_OK;
    ZK_TRY(hipMalloc(d_ptr, bytes));
    return ZKIE_OK;
}

int zkie_dev_free(void* d_ptr)
{
    if (!d_ptr) return ZKIE_OK;
    ZK_TRY(hipFree(d_ptr));
    return ZKIE_OK;
}

int zkie_memcpy_htod(void* d_dst, const void* src, size_t bytes)
{
    if (bytes == 0) return ZKIE_OK;
    ZK_TRY(hipMemcpy(d_dst, src, bytes, hipMemcpyHostToDevice));
    return ZKIE_OK;
}

int zkie_memcpy_dtoh(void* dst, const void* d_src, size_t bytes)
{
    if (bytes == 0) return ZKIE_OK;
    ZK_TRY(hipMemcpy(dst, d_src, bytes, hipMemcpyDeviceToHost));
    return ZKIE_OK;
}

int zkie_memcpy_dtod(void* d_dst, const void* d_src, size_t bytes, void* stream)
{
    if (bytes == 0) return ZKIE_OK;
    ZK_TRY(hipMemcpyAsync(d_dst, d_src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)));
    return ZKIE_OK;
}

int zkie_memset(void* d_ptr, int value, size_t bytes)
{
    if (bytes == 0) return ZKIE_OK;
    ZK_TRY(hipMemset(d_ptr, value, bytes));
    return ZKIE_OK;
}

int zkie_device_synchronize(void)
{
    ZK_TRY(hipDeviceSynchronize());
    return ZKIE_OK;
}

int zkie_stream_synchronize(void* stream)
{
    ZK_TRY(hipStreamSynchronize(as_stream(stream)));
    return ZKIE_OK;
}

// Streams of the default priority that do not synchronise with the null
// stream, so that work queued on two of them can overlap.
int zkie_stream_create(void** stream)
{
    if (!stream) return ZKIE_ERR_INVALID;
    hipStream_t s = nullptr;
    ZK_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return ZKIE_OK;
}

int zkie_stream_destroy(void* stream)
{
    if (!stream) return ZKIE_ERR_INVALID;
    ZK_TRY(hipStreamDestroy(as_stream(stream)));
    return ZKIE_OK;
}

// Work queued on `waiter` after this call starts once the work queued on
// `signaler` so far has finished.
int zkie_stream_wait(void* waiter, void* signaler)
{
    hipEvent_t e = nullptr;
    ZK_TRY(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    hipError_t rc = hipEventRecord(e, as_stream(signaler));
    if (rc == hipSuccess) rc = hipStreamWaitEvent(as_stream(waiter), e, 0);
    (void)hipEventDestroy(e);  // released once the wait has been satisfied
    ZK_TRY(rc);
    return ZKIE_OK;
}

// Inputs of the synthetic workloads (common/field.rs:17-36 XorShift64,
// common/fixed_point.rs:11-38 signed embedding v < 0 -> p - |v|).
int zkie_gen_inputs(uint64_t seed, uint64_t n, int kind, uint64_t* out)
{
    if (!out && n) return ZKIE_ERR_INVALID;
    const uint64_t P = 0xFFFFFFFF00000001ull;
    uint64_t x = seed + 0x9e3779b97f4a7c15ull;
    auto next = [&x]() {
        x ^= x << 13;
        x ^= x >> 7;
        x ^= x << 17;
        return x;
    };
    auto embed = [P](int64_t v) { return v >= 0 ? (uint64_t)v : P - (uint64_t)(-v); };
    switch (kind) {
        case ZKIE_GEN_UNIFORM:
            for (uint64_t i = 0; i < n; i++) out[i] = next() % P;
            return ZKIE_OK;
        case ZKIE_GEN_I16:
            for (uint64_t i = 0; i < n; i++) out[i] = embed((int16_t)(uint16_t)(next() % 65536));
            return ZKIE_OK;
        case ZKIE_GEN_I8:
            for (uint64_t i = 0; i < n; i++) out[i] = embed((int64_t)(next() % 255) - 127);
            return ZKIE_OK;
        case ZKIE_GEN_GAUSS_I16: {
            // Irwin-Hall sum of 12 53-bit uniforms, g = S 2^-53 - 6, value =
            // floor(g * 0.02 * 2^12 + 1/2) clamped to int16, in exact integers.
            const __int128 two53 = (__int128)1 << 53;
            for (uint64_t i = 0; i < n; i++) {
                __int128 S = 0;
                for (int k = 0; k < 12; k++) S += (__int128)(next() >> 11);
                const __int128 num = 2 * (S - 6 * two53) * 4096 + 50 * two53;
                const __int128 den = 2 * 50 * two53;
                __int128 q = num / den;
                if ((num % den != 0) && (num < 0)) q -= 1;
                if (q > 32767) q = 32767;
                if (q < -32768) q = -32768;
                out[i] = embed((int64_t)q);
            }
            return ZKIE_OK;
        }
        default:
            return ZKIE_ERR_INVALID;
    }
}

int zkie_profile_enable(int on)
{
    ProfState& P = prof();
    std::lock_guard<std::mutex> g(P.mu);
    P.on = on != 0;
    return ZKIE_OK;
}

int zkie_profile_reset(void)
{
    ZK_TRY(hipDeviceSynchronize());
    ProfState& P = prof();
    std::lock_guard<std::mutex> g(P.mu);
    prof_drain(P);
    for (auto& x : P.launches) x = 0;
    for (auto& x : P.total_ms) x = 0.0;
    return ZKIE_OK;
}

int zkie_profile_query(const char* kernel, uint64_t* launches, double* total_ms)
{
    if (!kernel) return ZKIE_ERR_INVALID;
    ZK_TRY(hipDeviceSynchronize());
    ProfState& P = prof();
    std::lock_guard<std::mutex> g(P.mu);
    prof_drain(P);
    auto it = P.ids.find(kernel);
    if (launches) *launches = it == P.ids.end() ? 0 : P.launches[it->second];
    if (total_ms) *total_ms = it == P.ids.end() ? 0.0 : P.total_ms[it->second];
    return ZKIE_OK;
}

int zkie_profile_names(char* buf, size_t cap)
{
    ProfState& P = prof();
    std::lock_guard<std::mutex> g(P.mu);
    std::string all;
    for (auto& n : P.names) {
        all += n;
        all += '\n';
    }
    if (!buf || cap == 0) return ZKIE_ERR_INVALID;
    size_t k = all.size() < cap - 1 ? all.size() : cap - 1;
    for (size_t i = 0; i < k; i++) buf[i] = all[i];
    buf[k] = 0;
    return all.size() < cap ? ZKIE_OK : ZKIE_ERR_INVALID;
}

}  // extern "C"
