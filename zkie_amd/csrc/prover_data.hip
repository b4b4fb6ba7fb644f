// Prover-data cache stream of one committed matrix: the bytes that follow the
// ZKIEBCH2 header in the reference's batch cache (crates/zkie-core/src/pcs/
// cache.rs:50-57 writes the header; whir.rs:542-560 then streams the tree).
//
// Layout (all integers u64 little-endian, the byte order of both the host
// and the device here):
//   1                      leaf-matrix count (whir.rs:547; WHIR commits one)
//   w, h*w                 width and value count of the matrix (whir.rs:549-550)
//   h*w values             the matrix rows, canonical Goldilocks (whir.rs:551-554)
//   L                      digest-layer count (merkle_tree.rs:229)
//   L layer lengths        digests per layer, leaves first (merkle_tree.rs:230-232)
//   L-1 arities            2 for every binary-tree transition (merkle_tree.rs:233-235)
//   the digest layers      8 values per digest, leaves first (merkle_tree.rs:236-241)
//
// The matrix and the layers already sit in HBM in exactly this order
// ([row 0 | row 1 | ...] and [layer0 | layer1 | ... | root]), so the writer
// only frames them: the payload goes device -> pinned staging -> callback in
// chunks, two staging buffers alternating so that the copy of chunk i + 1 is
// in flight while the callback consumes chunk i. The reader is the mirror
// (whir.rs:572-602 with merkle_tree.rs:247-276): framing is parsed on the
// host and checked against the caller's shape before any payload is copied.
#include <algorithm>
#include <vector>

#include "runtime.hpp"

namespace zk {
namespace {

constexpr uint64_t kChunkBytes = 16ull << 20;

// Two pinned staging buffers and their copy-done events. The destructor
// drains the stream first, so no copy can still target freed host memory on
// any return path.
struct Staging {
    hipStream_t s = nullptr;
    void* buf[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};

    ~Staging()
    {
        (void)hipStreamSynchronize(s);
        for (int i = 0; i < 2; i++) {
            if (buf[i]) (void)hipHostFree(buf[i]);
            if (ev[i]) (void)hipEventDestroy(ev[i]);
        }
    }
    int init(hipStream_t stream, uint64_t bytes)
    {
        s = stream;
        for (int i = 0; i < 2; i++) {
            ZK_TRY(hipHostMalloc(&buf[i], bytes ? bytes : 8, hipHostMallocDefault));
            ZK_TRY(hipEventCreateWithFlags(&ev[i], hipEventDisableTiming));
        }
        return 0;
    }
};

struct Framing {
    std::vector<uint64_t> head;  // 1, w, h*w
    std::vector<uint64_t> tree;  // L, lengths, arities
    uint64_t mat_bytes = 0;
    uint64_t layer_bytes = 0;
};

int make_framing(uint64_t h, uint64_t w, Framing& f)
{
    if (h == 0 || w == 0) return ZKIE_ERR_INVALID;
    if (h > UINT64_MAX / 8 / w) return ZKIE_ERR_INVALID;
    uint32_t nl = 0;
    uint64_t lens[65];
    const int rc = zkie_merkle_layout(h, &nl, lens);
    if (rc != 0) return rc;
    uint64_t digests = 0;
    for (uint32_t i = 0; i < nl; i++) digests += lens[i];
    f.head = {1, w, h * w};
    f.tree.clear();
    f.tree.push_back(nl);
    for (uint32_t i = 0; i < nl; i++) f.tree.push_back(lens[i]);
    for (uint32_t i = 0; i + 1 < nl; i++) f.tree.push_back(2);
    f.mat_bytes = h * w * 8;
    f.layer_bytes = digests * 64;
    return 0;
}

uint64_t chunk_len(uint64_t total, uint64_t i)
{
    const uint64_t off = i * kChunkBytes;
    return total - off < kChunkBytes ? total - off : kChunkBytes;
}

int stream_out(Staging& st, const uint8_t* d_src, uint64_t bytes, zkie_write_fn write, void* ctx)
{
    const uint64_t n = (bytes + kChunkBytes - 1) / kChunkBytes;
    auto issue = [&](uint64_t i) -> int {
        const int b = (int)(i & 1);
        ZK_TRY(hipMemcpyAsync(st.buf[b], d_src + i * kChunkBytes, chunk_len(bytes, i),
                              hipMemcpyDeviceToHost, st.s));
        ZK_TRY(hipEventRecord(st.ev[b], st.s));
        return 0;
    };
    if (n) {
        const int rc = issue(0);
        if (rc) return rc;
    }
    for (uint64_t i = 0; i < n; i++) {
        // buffer (i + 1) & 1 last held chunk i - 1, already consumed
        if (i + 1 < n) {
            const int rc = issue(i + 1);
            if (rc) return rc;
        }
        ZK_TRY(hipEventSynchronize(st.ev[i & 1]));
        if (write(ctx, st.buf[i & 1], chunk_len(bytes, i)) != 0) return ZKIE_ERR_IO;
    }
    return 0;
}

int stream_in(Staging& st, uint8_t* d_dst, uint64_t bytes, zkie_read_fn read, void* ctx)
{
    const uint64_t n = (bytes + kChunkBytes - 1) / kChunkBytes;
    for (uint64_t i = 0; i < n; i++) {
        const int b = (int)(i & 1);
        // the last copy out of this buffer (chunk i - 2, or a chunk of the
        // previous region) must be done before it is refilled; an event that
        // was never recorded is complete
        ZK_TRY(hipEventSynchronize(st.ev[b]));
        const uint64_t len = chunk_len(bytes, i);
        if (read(ctx, st.buf[b], len) != 0) return ZKIE_ERR_IO;
        ZK_TRY(hipMemcpyAsync(d_dst + i * kChunkBytes, st.buf[b], len, hipMemcpyHostToDevice, st.s));
        ZK_TRY(hipEventRecord(st.ev[b], st.s));
    }
    return 0;
}

uint64_t staging_bytes(const Framing& f)
{
    const uint64_t big = f.mat_bytes > f.layer_bytes ? f.mat_bytes : f.layer_bytes;
    return big < kChunkBytes ? big : kChunkBytes;
}

}  // namespace
}  // namespace zk

using namespace zk;

extern "C" int zkie_prover_data_size(uint64_t h, uint64_t w, uint64_t* bytes)
{
    if (!bytes) return ZKIE_ERR_INVALID;
    Framing f;
    const int rc = make_framing(h, w, f);
    if (rc) return rc;
    *bytes = 8 * (f.head.size() + f.tree.size()) + f.mat_bytes + f.layer_bytes;
    return 0;
}

extern "C" int zkie_prover_data_write(const uint64_t* d_mat, uint64_t h, uint64_t w,
                                      const uint64_t* d_layers, zkie_write_fn write, void* ctx,
                                      void* stream)
{
    if (!d_mat || !d_layers || !write) return ZKIE_ERR_INVALID;
    Framing f;
    int rc = make_framing(h, w, f);
    if (rc) return rc;
    Staging st;
    rc = st.init(as_stream(stream), staging_bytes(f));
    if (rc) return rc;
    if (write(ctx, f.head.data(), 8 * f.head.size()) != 0) return ZKIE_ERR_IO;
    rc = stream_out(st, reinterpret_cast<const uint8_t*>(d_mat), f.mat_bytes, write, ctx);
    if (rc) return rc;
    if (write(ctx, f.tree.data(), 8 * f.tree.size()) != 0) return ZKIE_ERR_IO;
    return stream_out(st, reinterpret_cast<const uint8_t*>(d_layers), f.layer_bytes, write, ctx);
}

extern "C" int zkie_prover_data_read(zkie_read_fn read, void* ctx, uint64_t h, uint64_t w,
                                     uint64_t* d_mat, uint64_t* d_layers, uint64_t* root,
                                     void* stream)
{
    if (!d_mat || !d_layers || !read) return ZKIE_ERR_INVALID;
    Framing f;
    int rc = make_framing(h, w, f);
    if (rc) return rc;
    std::vector<uint64_t> got(f.head.size());
    if (read(ctx, got.data(), 8 * got.size()) != 0) return ZKIE_ERR_IO;
    if (got != f.head) return ZKIE_ERR_INVALID;
    Staging st;
    rc = st.init(as_stream(stream), staging_bytes(f));
    if (rc) return rc;
    rc = stream_in(st, reinterpret_cast<uint8_t*>(d_mat), f.mat_bytes, read, ctx);
    if (rc) return rc;
    // The layer count comes first; the lengths and arities it announces are
    // read only when it matches the caller's geometry.
    uint64_t nl = 0;
    if (read(ctx, &nl, 8) != 0) return ZKIE_ERR_IO;
    if (nl != f.tree[0]) return ZKIE_ERR_INVALID;
    got.assign(f.tree.size() - 1, 0);
    if (!got.empty() && read(ctx, got.data(), 8 * got.size()) != 0) return ZKIE_ERR_IO;
    if (!std::equal(got.begin(), got.end(), f.tree.begin() + 1)) return ZKIE_ERR_INVALID;
    rc = stream_in(st, reinterpret_cast<uint8_t*>(d_layers), f.layer_bytes, read, ctx);
    if (rc) return rc;
    ZK_TRY(hipStreamSynchronize(st.s));
    if (root) {
        const uint64_t* d_root = d_layers + (f.layer_bytes / 8 - 8);
        ZK_TRY(hipMemcpyAsync(root, d_root, 64, hipMemcpyDeviceToHost, st.s));
        ZK_TRY(hipStreamSynchronize(st.s));
    }
    return 0;
}
