// Poseidon2 Merkle commitment on MI355X.
//
// Replaces crates/zkie-core/cuda/poseidon2_merkle.cu and the host schedule of
// crates/zkie-core/src/pcs/merkle_cuda.rs:177-312. Design:
//  * one row (leaf) or one parent (compression) per lane, so a wave of 64
//    lanes runs 64 independent permutations; the reference kernel instead
//    hashes 8 rows serially per thread (poseidon2_merkle.cu:187-196);
//  * levels with few parents, whose time is one permutation's latency, run
//    one permutation per 16-lane row (poseidon2_x16.hpp), and above a
//    power-of-two layer of at most 2^16 digests seven levels at a time are
//    reduced by one workgroup per subtree inside LDS (a level per barrier)
//    instead of one kernel launch per level (merkle_cuda.rs:250-280);
//  * the digest layers stay in HBM; openings gather rows and siblings on the
//    device and copy only what was asked for.
#include <algorithm>
#include <mutex>
#include <vector>

#include "last_leaf.hpp"
#include "ntt_plan.hpp"
#include "poseidon2.hpp"
#include "poseidon2_x16.hpp"
#include "row_stage.hpp"
#include "runtime.hpp"

namespace zk {

__constant__ P2Consts c_p2;

namespace {

constexpr int kMaxDevices = 64;
bool g_uploaded[kMaxDevices];
bool g_diag_fast[kMaxDevices];
std::mutex g_const_mu;

// ---- host derivation of the constants (merkle_cuda.rs:54-85) -------------
// rand 0.10 SmallRng = Xoshiro256++ seeded through SplitMix64; p3-goldilocks
// samples a field element by rejecting u64 >= p.
struct Xoshiro {
    uint64_t s[4];
    explicit Xoshiro(uint64_t seed)
    {
        uint64_t st = seed;
        for (int i = 0; i < 4; i++) {
            st += 0x9e3779b97f4a7c15ull;
            uint64_t z = st;
            z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
            z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
            s[i] = z ^ (z >> 31);
        }
    }
    static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
    uint64_t next()
    {
        const uint64_t res = rotl(s[0] + s[3], 23) + s[0];
        const uint64_t t = s[1] << 17;
        s[2] ^= s[0];
        s[3] ^= s[1];
        s[1] ^= s[2];
        s[0] ^= s[3];
        s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return res;
    }
    uint64_t field()
    {
        for (;;) {
            uint64_t x = next();
            if (x < P) return x;
        }
    }
};

void derive_default(P2Consts& c)
{
    Xoshiro r(1);
    for (int k = 0; k < 4; k++)
        for (int i = 0; i < 16; i++) c.ext[k][i] = r.field();
    for (int k = 4; k < 8; k++)
        for (int i = 0; i < 16; i++) c.ext[k][i] = r.field();
    for (int k = 0; k < 22; k++) c.internal[k] = r.field();
    c.diag15 = INV_2_32;
}

int upload(const P2Consts& in)
{
    const int dev = current_device();
    if (dev < 0 || dev >= kMaxDevices) return ZKIE_ERR_INVALID;
    P2Consts c = in;
    p2_set_diag(c);
    ZK_TRY(hipMemcpyToSymbol(HIP_SYMBOL(c_p2), &c, sizeof(P2Consts), 0, hipMemcpyHostToDevice));
    g_uploaded[dev] = true;
    g_diag_fast[dev] = p2_fast_constants(c);
    return ZKIE_OK;
}

// Upload the default constants on first use of a device; report whether
// the fast path applies (2^-32 diagonal, linear-layer constants below
// kRcLimit: p2_fast_constants).
int ensure_constants(bool* diag_fast)
{
    std::lock_guard<std::mutex> g(g_const_mu);
    const int dev = current_device();
    if (dev < 0 || dev >= kMaxDevices) return ZKIE_ERR_INVALID;
    if (!g_uploaded[dev]) {
        P2Consts c;
        derive_default(c);
        int rc = upload(c);
        if (rc) return rc;
    }
    *diag_fast = g_diag_fast[dev];
    return ZKIE_OK;
}

// ---- device helpers --------------------------------------------------------
__device__ __forceinline__ void store_digest(uint64_t* dst, const uint64_t* st)
{
    ulonglong2* d = reinterpret_cast<ulonglong2*>(dst);
#pragma unroll
    for (int k = 0; k < 4; k++) d[k] = make_ulonglong2(gl_canon(st[2 * k]), gl_canon(st[2 * k + 1]));
}

__device__ __forceinline__ void load8(uint64_t* st, const uint64_t* src)
{
    const ulonglong2* s = reinterpret_cast<const ulonglong2*>(src);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const ulonglong2 v = s[k];
        st[2 * k] = v.x;
        st[2 * k + 1] = v.y;
    }
}

// Sponge absorption of one row of W elements (W known at compile time when
// W > 0, else the runtime width w): PaddingFreeSponge<Perm, 16, 8, 8>.
template <int W, bool D15>
__device__ __forceinline__ void hash_row(const uint64_t* __restrict__ row, uint64_t w, uint64_t* st)
{
#pragma unroll
    for (int i = 0; i < 16; i++) st[i] = 0;
    if (W > 0) {
        constexpr int kFull = W / 8, kRem = W % 8;
#pragma unroll 1
        for (int b = 0; b < kFull; b++) {
            if ((W % 2) == 0) {
                load8(st, row + 8 * b);
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) st[i] = row[8 * b + i];
            }
            // a partial last chunk keeps the rate words it does not overwrite
            if constexpr (kRem == 0)
                p2_permute<D15, kOutAbsorb>(st, c_p2, b == kFull - 1);
            else
                p2_permute<D15>(st, c_p2);
        }
        if (kRem) {
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (i < kRem) st[i] = row[8 * kFull + i];
            p2_permute<D15, kOutDigest>(st, c_p2);
        }
    } else {
#pragma unroll 1
        for (uint64_t pos = 0; pos < w; pos += 8) {
            const uint64_t len = w - pos < 8 ? w - pos : 8;
#pragma unroll
            for (int i = 0; i < 8; i++)
                if ((uint64_t)i < len) st[i] = row[pos + i];
            p2_permute<D15>(st, c_p2);
        }
    }
}

// Leaf digests of rows [row0, row_end). Rows of 8 or 16 elements are staged
// through LDS (row_stage.hpp) so HBM serves each row once.
template <int W, bool D15>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void leaf_kernel(
    const uint64_t* __restrict__ mat, uint64_t* __restrict__ digests, uint64_t row0, uint64_t row_end,
    uint64_t w)
{
    uint64_t st[16];
    if constexpr (W == 8 || W == 16) {
        __shared__ uint64_t tile[256 * (W + 1)];
        const uint64_t first = row0 + flat_block() * 256;
        if (first >= row_end) return;  // the last row of a two-dimensional grid
        const uint32_t nrows = row_end - first < 256 ? (uint32_t)(row_end - first) : 256u;
        stage_rows<W>(mat, first, nrows, tile);
        if (threadIdx.x >= nrows) return;
        const uint64_t* row = tile + threadIdx.x * (W + 1);
#pragma unroll
        for (int i = 8; i < 16; i++) st[i] = 0;
#pragma unroll 1
        for (int b = 0; b < W / 8; b++) {
#pragma unroll
            for (int i = 0; i < 8; i++) st[i] = row[8 * b + i];
            p2_permute<D15, kOutAbsorb>(st, c_p2, b == W / 8 - 1);
        }
        store_digest(digests + (first + threadIdx.x) * 8, st);
    } else {
        const uint64_t row = row0 + flat_block() * blockDim.x + threadIdx.x;
        if (row >= row_end) return;
        hash_row<W, D15>(mat + row * (W > 0 ? (uint64_t)W : w), w, st);
        store_digest(digests + row * 8, st);
    }
}

// The last pass of a 16-wide LDE fused with the leaf hash (last_leaf.hpp):
// one workgroup per tile of the pass, 256 threads (four workgroups per CU
// for tiles of up to 256 rows).

template <int S, bool D15>
__global__ __launch_bounds__(fuse_threads<S>()) __attribute__((amdgpu_waves_per_eu(4))) void ntt_last_leaf_kernel(
    PassArgs a, uint64_t* __restrict__ digests)
{
    extern __shared__ uint64_t lds[];
    constexpr uint32_t T = fuse_threads<S>();
    const uint32_t tid = threadIdx.x;
    __builtin_assume(tid < T);
    const uint64_t bid = flat_block();
    if (bid >= pass_blocks(a)) return;  // the last row of a two-dimensional grid
    const PassTile t = pass_tile(a, bid);
    const PassLane l = pass_lane(a, t, tid);
    pass_tables<S, kRoleLast>(a, t, tid, T, lds);
    __syncthreads();
    pass_step<S, 8, false, kRoleLast, kFuseLogV>(0, a, t, l, tid, T, lds);
    __syncthreads();
    if constexpr (Radix<S>::n == 3) {
        pass_step<S, 8, false, kRoleLast, kFuseLogV>(1, a, t, l, tid, T, lds);
        __syncthreads();
    }
    uint64_t keep[LastLeaf<S>::template rounds<T>()][kStepU][LastLeaf<S>::R];
    last_leaf_step<S, T>(a, t, l, tid, lds, keep);
    __syncthreads();
    last_leaf_rows<S, T>(l, tid, lds, keep);
    __syncthreads();
    last_leaf_hash<S, T, D15>(tid, lds, c_p2);
    __syncthreads();
    last_leaf_store<S, T>(a, t, tid, lds, digests, 0);
}

// Parents [from, to) of `step` children each; slots [to, pad_to) get the
// zero digest (merkle_tree.rs:393-396 default digest padding).
template <bool D15>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void compress_kernel(const uint64_t* __restrict__ prev,
                                                       uint64_t* __restrict__ next, uint64_t from,
                                                       uint64_t to, uint64_t pad_to, uint32_t step)
{
    const uint64_t i = from + flat_block() * blockDim.x + threadIdx.x;
    if (i >= pad_to) return;
    uint64_t st[16];
    if (i >= to) {
#pragma unroll
        for (int k = 0; k < 16; k++) st[k] = 0;
        store_digest(next + i * 8, st);
        return;
    }
    load8(st, prev + (uint64_t)step * i * 8);
    if (step == 2) {
        load8(st + 8, prev + ((uint64_t)step * i + 1) * 8);
    } else {
#pragma unroll
        for (int k = 8; k < 16; k++) st[k] = 0;
    }
    p2_permute<D15, kOutDigest>(st, c_p2);
    store_digest(next + i * 8, st);
}

// compress_kernel for levels with few parents: one parent per 16-lane row,
// lane i holding state word i (the 16 words of two adjacent children are
// contiguous). Same slots and zero padding as compress_kernel; a row's lanes
// always take the same path.
__global__ __launch_bounds__(256) void compress_x16_kernel(const uint64_t* __restrict__ prev,
                                                           uint64_t* __restrict__ next, uint64_t from,
                                                           uint64_t to, uint64_t pad_to, uint32_t step)
{
    const uint64_t p = from + (flat_block() * blockDim.x + threadIdx.x) / 16;
    const uint32_t i = threadIdx.x & 15;
    if (p >= pad_to) return;
    if (p >= to) {
        if (i < 8) next[p * 8 + i] = 0;
        return;
    }
    uint64_t x;
    if (step == 2)
        x = prev[p * 16 + i];
    else
        x = i < 8 ? prev[p * 8 + i] : 0;
    const X16Lane L = x16_lane(c_p2, i);
    x = p2_permute_x16(x, L, c_p2);
    if (i < 8) next[p * 8 + i] = gl_canon(x);
}

// One workgroup reduces 2^levels consecutive digests of a layer to one
// digest, writing every intermediate layer: the top of the tree in LDS, one
// level per barrier, one parent per 16-lane row. Parent j of level t
// (t = 1..levels) of subtree g is written to out_layers[t-1] +
// (g << (levels - t)) + j.
constexpr uint32_t kSubLevels = 7;  // at most 128 digests: 64 parents, one row each
constexpr uint32_t kSubThreads = 1024;
struct SubtreeArgs {
    const uint64_t* in;    // first layer (already computed), 2^levels * groups digests
    uint64_t* out[24];     // output layer base pointers, level 1..levels
    uint32_t levels;
};

__global__ __launch_bounds__(kSubThreads) void subtree_kernel(SubtreeArgs a)
{
    // level t's digests in buf[t & 1]; level t + 1 reads them after the barrier
    __shared__ uint64_t buf[2][(1u << (kSubLevels - 1)) * 8];
    const uint32_t g = blockIdx.x;
    const uint32_t row = threadIdx.x / 16, i = threadIdx.x & 15, rows = blockDim.x / 16;
    const X16Lane L = x16_lane(c_p2, i);
    const uint64_t* src = a.in + ((uint64_t)g << a.levels) * 8;
    uint32_t n = 1u << a.levels;
    for (uint32_t t = 1; t <= a.levels; t++) {
        const uint32_t parents = n >> 1;
        for (uint32_t p = row; p < parents; p += rows) {
            uint64_t x = t == 1 ? src[16 * p + i] : buf[(t - 1) & 1][16 * p + i];
            x = p2_permute_x16(x, L, c_p2);
            if (i < 8) {
                const uint64_t c = gl_canon(x);
                buf[t & 1][8 * p + i] = c;
                a.out[t - 1][(((uint64_t)g << (a.levels - t)) + p) * 8 + i] = c;
            }
        }
        __syncthreads();
        n = parents;
    }
}

// Gather `count` records of `len` u64 at record ids ids[k] from src (record
// stride `stride` u64) into dst (contiguous).
__global__ __launch_bounds__(256) void gather_kernel(const uint64_t* __restrict__ src,
                                                     uint64_t stride, uint64_t len,
                                                     const uint64_t* __restrict__ ids,
                                                     uint64_t count, uint64_t* __restrict__ dst)
{
    const uint64_t t = flat_block() * blockDim.x + threadIdx.x;
    if (t >= count * len) return;
    const uint64_t k = t / len, e = t % len;
    dst[t] = src[ids[k] * stride + e];
}

dim3 grid_for(uint64_t n, unsigned block = 256) { return grid_of((n + block - 1) / block, block); }

// Launch the leaf kernel for rows [r0, r1) with a width specialisation.
int launch_leaves(const uint64_t* mat, uint64_t* dig, uint64_t r0, uint64_t r1, uint64_t w,
                  bool fast, hipStream_t s)
{
    if (r1 <= r0) return ZKIE_OK;
    // Even-width rows are read with 16-byte loads; digests are stored as 16-byte pairs.
    if (((uintptr_t)dig & 15) || ((w % 2) == 0 && ((uintptr_t)mat & 15))) return ZKIE_ERR_INVALID;
    const dim3 grid = grid_for(r1 - r0);
    ProfMark m = prof_begin("p2_leaf", s);
#define ZK_LEAF(WW)                                                                                   \
    do {                                                                                              \
        if (fast)                                                                                     \
            leaf_kernel<WW, true><<<grid, 256, 0, s>>>(mat, dig, r0, r1, w);                          \
        else                                                                                          \
            leaf_kernel<WW, false><<<grid, 256, 0, s>>>(mat, dig, r0, r1, w);                         \
    } while (0)
    switch (w) {
        case 1: ZK_LEAF(1); break;
        case 8: ZK_LEAF(8); break;
        case 16: ZK_LEAF(16); break;
        case 32: ZK_LEAF(32); break;
        case 128: ZK_LEAF(128); break;
        default: ZK_LEAF(0); break;
    }
#undef ZK_LEAF
    prof_end(m, s);
    ZK_LAUNCHED();
    return ZKIE_OK;
}

// Up to this many parent slots a level runs one permutation per 16-lane row:
// below it, a launch with one permutation per lane takes the latency of one
// permutation whatever its size, and the row form has a fifth of that
// latency for about three times the instructions.
constexpr uint64_t kX16MaxParents = 1ull << 15;

int launch_compress(const uint64_t* prev, uint64_t* next, uint64_t from, uint64_t to,
                    uint64_t pad_to, uint32_t step, bool fast, hipStream_t s)
{
    if (pad_to <= from) return ZKIE_OK;
    if (((uintptr_t)prev | (uintptr_t)next) & 15) return ZKIE_ERR_INVALID;  // 16-byte digest loads and stores
    ProfMark m = prof_begin("p2_compress", s);
    if (pad_to - from <= kX16MaxParents)
        compress_x16_kernel<<<grid_for((pad_to - from) * 16), 256, 0, s>>>(prev, next, from, to, pad_to, step);
    else if (fast)
        compress_kernel<true><<<grid_for(pad_to - from), 256, 0, s>>>(prev, next, from, to, pad_to, step);
    else
        compress_kernel<false><<<grid_for(pad_to - from), 256, 0, s>>>(prev, next, from, to, pad_to, step);
    prof_end(m, s);
    ZK_LAUNCHED();
    return ZKIE_OK;
}

std::vector<uint64_t> layer_lens(uint64_t h)
{
    auto padded = [](uint64_t raw) -> uint64_t {
        if (raw <= 1) return raw;
        return (raw + 1) / 2 * 2;
    };
    std::vector<uint64_t> lens;
    uint64_t len = padded(h);
    lens.push_back(len);
    while (len > 1) {
        len = padded(len / 2);
        lens.push_back(len);
    }
    return lens;
}

// Build every layer above layer 0 (layer 0 already filled and padded).
// Levels whose parent count is a power of two and small enough are reduced
// by the LDS subtree kernel; the rest go one launch per level.
int build_upper(uint64_t* d_layers, const std::vector<uint64_t>& lens, bool fast, hipStream_t s)
{
    std::vector<uint64_t> off(lens.size());
    uint64_t acc = 0;
    for (size_t i = 0; i < lens.size(); i++) {
        off[i] = acc;
        acc += lens[i] * 8;
    }
    size_t i = 0;
    const size_t top = lens.size() - 1;
    while (i < top) {
        const uint64_t len = lens[i];
        // Subtree path: every level above a power-of-two layer is an exact
        // halving (no padding), so a layer of at most 2^kSubLevels digests
        // reduces to the root in one launch, and a layer of at most
        // kX16MaxParents * 2 digests loses kSubLevels levels in one launch of
        // one workgroup per 2^kSubLevels-digest subtree.
        if ((len & (len - 1)) == 0 && len >= 2 && len <= 2 * kX16MaxParents) {
            uint32_t lg = 0;
            while ((1ull << lg) < len) lg++;
            const uint32_t levels = lg < kSubLevels ? lg : kSubLevels;
            SubtreeArgs a;
            a.in = d_layers + off[i];
            a.levels = levels;
            for (uint32_t t = 1; t <= levels; t++) a.out[t - 1] = d_layers + off[i + t];
            const unsigned groups = (unsigned)(len >> levels);
            ProfMark m = prof_begin("p2_subtree", s);
            subtree_kernel<<<groups, kSubThreads, 0, s>>>(a);
            prof_end(m, s);
            ZK_LAUNCHED();
            i += levels;
            continue;
        }
        const uint64_t raw = len / 2;
        int rc = launch_compress(d_layers + off[i], d_layers + off[i + 1], 0, raw, lens[i + 1], 2,
                                 fast, s);
        if (rc) return rc;
        i++;
    }
    return ZKIE_OK;
}

// Launch the fused last pass + leaf hash for pass arguments `a` (the LDS
// limit raised per device above the 64 KB default).
template <int S, bool D15>
hipError_t launch_last_leaf_s(const PassArgs& a, uint64_t* digests, hipStream_t s)
{
    const size_t shmem = (size_t)LastLeaf<S>::lds_words() * 8;
    static std::mutex mu;
    static size_t raised[kMaxDevices];
    if (shmem > 64 * 1024) {
        const int dev = current_device();
        if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
        std::lock_guard<std::mutex> g(mu);
        if (shmem > raised[dev]) {
            const hipError_t e = hipFuncSetAttribute((const void*)&ntt_last_leaf_kernel<S, D15>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)shmem);
            if (e != hipSuccess) return e;
            raised[dev] = shmem;
        }
    }
    ntt_last_leaf_kernel<S, D15><<<grid_of(pass_blocks(a), fuse_threads<S>()), fuse_threads<S>(), shmem, s>>>(a, digests);
    return hipGetLastError();
}

template <bool D15>
hipError_t launch_last_leaf(const PassArgs& a, uint64_t* digests, hipStream_t s)
{
    switch (a.s) {
        case 4: return launch_last_leaf_s<4, D15>(a, digests, s);
        case 5: return launch_last_leaf_s<5, D15>(a, digests, s);
        case 6: return launch_last_leaf_s<6, D15>(a, digests, s);
        case 7: return launch_last_leaf_s<7, D15>(a, digests, s);
        case 8: return launch_last_leaf_s<8, D15>(a, digests, s);
        default: return launch_last_leaf_s<9, D15>(a, digests, s);
    }
}

// The fused pass applies (last_leaf_fusable) and the digests can take
// 16-byte stores.
bool fusable_last_pass(const PassArgs& a, const uint64_t* digests)
{
    return last_leaf_fusable(a) && ((uintptr_t)digests & 15) == 0;
}

struct FuseCtx {
    uint64_t* digests;
    bool fast;
    bool used;
};

int fuse_hook(const PassArgs& a, hipStream_t s, void* ctx)
{
    FuseCtx& c = *static_cast<FuseCtx*>(ctx);
    if (!fusable_last_pass(a, c.digests)) return ZKIE_PASS_NOT_TAKEN;
    ProfMark m = prof_begin("ntt_last_leaf", s);
    const hipError_t e = c.fast ? launch_last_leaf<true>(a, c.digests, s) : launch_last_leaf<false>(a, c.digests, s);
    prof_end(m, s);
    ZK_TRY(e);
    c.used = true;
    return ZKIE_OK;
}

}  // namespace

// Exposed to the other translation units of the library.
int merkle_commit_device(const uint64_t* d_mat, uint64_t h, uint64_t w, uint64_t* d_layers,
                         hipStream_t s)
{
    bool fast = false;
    int rc = ensure_constants(&fast);
    if (rc) return rc;
    const std::vector<uint64_t> lens = layer_lens(h);
    rc = launch_leaves(d_mat, d_layers, 0, h, w, fast, s);
    if (rc) return rc;
    if (lens[0] > h) {
        rc = launch_compress(nullptr, d_layers, h, h, lens[0], 2, fast, s);  // zero digests only
        if (rc) return rc;
    }
    if (lens.size() == 1) return ZKIE_OK;
    return build_upper(d_layers, lens, fast, s);
}

// The LDE of d_in into d_cw followed by the commitment of its rows into
// d_layers: the last NTT pass hashes the rows it produces when it can
// (fusable_last_pass), otherwise the leaf kernel hashes the finished codeword.
int lde_commit_device(const uint64_t* d_in, uint64_t h, uint64_t in_rows, uint64_t w, uint32_t log_blowup,
                      uint64_t shift, uint64_t* d_cw, uint64_t* d_layers, hipStream_t s)
{
    if (h == 0 || (h & (h - 1)) != 0 || log_blowup > 32 || !d_layers || (w > 0 && (!d_in || !d_cw)))
        return ZKIE_ERR_INVALID;
    uint32_t lgh = 0;
    while ((1ull << lgh) < h) lgh++;
    if (lgh + log_blowup > 32) return ZKIE_ERR_INVALID;
    const uint64_t n = h << log_blowup;
    bool fast = false;
    int rc = ensure_constants(&fast);
    if (rc) return rc;
    FuseCtx ctx{d_layers, fast, false};
    const LastPassHook hook{fuse_hook, &ctx};
    if (w > 0) {
        rc = lde_run_rows(d_in, h, in_rows, w, log_blowup, shift, d_cw, s, nullptr, &hook);
        if (rc) return rc;
    }
    const std::vector<uint64_t> lens = layer_lens(n);
    if (!ctx.used) {
        rc = launch_leaves(d_cw, d_layers, 0, n, w, fast, s);
        if (rc) return rc;
    }
    if (lens[0] > n) {
        rc = launch_compress(nullptr, d_layers, n, n, lens[0], 2, fast, s);  // zero digests only
        if (rc) return rc;
    }
    if (lens.size() == 1) return ZKIE_OK;
    return build_upper(d_layers, lens, fast, s);
}

// The root of an n-row tree (its last layer) into host memory, after the
// work queued on s.
int root_to_host(const uint64_t* d_layers, uint64_t n, uint64_t* root, hipStream_t s)
{
    if (!root) return ZKIE_OK;
    const std::vector<uint64_t> lens = layer_lens(n);
    uint64_t off = 0;
    for (size_t i = 0; i + 1 < lens.size(); i++) off += lens[i] * 8;
    ZK_TRY(hipMemcpyAsync(root, d_layers + off, 64, hipMemcpyDeviceToHost, s));
    ZK_TRY(hipStreamSynchronize(s));
    return ZKIE_OK;
}

__global__ __launch_bounds__(256) void zero_kernel(uint64_t* __restrict__ p, uint64_t n)
{
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        p[i] = 0;
}

unsigned stride_blocks(uint64_t n)
{
    const uint64_t g = (n + 255) / 256;
    return (unsigned)(g < (1ull << 16) ? (g ? g : 1) : (1ull << 16));
}

}  // namespace zk

using namespace zk;

extern "C" {

int zkie_p2_default_constants(uint64_t rc_init[64], uint64_t rc_final[64], uint64_t rc_internal[22],
                              uint64_t* diag15)
{
    if (!rc_init || !rc_final || !rc_internal || !diag15) return ZKIE_ERR_INVALID;
    P2Consts c;
    derive_default(c);
    for (int k = 0; k < 4; k++)
        for (int i = 0; i < 16; i++) {
            rc_init[16 * k + i] = c.ext[k][i];
            rc_final[16 * k + i] = c.ext[4 + k][i];
        }
    for (int k = 0; k < 22; k++) rc_internal[k] = c.internal[k];
    *diag15 = c.diag15;
    return ZKIE_OK;
}

int zkie_p2_upload_constants(const uint64_t* rc_init, const uint64_t* rc_final,
                             const uint64_t* rc_internal, uint64_t diag15)
{
    if (!rc_init || !rc_final || !rc_internal) return ZKIE_ERR_INVALID;
    P2Consts c;
    for (int k = 0; k < 4; k++)
        for (int i = 0; i < 16; i++) {
            c.ext[k][i] = gl_canon(rc_init[16 * k + i]);
            c.ext[4 + k][i] = gl_canon(rc_final[16 * k + i]);
        }
    for (int k = 0; k < 22; k++) c.internal[k] = gl_canon(rc_internal[k]);
    c.diag15 = gl_canon(diag15);
    std::lock_guard<std::mutex> g(g_const_mu);
    return upload(c);
}

int zkie_p2_leaf_batch(const uint64_t* d_mat, uint64_t* d_digests, uint32_t h, uint32_t w)
{
    bool fast = false;
    int rc = ensure_constants(&fast);
    if (rc) return rc;
    return launch_leaves(d_mat, d_digests, 0, (uint64_t)(h / 8) * 8, w, fast, 0);
}

int zkie_p2_leaf_scalar(const uint64_t* d_mat, uint64_t* d_digests, uint32_t start_row, uint32_t h,
                        uint32_t w)
{
    bool fast = false;
    int rc = ensure_constants(&fast);
    if (rc) return rc;
    return launch_leaves(d_mat, d_digests, start_row, h, w, fast, 0);
}

int zkie_p2_compress_batch(const uint64_t* d_prev, uint64_t* d_next, uint32_t next_len, uint32_t step)
{
    if (step != 1 && step != 2) return ZKIE_ERR_INVALID;
    bool fast = false;
    int rc = ensure_constants(&fast);
    if (rc) return rc;
    const uint64_t end = (uint64_t)(next_len / 8) * 8;
    return launch_compress(d_prev, d_next, 0, end, end, step, fast, 0);
}

int zkie_p2_compress_scalar(const uint64_t* d_prev, uint64_t* d_next, uint32_t from, uint32_t to,
                            uint32_t step)
{
    if (step != 1 && step != 2) return ZKIE_ERR_INVALID;
    bool fast = false;
    int rc = ensure_constants(&fast);
    if (rc) return rc;
    return launch_compress(d_prev, d_next, from, to, to, step, fast, 0);
}

int zkie_merkle_layout(uint64_t h, uint32_t* num_layers, uint64_t* layer_lens_out)
{
    if (h == 0 || !num_layers) return ZKIE_ERR_INVALID;
    const std::vector<uint64_t> lens = layer_lens(h);
    *num_layers = (uint32_t)lens.size();
    if (layer_lens_out)
        for (size_t i = 0; i < lens.size(); i++) layer_lens_out[i] = lens[i];
    return ZKIE_OK;
}

int zkie_merkle_commit(const uint64_t* d_mat, uint64_t h, uint64_t w, uint64_t* d_layers,
                       uint64_t* root, void* stream)
{
    if (h == 0 || !d_layers || (w > 0 && !d_mat)) return ZKIE_ERR_INVALID;
    hipStream_t s = as_stream(stream);
    int rc = merkle_commit_device(d_mat, h, w, d_layers, s);
    if (rc) return rc;
    if (root) {
        const std::vector<uint64_t> lens = layer_lens(h);
        uint64_t off = 0;
        for (size_t i = 0; i + 1 < lens.size(); i++) off += lens[i] * 8;
        ZK_TRY(hipMemcpyAsync(root, d_layers + off, 64, hipMemcpyDeviceToHost, s));
        ZK_TRY(hipStreamSynchronize(s));
    }
    return ZKIE_OK;
}

int zkie_lde_commit(const uint64_t* d_in, uint64_t h, uint64_t w, uint32_t log_blowup, uint64_t shift,
                    uint64_t* d_out, uint64_t* d_layers, uint64_t* root, void* stream)
{
    hipStream_t s = as_stream(stream);
    int rc = lde_commit_device(d_in, h, h, w, log_blowup, shift, d_out, d_layers, s);
    if (rc) return rc;
    return root_to_host(d_layers, h << log_blowup, root, s);
}

int zkie_commit_batch(const uint64_t* const* d_tables, uint32_t count, uint32_t arity, uint32_t log_width,
                      uint32_t log_blowup, uint64_t* d_stack, uint64_t* d_codeword, uint64_t* d_layers,
                      uint64_t* root, void* stream)
{
    if (!d_tables || count == 0 || arity > 40 || log_width > 16 || !d_stack || !d_codeword || !d_layers)
        return ZKIE_ERR_INVALID;
    // at most 2^48 stacked entries (a codeword row count of at most 2^32
    // with rows of at most 2^16), so every size below fits in 64 bits
    if ((uint64_t)count > (1ull << (48 - arity))) return ZKIE_ERR_INVALID;
    const uint64_t len = 1ull << arity;
    const uint64_t total = (uint64_t)count << arity;
    uint32_t vars = 0;  // total_num_vars: the stacked witness has 2^vars entries
    while ((1ull << vars) < total) vars++;
    if (vars < log_width || vars - log_width + log_blowup > 32) return ZKIE_ERR_INVALID;
    const uint64_t w = 1ull << log_width;
    const uint64_t h = 1ull << (vars - log_width);
    // rows holding table entries; with no blowup every row is read, so the
    // zero padding is written out
    const uint64_t data_rows = log_blowup ? (total + w - 1) / w : h;
    const uint64_t end = data_rows * w;
    // A table already in its slot of the stack is not copied; one that
    // overlaps any other part of the stack would be overwritten while read.
    const uintptr_t s0 = (uintptr_t)d_stack, s1 = s0 + end * 8;
    for (uint32_t i = 0; i < count; i++) {
        const uint64_t* t = d_tables[i];
        if (!t) return ZKIE_ERR_INVALID;
        if (t == d_stack + (uint64_t)i * len) continue;
        const uintptr_t t0 = (uintptr_t)t, t1 = t0 + len * 8;
        if (t0 < s1 && s0 < t1) return ZKIE_ERR_INVALID;
    }
    hipStream_t s = as_stream(stream);
    for (uint32_t i = 0; i < count; i++) {
        if (d_tables[i] == d_stack + (uint64_t)i * len) continue;
        ZK_TRY(hipMemcpyAsync(d_stack + (uint64_t)i * len, d_tables[i], len * 8, hipMemcpyDeviceToDevice, s));
    }
    if (end > total) {
        zero_kernel<<<stride_blocks(end - total), 256, 0, s>>>(d_stack + total, end - total);
        ZK_LAUNCHED();
    }
    const int rc = lde_commit_device(d_stack, h, data_rows, w, log_blowup, 1, d_codeword, d_layers, s);
    if (rc) return rc;
    return root_to_host(d_layers, h << log_blowup, root, s);
}

namespace {

// Copy `ids.size()` records of `len` u64 from src into host memory `out`.
int gather_to_host(const uint64_t* d_src, uint64_t stride, uint64_t len,
                   const std::vector<uint64_t>& ids, uint64_t* out, hipStream_t s)
{
    if (ids.empty() || len == 0) return ZKIE_OK;
    const uint64_t count = ids.size();
    const size_t bytes_ids = count * 8, bytes_out = count * len * 8;
    Scratch lease(WS_MISC, bytes_ids + bytes_out, s);
    if (lease.status()) return lease.status();
    uint8_t* ws = (uint8_t*)lease.get();
    uint64_t* d_ids = (uint64_t*)ws;
    uint64_t* d_out = (uint64_t*)(ws + bytes_ids);
    ZK_TRY(hipMemcpyAsync(d_ids, ids.data(), bytes_ids, hipMemcpyHostToDevice, s));
    gather_kernel<<<grid_for(count * len), 256, 0, s>>>(d_src, stride, len, d_ids, count, d_out);
    ZK_LAUNCHED();
    ZK_TRY(hipMemcpyAsync(out, d_out, bytes_out, hipMemcpyDeviceToHost, s));
    ZK_TRY(hipStreamSynchronize(s));
    return ZKIE_OK;
}

}  // namespace

int zkie_merkle_open_batch(const uint64_t* d_mat, uint64_t h, uint64_t w, const uint64_t* d_layers,
                           const uint64_t* indices, uint64_t n, uint64_t* rows_out,
                           uint64_t* siblings_out, void* stream)
{
    if (h == 0 || !d_layers || (n && !indices)) return ZKIE_ERR_INVALID;
    for (uint64_t k = 0; k < n; k++)
        if (indices[k] >= h) return ZKIE_ERR_INVALID;
    hipStream_t s = as_stream(stream);
    const std::vector<uint64_t> lens = layer_lens(h);
    if (rows_out && w > 0) {
        std::vector<uint64_t> rows(indices, indices + n);
        int rc = gather_to_host(d_mat, w, w, rows, rows_out, s);
        if (rc) return rc;
    }
    if (siblings_out && lens.size() > 1) {
        std::vector<uint64_t> ids;
        ids.reserve(n * (lens.size() - 1));
        for (uint64_t k = 0; k < n; k++) {
            uint64_t idx = indices[k], base = 0;
            for (size_t l = 0; l + 1 < lens.size(); l++) {
                ids.push_back(base + (idx ^ 1));
                base += lens[l];
                idx >>= 1;
            }
        }
        int rc = gather_to_host(d_layers, 8, 8, ids, siblings_out, s);
        if (rc) return rc;
    }
    return ZKIE_OK;
}

int zkie_merkle_open_pruned(const uint64_t* d_mat, uint64_t h, uint64_t w, const uint64_t* d_layers,
                            const uint64_t* indices, uint64_t n, uint64_t* rows_out,
                            uint64_t* pruned_out, uint64_t cap, uint64_t* count, void* stream)
{
    if (h == 0 || !d_layers || !count || (n && !indices)) return ZKIE_ERR_INVALID;
    for (uint64_t k = 0; k < n; k++)
        if (indices[k] >= h) return ZKIE_ERR_INVALID;
    hipStream_t s = as_stream(stream);
    const std::vector<uint64_t> lens = layer_lens(h);
    if (rows_out && w > 0) {
        std::vector<uint64_t> rows(indices, indices + n);
        int rc = gather_to_host(d_mat, w, w, rows, rows_out, s);
        if (rc) return rc;
    }
    // walk_frontier (pruning.rs:130-170), arity 2 at every level.
    std::vector<uint64_t> nodes(indices, indices + n);
    std::sort(nodes.begin(), nodes.end());
    nodes.erase(std::unique(nodes.begin(), nodes.end()), nodes.end());
    std::vector<uint64_t> ids;
    uint64_t base = 0;
    for (size_t l = 0; l + 1 < lens.size() && !nodes.empty(); l++) {
        std::vector<uint64_t> parents;
        size_t i = 0;
        while (i < nodes.size()) {
            const uint64_t group = nodes[i] / 2, start = group * 2;
            size_t member = i;
            for (uint64_t k = 0; k < 2; k++) {
                if (member < nodes.size() && nodes[member] == start + k)
                    member++;
                else
                    ids.push_back(base + start + k);
            }
            parents.push_back(group);
            i = member;
        }
        nodes.swap(parents);
        base += lens[l];
    }
    *count = ids.size();
    if (ids.size() > cap) return ZKIE_ERR_INVALID;
    if (!pruned_out) return ids.empty() ? ZKIE_OK : ZKIE_ERR_INVALID;
    return gather_to_host(d_layers, 8, 8, ids, pruned_out, s);
}

}  // extern "C"
