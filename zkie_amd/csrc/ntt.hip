// Batched Goldilocks NTT on MI355X.
//
// Replaces crates/zkie-core/cuda/goldilocks_ntt.cu (lg_h full-HBM radix-2
// passes plus a scattered gather and scatter, capped at 2^18 rows by
// dft_cuda.rs:96) with a four-step decomposition:
//   n = 2^L is split into P passes of s_p bits (s_p <= 9). Pass p treats the
//   array as independent blocks of N = 2^B rows (B = L - s_0 - ... - s_{p-1}),
//   splits N = N1 * N2 with N1 = 2^(s_p) and computes, for every j2 < N2,
//       Y[i1][j2] = w_N^(i1 j2) * sum_j1 x[j1 N2 + j2] w_N1^(i1 j1)
//   into position i1 N2 + j2 of the block (in place), with the N1-point DFT
//   done as radix-2 decimation-in-frequency stages inside LDS. The last pass
//   (N2 = 1) writes each result straight to its natural row.
// A workgroup owns an N1 x V tile, V = C columns x J consecutive j2 values,
// chosen so that every global access of one point is a contiguous run of
// C*J*8 = 128 bytes (16 columns of a row, or 16 consecutive rows of a
// single column), i.e. whole cache lines.
// The first pass of an LDE reads only the h non-zero input rows; the zero
// rows of the padded matrix are never materialised or read.
#include <mutex>
#include <vector>

#include "ntt_plan.hpp"
#include "runtime.hpp"

namespace zk {
namespace {

constexpr int kMaxDevices = 64;

// The twiddle tables live in device memory of the code object itself (one
// copy per device, held until the process ends), filled from the host on
// the first transform on each device: no allocation after that first call.
__device__ __align__(256) uint64_t g_twiddles[kTableLen];
const uint64_t* g_tables[kMaxDevices];
std::mutex g_tab_mu;

int ensure_tables(const uint64_t** out)
{
    std::lock_guard<std::mutex> g(g_tab_mu);
    const int dev = current_device();
    if (dev < 0 || dev >= kMaxDevices) return ZKIE_ERR_INVALID;
    if (!g_tables[dev]) {
        const std::vector<uint64_t> h = build_twiddle_tables();
        void* d = nullptr;
        ZK_TRY(hipGetSymbolAddress(&d, HIP_SYMBOL(g_twiddles)));
        ZK_TRY(hipMemcpy(d, h.data(), h.size() * 8, hipMemcpyHostToDevice));
        g_tables[dev] = (const uint64_t*)d;
    }
    *out = g_tables[dev];
    return ZKIE_OK;
}

template <int S, int KNZ, bool INV, int ROLE, int LOGV, int ROWS>
__global__ __launch_bounds__(kNttThreads) void ntt_pass_kernel(PassArgs a)
{
    extern __shared__ uint64_t lds[];
    // The launch always uses kNttThreads threads; a compile-time count lets
    // the step loops unroll to their exact number of rounds.
    constexpr uint32_t T = kNttThreads;
    const uint32_t tid = threadIdx.x;
    __builtin_assume(tid < T);  // lets the step loops drop their item-count checks
    constexpr int n = pass_steps<S>();
    const uint64_t bid = flat_block();
    if (bid >= pass_blocks(a)) return;  // the last row of a two-dimensional grid
    const PassTile t = pass_tile(a, bid);
    const PassLane l = pass_lane(a, t, tid);
    if constexpr (n == 1) {
        pass_step<S, KNZ, INV, ROLE, LOGV>(0, a, t, l, tid, T, lds);
    } else {
        static_assert(((1u << (S - Radix<S>::r0)) << kNttLogV) <= kStepU * T, "step 0 in one round");
        // The table words are read first and the tile right after; the
        // tables are written to LDS (and the inter-pass table formed) while
        // the tile is still in flight, so the latencies overlap. The code is
        // straight-line from the table loads to their LDS writes (the row
        // check is a template choice), so the wait before the writes counts
        // the tile's loads as still in flight.
        static_assert(pass_table_entries<S, ROLE>() <= T, "a thread per table entry");
        const PassTabFetch tf = pass_tables_fetch<S, ROLE>(a, t, tid);
        __builtin_amdgcn_sched_barrier(0);  // keep the table loads ahead of the tile's
        uint64_t x[kStepU][1 << Radix<S>::r0];
        pass_step0_gather<S, KNZ, LOGV, ROWS>(a, t, l, tid, T, x);
        pass_tables_put<S, ROLE>(tf, t, tid, lds);
        __syncthreads();  // step twiddles in LDS before step 0 reads them
        if constexpr (ROLE == kRoleTable) {
            pass_tables_tab<S, ROLE>(t, tid, T, lds);
            __syncthreads();  // small tables read before step 0 overwrites them
        }
        pass_step0_finish<S, KNZ, INV, ROLE, LOGV>(a, t, l, tid, T, lds, x);
        __syncthreads();
        pass_step<S, KNZ, INV, ROLE, LOGV>(1, a, t, l, tid, T, lds);
    }
    if (n > 2) {
        __syncthreads();
        pass_step<S, KNZ, INV, ROLE, LOGV>(2, a, t, l, tid, T, lds);
    }
}

// Launch one instantiation, one workgroup per tile; dynamic LDS above the
// 64 KB default needs the kernel's limit raised first (gfx950 has 160 KB of
// LDS per CU).
template <int S, int KNZ, bool INV, int ROLE, int LOGV, int ROWS>
hipError_t launch_one(const PassArgs& a, uint64_t blocks, size_t shmem, hipStream_t s)
{
    // The raised limit is kept per device (the attribute is set with that
    // device current) and under a lock, so concurrent callers never record a
    // limit larger than the one actually set.
    static std::mutex mu;
    static size_t raised[kMaxDevices];
    if (shmem > 64 * 1024) {
        const int dev = current_device();
        if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
        std::lock_guard<std::mutex> g(mu);
        if (shmem > raised[dev]) {
            hipError_t e = hipFuncSetAttribute((const void*)&ntt_pass_kernel<S, KNZ, INV, ROLE, LOGV, ROWS>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)shmem);
            if (e != hipSuccess) return e;
            raised[dev] = shmem;
        }
    }
    ntt_pass_kernel<S, KNZ, INV, ROLE, LOGV, ROWS><<<grid_of(blocks, kNttThreads), kNttThreads, shmem, s>>>(a);
    return hipGetLastError();
}

// A first pass whose input has fewer rows than its read pattern covers
// checks rows (a separate instance); every other pass reads whole tiles. A
// pass reading all R inputs of its step-0 items (KNZ = 8) covers exactly the
// input's rows.
template <int S, int KNZ, bool INV, int ROLE, int LOGV>
hipError_t launch_rows(const PassArgs& a, uint64_t blocks, size_t shmem, hipStream_t s)
{
    if (!a.check_rows) return launch_one<S, KNZ, INV, ROLE, LOGV, kRowsAll>(a, blocks, shmem, s);
    if constexpr (KNZ < 8 && !INV)
        return launch_one<S, KNZ, INV, ROLE, LOGV, kRowsChecked>(a, blocks, shmem, s);
    else
        return hipErrorInvalidValue;
}

// Tiles of 16 vector lanes (the usual case) address LDS with immediate offsets.
template <int S, int KNZ, bool INV, int ROLE>
hipError_t launch_v(const PassArgs& a, uint64_t blocks, size_t shmem, hipStream_t s)
{
    if (a.logC + a.logJ == kNttLogV) return launch_rows<S, KNZ, INV, ROLE, (int)kNttLogV>(a, blocks, shmem, s);
    return launch_rows<S, KNZ, INV, ROLE, -1>(a, blocks, shmem, s);
}

// Instances: forward passes prune zero inputs of an LDE (KNZ < 8) and never
// scale; inverse passes read full inputs and scale in the last pass.
template <int S, bool INV, int ROLE>
hipError_t launch_pass_r(const PassArgs& a, int knz, uint64_t blocks, size_t shmem, hipStream_t s)
{
    if (INV) return launch_v<S, 8, INV, ROLE>(a, blocks, shmem, s);
    switch (knz) {
        case 1: return launch_v<S, 1, INV, ROLE>(a, blocks, shmem, s);
        case 2: return launch_v<S, 2, INV, ROLE>(a, blocks, shmem, s);
        case 4: return launch_v<S, 4, INV, ROLE>(a, blocks, shmem, s);
        default: return launch_v<S, 8, INV, ROLE>(a, blocks, shmem, s);
    }
}

template <int S, bool INV>
hipError_t launch_pass_s(const PassArgs& a, int knz, uint64_t blocks, size_t shmem, hipStream_t s)
{
    switch (pass_role(a)) {
        case kRoleTwiddle: return launch_pass_r<S, INV, kRoleTwiddle>(a, knz, blocks, shmem, s);
        case kRoleTable: return launch_pass_r<S, INV, kRoleTable>(a, knz, blocks, shmem, s);
        default:
            // A forward last pass never scales and an inverse one always does (1/n, n > 1).
            if constexpr (INV) {
                if (pass_role(a) != kRoleLastScale) return hipErrorInvalidValue;
                return launch_pass_r<S, INV, kRoleLastScale>(a, knz, blocks, shmem, s);
            } else {
                if (pass_role(a) != kRoleLast) return hipErrorInvalidValue;
                return launch_pass_r<S, INV, kRoleLast>(a, knz, blocks, shmem, s);
            }
    }
}

template <bool INV>
hipError_t launch_pass(const PassArgs& a, int knz, uint64_t blocks, size_t shmem, hipStream_t s)
{
    switch (a.s) {
        case 1: return launch_pass_s<1, INV>(a, knz, blocks, shmem, s);
        case 2: return launch_pass_s<2, INV>(a, knz, blocks, shmem, s);
        case 3: return launch_pass_s<3, INV>(a, knz, blocks, shmem, s);
        case 4: return launch_pass_s<4, INV>(a, knz, blocks, shmem, s);
        case 5: return launch_pass_s<5, INV>(a, knz, blocks, shmem, s);
        case 6: return launch_pass_s<6, INV>(a, knz, blocks, shmem, s);
        case 7: return launch_pass_s<7, INV>(a, knz, blocks, shmem, s);
        case 8: return launch_pass_s<8, INV>(a, knz, blocks, shmem, s);
        default: return launch_pass_s<9, INV>(a, knz, blocks, shmem, s);
    }
}

// Grid of a grid-stride launch over n items (256 threads per workgroup).
unsigned stride_grid(uint64_t n)
{
    const uint64_t g = (n + 255) / 256;
    return (unsigned)(g < (1ull << 20) ? (g ? g : 1) : (1ull << 20));
}

// Powers of the coset shift, formed on the device: lo[k] = shift^k and
// hi[k] = shift^(k 2^16) for k < 2^16, so shift^j = lo[j mod 2^16] hi[j >> 16].
__global__ __launch_bounds__(256) void coset_tables_kernel(uint64_t shift, uint64_t* __restrict__ lo,
                                                           uint64_t* __restrict__ hi)
{
    const uint64_t k = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= kBigLen) return;
    lo[k] = gl_pow(shift, k);
    hi[k] = gl_pow(shift, k << 16);
}

// Multiply row j of an h x w matrix by shift^j, shift^j = lo[j & 0xFFFF] * hi[j >> 16].
__global__ __launch_bounds__(256) void coset_scale_kernel(const uint64_t* __restrict__ in,
                                                          uint64_t* __restrict__ out, uint64_t h,
                                                          uint64_t w, const uint64_t* __restrict__ lo,
                                                          const uint64_t* __restrict__ hi)
{
    const uint64_t total = h * w;
    for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t j = t / w;
        const uint64_t sj = gl_mul(lo[j & 0xFFFF], hi[j >> 16]);
        out[t] = gl_canon(gl_mul(in[t], sj));
    }
}

// Run all passes (see pass_args for the buffer roles). A hook, when given,
// is offered the last pass of a multi-pass plan first; it returns
// ZKIE_PASS_NOT_TAKEN to leave that pass to the plain kernel.
int run_passes(const Plan& p, uint64_t w, const uint64_t* in, uint64_t in_rows, uint64_t* tmp,
               uint64_t* out, bool inverse, hipStream_t s, const LastPassHook* hook = nullptr)
{
    const uint64_t* tables = nullptr;
    int rc = ensure_tables(&tables);
    if (rc) return rc;
    uint32_t B = p.L;
    for (uint32_t i = 0; i < p.np; i++) {
        const PassArgs a = pass_args(p, i, B, w, in, in_rows, tmp, out, tables, inverse);
        B -= a.s;
        if (hook && a.last && p.np > 1) {
            rc = hook->fn(a, s, hook->ctx);
            if (rc != ZKIE_PASS_NOT_TAKEN) return rc;
        }
        const uint64_t blocks = pass_blocks(a);
        ProfMark m = prof_begin(a.last ? "ntt_pass_last" : (i == 0 ? "ntt_pass_first" : "ntt_pass_mid"), s);
        const hipError_t e = inverse ? launch_pass<true>(a, pass_knz(a), blocks, pass_lds_bytes(a), s)
                                     : launch_pass<false>(a, pass_knz(a), blocks, pass_lds_bytes(a), s);
        prof_end(m, s);
        ZK_TRY(e);
    }
    return ZKIE_OK;
}

int dft_inplace(uint64_t* d_mat, uint64_t* d_tmp, uint32_t lg, uint64_t w, bool inverse, hipStream_t s)
{
    if (lg > 32 || (w > 0 && !d_mat)) return ZKIE_ERR_INVALID;
    if (lg == 0 || w == 0) return ZKIE_OK;
    const Plan p = make_plan(lg, w);
    if (!plan_fits(p, w)) return ZKIE_ERR_INVALID;
    const uint64_t n = 1ull << lg;
    if (p.np == 1) return run_passes(p, w, d_mat, n, nullptr, d_mat, inverse, s);
    if (d_tmp) return run_passes(p, w, d_mat, n, d_tmp, d_mat, inverse, s);
    Scratch ws(WS_NTT, n * w * 8, s);
    if (ws.status()) return ws.status();
    return run_passes(p, w, d_mat, n, (uint64_t*)ws.get(), d_mat, inverse, s);
}

}  // namespace

int lde_run_rows(const uint64_t* d_in, uint64_t h, uint64_t in_rows, uint64_t w, uint32_t log_blowup,
                 uint64_t shift, uint64_t* d_out, hipStream_t s, const LdeWorkspace* ws,
                 const LastPassHook* hook)
{
    if (h == 0 || (h & (h - 1)) != 0 || !d_in || !d_out) return ZKIE_ERR_INVALID;
    // A first pass that reads fewer rows than its tile covers prunes inputs
    // of a step-0 radix below 8; with no blowup every input can be non-zero.
    if (in_rows == 0 || in_rows > h || (in_rows < h && log_blowup == 0)) return ZKIE_ERR_INVALID;
    uint32_t lgh = 0;
    while ((1ull << lgh) < h) lgh++;
    const uint32_t L = lgh + log_blowup;
    if (L > 32) return ZKIE_ERR_INVALID;
    if (w == 0) return ZKIE_OK;
    const uint64_t n = 1ull << L;
    const Plan p = make_plan(L, w);
    if (!plan_fits(p, w)) return ZKIE_ERR_INVALID;
    if (ws && p.np > 1 && n * w > ws->ntt_words) return ZKIE_ERR_INVALID;
    const uint64_t* src = d_in;
    shift = gl_canon(shift);
    if (shift != 1) {
        // coset: x_j <- x_j shift^j, staged in the head of d_out. The powers
        // are formed on the device on the call's stream, so nothing waits
        // for the host.
        auto scale = [&](uint64_t* d_tab) -> int {
            coset_tables_kernel<<<(unsigned)(kBigLen / 256), 256, 0, s>>>(shift, d_tab, d_tab + kBigLen);
            ZK_LAUNCHED();
            coset_scale_kernel<<<stride_grid(in_rows * w), 256, 0, s>>>(d_in, d_out, in_rows, w, d_tab,
                                                                       d_tab + kBigLen);
            ZK_LAUNCHED();
            return ZKIE_OK;
        };
        int rc;
        if (ws) {
            rc = scale(ws->coset);
        } else {
            Scratch lease(WS_MISC, 2 * kBigLen * 8, s);  // released before the WS_NTT lease below
            if (lease.status()) return lease.status();
            rc = scale((uint64_t*)lease.get());
        }
        if (rc) return rc;
        src = d_out;
    }
    if (p.np == 1) {
        if (src == d_out) {
            // in place, single pass: rows >= in_rows are treated as zero
            return run_passes(p, w, d_out, in_rows, nullptr, d_out, false, s);
        }
        return run_passes(p, w, src, in_rows, nullptr, d_out, false, s);
    }
    if (ws) return run_passes(p, w, src, in_rows, ws->ntt, d_out, false, s, hook);
    Scratch lease(WS_NTT, n * w * 8, s);
    if (lease.status()) return lease.status();
    return run_passes(p, w, src, in_rows, (uint64_t*)lease.get(), d_out, false, s, hook);
}

// Exposed to the other translation units of the library.
int lde_device(const uint64_t* d_in, uint64_t h, uint64_t w, uint32_t log_blowup, uint64_t shift,
               uint64_t* d_out, hipStream_t s)
{
    return lde_run(d_in, h, w, log_blowup, shift, d_out, s, nullptr, nullptr);
}

// Prefix order (writer.rs:43-71): entry (i, j) of the committed matrix, row
// i < 2^lrows and column j < 2^k, is poly[j 2^lrows + i]; E u64 per entry.
// `total` = E 2^(lrows + k) u64 (up to 2^33 for a 32-variable EF table).
__global__ __launch_bounds__(256) void prefix_transpose_kernel(const uint64_t* __restrict__ in,
                                                               uint64_t* __restrict__ out, uint64_t total,
                                                               uint32_t lrows, uint32_t k, uint32_t E)
{
    for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (uint64_t)gridDim.x * blockDim.x)
        out[t] = in[prefix_source(t, lrows, k, E)];
}

// commit_extension's encoding (writer.rs:21-86): the 2^n-entry table as a
// 2^(n-k) x 2^k matrix (Suffix: row-major as stored; Prefix: transposed),
// zero-padded to 2^log_inv_rate times the height and transformed per column
// (an EF table transforms per base component, dft_algebra_batch).
int whir_encode_device(const uint64_t* d_poly, uint32_t n_vars, int is_ext, uint32_t k,
                       uint32_t log_inv_rate, int prefix, uint64_t* d_out, hipStream_t s)
{
    if (k > n_vars || n_vars > 32 || !d_poly || !d_out) return ZKIE_ERR_INVALID;
    const uint64_t E = is_ext ? 2 : 1;
    const uint64_t h = 1ull << (n_vars - k), w = E << k;
    if (!prefix) return lde_device(d_poly, h, w, log_inv_rate, 1, d_out, s);
    const uint64_t total = h * w;
    if (d_poly < d_out + total && d_out < d_poly + total) return ZKIE_ERR_INVALID;  // no in-place transpose
    prefix_transpose_kernel<<<stride_grid(total), 256, 0, s>>>(d_poly, d_out, total, n_vars - k, k,
                                                               (uint32_t)E);
    ZK_LAUNCHED();
    return lde_device(d_out, h, w, log_inv_rate, 1, d_out, s);
}

}  // namespace zk

using namespace zk;

extern "C" {

int zkie_ntt_forward_goldilocks(uint64_t* d_mat, uint64_t* d_temp, uint32_t lg_h, uint64_t w,
                                const uint64_t* d_tw)
{
    (void)d_tw;  // twiddles are generated internally (identical values)
    return dft_inplace(d_mat, d_temp, lg_h, w, false, 0);
}

int zkie_dft_batch(uint64_t* d_mat, uint32_t lg_h, uint64_t w, void* stream)
{
    return dft_inplace(d_mat, nullptr, lg_h, w, false, as_stream(stream));
}

int zkie_idft_batch(uint64_t* d_mat, uint32_t lg_h, uint64_t w, void* stream)
{
    return dft_inplace(d_mat, nullptr, lg_h, w, true, as_stream(stream));
}

int zkie_whir_encode(const uint64_t* d_poly, uint32_t num_vars, int is_ext, uint32_t log_width,
                     uint32_t log_inv_rate, int prefix, uint64_t* d_out, void* stream)
{
    return whir_encode_device(d_poly, num_vars, is_ext, log_width, log_inv_rate, prefix, d_out,
                              as_stream(stream));
}

int zkie_lde_batch(const uint64_t* d_in, uint64_t h, uint64_t w, uint32_t log_blowup, uint64_t shift,
                   uint64_t* d_out, void* stream)
{
    return lde_device(d_in, h, w, log_blowup, shift, d_out, as_stream(stream));
}

}  // extern "C"
