// WHIR/FRI row fold on MI355X.
//
// out[t] = sum_j eq(r, j) * row_t[j], eq(r, j) = prod_b (j_b ? r_b : 1 - r_b),
// bit 0 the least-significant index bit. This is zkIE's mle::eval
// (common/mle.rs:8-22) applied to every row, i.e. the codeword row fold of
// the WHIR prover (p3-whir src/pcs/prover/mod.rs:257-290, Suffix order) and,
// applied to the table viewed as 2^(n-k) rows of 2^k, the table fold over
// the low k variables (mle.rs:25-38 partial_eval).
// One row per lane; the 2^k eq weights are computed once on the host and
// read as wave-uniform values; each output is an exact dot product of the
// row with the weights (DotAcc: 32 x 32 partial products, one reduction per
// output); the codeword is streamed exactly once.
#include <vector>

#include "gl64.hpp"
#include "runtime.hpp"

namespace zk {
namespace {

// eq weights of a fold with k <= 6 (at most 64 EF values), passed by value
// as a kernel argument: they reach the kernel as scalar loads from the
// argument segment, and no device buffer has to outlive the launch, so the
// call does not synchronise its stream. Entry j is [e.c0, e.c1, 7 e.c1].
struct EqArg {
    uint64_t v[192];
};

template <int K, bool EXT>
__global__ __launch_bounds__(256) void fold_kernel(const uint64_t* __restrict__ mat, uint64_t h,
                                                   const EqArg eqa, uint64_t* __restrict__ out)
{
    const uint64_t* eq = eqa.v;
    constexpr int Wd = 1 << K;
    constexpr int RW = EXT ? 2 * Wd : Wd;  // u64 per row
    const uint64_t* row;
    uint64_t t;
    uint64_t rowv[RW % 2 == 0 && RW <= 16 ? RW : 2];
    if constexpr (RW % 2 == 0 && RW <= 16) {
        // rows of at most 128 bytes: each lane issues all of its row's 16-byte
        // loads at once (the 16-byte pieces of a wave's rows cover whole
        // lines across the loads, so HBM serves each line once)
        t = flat_block() * blockDim.x + threadIdx.x;
        if (t >= h) return;
        const ulonglong2* src = reinterpret_cast<const ulonglong2*>(mat + t * RW);
#pragma unroll
        for (int i = 0; i < RW / 2; i++) {
            const ulonglong2 v = src[i];
            rowv[2 * i] = v.x;
            rowv[2 * i + 1] = v.y;
        }
        row = rowv;
    } else {
        t = flat_block() * blockDim.x + threadIdx.x;
        if (t >= h) return;
        row = mat + t * RW;
    }
    // (e0 + e1 x)(y0 + y1 x) = (e0 y0 + 7 e1 y1) + (e0 y1 + e1 y0) x
    DotAcc s0, s1;
    if (!EXT) {
#pragma unroll
        for (int j = 0; j < Wd; j++) {
            const uint64_t x = row[j];
            dot_add(s0, eq[3 * j], x);
            dot_add(s1, eq[3 * j + 1], x);
        }
    } else {
#pragma unroll
        for (int j = 0; j < Wd; j++) {
            const uint64_t y0 = row[2 * j], y1 = row[2 * j + 1];
            dot_add(s0, eq[3 * j], y0);
            dot_add(s0, eq[3 * j + 2], y1);
            dot_add(s1, eq[3 * j], y1);
            dot_add(s1, eq[3 * j + 1], y0);
        }
    }
    reinterpret_cast<ulonglong2*>(out)[t] = make_ulonglong2(gl_canon(dot_reduce(s0)), gl_canon(dot_reduce(s1)));
}

// Generic width (K > 6): runtime loop.
template <bool EXT>
__global__ __launch_bounds__(256) void fold_kernel_rt(const uint64_t* __restrict__ mat, uint64_t h,
                                                      uint32_t k, const uint64_t* __restrict__ eq,
                                                      uint64_t* __restrict__ out)
{
    const uint64_t t = flat_block() * blockDim.x + threadIdx.x;
    if (t >= h) return;
    const uint64_t Wd = 1ull << k;
    uint64_t s0 = 0, s1 = 0;
    for (uint64_t j = 0; j < Wd; j++) {
        const uint64_t e0 = eq[2 * j], e1 = eq[2 * j + 1];
        if (!EXT) {
            const uint64_t x = mat[t * Wd + j];
            s0 = gl_add(s0, gl_mul(e0, x));
            s1 = gl_add(s1, gl_mul(e1, x));
        } else {
            const uint64_t y0 = mat[(t * Wd + j) * 2], y1 = mat[(t * Wd + j) * 2 + 1];
            s0 = gl_add(s0, gl_add(gl_mul(e0, y0), gl_mul7(gl_mul(e1, y1))));
            s1 = gl_add(s1, gl_add(gl_mul(e0, y1), gl_mul(e1, y0)));
        }
    }
    out[2 * t] = gl_canon(s0);
    out[2 * t + 1] = gl_canon(s1);
}

// eq table on the host: eq[j] = prod_b (bit_b(j) ? r_b : 1 - r_b) (mle.rs:44-56).
std::vector<uint64_t> eq_table(const uint64_t* r, uint32_t k)
{
    const uint64_t n = 1ull << k;
    std::vector<Ef> e(n, Ef{1, 0});
    for (uint32_t b = 0; b < k; b++) {
        const Ef rb{gl_canon(r[2 * b]), gl_canon(r[2 * b + 1])};
        const Ef one_minus = ef_sub(Ef{1, 0}, rb);
        for (uint64_t j = 0; j < n; j++) e[j] = ef_mul(e[j], ((j >> b) & 1) ? rb : one_minus);
    }
    std::vector<uint64_t> flat(2 * n);
    for (uint64_t j = 0; j < n; j++) {
        flat[2 * j] = gl_canon(e[j].c0);
        flat[2 * j + 1] = gl_canon(e[j].c1);
    }
    return flat;
}

}  // namespace

int fold_device(const uint64_t* d_mat, uint64_t h, uint32_t k, int is_ext, const uint64_t* r,
                uint64_t* d_out, hipStream_t s)
{
    if (k > 8 || !r || (h && (!d_mat || !d_out))) return ZKIE_ERR_INVALID;
    // Rows are staged with 16-byte loads and outputs stored as 16-byte pairs.
    if (((uintptr_t)d_mat | (uintptr_t)d_out) & 15) return ZKIE_ERR_INVALID;
    if (h == 0) return ZKIE_OK;
    const std::vector<uint64_t> eq = eq_table(r, k);
    const dim3 grid = grid_of((h + 255) / 256, 256);
    if (k <= 6) {
        EqArg ea{};
        for (size_t j = 0; 2 * j < eq.size(); j++) {
            ea.v[3 * j] = eq[2 * j];
            ea.v[3 * j + 1] = eq[2 * j + 1];
            ea.v[3 * j + 2] = gl_canon(gl_mul7(eq[2 * j + 1]));
        }
        ProfMark m = prof_begin("fold_rows", s);
#define ZK_FOLD(KK)                                                                  \
    case KK:                                                                         \
        if (is_ext)                                                                  \
            fold_kernel<KK, true><<<grid, 256, 0, s>>>(d_mat, h, ea, d_out);         \
        else                                                                         \
            fold_kernel<KK, false><<<grid, 256, 0, s>>>(d_mat, h, ea, d_out);        \
        break;
        switch (k) {
            ZK_FOLD(0)
            ZK_FOLD(1)
            ZK_FOLD(2)
            ZK_FOLD(3)
            ZK_FOLD(4)
            ZK_FOLD(5)
            default: ZK_FOLD(6)
        }
#undef ZK_FOLD
        prof_end(m, s);
        ZK_LAUNCHED();
        return ZKIE_OK;
    }
    Scratch ws(WS_MISC, eq.size() * 8, s);
    if (ws.status()) return ws.status();
    uint64_t* d_eq = (uint64_t*)ws.get();
    ZK_TRY(hipMemcpyAsync(d_eq, eq.data(), eq.size() * 8, hipMemcpyHostToDevice, s));
    ProfMark m = prof_begin("fold_rows", s);
    if (is_ext)
        fold_kernel_rt<true><<<grid, 256, 0, s>>>(d_mat, h, k, d_eq, d_out);
    else
        fold_kernel_rt<false><<<grid, 256, 0, s>>>(d_mat, h, k, d_eq, d_out);
    prof_end(m, s);
    ZK_LAUNCHED();
    // The eq weights were copied from a host vector that ends with this call.
    ZK_TRY(hipStreamSynchronize(s));
    return ZKIE_OK;
}

// Rows ids[0..n) (each `width` u64) gathered into dst.
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint64_t* __restrict__ src, uint64_t width,
                                                          const uint64_t* __restrict__ ids, uint64_t n,
                                                          uint64_t* __restrict__ dst)
{
    const uint64_t t = flat_block() * blockDim.x + threadIdx.x;
    if (t >= n * width) return;
    const uint64_t k = t / width, e = t % width;
    dst[t] = src[ids[k] * width + e];
}

// Multilinear evaluation of a table of 2^t entries at r (t EF coordinates,
// variable 0 the least-significant index bit): folds of at most six
// variables at a time, each reading the previous EF table once.
int mle_eval_device(const uint64_t* d_vals, uint32_t t, int is_ext, const uint64_t* r, uint64_t* out,
                    hipStream_t s)
{
    if (t > 40 || !d_vals || !r || !out) return ZKIE_ERR_INVALID;
    if (t == 0) {
        out[1] = 0;
        ZK_TRY(hipMemcpyAsync(out, d_vals, is_ext ? 16 : 8, hipMemcpyDeviceToHost, s));
        ZK_TRY(hipStreamSynchronize(s));
        out[0] = gl_canon(out[0]);
        out[1] = gl_canon(out[1]);
        return ZKIE_OK;
    }
    const uint32_t k0 = t < 6 ? t : 6;
    const uint64_t first = 1ull << (t - k0);  // EF entries after the first fold
    Scratch ws(WS_FOLD, 2 * first * 16, s);
    if (ws.status()) return ws.status();
    uint64_t* buf = (uint64_t*)ws.get();
    uint64_t* ping = buf;
    uint64_t* pong = buf + 2 * first;
    const uint64_t* cur = d_vals;
    int ext = is_ext;
    uint32_t left = t, done = 0;
    while (left > 0) {
        const uint32_t k = left < 6 ? left : 6;
        uint64_t* dst = (cur == ping) ? pong : ping;
        const int rc = fold_device(cur, 1ull << (left - k), k, ext, r + 2 * done, dst, s);
        if (rc) return rc;
        cur = dst;
        ext = 1;
        left -= k;
        done += k;
    }
    ZK_TRY(hipMemcpyAsync(out, cur, 16, hipMemcpyDeviceToHost, s));
    ZK_TRY(hipStreamSynchronize(s));
    return ZKIE_OK;
}

// Fold of the listed rows only (the queried-row fold of a STIR round).
int fold_rows_at_device(const uint64_t* d_mat, uint64_t h, uint32_t k, int is_ext, const uint64_t* ids,
                        uint64_t n, const uint64_t* r, uint64_t* out, hipStream_t s)
{
    if (k > 8 || !r || (n && (!d_mat || !ids || !out))) return ZKIE_ERR_INVALID;
    if (n == 0) return ZKIE_OK;
    for (uint64_t i = 0; i < n; i++)
        if (ids[i] >= h) return ZKIE_ERR_INVALID;
    const uint64_t width = (is_ext ? 2ull : 1ull) << k;
    // ids | rows | out, each region starting on a 256-byte boundary (the
    // fold stages rows with 16-byte loads and stores 16-byte outputs).
    auto round256 = [](uint64_t words) { return (words + 31) / 32 * 32; };
    const uint64_t ids_words = round256(n), rows_words = round256(n * width);
    Scratch ws(WS_FOLD, (ids_words + rows_words + 2 * n) * 8, s);
    if (ws.status()) return ws.status();
    uint64_t* buf = (uint64_t*)ws.get();
    uint64_t* d_ids = buf;
    uint64_t* d_rows = buf + ids_words;
    uint64_t* d_out = d_rows + rows_words;
    ZK_TRY(hipMemcpyAsync(d_ids, ids, n * 8, hipMemcpyHostToDevice, s));
    gather_rows_kernel<<<grid_of((n * width + 255) / 256, 256), 256, 0, s>>>(d_mat, width, d_ids, n, d_rows);
    ZK_LAUNCHED();
    const int rc = fold_device(d_rows, n, k, is_ext, r, d_out, s);
    if (rc) return rc;
    ZK_TRY(hipMemcpyAsync(out, d_out, 2 * n * 8, hipMemcpyDeviceToHost, s));
    ZK_TRY(hipStreamSynchronize(s));
    return ZKIE_OK;
}

}  // namespace zk

extern "C" int zkie_mle_eval(const uint64_t* d_vals, uint32_t num_vars, int is_ext, const uint64_t* r,
                             uint64_t* out, void* stream)
{
    return zk::mle_eval_device(d_vals, num_vars, is_ext, r, out, zk::as_stream(stream));
}

extern "C" int zkie_fold_rows_at(const uint64_t* d_mat, uint64_t h, uint32_t log_width, int is_ext,
                                 const uint64_t* indices, uint64_t n, const uint64_t* r, uint64_t* out,
                                 void* stream)
{
    return zk::fold_rows_at_device(d_mat, h, log_width, is_ext, indices, n, r, out, zk::as_stream(stream));
}

extern "C" int zkie_fold_rows(const uint64_t* d_mat, uint64_t h, uint32_t log_width, int is_ext,
                              const uint64_t* r, uint64_t* d_out, void* stream)
{
    return zk::fold_device(d_mat, h, log_width, is_ext, r, d_out, zk::as_stream(stream));
}
