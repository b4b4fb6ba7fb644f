// Sumcheck rounds of a product of two multilinear tables on MI355X: the
// round polynomials the WHIR prover sends before each fold
// (compute_sumcheck_polynomials, p3-whir src/pcs/prover/mod.rs:309-315),
// with the round and fold rules of zkIE's own sumcheck::prove
// (crates/zkie-core/src/common/sumcheck.rs:33-89):
//   round: pair the entries (2s, 2s + 1) (variable 0 = the least-significant
//          index bit), y_X = sum_s f(X) h(X) at X = 0, 1, 2 with
//          f(2) = 2 f1 - f0; c0 = y0, c1 = (4 y1 - y2 - 3 y0) / 2,
//          c2 = (y2 - 2 y1 + y0) / 2;
//   fold:  b[s] = a[2s] + r (a[2s + 1] - a[2s]) for both tables.
// f is base or EF, h and every folded table EF = F[x]/(x^2 - 7) flattened
// [c0, c1]; challenges are EF. The round-by-round entry points (the
// interactive form: each challenge drawn from the previous round's message)
// stream the tables once per round, the round kernel reducing its three EF
// sums per workgroup in LDS and one small workgroup adding the partial sums.
// zkie_sumcheck_prove, whose challenges are all given (sumcheck.rs:33-38),
// runs several rounds per pass over the tables (sc_multi_kernel).
#include <algorithm>
#include <vector>

#include "gl64.hpp"
#include "runtime.hpp"

namespace zk {
namespace {

constexpr int kScThreads = 256;
constexpr uint32_t kScMaxBlocks = 2048;  // workgroups of a round kernel (partial sums)

template <bool FEXT>
__device__ __forceinline__ Ef sc_load_f(const uint64_t* __restrict__ f, uint64_t i)
{
    if constexpr (FEXT)
        return Ef{f[2 * i], f[2 * i + 1]};
    else
        return Ef{f[i], 0};
}

template <bool FEXT>
__device__ __forceinline__ Ef sc_mul(Ef f, Ef h)
{
    if constexpr (FEXT)
        return ef_mul(f, h);
    else
        return ef_mul_base(h, f.c0);
}

// Six u64 per thread reduced over the workgroup; thread 0 gets the sums.
__device__ __forceinline__ void sc_block_reduce(uint64_t v[6], uint64_t (*red)[kScThreads])
{
    const uint32_t tid = threadIdx.x;
#pragma unroll
    for (int e = 0; e < 6; e++) red[e][tid] = v[e];
    __syncthreads();
#pragma unroll 1
    for (uint32_t w = kScThreads / 2; w > 0; w >>= 1) {
        if (tid < w) {
#pragma unroll
            for (int e = 0; e < 6; e++) red[e][tid] = gl_add(red[e][tid], red[e][tid + w]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int e = 0; e < 6; e++) v[e] = red[e][0];
}

// Partial sums [y0, y1, y2] (EF each) of the pairs s = gid, gid + stride, ...
// below `half`; one record of 6 u64 per workgroup.
template <bool FEXT>
__global__ __launch_bounds__(kScThreads) void sc_round_kernel(const uint64_t* __restrict__ f,
                                                              const uint64_t* __restrict__ h, uint64_t half,
                                                              uint64_t* __restrict__ partial)
{
    __shared__ uint64_t red[6][kScThreads];
    Ef y0{0, 0}, y1{0, 0}, y2{0, 0};
    const uint64_t stride = (uint64_t)gridDim.x * kScThreads;
    for (uint64_t s = (uint64_t)blockIdx.x * kScThreads + threadIdx.x; s < half; s += stride) {
        const Ef f0 = sc_load_f<FEXT>(f, 2 * s), f1 = sc_load_f<FEXT>(f, 2 * s + 1);
        const Ef h0{h[4 * s], h[4 * s + 1]}, h1{h[4 * s + 2], h[4 * s + 3]};
        const Ef f2 = ef_sub(ef_add(f1, f1), f0), h2 = ef_sub(ef_add(h1, h1), h0);
        y0 = ef_add(y0, sc_mul<FEXT>(f0, h0));
        y1 = ef_add(y1, sc_mul<FEXT>(f1, h1));
        y2 = ef_add(y2, sc_mul<FEXT>(f2, h2));
    }
    uint64_t v[6] = {y0.c0, y0.c1, y1.c0, y1.c1, y2.c0, y2.c1};
    sc_block_reduce(v, red);
    if (threadIdx.x == 0) {
#pragma unroll
        for (int e = 0; e < 6; e++) partial[6 * (uint64_t)blockIdx.x + e] = gl_canon(v[e]);
    }
}

// One workgroup of kFinThreads: the sum of `nblocks` partial records into
// out[0..6). Thread t adds component t % 6 of the records t / 6,
// t / 6 + kFinThreads / 6, ... (consecutive threads read consecutive words),
// then the kFinThreads / 6 threads of each component reduce in LDS.
// Workgroup g handles the records of round g: counts.n[g] records from
// partial + g * 6 * kScMaxBlocks, sums to out + 6 g.
constexpr int kFinThreads = 768;
constexpr int kFinPer = kFinThreads / 6;
constexpr uint32_t kScMaxRounds = 34;

struct FinCounts {
    uint32_t n[kScMaxRounds];
};

__global__ __launch_bounds__(kFinThreads) void sc_finish_kernel(const uint64_t* __restrict__ partial,
                                                                const FinCounts counts, uint64_t* __restrict__ out)
{
    __shared__ uint64_t red[kFinThreads];
    const uint32_t tid = threadIdx.x;
    const uint32_t nblocks = counts.n[blockIdx.x];
    partial += 6ull * kScMaxBlocks * blockIdx.x;
    out += 6 * blockIdx.x;
    uint64_t v = 0;
    for (uint64_t i = tid; i < 6ull * nblocks; i += kFinThreads) v = gl_add(v, partial[i]);
    red[tid] = v;
    __syncthreads();
    // component e = tid % 6 of lane j = tid / 6 lives at red[6 j + e]
    const uint32_t e = tid % 6, j = tid / 6;
#pragma unroll 1
    for (uint32_t w = kFinPer / 2; w > 0; w >>= 1) {
        uint64_t x = 0;
        const bool act = j < w;
        if (act) x = gl_add(red[6 * j + e], red[6 * (j + w) + e]);
        __syncthreads();
        if (act) red[6 * j + e] = x;
        __syncthreads();
    }
    if (tid < 6) out[tid] = gl_canon(red[tid]);
}

// Both tables bound at variable 0: out[s] = a[2s] + r (a[2s + 1] - a[2s]),
// s < half, outputs EF.
template <bool FEXT>
__global__ __launch_bounds__(kScThreads) void sc_fold_kernel(const uint64_t* __restrict__ f,
                                                             const uint64_t* __restrict__ h, uint64_t half,
                                                             uint64_t r0, uint64_t r1,
                                                             uint64_t* __restrict__ f_out,
                                                             uint64_t* __restrict__ h_out)
{
    const uint64_t s = flat_block() * kScThreads + threadIdx.x;
    if (s >= half) return;
    const Ef r{r0, r1};
    const Ef f0 = sc_load_f<FEXT>(f, 2 * s), f1 = sc_load_f<FEXT>(f, 2 * s + 1);
    const Ef h0{h[4 * s], h[4 * s + 1]}, h1{h[4 * s + 2], h[4 * s + 3]};
    const Ef fo = ef_add(f0, ef_mul(r, ef_sub(f1, f0)));
    const Ef ho = ef_add(h0, ef_mul(r, ef_sub(h1, h0)));
    f_out[2 * s] = gl_canon(fo.c0);
    f_out[2 * s + 1] = gl_canon(fo.c1);
    h_out[2 * s] = gl_canon(ho.c0);
    h_out[2 * s + 1] = gl_canon(ho.c1);
}

// Bind variable 0 of both tables (2^m entries, m >= 2) to r and, in the
// same pass, the next round's partial sums over the folded tables: lane s
// reads entries 4s .. 4s + 3, writes folded entries 2s and 2s + 1 (one pair
// of the next round) and adds that pair's y0, y1, y2.
template <bool FEXT>
__global__ __launch_bounds__(kScThreads) void sc_fold_round_kernel(const uint64_t* __restrict__ f,
                                                                   const uint64_t* __restrict__ h,
                                                                   uint64_t quarter, uint64_t r0, uint64_t r1,
                                                                   uint64_t* __restrict__ f_out,
                                                                   uint64_t* __restrict__ h_out,
                                                                   uint64_t* __restrict__ partial)
{
    __shared__ uint64_t red[6][kScThreads];
    const Ef r{r0, r1};
    Ef y0{0, 0}, y1{0, 0}, y2{0, 0};
    const uint64_t stride = (uint64_t)gridDim.x * kScThreads;
    for (uint64_t s = (uint64_t)blockIdx.x * kScThreads + threadIdx.x; s < quarter; s += stride) {
        Ef fa[4], ha[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            fa[q] = sc_load_f<FEXT>(f, 4 * s + q);
            ha[q] = Ef{h[8 * s + 2 * q], h[8 * s + 2 * q + 1]};
        }
        const Ef f0 = ef_add(fa[0], ef_mul(r, ef_sub(fa[1], fa[0])));
        const Ef f1 = ef_add(fa[2], ef_mul(r, ef_sub(fa[3], fa[2])));
        const Ef h0 = ef_add(ha[0], ef_mul(r, ef_sub(ha[1], ha[0])));
        const Ef h1 = ef_add(ha[2], ef_mul(r, ef_sub(ha[3], ha[2])));
        f_out[4 * s] = gl_canon(f0.c0);
        f_out[4 * s + 1] = gl_canon(f0.c1);
        f_out[4 * s + 2] = gl_canon(f1.c0);
        f_out[4 * s + 3] = gl_canon(f1.c1);
        h_out[4 * s] = gl_canon(h0.c0);
        h_out[4 * s + 1] = gl_canon(h0.c1);
        h_out[4 * s + 2] = gl_canon(h1.c0);
        h_out[4 * s + 3] = gl_canon(h1.c1);
        const Ef f2 = ef_sub(ef_add(f1, f1), f0), h2 = ef_sub(ef_add(h1, h1), h0);
        y0 = ef_add(y0, ef_mul(f0, h0));
        y1 = ef_add(y1, ef_mul(f1, h1));
        y2 = ef_add(y2, ef_mul(f2, h2));
    }
    uint64_t v[6] = {y0.c0, y0.c1, y1.c0, y1.c1, y2.c0, y2.c1};
    sc_block_reduce(v, red);
    if (threadIdx.x == 0) {
#pragma unroll
        for (int e = 0; e < 6; e++) partial[6 * (uint64_t)blockIdx.x + e] = gl_canon(v[e]);
    }
}

// ---- several rounds in one pass (challenges known in advance) --------------
// sumcheck::prove takes all its challenges at once (sumcheck.rs:33-38), so K
// consecutive rounds need no reduction between them: the entries of a block
// of 2^K consecutive indices pair up in round 1 (bit 0), their folds pair up
// in round 2 (bit 1), and so on, and the whole tree of one block is formed in
// registers. Each lane takes whole blocks, adds every pair's products to its
// round's three sums, and writes the block's fully folded entry of both
// tables; the tables are streamed once for K rounds.
constexpr int kScMultiMax = 4;  // rounds per pass
// Rounds of a pass over a table of 2^m entries: four rounds in one pass keep
// a 16-entry tree per lane (about 110 VGPRs, four waves per SIMD), which
// is latency-bound on large tables; there two passes of two rounds stream
// faster (2^22 base entries x EF weights, 4 rounds: 89 us against 112 us of
// kernel time), while small tables are bound by the launches.
constexpr uint32_t kScWideLog = 20;
uint32_t sc_pass_rounds(uint32_t m, uint32_t left)
{
    return std::min<uint32_t>(m >= kScWideLog ? 2 : kScMultiMax, left);
}

struct ScChallenges {
    uint64_t r[2 * kScMultiMax];  // EF challenges of the pass's rounds, canonical
};

// The folded entry of the 2^J-entry sub-block at `off`, adding the products
// of its rounds 1..J (tree order) to acc[0..J). BASE: f entries of the block
// are base-field values (f not EF and J = 1, so both pair members are loads).
template <bool FEXT, int J, int K>
__device__ __forceinline__ void sc_tree(const uint64_t* __restrict__ f, const uint64_t* __restrict__ h,
                                        uint64_t off, const ScChallenges& c, Ef (&acc)[K][3], Ef& fo, Ef& ho)
{
    if constexpr (J == 0) {
        fo = sc_load_f<FEXT>(f, off);
        ho = Ef{h[2 * off], h[2 * off + 1]};
    } else {
        Ef fa, ha, fb, hb;
        sc_tree<FEXT, J - 1, K>(f, h, off, c, acc, fa, ha);
        sc_tree<FEXT, J - 1, K>(f, h, off + (1ull << (J - 1)), c, acc, fb, hb);
        constexpr bool BASE = !FEXT && J == 1;
        const Ef r{c.r[2 * (J - 1)], c.r[2 * (J - 1) + 1]};
        const Ef f2 = ef_sub(ef_add(fb, fb), fa), h2 = ef_sub(ef_add(hb, hb), ha);
        acc[J - 1][0] = ef_add(acc[J - 1][0], sc_mul<!BASE>(fa, ha));
        acc[J - 1][1] = ef_add(acc[J - 1][1], sc_mul<!BASE>(fb, hb));
        acc[J - 1][2] = ef_add(acc[J - 1][2], sc_mul<!BASE>(f2, h2));
        const Ef df = ef_sub(fb, fa);
        fo = ef_add(fa, BASE ? ef_mul_base(r, df.c0) : ef_mul(r, df));
        ho = ef_add(ha, ef_mul(r, ef_sub(hb, ha)));
    }
}

// K rounds over tables of nblk 2^K entries: the folded tables (nblk EF
// entries each) and, per round j, one record of its three EF sums per
// workgroup at partial + 6 (j kScMaxBlocks + workgroup).
template <bool FEXT, int K>
__global__ __launch_bounds__(kScThreads) void sc_multi_kernel(const uint64_t* __restrict__ f,
                                                              const uint64_t* __restrict__ h, uint64_t nblk,
                                                              const ScChallenges c, uint64_t* __restrict__ f_out,
                                                              uint64_t* __restrict__ h_out,
                                                              uint64_t* __restrict__ partial)
{
    __shared__ uint64_t red[6][kScThreads];
    Ef acc[K][3];
#pragma unroll
    for (int j = 0; j < K; j++)
#pragma unroll
        for (int e = 0; e < 3; e++) acc[j][e] = Ef{0, 0};
    const uint64_t stride = (uint64_t)gridDim.x * kScThreads;
    for (uint64_t b = (uint64_t)blockIdx.x * kScThreads + threadIdx.x; b < nblk; b += stride) {
        Ef fo, ho;
        sc_tree<FEXT, K, K>(f, h, b << K, c, acc, fo, ho);
        f_out[2 * b] = gl_canon(fo.c0);
        f_out[2 * b + 1] = gl_canon(fo.c1);
        h_out[2 * b] = gl_canon(ho.c0);
        h_out[2 * b + 1] = gl_canon(ho.c1);
    }
#pragma unroll
    for (int j = 0; j < K; j++) {
        uint64_t v[6] = {acc[j][0].c0, acc[j][0].c1, acc[j][1].c0, acc[j][1].c1, acc[j][2].c0, acc[j][2].c1};
        sc_block_reduce(v, red);
        if (threadIdx.x == 0) {
#pragma unroll
            for (int e = 0; e < 6; e++) partial[6 * ((uint64_t)j * kScMaxBlocks + blockIdx.x) + e] = gl_canon(v[e]);
        }
        __syncthreads();  // the reduction area is reused by the next round
    }
}

uint32_t sc_blocks(uint64_t items)
{
    const uint64_t want = (items + kScThreads - 1) / kScThreads;
    return (uint32_t)(want < kScMaxBlocks ? want : kScMaxBlocks);
}

// Adds the `blocks` partial records at `partial` into d_sums (6 u64).
int sc_finish(const uint64_t* partial, uint32_t blocks, uint64_t* d_sums, hipStream_t s)
{
    FinCounts c{};
    c.n[0] = blocks;
    ProfMark pm = prof_begin("sumcheck_finish", s);
    sc_finish_kernel<<<1, kFinThreads, 0, s>>>(partial, c, d_sums);
    prof_end(pm, s);
    ZK_LAUNCHED();
    return ZKIE_OK;
}

// Partial round sums of tables of 2^m entries (m >= 1) into `partial`
// (kScMaxBlocks records of 6 u64); *blocks receives the record count.
int sc_sums(const uint64_t* d_f, bool f_ext, const uint64_t* d_h, uint32_t m, uint64_t* partial,
            uint32_t* blocks, hipStream_t s)
{
    const uint64_t half = 1ull << (m - 1);
    *blocks = sc_blocks(half);
    ProfMark pm = prof_begin("sumcheck_round", s);
    if (f_ext)
        sc_round_kernel<true><<<*blocks, kScThreads, 0, s>>>(d_f, d_h, half, partial);
    else
        sc_round_kernel<false><<<*blocks, kScThreads, 0, s>>>(d_f, d_h, half, partial);
    prof_end(pm, s);
    ZK_LAUNCHED();
    return ZKIE_OK;
}

// Fold of tables of 2^m entries (m >= 2) by r with the next round's partial
// sums into `partial`; *blocks receives the record count.
int sc_fold_sums(const uint64_t* d_f, bool f_ext, const uint64_t* d_h, uint32_t m, const uint64_t* r,
                 uint64_t* d_f_out, uint64_t* d_h_out, uint64_t* partial, uint32_t* blocks, hipStream_t s)
{
    const uint64_t quarter = 1ull << (m - 2);
    *blocks = sc_blocks(quarter);
    const uint64_t r0 = gl_canon(r[0]), r1 = gl_canon(r[1]);
    ProfMark pm = prof_begin("sumcheck_fold_round", s);
    if (f_ext)
        sc_fold_round_kernel<true><<<*blocks, kScThreads, 0, s>>>(d_f, d_h, quarter, r0, r1, d_f_out, d_h_out,
                                                                  partial);
    else
        sc_fold_round_kernel<false><<<*blocks, kScThreads, 0, s>>>(d_f, d_h, quarter, r0, r1, d_f_out, d_h_out,
                                                                   partial);
    prof_end(pm, s);
    ZK_LAUNCHED();
    return ZKIE_OK;
}

// c0, c1, c2 (EF each, canonical) from y0, y1, y2 (sumcheck.rs:65-67).
void sc_coefficients(const uint64_t y[6], uint64_t poly[6])
{
    for (int e = 0; e < 2; e++) {
        const uint64_t y0 = y[e], y1 = y[2 + e], y2 = y[4 + e];
        const uint64_t c1 = gl_halve(gl_sub(gl_sub(gl_mul(4, y1), y2), gl_mul(3, y0)));
        const uint64_t c2 = gl_halve(gl_add(gl_sub(y2, gl_add(y1, y1)), y0));
        poly[e] = gl_canon(y0);
        poly[2 + e] = gl_canon(c1);
        poly[4 + e] = gl_canon(c2);
    }
}

int sc_fold(const uint64_t* d_f, bool f_ext, const uint64_t* d_h, uint32_t m, const uint64_t* r,
            uint64_t* d_f_out, uint64_t* d_h_out, hipStream_t s)
{
    const uint64_t half = 1ull << (m - 1);
    const uint64_t blocks = (half + kScThreads - 1) / kScThreads;
    const uint64_t r0 = gl_canon(r[0]), r1 = gl_canon(r[1]);
    ProfMark pm = prof_begin("sumcheck_fold", s);
    if (f_ext)
        sc_fold_kernel<true><<<grid_of(blocks, kScThreads), kScThreads, 0, s>>>(d_f, d_h, half, r0, r1, d_f_out, d_h_out);
    else
        sc_fold_kernel<false><<<grid_of(blocks, kScThreads), kScThreads, 0, s>>>(d_f, d_h, half, r0, r1, d_f_out, d_h_out);
    prof_end(pm, s);
    ZK_LAUNCHED();
    return ZKIE_OK;
}

// eq(p, x) = prod_b (x_b ? p_b : 1 - p_b) for x < 2^n (bit 0 first):
// lo[x mod 2^L] * hi[x >> L], both halves formed on the host.
// [a, a + n) and [b, b + m) (u64 counts) share memory.
bool overlaps(const uint64_t* a, uint64_t n, const uint64_t* b, uint64_t m) { return a < b + m && b < a + n; }

// ---- batched constraint weights of a WHIR round -----------------------------
// w[x] (+)= sum_c g_c T_c(x) over constraints c: an evaluation constraint at a
// point p has T(x) = eq(p, x) = prod_b (x_b ? p_b : 1 - p_b), a selection
// constraint at a univariate point z has T(x) = z^x = prod_b (x_b ? z^(2^b) :
// 1), and g_c = gamma^c. Both are products of one factor per bit of x, so
// with x = x_lo + 2^h x_hi each table splits into lo_c[x_lo] hi_c[x_hi]: one
// kernel forms those small tables, a second sums lo_c[x_lo] hi_c[x_hi] over
// c for every x as exact dot products (DotAcc), with hi_c (gamma folded in)
// read as wave-uniform scalars. The inputs travel as kernel arguments, so
// the call queues its work without waiting for the host.
constexpr uint32_t kCwMaxValues = 96;  // EF values per launch: eq coordinates + selection points

struct CwArgs {
    uint64_t g0[2];     // gamma^(index of the launch's first constraint)
    uint64_t gamma[2];
    uint32_t n, h, m, q;  // variables, low bits of the split, eq points, selection points
    uint64_t v[2 * kCwMaxValues];  // m points of n EF coordinates (variable 0 first), then q EF points
};

// lo[c][t] (t < 2^h) and hi[c][u] (u < 2^(n-h), stored [c0, c1, 7 c1], times g_c).
__global__ __launch_bounds__(kScThreads) void cw_tables_kernel(const CwArgs a, uint64_t* __restrict__ lo,
                                                              uint64_t* __restrict__ hi)
{
    const uint32_t C = a.m + a.q;
    const uint64_t nlo = (uint64_t)C << a.h, nhi = (uint64_t)C << (a.n - a.h);
    const uint64_t t = (uint64_t)blockIdx.x * kScThreads + threadIdx.x;
    if (t >= nlo + nhi) return;
    const bool is_lo = t < nlo;
    const uint64_t e = is_lo ? t : t - nlo;
    const uint32_t bits = is_lo ? a.h : a.n - a.h, b0 = is_lo ? 0 : a.h;
    const uint32_t c = (uint32_t)(e >> bits);
    const uint64_t x = e & ((1ull << bits) - 1);
    Ef acc{1, 0};
    if (c < a.m) {
        const uint64_t* p = a.v + 2 * ((uint64_t)c * a.n + b0);
        for (uint32_t b = 0; b < bits; b++) {
            const Ef pb{p[2 * b], p[2 * b + 1]};
            acc = ef_mul(acc, ((x >> b) & 1) ? pb : ef_sub(Ef{1, 0}, pb));
        }
    } else {
        const uint64_t* zp = a.v + 2 * ((uint64_t)a.m * a.n + (c - a.m));
        Ef z{zp[0], zp[1]};
        for (uint32_t b = 0; b < b0; b++) z = ef_mul(z, z);  // z^(2^h) for the high bits
        for (uint32_t b = 0; b < bits; b++) {
            if ((x >> b) & 1) acc = ef_mul(acc, z);
            z = ef_mul(z, z);
        }
    }
    if (is_lo) {
        lo[2 * e] = gl_canon(acc.c0);
        lo[2 * e + 1] = gl_canon(acc.c1);
    } else {
        Ef g{a.g0[0], a.g0[1]};
        const Ef gm{a.gamma[0], a.gamma[1]};
        for (uint32_t i = 0; i < c; i++) g = ef_mul(g, gm);
        acc = ef_mul(acc, g);
        const uint64_t c0 = gl_canon(acc.c0), c1 = gl_canon(acc.c1);
        hi[3 * e] = c0;
        hi[3 * e + 1] = c1;
        hi[3 * e + 2] = gl_canon(gl_mul7(c1));
    }
}

// w[x] (+)= sum_{c < C} lo_c[x_lo] hi_c[x_hi] for x < 2^n. Every x of a
// 256-entry block shares x_hi (2^h >= 256, or h = n), so hi is read at a
// wave-uniform address.
__global__ __launch_bounds__(kScThreads) void cw_apply_kernel(const uint64_t* __restrict__ lo,
                                                             const uint64_t* __restrict__ hi, uint32_t C,
                                                             uint32_t n, uint32_t h, int accumulate,
                                                             uint64_t* __restrict__ w)
{
    const uint64_t N = 1ull << n, nhi = 1ull << (n - h), lmask = (1ull << h) - 1;
    for (uint64_t base = (uint64_t)blockIdx.x * kScThreads; base < N; base += (uint64_t)gridDim.x * kScThreads) {
        const uint64_t x = base + threadIdx.x;
        if (x >= N) continue;
        const uint64_t xh = base >> h, xl = x & lmask;
        DotAcc s0, s1;
#pragma unroll 2
        for (uint32_t c = 0; c < C; c++) {
            const uint64_t* H = hi + 3 * ((uint64_t)c * nhi + xh);
            const uint64_t h0 = H[0], h1 = H[1], h7 = H[2];
            const uint64_t* Lp = lo + 2 * (((uint64_t)c << h) + xl);
            const uint64_t l0 = Lp[0], l1 = Lp[1];
            // (h0 + h1 X)(l0 + l1 X) = (h0 l0 + 7 h1 l1) + (h0 l1 + h1 l0) X
            dot_add(s0, h0, l0);
            dot_add(s0, h7, l1);
            dot_add(s1, h0, l1);
            dot_add(s1, h1, l0);
        }
        uint64_t c0 = gl_canon(dot_reduce(s0)), c1 = gl_canon(dot_reduce(s1));
        if (accumulate) {
            c0 = gl_canon(gl_add(w[2 * x], c0));
            c1 = gl_canon(gl_add(w[2 * x + 1], c1));
        }
        w[2 * x] = c0;
        w[2 * x + 1] = c1;
    }
}

// Launch the weights of m eq points and q selection points (gamma^0 for the
// first eq point); the inputs are host arrays, copied into kernel arguments.
int constraint_weights(const uint64_t* eq_points, uint32_t m, const uint64_t* sel, uint32_t q, const uint64_t* gamma,
                       uint32_t n, int accumulate, uint64_t* d_w, hipStream_t s)
{
    const uint32_t h = n <= 8 ? n : (((n + 1) / 2) > 8 ? (n + 1) / 2 : 8);
    const uint64_t N = 1ull << n;
    const unsigned apply_grid = (unsigned)std::min<uint64_t>((N + kScThreads - 1) / kScThreads, 65536);
    const uint32_t total = m + q;
    if (total == 0) {
        if (!accumulate) {
            cw_apply_kernel<<<apply_grid, kScThreads, 0, s>>>(nullptr, nullptr, 0, n, h, 0, d_w);
            ZK_LAUNCHED();
        }
        return ZKIE_OK;
    }
    // most constraints one launch can hold (selection points take one value each)
    const uint64_t per = ((1ull << h) * 2 + (1ull << (n - h)) * 3) * 8;
    Scratch ws(WS_MISC, (size_t)kCwMaxValues * per, s);
    if (ws.status()) return ws.status();
    uint64_t* d_lo = (uint64_t*)ws.get();
    const Ef gm{gl_canon(gamma[0]), gl_canon(gamma[1])};
    Ef g{1, 0};
    uint32_t c = 0;
    bool first = true;
    while (c < total) {
        CwArgs a{};
        a.gamma[0] = gm.c0;
        a.gamma[1] = gm.c1;
        a.g0[0] = gl_canon(g.c0);
        a.g0[1] = gl_canon(g.c1);
        a.n = n;
        a.h = h;
        // eq points first, then selection points, as many as fit: at most
        // kCwMaxValues values (the argument block) and kCwMaxValues
        // constraints (the small-table workspace; 0-variable eq points take
        // no values)
        uint32_t used = 0;
        while (c < m && used + n <= kCwMaxValues && a.m < kCwMaxValues) {
            for (uint32_t b = 0; b < n; b++) {
                a.v[2 * (used + b)] = gl_canon(eq_points[2 * ((uint64_t)c * n + b)]);
                a.v[2 * (used + b) + 1] = gl_canon(eq_points[2 * ((uint64_t)c * n + b) + 1]);
            }
            used += n;
            a.m++;
            c++;
        }
        if (c >= m) {
            while (c < total && used < kCwMaxValues && a.m + a.q < kCwMaxValues) {
                a.v[2 * used] = gl_canon(sel[2 * (c - m)]);
                a.v[2 * used + 1] = gl_canon(sel[2 * (c - m) + 1]);
                used++;
                a.q++;
                c++;
            }
        }
        const uint32_t C = a.m + a.q;
        uint64_t* d_hi = d_lo + ((uint64_t)C << h) * 2;
        const uint64_t entries = ((uint64_t)C << h) + ((uint64_t)C << (n - h));
        ProfMark pm = prof_begin("constraint_weights", s);
        cw_tables_kernel<<<(unsigned)((entries + kScThreads - 1) / kScThreads), kScThreads, 0, s>>>(a, d_lo, d_hi);
        cw_apply_kernel<<<apply_grid, kScThreads, 0, s>>>(d_lo, d_hi, C, n, h, first ? accumulate : 1, d_w);
        prof_end(pm, s);
        ZK_LAUNCHED();
        for (uint32_t i = 0; i < C; i++) g = ef_mul(g, gm);
        first = false;
    }
    return ZKIE_OK;
}

}  // namespace
}  // namespace zk

using namespace zk;

extern "C" {

int zkie_sumcheck_round(const uint64_t* d_f, int f_is_ext, const uint64_t* d_h, uint32_t num_vars,
                        uint64_t* poly, void* stream)
{
    if (num_vars < 1 || num_vars > 34 || !d_f || !d_h || !poly) return ZKIE_ERR_INVALID;
    hipStream_t s = as_stream(stream);
    Scratch ws(WS_MISC, (kScMaxBlocks + 1) * 6 * 8, s);
    if (ws.status()) return ws.status();
    uint64_t* partial = (uint64_t*)ws.get();
    uint64_t* d_sums = partial + 6 * kScMaxBlocks;
    uint32_t blocks = 0;
    int rc = sc_sums(d_f, f_is_ext != 0, d_h, num_vars, partial, &blocks, s);
    if (!rc) rc = sc_finish(partial, blocks, d_sums, s);
    if (rc) return rc;
    uint64_t y[6];
    ZK_TRY(hipMemcpyAsync(y, d_sums, sizeof(y), hipMemcpyDeviceToHost, s));
    ZK_TRY(hipStreamSynchronize(s));
    sc_coefficients(y, poly);
    return ZKIE_OK;
}

int zkie_sumcheck_fold(const uint64_t* d_f, int f_is_ext, const uint64_t* d_h, uint32_t num_vars,
                       const uint64_t* r, uint64_t* d_f_out, uint64_t* d_h_out, uint64_t* next_poly,
                       void* stream)
{
    if (num_vars < 1 || num_vars > 34 || !d_f || !d_h || !r || !d_f_out || !d_h_out) return ZKIE_ERR_INVALID;
    if (next_poly && num_vars < 2) return ZKIE_ERR_INVALID;
    const uint64_t n = 1ull << num_vars, half = n >> 1;
    const uint64_t nf = f_is_ext ? 2 * n : n;
    if (overlaps(d_f_out, 2 * half, d_f, nf) || overlaps(d_f_out, 2 * half, d_h, 2 * n) ||
        overlaps(d_h_out, 2 * half, d_f, nf) || overlaps(d_h_out, 2 * half, d_h, 2 * n) ||
        overlaps(d_f_out, 2 * half, d_h_out, 2 * half))
        return ZKIE_ERR_INVALID;
    hipStream_t s = as_stream(stream);
    if (!next_poly) return sc_fold(d_f, f_is_ext != 0, d_h, num_vars, r, d_f_out, d_h_out, s);
    Scratch ws(WS_MISC, (kScMaxBlocks + 1) * 6 * 8, s);
    if (ws.status()) return ws.status();
    uint64_t* partial = (uint64_t*)ws.get();
    uint64_t* d_sums = partial + 6 * kScMaxBlocks;
    uint32_t blocks = 0;
    int rc = sc_fold_sums(d_f, f_is_ext != 0, d_h, num_vars, r, d_f_out, d_h_out, partial, &blocks, s);
    if (!rc) rc = sc_finish(partial, blocks, d_sums, s);
    if (rc) return rc;
    uint64_t y[6];
    ZK_TRY(hipMemcpyAsync(y, d_sums, sizeof(y), hipMemcpyDeviceToHost, s));
    ZK_TRY(hipStreamSynchronize(s));
    sc_coefficients(y, next_poly);
    return ZKIE_OK;
}

int zkie_eq_table(const uint64_t* point, uint32_t num_vars, uint64_t* d_out, void* stream)
{
    if (num_vars > 34 || !d_out || (num_vars && !point)) return ZKIE_ERR_INVALID;
    // one evaluation constraint with weight gamma^0 = 1 (no host wait)
    const uint64_t one[2] = {1, 0};
    return constraint_weights(point, 1, nullptr, 0, one, num_vars, 0, d_out, as_stream(stream));
}

int zkie_constraint_weights(const uint64_t* eq_points, uint32_t m, const uint64_t* sel_points, uint32_t q,
                            const uint64_t* gamma, uint32_t num_vars, int accumulate, uint64_t* d_w, void* stream)
{
    if (num_vars > 34 || !d_w || !gamma || (m && !eq_points) || (q && !sel_points)) return ZKIE_ERR_INVALID;
    return constraint_weights(eq_points, m, sel_points, q, gamma, num_vars, accumulate != 0, d_w, as_stream(stream));
}

int zkie_sumcheck_prove(const uint64_t* d_f, int f_is_ext, const uint64_t* d_h, uint32_t num_vars,
                        uint32_t rounds, const uint64_t* r, uint64_t* polys, uint64_t* d_f_out,
                        uint64_t* d_h_out, void* stream)
{
    if (num_vars > 34 || rounds > num_vars || !d_f || !d_h || !d_f_out || !d_h_out ||
        (rounds && (!r || !polys)))
        return ZKIE_ERR_INVALID;
    hipStream_t s = as_stream(stream);
    const uint64_t n = 1ull << num_vars, nout = n >> rounds;
    const uint64_t nf = f_is_ext ? 2 * n : n;
    if (overlaps(d_f_out, 2 * nout, d_f, nf) || overlaps(d_f_out, 2 * nout, d_h, 2 * n) ||
        overlaps(d_h_out, 2 * nout, d_f, nf) || overlaps(d_h_out, 2 * nout, d_h, 2 * n) ||
        overlaps(d_f_out, 2 * nout, d_h_out, 2 * nout))
        return ZKIE_ERR_INVALID;
    if (rounds == 0) {
        // no round: the tables themselves, f lifted to EF
        if (f_is_ext) {
            ZK_TRY(hipMemcpyAsync(d_f_out, d_f, 16 * n, hipMemcpyDeviceToDevice, s));
        } else {
            ZK_TRY(hipMemsetAsync(d_f_out, 0, 16 * n, s));
            ZK_TRY(hipMemcpy2DAsync(d_f_out, 16, d_f, 8, 8, n, hipMemcpyDeviceToDevice, s));
        }
        ZK_TRY(hipMemcpyAsync(d_h_out, d_h, 16 * n, hipMemcpyDeviceToDevice, s));
        return ZKIE_OK;
    }
    // Workspace: partial sums, then every round's y sums (6 u64 each), then
    // the folded tables between passes: even passes write region A (f and h
    // of the first pass's output size, EF), odd passes region B after it
    // (the second pass's output size); the last pass writes the outputs.
    const uint32_t k0 = sc_pass_rounds(num_vars, rounds);
    const uint32_t k1 = rounds > k0 ? sc_pass_rounds(num_vars - k0, rounds - k0) : 0;
    const uint64_t out_a = rounds > k0 ? n >> k0 : 0;
    const uint64_t out_b = rounds > k0 + k1 ? n >> (k0 + k1) : 0;
    const uint64_t pool_u64 = 4 * out_a + 4 * out_b;
    // Every round keeps its own partial records, added by one launch at the end.
    Scratch ws(WS_FOLD, (6 * (kScMaxBlocks + 1) * rounds + pool_u64) * 8, s);
    if (ws.status()) return ws.status();
    uint64_t* partial = (uint64_t*)ws.get();
    uint64_t* d_y = partial + 6 * kScMaxBlocks * rounds;
    uint64_t* pool = d_y + 6 * rounds;
    FinCounts counts{};
    const uint64_t* cf = d_f;
    const uint64_t* ch = d_h;
    bool ext = f_is_ext != 0;
    // passes of up to kScMultiMax rounds, each streaming the tables once
    for (uint32_t i = 0, p = 0; i < rounds; p++) {
        const uint32_t K = sc_pass_rounds(num_vars - i, rounds - i);
        const uint64_t nblk = 1ull << (num_vars - i - K);
        uint64_t *nf_, *nh_;
        if (i + K == rounds) {
            nf_ = d_f_out;
            nh_ = d_h_out;
        } else {
            // passes shrink the table, so later passes fit their region
            uint64_t* base = (p % 2 == 0) ? pool : pool + 4 * out_a;
            nf_ = base;
            nh_ = base + 2 * nblk;
        }
        ScChallenges c{};
        for (uint32_t j = 0; j < K; j++) {
            c.r[2 * j] = gl_canon(r[2 * (i + j)]);
            c.r[2 * j + 1] = gl_canon(r[2 * (i + j) + 1]);
        }
        const uint32_t blocks = sc_blocks(nblk);
        for (uint32_t j = 0; j < K; j++) counts.n[i + j] = blocks;
        uint64_t* part = partial + 6ull * kScMaxBlocks * i;
        ProfMark pm = prof_begin("sumcheck_pass", s);
        switch (K * 2 + (ext ? 1 : 0)) {
            case 2: sc_multi_kernel<false, 1><<<blocks, kScThreads, 0, s>>>(cf, ch, nblk, c, nf_, nh_, part); break;
            case 3: sc_multi_kernel<true, 1><<<blocks, kScThreads, 0, s>>>(cf, ch, nblk, c, nf_, nh_, part); break;
            case 4: sc_multi_kernel<false, 2><<<blocks, kScThreads, 0, s>>>(cf, ch, nblk, c, nf_, nh_, part); break;
            case 5: sc_multi_kernel<true, 2><<<blocks, kScThreads, 0, s>>>(cf, ch, nblk, c, nf_, nh_, part); break;
            case 6: sc_multi_kernel<false, 3><<<blocks, kScThreads, 0, s>>>(cf, ch, nblk, c, nf_, nh_, part); break;
            case 7: sc_multi_kernel<true, 3><<<blocks, kScThreads, 0, s>>>(cf, ch, nblk, c, nf_, nh_, part); break;
            case 8: sc_multi_kernel<false, 4><<<blocks, kScThreads, 0, s>>>(cf, ch, nblk, c, nf_, nh_, part); break;
            default: sc_multi_kernel<true, 4><<<blocks, kScThreads, 0, s>>>(cf, ch, nblk, c, nf_, nh_, part); break;
        }
        prof_end(pm, s);
        ZK_LAUNCHED();
        cf = nf_;
        ch = nh_;
        ext = true;
        i += K;
    }
    ProfMark pm = prof_begin("sumcheck_finish", s);
    sc_finish_kernel<<<rounds, kFinThreads, 0, s>>>(partial, counts, d_y);
    prof_end(pm, s);
    ZK_LAUNCHED();
    std::vector<uint64_t> y(6 * rounds);
    ZK_TRY(hipMemcpyAsync(y.data(), d_y, y.size() * 8, hipMemcpyDeviceToHost, s));
    ZK_TRY(hipStreamSynchronize(s));
    for (uint32_t i = 0; i < rounds; i++) sc_coefficients(y.data() + 6 * i, polys + 6 * i);
    return ZKIE_OK;
}

}  // extern "C"
