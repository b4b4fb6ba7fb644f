// Host-side NTT planning and twiddle tables, shared by the library and the
// CPU emulator of the device passes.
#pragma once

#include <vector>

#include "ntt_pass.hpp"

namespace zk {

constexpr uint32_t kMaxPassBits = 9;
// Threads of a pass workgroup: a 512 x 16 tile (64 KB of LDS) with 512
// threads keeps four waves per SIMD on a CU holding two such workgroups.
#ifndef ZK_NTT_THREADS
#define ZK_NTT_THREADS 512
#endif
constexpr uint32_t kNttThreads = ZK_NTT_THREADS;
// log2 of the tile's vector lanes V (columns times j2 values per tile).
#ifndef ZK_NTT_LOGV
#define ZK_NTT_LOGV 4
#endif
constexpr uint32_t kNttLogV = ZK_NTT_LOGV;
constexpr uint64_t kW512Len = 1ull << kStepTableLg;  // w_512^k, k < 512
constexpr uint64_t kBigLen = 1ull << 16;             // two-level table of w_{2^32}
constexpr uint64_t kTableLen = 2 * kW512Len + 4 * kBigLen;

// Table layout: [w512_fwd | w512_inv | lo_fwd | hi_fwd | lo_inv | hi_inv].
inline const uint64_t* tab_w512(const uint64_t* base, bool inv) { return base + (inv ? kW512Len : 0); }
inline const uint64_t* tab_lo(const uint64_t* base, bool inv) { return base + 2 * kW512Len + (inv ? 2 * kBigLen : 0); }
inline const uint64_t* tab_hi(const uint64_t* base, bool inv) { return tab_lo(base, inv) + kBigLen; }

// TWO_ADIC_GENERATORS[k] = 7^((p-1)/2^k), the table dft_cuda.rs:49 reads.
inline uint64_t two_adic_generator(uint32_t k) { return gl_pow(7, (P - 1) >> k); }

inline std::vector<uint64_t> build_twiddle_tables()
{
    std::vector<uint64_t> h(kTableLen, 0);
    for (int inv = 0; inv < 2; inv++) {
        uint64_t* w512 = h.data() + (inv ? kW512Len : 0);
        uint64_t root = two_adic_generator(kStepTableLg);
        if (inv) root = gl_inv(root);
        uint64_t x = 1;
        for (uint64_t k = 0; k < kW512Len; k++) {
            w512[k] = x;
            x = gl_canon(gl_mul(x, root));
        }
        uint64_t g32 = two_adic_generator(32);
        if (inv) g32 = gl_inv(g32);
        uint64_t* lo = h.data() + 2 * kW512Len + (inv ? 2 * kBigLen : 0);
        uint64_t* hi = lo + kBigLen;
        x = 1;
        for (uint64_t k = 0; k < kBigLen; k++) {
            lo[k] = x;
            x = gl_canon(gl_mul(x, g32));
        }
        const uint64_t step = x;  // g32^(2^16)
        x = 1;
        for (uint64_t k = 0; k < kBigLen; k++) {
            hi[k] = x;
            x = gl_canon(gl_mul(x, step));
        }
    }
    return h;
}

struct Plan {
    uint32_t L = 0, np = 0, logC = 0;
    uint32_t sb[8] = {0};
};

inline Plan make_plan(uint32_t L, uint64_t w)
{
    Plan p;
    p.L = L;
    uint32_t logC = 0;
    while (logC < kNttLogV && (w % (2ull << logC)) == 0) logC++;
    p.logC = logC;
    p.np = L == 0 ? 0 : (L + kMaxPassBits - 1) / kMaxPassBits;
    for (uint32_t i = 0; i < p.np; i++) p.sb[i] = L / p.np + (i < L % p.np ? 1 : 0);
    return p;
}

// Non-zero inputs among the R = 2^r0 inputs of a step-0 radix DFT: an LDE's
// first pass reads h = n / blowup rows, so inputs k >= R / blowup are zero.
inline int pass_knz(const PassArgs& a)
{
    const int r0 = a.s <= 3 ? (int)a.s : 3;
    const uint64_t n = 1ull << a.L;
    const uint64_t R = 1ull << r0;
    if (a.in_rows >= n || a.B != a.L) return (int)R;
    // rows j1 N2 + j2 < in_rows <=> j1 < in_rows / N2 (a power of two here)
    const uint64_t n2 = 1ull << (a.B - a.s);
    const uint64_t j1_nz = (a.in_rows + n2 - 1) / n2;  // j1 < j1_nz can be non-zero
    const uint64_t q_span = 1ull << (a.s - r0);
    uint64_t knz = (j1_nz + q_span - 1) / q_span;
    if (knz > R) knz = R;
    if (knz < 1) knz = 1;
    // round up to a power of two (template instances exist for 1, 2, 4, 8)
    uint64_t p2 = 1;
    while (p2 < knz) p2 <<= 1;
    return (int)p2;
}

// Arguments of pass i. Passes 0..np-2 read `in` (pass 0) or `tmp` and write
// `tmp` in place; the last pass reads `tmp` (or `in` when np == 1) and writes
// `out` in natural order. B is the block log-size entering pass i.
inline PassArgs pass_args(const Plan& p, uint32_t i, uint32_t B, uint64_t w, const uint64_t* in,
                          uint64_t in_rows, uint64_t* tmp, uint64_t* out, const uint64_t* tables,
                          bool inverse)
{
    PassArgs a;
    const uint64_t n = 1ull << p.L;
    const bool last = (i + 1 == p.np);
    a.in = i == 0 ? in : tmp;
    a.out = last ? out : tmp;
    a.in_rows = i == 0 ? in_rows : n;
    a.w = w;
    a.scale = last && inverse ? gl_inv(n % P) : 1;
    a.w512 = tab_w512(tables, inverse);
    a.twlo = tab_lo(tables, inverse);
    a.twhi = tab_hi(tables, inverse);
    a.in_len = (i == 0 ? in_rows : n) * w;
    a.out_len = n * w;
    a.L = p.L;
    a.B = B;
    a.s = p.sb[i];
    a.logC = p.logC;
    const uint32_t logN2 = B - a.s;
    uint32_t logJ = kNttLogV - p.logC;
    if (logJ > logN2) logJ = logN2;
    a.logJ = logJ;
    a.last = last ? 1 : 0;
    a.np = p.np;
    for (int k = 0; k < 8; k++) a.sb[k] = p.sb[k];
    const uint64_t N2 = 1ull << logN2;
    a.in_stride = (uint32_t)(N2 * w);
    a.out_stride = (uint32_t)((last ? (n >> a.s) : N2) * w);
    // Step 0 reads points j1 < KNZ 2^(s - r0) of each tile, i.e. rows below
    // KNZ 2^(s - r0) N2 (first pass, a single block); they all hold data unless
    // the input is shorter.
    const uint32_t r0 = a.s <= 3 ? a.s : 3;
    const uint64_t knz = (uint64_t)pass_knz(a);
    a.check_rows = (knz << (a.s - r0)) * N2 > a.in_rows ? 1 : 0;
    return a;
}

// The pass strides of a plan fit the 32-bit fields of PassArgs.
inline bool plan_fits(const Plan& p, uint64_t w)
{
    const uint64_t n = 1ull << p.L;
    return w < (1ull << 32) && (n / (1ull << p.sb[p.np - 1])) * w < (1ull << 32) &&
           (n >> p.sb[0]) * w < (1ull << 32);
}

// Prefix order (writer.rs:43-71): output word t of the committed matrix
// (E u64 per entry, rows i < 2^lrows, columns j < 2^k) reads word
// ((j 2^lrows + i) E + c) of the table; all in 64 bits (up to 2^33 words
// for a 32-variable EF table).
__host__ __device__ __forceinline__ uint64_t prefix_source(uint64_t t, uint32_t lrows, uint32_t k, uint32_t E)
{
    const uint64_t c = t % E, e = t / E;
    const uint64_t j = e & ((1ull << k) - 1), i = e >> k;
    return ((j << lrows) | i) * E + c;
}

// LDS of a pass: the N1 x V tile, the inter-pass twiddle table (kRoleTable)
// and the step twiddles, unless the sub-DFT is a single step.
inline size_t pass_lds_bytes(const PassArgs& a)
{
    if (a.s <= 3) return 0;
    size_t words = (size_t)1 << (a.s + a.logC + a.logJ);
    if (pass_uses_twtab(a)) words += (size_t)1 << a.s;
    words += kW512Words;
    return words * 8;
}

}  // namespace zk
