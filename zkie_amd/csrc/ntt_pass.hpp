// One four-step NTT pass, written as host/device functions so the same code
// runs in the HIP kernel and in the CPU emulator used by the tests (which
// executes each step for every thread of a workgroup in barrier order and
// checks every address against its buffer).
//
// Pass geometry: the array of n = 2^L rows is a set of blocks of N = 2^B
// rows. A workgroup owns block b, a tile of J = 2^logJ consecutive j2 values
// and a tile of C = 2^logC columns (V = C J vector lanes); it computes the
// N1 = 2^S point DFT over j1 of x[b N + j1 N2 + j2][c] (N2 = N / N1),
// multiplies output i1 by w_N^(i1 j2) and stores it at row b N + i1 N2 + j2
// (or, in the last pass where N2 = 1, at the natural row of b N1 + i1).
//
// The N1-point DFT runs as radix-8/4/2 decimation-in-frequency steps with
// the small DFTs in registers: step 0 reads its R inputs straight from HBM,
// intermediate steps exchange through LDS (in place, one barrier between
// steps), and the last step writes straight to HBM. Step t works on
// sub-problems of 2^BS points: for each (blk, q < 2^(BS - r), v) it loads the
// R = 2^r points q + k 2^(BS - r), computes their R-point DFT, multiplies
// frequency f by w_{2^BS}^(f q) and stores it at q + f 2^(BS - r). After the
// last step, position pos = f_0 2^(S - r_0) + f_1 2^(S - r_0 - r_1) + ... holds
// frequency i1 = f_0 + f_1 2^(r_0) + ... (mixed-radix digit reversal).
#pragma once

#include "gl64.hpp"

#if defined(ZK_EMU_BOUNDS)
#include <cstdio>
#include <cstdlib>
#define ZK_BOUND(idx, len)                                                                  \
    do {                                                                                    \
        if ((uint64_t)(idx) >= (uint64_t)(len)) {                                           \
            std::fprintf(stderr, "out of bounds %s:%d %llu >= %llu\n", __FILE__, __LINE__, \
                         (unsigned long long)(idx), (unsigned long long)(len));             \
            std::abort();                                                                   \
        }                                                                                   \
    } while (0)
#else
#define ZK_BOUND(idx, len) \
    do {                   \
    } while (0)
#endif

namespace zk {

constexpr int kStepTableLg = 9;  // in-pass twiddles come from w_512^k, k < 512

struct PassArgs {
    const uint64_t* in;
    uint64_t* out;
    uint64_t in_rows;  // rows of `in` holding data; rows beyond read as zero
    uint64_t w;
    uint64_t scale;        // last pass: multiply by this (1 = forward)
    const uint64_t* w512;  // w_512^k, k < 512 (forward or inverse)
    const uint64_t* twlo;  // w_{2^32}^x, x < 2^16
    const uint64_t* twhi;  // w_{2^32}^(x 2^16), x < 2^16
    uint64_t in_len, out_len;  // element counts, checked by the emulator only
    uint32_t L, B, s;
    uint32_t logC, logJ;
    uint32_t last;
    uint32_t np;
    uint32_t sb[8];
    uint32_t check_rows;  // step 0 may read rows >= in_rows (read as zero)
    uint32_t in_stride;   // elements between points j1 and j1 + 1 of a tile (N2 w)
    uint32_t out_stride;  // elements between frequencies i1 and i1 + 1 (N2 w, last pass 2^(L-s) w)
};

struct PassTile {
    uint64_t blk;  // first row of the block
    uint64_t c0;   // first column
    uint64_t j20;  // first j2
    uint64_t N2;
    uint64_t nat0;  // last pass: natural row of blk (frequency i1 adds i1 2^(L - s))
    uint32_t logV;
};

// What the last step of a pass does with each output (a compile-time choice,
// so that a pass carries no per-element branches):
//   kRoleTwiddle  non-last pass, w_N^(i1 j2) formed from the two-level table;
//   kRoleTable    non-last pass with one j2 per tile, w_N^(i1 j2) from LDS;
//   kRoleLast     last pass, natural row order, canonical output;
//   kRoleLastScale  the same, times the pass scale (1/n of an inverse DFT).
enum PassRole { kRoleTwiddle = 0, kRoleTable = 1, kRoleLast = 2, kRoleLastScale = 3 };

// The first pass of a zero-padded LDE (fewer than 8 non-zero step-0 inputs)
// reads its input once and writes 8 / KNZ times as much: its HBM loads and
// stores carry the non-temporal hint (ld_nt, st_nt), which measured faster
// there and not in the other passes.
template <int KNZ>
__host__ __device__ constexpr bool pass_streams()
{
    return KNZ < 8;
}

__host__ __device__ __forceinline__ uint32_t bit_reverse(uint32_t x, uint32_t bits)
{
    return bits ? (__builtin_bitreverse32(x) >> (32 - bits)) : 0u;
}

__host__ __device__ __forceinline__ uint64_t pass_blocks(const PassArgs& a)
{
    const uint32_t logN2 = a.B - a.s;
    return ((1ull << a.L) >> a.B) * ((1ull << logN2) >> a.logJ) * (a.w >> a.logC);
}

// Natural row of position pos after all passes: the digit of pass p (its
// s_p bits, taken from the top of pos) lands at bit s_0 + ... + s_(p-1).
__host__ __device__ __forceinline__ uint64_t pass_natural_row(const PassArgs& a, uint64_t pos)
{
    uint64_t nat = 0;
    uint32_t rem = a.L, shift_nat = 0;
    for (uint32_t p = 0; p < a.np; p++) {
        const uint32_t sp = a.sb[p];
        rem -= sp;
        nat |= ((pos >> rem) & ((1ull << sp) - 1)) << shift_nat;
        shift_nat += sp;
    }
    return nat;
}

__host__ __device__ __forceinline__ PassTile pass_tile(const PassArgs& a, uint64_t bid)
{
    PassTile t;
    t.N2 = 1ull << (a.B - a.s);
    const uint64_t CT = a.w >> a.logC;
    const uint64_t JT = t.N2 >> a.logJ;
    const uint64_t ct = bid % CT;
    bid /= CT;
    const uint64_t jt = bid % JT;
    const uint64_t b = bid / JT;
    t.blk = b << a.B;
    t.c0 = ct << a.logC;
    t.j20 = jt << a.logJ;
    t.logV = a.logC + a.logJ;
    t.nat0 = a.last ? pass_natural_row(a, t.blk) : 0;
    return t;
}

// w_{2^B}^e for e < 2^B.
__host__ __device__ __forceinline__ uint64_t pass_root_pow(const PassArgs& a, uint64_t e)
{
    const uint64_t E = e << (32 - a.B);
    return gl_mul(a.twlo[E & 0xFFFF], a.twhi[E >> 16]);
}

// Radix decomposition of an S-point sub-DFT: digits r_0, r_1, r_2 (bits).
template <int S>
struct Radix {
    static constexpr int n = S <= 3 ? 1 : (S <= 6 ? 2 : 3);
    static constexpr int r0 = S <= 3 ? S : 3;
    static constexpr int r1 = S <= 3 ? 0 : (S <= 6 ? S - 3 : (S == 7 ? 2 : 3));
    static constexpr int r2 = S - r0 - r1;
};
// S=9: 3,3,3  S=8: 3,3,2  S=7: 3,2,2  S=6: 3,3  S=5: 3,2  S=4: 3,1 ... all digits <= 3.

// Frequency of position pos for the digit sequence of Radix<S>.
template <int S>
__host__ __device__ __forceinline__ uint32_t digit_reverse(uint32_t pos)
{
    using Rd = Radix<S>;
    uint32_t f = 0, sh = 0, rem = S;
    rem -= Rd::r0;
    f |= ((pos >> rem) & ((1u << Rd::r0) - 1)) << sh;
    sh += Rd::r0;
    if (Rd::r1) {
        rem -= Rd::r1;
        f |= ((pos >> rem) & ((1u << Rd::r1) - 1)) << sh;
        sh += Rd::r1;
    }
    if (Rd::r2) {
        rem -= Rd::r2;
        f |= ((pos >> rem) & ((1u << Rd::r2) - 1)) << sh;
    }
    return f;
}

// Roots of unity inside the 8- and 4-point DFTs are signed powers of two:
// forward w4 = 2^48, w8 = -2^24, w8^3 = -2^72 = 2^-24; inverse w4 = -2^48,
// w8 = 2^72 = -2^-24, w8^3 = 2^24 (2^96 = -1). A butterfly output
// (u - v) w with w = -2^k is formed as (v - u) 2^k, so every twiddle inside
// a small DFT is a shift form (gl_mul_2e24, gl_mul_2e48, gl_mul_inv_pow2<24>).
template <bool INV, int P8>
__host__ __device__ __forceinline__ uint64_t dif_lower8(uint64_t u, uint64_t v)
{
    // lower output of a radix-2 butterfly of the 8-point DFT, twiddle w8^P8
    if (P8 == 0) return gl_sub2(u, v);
    if (!INV) {
        if (P8 == 1) return gl_mul_2e24(gl_sub2(v, u));         // -2^24
        if (P8 == 2) return gl_mul_2e48(gl_sub2(u, v));         //  2^48
        return gl_mul_inv_pow2<24>(gl_sub2(u, v));              //  2^-24
    } else {
        if (P8 == 1) return gl_mul_inv_pow2<24>(gl_sub2(v, u)); // -2^-24
        if (P8 == 2) return gl_mul_2e48(gl_sub2(v, u));         // -2^48
        return gl_mul_2e24(gl_sub2(u, v));                      //  2^24
    }
}

// In-register R-point DFT (radix-2 DIF); x[idx] ends up holding frequency
// bit_reverse(idx, log2 R). Inputs x[k] with k >= NZ are known to be zero
// (the zero padding of an LDE): they enter as literal zeros, so that the
// butterflies they reach fold away at compile time.
template <int RLOG, bool INV, int NZ = (1 << RLOG)>
__host__ __device__ __forceinline__ void dft_small(uint64_t* x)
{
    if (RLOG == 3) {
        const uint64_t a0 = x[0], a1 = NZ > 1 ? x[1] : 0, a2 = NZ > 2 ? x[2] : 0, a3 = NZ > 3 ? x[3] : 0;
        const uint64_t a4 = NZ > 4 ? x[4] : 0, a5 = NZ > 5 ? x[5] : 0, a6 = NZ > 6 ? x[6] : 0,
                       a7 = NZ > 7 ? x[7] : 0;
        const uint64_t b0 = gl_add(a0, a4), b1 = gl_add(a1, a5), b2 = gl_add(a2, a6), b3 = gl_add(a3, a7);
        const uint64_t b4 = dif_lower8<INV, 0>(a0, a4), b5 = dif_lower8<INV, 1>(a1, a5);
        const uint64_t b6 = dif_lower8<INV, 2>(a2, a6), b7 = dif_lower8<INV, 3>(a3, a7);
        const uint64_t c0 = gl_add(b0, b2), c1 = gl_add(b1, b3);
        const uint64_t c2 = dif_lower8<INV, 0>(b0, b2), c3 = dif_lower8<INV, 2>(b1, b3);  // w4 = w8^2
        const uint64_t c4 = gl_add(b4, b6), c5 = gl_add(b5, b7);
        const uint64_t c6 = dif_lower8<INV, 0>(b4, b6), c7 = dif_lower8<INV, 2>(b5, b7);
        x[0] = gl_add(c0, c1);
        x[1] = gl_sub2(c0, c1);
        x[2] = gl_add(c2, c3);
        x[3] = gl_sub2(c2, c3);
        x[4] = gl_add(c4, c5);
        x[5] = gl_sub2(c4, c5);
        x[6] = gl_add(c6, c7);
        x[7] = gl_sub2(c6, c7);
    } else if (RLOG == 2) {
        const uint64_t a0 = x[0], a1 = NZ > 1 ? x[1] : 0, a2 = NZ > 2 ? x[2] : 0, a3 = NZ > 3 ? x[3] : 0;
        const uint64_t b0 = gl_add(a0, a2), b1 = gl_add(a1, a3);
        const uint64_t b2 = dif_lower8<INV, 0>(a0, a2), b3 = dif_lower8<INV, 2>(a1, a3);
        x[0] = gl_add(b0, b1);
        x[1] = gl_sub2(b0, b1);
        x[2] = gl_add(b2, b3);
        x[3] = gl_sub2(b2, b3);
    } else if (RLOG == 1) {
        const uint64_t u = x[0], v = NZ > 1 ? x[1] : 0;
        x[0] = gl_add(u, v);
        x[1] = gl_sub2(u, v);
    }
}

// Per-thread addressing of a pass, fixed for all its items: a thread always
// serves the same vector lane v (the thread count is a multiple of V), so the
// element index of point j1 is in_base + j1 in_stride and that of frequency i1
// is out_base + i1 out_stride.
struct PassLane {
    uint32_t v;
    uint64_t in_base, out_base;
    uint32_t pos_lim;  // step 0: points j1 >= pos_lim lie beyond in_rows
    uint64_t j2;
};

__host__ __device__ __forceinline__ PassLane pass_lane(const PassArgs& a, const PassTile& t, uint32_t tid)
{
    PassLane l;
    l.v = tid & ((1u << t.logV) - 1);
    const uint64_t c = t.c0 + (l.v & ((1u << a.logC) - 1));
    l.j2 = t.j20 + (l.v >> a.logC);
    const uint64_t row0 = t.blk + l.j2;  // row of point 0
    l.in_base = row0 * a.w + c;
    l.out_base = (a.last ? t.nat0 : row0) * a.w + c;
    const uint32_t logN2 = a.B - a.s;
    if (row0 >= a.in_rows)
        l.pos_lim = 0;
    else {
        const uint64_t lim = ((a.in_rows - row0) + t.N2 - 1) >> logN2;
        l.pos_lim = lim > (1ull << a.s) ? (1u << a.s) : (uint32_t)lim;
    }
    return l;
}

// Items of a step (one per sub-problem q and vector lane): item `it` works
// on the points base + k 2^(BS - RL) of its block.
template <int RL, int BS>
__host__ __device__ __forceinline__ void step_item(uint32_t it, uint32_t logV, uint32_t& base, uint32_t& q)
{
    constexpr int QL = BS - RL;
    const uint32_t rest = it >> logV;
    q = rest & ((1u << QL) - 1);
    base = ((rest >> QL) << BS) + q;
}

// A thread takes U items per round and issues all their reads before any
// arithmetic, so that U * R reads are in flight per thread.
constexpr int kStepU = 2;

// Reads of one round of a radix-2^RL DIF step on sub-problems of 2^BS points
// of an S-point DFT: the R points of items it0 and it0 + T into x.
// FROM_GLOBAL: from HBM (step 0; only the first KNZ of the R inputs can be
// non-zero, the rest are the zero padding of an LDE), else from the LDS tile.
// LOGV is the tile's log2 vector width when known at compile time (then LDS
// addresses are a base plus immediate offsets), or -1 to read it from the tile.
// ROWS (FROM_GLOBAL): kRowsAll when every input row exists (a.check_rows
// clear), kRowsChecked when rows past the input read as zero, kRowsAny to
// decide at run time.
enum { kRowsAny = 0, kRowsAll = 1, kRowsChecked = 2 };

template <int S, int RL, int BS, int KNZ, bool FROM_GLOBAL, int LOGV, int ROWS = kRowsAny>
__host__ __device__ __forceinline__ void step_gather(const PassArgs& a, const PassTile& t, const PassLane& l,
                                                     uint32_t it0, uint32_t T, const uint64_t* lds,
                                                     uint64_t (&x)[kStepU][1 << RL])
{
    constexpr int R = 1 << RL;
    constexpr int QL = BS - RL;
    const uint32_t logV = LOGV >= 0 ? (uint32_t)LOGV : t.logV;
    const uint32_t items = (1u << (S - RL)) << logV;
    const uint32_t v = l.v;
    if (FROM_GLOBAL && ROWS != kRowsChecked && (ROWS == kRowsAll || !a.check_rows)) {
        // Every input row exists: straight-line loads with no branch or
        // select after them, so that a later wait for an older load (the
        // LDS tables) can leave the whole tile in flight.
#pragma unroll
        for (int u = 0; u < kStepU; u++) {
            const uint32_t it = it0 + (uint32_t)u * T;
            if (it >= items) continue;
            uint32_t base, q;
            step_item<RL, BS>(it, logV, base, q);
            const uint64_t gbase = l.in_base + (uint64_t)base * a.in_stride;
#pragma unroll
            for (int k = 0; k < R; k++) {
                if (k < KNZ) {
                    const uint64_t idx = gbase + (uint64_t)((uint32_t)k << QL) * a.in_stride;
                    ZK_BOUND(idx, a.in_len);
                    x[u][k] = pass_streams<KNZ>() ? ld_nt(a.in + idx) : a.in[idx];
                } else {
                    x[u][k] = 0;
                }
            }
        }
        return;
    }
#pragma unroll
    for (int u = 0; u < kStepU; u++) {
        const uint32_t it = it0 + (uint32_t)u * T;
        if (it >= items) continue;
        uint32_t base, q;
        step_item<RL, BS>(it, logV, base, q);
        const uint64_t gbase = l.in_base + (uint64_t)base * a.in_stride;
        const uint32_t lbase = (base << logV) | v;
#pragma unroll
        for (int k = 0; k < R; k++) {
            const uint32_t pos = base + ((uint32_t)k << QL);
            if (FROM_GLOBAL) {
                if (k < KNZ) {
                    // A row past the input reads element 0 and keeps 0: the
                    // same number of loads as the straight-line form above.
                    const bool in = pos < l.pos_lim;
                    const uint64_t idx = in ? gbase + (uint64_t)((uint32_t)k << QL) * a.in_stride : 0;
                    ZK_BOUND(idx, a.in_len);
                    const uint64_t val = pass_streams<KNZ>() ? ld_nt(a.in + idx) : a.in[idx];
                    x[u][k] = in ? val : 0;
                } else {
                    x[u][k] = 0;
                }
            } else {
                const uint32_t li = lbase + (((uint32_t)k << QL) << logV);
                ZK_BOUND(li, (1u << S) << logV);
                x[u][k] = lds[li];
            }
        }
    }
}

// The rest of the round: R-point DFT of each item, step twiddles
// w_{2^BS}^(f q) from the LDS table wtab (w_512^k), then the outputs to the
// LDS tile or, in the last step (TO_GLOBAL), with the pass role's treatment
// to HBM.
template <int S, int RL, int BS, bool INV, bool TO_GLOBAL, int ROLE, int LOGV, int NZ = (1 << RL),
          bool STREAM = false>
__host__ __device__ __forceinline__ void step_finish(const PassArgs& a, const PassTile& t, const PassLane& l,
                                                     uint32_t it0, uint32_t T, uint64_t* lds,
                                                     const uint64_t* wtab, const uint64_t* twtab,
                                                     uint64_t (&x)[kStepU][1 << RL])
{
    constexpr int R = 1 << RL;
    constexpr int QL = BS - RL;
    const uint32_t logV = LOGV >= 0 ? (uint32_t)LOGV : t.logV;
    const uint32_t items = (1u << (S - RL)) << logV;
    const uint32_t v = l.v;
#pragma unroll
    for (int u = 0; u < kStepU; u++) {
        const uint32_t it = it0 + (uint32_t)u * T;
        if (it >= items) continue;
        uint32_t base, q;
        step_item<RL, BS>(it, logV, base, q);
        uint64_t tw[R];
        if (QL > 0) {
#pragma unroll
            for (int idx = 1; idx < R; idx++) {
                const uint32_t f = bit_reverse((uint32_t)idx, RL);
                const uint32_t wi = (f * q) << (kStepTableLg - BS);
                ZK_BOUND(wi, 1u << kStepTableLg);
                tw[idx] = wtab[wi];
            }
        }
        dft_small<RL, INV, (NZ < (1 << RL) ? NZ : (1 << RL))>(x[u]);
        if (QL > 0) {
            if constexpr (NZ >= (1 << RL)) {
                // independent products in interleaved pairs (each fills the
                // other's wait states)
#pragma unroll
                for (int idx = 1; idx + 1 < R; idx += 2)
                    gl_mul2(x[u][idx], tw[idx], x[u][idx + 1], tw[idx + 1], x[u][idx], x[u][idx + 1]);
                if ((R - 1) % 2) x[u][R - 1] = gl_mul(x[u][R - 1], tw[R - 1]);
            } else {
                // a pruned step 0 (zero inputs): its products one by one,
                // which measured faster in the LDE's first pass
#pragma unroll
                for (int idx = 1; idx < R; idx++) x[u][idx] = gl_mul(x[u][idx], tw[idx]);
            }
        }
        if (TO_GLOBAL) {
            // QL == 0 here: base holds the leading digits, f the last one,
            // which digit reversal moves to the top of i1.
            const uint32_t i1b = digit_reverse<S>(base);
            const uint64_t obase = l.out_base + (uint64_t)i1b * a.out_stride;
#pragma unroll
            for (int idx = 0; idx < R; idx++) {
                const uint32_t f = bit_reverse((uint32_t)idx, RL);
                const uint32_t fi = f << (S - RL);
                const uint32_t i1 = i1b + fi;
                uint64_t val = x[u][idx];
                if (ROLE == kRoleTable) {
                    // w_N^(i1 j2) for the tile's single j2, each product
                    // stored as soon as it is formed (pairing these measured
                    // slower in the LDE's first pass)
                    ZK_BOUND(i1, 1u << a.s);
                    val = gl_mul(val, twtab[i1]);
                } else if (ROLE == kRoleTwiddle) {
                    const uint64_t ex = (uint64_t)i1 * l.j2;
                    if (ex) val = gl_mul(val, pass_root_pow(a, ex));
                } else {
                    if (ROLE == kRoleLastScale) val = gl_mul(val, a.scale);
                    val = gl_canon(val);
                }
                const uint64_t oidx = obase + (uint64_t)fi * a.out_stride;
                ZK_BOUND(oidx, a.out_len);
                if (STREAM)
                    st_nt(a.out + oidx, val);
                else
                    a.out[oidx] = val;
            }
        } else {
            const uint32_t lbase = (base << logV) | v;
#pragma unroll
            for (int idx = 0; idx < R; idx++) {
                const uint32_t f = bit_reverse((uint32_t)idx, RL);
                const uint32_t li = lbase + ((f << QL) << logV);
                ZK_BOUND(li, (1u << S) << logV);
                lds[li] = x[u][idx];
            }
        }
    }
}

// One radix-2^RL DIF step: every round of gather + finish.
template <int S, int RL, int BS, int KNZ, bool INV, bool FROM_GLOBAL, bool TO_GLOBAL, int ROLE, int LOGV,
          bool STREAM = pass_streams<KNZ>()>
__host__ __device__ __forceinline__ void ntt_step(const PassArgs& a, const PassTile& t, const PassLane& l,
                                                  uint32_t tid, uint32_t T, uint64_t* lds, const uint64_t* wtab,
                                                  const uint64_t* twtab)
{
    const uint32_t logV = LOGV >= 0 ? (uint32_t)LOGV : t.logV;
    const uint32_t items = (1u << (S - RL)) << logV;
    for (uint32_t it0 = tid; it0 < items; it0 += kStepU * T) {
        uint64_t x[kStepU][1 << RL];
        step_gather<S, RL, BS, KNZ, FROM_GLOBAL, LOGV>(a, t, l, it0, T, lds, x);
        step_finish<S, RL, BS, INV, TO_GLOBAL, ROLE, LOGV, FROM_GLOBAL ? KNZ : 8, STREAM>(a, t, l, it0, T, lds,
                                                                                      wtab, twtab, x);
    }
}

// Number of barrier-separated steps of an S-point sub-DFT.
template <int S>
constexpr int pass_steps()
{
    return Radix<S>::n;
}

// Whether the pass keeps a table of its inter-pass twiddles in LDS: a
// multi-step, non-last pass whose tile holds a single j2 (J = 1). Then every
// output i1 is multiplied by w_N^(i1 j2) with the same j2, and the 2^S powers
// are formed once per workgroup after the tile data (LDS words
// [2^S V, 2^S V + 2^S)).
__host__ __device__ __forceinline__ bool pass_uses_twtab(const PassArgs& a)
{
    return a.s > 3 && !a.last && a.logJ == 0;
}

// LDS words of a multi-step pass: the 2^S x V tile, the inter-pass twiddle
// table (kRoleTable), then the step twiddles w_512^k (kW512Words).
constexpr uint32_t kW512Words = 1u << kStepTableLg;
template <int S, int ROLE>
__host__ __device__ __forceinline__ uint32_t pass_wtab_offset(uint32_t logV)
{
    return ((1u << S) << logV) + (ROLE == kRoleTable ? (1u << S) : 0u);
}

// The inter-pass table of a kRoleTable tile, tab[i] = w_N^(i j2) for
// i < 2^S, is formed as lo[i mod 32] hi[i / 32] from two small power tables
// (lo[k] = w_N^(k j2), hi[m] = w_N^(32 m j2)), so a workgroup reads 2 (32 +
// 2^(S-5)) entries of the two-level root table instead of 2^(S+1), which
// the streaming codeword would evict from L2 between workgroups. The small
// tables sit at the start of the tile region, which step 0 writes only after
// the inter-pass table is formed (a barrier separates the two).
constexpr uint32_t kTabLoLg = 5;
template <int S>
__host__ __device__ __forceinline__ constexpr uint32_t pass_tab_lo_lg()
{
    return S <= (int)kTabLoLg ? (uint32_t)S - 1 : kTabLoLg;
}

// Before step 0, first half (a barrier follows): the step twiddles w_512^k
// into LDS and, for kRoleTable, the two small power tables. Entry i comes
// from pass_tables_fetch (its HBM words) and pass_tables_put (the LDS
// write), so that a kernel with a thread per entry can issue these loads
// before its tile's and write the tables while the tile is still in flight.
struct PassTabFetch {
    uint64_t w;       // w_512^i
    uint64_t r0, r1;  // the two root-table factors of small-table entry i (1, 1 for w^0 or none)
};

template <int S, int ROLE>
__host__ __device__ __forceinline__ PassTabFetch pass_tables_fetch(const PassArgs& a, const PassTile& t,
                                                                   uint32_t i)
{
    // No branch around the loads (entries past the tables read w^0 = lo[0]
    // hi[0] = 1), so a kernel's later wait for them can leave its tile's
    // loads in flight.
    PassTabFetch f{0, 1, 1};
    if (S <= 3) return f;
    if (i < kW512Words) f.w = a.w512[i];
    if (ROLE == kRoleTable) {
        constexpr uint32_t LO = pass_tab_lo_lg<S>();
        constexpr uint32_t nlo = 1u << LO, nhi = 1u << (S - LO);
        const uint64_t ex =
            i < nlo + nhi ? (i < nlo ? (uint64_t)i : (uint64_t)(i - nlo) << LO) * t.j20 : 0;
        const uint64_t E = ex << (32 - a.B);  // w_{2^B}^ex = lo[E mod 2^16] hi[E >> 16]
        f.r0 = a.twlo[E & 0xFFFF];
        f.r1 = a.twhi[E >> 16];
    }
    return f;
}

template <int S, int ROLE>
__host__ __device__ __forceinline__ void pass_tables_put(const PassTabFetch& f, const PassTile& t, uint32_t i,
                                                         uint64_t* lds)
{
    if (S <= 3) return;
    if (i < kW512Words) lds[pass_wtab_offset<S, ROLE>(t.logV) + i] = f.w;
    if (ROLE == kRoleTable) {
        constexpr uint32_t LO = pass_tab_lo_lg<S>();
        constexpr uint32_t nlo = 1u << LO, nhi = 1u << (S - LO);
        static_assert(S <= 3 || nlo + nhi <= (1u << S), "small tables fit the tile region");
        if (i < nlo + nhi) lds[i] = gl_mul(f.r0, f.r1);  // [lo | hi], in the tile region
    }
}

// Entries needed per workgroup (a thread per entry in the kernel).
template <int S, int ROLE>
__host__ __device__ __forceinline__ constexpr uint32_t pass_table_entries()
{
    return ROLE == kRoleTable && (1u << S) > kW512Words ? (1u << S) : kW512Words;
}

template <int S, int ROLE>
__host__ __device__ __forceinline__ void pass_tables(const PassArgs& a, const PassTile& t, uint32_t tid,
                                                     uint32_t T, uint64_t* lds)
{
    if (S <= 3) return;
    for (uint32_t i = tid; i < pass_table_entries<S, ROLE>(); i += T)
        pass_tables_put<S, ROLE>(pass_tables_fetch<S, ROLE>(a, t, i), t, i, lds);
}

// Before step 0, second half (after a barrier; a barrier separates it from
// the last step, the reader): tab[i] = lo[i mod 2^LO] hi[i >> LO].
template <int S, int ROLE>
__host__ __device__ __forceinline__ void pass_tables_tab(const PassTile& t, uint32_t tid, uint32_t T,
                                                         uint64_t* lds)
{
    if (ROLE != kRoleTable || S <= 3) return;
    constexpr uint32_t LO = pass_tab_lo_lg<S>();
    const uint64_t* small = lds;
    uint64_t* tab = lds + ((1u << S) << t.logV);
    for (uint32_t i = tid; i < (1u << S); i += T)
        tab[i] = gl_mul(small[i & ((1u << LO) - 1)], small[(1u << LO) + (i >> LO)]);
}

// Step `k` of the S-point sub-DFT (k < pass_steps<S>()). The caller puts a
// workgroup barrier between consecutive steps.
template <int S, int KNZ, bool INV, int ROLE, int LOGV>
__host__ __device__ __forceinline__ void pass_step(int k, const PassArgs& a, const PassTile& t,
                                                   const PassLane& l, uint32_t tid, uint32_t T,
                                                   uint64_t* lds)
{
    using Rd = Radix<S>;
    constexpr int n = Rd::n;
    const uint64_t* tab = ROLE == kRoleTable ? lds + ((1u << S) << t.logV) : nullptr;
    const uint64_t* wtab = lds + pass_wtab_offset<S, ROLE>(t.logV);
    if (k == 0) {
        if (n == 1)
            ntt_step<S, Rd::r0, S, KNZ, INV, true, true, ROLE, LOGV>(a, t, l, tid, T, lds, wtab, nullptr);
        else
            ntt_step<S, Rd::r0, S, KNZ, INV, true, false, ROLE, LOGV>(a, t, l, tid, T, lds, wtab, nullptr);
    } else if (k == 1) {
        if (n == 2)
            ntt_step<S, Rd::r1, S - Rd::r0, 8, INV, false, true, ROLE, LOGV, pass_streams<KNZ>()>(a, t, l, tid, T,
                                                                                                   lds, wtab, tab);
        else if (n == 3)
            ntt_step<S, Rd::r1, S - Rd::r0, 8, INV, false, false, ROLE, LOGV>(a, t, l, tid, T, lds, wtab, nullptr);
    } else if (k == 2) {
        if (n == 3)
            ntt_step<S, Rd::r2, Rd::r2, 8, INV, false, true, ROLE, LOGV, pass_streams<KNZ>()>(a, t, l, tid, T, lds,
                                                                                              wtab, tab);
    }
}

// Step 0 of a multi-step pass in two halves, so that a kernel can issue its
// HBM reads before the LDS tables are filled: the reads of all items (one
// round: 2^(S - r0) V <= kStepU T) and, after a barrier, the rest.
template <int S, int KNZ, int LOGV, int ROWS = kRowsAny>
__host__ __device__ __forceinline__ void pass_step0_gather(const PassArgs& a, const PassTile& t,
                                                           const PassLane& l, uint32_t tid, uint32_t T,
                                                           uint64_t (&x)[kStepU][1 << Radix<S>::r0])
{
    step_gather<S, Radix<S>::r0, S, KNZ, true, LOGV, ROWS>(a, t, l, tid, T, nullptr, x);
}

template <int S, int KNZ, bool INV, int ROLE, int LOGV>
__host__ __device__ __forceinline__ void pass_step0_finish(const PassArgs& a, const PassTile& t,
                                                           const PassLane& l, uint32_t tid, uint32_t T,
                                                           uint64_t* lds,
                                                           uint64_t (&x)[kStepU][1 << Radix<S>::r0])
{
    static_assert(Radix<S>::n > 1, "a single-step pass writes HBM from step 0");
    const uint64_t* wtab = lds + pass_wtab_offset<S, ROLE>(t.logV);
    step_finish<S, Radix<S>::r0, S, INV, false, ROLE, LOGV, KNZ>(a, t, l, tid, T, lds, wtab, nullptr, x);
}

// Role of a pass (see PassRole).
__host__ __device__ __forceinline__ int pass_role(const PassArgs& a)
{
    if (a.last) return a.scale != 1 ? kRoleLastScale : kRoleLast;
    return pass_uses_twtab(a) ? kRoleTable : kRoleTwiddle;
}

}  // namespace zk
