// Poseidon2-Goldilocks-16 on CDNA4: one permutation per lane, state in 16
// u64 registers. Restates poseidon2_merkle.cu:37-155 (the reference device
// permutation that mirrors p3-poseidon2 / p3-goldilocks 0.7.0):
//   initial mds_light16, 4 external rounds (rc, x^7 on all lanes,
//   mds_light16), 22 internal rounds (rc and x^7 on lane 0, then
//   st_i = sum + V_i st_i), 4 external rounds.
// V = [-2, 1, 2, 1/2, 3, 4, -1/2, -3, -4, 1/2^3, 1/2^4, 1/2^5, -1/2^3,
//      -1/2^4, -1/2^5, diag15] (poseidon2_merkle.cu:111-142).
//
// MI355X choices:
//  * round constants sit in __constant__ memory indexed by wave-uniform
//    loop counters, so the compiler reads them with scalar loads into SGPRs
//    and every VALU op takes them as a scalar operand;
//  * the linear layers work on the 32-bit halves of the state as exact
//    64-bit sums (one v_mad_u64_u32 per term) and reduce once per output,
//    folding the next round's constants into that same reduction;
//  * corrections that a lane needs only with probability about 2^-32 (the
//    multiply's final borrow, second wraps, the linear-layer folds) run
//    behind wave-uniform branches (gl64.hpp);
//  * the external layer is M4 (x_g + S) per group of four words, S the sum of
//    the four groups (mds_light16 = circ(2 M4, M4, M4, M4));
//  * the internal diagonal is applied without multiplies: every output of an
//    internal round is an exact sum of 32-bit halves built on the unreduced
//    round sum (2^-k splits x into x >> k and the shifted-out bits, -v x uses
//    the complement ~x), and the constant that the next step adds to a word
//    (the next round's rc0, or the terminal round's constants after the last
//    internal round) joins those sums instead of a separate modular add;
//  * round loops stay rolled (one copy of the external round body) to keep
//    the code inside the instruction cache.
#pragma once

#include "gl64.hpp"

namespace zk {

struct P2Consts {
    uint64_t ext[8][16];  // [0..4) initial, [4..8) terminal external rounds
    uint64_t internal[22];
    uint64_t diag15;
    uint64_t diag[16];  // the whole internal diagonal V (p2_set_diag)
};

// V = [-2, 1, 2, 1/2, 3, 4, -1/2, -3, -4, 1/2^3, 1/2^4, 1/2^5, -1/2^3,
// -1/2^4, -1/2^5, diag15] (poseidon2_merkle.cu:111-142), canonical.
inline void p2_set_diag(P2Consts& c)
{
    const uint64_t i2 = gl_inv(2), i8 = gl_inv(8), i16 = gl_inv(16), i32 = gl_inv(32);
    const uint64_t V[16] = {P - 2, 1, 2, i2, 3, 4, P - i2, P - 3, P - 4, i8, i16, i32, P - i8, P - i16, P - i32,
                            gl_canon(c.diag15)};
    for (int i = 0; i < 16; i++) c.diag[i] = V[i];
}

__host__ __device__ __forceinline__ uint64_t sbox7(uint64_t x)
{
    const uint64_t x2 = gl_sqr(x);
    uint64_t x3, x4;
    gl_mul2(x2, x, x2, x2, x3, x4);
    return gl_mul(x3, x4);
}

// x^7 and y^7, the two addition chains interleaved product by product.
__host__ __device__ __forceinline__ void sbox7_2(uint64_t& x, uint64_t& y)
{
    uint64_t x2, y2, x3, y3, x4, y4;
    gl_mul2(x, x, y, y, x2, y2);
    gl_mul2(x2, x, y2, y, x3, y3);
    gl_mul2(x2, x2, y2, y2, x4, y4);
    gl_mul2(x3, x4, y3, y4, x, y);
}

// mat4 = [2 3 1 1; 1 2 3 1; 1 1 2 3; 3 1 1 2] (the addition chain of
// poseidon2_merkle.cu:63-76) on one 32-bit half of four lanes, into 64-bit
// sums (coefficients 1, 2, 3, so no sum can carry).
__host__ __device__ __forceinline__ void mat4_half(uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3,
                                                   uint64_t* y)
{
    const uint64_t t01 = acc32m<1>(x0, x1);
    const uint64_t t23 = acc32m<1>(x2, x3);
    const uint64_t t0123 = t01 + t23;
    const uint64_t t01123 = acc32m<1>(t0123, x1);
    const uint64_t t01233 = acc32m<1>(t0123, x3);
    y[3] = acc32m<2>(t01233, x0);  // 3x0 + x1 + x2 + 2x3
    y[1] = acc32m<2>(t01123, x2);  // x0 + 2x1 + 3x2 + x3
    y[0] = t01123 + t01;           // 2x0 + 3x1 + x2 + x3
    y[2] = t01233 + t23;           // x0 + x1 + 2x2 + 3x3
}

// mat4 on 64-bit sums (used on the column sums of the four lane groups).
__host__ __device__ __forceinline__ void mat4_wide(const uint64_t* x, uint64_t* y)
{
    const uint64_t t01 = x[0] + x[1];
    const uint64_t t23 = x[2] + x[3];
    const uint64_t t0123 = t01 + t23;
    const uint64_t t01123 = t0123 + x[1];
    const uint64_t t01233 = t0123 + x[3];
    y[3] = t01233 + (x[0] << 1);  // 3x0 + x1 + x2 + 2x3
    y[1] = t01123 + (x[2] << 1);  // x0 + 2x1 + 3x2 + x3
    y[0] = t01123 + t01;          // 2x0 + 3x1 + x2 + x3
    y[2] = t01233 + t23;          // x0 + x1 + 2x2 + 3x3
}

// st <- mds_light16(st) (+ constants). mds_light16 is circ(2 M4, M4, M4, M4):
// output group g is M4 x_g + sum_h M4 x_h = M4 (x_g + S) with S the sum of
// the four groups (M4 is linear), so the column sums S come first and each
// group is then z = x_g + S and M4 z, written on its own (only one group's
// intermediate sums are live at a time). Both 32-bit halves of the state go
// through the layer as exact 64-bit sums (z below 5 2^32, M4 z below 35 2^32
// plus a constant's half), and each output is reduced once from its two
// sums. RC: kRcNone, kRcAll (rc[i] added to word i), kRcLane0 (rc[0] added
// to word 0 only, the constant of the first internal round). GROUPS selects
// the output groups of four words that are formed (bit g: words 4g..4g+3);
// the other words are left holding their inputs, for a caller that never
// reads them (the last layer of a permutation whose caller keeps only the
// digest, or only the capacity before the next absorb overwrites the rate).
// RC64: every constant is below kRcLimit, so it joins the low sum whole
// (A < 2^38 there, so A + rc cannot carry) instead of as two halves.
enum { kRcNone = 0, kRcAll = 1, kRcLane0 = 2 };
enum { kOutAll = 0xF, kOutDigest = 0x3, kOutCapacity = 0xC };
constexpr uint64_t kRcLimit = 0xFFFFFFC000000000ull;  // 2^64 - 2^38

template <int RC, int GROUPS = kOutAll, bool RC64 = false>
__host__ __device__ __forceinline__ void mds_light16_rc(uint64_t* st, const uint64_t* rc)
{
    uint64_t sl[4], sh[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        sl[k] = acc32(acc32(acc32m<1>((uint32_t)st[k], (uint32_t)st[4 + k]), (uint32_t)st[8 + k]),
                      (uint32_t)st[12 + k]);
        sh[k] = acc32(acc32(acc32m<1>((uint32_t)(st[k] >> 32), (uint32_t)(st[4 + k] >> 32)),
                            (uint32_t)(st[8 + k] >> 32)),
                      (uint32_t)(st[12 + k] >> 32));
    }
    uint64_t w[16];  // lanes whose output still needs + eps (one shared rare branch)
#pragma unroll
    for (int j = 0; j < 16; j += 4) {
        if (!((GROUPS >> (j >> 2)) & 1)) continue;
        uint64_t zl[4], zh[4], yl[4], yh[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            zl[k] = acc32(sl[k], (uint32_t)st[j + k]);
            zh[k] = acc32(sh[k], (uint32_t)(st[j + k] >> 32));
        }
        mat4_wide(zl, yl);
        mat4_wide(zh, yh);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint64_t A = yl[k], B = yh[k];
            if (RC == kRcAll || (RC == kRcLane0 && j + k == 0)) {
                if (RC64) {
                    A += rc[j + k];
                } else {
                    A = acc32s(A, (uint32_t)rc[j + k]);
                    B = acc32s(B, (uint32_t)(rc[j + k] >> 32));
                }
            }
            st[j + k] = gl_from_halves_defer(A, B, w[j + k]);
        }
    }
    uint64_t any = 0;
#pragma unroll
    for (int i = 0; i < 16; i++)
        if ((GROUPS >> (i >> 2)) & 1) any |= w[i];
    if (__builtin_expect(any != 0, 0)) {
#pragma unroll
        for (int i = 0; i < 16; i++)
            if ((GROUPS >> (i >> 2)) & 1) gl_fold_eps(st[i], w[i]);
    }
}

template <bool ADD_RC>
__host__ __device__ __forceinline__ void mds_light16(uint64_t* st, const uint64_t* rc)
{
    mds_light16_rc<ADD_RC ? kRcAll : kRcNone>(st, rc);
}

// One internal round on a state whose word 0 already includes the round's
// constant: st0 <- st0^7, then st_i <- sum + V_i st_i. The round sum is kept
// as two 64-bit sums of 32-bit halves, SL + SH 2^32 (one v_mad_u64_u32 per
// half, never reduced), and every output is an exact sum of halves
// A + B 2^32 (A, B below 2^38) reduced once, with the final fold of all of
// them deferred to one shared rare branch. With ~x = 2^64 - 1 - x, q = x >> k
// and m = (x mod 2^k) 2^(32-k):
//   V = 1, 2, 3, 4:  A = SL + V x.lo,             B = SH + V x.hi;
//   V = -v (v = 2, 3, 4): -v x = v ~x - v (eps - 1) and -v (eps - 1) =
//                    (2^32 - 1 - v) 2^32 + 1 + 2v (mod p), so
//                    A = SL + 1 + 2v + v ~x.lo,   B = SH + 2^32 - 1 - v + v ~x.hi;
//   V = 2^-k (k = 1, 3, 4, 5, 32): x 2^-k = q - m eps = q + m + ~m 2^32 + 1, so
//                    A = SL + 1 + q.lo + m,       B = SH + q.hi + ~m;
//   V = -2^-k (k = 1, 3, 4, 5): -x 2^-k = m eps - q = (~m + ~q.lo + 3) +
//                    (m + ~q.hi - 2) 2^32 (mod p), and ~q.hi - 2 = ~(q.hi + 2), so
//                    A = SL + 3 + ~m + ~q.lo,     B = SH + m + ~(q.hi + 2);
//   V = diag15 otherwise: y = x15 diag15, A = SL + y.lo, B = SH + y.hi.
// The next round's constant rc0_next joins the sums of word 0 (its only
// use is the next S-box input); the constant parts of the A and B addends
// are formed on the scalar unit. (Folding the terminal round's constants
// into all sixteen outputs of the last round as well keeps sixteen more
// constants live and makes the leaf kernels spill registers.)
template <int K>
__host__ __device__ __forceinline__ void inv_pow2_pos(uint64_t x, uint64_t SL, uint64_t SH, uint64_t& A, uint64_t& B)
{
    const uint64_t q = x >> K;
    const uint32_t m = (uint32_t)x << (32 - K);
    A = acc32(acc32(SL + 1, (uint32_t)q), m);
    B = acc32(acc32(SH, (uint32_t)(q >> 32)), ~m);
}

template <int K>
__host__ __device__ __forceinline__ void inv_pow2_neg(uint64_t x, uint64_t SL, uint64_t SH, uint64_t& A, uint64_t& B)
{
    const uint64_t q = x >> K;
    const uint32_t m = (uint32_t)x << (32 - K);
    A = acc32(acc32(SL + 3, ~m), ~(uint32_t)q);
    B = acc32(acc32(SH, m), ~((uint32_t)(q >> 32) + 2u));
}

template <bool DIAG15_IS_INV_2_32, bool TERM = false>
__host__ __device__ __forceinline__ void internal_round_core(uint64_t* st, uint64_t rc0_next, uint64_t diag15,
                                                             const uint64_t* term = nullptr)
{
    uint64_t SL = (uint32_t)st[1], SH = st[1] >> 32;
#pragma unroll
    for (int i = 2; i < 16; i++) {
        SL = acc32(SL, (uint32_t)st[i]);
        SH = acc32(SH, (uint32_t)(st[i] >> 32));
    }
    const uint64_t x0 = sbox7(st[0]);
    SL = acc32(SL, (uint32_t)x0);
    SH = acc32(SH, (uint32_t)(x0 >> 32));
    // the constant added to output i: the next round's rc0 on word 0, or
    // (TERM, the last internal round on the fast path) the first terminal
    // round's constant term[i] on every word, whole in the low sum
    auto cl = [&](int i) -> uint64_t {
        if (TERM) return term[i];
        return i == 0 ? (uint64_t)(uint32_t)rc0_next : 0;
    };
    auto ch = [&](int i) -> uint64_t { return !TERM && i == 0 ? rc0_next >> 32 : 0; };
    // Each output is finished as soon as its sums are formed (few sums live
    // at once); the rare final folds are applied per group of four words.
    uint64_t w[4];
    auto finish = [&](int i, uint64_t A, uint64_t B) { st[i] = gl_from_halves_defer(A, B, w[i & 3]); };
    auto fold4 = [&](int j) {
        const uint64_t any = mask_or(mask_or(w[0], w[1]), mask_or(w[2], w[3]));
        if (__builtin_expect(any != 0, 0)) {
#pragma unroll
            for (int i = 0; i < 4; i++) gl_fold_eps(st[j + i], w[i]);
        }
#if defined(__HIP_DEVICE_COMPILE__)
        // TERM: the next group's constants are loaded after this point, so
        // that at most four of them are live at once (scalar registers)
        if (TERM) asm volatile("" ::: "memory");
#endif
    };
    uint64_t A, B;
    {
        const uint64_t nx = ~x0;  // -2
        finish(0, acc32m<2>(SL + (5 + cl(0)), (uint32_t)nx), acc32m<2>(SH + (0xFFFFFFFDull + ch(0)), (uint32_t)(nx >> 32)));
    }
    finish(1, acc32(SL + cl(1), (uint32_t)st[1]), acc32(SH + ch(1), (uint32_t)(st[1] >> 32)));        //  1
    finish(2, acc32m<2>(SL + cl(2), (uint32_t)st[2]), acc32m<2>(SH + ch(2), (uint32_t)(st[2] >> 32)));  //  2
    inv_pow2_pos<1>(st[3], SL + cl(3), SH + ch(3), A, B);                                             //  1/2
    finish(3, A, B);
    fold4(0);
    finish(4, acc32m<3>(SL + cl(4), (uint32_t)st[4]), acc32m<3>(SH + ch(4), (uint32_t)(st[4] >> 32)));  //  3
    finish(5, acc32m<4>(SL + cl(5), (uint32_t)st[5]), acc32m<4>(SH + ch(5), (uint32_t)(st[5] >> 32)));  //  4
    inv_pow2_neg<1>(st[6], SL + cl(6), SH + ch(6), A, B);                                             // -1/2
    finish(6, A, B);
    {
        const uint64_t nx = ~st[7];  // -3
        finish(7, acc32m<3>(SL + (7 + cl(7)), (uint32_t)nx), acc32m<3>(SH + (0xFFFFFFFCull + ch(7)), (uint32_t)(nx >> 32)));
    }
    fold4(4);
    {
        const uint64_t nx = ~st[8];  // -4
        finish(8, acc32m<4>(SL + (9 + cl(8)), (uint32_t)nx), acc32m<4>(SH + (0xFFFFFFFBull + ch(8)), (uint32_t)(nx >> 32)));
    }
    inv_pow2_pos<3>(st[9], SL + cl(9), SH + ch(9), A, B);  //  1/2^3
    finish(9, A, B);
    inv_pow2_pos<4>(st[10], SL + cl(10), SH + ch(10), A, B);  //  1/2^4
    finish(10, A, B);
    inv_pow2_pos<5>(st[11], SL + cl(11), SH + ch(11), A, B);  //  1/2^5
    finish(11, A, B);
    fold4(8);
    inv_pow2_neg<3>(st[12], SL + cl(12), SH + ch(12), A, B);  // -1/2^3
    finish(12, A, B);
    inv_pow2_neg<4>(st[13], SL + cl(13), SH + ch(13), A, B);  // -1/2^4
    finish(13, A, B);
    inv_pow2_neg<5>(st[14], SL + cl(14), SH + ch(14), A, B);  // -1/2^5
    finish(14, A, B);
    if (DIAG15_IS_INV_2_32) {
        // x 2^-32 = x.hi + x.lo + ~x.lo 2^32 + 1 (k = 32: q = x.hi, m = x.lo)
        const uint64_t x = st[15];
        finish(15, acc32(acc32(SL + (1 + cl(15)), (uint32_t)(x >> 32)), (uint32_t)x), acc32(SH + ch(15), ~(uint32_t)x));
    } else {
        const uint64_t y = gl_mul(st[15], diag15);
        finish(15, acc32(SL + cl(15), (uint32_t)y), acc32(SH + ch(15), (uint32_t)(y >> 32)));
    }
    fold4(12);
}

// One internal round as a unit: st0 <- (st0 + rc)^7, then st_i <- sum + V_i st_i.
template <bool DIAG15_IS_INV_2_32>
__host__ __device__ __forceinline__ void internal_round(uint64_t* st, uint64_t rc, uint64_t diag15)
{
    st[0] = gl_add_small(st[0], rc);
    internal_round_core<DIAG15_IS_INV_2_32>(st, 0, diag15);
}

// FAST: the constant set has diag15 = 2^-32 and every constant that a
// linear layer adds (ext[0..8), internal[0]) below kRcLimit
// (p2_fast_constants); the caller checks this on the host. OUT: the output
// words the caller reads (kOutAll, kOutDigest for words 0..7, kOutCapacity
// for words 8..15), or kOutAbsorb: the caller passes last = whether this is
// the last absorb of a sponge (digest) or not (capacity), a value uniform
// over the wave. Words outside OUT are left undefined.
enum { kOutAbsorb = 0 };

inline bool p2_fast_constants(const P2Consts& c)
{
    if (gl_canon(c.diag15) != INV_2_32) return false;
    for (int k = 0; k < 8; k++)
        for (int i = 0; i < 16; i++)
            if (c.ext[k][i] >= kRcLimit) return false;
    return c.internal[0] < kRcLimit;
}

template <bool FAST, int OUT = kOutAll>
__host__ __device__ __forceinline__ void p2_permute(uint64_t* st, const P2Consts& C, bool last = true)
{
    // Initial linear layer fused with the first round's constants.
    mds_light16_rc<kRcAll, kOutAll, FAST>(st, C.ext[0]);
#pragma unroll 1
    for (int r = 0; r < 8; r++) {
#pragma unroll
        for (int i = 0; i < 16; i += 2) sbox7_2(st[i], st[i + 1]);
        if (r == 3) {
            // the linear layer adds the first internal round's constant to
            // word 0 and every internal round the next one's
            mds_light16_rc<kRcLane0, kOutAll, FAST>(st, C.internal);
            if (FAST) {
                // the last internal round adds the first terminal round's
                // constants (st += rc before its S-box) to its sums
#pragma unroll 1
                for (int k = 0; k < 21; k++) internal_round_core<FAST>(st, C.internal[k + 1], C.diag15);
                internal_round_core<FAST, true>(st, 0, C.diag15, C.ext[4]);
            } else {
#pragma unroll 1
                for (int k = 0; k < 22; k++)
                    internal_round_core<FAST>(st, k < 21 ? C.internal[k + 1] : 0, C.diag15);
                // constants of the first terminal round (st += rc) before its S-box
#pragma unroll
                for (int i = 0; i < 16; i++) st[i] = gl_add_small(st[i], C.ext[4][i]);
            }
        } else if (r == 7) {
            if (OUT != kOutAbsorb)
                mds_light16_rc<kRcNone, OUT>(st, nullptr);
            else if (last)
                mds_light16_rc<kRcNone, kOutDigest>(st, nullptr);
            else
                mds_light16_rc<kRcNone, kOutCapacity>(st, nullptr);
        } else {
            mds_light16_rc<kRcAll, kOutAll, FAST>(st, C.ext[r + 1]);
        }
    }
}

}  // namespace zk
