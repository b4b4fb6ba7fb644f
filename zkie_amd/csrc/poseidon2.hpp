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
//  * the internal diagonal is applied without multiplies: 2^-k splits x
//    into x >> k and the shifted-out bits, the 2^-32 entry uses a closed form
//    when diag15 has that value, and 2x, 3x, 4x, -3x are exact sums of
//    halves or shifts with the wrapped bits folded back once;
//  * in the internal rounds the work that does not depend on the S-box is
//    issued before it, and the round sum is made canonical so the sixteen
//    "sum + t" additions need one wrap correction each;
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

// st <- mds_light16(st) (+ rc if given). Output 4g + k is mat4(x_g)[k] +
// sum_h mat4(x_h)[k], and the column sum equals mat4(sum_h x_h)[k] (mat4
// is linear), so the sums come from the four-lane group sums first and each
// group is then transformed and written on its own: only one group's
// intermediate sums are live at a time. Both 32-bit halves of the state go
// through the layer as exact 64-bit sums (at most 35 (2^32 - 1) + 2^32
// each), and each output is reduced once from its two sums.
template <bool ADD_RC>
__host__ __device__ __forceinline__ void mds_light16(uint64_t* st, const uint64_t* rc)
{
    uint64_t gl[4], gh[4], sl[4], sh[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        gl[k] = acc32(acc32(acc32m<1>((uint32_t)st[k], (uint32_t)st[4 + k]), (uint32_t)st[8 + k]),
                      (uint32_t)st[12 + k]);
        gh[k] = acc32(acc32(acc32m<1>((uint32_t)(st[k] >> 32), (uint32_t)(st[4 + k] >> 32)),
                            (uint32_t)(st[8 + k] >> 32)),
                      (uint32_t)(st[12 + k] >> 32));
    }
    mat4_wide(gl, sl);
    mat4_wide(gh, sh);
    uint64_t w[16];  // lanes whose output still needs + eps (one shared rare branch)
#pragma unroll
    for (int j = 0; j < 16; j += 4) {
        uint64_t yl[4], yh[4];
        mat4_half((uint32_t)st[j], (uint32_t)st[j + 1], (uint32_t)st[j + 2], (uint32_t)st[j + 3], yl);
        mat4_half((uint32_t)(st[j] >> 32), (uint32_t)(st[j + 1] >> 32), (uint32_t)(st[j + 2] >> 32),
                  (uint32_t)(st[j + 3] >> 32), yh);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint64_t A = yl[k] + sl[k], B = yh[k] + sh[k];
            if (ADD_RC) {
                A = acc32s(A, (uint32_t)rc[j + k]);
                B = acc32s(B, (uint32_t)(rc[j + k] >> 32));
            }
            st[j + k] = gl_from_halves_defer(A, B, w[j + k]);
        }
    }
    uint64_t any = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) any |= w[i];
    if (__builtin_expect(any != 0, 0)) {
#pragma unroll
        for (int i = 0; i < 16; i++) gl_fold_eps(st[i], w[i]);
    }
}

// One internal round: st0 <- (st0 + rc)^7, then st_i <- sum + V_i st_i.
// The round sum is formed from 32-bit halves (two 64-bit running sums, one
// v_mad_u64_u32 per half) and made canonical, sum = s0 + s1 2^32. Lanes then
// use the cheapest of two kinds of form:
//  * exact sums of halves A + B 2^32 (A, B below 2^35), reduced once with the
//    final fold deferred to one shared rare branch:
//      V = 2, 3, 4:  A = s0 + V x.lo, B = s1 + V x.hi;
//      V = -v (v = 2, 3, 4): -v x = v ~x - v (eps - 1) with ~x = 2^64 - 1 - x,
//                    and -v (eps - 1) = (2^32 - 1 - v) 2^32 + 1 + 2v mod p, so
//                    A = s0 + 1 + 2v + v ~x.lo, B = s1 + 2^32 - 1 - v + v ~x.hi;
//      V = 2^-k (k = 3, 4, 5): x 2^-k = q - m eps with q = x >> k and
//                    m = (x mod 2^k) 2^(32-k), and -m 2^32 = ~m 2^32 + 1
//                    (2^32 eps = -1), so A = s0 + q.lo + m + 1,
//                    B = s1 + q.hi + ~m (~m = 2^32 - 1 - m);
//  * single-correction forms on the canonical sum:
//      V = -2^-k: sum - x 2^-k = (sum + m eps) - q;
//      V = 2^-32: sum + x 2^-32 = (sum + x.hi) - x.lo eps, where sum + x.hi
//                 cannot wrap (sum <= p - 1) and x.lo eps < p;
//      V = 1, 1/2: sum + t with one wrap correction; V = -1/2: gl_sub2.
template <int K>
__host__ __device__ __forceinline__ uint64_t lane_inv_pow2(uint64_t SL1, uint64_t SH, uint64_t x, uint64_t& w)
{
    const uint32_t ql = (uint32_t)(x >> K), qh = (uint32_t)(x >> 32) >> K;
    const uint32_t m = (uint32_t)x << (32 - K);
    const uint64_t A = acc32(acc32(SL1, ql), m);
    const uint64_t B = acc32(acc32(SH, qh), ~m);
    return gl_from_halves_defer(A, B, w);
}

template <bool DIAG15_IS_INV_2_32>
__host__ __device__ __forceinline__ void internal_round(uint64_t* st, uint64_t rc, uint64_t diag15)
{
    uint64_t slo = (uint32_t)st[1], shi = st[1] >> 32;
#pragma unroll
    for (int i = 2; i < 16; i++) {
        slo = acc32(slo, (uint32_t)st[i]);
        shi = acc32(shi, (uint32_t)(st[i] >> 32));
    }
    const uint64_t x0 = sbox7(gl_add_small(st[0], rc));
    slo = acc32(slo, (uint32_t)x0);
    shi = acc32(shi, (uint32_t)(x0 >> 32));
    // sum = slo + shi 2^32 = slo + (shi.lo << 32) + shi.hi 2^64, and 2^64 = eps
    const uint64_t t = slo + (shi << 32);
    const uint32_t k = (uint32_t)(shi >> 32) + (t < slo ? 1u : 0u);
    const uint64_t sum = gl_canon_fast(gl_add_meps_rare(t, k));
    const uint64_t SL = (uint32_t)sum, SH = sum >> 32;  // the halves of the sum, zero-extended

    const uint64_t x15 = st[15];
    uint64_t w[9];
    {
        const uint64_t nx = ~x0;                                                              // -2
        st[0] = gl_from_halves_defer(acc32m<2>(SL + 5, (uint32_t)nx),
                                     acc32m<2>(SH + 0xFFFFFFFDull, (uint32_t)(nx >> 32)), w[7]);
    }
    st[1] = gl_add_small(st[1], sum);                                                         //  1
    st[2] = gl_from_halves_defer(acc32m<2>(SL, (uint32_t)st[2]), acc32m<2>(SH, (uint32_t)(st[2] >> 32)),
                                 w[0]);                                                       //  2
    st[3] = gl_add_small(gl_halve(st[3]), sum);                                               //  1/2
    st[4] = gl_from_halves_defer(acc32m<3>(SL, (uint32_t)st[4]), acc32m<3>(SH, (uint32_t)(st[4] >> 32)),
                                 w[1]);                                                       //  3
    st[5] = gl_from_halves_defer(acc32m<4>(SL, (uint32_t)st[5]), acc32m<4>(SH, (uint32_t)(st[5] >> 32)),
                                 w[2]);                                                       //  4
    st[6] = gl_sub2(sum, gl_halve(st[6]));                                                    // -1/2
    {
        const uint64_t nx = ~st[7];                                                           // -3
        st[7] = gl_from_halves_defer(acc32m<3>(SL + 7, (uint32_t)nx),
                                     acc32m<3>(SH + 0xFFFFFFFCull, (uint32_t)(nx >> 32)), w[3]);
    }
    {
        const uint64_t nx = ~st[8];                                                           // -4
        st[8] = gl_from_halves_defer(acc32m<4>(SL + 9, (uint32_t)nx),
                                     acc32m<4>(SH + 0xFFFFFFFBull, (uint32_t)(nx >> 32)), w[8]);
    }
    const uint64_t SL1 = SL + 1;
    st[9] = lane_inv_pow2<3>(SL1, SH, st[9], w[4]);                                           //  1/2^3
    st[10] = lane_inv_pow2<4>(SL1, SH, st[10], w[5]);                                         //  1/2^4
    st[11] = lane_inv_pow2<5>(SL1, SH, st[11], w[6]);                                         //  1/2^5
    st[12] = gl_sub_small(gl_add_meps(sum, (uint32_t)st[12] << 29), st[12] >> 3);            // -1/2^3
    st[13] = gl_sub_small(gl_add_meps(sum, (uint32_t)st[13] << 28), st[13] >> 4);            // -1/2^4
    st[14] = gl_sub_small(gl_add_meps(sum, (uint32_t)st[14] << 27), st[14] >> 5);            // -1/2^5
    if (DIAG15_IS_INV_2_32)
        st[15] = gl_sub_small(acc32(sum, (uint32_t)(x15 >> 32)), (uint64_t)(uint32_t)x15 * EPS);
    else
        st[15] = gl_add_small(gl_mul(x15, diag15), sum);
    const uint64_t any = mask_or(mask_or(mask_or(w[0], w[1]), mask_or(w[2], w[3])),
                                 mask_or(mask_or(w[4], w[5]), mask_or(mask_or(w[6], w[7]), w[8])));
    if (__builtin_expect(any != 0, 0)) {
        gl_fold_eps(st[0], w[7]);
        gl_fold_eps(st[8], w[8]);
        gl_fold_eps(st[2], w[0]);
        gl_fold_eps(st[4], w[1]);
        gl_fold_eps(st[5], w[2]);
        gl_fold_eps(st[7], w[3]);
        gl_fold_eps(st[9], w[4]);
        gl_fold_eps(st[10], w[5]);
        gl_fold_eps(st[11], w[6]);
    }
}

template <bool DIAG15_IS_INV_2_32>
__host__ __device__ __forceinline__ void p2_permute(uint64_t* st, const P2Consts& C)
{
    // Initial linear layer fused with the first round's constants.
    mds_light16<true>(st, C.ext[0]);
#pragma unroll 1
    for (int r = 0; r < 8; r++) {
#pragma unroll
        for (int i = 0; i < 16; i += 2) sbox7_2(st[i], st[i + 1]);
        if (r == 3) {
            mds_light16<false>(st, nullptr);
#pragma unroll 1
            for (int k = 0; k < 22; k++) internal_round<DIAG15_IS_INV_2_32>(st, C.internal[k], C.diag15);
            // Constants of the first terminal round (st += rc) before its S-box.
#pragma unroll
            for (int i = 0; i < 16; i++) st[i] = gl_add_small(st[i], C.ext[4][i]);
        } else if (r == 7) {
            mds_light16<false>(st, nullptr);
        } else {
            mds_light16<true>(st, C.ext[r + 1]);
        }
    }
}

}  // namespace zk
