// Poseidon2-Goldilocks-16 with one permutation spread over the 16 lanes of a
// DPP row (lane i of the row holds state word i), for the upper Merkle levels,
// whose few parents cannot fill the GPU with one permutation per lane: there
// the time of a level is the latency of one permutation, and spreading it
// over 16 lanes cuts that latency about five-fold (the 16 S-boxes of an
// external round run side by side; the linear layers exchange words with
// DPP row and quad moves). Same rounds, constants and results as
// p2_permute (poseidon2_merkle.cu:37-155 restated).
//
// Every lane of a row must be active whenever these functions run (a DPP
// move reads its source lane's register).
#pragma once

#include "poseidon2.hpp"

namespace zk {

// DPP controls (GFX9 encoding): quad_perm selectors and row rotations.
constexpr int kDppQuadRot1 = 0x39;  // lane k of a quad reads lane (k + 1) mod 4
constexpr int kDppQuadRot2 = 0x4E;  // (k + 2) mod 4
constexpr int kDppQuadRot3 = 0x93;  // (k + 3) mod 4
constexpr int kDppRowRor1 = 0x121;
constexpr int kDppRowRor2 = 0x122;
constexpr int kDppRowRor4 = 0x124;
constexpr int kDppRowRor8 = 0x128;

template <int CTRL>
__device__ __forceinline__ uint64_t dpp64(uint64_t v)
{
    // every source lane of these controls is inside the row and active
    const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)v, CTRL, 0xF, 0xF, true);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, true);
    return ((uint64_t)hi << 32) | lo;
}

// This lane's share of the constants: its word's external round constants
// and internal diagonal entry.
struct X16Lane {
    uint64_t rc[8];  // ext[r][i], r = 0..7
    uint64_t v;      // V_i
    bool lane0;      // word 0 (the internal S-box)
};

__device__ __forceinline__ X16Lane x16_lane(const P2Consts& C, uint32_t i)
{
    X16Lane L;
#pragma unroll
    for (int r = 0; r < 8; r++) L.rc[r] = C.ext[r][i];
    L.v = C.diag[i];
    L.lane0 = i == 0;
    return L;
}

// mds_light16 for the lane's word i = 4g + k: mat4 row k of its group
// (m = 2 x_k + 3 x_{k+1} + x_{k+2} + x_{k+3}, indices mod 4 in the quad),
// plus the sum of m over the four groups (lanes i, i +- 4, i +- 8), all on
// exact 64-bit sums of 32-bit halves, reduced once (+ rc if given).
template <bool ADD_RC>
__device__ __forceinline__ uint64_t mds_x16(uint64_t x, uint64_t rc)
{
    const uint64_t z1 = dpp64<kDppQuadRot1>(x), z2 = dpp64<kDppQuadRot2>(x), z3 = dpp64<kDppQuadRot3>(x);
    const uint64_t ml = acc32m<3>(acc32m<2>(acc32((uint32_t)z2, (uint32_t)z3), (uint32_t)x), (uint32_t)z1);
    const uint64_t mh = acc32m<3>(acc32m<2>(acc32(z2 >> 32, (uint32_t)(z3 >> 32)), (uint32_t)(x >> 32)),
                                  (uint32_t)(z1 >> 32));
    uint64_t sl = ml + dpp64<kDppRowRor4>(ml), sh = mh + dpp64<kDppRowRor4>(mh);
    sl += dpp64<kDppRowRor8>(sl);
    sh += dpp64<kDppRowRor8>(sh);
    uint64_t A = ml + sl, B = mh + sh;  // each below 35 (2^32 - 1)
    if (ADD_RC) {
        A = acc32(A, (uint32_t)rc);
        B = acc32(B, (uint32_t)(rc >> 32));
    }
    return gl_from_halves(A, B);
}

// One internal round: word 0 <- (word 0 + rc)^7, then every word <-
// sum + V_i word (the S-box runs in every lane; word 0 keeps it).
__device__ __forceinline__ uint64_t internal_x16(uint64_t x, uint64_t rc, const X16Lane& L)
{
    const uint64_t y = sbox7(gl_add_small(x, rc));
    x = L.lane0 ? y : x;
    uint64_t sl = (uint32_t)x, sh = x >> 32;
    sl += dpp64<kDppRowRor8>(sl);
    sh += dpp64<kDppRowRor8>(sh);
    sl += dpp64<kDppRowRor4>(sl);
    sh += dpp64<kDppRowRor4>(sh);
    sl += dpp64<kDppRowRor2>(sl);
    sh += dpp64<kDppRowRor2>(sh);
    sl += dpp64<kDppRowRor1>(sl);
    sh += dpp64<kDppRowRor1>(sh);  // each below 16 (2^32 - 1)
    return gl_add(gl_from_halves(sl, sh), gl_mul(x, L.v));
}

// The permutation of the row's 16-word state; returns this lane's word.
__device__ __forceinline__ uint64_t p2_permute_x16(uint64_t x, const X16Lane& L, const P2Consts& C)
{
    x = mds_x16<true>(x, L.rc[0]);
#pragma unroll
    for (int r = 0; r < 8; r++) {
        x = sbox7(x);
        if (r == 3) {
            x = mds_x16<false>(x, 0);
#pragma unroll 1
            for (int k = 0; k < 22; k++) x = internal_x16(x, C.internal[k], L);
            x = gl_add_small(x, L.rc[4]);
        } else if (r == 7) {
            x = mds_x16<false>(x, 0);
        } else {
            x = mds_x16<true>(x, L.rc[r + 1]);
        }
    }
    return x;
}

}  // namespace zk
