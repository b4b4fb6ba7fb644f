// One four-step NTT pass, written as phases separated by workgroup barriers
// so the same code runs in the HIP kernel and in the CPU emulator used by the
// tests (which executes each phase for every thread of a workgroup in turn
// and checks every address against its buffer).
//
// Pass geometry: the array of n = 2^L rows is a set of blocks of N = 2^B
// rows. A workgroup owns block b, a tile of J = 2^logJ consecutive j2 values
// and a tile of C = 2^logC columns; it loads the N1 = 2^s points
// x[b N + j1 N2 + j2][c] (N2 = N / N1) into LDS as lds[j1][v] with
// v = (j2 - j20) C + (c - c0), runs radix-2 decimation-in-frequency over j1,
// multiplies output i1 by w_N^(i1 j2) and stores it at row b N + i1 N2 + j2
// (or, in the last pass where N2 = 1, at the natural row of position
// b N1 + i1).
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

struct PassArgs {
    const uint64_t* in;
    uint64_t* out;
    uint64_t in_rows;  // rows of `in` holding data; rows beyond read as zero
    uint64_t w;
    uint64_t scale;  // last pass: multiply by this (1 = forward)
    const uint64_t* tws;   // small tables: w_{2^lg}^k at offset 2^(lg-1) - 1
    const uint64_t* twlo;  // w_{2^32}^x, x < 2^16
    const uint64_t* twhi;  // w_{2^32}^(x 2^16), x < 2^16
    uint64_t in_len, out_len;  // element counts, checked by the emulator only
    uint32_t L, B, s;
    uint32_t logC, logJ;
    uint32_t last;
    uint32_t np;
    uint32_t sb[8];
};

struct PassTile {
    uint64_t blk;  // first row of the block
    uint64_t c0;   // first column
    uint64_t j20;  // first j2
    uint64_t N2;
    uint32_t logV, E;
};

__host__ __device__ __forceinline__ uint32_t bit_reverse(uint32_t x, uint32_t bits)
{
    return bits ? (__builtin_bitreverse32(x) >> (32 - bits)) : 0u;
}

__host__ __device__ __forceinline__ uint64_t pass_blocks(const PassArgs& a)
{
    const uint32_t logN2 = a.B - a.s;
    return ((1ull << a.L) >> a.B) * ((1ull << logN2) >> a.logJ) * (a.w >> a.logC);
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
    t.E = (1u << a.s) << t.logV;
    return t;
}

// w_{2^B}^e for e < 2^B.
__host__ __device__ __forceinline__ uint64_t pass_root_pow(const PassArgs& a, uint64_t e)
{
    const uint64_t E = e << (32 - a.B);
    return gl_mul(a.twlo[E & 0xFFFF], a.twhi[E >> 16]);
}

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

__host__ __device__ __forceinline__ void pass_load(const PassArgs& a, const PassTile& t, uint32_t tid,
                                                   uint32_t T, uint64_t* lds)
{
    const uint32_t V = 1u << t.logV;
    const uint32_t cmask = (1u << a.logC) - 1;
    for (uint32_t e = tid; e < t.E; e += T) {
        const uint32_t i = e >> t.logV, v = e & (V - 1);
        const uint64_t row = t.blk + (uint64_t)i * t.N2 + t.j20 + (v >> a.logC);
        uint64_t x = 0;
        if (row < a.in_rows) {
            const uint64_t idx = row * a.w + t.c0 + (v & cmask);
            ZK_BOUND(idx, a.in_len);
            x = a.in[idx];
        }
        lds[e] = x;
    }
}

// Radix-2 DIF stage with half-size m = 2^lm over the N1 points of every v.
__host__ __device__ __forceinline__ void pass_stage(const PassArgs& a, const PassTile& t, int lm,
                                                    uint32_t tid, uint32_t T, uint64_t* lds)
{
    const uint32_t V = 1u << t.logV;
    const uint32_t nbf = t.E >> 1;
    const uint32_t m = 1u << lm;
    for (uint32_t q = tid; q < nbf; q += T) {
        const uint32_t v = q & (V - 1), k = q >> t.logV;
        const uint32_t pos = k & (m - 1);
        const uint32_t i0 = ((k >> lm) << (lm + 1)) | pos;
        const uint32_t x0 = (i0 << t.logV) | v, x1 = ((i0 + m) << t.logV) | v;
        ZK_BOUND(x1, t.E);
        const uint64_t u = lds[x0], w = lds[x1];
        lds[x0] = gl_add(u, w);
        const uint64_t d = gl_sub(u, w);
        lds[x1] = lm ? gl_mul(d, a.tws[(m - 1) + pos]) : d;
    }
}

__host__ __device__ __forceinline__ void pass_store(const PassArgs& a, const PassTile& t, uint32_t tid,
                                                    uint32_t T, const uint64_t* lds)
{
    const uint32_t V = 1u << t.logV;
    const uint32_t cmask = (1u << a.logC) - 1;
    for (uint32_t e = tid; e < t.E; e += T) {
        const uint32_t pos = e >> t.logV, v = e & (V - 1);
        const uint32_t i1 = bit_reverse(pos, a.s);
        uint64_t val = lds[e];
        const uint64_t c = t.c0 + (v & cmask);
        if (!a.last) {
            const uint64_t j2 = t.j20 + (v >> a.logC);
            const uint64_t ex = (uint64_t)i1 * j2;
            if (ex) val = gl_mul(val, pass_root_pow(a, ex));
            const uint64_t idx = (t.blk + (uint64_t)i1 * t.N2 + j2) * a.w + c;
            ZK_BOUND(idx, a.out_len);
            a.out[idx] = val;
        } else {
            if (a.scale != 1) val = gl_mul(val, a.scale);
            const uint64_t idx = pass_natural_row(a, t.blk + i1) * a.w + c;
            ZK_BOUND(idx, a.out_len);
            a.out[idx] = gl_canon(val);
        }
    }
}

}  // namespace zk
