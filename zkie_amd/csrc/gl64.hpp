// Goldilocks arithmetic for CDNA4 (gfx950) and the host.
//
// p = 2^64 - 2^32 + 1, eps = 2^64 mod p = 2^32 - 1, 2^96 = -1 (mod p).
// Device values live in [0, 2^64) and need not be canonical; every helper
// accepts any u64 and returns a u64 congruent to the exact result. Only
// `gl_canon` produces the canonical representative; every value that leaves
// a kernel goes through it, so all outputs are canonical u64 exactly like the
// reference ABI (goldilocks_ntt.cu:92, poseidon2_merkle.cu:183).
//
// The 64x64 product is built from four v_mad_u64_u32 (32x32+64 -> 64) and
// reduced with the special form of p; there is no MFMA path here because
// nothing in this field is a dense float contraction. Defining
// ZK_LIMB_MUL_ON_HOST makes host builds run the same 32-bit-limb product
// (used by the CPU emulation tests of the device code).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace zk {

// Streaming global accesses (codeword passes read and write every word
// once): loads and stores with the non-temporal hint, plain on the host.

template <class T>
__host__ __device__ __forceinline__ T ld_nt(const T* p)
{
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_nontemporal_load(p);
#else
    return *p;
#endif
}

template <class T>
__host__ __device__ __forceinline__ void st_nt(T* p, T v)
{
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_nontemporal_store(v, p);
#else
    *p = v;
#endif
}

constexpr uint64_t P = 0xFFFFFFFF00000001ull;
constexpr uint64_t EPS = 0xFFFFFFFFull;
constexpr uint64_t HALF = 0x7FFFFFFF80000001ull;  // (p + 1) / 2
constexpr uint64_t INV_2_32 = 0xFFFFFFFE00000002ull;  // 2^-32 mod p

__host__ __device__ __forceinline__ uint64_t gl_canon(uint64_t a) { return a >= P ? a - P : a; }

// Device forms written with gfx950 carry/borrow masks in inline assembly
// (1); 0 builds the portable C forms on the device as well.
#ifndef ZK_MUL_ASM
#define ZK_MUL_ASM 1
#endif

// Rare corrections. Several reductions end in a correction that a lane needs
// with probability about 2^-32 or less (a second wrap or borrow that only
// operands near 2^64 can cause). On the device such a correction runs behind
// a branch on the wave's mask of the lanes that need it: one scalar compare
// and a branch that is almost never taken, instead of vector instructions in
// every lane. On the host it is an ordinary conditional. Either way every
// lane that needs the correction gets it.
__host__ __device__ __forceinline__ bool any_lane(bool c)
{
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_ballot_w64(c) != 0;
#else
    return c;
#endif
}
#define ZK_RARE(c) __builtin_expect(any_lane(c), 0)

// An operand the compiler has proven to be 0 after inlining (e.g. the
// zero-padded inputs of a DFT): the assembly forms below, which the compiler
// cannot fold, return early for it.
#define ZK_ZERO(x) (__builtin_constant_p(x) && (x) == 0)

__host__ __device__ __forceinline__ void gl_fold_eps(uint64_t& r, uint64_t w);

// a + b for any a, b < 2^64.
__host__ __device__ __forceinline__ uint64_t gl_add(uint64_t a, uint64_t b)
{
#if defined(__HIP_DEVICE_COMPILE__) && ZK_MUL_ASM
    // The carry of the 64-bit add (v_addc's carry-out) selects + eps, added
    // by a product-add whose own carry-out marks the rare second wrap.
    if (ZK_ZERO(b)) return a;
    if (ZK_ZERO(a)) return b;
    uint32_t s0, s1, c;
    uint64_t k, w;
    asm("v_add_co_u32_e64 %0, %3, %4, %5\n\t"
        "s_nop 1\n\t"
        "v_addc_co_u32_e64 %1, %3, %6, %7, %3\n\t"
        "s_nop 1\n\t"
        "v_cndmask_b32_e64 %2, 0, 1, %3"
        : "=&v"(s0), "=&v"(s1), "=&v"(c), "=&s"(k)
        : "v"((uint32_t)a), "v"((uint32_t)b), "v"((uint32_t)(a >> 32)), "v"((uint32_t)(b >> 32)));
    uint64_t t;
    asm("v_mad_u64_u32 %0, %1, %2, -1, %3" : "=&v"(t), "=s"(w) : "v"(c), "v"(((uint64_t)s1 << 32) | s0));
    if (__builtin_expect(w != 0, 0)) gl_fold_eps(t, w);
    return t;
#else
    uint64_t s = a + b;
    uint64_t t = s + ((s < a) ? EPS : 0);
    // A second wrap needs both operands at least p: rare, folded the same way.
    const bool w2 = t < s;
    if (ZK_RARE(w2)) t += w2 ? EPS : 0;
    return t;
#endif
}

// a + b where b < p (or any b <= 2^64 - 2^32): a single wrap at most.
__host__ __device__ __forceinline__ uint64_t gl_add_small(uint64_t a, uint64_t b)
{
    uint64_t s = a + b;
    return s + ((s < b) ? EPS : 0);
}

// a - b for any a, b < 2^64.
__host__ __device__ __forceinline__ uint64_t gl_sub(uint64_t a, uint64_t b)
{
    uint64_t d = a - b;
    uint64_t t = d - ((a < b) ? EPS : 0);
    // A second borrow needs b >= p + a: rare.
    const bool b2 = t > d;
    if (ZK_RARE(b2)) t -= b2 ? EPS : 0;
    return t;
}

__host__ __device__ __forceinline__ uint64_t gl_neg(uint64_t a) { return gl_sub(0, a); }

__host__ __device__ __forceinline__ uint64_t gl_double(uint64_t a) { return gl_add(a, a); }

// Reduce the 128-bit value (r3:r2:r1:r0, 32-bit limbs) mod p:
// x = lo64 + r2 * 2^64 + r3 * 2^96 = lo64 + r2 * eps - r3.
__host__ __device__ __forceinline__ uint64_t gl_reduce128(uint64_t lo, uint64_t hi)
{
    const uint64_t r3 = hi >> 32;
    const uint64_t r2 = hi & 0xFFFFFFFFull;
    uint64_t t0 = lo - r3;
    if (lo < r3) t0 -= EPS;  // borrow: t0 >= 2^64 - 2^32 + 1 > eps, no second wrap
    const uint64_t t1 = (r2 << 32) - r2;  // r2 * eps < p
    uint64_t r = t0 + t1;
    if (r < t1) r += EPS;  // carry: result < t1 < p - eps, no second wrap
    return r;
}

#if defined(__HIP_DEVICE_COMPILE__) && ZK_MUL_ASM
// a * b mod p in 12 VALU instructions on gfx950, using the carry-out of
// v_mad_u64_u32, which the compiler does not use on its own:
//   P = a0 b0,  T = a0 b1 + P.hi,  U + c 2^64 = a1 b0 + T  (carry c kept as a lane mask),
//   H = a1 b1 + U.hi,  L = U.lo 2^32 + P.lo,
//   a b = L + 2^64 H + 2^96 c = L + eps H.lo - H.hi - c   (2^64 = eps, 2^96 = -1).
// S = L + eps H.lo wraps at most once (carry folds back as + eps, no second
// wrap); S - H.hi - c borrows at most once (borrow folds back as - eps on a
// value >= 2^64 - 2^32, no second borrow). That borrow needs S < 2^32, i.e.
// H.lo = 0 and L < 2^32, so it is a rare correction (gl_fix_borrow behind a
// wave-uniform branch). A VALU write of an SGPR needs two wait states before a
// VALU reads it as carry-in or lane mask (s_nop 1).

// d -= eps in the lanes of mask k, where a borrow left d >= 2^64 - 2^32.
__device__ __forceinline__ void gl_fix_borrow(uint32_t& d0, uint32_t& d1, uint64_t k)
{
    uint32_t e;
    uint64_t kk;
    asm("s_nop 1\n\t"
        "v_cndmask_b32_e64 %2, 0, -1, %4\n\t"
        "v_sub_co_u32_e64 %0, %3, %0, %2\n\t"
        "s_nop 1\n\t"
        "v_subb_co_u32_e64 %1, %3, %1, 0, %3"
        : "+v"(d0), "+v"(d1), "=&v"(e), "=&s"(kk)
        : "s"(k));
}

__device__ __forceinline__ uint64_t gl_mul_dev(uint64_t a, uint64_t b)
{
    const uint32_t a0 = (uint32_t)a, a1 = (uint32_t)(a >> 32);
    const uint32_t b0 = (uint32_t)b, b1 = (uint32_t)(b >> 32);
    const uint64_t P = (uint64_t)a0 * b0;
    const uint64_t T = (uint64_t)a0 * b1 + (P >> 32);
    uint64_t U, m;
    asm("v_mad_u64_u32 %0, %1, %2, %3, %4" : "=&v"(U), "=s"(m) : "v"(a1), "v"(b0), "v"(T));
    const uint64_t H = (uint64_t)a1 * b1 + (U >> 32);
    const uint64_t L = (U << 32) | (uint32_t)P;
    uint64_t S, m1;
    uint32_t c1;
    asm("v_mad_u64_u32 %0, %1, %3, -1, %4\n\t"
        "s_nop 1\n\t"
        "v_cndmask_b32_e64 %2, 0, 1, %1\n\t"
        "v_mad_u64_u32 %0, %1, %2, -1, %0"
        : "=&v"(S), "=&s"(m1), "=&v"(c1)
        : "v"((uint32_t)H), "v"(L));
    uint32_t d0, d1;
    uint64_t k;
    asm("v_subb_co_u32_e64 %0, %2, %3, %5, %6\n\t"
        "s_nop 1\n\t"
        "v_subb_co_u32_e64 %1, %2, %4, 0, %2"
        : "=&v"(d0), "=&v"(d1), "=&s"(k)
        : "v"((uint32_t)S), "v"((uint32_t)(S >> 32)), "v"((uint32_t)(H >> 32)), "s"(m));
    if (__builtin_expect(k != 0, 0)) gl_fix_borrow(d0, d1, k);
    return ((uint64_t)d1 << 32) | d0;
}
#endif

__host__ __device__ __forceinline__ uint64_t gl_mul(uint64_t a, uint64_t b)
{
#if defined(__HIP_DEVICE_COMPILE__) && ZK_MUL_ASM
    return gl_mul_dev(a, b);
#elif defined(__HIP_DEVICE_COMPILE__) || defined(ZK_LIMB_MUL_ON_HOST)
    const uint32_t a0 = (uint32_t)a, a1 = (uint32_t)(a >> 32);
    const uint32_t b0 = (uint32_t)b, b1 = (uint32_t)(b >> 32);
    const uint64_t p00 = (uint64_t)a0 * b0;
    const uint64_t p01 = (uint64_t)a0 * b1 + (p00 >> 32);
    const uint64_t p10 = (uint64_t)a1 * b0 + (uint32_t)p01;
    const uint64_t p11 = (uint64_t)a1 * b1 + (p01 >> 32) + (p10 >> 32);
    const uint64_t lo = (p10 << 32) | (uint32_t)p00;
    return gl_reduce128(lo, p11);
#else
    const unsigned __int128 x = (unsigned __int128)a * b;
    return gl_reduce128((uint64_t)x, (uint64_t)(x >> 64));
#endif
}

__host__ __device__ __forceinline__ uint64_t gl_sqr(uint64_t a)
{
#if defined(__HIP_DEVICE_COMPILE__) && ZK_MUL_ASM
    return gl_mul_dev(a, a);
#elif defined(__HIP_DEVICE_COMPILE__) || defined(ZK_LIMB_MUL_ON_HOST)
    const uint32_t a0 = (uint32_t)a, a1 = (uint32_t)(a >> 32);
    const uint64_t p00 = (uint64_t)a0 * a0;
    const uint64_t c = (uint64_t)a0 * a1;  // cross term, counted twice
    const uint64_t p01 = c + (p00 >> 32);
    const uint64_t p10 = c + (uint32_t)p01;
    const uint64_t p11 = (uint64_t)a1 * a1 + (p01 >> 32) + (p10 >> 32);
    const uint64_t lo = (p10 << 32) | (uint32_t)p00;
    return gl_reduce128(lo, p11);
#else
    return gl_mul(a, a);
#endif
}

// Two independent products (x = a b, y = c d) with the steps of gl_mul_dev
// interleaved, so that each product's instructions fill the other's SGPR
// wait states instead of s_nop cycles.
__host__ __device__ __forceinline__ void gl_mul2(uint64_t a, uint64_t b, uint64_t c, uint64_t d,
                                                 uint64_t& x, uint64_t& y)
{
#if defined(__HIP_DEVICE_COMPILE__) && ZK_MUL_ASM
    const uint32_t a0 = (uint32_t)a, a1 = (uint32_t)(a >> 32), b0 = (uint32_t)b, b1 = (uint32_t)(b >> 32);
    const uint32_t c0 = (uint32_t)c, c1 = (uint32_t)(c >> 32), d0 = (uint32_t)d, d1 = (uint32_t)(d >> 32);
    const uint64_t Pa = (uint64_t)a0 * b0, Pb = (uint64_t)c0 * d0;
    const uint64_t Ta = (uint64_t)a0 * b1 + (Pa >> 32), Tb = (uint64_t)c0 * d1 + (Pb >> 32);
    uint64_t Ua, Ub, ma, mb;
    asm("v_mad_u64_u32 %0, %2, %4, %5, %6\n\t"
        "v_mad_u64_u32 %1, %3, %7, %8, %9"
        : "=&v"(Ua), "=&v"(Ub), "=&s"(ma), "=&s"(mb)
        : "v"(a1), "v"(b0), "v"(Ta), "v"(c1), "v"(d0), "v"(Tb));
    const uint64_t Ha = (uint64_t)a1 * b1 + (Ua >> 32), Hb = (uint64_t)c1 * d1 + (Ub >> 32);
    const uint64_t La = (Ua << 32) | (uint32_t)Pa, Lb = (Ub << 32) | (uint32_t)Pb;
    uint64_t Sa, Sb, ka, kb;
    uint32_t ca, cb;
    asm("v_mad_u64_u32 %0, %2, %6, -1, %7\n\t"
        "v_mad_u64_u32 %1, %3, %8, -1, %9\n\t"
        "s_nop 0\n\t"
        "v_cndmask_b32_e64 %4, 0, 1, %2\n\t"
        "v_cndmask_b32_e64 %5, 0, 1, %3\n\t"
        "v_mad_u64_u32 %0, %2, %4, -1, %0\n\t"
        "v_mad_u64_u32 %1, %3, %5, -1, %1"
        : "=&v"(Sa), "=&v"(Sb), "=&s"(ka), "=&s"(kb), "=&v"(ca), "=&v"(cb)
        : "v"((uint32_t)Ha), "v"(La), "v"((uint32_t)Hb), "v"(Lb));
    uint32_t xa0, xa1, xb0, xb1;
    asm("v_subb_co_u32_e64 %0, %4, %6, %8, %9\n\t"
        "v_subb_co_u32_e64 %2, %5, %10, %12, %13\n\t"
        "s_nop 0\n\t"
        "v_subb_co_u32_e64 %1, %4, %7, 0, %4\n\t"
        "v_subb_co_u32_e64 %3, %5, %11, 0, %5"
        : "=&v"(xa0), "=&v"(xa1), "=&v"(xb0), "=&v"(xb1), "=&s"(ka), "=&s"(kb)
        : "v"((uint32_t)Sa), "v"((uint32_t)(Sa >> 32)), "v"((uint32_t)(Ha >> 32)), "s"(ma),
          "v"((uint32_t)Sb), "v"((uint32_t)(Sb >> 32)), "v"((uint32_t)(Hb >> 32)), "s"(mb));
    if (__builtin_expect((ka | kb) != 0, 0)) {
        gl_fix_borrow(xa0, xa1, ka);
        gl_fix_borrow(xb0, xb1, kb);
    }
    x = ((uint64_t)xa1 << 32) | xa0;
    y = ((uint64_t)xb1 << 32) | xb0;
#else
    x = gl_mul(a, b);
    y = gl_mul(c, d);
#endif
}

// --- Linear-layer helpers whose device forms use the carry and borrow masks
// of the 32-bit add/sub instructions directly (two wait states between the
// VALU that writes a mask and the VALU that reads it).

// a - b for b <= p and any a: one borrow at most (a - b + 2^64 >= eps).
__host__ __device__ __forceinline__ uint64_t gl_sub_small(uint64_t a, uint64_t b)
{
#if defined(__HIP_DEVICE_COMPILE__) && ZK_MUL_ASM
    if (ZK_ZERO(b)) return a;
    uint32_t d0, d1, e;
    uint64_t k;
    asm("v_sub_co_u32_e64 %0, %3, %4, %6\n\t"
        "s_nop 1\n\t"
        "v_subb_co_u32_e64 %1, %3, %5, %7, %3\n\t"
        "s_nop 1\n\t"
        "v_cndmask_b32_e64 %2, 0, -1, %3\n\t"
        "v_sub_co_u32_e64 %0, %3, %0, %2\n\t"
        "s_nop 1\n\t"
        "v_subb_co_u32_e64 %1, %3, %1, 0, %3"
        : "=&v"(d0), "=&v"(d1), "=&v"(e), "=&s"(k)
        : "v"((uint32_t)a), "v"((uint32_t)(a >> 32)), "v"((uint32_t)b), "v"((uint32_t)(b >> 32)));
    return ((uint64_t)d1 << 32) | d0;
#else
    const uint64_t d = a - b;
    return a < b ? d - EPS : d;
#endif
}

// a - b for any a, b: the first borrow folds back as - eps, which borrows
// again only when a - b + 2^64 < eps, i.e. b >= p + a (rare: gl_fix_borrow
// behind a wave-uniform branch); the third subtraction cannot borrow.
__host__ __device__ __forceinline__ uint64_t gl_sub2(uint64_t a, uint64_t b)
{
#if defined(__HIP_DEVICE_COMPILE__) && ZK_MUL_ASM
    if (ZK_ZERO(b)) return a;
    uint32_t d0, d1, e;
    uint64_t k;
    asm("v_sub_co_u32_e64 %0, %3, %4, %6\n\t"
        "s_nop 1\n\t"
        "v_subb_co_u32_e64 %1, %3, %5, %7, %3\n\t"
        "s_nop 1\n\t"
        "v_cndmask_b32_e64 %2, 0, -1, %3\n\t"
        "v_sub_co_u32_e64 %0, %3, %0, %2\n\t"
        "s_nop 1\n\t"
        "v_subb_co_u32_e64 %1, %3, %1, 0, %3"
        : "=&v"(d0), "=&v"(d1), "=&v"(e), "=&s"(k)
        : "v"((uint32_t)a), "v"((uint32_t)(a >> 32)), "v"((uint32_t)b), "v"((uint32_t)(b >> 32)));
    if (__builtin_expect(k != 0, 0)) gl_fix_borrow(d0, d1, k);
    return ((uint64_t)d1 << 32) | d0;
#else
    return gl_sub(a, b);
#endif
}

// s + m eps for any s and m < 2^32: the product-add wraps at most once, and
// after a wrap the value is below m eps <= 2^64 - 2^33, so + eps cannot wrap.
__host__ __device__ __forceinline__ uint64_t gl_add_meps(uint64_t s, uint32_t m)
{
#if defined(__HIP_DEVICE_COMPILE__) && ZK_MUL_ASM
    if (ZK_ZERO(m)) return s;
    uint64_t S, k;
    uint32_t c;
    asm("v_mad_u64_u32 %0, %1, %3, -1, %4\n\t"
        "s_nop 1\n\t"
        "v_cndmask_b32_e64 %2, 0, 1, %1\n\t"
        "v_mad_u64_u32 %0, %1, %2, -1, %0"
        : "=&v"(S), "=&s"(k), "=&v"(c)
        : "v"(m), "v"(s));
    return S;
#else
    return gl_add(s, (uint64_t)m * EPS);
#endif
}

// s + m eps where the product-add rarely wraps (m eps far below 2^64 - s,
// e.g. m a small count of wraps): the wrap folds back behind a
// wave-uniform branch.
__host__ __device__ __forceinline__ uint64_t gl_add_meps_rare(uint64_t s, uint32_t m)
{
#if defined(__HIP_DEVICE_COMPILE__) && ZK_MUL_ASM
    uint64_t S, k;
    asm("v_mad_u64_u32 %0, %1, %2, -1, %3" : "=&v"(S), "=s"(k) : "v"(m), "v"(s));
    if (__builtin_expect(k != 0, 0)) {
        uint64_t kk;
        uint32_t c;
        asm("s_nop 1\n\t"
            "v_cndmask_b32_e64 %1, 0, 1, %3\n\t"
            "v_mad_u64_u32 %0, %2, %1, -1, %0"
            : "+v"(S), "=&v"(c), "=&s"(kk)
            : "s"(k));
    }
    return S;
#else
    return gl_add(s, (uint64_t)m * EPS);
#endif
}

// acc + x for a 64-bit running sum of 32-bit values (one v_mad_u64_u32).
__host__ __device__ __forceinline__ uint64_t acc32(uint64_t acc, uint32_t x)
{
#if defined(__HIP_DEVICE_COMPILE__) && ZK_MUL_ASM
    uint64_t r, k;
    asm("v_mad_u64_u32 %0, %1, %2, 1, %3" : "=&v"(r), "=s"(k) : "v"(x), "v"(acc));
    return r;
#else
    return acc + x;
#endif
}

// acc + x * M for a 64-bit running sum of 32-bit values, M a small constant.
template <int M>
__host__ __device__ __forceinline__ uint64_t acc32m(uint64_t acc, uint32_t x)
{
#if defined(__HIP_DEVICE_COMPILE__) && ZK_MUL_ASM
    static_assert(M >= 1 && M <= 64, "inline constant");
    uint64_t r, k;
    asm("v_mad_u64_u32 %0, %1, %2, %4, %3" : "=&v"(r), "=s"(k) : "v"(x), "v"(acc), "i"(M));
    return r;
#else
    return acc + (uint64_t)x * M;
#endif
}

// acc + x for a wave-uniform x (an SGPR operand, e.g. a round constant).
__host__ __device__ __forceinline__ uint64_t acc32s(uint64_t acc, uint32_t x)
{
#if defined(__HIP_DEVICE_COMPILE__) && ZK_MUL_ASM
    uint64_t r, k;
    asm("v_mad_u64_u32 %0, %1, %2, 1, %3" : "=&v"(r), "=s"(k) : "s"(x), "v"(acc));
    return r;
#else
    return acc + x;
#endif
}

// A + B 2^32 mod p for A, B < 2^63 (sums of 32-bit halves): with
// Bp = B + A.hi (one v_mad_u64_u32) the value is A.lo + Bp.lo 2^32 +
// Bp.hi 2^64, and 2^64 = eps. For the sums of a linear layer Bp.hi is a
// small count, so the final fold is a rare correction.
__host__ __device__ __forceinline__ uint64_t gl_from_halves(uint64_t A, uint64_t B)
{
#if defined(__HIP_DEVICE_COMPILE__) && ZK_MUL_ASM
    const uint64_t Bp = acc32(B, (uint32_t)(A >> 32));
    return gl_add_meps_rare(((uint64_t)(uint32_t)Bp << 32) | (uint32_t)A, (uint32_t)(Bp >> 32));
#else
    const uint64_t t = A + (B << 32);
    const uint32_t k = (uint32_t)(B >> 32) + (t < A ? 1u : 0u);
    return gl_add(t, (uint64_t)k * EPS);
#endif
}

// gl_from_halves without its final fold: returns A + B 2^32 folded once, and
// w (device) the mask of the lanes in which the fold's product-add wrapped
// and + eps is still due (gl_fold_eps), so that several outputs can share
// one rare-correction branch. On the host the value is complete and w = 0.
__host__ __device__ __forceinline__ uint64_t gl_from_halves_defer(uint64_t A, uint64_t B, uint64_t& w)
{
#if defined(__HIP_DEVICE_COMPILE__) && ZK_MUL_ASM
    const uint64_t Bp = acc32(B, (uint32_t)(A >> 32));
    uint64_t S;
    asm("v_mad_u64_u32 %0, %1, %2, -1, %3"
        : "=&v"(S), "=s"(w)
        : "v"((uint32_t)(Bp >> 32)), "v"(((uint64_t)(uint32_t)Bp << 32) | (uint32_t)A));
    return S;
#else
    w = 0;
    return gl_from_halves(A, B);
#endif
}

// a | b of two lane masks held in scalar registers, formed on the scalar
// unit (several deferred-fold masks are merged so that one branch serves
// them all).
__host__ __device__ __forceinline__ uint64_t mask_or(uint64_t a, uint64_t b)
{
#if defined(__HIP_DEVICE_COMPILE__) && ZK_MUL_ASM
    uint64_t r;
    asm("s_or_b64 %0, %1, %2" : "=s"(r) : "s"(a), "s"(b) : "scc");
    return r;
#else
    return a | b;
#endif
}

// r += eps in the lanes of mask w (a product-add of at most 2^32 eps wrapped
// there, so the value is below 2^64 - 2^33 and + eps cannot wrap again).
__host__ __device__ __forceinline__ void gl_fold_eps(uint64_t& r, uint64_t w)
{
#if defined(__HIP_DEVICE_COMPILE__) && ZK_MUL_ASM
    uint64_t kk;
    uint32_t c;
    asm("s_nop 1\n\t"
        "v_cndmask_b32_e64 %1, 0, 1, %3\n\t"
        "v_mad_u64_u32 %0, %2, %1, -1, %0"
        : "+v"(r), "=&v"(c), "=&s"(kk)
        : "s"(w));
#else
    (void)r;
    (void)w;
#endif
}

// x * 2^-k for 1 <= k <= 32, any x < 2^64:
// x = q 2^k + r, r 2^-k = -r 2^(96-k) = -(m * eps) with m = r 2^(32-k) < 2^32,
// and -(m * eps) = p - m 2^32 + m = (2^32 - 1 - m) 2^32 + (m + 1).
template <int K>
__host__ __device__ __forceinline__ uint64_t gl_mul_inv_pow2(uint64_t x)
{
    static_assert(K >= 1 && K <= 32, "shift range");
    if (ZK_ZERO(x)) return 0;
    const uint64_t q = x >> K;
    const uint64_t m = (K == 32) ? (x & 0xFFFFFFFFull) : ((x & ((1ull << K) - 1)) << (32 - K));
    const uint64_t y = ((0xFFFFFFFFull - m) << 32) + (m + 1);
    return gl_add_small(q, y) ;
}

// x * 2^24: x << 24 plus the shifted-out bits hi < 2^24 at weight 2^64 = eps.
__host__ __device__ __forceinline__ uint64_t gl_mul_2e24(uint64_t x)
{
    if (ZK_ZERO(x)) return 0;
#if defined(__HIP_DEVICE_COMPILE__)
    // x << 24 from the halves directly: (lo << 24, hi:lo >> 8)
    const uint32_t lo = (uint32_t)x, hi = (uint32_t)(x >> 32);
    const uint64_t s = ((uint64_t)__builtin_amdgcn_alignbit(hi, lo, 8) << 32) | (uint32_t)(lo << 24);
    return gl_add_meps(s, hi >> 8);
#else
    return gl_add_meps(x << 24, (uint32_t)(x >> 40));
#endif
}

// x * 2^48: hi = x >> 16 (48 bits) at weight 2^64; hi eps = hi.lo eps + hi.hi 2^32 eps
// and 2^32 eps = 2^64 - 2^32 = -1, so x 2^48 = (x << 48) + hi.lo eps - hi.hi.
__host__ __device__ __forceinline__ uint64_t gl_mul_2e48(uint64_t x)
{
    if (ZK_ZERO(x)) return 0;
    const uint64_t hi = x >> 16;
    return gl_sub_small(gl_add_meps(x << 48, (uint32_t)hi), hi >> 32);
}

// Canonical representative of a value that is rarely >= p (x - p = x + eps
// mod 2^64, behind a wave-uniform branch).
__host__ __device__ __forceinline__ uint64_t gl_canon_fast(uint64_t x)
{
    const bool big = x >= P;
    if (ZK_RARE(big)) x = big ? x + EPS : x;
    return x;
}

// x * 2^S for S in {1, 2}: lo + k 2^64 with k < 2^S, and k eps < p folds in
// with one wrap at most.
template <int S>
__host__ __device__ __forceinline__ uint64_t gl_shl(uint64_t x)
{
    static_assert(S >= 1 && S <= 2, "shift range");
    const uint64_t lo = x << S;
    uint64_t r = lo + (x >> (64 - S)) * EPS;
    const bool w = r < lo;  // rare: lo within 3 eps of 2^64
    if (ZK_RARE(w)) r += w ? EPS : 0;
    return r;
}

// sum + x * 2^S for S in {1, 2}: the two wraps (shifted-out bits and the
// addition carry) are counted into k <= 2^S, then k eps folds in once.
template <int S>
__host__ __device__ __forceinline__ uint64_t gl_add_shl(uint64_t sum, uint64_t x)
{
    static_assert(S >= 1 && S <= 2, "shift range");
    const uint64_t lo = (x << S) + sum;
    const uint64_t k = (x >> (64 - S)) + (lo < sum ? 1 : 0);
    uint64_t r = lo + k * EPS;
    const bool w = r < lo;  // rare: lo within 5 eps of 2^64
    if (ZK_RARE(w)) r += w ? EPS : 0;
    return r;
}

__host__ __device__ __forceinline__ uint64_t gl_halve(uint64_t x)
{
    return (x >> 1) + ((x & 1) ? HALF : 0);
}

__host__ __device__ inline uint64_t gl_pow(uint64_t a, uint64_t e)
{
    uint64_t r = 1;
    while (e) {
        if (e & 1) r = gl_mul(r, a);
        a = gl_mul(a, a);
        e >>= 1;
    }
    return gl_canon(r);
}

__host__ __device__ inline uint64_t gl_inv(uint64_t a) { return gl_pow(a, P - 2); }

// Lazy sum of up to 2^32 u64 terms: value = lo + hi * 2^64.
struct Acc {
    uint64_t lo;
    uint32_t hi;
};

__host__ __device__ __forceinline__ Acc acc_of(uint64_t x) { return Acc{x, 0u}; }

__host__ __device__ __forceinline__ Acc acc_add(Acc a, uint64_t x)
{
    const uint64_t s = a.lo + x;
    return Acc{s, a.hi + (s < x ? 1u : 0u)};
}

__host__ __device__ __forceinline__ Acc acc_add(Acc a, Acc b)
{
    const uint64_t s = a.lo + b.lo;
    return Acc{s, a.hi + b.hi + (s < b.lo ? 1u : 0u)};
}

// lo + hi * eps with hi * eps < p: one wrap at most.
__host__ __device__ __forceinline__ uint64_t acc_reduce(Acc a)
{
    const uint64_t t = ((uint64_t)a.hi << 32) - (uint64_t)a.hi;
    return gl_add_small(a.lo, t);
}

// Exact running sum of products e * x, e wave-uniform (on the device it is
// taken as a scalar operand, so it must be the same in every lane) and x per
// lane, for
// dot products that are reduced once at the end: the four 32 x 32 partial
// products accumulate in three 64-bit sums with carry counts,
//   sum = a0 + a1 2^32 + a2 2^64 + c0 2^64 + c1 2^96 + c2 2^128,
// 8 VALU instructions per term instead of a reduced multiply and addition.
// The counts stay below 2^32 for up to 2^31 terms.
struct DotAcc {
    uint64_t a0 = 0, a1 = 0, a2 = 0;
    uint32_t c0 = 0, c1 = 0, c2 = 0;
};

__host__ __device__ __forceinline__ void dot_add(DotAcc& d, uint64_t e, uint64_t x)
{
#if defined(__HIP_DEVICE_COMPILE__) && ZK_MUL_ASM
    const uint32_t el = (uint32_t)e, eh = (uint32_t)(e >> 32);
    const uint32_t xl = (uint32_t)x, xh = (uint32_t)(x >> 32);
    uint64_t k0, k1, k2, k3, kx;
    // each carry mask is read at least two instructions after its write
    asm("v_mad_u64_u32 %0, %6, %11, %13, %0\n\t"
        "v_mad_u64_u32 %1, %7, %12, %13, %1\n\t"
        "v_mad_u64_u32 %2, %9, %12, %14, %2\n\t"
        "v_mad_u64_u32 %1, %8, %11, %14, %1\n\t"
        "v_addc_co_u32_e64 %3, %10, %3, 0, %6\n\t"
        "v_addc_co_u32_e64 %4, %10, %4, 0, %7\n\t"
        "v_addc_co_u32_e64 %5, %10, %5, 0, %9\n\t"
        "v_addc_co_u32_e64 %4, %10, %4, 0, %8"
        : "+v"(d.a0), "+v"(d.a1), "+v"(d.a2), "+v"(d.c0), "+v"(d.c1), "+v"(d.c2), "=&s"(k0), "=&s"(k1),
          "=&s"(k2), "=&s"(k3), "=&s"(kx)
        : "v"(xl), "v"(xh), "s"(el), "s"(eh));
#else
    const uint64_t el = e & 0xFFFFFFFFull, eh = e >> 32, xl = x & 0xFFFFFFFFull, xh = x >> 32;
    uint64_t p = xl * el;
    d.a0 += p;
    d.c0 += d.a0 < p ? 1u : 0u;
    p = xh * el;
    d.a1 += p;
    d.c1 += d.a1 < p ? 1u : 0u;
    p = xh * eh;
    d.a2 += p;
    d.c2 += d.a2 < p ? 1u : 0u;
    p = xl * eh;
    d.a1 += p;
    d.c1 += d.a1 < p ? 1u : 0u;
#endif
}

// The accumulated sum mod p: with lo = a0 + (a1 << 32) and its carry, and
// mid = (a1 >> 32) + a2 + c0 + carry (its own carry counted into the
// 2^128 term), sum = lo + mid 2^64 + c1 2^96 + c2' 2^128, and 2^64 = eps,
// 2^96 = -1, 2^128 = -2^32 give lo + mid.lo eps - (mid.hi + c1 + c2' 2^32).
__host__ __device__ __forceinline__ uint64_t dot_reduce(const DotAcc& d)
{
    const uint64_t lo = d.a0 + (d.a1 << 32);
    const uint64_t t = (d.a1 >> 32) + d.c0 + (lo < d.a0 ? 1u : 0u);
    const uint64_t mid = d.a2 + t;
    const uint64_t c2 = (uint64_t)d.c2 + (mid < t ? 1u : 0u);
    const uint64_t q = (mid >> 32) + d.c1 + (c2 << 32);  // < p for counts below 2^31
    return gl_sub_small(gl_add_meps(lo, (uint32_t)mid), q);
}

// Quadratic extension EF = F[x]/(x^2 - 7).
struct Ef {
    uint64_t c0, c1;
};

__host__ __device__ __forceinline__ Ef ef_add(Ef a, Ef b) { return Ef{gl_add(a.c0, b.c0), gl_add(a.c1, b.c1)}; }
__host__ __device__ __forceinline__ Ef ef_sub(Ef a, Ef b) { return Ef{gl_sub(a.c0, b.c0), gl_sub(a.c1, b.c1)}; }

// 7 x = 8 x - x, with 8 x = (x << 3) + (x >> 61) eps (2^64 = eps).
__host__ __device__ __forceinline__ uint64_t gl_mul7(uint64_t x)
{
    return gl_sub(gl_add_meps(x << 3, (uint32_t)(x >> 61)), x);
}

// The four products run as two interleaved pairs (gl_mul2), so that each
// fills the other's wait states.
__host__ __device__ __forceinline__ Ef ef_mul(Ef a, Ef b)
{
    uint64_t p00, p11, p01, p10;
    gl_mul2(a.c0, b.c0, a.c1, b.c1, p00, p11);
    gl_mul2(a.c0, b.c1, a.c1, b.c0, p01, p10);
    return Ef{gl_add(p00, gl_mul7(p11)), gl_add(p01, p10)};
}

__host__ __device__ __forceinline__ Ef ef_mul_base(Ef a, uint64_t b)
{
    Ef r;
    gl_mul2(a.c0, b, a.c1, b, r.c0, r.c1);
    return r;
}

}  // namespace zk
