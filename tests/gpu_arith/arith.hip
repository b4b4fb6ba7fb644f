// Test kernels for the device forms of the field arithmetic and of the
// Poseidon2 building blocks (the inline-assembly paths and their rare
// corrections, which the host emulation of the device code does not run).
// Test infrastructure: built beside the tests, called by
// tests/test_gpu_arith.py with crafted operands, never part of the library.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../zkie_amd/csrc/poseidon2.hpp"
#include "../../zkie_amd/csrc/poseidon2_x16.hpp"

using namespace zk;

namespace {

constexpr int kOps = 16;

__global__ void binary_kernel(const uint64_t* a, const uint64_t* b, uint64_t* out, uint64_t n)
{
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n) return;
    const uint64_t x = a[t], y = b[t];
    uint64_t* o = out + t * kOps;
    o[0] = gl_canon(gl_add(x, y));
    o[1] = gl_canon(gl_sub2(x, y));
    o[2] = gl_canon(gl_mul(x, y));
    o[3] = gl_canon(gl_sqr(x));
    o[4] = gl_canon(gl_mul_2e24(x));
    o[5] = gl_canon(gl_mul_2e48(x));
    o[6] = gl_canon(gl_mul_inv_pow2<24>(x));
    o[7] = gl_canon(gl_from_halves(x >> 29, y >> 29));  // sums of halves below 2^35
    uint64_t w;
    uint64_t r = gl_from_halves_defer(x >> 29, y >> 29, w);
    gl_fold_eps(r, w);
    o[8] = gl_canon(r);
    uint64_t p, q;
    gl_mul2(x, y, x, x, p, q);  // two different products through the interleaved form
    o[9] = gl_canon(p);
    o[10] = gl_canon(q);
    o[11] = gl_canon(gl_mul7(x));
    const Ef e = ef_mul(Ef{x, y}, Ef{y, x});  // (x + y X)(y + x X) in F[X]/(X^2 - 7)
    o[12] = gl_canon(e.c0);
    o[13] = gl_canon(e.c1);
    const Ef eb = ef_mul_base(Ef{x, y}, y);
    o[14] = gl_canon(eb.c0);
    o[15] = gl_canon(eb.c1);
}

// st: n states of 16 words; mode 0 mds_light16, 1 internal round (rc, diag15
// = 2^-32), 2 the permutation one lane per state with diag15 = 2^-32, 3 the
// permutation one 16-lane row per state, 4 the permutation one lane per
// state with a general diag15.
__global__ void state_kernel(uint64_t* st, uint64_t n, int mode, uint64_t rc, const P2Consts* C)
{
    const uint64_t g = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (mode == 3) {
        const uint64_t s = g / 16;
        const uint32_t i = threadIdx.x & 15;
        if (s >= n) return;  // whole rows
        const X16Lane L = x16_lane(*C, i);
        st[s * 16 + i] = gl_canon(p2_permute_x16(st[s * 16 + i], L, *C));
        return;
    }
    if (g >= n) return;
    uint64_t x[16];
    for (int i = 0; i < 16; i++) x[i] = st[g * 16 + i];
    if (mode == 0) mds_light16<false>(x, nullptr);
    if (mode == 1) internal_round<true>(x, rc, INV_2_32);
    if (mode == 2) p2_permute<true>(x, *C);
    if (mode == 4) p2_permute<false>(x, *C);
    for (int i = 0; i < 16; i++) st[g * 16 + i] = gl_canon(x[i]);
}

int ok(hipError_t e) { return e == hipSuccess ? 0 : (int)e; }

}  // namespace

extern "C" {

int arith_ops() { return kOps; }

// out[t * kOps + k] = op k on (a[t], b[t]) (host arrays).
int arith_binary(const uint64_t* a, const uint64_t* b, uint64_t* out, uint64_t n)
{
    uint64_t *da = nullptr, *db = nullptr, *dout = nullptr;
    int rc = ok(hipMalloc(&da, n * 8));
    if (!rc) rc = ok(hipMalloc(&db, n * 8));
    if (!rc) rc = ok(hipMalloc(&dout, n * 8 * kOps));
    if (!rc) rc = ok(hipMemcpy(da, a, n * 8, hipMemcpyHostToDevice));
    if (!rc) rc = ok(hipMemcpy(db, b, n * 8, hipMemcpyHostToDevice));
    if (!rc) {
        binary_kernel<<<(unsigned)((n + 255) / 256), 256>>>(da, db, dout, n);
        rc = ok(hipGetLastError());
    }
    if (!rc) rc = ok(hipMemcpy(out, dout, n * 8 * kOps, hipMemcpyDeviceToHost));
    hipFree(da);
    hipFree(db);
    hipFree(dout);
    return rc;
}

// States st[n][16] in place (host array); constants in the P2Consts layout
// (ext[8][16], internal[22], diag15) from the caller, the diagonal derived.
int arith_states(uint64_t* st, uint64_t n, int mode, uint64_t rc, const uint64_t* ext128,
                 const uint64_t* internal22, uint64_t diag15)
{
    P2Consts c{};
    for (int r = 0; r < 8; r++)
        for (int i = 0; i < 16; i++) c.ext[r][i] = ext128[16 * r + i];
    for (int k = 0; k < 22; k++) c.internal[k] = internal22[k];
    c.diag15 = diag15;
    p2_set_diag(c);
    uint64_t* dst = nullptr;
    P2Consts* dc = nullptr;
    int e = ok(hipMalloc(&dst, n * 128));
    if (!e) e = ok(hipMalloc(&dc, sizeof c));
    if (!e) e = ok(hipMemcpy(dst, st, n * 128, hipMemcpyHostToDevice));
    if (!e) e = ok(hipMemcpy(dc, &c, sizeof c, hipMemcpyHostToDevice));
    if (!e) {
        const uint64_t threads = mode == 3 ? n * 16 : n;
        state_kernel<<<(unsigned)((threads + 255) / 256), 256>>>(dst, n, mode, rc, dc);
        e = ok(hipGetLastError());
    }
    if (!e) e = ok(hipMemcpy(st, dst, n * 128, hipMemcpyDeviceToHost));
    hipFree(dst);
    hipFree(dc);
    return e;
}

}  // extern "C"
