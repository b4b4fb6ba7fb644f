// VALU issue-rate probe for gfx950 (diagnostics, built as its own library,
// libzkie_valu_probe.so; the commitment library does not contain it).
//
// Each kernel runs `iters` iterations of a block of 16 VALU instructions of
// one kind over 8 independent register chains per lane, with enough waves
// resident (8 per SIMD) that no chain's latency is exposed. The launch is
// timed with HIP events on its stream; the wave-instruction count is known
// exactly (16 per iteration per wave, plus the handful around the loop), so
//   rate = waves * 16 * iters / time
// is the issue peak of that instruction kind in wave-instructions per second,
// the denominator of a kernel's VALU roofline. rocprofv3 (SQ_INSTS_VALU,
// GRBM_GUI_ACTIVE) confirms the count and the clock of the same launches.
//
// Kinds (the instruction forms the commitment kernels are built from):
//   0  v_add_u32 (VOP2, 4 bytes)
//   1  v_add_co_u32 with an SGPR carry-out (VOP3, 8 bytes)
//   2  v_mad_u64_u32 (VOP3, 64-bit result, SGPR carry-out)
//   3  v_mul_lo_u32 (VOP3)
//   4  v_addc_co_u32 with SGPR carry-in and carry-out (VOP3)
//   5  v_cndmask_b32 on an SGPR mask (VOP3)
//   6  the field-multiply mix: 6 v_mad_u64_u32, 1 v_cndmask_b32, 2
//      v_subb_co_u32, 3 v_mov_b32 per 12, the instruction mix of the
//      Goldilocks product in the Poseidon2 kernels (repeated, 12 + 4 adds = 16)
//   7  v_add_u32 in its VOP3 encoding (_e64, 8 bytes)
//   8  v_add_co_u32 with VCC carry-out (VOP2, 4 bytes)
//   9  64-bit adds on VCC: v_add_co_u32, two v_add_u32, v_addc_co_u32 (VOP2)
//  10  v_cndmask_b32 on VCC (VOP2)
//  11  v_mov_b32 (VOP1)
//  12  v_mov_b64 (VOP1, 64-bit)
//  13  v_lshl_add_u64 (VOP3, 64-bit add)
//  14  v_add_u32 with a 32-bit literal operand (VOP2 + literal, 8 bytes)
//  15  v_add_u32 and s_nop 0 alternating (8 of each)
//  16  v_xor_b32 (VOP2)
//  17  v_add3_u32 (VOP3, three sources)
//  18  v_lshlrev_b32 (VOP2 shift)
//  19  64-bit subtractions on VCC: v_sub_co_u32, s_nop 1, v_subb_co_u32 (VOP2)
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kThreads = 256;

#define ZKP_REP8(X) X(0) X(1) X(2) X(3) X(4) X(5) X(6) X(7)

template <int KIND>
__global__ __launch_bounds__(kThreads) void valu_probe_kernel(uint32_t iters, uint32_t* __restrict__ out)
{
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    uint32_t a0 = t, a1 = t + 1, a2 = t + 2, a3 = t + 3, a4 = t + 4, a5 = t + 5, a6 = t + 6, a7 = t + 7;
    uint32_t b = t * 3 + 1;
    uint64_t m0 = t, m1 = t + 11, m2 = t + 12, m3 = t + 13, m4 = t + 14, m5 = t + 15, m6 = t + 16, m7 = t + 17;
    uint64_t k0, k1, k2, k3;
#pragma unroll 1
    for (uint32_t i = 0; i < iters; i++) {
        if constexpr (KIND == 0) {
            asm volatile(
#define ZKP_ADD(n) "v_add_u32_e32 %" #n ", %8, %" #n "\n\t"
                ZKP_REP8(ZKP_ADD) ZKP_REP8(ZKP_ADD)
#undef ZKP_ADD
                : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7)
                : "v"(b));
        } else if constexpr (KIND == 1) {
            asm volatile(
#define ZKP_ADDCO(n) "v_add_co_u32_e64 %" #n ", %8, %" #n ", %9\n\t"
                ZKP_REP8(ZKP_ADDCO) ZKP_REP8(ZKP_ADDCO)
#undef ZKP_ADDCO
                : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7), "=&s"(k0)
                : "v"(b));
        } else if constexpr (KIND == 2) {
            asm volatile(
#define ZKP_MAD(n) "v_mad_u64_u32 %" #n ", %8, %9, %10, %" #n "\n\t"
                ZKP_REP8(ZKP_MAD) ZKP_REP8(ZKP_MAD)
#undef ZKP_MAD
                : "+v"(m0), "+v"(m1), "+v"(m2), "+v"(m3), "+v"(m4), "+v"(m5), "+v"(m6), "+v"(m7), "=&s"(k0)
                : "v"(a0), "v"(b));
        } else if constexpr (KIND == 3) {
            asm volatile(
#define ZKP_MUL(n) "v_mul_lo_u32 %" #n ", %" #n ", %8\n\t"
                ZKP_REP8(ZKP_MUL) ZKP_REP8(ZKP_MUL)
#undef ZKP_MUL
                : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7)
                : "v"(b));
        } else if constexpr (KIND == 4) {
            // carry-in from a mask written 16 instructions earlier (no wait states)
            asm volatile(
#define ZKP_ADDC(n) "v_addc_co_u32_e64 %" #n ", %8, %" #n ", %9, %10\n\t"
                ZKP_REP8(ZKP_ADDC) ZKP_REP8(ZKP_ADDC)
#undef ZKP_ADDC
                : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7), "=&s"(k0)
                : "v"(b), "s"(0ull));
        } else if constexpr (KIND == 5) {
            asm volatile(
#define ZKP_CND(n) "v_cndmask_b32_e64 %" #n ", %" #n ", %8, %9\n\t"
                ZKP_REP8(ZKP_CND) ZKP_REP8(ZKP_CND)
#undef ZKP_CND
                : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7)
                : "v"(b), "s"(0x5555555555555555ull));
        } else if constexpr (KIND == 7) {
            asm volatile(
#define ZKP_ADD3(n) "v_add_u32_e64 %" #n ", %8, %" #n "\n\t"
                ZKP_REP8(ZKP_ADD3) ZKP_REP8(ZKP_ADD3)
#undef ZKP_ADD3
                : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7)
                : "v"(b));
        } else if constexpr (KIND == 8) {
            asm volatile(
#define ZKP_ADDCOV(n) "v_add_co_u32_e32 %" #n ", vcc, %8, %" #n "\n\t"
                ZKP_REP8(ZKP_ADDCOV) ZKP_REP8(ZKP_ADDCOV)
#undef ZKP_ADDCOV
                : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7)
                : "v"(b)
                : "vcc");
        } else if constexpr (KIND == 9) {
            // add_co, two independent adds (the two wait states before a VALU
            // reads VCC as carry-in), addc: four 64-bit adds on VCC
            asm volatile(
#define ZKP_ADD64(n, m, x, y) "v_add_co_u32_e32 %" #n ", vcc, %8, %" #n "\n\tv_add_u32_e32 %" #x ", %8, %" #x \
    "\n\tv_add_u32_e32 %" #y ", %8, %" #y "\n\tv_addc_co_u32_e32 %" #m ", vcc, %8, %" #m ", vcc\n\t"
                ZKP_ADD64(0, 1, 2, 3) ZKP_ADD64(4, 5, 6, 7) ZKP_ADD64(2, 3, 0, 1) ZKP_ADD64(6, 7, 4, 5)
#undef ZKP_ADD64
                : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7)
                : "v"(b)
                : "vcc");
        } else if constexpr (KIND == 10) {
            asm volatile(
                "s_mov_b64 vcc, %9\n\t"
#define ZKP_CNDV(n) "v_cndmask_b32_e32 %" #n ", %" #n ", %8, vcc\n\t"
                ZKP_REP8(ZKP_CNDV) ZKP_REP8(ZKP_CNDV)
#undef ZKP_CNDV
                : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7)
                : "v"(b), "s"(0x5555555555555555ull)
                : "vcc");
        } else if constexpr (KIND == 11) {
            asm volatile(
#define ZKP_MOV(n) "v_mov_b32_e32 %" #n ", %8\n\t"
                ZKP_REP8(ZKP_MOV) ZKP_REP8(ZKP_MOV)
#undef ZKP_MOV
                : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7)
                : "v"(b));
        } else if constexpr (KIND == 12) {
            asm volatile(
#define ZKP_MOV64(n) "v_mov_b64_e32 %" #n ", %8\n\t"
                ZKP_REP8(ZKP_MOV64) ZKP_REP8(ZKP_MOV64)
#undef ZKP_MOV64
                : "+v"(m0), "+v"(m1), "+v"(m2), "+v"(m3), "+v"(m4), "+v"(m5), "+v"(m6), "+v"(m7)
                : "v"((uint64_t)b));
        } else if constexpr (KIND == 13) {
            asm volatile(
#define ZKP_LSHLADD(n) "v_lshl_add_u64 %" #n ", %8, 1, %" #n "\n\t"
                ZKP_REP8(ZKP_LSHLADD) ZKP_REP8(ZKP_LSHLADD)
#undef ZKP_LSHLADD
                : "+v"(m0), "+v"(m1), "+v"(m2), "+v"(m3), "+v"(m4), "+v"(m5), "+v"(m6), "+v"(m7)
                : "v"((uint64_t)b));
        } else if constexpr (KIND == 14) {
            asm volatile(
#define ZKP_ADDLIT(n) "v_add_u32_e32 %" #n ", 0x12345678, %" #n "\n\t"
                ZKP_REP8(ZKP_ADDLIT) ZKP_REP8(ZKP_ADDLIT)
#undef ZKP_ADDLIT
                : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7));
        } else if constexpr (KIND == 15) {
            // 8 adds and 8 s_nop 0: only the adds are VALU (counted 8, not 16)
            asm volatile(
#define ZKP_ADDNOP(n) "v_add_u32_e32 %" #n ", %8, %" #n "\n\ts_nop 0\n\t"
                ZKP_REP8(ZKP_ADDNOP)
#undef ZKP_ADDNOP
                : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7)
                : "v"(b));
        } else if constexpr (KIND == 16) {
            asm volatile(
#define ZKP_XOR(n) "v_xor_b32_e32 %" #n ", %8, %" #n "\n\t"
                ZKP_REP8(ZKP_XOR) ZKP_REP8(ZKP_XOR)
#undef ZKP_XOR
                : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7)
                : "v"(b));
        } else if constexpr (KIND == 17) {
            asm volatile(
#define ZKP_ADD3S(n) "v_add3_u32 %" #n ", %8, %" #n ", %8\n\t"
                ZKP_REP8(ZKP_ADD3S) ZKP_REP8(ZKP_ADD3S)
#undef ZKP_ADD3S
                : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7)
                : "v"(b));
        } else if constexpr (KIND == 18) {
            asm volatile(
#define ZKP_SHL(n) "v_lshlrev_b32_e32 %" #n ", 1, %" #n "\n\t"
                ZKP_REP8(ZKP_SHL) ZKP_REP8(ZKP_SHL)
#undef ZKP_SHL
                : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7));
        } else if constexpr (KIND == 19) {
            // eight 64-bit subtractions on VCC, s_nop 1 for the carry-in's two wait states
            asm volatile(
#define ZKP_SUB64(n, m) "v_sub_co_u32_e32 %" #n ", vcc, %" #n ", %8\n\ts_nop 1\n\tv_subb_co_u32_e32 %" #m ", vcc, %" #m ", %8, vcc\n\t"
                ZKP_SUB64(0, 1) ZKP_SUB64(2, 3) ZKP_SUB64(4, 5) ZKP_SUB64(6, 7)
                ZKP_SUB64(0, 1) ZKP_SUB64(2, 3) ZKP_SUB64(4, 5) ZKP_SUB64(6, 7)
#undef ZKP_SUB64
                : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7)
                : "v"(b)
                : "vcc");
        } else {
            // 6 mad, 1 cndmask, 2 subb, 3 mov, 4 add per 16, over independent registers
            asm volatile(
                "v_mad_u64_u32 %0, %8, %12, %13, %0\n\t"
                "v_mad_u64_u32 %1, %9, %12, %13, %1\n\t"
                "v_mov_b32 %4, %12\n\t"
                "v_mad_u64_u32 %2, %10, %12, %13, %2\n\t"
                "v_add_u32_e32 %5, %13, %5\n\t"
                "v_mad_u64_u32 %3, %11, %12, %13, %3\n\t"
                "v_mov_b32 %6, %13\n\t"
                "v_mad_u64_u32 %0, %8, %13, %12, %0\n\t"
                "v_cndmask_b32_e64 %7, %7, %13, %14\n\t"
                "v_mad_u64_u32 %1, %9, %13, %12, %1\n\t"
                "v_subb_co_u32_e64 %5, %10, %5, %13, %14\n\t"
                "v_add_u32_e32 %4, %13, %4\n\t"
                "v_subb_co_u32_e64 %6, %11, %6, %12, %14\n\t"
                "v_mov_b32 %7, %12\n\t"
                "v_add_u32_e32 %5, %12, %5\n\t"
                "v_add_u32_e32 %6, %12, %6\n\t"
                : "+v"(m0), "+v"(m1), "+v"(m2), "+v"(m3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7),
                  "=&s"(k0), "=&s"(k1), "=&s"(k2), "=&s"(k3)
                : "v"(a0), "v"(b), "s"(0x3333333333333333ull));
        }
    }
    (void)k0;
    (void)k1;
    (void)k2;
    (void)k3;
    out[t] = a0 ^ a1 ^ a2 ^ a3 ^ a4 ^ a5 ^ a6 ^ a7 ^ (uint32_t)(m0 ^ m1 ^ m2 ^ m3 ^ m4 ^ m5 ^ m6 ^ m7);
}

template <int KIND>
hipError_t launch(uint32_t blocks, uint32_t iters, uint32_t* out, hipStream_t s)
{
    valu_probe_kernel<KIND><<<blocks, kThreads, 0, s>>>(iters, out);
    return hipGetLastError();
}

}  // namespace

extern "C" {

// Number of kinds.
int zkie_valu_probe_kinds(void) { return 20; }

// Run kind `kind` on `blocks` workgroups of 256 threads for `iters`
// iterations; *ms receives the launch's duration (HIP events on a stream of
// its own), *wave_instr the VALU wave-instructions of the timed loop
// (blocks * 4 waves * 16 * iters). out: a device buffer of blocks * 256 u32.
int zkie_valu_probe_run(int kind, uint32_t blocks, uint32_t iters, uint32_t* d_out, double* ms,
                        uint64_t* wave_instr)
{
    if (kind < 0 || kind > 19 || blocks == 0 || !d_out || !ms || !wave_instr) return -1;
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) return (int)e;
    hipEvent_t a = nullptr, b = nullptr;
    if ((e = hipEventCreate(&a)) != hipSuccess || (e = hipEventCreate(&b)) != hipSuccess) {
        (void)hipStreamDestroy(s);
        return (int)e;
    }
    (void)hipEventRecord(a, s);
    switch (kind) {
        case 0: e = launch<0>(blocks, iters, d_out, s); break;
        case 1: e = launch<1>(blocks, iters, d_out, s); break;
        case 2: e = launch<2>(blocks, iters, d_out, s); break;
        case 3: e = launch<3>(blocks, iters, d_out, s); break;
        case 4: e = launch<4>(blocks, iters, d_out, s); break;
        case 5: e = launch<5>(blocks, iters, d_out, s); break;
        case 6: e = launch<6>(blocks, iters, d_out, s); break;
        case 7: e = launch<7>(blocks, iters, d_out, s); break;
        case 8: e = launch<8>(blocks, iters, d_out, s); break;
        case 9: e = launch<9>(blocks, iters, d_out, s); break;
        case 10: e = launch<10>(blocks, iters, d_out, s); break;
        case 11: e = launch<11>(blocks, iters, d_out, s); break;
        case 12: e = launch<12>(blocks, iters, d_out, s); break;
        case 13: e = launch<13>(blocks, iters, d_out, s); break;
        case 14: e = launch<14>(blocks, iters, d_out, s); break;
        case 15: e = launch<15>(blocks, iters, d_out, s); break;
        case 16: e = launch<16>(blocks, iters, d_out, s); break;
        case 17: e = launch<17>(blocks, iters, d_out, s); break;
        case 18: e = launch<18>(blocks, iters, d_out, s); break;
        default: e = launch<19>(blocks, iters, d_out, s); break;
    }
    (void)hipEventRecord(b, s);
    if (e == hipSuccess) e = hipEventSynchronize(b);
    float t = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&t, a, b);
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    (void)hipStreamDestroy(s);
    if (e != hipSuccess) return (int)e;
    *ms = t;
    *wave_instr = (uint64_t)blocks * (kThreads / 64) * (kind == 15 ? 8ull : 16ull) * iters;
    return 0;
}

}  // extern "C"
