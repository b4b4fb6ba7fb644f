// CPU emulation of the device code of libzkie_hip.so (test infrastructure).
//
// Built host-only from the same headers the kernels use, with the device
// 32-bit-limb multiply (ZK_LIMB_MUL_ON_HOST) and bounds checks on every
// global and LDS access (ZK_EMU_BOUNDS). Each NTT pass is executed phase by
// phase for every thread of every workgroup, in the order the barriers
// impose, so index mistakes abort here instead of faulting a GPU.
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../zkie_amd/csrc/last_leaf.hpp"
#include "../../zkie_amd/csrc/ntt_plan.hpp"
#include "../../zkie_amd/csrc/poseidon2.hpp"

using namespace zk;

namespace {

template <int S, int KNZ, bool INV, int ROLE, int LOGV>
void run_pass_t(const PassArgs& a, uint32_t T)
{
    const uint64_t blocks = pass_blocks(a);
    std::vector<uint64_t> lds(pass_lds_bytes(a) / 8 + 1);
    constexpr int n = pass_steps<S>();
    const uint32_t logV = a.logC + a.logJ;
    if (T % (1u << logV) != 0) std::abort();  // a thread keeps one vector lane
    // the kernel's order: step-0 reads, LDS tables, [barrier] the rest of
    // step 0, then [barrier] each later step (one round of step-0 items when
    // T is the kernel's thread count; more rounds go through pass_step)
    const bool split0 = n > 1 && ((1u << (S - Radix<S>::r0)) << logV) <= kStepU * T;
    using Regs = uint64_t[kStepU][1 << Radix<S>::r0];
    std::vector<Regs> x(T);
    for (uint64_t bid = 0; bid < blocks; bid++) {
        const PassTile t = pass_tile(a, bid);
        if (split0)
            for (uint32_t tid = 0; tid < T; tid++)
                pass_step0_gather<S, KNZ, LOGV>(a, t, pass_lane(a, t, tid), tid, T, x[tid]);
        for (uint32_t tid = 0; tid < T; tid++) pass_tables<S, ROLE>(a, t, tid, T, lds.data());
        for (uint32_t tid = 0; tid < T; tid++) pass_tables_tab<S, ROLE>(t, tid, T, lds.data());
        for (int k = 0; k < n; k++)
            for (uint32_t tid = 0; tid < T; tid++) {
                const PassLane l = pass_lane(a, t, tid);
                if (k == 0 && split0) {
                    if constexpr (n > 1) pass_step0_finish<S, KNZ, INV, ROLE, LOGV>(a, t, l, tid, T, lds.data(), x[tid]);
                } else {
                    pass_step<S, KNZ, INV, ROLE, LOGV>(k, a, t, l, tid, T, lds.data());
                }
            }
    }
}

template <int S, int KNZ, bool INV, int ROLE>
void run_pass_v(const PassArgs& a, uint32_t T)
{
    if (a.logC + a.logJ == kNttLogV)
        run_pass_t<S, KNZ, INV, ROLE, (int)kNttLogV>(a, T);
    else
        run_pass_t<S, KNZ, INV, ROLE, -1>(a, T);
}

template <int S, bool INV, int ROLE>
void run_pass_r(const PassArgs& a, int knz, uint32_t T)
{
    switch (knz) {
        case 1: run_pass_v<S, 1, INV, ROLE>(a, T); break;
        case 2: run_pass_v<S, 2, INV, ROLE>(a, T); break;
        case 4: run_pass_v<S, 4, INV, ROLE>(a, T); break;
        default: run_pass_v<S, 8, INV, ROLE>(a, T); break;
    }
}

template <int S, bool INV>
void run_pass_s(const PassArgs& a, int knz, uint32_t T)
{
    switch (pass_role(a)) {
        case kRoleTwiddle: run_pass_r<S, INV, kRoleTwiddle>(a, knz, T); break;
        case kRoleTable: run_pass_r<S, INV, kRoleTable>(a, knz, T); break;
        case kRoleLast: run_pass_r<S, INV, kRoleLast>(a, knz, T); break;
        default: run_pass_r<S, INV, kRoleLastScale>(a, knz, T); break;
    }
}

template <bool INV>
void run_pass_inv(const PassArgs& a, uint32_t T)
{
    const int knz = pass_knz(a);
    switch (a.s) {
        case 1: run_pass_s<1, INV>(a, knz, T); break;
        case 2: run_pass_s<2, INV>(a, knz, T); break;
        case 3: run_pass_s<3, INV>(a, knz, T); break;
        case 4: run_pass_s<4, INV>(a, knz, T); break;
        case 5: run_pass_s<5, INV>(a, knz, T); break;
        case 6: run_pass_s<6, INV>(a, knz, T); break;
        case 7: run_pass_s<7, INV>(a, knz, T); break;
        case 8: run_pass_s<8, INV>(a, knz, T); break;
        default: run_pass_s<9, INV>(a, knz, T); break;
    }
}

// The fused last pass + leaf hash (last_leaf.hpp) of the commitment, phase
// by phase for every thread of every workgroup, kernel thread count.
template <int S>
void run_last_leaf_s(const PassArgs& a, uint64_t* digests, uint64_t digests_len, const P2Consts& C, bool d15)
{
    constexpr uint32_t T = fuse_threads<S>();
    using LL = LastLeaf<S>;
    const uint64_t blocks = pass_blocks(a);
    std::vector<uint64_t> lds(LL::lds_words());
    using Keep = uint64_t[LL::template rounds<T>()][kStepU][LL::R];
    std::vector<Keep> keep(T);
    for (uint64_t bid = 0; bid < blocks; bid++) {
        const PassTile t = pass_tile(a, bid);
        for (uint32_t tid = 0; tid < T; tid++) pass_tables<S, kRoleLast>(a, t, tid, T, lds.data());
        for (int k = 0; k + 1 < pass_steps<S>(); k++)
            for (uint32_t tid = 0; tid < T; tid++)
                pass_step<S, 8, false, kRoleLast, kFuseLogV>(k, a, t, pass_lane(a, t, tid), tid, T, lds.data());
        for (uint32_t tid = 0; tid < T; tid++) last_leaf_step<S, T>(a, t, pass_lane(a, t, tid), tid, lds.data(), keep[tid]);
        for (uint32_t tid = 0; tid < T; tid++) last_leaf_rows<S, T>(pass_lane(a, t, tid), tid, lds.data(), keep[tid]);
        for (uint32_t tid = 0; tid < T; tid++) {
            if (d15)
                last_leaf_hash<S, T, true>(tid, lds.data(), C);
            else
                last_leaf_hash<S, T, false>(tid, lds.data(), C);
        }
        for (uint32_t tid = 0; tid < T; tid++) last_leaf_store<S, T>(a, t, tid, lds.data(), digests, digests_len);
    }
}

void run_last_leaf(const PassArgs& a, uint64_t* digests, uint64_t digests_len, const P2Consts& C, bool d15)
{
    switch (a.s) {
        case 4: run_last_leaf_s<4>(a, digests, digests_len, C, d15); break;
        case 5: run_last_leaf_s<5>(a, digests, digests_len, C, d15); break;
        case 6: run_last_leaf_s<6>(a, digests, digests_len, C, d15); break;
        case 7: run_last_leaf_s<7>(a, digests, digests_len, C, d15); break;
        case 8: run_last_leaf_s<8>(a, digests, digests_len, C, d15); break;
        default: run_last_leaf_s<9>(a, digests, digests_len, C, d15); break;
    }
}

void run_pass(const PassArgs& a, uint32_t T, bool inverse)
{
    if (inverse)
        run_pass_inv<true>(a, T);
    else
        run_pass_inv<false>(a, T);
}

}  // namespace

extern "C" {

uint64_t emu_gl_add(uint64_t a, uint64_t b) { return gl_add(a, b); }
uint64_t emu_gl_sub(uint64_t a, uint64_t b) { return gl_sub(a, b); }
uint64_t emu_gl_mul(uint64_t a, uint64_t b) { return gl_mul(a, b); }
uint64_t emu_gl_sqr(uint64_t a) { return gl_sqr(a); }
uint64_t emu_gl_halve(uint64_t a) { return gl_halve(a); }
uint64_t emu_gl_inv_pow2(uint64_t a, int k)
{
    switch (k) {
        case 3: return gl_mul_inv_pow2<3>(a);
        case 4: return gl_mul_inv_pow2<4>(a);
        case 5: return gl_mul_inv_pow2<5>(a);
        case 32: return gl_mul_inv_pow2<32>(a);
        default: return 0;
    }
}
uint64_t emu_acc_sum(const uint64_t* x, uint64_t n)
{
    Acc a = acc_of(0);
    for (uint64_t i = 0; i < n; i++) a = acc_add(a, x[i]);
    return acc_reduce(a);
}
uint64_t emu_gl_canon(uint64_t a) { return gl_canon(a); }
uint64_t emu_dot(const uint64_t* e, const uint64_t* x, uint64_t n)
{
    DotAcc d;
    for (uint64_t i = 0; i < n; i++) dot_add(d, e[i], x[i]);
    return gl_canon(dot_reduce(d));
}
uint64_t emu_gl_canon_fast(uint64_t a) { return gl_canon_fast(a); }
uint64_t emu_gl_shl(uint64_t a, int s) { return s == 1 ? gl_shl<1>(a) : gl_shl<2>(a); }
uint64_t emu_gl_add_shl(uint64_t sum, uint64_t a, int s)
{
    return s == 1 ? gl_add_shl<1>(sum, a) : gl_add_shl<2>(sum, a);
}
uint64_t emu_gl_add_small(uint64_t a, uint64_t b) { return gl_add_small(a, b); }

// Permutation with explicit constants (layout of zkie_p2_upload_constants).
void emu_p2_permute(uint64_t* st, const uint64_t* rc_init, const uint64_t* rc_final,
                    const uint64_t* rc_internal, uint64_t diag15, int fast_diag)
{
    P2Consts c;
    for (int k = 0; k < 4; k++)
        for (int i = 0; i < 16; i++) {
            c.ext[k][i] = rc_init[16 * k + i];
            c.ext[4 + k][i] = rc_final[16 * k + i];
        }
    for (int k = 0; k < 22; k++) c.internal[k] = rc_internal[k];
    c.diag15 = diag15;
    if (fast_diag && p2_fast_constants(c))
        p2_permute<true>(st, c);
    else
        p2_permute<false>(st, c);
    for (int i = 0; i < 16; i++) st[i] = gl_canon(st[i]);
}

// One internal round of the device code (st0 <- (st0 + rc)^7, then the
// internal linear layer), canonical outputs.
void emu_p2_internal_round(uint64_t* st, uint64_t rc, uint64_t diag15, int fast_diag)
{
    if (fast_diag)
        internal_round<true>(st, rc, diag15);
    else
        internal_round<false>(st, rc, diag15);
    for (int i = 0; i < 16; i++) st[i] = gl_canon(st[i]);
}

// One external linear layer (mds_light16, no constants), canonical outputs.
void emu_p2_mds_light(uint64_t* st)
{
    mds_light16<false>(st, nullptr);
    for (int i = 0; i < 16; i++) st[i] = gl_canon(st[i]);
}

// DFT (in place) / LDE through the device pass code. Returns 0 on success.
int emu_dft(uint64_t* mat, uint32_t lg, uint64_t w, int inverse, uint32_t threads)
{
    if (lg == 0 || w == 0) return 0;
    const std::vector<uint64_t> tab = build_twiddle_tables();
    const Plan p = make_plan(lg, w);
    const uint64_t n = 1ull << lg;
    std::vector<uint64_t> tmp(n * w);
    uint32_t B = lg;
    for (uint32_t i = 0; i < p.np; i++) {
        PassArgs a = pass_args(p, i, B, w, mat, n, tmp.data(), mat, tab.data(), inverse != 0);
        if (p.np == 1) {
            // single pass in place: every workgroup reads all its rows before
            // its last step writes them; a copy of the input stands for that order
            std::vector<uint64_t> src(mat, mat + n * w);
            a.in = src.data();
            run_pass(a, threads, inverse != 0);
        } else {
            run_pass(a, threads, inverse != 0);
        }
        B -= a.s;
    }
    return 0;
}

// LDE reading only the first in_rows rows of `in` (the rest are zero
// coefficients), as the library's batch commit does.
int emu_lde_rows(const uint64_t* in, uint64_t h, uint64_t in_rows, uint64_t w, uint32_t log_blowup,
                 uint64_t* out, uint32_t threads)
{
    uint32_t lgh = 0;
    while ((1ull << lgh) < h) lgh++;
    const uint32_t L = lgh + log_blowup;
    const std::vector<uint64_t> tab = build_twiddle_tables();
    const Plan p = make_plan(L, w);
    const uint64_t n = 1ull << L;
    std::vector<uint64_t> tmp(n * w);
    uint32_t B = L;
    for (uint32_t i = 0; i < p.np; i++) {
        const PassArgs a = pass_args(p, i, B, w, in, in_rows, tmp.data(), out, tab.data(), false);
        run_pass(a, threads, false);
        B -= a.s;
    }
    return 0;
}

// The source word of output word t of the Prefix-order transpose.
uint64_t emu_prefix_source(uint64_t t, uint32_t lrows, uint32_t k, uint32_t E) { return prefix_source(t, lrows, k, E); }

int emu_lde(const uint64_t* in, uint64_t h, uint64_t w, uint32_t log_blowup, uint64_t* out,
            uint32_t threads)
{
    return emu_lde_rows(in, h, h, w, log_blowup, out, threads);
}

// LDE of 16-wide rows with the last pass fused with the leaf hash: out gets
// the codeword, digests (n * 8 u64) the leaf digests. Returns 1 when the
// plan's last pass is not fusable (nothing written), 0 on success.
int emu_lde_leaf(const uint64_t* in, uint64_t h, uint64_t w, uint32_t log_blowup, uint64_t* out,
                 uint64_t* digests, const uint64_t* rc_init, const uint64_t* rc_final, const uint64_t* rc_internal,
                 uint64_t diag15, int fast_diag)
{
    uint32_t lgh = 0;
    while ((1ull << lgh) < h) lgh++;
    const uint32_t L = lgh + log_blowup;
    const std::vector<uint64_t> tab = build_twiddle_tables();
    const Plan p = make_plan(L, w);
    const uint64_t n = 1ull << L;
    std::vector<uint64_t> tmp(n * w);
    P2Consts c;
    for (int k = 0; k < 4; k++)
        for (int i = 0; i < 16; i++) {
            c.ext[k][i] = rc_init[16 * k + i];
            c.ext[4 + k][i] = rc_final[16 * k + i];
        }
    for (int k = 0; k < 22; k++) c.internal[k] = rc_internal[k];
    c.diag15 = diag15;
    uint32_t B = L;
    for (uint32_t i = 0; i < p.np; i++) {
        const PassArgs a = pass_args(p, i, B, w, in, h, tmp.data(), out, tab.data(), false);
        if (a.last) {
            if (!last_leaf_fusable(a)) return 1;
            run_last_leaf(a, digests, n * 8, c, fast_diag != 0 && p2_fast_constants(c));
        } else {
            run_pass(a, 512, false);
        }
        B -= a.s;
    }
    return 0;
}

}  // extern "C"
