// The last pass of a multi-pass LDE of 16-wide rows fused with the leaf
// hash of the commitment (PaddingFreeSponge<Perm, 16, 8, 8> of each row,
// merkle_tree.rs:372-442 first_digest_layer), written as host/device phases
// so the kernel (merkle.hip) and the CPU emulator of the tests run the same
// code, the emulator with bounds checks on every access.
//
// A workgroup owns one tile of the last pass: 2^S complete codeword rows (16
// columns, one j2), whose natural rows are nat0 + i 2^(L - S). The pass's
// earlier steps run as in the plain pass (ntt_pass.hpp); then
//   step:  the last radix step reads the LDS tile, writes the codeword rows
//          to HBM (natural order, canonical) and keeps its outputs;
//   rows:  (after a barrier) the kept outputs go to a row tile in the same
//          LDS, row i at words [17 i, 17 i + 16) (the odd stride puts the
//          later reads of one element of 64 rows on different banks);
//   hash:  (after a barrier) each thread hashes whole rows from LDS and
//          leaves their digests in LDS, so the codeword is never read back
//          from HBM;
//   store: (after a barrier) lanes write the digests to layer 0, four lanes
//          per 64-byte digest.
#pragma once

#include "ntt_pass.hpp"
#include "poseidon2.hpp"

namespace zk {

constexpr int kFuseLogV = 4;  // 16 columns of one j2

// Threads of a fused workgroup: one per row of the tile (every lane hashes
// in the last phase, which holds most of the work), at least one wave. With
// one row per thread the last step keeps at most 16 outputs per thread.
template <int S>
__host__ __device__ constexpr uint32_t fuse_threads()
{
    return S <= 6 ? 64u : (1u << S);
}

template <int S>
struct LastLeaf {
    using Rd = Radix<S>;
    static_assert(Rd::n >= 2, "a multi-step pass");
    static constexpr int RL = Rd::n == 2 ? Rd::r1 : Rd::r2;  // digit bits of the last step
    static constexpr int R = 1 << RL;
    static constexpr uint32_t items = (1u << (S - RL)) << kFuseLogV;
    template <uint32_t T>
    static constexpr uint32_t rounds()
    {
        return (items + kStepU * T - 1) / (kStepU * T);
    }
    // LDS words: the pass's tile and step twiddles, or the row tile if larger
    static constexpr uint32_t lds_words()
    {
        return (1u << S) * 17 > ((1u << S) << kFuseLogV) + kW512Words ? (1u << S) * 17
                                                                       : ((1u << S) << kFuseLogV) + kW512Words;
    }
};

// The last step for thread tid: as ntt_step does for the last pass, with the
// outputs also kept (keep[r][u][idx] for round r, item u, output idx).
template <int S, uint32_t T>
__host__ __device__ __forceinline__ void last_leaf_step(const PassArgs& a, const PassTile& t, const PassLane& l,
                                                        uint32_t tid, const uint64_t* lds,
                                                        uint64_t (&keep)[LastLeaf<S>::template rounds<T>()][kStepU]
                                                                        [LastLeaf<S>::R])
{
    using LL = LastLeaf<S>;
    constexpr int RL = LL::RL, R = LL::R;
#pragma unroll
    for (uint32_t r = 0; r < LL::template rounds<T>(); r++) {
        const uint32_t it0 = tid + r * kStepU * T;
        uint64_t x[kStepU][R];
        step_gather<S, RL, RL, 8, false, kFuseLogV>(a, t, l, it0, T, lds, x);
#pragma unroll
        for (int u = 0; u < kStepU; u++) {
            const uint32_t it = it0 + (uint32_t)u * T;
            if (it >= LL::items) continue;
            uint32_t base, q;
            step_item<RL, RL>(it, kFuseLogV, base, q);
            dft_small<RL, false>(x[u]);
            const uint64_t obase = l.out_base + (uint64_t)digit_reverse<S>(base) * a.out_stride;
#pragma unroll
            for (int idx = 0; idx < R; idx++) {
                const uint32_t fi = bit_reverse((uint32_t)idx, RL) << (S - RL);
                const uint64_t val = gl_canon(x[u][idx]);
                const uint64_t oidx = obase + (uint64_t)fi * a.out_stride;
                ZK_BOUND(oidx, a.out_len);
                a.out[oidx] = val;
                keep[r][u][idx] = val;
            }
        }
    }
}

// The kept outputs of thread tid into the row tile (after a barrier that
// ends every read of the pass's tile).
template <int S, uint32_t T>
__host__ __device__ __forceinline__ void last_leaf_rows(const PassLane& l, uint32_t tid, uint64_t* lds,
                                                        const uint64_t (&keep)[LastLeaf<S>::template rounds<T>()]
                                                                              [kStepU][LastLeaf<S>::R])
{
    using LL = LastLeaf<S>;
    constexpr int RL = LL::RL, R = LL::R;
#pragma unroll
    for (uint32_t r = 0; r < LL::template rounds<T>(); r++) {
#pragma unroll
        for (int u = 0; u < kStepU; u++) {
            const uint32_t it = tid + r * kStepU * T + (uint32_t)u * T;
            if (it >= LL::items) continue;
            uint32_t base, q;
            step_item<RL, RL>(it, kFuseLogV, base, q);
            const uint32_t i1b = digit_reverse<S>(base);
#pragma unroll
            for (int idx = 0; idx < R; idx++) {
                const uint32_t i1 = i1b + (bit_reverse((uint32_t)idx, RL) << (S - RL));
                ZK_BOUND(i1 * 17 + l.v, (1u << S) * 17);
                lds[i1 * 17 + l.v] = keep[r][u][idx];
            }
        }
    }
}

// Leaf digests of the rows of thread tid (rows tid, tid + T, ...), from the
// row tile (after a barrier that ends the row tile's writes), each written
// canonical over the first 8 words of its own row in the tile (the row is
// consumed by then, and no other thread reads it).
template <int S, uint32_t T, bool D15>
__host__ __device__ __forceinline__ void last_leaf_hash(uint32_t tid, uint64_t* lds, const P2Consts& C)
{
#pragma unroll 1
    for (uint32_t row = tid; row < (1u << S); row += T) {
        uint64_t* rp = lds + row * 17;
        uint64_t st[16];
#pragma unroll
        for (int i = 8; i < 16; i++) st[i] = 0;
#pragma unroll 1
        for (int b = 0; b < 2; b++) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                ZK_BOUND(row * 17 + 8 * b + i, (1u << S) * 17);
                st[i] = rp[8 * b + i];
            }
            p2_permute<D15, kOutAbsorb>(st, C, b == 1);
        }
#pragma unroll
        for (int i = 0; i < 8; i++) rp[i] = gl_canon(st[i]);
    }
}

// The tile's digests from LDS to layer 0 (after a barrier that ends the
// digest writes): four consecutive lanes write the four 16-byte quarters of
// one 64-byte digest, so each digest reaches the L2 as one piece (a tile's
// rows are 2^(L - s) rows apart in natural order, so its digests are too).
template <int S, uint32_t T>
__host__ __device__ __forceinline__ void last_leaf_store(const PassArgs& a, const PassTile& t, uint32_t tid,
                                                         const uint64_t* lds, uint64_t* digests, uint64_t digests_len)
{
    (void)digests_len;
    const uint32_t shift = a.L - a.s;
#pragma unroll 1
    for (uint32_t q = tid; q < (4u << S); q += T) {
        const uint32_t row = q >> 2, k = q & 3;
        ZK_BOUND(row * 17 + 2 * k + 1, (1u << S) * 17);
        const uint64_t* rp = lds + row * 17 + 2 * k;
        const uint64_t d = (t.nat0 + ((uint64_t)row << shift)) * 8 + 2 * k;
        ZK_BOUND(d + 1, digests_len);
#if defined(__HIP_DEVICE_COMPILE__)
        *reinterpret_cast<ulonglong2*>(digests + d) = make_ulonglong2(rp[0], rp[1]);
#else
        digests[d] = rp[0];
        digests[d + 1] = rp[1];
#endif
    }
}

// Whether the last pass of an LDE can hash its rows: 16-wide rows held
// whole by one tile (16 columns, one j2), a multi-step pass, no scale.
__host__ __device__ __forceinline__ bool last_leaf_fusable(const PassArgs& a)
{
    return a.last && a.np > 1 && a.w == 16 && a.logC == 4 && a.logJ == 0 && a.s >= 4 && a.s <= 9 && a.scale == 1;
}

}  // namespace zk
