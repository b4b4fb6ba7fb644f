// Parity test of the C++ host interface (include/zkie_hip.hpp) against the
// oracle, written like the reference's own engine tests: transform and
// inverse round trip, encode, commit, open, verify, pruned multi-opening,
// fold, the prover-data cache stream, and the error paths. Needs a HIP device; prints one line per check and
// exits non-zero on the first mismatch.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <sstream>
#include <string>
#include <vector>

#include "zkie_hip.hpp"

extern "C" {
#include "zkie_oracle.h"
}

using zkie::F;

static int g_checks = 0;
#define EXPECT(cond, what)                                                   \
    do {                                                                     \
        if (!(cond)) {                                                       \
            std::printf("FAIL %s (line %d)\n", what, __LINE__);              \
            std::exit(1);                                                    \
        }                                                                    \
        std::printf("ok   %s\n", what);                                      \
        std::fflush(stdout);                                                 \
        g_checks++;                                                          \
    } while (0)

static zkie::RowMajorMatrix random_matrix(uint64_t seed, size_t h, size_t w)
{
    zkie::RowMajorMatrix m{std::vector<F>(h * w), w};
    or_gen_uniform(seed, h * w, m.values.data());
    return m;
}

int main()
{
    or_set_threads(4);
    std::printf("CASE C++ host interface\n");
    std::fflush(stdout);
    if (zkie_device_count() < 1) {
        std::printf("FAIL no HIP device\n");
        return 1;
    }
    zkie::HipDft dft;
    zkie::HipMerkleTreeMmcs mmcs;

    // dft_batch / idft_batch
    const auto m = random_matrix(1, 1 << 10, 8);
    const auto ev = dft.dft_batch(m);
    std::vector<F> ref = m.values;
    or_dft_batch(ref.data(), 10, 8);
    EXPECT(ev.values == ref, "dft_batch 2^10 x 8 equals the oracle");
    EXPECT(dft.idft_batch(ev).values == m.values, "idft_batch inverts dft_batch");
    EXPECT(dft.dft_batch(random_matrix(2, 1, 5)).values == random_matrix(2, 1, 5).values,
           "dft_batch of one row is the identity");

    // lde_batch (commit_extension's encoding)
    const auto c = random_matrix(3, 1 << 9, 16);
    const auto cw = dft.lde_batch(c, 2);
    std::vector<F> cw_ref((size_t(1) << 11) * 16);
    or_lde_batch(c.values.data(), 1 << 9, 16, 2, 1, cw_ref.data());
    EXPECT(cw.values == cw_ref && cw.height() == (1u << 11), "lde_batch blowup 4 equals the oracle");

    // commit / open_batch / verify
    const size_t h = cw.height();
    auto [cap, tree] = mmcs.commit(cw);
    std::vector<F> layers_ref(8 * (2 * h));
    zkie::Digest root_ref{};
    or_merkle_commit(cw.values.data(), h, 16, layers_ref.data(), root_ref.data());
    EXPECT(cap.size() == 1 && cap[0] == root_ref, "commit root equals the oracle");
    for (size_t idx : {size_t(0), size_t(1), size_t(777), h - 1}) {
        const auto o = mmcs.open_batch(idx, tree);
        std::vector<F> sib(8 * (tree.layer_lens.size() - 1));
        or_merkle_open(layers_ref.data(), h, idx, sib.data());
        bool same = o.opened_values[0] == std::vector<F>(cw.row(idx), cw.row(idx) + 16);
        for (size_t l = 0; l < o.opening_proof.size(); l++)
            for (int e = 0; e < 8; e++) same = same && o.opening_proof[l][e] == sib[8 * l + e];
        EXPECT(same, "open_batch row and path equal the oracle");
        EXPECT(or_merkle_verify(cap[0].data(), h, idx, o.opened_values[0].data(), 16,
                                o.opening_proof[0].data()) == 1,
               "open_batch verifies against the root");
    }

    // open_multi_batch (pruned)
    const std::vector<size_t> q = {3, 4, 100, 1024, 2047};
    auto [rows, pruned] = mmcs.open_multi_batch(q, tree);
    std::vector<uint64_t> qi(q.begin(), q.end());
    std::vector<F> pref(8 * q.size() * 16);
    const uint64_t n = or_merkle_open_pruned(layers_ref.data(), h, qi.data(), qi.size(), pref.data(),
                                             q.size() * 16);
    bool same = pruned.digests.size() == n;
    for (size_t i = 0; same && i < n; i++)
        for (int e = 0; e < 8; e++) same = same && pruned.digests[i][e] == pref[8 * i + e];
    for (size_t i = 0; i < q.size(); i++)
        same = same && rows[i][0] == std::vector<F>(cw.row(q[i]), cw.row(q[i]) + 16);
    EXPECT(same, "open_multi_batch rows and pruned proof equal the oracle");

    // commit_batch: three tables of 2^9, stacked table-major into 2^11 (one
    // zero table of padding), rows of 16, blowup 4
    {
        std::vector<std::vector<F>> tabs;
        std::vector<F> stacked(size_t(1) << 11, 0);
        for (int i = 0; i < 3; i++) {
            tabs.push_back(random_matrix(40 + i, 1 << 9, 1).values);
            std::memcpy(stacked.data() + (size_t(i) << 9), tabs.back().data(), (size_t(1) << 9) * sizeof(F));
        }
        auto [bcap, btree] = mmcs.commit_batch(tabs, 4, 2);
        std::vector<F> bcw((size_t(1) << 9) * 16);
        or_lde_batch(stacked.data(), 1 << 7, 16, 2, 1, bcw.data());
        std::vector<uint64_t> blens(65);
        const uint32_t bnl = or_merkle_num_layers(1 << 9);
        or_merkle_layer_lens(1 << 9, blens.data());
        size_t btotal = 0;
        for (uint32_t i = 0; i < bnl; i++) btotal += blens[i];
        std::vector<uint64_t> blayers(btotal * 8);
        zkie::Digest broot{};
        or_merkle_commit(bcw.data(), 1 << 9, 16, blayers.data(), broot.data());
        EXPECT(btree.height == (1u << 9) && btree.mat.download() == bcw, "commit_batch codeword equals the oracle");
        EXPECT(bcap.size() == 1 && bcap[0] == broot, "commit_batch root equals the oracle");
        bool threw = false;
        try {
            mmcs.commit_batch({std::vector<F>(8), std::vector<F>(4)}, 1, 1);
        } catch (const zkie::Error&) {
            threw = true;
        }
        EXPECT(threw, "commit_batch refuses tables of different sizes");
    }

    // fold of the committed codeword
    std::vector<zkie::Ef> r(4);
    for (int b = 0; b < 4; b++) r[b] = {F(1000 + b), F(7 * b + 1)};
    const auto f = zkie::fold_rows(tree.mat, h, 4, false, r);
    std::vector<F> fref(2 * h);
    or_fold_rows(cw.values.data(), h, 4, 0, &r[0][0], fref.data());
    same = true;
    for (size_t i = 0; i < h; i++) same = same && f[i][0] == fref[2 * i] && f[i][1] == fref[2 * i + 1];
    EXPECT(same, "fold_rows equals the oracle");

    // sumcheck::prove over the committed codeword's first 2^12 entries and an EF weight table
    {
        const uint32_t t = 12;
        std::vector<F> fv(cw.values.begin(), cw.values.begin() + (size_t(1) << t));
        std::vector<F> hv(size_t(2) << t);
        or_gen_uniform(77, hv.size(), hv.data());
        std::vector<zkie::Ef> ch(t);
        for (uint32_t b = 0; b < t; b++) ch[b] = {F(31 * b + 5), F(b + 2)};
        const zkie::DeviceBuffer d_f = zkie::DeviceBuffer::upload(fv), d_h = zkie::DeviceBuffer::upload(hv);
        const zkie::SumcheckProof pr = zkie::sumcheck_prove(d_f, false, d_h, t, ch);
        std::vector<F> polys(6 * t), fo(2), ho(2);
        or_sumcheck_prove(fv.data(), 0, hv.data(), t, t, &ch[0][0], polys.data(), fo.data(), ho.data());
        same = pr.rounds.size() == t && pr.f_eval == zkie::Ef{fo[0], fo[1]} && pr.h_eval == zkie::Ef{ho[0], ho[1]};
        for (uint32_t i = 0; same && i < t; i++)
            same = pr.rounds[i].c0 == zkie::Ef{polys[6 * i], polys[6 * i + 1]} &&
                   pr.rounds[i].c1 == zkie::Ef{polys[6 * i + 2], polys[6 * i + 3]} &&
                   pr.rounds[i].c2 == zkie::Ef{polys[6 * i + 4], polys[6 * i + 5]};
        EXPECT(same, "sumcheck_prove equals the oracle");
    }
    bool threw = false;

    // prover-data cache stream (whir.rs:542-602): framing, payload, round trip
    std::stringstream ss(std::ios::in | std::ios::out | std::ios::binary);
    zkie::serialize_batch_prover_data_into(tree, ss);
    const std::string bytes = ss.str();
    uint64_t size = 0;
    zkie::check(zkie_prover_data_size(h, 16, &size), "zkie_prover_data_size");
    auto u64_at = [&](size_t i) {
        uint64_t v = 0;
        std::memcpy(&v, bytes.data() + 8 * i, 8);
        return v;
    };
    const size_t L = tree.layer_lens.size(), t0 = 3 + h * 16, d0 = t0 + 2 * L;
    size_t total = 0;
    for (uint64_t l : tree.layer_lens) total += l;
    same = bytes.size() == size && size == 8 * (d0 + 8 * total);
    same = same && u64_at(0) == 1 && u64_at(1) == 16 && u64_at(2) == h * 16 && u64_at(t0) == L;
    for (size_t i = 0; same && i < h * 16; i++) same = u64_at(3 + i) == cw.values[i];
    for (size_t i = 0; same && i < L; i++) same = u64_at(t0 + 1 + i) == tree.layer_lens[i];
    for (size_t i = 0; same && i + 1 < L; i++) same = u64_at(t0 + 1 + L + i) == 2;
    for (size_t i = 0; same && i < 8 * total; i++) same = u64_at(d0 + i) == layers_ref[i];
    EXPECT(same, "serialize_batch_prover_data_into frames the codeword and the oracle's layers");
    ss.seekg(0);
    const auto back = zkie::restore_batch_prover_data_from(ss, h, 16);
    EXPECT(back.root == cap[0] && back.mat.download() == cw.values && back.layers.download() == tree.layers.download(),
           "restore_batch_prover_data_from returns the committed tree");
    const auto o1 = mmcs.open_batch(777, tree), o2 = mmcs.open_batch(777, back);
    EXPECT(o1.opened_values == o2.opened_values && o1.opening_proof == o2.opening_proof,
           "the restored tree opens like the committed one");
    std::stringstream other(bytes);
    threw = false;
    try {
        (void)zkie::restore_batch_prover_data_from(other, h, 8);
    } catch (const zkie::Error& e) {
        threw = e.code == ZKIE_ERR_INVALID;
    }
    EXPECT(threw, "restoring a stream of another shape throws zkie::Error(ZKIE_ERR_INVALID)");

    // the whole batch cache, as the reference's round trip writes it
    // (whir.rs:866-905): header, then the prover data; read back in order
    {
        zkie::BatchCacheMetadata meta;
        meta.model_id = "test-model";
        meta.group_id = "group-0";
        meta.table_ids = {"layer-0-weight"};
        meta.table_arity = 13;
        meta.num_tables = 1;
        meta.security_level = 32;
        meta.pow_bits = 10;
        meta.source_digest.fill(7);
        std::stringstream file;
        zkie::write_header(file, meta, cap);
        zkie::serialize_batch_prover_data_into(tree, file);
        const auto hdr = zkie::read_header(file);
        const auto again = zkie::restore_batch_prover_data_from(file, h, 16);
        EXPECT(hdr.first == meta && hdr.second == cap && again.root == tree.root &&
                   again.mat.download() == tree.mat.download(),
               "cache file: header then prover data read back in order");
    }

    // error path: an index outside the tree is a status, thrown as zkie::Error
    threw = false;
    try {
        (void)mmcs.open_batch(h, tree);
    } catch (const zkie::Error& e) {
        threw = e.code == ZKIE_ERR_INVALID;
    }
    EXPECT(threw, "open_batch past the last row throws zkie::Error(ZKIE_ERR_INVALID)");

    std::printf("ALL PASS %d\n", g_checks);
    return 0;
}
