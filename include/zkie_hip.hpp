/* C++ host interface over the C ABI of libzkie_hip.so (header only).
 *
 * Mirrors the engines zkIE plugs into its WHIR PCS (crates/zkie-core/src/pcs):
 *   zkie::HipDft             <- CudaDft, TwoAdicSubgroupDft<Goldilocks>
 *                               (dft_cuda.rs:122-222): dft_batch over
 *                               row-major matrices, natural order in and out;
 *   zkie::HipMerkleTreeMmcs  <- CudaMerkleTreeMmcs, Mmcs<F> (merkle_cuda.rs:
 *                               315-395): commit, open_batch, open_multi_batch;
 *   zkie::MerkleTree         <- the MerkleTree prover data (p3-merkle-tree
 *                               merkle_tree.rs:32-70), kept in device memory;
 *   zkie::fold_rows, zkie::mle_eval <- the WHIR row fold and out-of-domain
 *                               evaluation (p3-whir prover/mod.rs:226-290);
 *   zkie::sumcheck_prove     <- sumcheck::prove (crates/zkie-core/src/common/
 *                               sumcheck.rs:33-79) over a device table and
 *                               weight table, EF rounds;
 *   zkie::serialize_batch_prover_data_into, zkie::restore_batch_prover_data_from
 *                            <- the prover-data part of the batch cache
 *                               (crates/zkie-core/src/pcs/whir.rs:542-602);
 *   zkie::write_header, zkie::read_header
 *                            <- the batch cache header (pcs/cache.rs:7-70).
 * Matrices are p3's RowMajorMatrix<F> (values row-major, canonical u64).
 * Errors: every non-zero status of the C ABI throws zkie::Error carrying it;
 * there is no CPU fallback here (the reference's Rust caller keeps its own,
 * dft_cuda.rs:174-177). Calls may come from several host threads: the
 * library orders its own scratch buffers between them. */
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <istream>
#include <ostream>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "zkie_hip.h"

namespace zkie {

using F = uint64_t;
using Digest = std::array<F, 8>;  // [F; DIGEST_ELEMS]
using Ef = std::array<F, 2>;      // BinomialExtensionField<F, 2>, [c0, c1]

struct Error : std::runtime_error {
    int code;
    Error(int rc, const std::string& what)
        : std::runtime_error(what + " failed with status " + std::to_string(rc)), code(rc)
    {
    }
};

inline void check(int rc, const char* what)
{
    if (rc != 0) throw Error(rc, what);
}

/* The EF coordinates of a possibly empty point, as the ABI's pointer. */
inline const F* ef_ptr(const std::vector<std::array<F, 2>>& r)
{
    static const F none[2] = {0, 0};
    return r.empty() ? none : r[0].data();
}

struct RowMajorMatrix {
    std::vector<F> values;
    size_t width = 0;
    size_t height() const { return width ? values.size() / width : 0; }
    const F* row(size_t r) const { return values.data() + r * width; }
};

/* Device allocation owned by this object (the CudaBuffer role of cuda_buffer.rs). */
class DeviceBuffer {
   public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t elems) : n_(elems)
    {
        check(zkie_dev_alloc(&ptr_, (elems ? elems : 1) * sizeof(F)), "zkie_dev_alloc");
    }
    static DeviceBuffer upload(const std::vector<F>& v)
    {
        DeviceBuffer b(v.size());
        if (!v.empty()) check(zkie_memcpy_htod(b.ptr_, v.data(), v.size() * sizeof(F)), "zkie_memcpy_htod");
        return b;
    }
    std::vector<F> download() const
    {
        std::vector<F> v(n_);
        if (n_) check(zkie_memcpy_dtoh(v.data(), ptr_, n_ * sizeof(F)), "zkie_memcpy_dtoh");
        return v;
    }
    DeviceBuffer(DeviceBuffer&& o) noexcept : ptr_(o.ptr_), n_(o.n_) { o.ptr_ = nullptr, o.n_ = 0; }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept
    {
        std::swap(ptr_, o.ptr_);
        std::swap(n_, o.n_);
        return *this;
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    ~DeviceBuffer()
    {
        if (ptr_) (void)zkie_dev_free(ptr_);
    }
    F* data() const { return static_cast<F*>(ptr_); }
    size_t size() const { return n_; }

   private:
    void* ptr_ = nullptr;
    size_t n_ = 0;
};

inline uint32_t log2_exact(size_t n, const char* what)
{
    uint32_t lg = 0;
    while ((size_t(1) << lg) < n) lg++;
    if ((size_t(1) << lg) != n) throw Error(ZKIE_ERR_INVALID, what);
    return lg;
}

/* TwoAdicSubgroupDft<Goldilocks> (dft_cuda.rs:161-222). */
class HipDft {
   public:
    /* out[i][c] = sum_j in[j][c] w_h^(ij), w_h = TWO_ADIC_GENERATORS[log h]. */
    RowMajorMatrix dft_batch(RowMajorMatrix mat) const { return run(std::move(mat), false); }
    /* The inverse transform, including the 1/h scale. */
    RowMajorMatrix idft_batch(RowMajorMatrix mat) const { return run(std::move(mat), true); }
    /* Coefficients zero-padded to height << added_bits, optionally scaled by
     * shift^i, then dft_batch: the encoding of commit_extension (writer.rs:21-86). */
    RowMajorMatrix lde_batch(const RowMajorMatrix& coeffs, uint32_t added_bits, F shift = 1) const
    {
        const size_t h = coeffs.height(), w = coeffs.width;
        (void)log2_exact(h, "lde_batch height");
        DeviceBuffer in = DeviceBuffer::upload(coeffs.values), out((h << added_bits) * w);
        check(zkie_lde_batch(in.data(), h, w, added_bits, shift, out.data(), nullptr), "zkie_lde_batch");
        return RowMajorMatrix{out.download(), w};
    }

   private:
    static RowMajorMatrix run(RowMajorMatrix mat, bool inverse)
    {
        const size_t h = mat.height(), w = mat.width;
        if (h <= 1) return mat;  // dft_cuda.rs:164-166
        const uint32_t lg = log2_exact(h, "dft_batch height");
        DeviceBuffer d = DeviceBuffer::upload(mat.values);
        check(inverse ? zkie_idft_batch(d.data(), lg, w, nullptr) : zkie_dft_batch(d.data(), lg, w, nullptr),
              inverse ? "zkie_idft_batch" : "zkie_dft_batch");
        mat.values = d.download();
        return mat;
    }
};

/* MerkleTree prover data (merkle_tree.rs:32-70), device resident. */
struct MerkleTree {
    DeviceBuffer mat;
    size_t height = 0, width = 0;
    DeviceBuffer layers;
    std::vector<uint64_t> layer_lens;  // digests per layer, leaves first
    Digest root{};
};

using MerkleCap = std::vector<Digest>;  // cap height 0: the root

/* BatchOpening (p3-commit): one opened row per matrix, the sibling path bottom-up. */
struct BatchOpening {
    std::vector<std::vector<F>> opened_values;
    std::vector<Digest> opening_proof;
};

/* PrunedMerklePaths (pruning.rs:83-89), as the frontier-ordered sibling list. */
struct PrunedMerklePaths {
    std::vector<Digest> digests;
};

/* Mmcs<F> with MerkleTree<F, F, M, 2, 8> prover data (merkle_cuda.rs:315-395). */
class HipMerkleTreeMmcs {
   public:
    /* One matrix per commitment (WHIR commits one, p3-whir pcs/proof.rs:114-121). */
    std::pair<MerkleCap, MerkleTree> commit(const RowMajorMatrix& m) const
    {
        MerkleTree t;
        t.height = m.height();
        t.width = m.width;
        uint32_t nl = 0;
        std::vector<uint64_t> lens(65);
        check(zkie_merkle_layout(t.height, &nl, lens.data()), "zkie_merkle_layout");
        lens.resize(nl);
        size_t total = 0;
        for (uint64_t l : lens) total += l;
        t.layer_lens = lens;
        t.mat = DeviceBuffer::upload(m.values);
        t.layers = DeviceBuffer(total * 8);
        check(zkie_merkle_commit(t.mat.data(), t.height, t.width, t.layers.data(), t.root.data(), nullptr),
              "zkie_merkle_commit");
        MerkleCap cap{t.root};
        return {std::move(cap), std::move(t)};
    }

    /* Whir::commit_batch (crates/zkie-core/src/pcs/whir.rs:476-525): same-size
     * tables of evaluations stacked table-major into one zero-padded witness,
     * viewed as rows of 2^log_width, encoded with blowup 2^log_blowup and
     * committed. The tree's matrix is the codeword. */
    std::pair<MerkleCap, MerkleTree> commit_batch(const std::vector<std::vector<F>>& evals_batch, uint32_t log_width,
                                                  uint32_t log_blowup) const
    {
        if (evals_batch.empty()) throw Error(ZKIE_ERR_INVALID, "commit_batch: batch must not be empty");
        const size_t len = evals_batch[0].size();
        uint32_t arity = 0;
        while ((size_t(1) << arity) < len) arity++;
        for (const auto& e : evals_batch)
            if (e.size() != len || (size_t(1) << arity) != len)
                throw Error(ZKIE_ERR_INVALID, "commit_batch: all tables must hold the same power-of-two count");
        const size_t total = evals_batch.size() * len;
        uint32_t vars = 0;
        while ((size_t(1) << vars) < total) vars++;
        if (vars < log_width) throw Error(ZKIE_ERR_INVALID, "commit_batch: the stacked witness fills no row");
        std::vector<DeviceBuffer> tables;
        std::vector<const uint64_t*> ptrs;
        for (const auto& e : evals_batch) {
            tables.push_back(DeviceBuffer::upload(e));
            ptrs.push_back(tables.back().data());
        }
        MerkleTree t;
        t.width = size_t(1) << log_width;
        t.height = (size_t(1) << (vars - log_width)) << log_blowup;
        uint32_t nl = 0;
        std::vector<uint64_t> lens(65);
        check(zkie_merkle_layout(t.height, &nl, lens.data()), "zkie_merkle_layout");
        lens.resize(nl);
        size_t digests = 0;
        for (uint64_t l : lens) digests += l;
        t.layer_lens = lens;
        DeviceBuffer stack(size_t(1) << vars);
        t.mat = DeviceBuffer(t.height * t.width);
        t.layers = DeviceBuffer(digests * 8);
        check(zkie_commit_batch(ptrs.data(), (uint32_t)ptrs.size(), arity, log_width, log_blowup, stack.data(),
                                t.mat.data(), t.layers.data(), t.root.data(), nullptr),
              "zkie_commit_batch");
        MerkleCap cap{t.root};
        return {std::move(cap), std::move(t)};
    }

    /* mmcs/batch.rs:75-121. */
    BatchOpening open_batch(size_t index, const MerkleTree& t) const
    {
        const uint64_t idx = index;
        BatchOpening o;
        o.opened_values.assign(1, std::vector<F>(t.width));
        o.opening_proof.resize(t.layer_lens.size() - 1);
        check(zkie_merkle_open_batch(t.mat.data(), t.height, t.width, t.layers.data(), &idx, 1,
                                     o.opened_values[0].data(), o.opening_proof.empty() ? nullptr : o.opening_proof[0].data(),
                                     nullptr),
              "zkie_merkle_open_batch");
        return o;
    }

    /* mmcs/mod.rs:309-461: opened rows per index (one matrix each) and the pruned proof. */
    std::pair<std::vector<std::vector<std::vector<F>>>, PrunedMerklePaths> open_multi_batch(
        const std::vector<size_t>& indices, const MerkleTree& t) const
    {
        std::vector<uint64_t> idx(indices.begin(), indices.end());
        std::vector<F> rows(idx.size() * t.width);
        // a pruned proof holds at most one sibling per index per level
        const uint64_t cap = (uint64_t)idx.size() * (t.layer_lens.size() - 1) + 1;
        std::vector<Digest> pruned(cap);
        uint64_t count = 0;
        check(zkie_merkle_open_pruned(t.mat.data(), t.height, t.width, t.layers.data(), idx.data(), idx.size(),
                                      rows.data(), pruned[0].data(), cap, &count, nullptr),
              "zkie_merkle_open_pruned");
        pruned.resize(count);
        std::vector<std::vector<std::vector<F>>> opened(idx.size());
        for (size_t i = 0; i < idx.size(); i++)
            opened[i].emplace_back(rows.begin() + i * t.width, rows.begin() + (i + 1) * t.width);
        return {std::move(opened), PrunedMerklePaths{std::move(pruned)}};
    }
};

/* Whir::serialize_batch_prover_data_into (whir.rs:542-560): the tree's
 * matrix and digest layers, framed as the batch cache stores them, streamed
 * from HBM to `os`. A failing stream throws zkie::Error (ZKIE_ERR_IO). */
inline void serialize_batch_prover_data_into(const MerkleTree& t, std::ostream& os)
{
    zkie_write_fn write = [](void* ctx, const void* bytes, uint64_t len) -> int {
        auto* s = static_cast<std::ostream*>(ctx);
        s->write(static_cast<const char*>(bytes), static_cast<std::streamsize>(len));
        return s->good() ? 0 : 1;
    };
    check(zkie_prover_data_write(t.mat.data(), t.height, t.width, t.layers.data(), write, &os, nullptr),
          "zkie_prover_data_write");
}

/* Whir::restore_batch_prover_data_from (whir.rs:572-602): a tree over an
 * h x w matrix (the table shape the caller knows) read from `is` into new
 * device buffers. Framing of another shape throws zkie::Error. */
inline MerkleTree restore_batch_prover_data_from(std::istream& is, size_t h, size_t w)
{
    MerkleTree t;
    t.height = h;
    t.width = w;
    uint32_t nl = 0;
    std::vector<uint64_t> lens(65);
    check(zkie_merkle_layout(h, &nl, lens.data()), "zkie_merkle_layout");
    lens.resize(nl);
    size_t total = 0;
    for (uint64_t l : lens) total += l;
    t.layer_lens = lens;
    t.mat = DeviceBuffer(h * w);
    t.layers = DeviceBuffer(total * 8);
    zkie_read_fn read = [](void* ctx, void* bytes, uint64_t len) -> int {
        auto* s = static_cast<std::istream*>(ctx);
        s->read(static_cast<char*>(bytes), static_cast<std::streamsize>(len));
        return s->gcount() == static_cast<std::streamsize>(len) ? 0 : 1;
    };
    check(zkie_prover_data_read(read, &is, h, w, t.mat.data(), t.layers.data(), t.root.data(), nullptr),
          "zkie_prover_data_read");
    return t;
}

/* The batch cache header (crates/zkie-core/src/pcs/cache.rs:7-70):
 * write_header stores (BATCH_CACHE_MAGIC, BatchCacheMetadata, Commitment) the
 * way bincode 1.3.3's serialize_into encodes that tuple (Cargo.lock pins
 * bincode 1.3.3): integers fixed-width little-endian, strings and sequences
 * preceded by their length as a u64, fixed-size arrays, tuples and structs
 * field by field in declaration order, nothing else. The commitment is
 * p3's MerkleCap<F, [F; 8]>, a sequence of digests (cap height 0: one), each
 * field element a u64. The prover data (serialize_batch_prover_data_into)
 * follows the header in the cache file (whir.rs:887-889). */
constexpr uint32_t kBatchCacheSchemaVersion = 2;  // cache.rs:7
constexpr char kBatchCacheMagic[8] = {'Z', 'K', 'I', 'E', 'B', 'C', 'H', '2'};

/* BatchCacheMetadata (cache.rs:10-22). */
struct BatchCacheMetadata {
    uint32_t schema_version = kBatchCacheSchemaVersion;
    std::string model_id;
    std::string group_id;
    std::vector<std::string> table_ids;  // ordered model tensors: position = committed table index
    uint32_t table_arity = 0;
    uint32_t num_tables = 0;
    uint32_t security_level = 0;
    uint32_t pow_bits = 0;
    std::array<uint8_t, 32> source_digest{};

    bool operator==(const BatchCacheMetadata& o) const
    {
        return schema_version == o.schema_version && model_id == o.model_id && group_id == o.group_id &&
               table_ids == o.table_ids && table_arity == o.table_arity && num_tables == o.num_tables &&
               security_level == o.security_level && pow_bits == o.pow_bits && source_digest == o.source_digest;
    }
};

namespace detail {
inline void put_u32(std::ostream& os, uint32_t v)
{
    char b[4];
    for (int i = 0; i < 4; i++) b[i] = static_cast<char>((v >> (8 * i)) & 0xFF);
    os.write(b, 4);
}
inline void put_u64(std::ostream& os, uint64_t v)
{
    char b[8];
    for (int i = 0; i < 8; i++) b[i] = static_cast<char>((v >> (8 * i)) & 0xFF);
    os.write(b, 8);
}
inline void put_str(std::ostream& os, const std::string& s)
{
    put_u64(os, s.size());
    os.write(s.data(), static_cast<std::streamsize>(s.size()));
}
inline void get_bytes(std::istream& is, char* dst, size_t n)
{
    is.read(dst, static_cast<std::streamsize>(n));
    if (is.gcount() != static_cast<std::streamsize>(n)) throw Error(ZKIE_ERR_IO, "read_header: short stream");
}
inline uint64_t get_uint(std::istream& is, int bytes)
{
    unsigned char b[8] = {0};
    get_bytes(is, reinterpret_cast<char*>(b), static_cast<size_t>(bytes));
    uint64_t v = 0;
    for (int i = bytes; i-- > 0;) v = (v << 8) | b[i];
    return v;
}
// Lengths beyond this are refused instead of allocated (a corrupt header).
constexpr uint64_t kMaxHeaderLen = uint64_t(1) << 24;
inline uint64_t get_len(std::istream& is)
{
    const uint64_t n = get_uint(is, 8);
    if (n > kMaxHeaderLen) throw Error(ZKIE_ERR_INVALID, "read_header: length out of range");
    return n;
}
inline std::string get_str(std::istream& is)
{
    std::string s(get_len(is), '\0');
    if (!s.empty()) get_bytes(is, &s[0], s.size());
    return s;
}
}  // namespace detail

/* cache::write_header (cache.rs:51-58). The metadata's table count must
 * match its table identifiers (BatchCacheMetadata::new, cache.rs:36). */
inline void write_header(std::ostream& os, const BatchCacheMetadata& m, const MerkleCap& commitment)
{
    if (m.schema_version != kBatchCacheSchemaVersion || m.table_ids.size() != m.num_tables)
        throw Error(ZKIE_ERR_INVALID, "write_header: metadata");
    os.write(kBatchCacheMagic, 8);
    detail::put_u32(os, m.schema_version);
    detail::put_str(os, m.model_id);
    detail::put_str(os, m.group_id);
    detail::put_u64(os, m.table_ids.size());
    for (const auto& id : m.table_ids) detail::put_str(os, id);
    detail::put_u32(os, m.table_arity);
    detail::put_u32(os, m.num_tables);
    detail::put_u32(os, m.security_level);
    detail::put_u32(os, m.pow_bits);
    os.write(reinterpret_cast<const char*>(m.source_digest.data()), 32);
    detail::put_u64(os, commitment.size());
    for (const auto& d : commitment)
        for (F x : d) detail::put_u64(os, x);
    if (!os.good()) throw Error(ZKIE_ERR_IO, "write_header");
}

/* cache::read_header (cache.rs:60-70): refuses another magic or schema
 * version, as the reference does. */
inline std::pair<BatchCacheMetadata, MerkleCap> read_header(std::istream& is)
{
    char magic[8];
    detail::get_bytes(is, magic, 8);
    BatchCacheMetadata m;
    m.schema_version = static_cast<uint32_t>(detail::get_uint(is, 4));
    if (std::string(magic, 8) != std::string(kBatchCacheMagic, 8) || m.schema_version != kBatchCacheSchemaVersion)
        throw Error(ZKIE_ERR_INVALID, "read_header: unsupported batch cache format");
    m.model_id = detail::get_str(is);
    m.group_id = detail::get_str(is);
    const uint64_t n = detail::get_len(is);
    for (uint64_t i = 0; i < n; i++) m.table_ids.push_back(detail::get_str(is));
    m.table_arity = static_cast<uint32_t>(detail::get_uint(is, 4));
    m.num_tables = static_cast<uint32_t>(detail::get_uint(is, 4));
    m.security_level = static_cast<uint32_t>(detail::get_uint(is, 4));
    m.pow_bits = static_cast<uint32_t>(detail::get_uint(is, 4));
    detail::get_bytes(is, reinterpret_cast<char*>(m.source_digest.data()), 32);
    MerkleCap cap(detail::get_len(is));
    for (auto& d : cap)
        for (F& x : d) x = detail::get_uint(is, 8);
    return {std::move(m), std::move(cap)};
}

/* Row fold (prover/mod.rs:257-290; mle.rs:8-22 with variable 0 the least
 * significant bit) of every row of a device matrix of 2^k (EF: 2^(k+1)) u64 per row. */
inline std::vector<Ef> fold_rows(const DeviceBuffer& d_mat, size_t h, uint32_t k, bool is_ext,
                                 const std::vector<Ef>& r)
{
    if (r.size() != k) throw Error(ZKIE_ERR_INVALID, "fold_rows challenges");
    DeviceBuffer out(2 * h);
    check(zkie_fold_rows(d_mat.data(), h, k, is_ext ? 1 : 0, ef_ptr(r), out.data(), nullptr),
          "zkie_fold_rows");
    const std::vector<F> v = out.download();
    std::vector<Ef> res(h);
    for (size_t i = 0; i < h; i++) res[i] = {v[2 * i], v[2 * i + 1]};
    return res;
}

/* Out-of-domain answer: the multilinear extension of a device table at r. */
inline Ef mle_eval(const DeviceBuffer& d_vals, uint32_t num_vars, bool is_ext, const std::vector<Ef>& r)
{
    if (r.size() != num_vars) throw Error(ZKIE_ERR_INVALID, "mle_eval point");
    Ef out{};
    check(zkie_mle_eval(d_vals.data(), num_vars, is_ext ? 1 : 0, ef_ptr(r), out.data(), nullptr), "zkie_mle_eval");
    return out;
}

/* sumcheck::prove's result (sumcheck.rs:10-30) with EF values: one round
 * polynomial c0 + c1 X + c2 X^2 per round and the two tables' final values. */
struct RoundPoly {
    Ef c0, c1, c2;
};
struct SumcheckProof {
    std::vector<RoundPoly> rounds;
    Ef f_eval, h_eval;
};

/* sumcheck::prove (sumcheck.rs:33-79) of sum_x f(x) h(x) over device tables of
 * 2^num_vars entries (f base or EF, h EF) with the challenges given up front,
 * one per variable. */
inline SumcheckProof sumcheck_prove(const DeviceBuffer& d_f, bool f_is_ext, const DeviceBuffer& d_h,
                                    uint32_t num_vars, const std::vector<Ef>& challenges)
{
    if (challenges.size() != num_vars) throw Error(ZKIE_ERR_INVALID, "sumcheck challenges");
    std::vector<F> polys(6 * (num_vars ? num_vars : 1));
    DeviceBuffer f_out(2), h_out(2);
    check(zkie_sumcheck_prove(d_f.data(), f_is_ext ? 1 : 0, d_h.data(), num_vars, num_vars,
                              num_vars ? ef_ptr(challenges) : polys.data(), polys.data(), f_out.data(),
                              h_out.data(), nullptr),
          "zkie_sumcheck_prove");
    SumcheckProof p;
    for (uint32_t i = 0; i < num_vars; i++)
        p.rounds.push_back({Ef{polys[6 * i], polys[6 * i + 1]}, Ef{polys[6 * i + 2], polys[6 * i + 3]},
                            Ef{polys[6 * i + 4], polys[6 * i + 5]}});
    const std::vector<F> fe = f_out.download(), he = h_out.download();
    p.f_eval = {fe[0], fe[1]};
    p.h_eval = {he[0], he[1]};
    return p;
}

}  // namespace zkie
