/*
 * zkie_hip.h — C ABI of the MI355X (gfx950) shard-commitment library
 * (libzkie_hip.so): coset/subgroup LDE over Goldilocks, Poseidon2 Merkle
 * commitment with openings, and the WHIR/FRI row fold.
 *
 * Conventions (same as the reference FFI, crates/zkie-core/src/pcs/cuda_ffi.rs):
 *  - every function returns int: 0 on success, a hipError_t value when the
 *    HIP runtime fails, or a negative ZKIE_ERR_* code for bad arguments. The
 *    library never falls back to a CPU path; callers that want one keep it on
 *    their side, as dft_cuda.rs:174-177 and merkle_cuda.rs:328-335 do;
 *  - matrices are row-major u64 arrays of canonical Goldilocks elements
 *    (p = 2^64 - 2^32 + 1), digests are 8 contiguous u64, digest layers are
 *    stored back to back ([layer0 | layer1 | ... | root]);
 *  - pointers named d_* are device pointers owned by the caller; other
 *    pointers are host memory;
 *  - `stream` is a hipStream_t (NULL = the null stream). Entry points that
 *    return host data synchronise that stream before returning.
 *
 * Reference paths are relative to the zkIE repository root.
 */
#ifndef ZKIE_HIP_H
#define ZKIE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ZKIE_OK 0
#define ZKIE_ERR_INVALID (-1)     /* argument out of range or inconsistent */
#define ZKIE_ERR_NO_DEVICE (-2)   /* no HIP device */
#define ZKIE_ERR_ALLOC (-3)       /* device workspace allocation failed */
#define ZKIE_ERR_IO (-4)          /* a caller's write or read callback failed */
#define ZKIE_ERR_SCRATCH_LIMIT (-5) /* larger than a no-alloc entry point's fixed scratch */

/* ------------------------------------------------------------------------
 * Device and memory. Replace the raw CUDA runtime imports of
 * crates/zkie-core/src/pcs/cuda_ffi.rs:41-45 (cudaMalloc, cudaFree,
 * cudaMemcpy, cudaDeviceSynchronize, cudaMemset) and the device count of
 * crates/zkie-core/cuda/poseidon2_merkle.cu:315-318 (zkie_cuda_device_count).
 * ---------------------------------------------------------------------- */
int zkie_device_count(void);
int zkie_dev_alloc(void **d_ptr, size_t bytes);
int zkie_dev_free(void *d_ptr);
int zkie_memcpy_htod(void *d_dst, const void *src, size_t bytes);
int zkie_memcpy_dtoh(void *dst, const void *d_src, size_t bytes);
int zkie_memcpy_dtod(void *d_dst, const void *d_src, size_t bytes, void *stream);
int zkie_memset(void *d_ptr, int value, size_t bytes);
int zkie_device_synchronize(void);
int zkie_stream_synchronize(void *stream);
/* Streams for overlapping independent stages (no reference counterpart: the
 * reference runs everything on the legacy default stream, merkle_cuda.rs:282).
 * zkie_stream_create makes a non-blocking stream of the default priority;
 * zkie_stream_wait makes work queued on `waiter` afterwards wait for the work
 * queued on `signaler` so far. */
int zkie_stream_create(void **stream);
int zkie_stream_destroy(void *stream);
int zkie_stream_wait(void *waiter, void *signaler);

/* ------------------------------------------------------------------------
 * Reference-compatible kernels (same names, arguments and semantics as
 * crates/zkie-core/src/pcs/cuda_ffi.rs:2-39).
 * ---------------------------------------------------------------------- */

/* goldilocks_ntt.cu:105-137. Forward DFT of every column of the row-major
 * h x w matrix d_mat (h = 2^lg_h), in place, natural order in and out, on
 * TWO_ADIC_GENERATORS[lg_h]; d_temp is caller scratch of h*w u64. d_tw is
 * accepted for ABI compatibility and may be NULL: the library generates the
 * identical twiddles itself (dft_cuda.rs:44-59) and has no 2^18 size cap. */
int zkie_ntt_forward_goldilocks(uint64_t *d_mat, uint64_t *d_temp, uint32_t lg_h, uint64_t w,
                                const uint64_t *d_tw);

/* poseidon2_merkle.cu:252-264. rc_init/rc_final: 4 rounds x 16 host u64 each,
 * rc_internal: 22 host u64, diag15: MATRIX_DIAG_16_GOLDILOCKS[15]. Applies to
 * the current device; every later hashing entry point uses them. */
int zkie_p2_upload_constants(const uint64_t *rc_init, const uint64_t *rc_final,
                             const uint64_t *rc_internal, uint64_t diag15);

/* poseidon2_merkle.cu:266-275: leaf digests of rows [0, 8*floor(h/8)). */
int zkie_p2_leaf_batch(const uint64_t *d_mat, uint64_t *d_digests, uint32_t h, uint32_t w);
/* poseidon2_merkle.cu:277-287: leaf digests of rows [start_row, h). */
int zkie_p2_leaf_scalar(const uint64_t *d_mat, uint64_t *d_digests, uint32_t start_row,
                        uint32_t h, uint32_t w);
/* poseidon2_merkle.cu:289-299: parents [0, 8*floor(next_len/8)) of `step`
 * children each (TruncatedPermutation<Perm, 2, 8, 16>). */
int zkie_p2_compress_batch(const uint64_t *d_prev, uint64_t *d_next, uint32_t next_len,
                           uint32_t step);
/* poseidon2_merkle.cu:301-311: parents [from, to). */
int zkie_p2_compress_scalar(const uint64_t *d_prev, uint64_t *d_next, uint32_t from,
                            uint32_t to, uint32_t step);

/* ------------------------------------------------------------------------
 * Device-resident path. The codeword and the digest layers stay in HBM
 * between stages, unlike the reference's per-stage H2D/D2H round trips
 * (dft_cuda.rs:203,213; merkle_cuda.rs:227,288-306).
 * ---------------------------------------------------------------------- */

/* merkle_cuda.rs:54-85 (derive_poseidon2_constants): the constants of
 * Poseidon2Goldilocks<16>::new_from_rng_128(SmallRng::seed_from_u64(1)),
 * derived on the host; pass them to zkie_p2_upload_constants. The library
 * uploads them by itself on first use when the caller never did. */
int zkie_p2_default_constants(uint64_t rc_init[64], uint64_t rc_final[64],
                              uint64_t rc_internal[22], uint64_t *diag15);

/* TwoAdicSubgroupDft::dft_batch (dft_cuda.rs:161-222, contract at
 * goldilocks_ntt.cu:3-23), in place on the device, any lg_h <= 32. */
int zkie_dft_batch(uint64_t *d_mat, uint32_t lg_h, uint64_t w, void *stream);
/* Inverse of zkie_dft_batch (evaluations -> coefficients), in place. */
int zkie_idft_batch(uint64_t *d_mat, uint32_t lg_h, uint64_t w, void *stream);
/* WHIR encode (p3-whir src/pcs/committer/writer.rs:73-81, Suffix order) and
 * coset LDE: treat the h x w matrix d_in as coefficient rows, zero-pad it to
 * n = h << log_blowup rows, scale row j by shift^j (shift = 1 is the
 * reference's plain subgroup encode), and write the n x w evaluations to
 * d_out. h must be a power of two. d_in and d_out must not overlap. */
int zkie_lde_batch(const uint64_t *d_in, uint64_t h, uint64_t w, uint32_t log_blowup,
                   uint64_t shift, uint64_t *d_out, void *stream);

/* No counterpart in the reference. zkie_lde_batch for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc. Same arguments, semantics and results as
 * zkie_lde_batch; its work buffers live in a fixed array in device memory of
 * the library (64 MiB plus 1 MiB per device that loads it, held until the
 * process ends) instead of being allocated, so it calls no hipMalloc or
 * hipFree. The first call on a device (with that device current) looks up the
 * array and fills the twiddle tables. Sizes with (h << log_blowup) * w above
 * 2^23 u64 return ZKIE_ERR_SCRATCH_LIMIT. All calls on one device share the
 * array: calls that overlap on one device (unordered streams, or host
 * threads) race; order them. */
int zkie_lde_batch_noalloc(const uint64_t *d_in, uint64_t h, uint64_t w, uint32_t log_blowup,
                           uint64_t shift, uint64_t *d_out, void *stream);

/* Tree geometry of MerkleTree::new for one matrix of height h, arity 2
 * (p3-merkle-tree merkle_tree.rs:95-178, padded_len at :577-585; the same
 * schedule as merkle_cuda.rs:203-209). layer_lens must hold 65 entries. */
int zkie_merkle_layout(uint64_t h, uint32_t *num_layers, uint64_t *layer_lens);
/* Mmcs::commit for one matrix (merkle_cuda.rs:177-312, mmcs/batch.rs:42-64):
 * hash every row of the h x w matrix d_mat with PaddingFreeSponge<Perm,16,8,8>,
 * compress layer by layer, zero digests in padded slots. d_layers holds
 * sum(layer_lens) * 8 u64. root (host, 8 u64, may be NULL) receives the cap
 * (cap height 0). */
int zkie_merkle_commit(const uint64_t *d_mat, uint64_t h, uint64_t w, uint64_t *d_layers,
                       uint64_t *root, void *stream);
/* The encode-then-commit of one WHIR commitment (p3-whir
 * src/pcs/committer/writer.rs:73-85, dft_batch then commit_matrix; the
 * initial round through adapter.rs:106-113) in one call: the results of
 * zkie_lde_batch(d_in, h, w, log_blowup, shift, d_out) followed by
 * zkie_merkle_commit(d_out, h << log_blowup, w, d_layers, root). For 16-wide
 * rows and a transform of more than one pass, the last NTT pass hashes the
 * rows it produces, so the codeword is not read back for the leaves. */
int zkie_lde_commit(const uint64_t *d_in, uint64_t h, uint64_t w, uint32_t log_blowup,
                    uint64_t shift, uint64_t *d_out, uint64_t *d_layers, uint64_t *root,
                    void *stream);
/* Whir::commit_batch (crates/zkie-core/src/pcs/whir.rs:476-525): `count`
 * tables of 2^arity evaluations each (device pointers, host array d_tables)
 * stacked table-major into one witness of total_vars = ceil(log2(count
 * 2^arity)) variables, zero-padded: entry j of table i is entry i 2^arity + j.
 * The witness, viewed as 2^(total_vars - log_width) rows of 2^log_width, is
 * committed as by zkie_lde_commit (shift 1). d_stack (2^total_vars u64) holds
 * the stacked witness on return, except that with log_blowup >= 1 the zero
 * rows past the tables are neither written nor read; a table already at its
 * place in d_stack is not copied, one overlapping another part of it is
 * refused. d_codeword holds 2^(total_vars - log_width + log_blowup) rows;
 * d_layers and root as for zkie_merkle_commit. The stacking order follows
 * the layout the reference hands to its external initial-round committer
 * (p3-whir adapter.rs:106-113); total_vars >= log_width. */
int zkie_commit_batch(const uint64_t *const *d_tables, uint32_t count, uint32_t arity,
                      uint32_t log_width, uint32_t log_blowup, uint64_t *d_stack,
                      uint64_t *d_codeword, uint64_t *d_layers, uint64_t *root, void *stream);
/* Mmcs::open_batch (p3-merkle-tree mmcs/batch.rs:75-121) for n indices at
 * once: rows_out (host, n*w u64) receives the opened rows, siblings_out
 * (host, n*(num_layers-1)*8 u64) the authentication paths, bottom-up. */
int zkie_merkle_open_batch(const uint64_t *d_mat, uint64_t h, uint64_t w,
                           const uint64_t *d_layers, const uint64_t *indices, uint64_t n,
                           uint64_t *rows_out, uint64_t *siblings_out, void *stream);
/* Mmcs::open_multi_batch / open_batch_pruned (p3-merkle-tree mmcs/mod.rs:309-461,
 * pruning.rs:130-232): rows_out as above (input order), pruned_out (host,
 * capacity `cap` digests) the boundary siblings in frontier order; *count is
 * the number of digests of the proof (may exceed cap, then nothing past cap
 * is written and ZKIE_ERR_INVALID is returned). */
int zkie_merkle_open_pruned(const uint64_t *d_mat, uint64_t h, uint64_t w,
                            const uint64_t *d_layers, const uint64_t *indices, uint64_t n,
                            uint64_t *rows_out, uint64_t *pruned_out, uint64_t cap,
                            uint64_t *count, void *stream);

/* Row fold of the WHIR prover (p3-whir src/pcs/prover/mod.rs:257-290, equal to
 * zkIE's mle::eval at common/mle.rs:8-22 with variable 0 the least-significant
 * index bit): out[t] = sum_j eq(r, j) * row_t[j] over the 2^log_width entries
 * of each of the h rows. Rows are base elements (is_ext = 0, 2^log_width u64)
 * or EF = F[x]/(x^2 - 7) elements flattened [c0, c1] (is_ext = 1). r (host)
 * holds log_width EF challenges (2*log_width u64); d_out receives h EF
 * elements (2h u64). log_width <= 8. */
int zkie_fold_rows(const uint64_t *d_mat, uint64_t h, uint32_t log_width, int is_ext,
                   const uint64_t *r, uint64_t *d_out, void *stream);

/* Queried-row fold of a STIR round (p3-whir src/pcs/prover/mod.rs:265-290,
 * Poly::eval_base / eval_ext of each opened row): the same fold as
 * zkie_fold_rows applied to rows indices[0..n) (host, each < h) of the
 * device matrix only; out (host) receives n EF elements (2n u64). */
int zkie_fold_rows_at(const uint64_t *d_mat, uint64_t h, uint32_t log_width, int is_ext,
                      const uint64_t *indices, uint64_t n, const uint64_t *r, uint64_t *out,
                      void *stream);

/* Multilinear evaluation of a device table of 2^num_vars entries (base, or
 * EF flattened [c0, c1] when is_ext) at an EF point: sum_j eq(r, j) * v[j]
 * with coordinate 0 the least-significant index bit (common/mle.rs:8-22).
 * This is the out-of-domain answer `sumcheck_prover.eval(&point)` of a WHIR
 * round (p3-whir src/pcs/prover/mod.rs:226-236); a p3 point, most
 * significant variable first, is passed reversed, as the row fold does
 * (prover/mod.rs:258-261). r (host): num_vars EF coordinates; out (host): one
 * EF element (2 u64). The table never leaves HBM. */
int zkie_mle_eval(const uint64_t *d_vals, uint32_t num_vars, int is_ext, const uint64_t *r,
                  uint64_t *out, void *stream);

/* Sumcheck of sum_x f(x) h(x) over tables of 2^num_vars entries, the round
 * polynomials a WHIR round sends before it folds (compute_sumcheck_polynomials,
 * p3-whir src/pcs/prover/mod.rs:309-315), with the round and fold rules of
 * zkIE's sumcheck::prove (crates/zkie-core/src/common/sumcheck.rs:33-89):
 * entries (2s, 2s+1) pair up (variable 0 is the least-significant index bit),
 * the round polynomial c0 + c1 X + c2 X^2 interpolates sum_s f(X) h(X) at
 * X = 0, 1, 2, and binding variable 0 to r maps a table a to
 * a[2s] + r (a[2s+1] - a[2s]). f is base (f_is_ext = 0) or EF, h is EF, all
 * EF flattened [c0, c1]; challenges and coefficients are EF.
 *
 * zkie_sumcheck_round: the current round's polynomial; poly (host) receives
 * c0, c1, c2 (6 u64). num_vars >= 1. */
int zkie_sumcheck_round(const uint64_t *d_f, int f_is_ext, const uint64_t *d_h, uint32_t num_vars,
                        uint64_t *poly, void *stream);
/* zkie_sumcheck_fold: both tables bound at variable 0 to r (host, one EF);
 * d_f_out and d_h_out receive 2^(num_vars-1) EF entries each and must not
 * overlap the inputs or each other. With next_poly (host, 6 u64) non-NULL
 * (num_vars >= 2) the same pass also forms the next round's polynomial, as
 * zkie_sumcheck_round on the outputs would, and the call synchronises;
 * with next_poly NULL it does not. */
int zkie_sumcheck_fold(const uint64_t *d_f, int f_is_ext, const uint64_t *d_h, uint32_t num_vars,
                       const uint64_t *r, uint64_t *d_f_out, uint64_t *d_h_out, uint64_t *next_poly,
                       void *stream);
/* zkie_eq_table: the weight table of one evaluation constraint,
 * d_out[x] = eq(point, x) = prod_b (x_b ? p_b : 1 - p_b) for x < 2^num_vars
 * (EF, bit 0 of x first, mle.rs:44-56), so that sum_x eq(p, x) f(x) = f(p)
 * (mle.rs:8-22). point (host): num_vars EF coordinates. */
int zkie_eq_table(const uint64_t *point, uint32_t num_vars, uint64_t *d_out, void *stream);
/* The batched constraint of a WHIR round (p3-whir src/pcs/prover/mod.rs:228-314):
 * the out-of-domain claims as evaluation constraints (Statements::Eq) and the
 * STIR openings as selection constraints (Statements::Select), combined by the
 * powers of gamma into one weight table over the round table of 2^num_vars
 * entries, the weights its sumcheck adds to its own:
 *   d_w[x] (+)= sum_{j<m} gamma^j eq(p_j, x) + sum_{k<q} gamma^(m+k) z_k^x
 * (EF flattened [c0, c1]; eq as zkie_eq_table, bit b of x variable b; z^x the
 * powers of a univariate point, so that sum_x f(x) z^x is the value at z of
 * the polynomial whose coefficients are the table, i.e. the queried-row fold).
 * eq_points (host): m points of num_vars EF coordinates; sel_points (host): q
 * EF points; gamma (host): one EF. accumulate = 1 adds to d_w, 0 overwrites
 * it. The call does not wait for the host or the device. The order of the
 * powers (the Eq group first, from gamma^0) restates Constraint::new of the
 * external p3-sumcheck crate. */
int zkie_constraint_weights(const uint64_t *eq_points, uint32_t m, const uint64_t *sel_points,
                            uint32_t q, const uint64_t *gamma, uint32_t num_vars, int accumulate,
                            uint64_t *d_w, void *stream);
/* zkie_sumcheck_prove: `rounds` rounds with the challenges r (host, rounds EF)
 * given up front, as sumcheck::prove takes them: polys (host) receives
 * 6 u64 per round, d_f_out / d_h_out the tables after the last fold
 * (2^(num_vars-rounds) EF entries each; with rounds = num_vars, f(r) and
 * h(r)). The outputs must not overlap the inputs or each other. */
int zkie_sumcheck_prove(const uint64_t *d_f, int f_is_ext, const uint64_t *d_h, uint32_t num_vars,
                        uint32_t rounds, const uint64_t *r, uint64_t *polys, uint64_t *d_f_out,
                        uint64_t *d_h_out, void *stream);

/* Encoding of commit_extension (p3-whir src/pcs/committer/writer.rs:21-86):
 * the 2^num_vars-entry table (base or EF) as a 2^(num_vars - log_width) x
 * 2^log_width matrix, rows as stored (prefix = 0, VariableOrder::Suffix) or
 * transposed (prefix = 1, VariableOrder::Prefix, writer.rs:43-71), zero-padded
 * to 2^log_inv_rate times its height and transformed per base column
 * (dft_algebra_batch). d_out receives 2^(num_vars + log_inv_rate) entries
 * (times 2 u64 for EF), row-major. For prefix = 1 the buffers must not overlap. */
int zkie_whir_encode(const uint64_t *d_poly, uint32_t num_vars, int is_ext, uint32_t log_width,
                     uint32_t log_inv_rate, int prefix, uint64_t *d_out, void *stream);

/* ------------------------------------------------------------------------
 * Prover-data cache stream. Replaces Whir::serialize_batch_prover_data_into
 * and Whir::restore_batch_prover_data_from (crates/zkie-core/src/pcs/
 * whir.rs:542-602, with MerkleTree::write_digest_layers / read_digest_layers
 * of vendor/p3-merkle-tree/src/merkle_tree.rs:223-276): the bytes of a
 * committed tree that follow the ZKIEBCH2 header of the batch cache
 * (pcs/cache.rs:50-57), streamed straight from and to HBM. All integers are
 * u64 little-endian:
 *   1 | w | h*w | the h x w matrix | L | L layer lengths | L-1 arities (2) |
 *   the digest layers (8 u64 per digest, leaves first).
 * The callbacks receive consecutive pieces of that stream, in order; they
 * return 0 to continue, anything else stops the call with ZKIE_ERR_IO. A read
 * callback must fill all `len` bytes. The payload moves through pinned
 * staging buffers, the copy of the next piece overlapping the callback.
 * ---------------------------------------------------------------------- */
typedef int (*zkie_write_fn)(void *ctx, const void *bytes, uint64_t len);
typedef int (*zkie_read_fn)(void *ctx, void *bytes, uint64_t len);
/* Total stream length for a tree over an h x w matrix. */
int zkie_prover_data_size(uint64_t h, uint64_t w, uint64_t *bytes);
/* whir.rs:542-560: the tree of zkie_merkle_commit (d_mat, d_layers) as bytes. */
int zkie_prover_data_write(const uint64_t *d_mat, uint64_t h, uint64_t w,
                           const uint64_t *d_layers, zkie_write_fn write, void *ctx,
                           void *stream);
/* whir.rs:572-602: reads a stream written for an h x w matrix back into
 * d_mat (h*w u64) and d_layers (sum(layer_lens) * 8 u64). Framing that does
 * not describe a tree of that shape (leaf-matrix count, width, value count,
 * layer count, layer lengths, arities) returns ZKIE_ERR_INVALID before any of
 * the part it announces is read. root (host, may be NULL) receives the last
 * digest layer. */
int zkie_prover_data_read(zkie_read_fn read, void *ctx, uint64_t h, uint64_t w, uint64_t *d_mat,
                          uint64_t *d_layers, uint64_t *root, void *stream);

/* ------------------------------------------------------------------------
 * Synthetic inputs (host): XorShift64 of common/field.rs:17-36 seeded with
 * `seed`, embedded like common/fixed_point.rs:11-38. ZKIE_GEN_UNIFORM:
 * next_u64() mod p; ZKIE_GEN_I16: (next_u64() % 65536) as i16;
 * ZKIE_GEN_I8: (next_u64() % 255) - 127; ZKIE_GEN_GAUSS_I16: integer
 * Irwin-Hall N(0,1) (sum of 12 next_u64() >> 11, scaled 2^-53, minus 6)
 * times 0.02 * 2^12, rounded half up, clamped to int16.
 * ---------------------------------------------------------------------- */
#define ZKIE_GEN_UNIFORM 0
#define ZKIE_GEN_I16 1
#define ZKIE_GEN_I8 2
#define ZKIE_GEN_GAUSS_I16 3
int zkie_gen_inputs(uint64_t seed, uint64_t n, int kind, uint64_t *out);

/* ------------------------------------------------------------------------
 * Kernel timers (no reference counterpart; stands in for the per-Whir
 * commit_stats counters of whir.rs:270-273,361-370). When enabled, each
 * kernel launch is bracketed by HIP events on its own stream.
 * ---------------------------------------------------------------------- */
int zkie_profile_enable(int on);
int zkie_profile_reset(void);
/* Totals for one kernel name since the last reset (synchronises the device). */
int zkie_profile_query(const char *kernel, uint64_t *launches, double *total_ms);
/* Newline-separated kernel names seen since the last reset. */
int zkie_profile_names(char *buf, size_t cap);

#ifdef __cplusplus
}
#endif
#endif /* ZKIE_HIP_H */
