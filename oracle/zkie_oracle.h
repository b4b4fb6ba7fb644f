/*
 * zkie_oracle.h — CPU restatement of the zkIE shard-commitment path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: it is loaded by
 * tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg, and
 * by nothing else. The product path (zkie_amd/, libzkie_hip.so) never links,
 * loads or calls it.
 *
 * Every function restates the reference algorithm it cites (paths relative to
 * the reference repository root). All values are canonical u64 Goldilocks
 * elements on input and output unless stated otherwise.
 */
#ifndef ZKIE_ORACLE_H
#define ZKIE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_P 0xFFFFFFFF00000001ULL

/* ---- field F = GF(p), p = 2^64 - 2^32 + 1 (external p3-goldilocks 0.7.0) ---- */
uint64_t or_add(uint64_t a, uint64_t b);
uint64_t or_sub(uint64_t a, uint64_t b);
uint64_t or_mul(uint64_t a, uint64_t b);
uint64_t or_pow(uint64_t a, uint64_t e);
uint64_t or_inv(uint64_t a);
/* EF = F[x]/(x^2 - 7): a = (a[0], a[1]) */
void or_ef_mul(const uint64_t a[2], const uint64_t b[2], uint64_t out[2]);

/* TWO_ADIC_GENERATORS[k] = 7^((p-1)/2^k), k <= 32 (dft_cuda.rs:44-59 uses the p3 table). */
uint64_t or_two_adic_generator(uint32_t k);

/* ---- DFT: TwoAdicSubgroupDft::dft_batch contract (goldilocks_ntt.cu:3-23) ---- */
/* In place over a row-major h x w matrix, h = 2^lg_h, column-wise, natural order. */
void or_dft_batch(uint64_t *mat, uint32_t lg_h, uint64_t w);
/* O(h^2) definition, out[i][c] = sum_j in[j][c] * w_h^(i*j). */
void or_dft_naive(const uint64_t *in, uint64_t *out, uint32_t lg_h, uint64_t w);
/* Horner evaluation of column c of an h x w coefficient matrix at x. */
uint64_t or_poly_eval(const uint64_t *mat, uint64_t h, uint64_t w, uint64_t c, uint64_t x);
/* Polynomial fingerprint sum_i v[i] z^i mod p. */
uint64_t or_checksum(const uint64_t *v, uint64_t n, uint64_t z);
/* Inverse DFT (evaluations -> coefficients), in place. */
void or_idft_batch(uint64_t *mat, uint32_t lg_h, uint64_t w);
/* WHIR encode / LDE (p3-whir writer.rs:73-81): zero-pad the h x w coefficient
 * matrix to (h << log_blowup) rows, optionally scale row j by shift^j (coset),
 * then dft_batch. out has (h << log_blowup) * w entries. */
void or_lde_batch(const uint64_t *in, uint64_t h, uint64_t w, uint32_t log_blowup,
                  uint64_t shift, uint64_t *out);

/* ---- Poseidon2-Goldilocks-16 (poseidon2_merkle.cu:31-155, merkle_cuda.rs:54-85) ---- */
void or_p2_derive_constants(uint64_t rc_init[64], uint64_t rc_final[64],
                            uint64_t rc_internal[22], uint64_t *diag15);
void or_p2_set_constants(const uint64_t rc_init[64], const uint64_t rc_final[64],
                         const uint64_t rc_internal[22], uint64_t diag15);
void or_p2_permute(uint64_t st[16]);
/* Linear layers alone (for structural checks). */
void or_p2_mds_light(uint64_t st[16]);
void or_p2_internal_linear(uint64_t st[16]);
/* PaddingFreeSponge<Perm,16,8,8>::hash_iter over one row (merkle_tree.rs:372-442). */
void or_leaf_hash(const uint64_t *row, uint64_t w, uint64_t out[8]);
/* TruncatedPermutation<Perm,2,8,16>::compress (merkle_tree.rs:594-642). */
void or_compress(const uint64_t left[8], const uint64_t right[8], uint64_t out[8]);

/* ---- rand 0.10 SmallRng (Xoshiro256++) seeded by SplitMix64 ---- */
typedef struct { uint64_t s[4]; } or_xoshiro;
void or_xoshiro_seed_u64(or_xoshiro *r, uint64_t seed);
void or_xoshiro_from_state(or_xoshiro *r, const uint64_t s[4]);
uint64_t or_xoshiro_next(or_xoshiro *r);
uint64_t or_splitmix64_next(uint64_t *state);

/* ---- Merkle tree geometry and openings (p3-merkle-tree, vendored) ---- */
/* padded_len(raw, 2) (merkle_tree.rs:577-585). */
uint64_t or_padded_len(uint64_t raw, uint64_t n);
/* Number of digest layers and their lengths for a single matrix of height h. */
uint32_t or_merkle_num_layers(uint64_t h);
void or_merkle_layer_lens(uint64_t h, uint64_t *lens);
/* Build all layers into `layers` (concatenated, 8 u64 per digest, zero
 * digests in padded slots). compressor: 0 = Poseidon2, 1 = XOR dummy
 * (merkle_tree.rs:661-672 test helper, digest-wise XOR). */
void or_merkle_build_layers(const uint64_t *layers0_digests, uint64_t h,
                            uint64_t *layers, int compressor);
/* compress() step alone (merkle_tree.rs:594-642): prev_len digests in, returns
 * padded_len(prev_len / 2, 2) digests written to next. */
uint64_t or_merkle_compress_layer(const uint64_t *prev, uint64_t prev_len, uint64_t *next,
                                  int compressor);
/* Leaf digests only: digests[i] = leaf_hash(row i), i < h (no padding). */
void or_merkle_leaf_digests(const uint64_t *mat, uint64_t h, uint64_t w, uint64_t *digests);
/* Full commit: layers (concatenated) + root copy. */
void or_merkle_commit(const uint64_t *mat, uint64_t h, uint64_t w, uint64_t *layers,
                      uint64_t root[8]);
/* open_batch (mmcs/batch.rs:75-121): siblings bottom-up, (num_layers-1) digests. */
void or_merkle_open(const uint64_t *layers, uint64_t h, uint64_t index, uint64_t *siblings);
/* open_batch_pruned sibling list (mmcs/mod.rs:309-461, pruning.rs:130-232).
 * Returns the number of digests written into out (capacity cap digests). */
uint64_t or_merkle_open_pruned(const uint64_t *layers, uint64_t h, const uint64_t *indices,
                               uint64_t n, uint64_t *out, uint64_t cap);
/* verify_batch for one row (mmcs/batch.rs:158-296), cap height 0: returns 1 if ok. */
int or_merkle_verify(const uint64_t root[8], uint64_t h, uint64_t index, const uint64_t *row,
                     uint64_t w, const uint64_t *siblings);

/* ---- fold (mle.rs:8-22; p3-whir prover/mod.rs:257-290) ---- */
/* out[t] = mle::eval(row_t, r) for each of h rows of 2^k elements; rows are base
 * (is_ext = 0, 2^k u64) or EF (is_ext = 1, 2^(k+1) u64 flattened [c0,c1]).
 * r holds k EF challenges (2k u64). out holds h EF elements (2h u64). */
void or_fold_rows(const uint64_t *mat, uint64_t h, uint32_t k, int is_ext, const uint64_t *r,
                  uint64_t *out);
/* mle::eval over base values and base point (mle.rs:8-22). */
uint64_t or_mle_eval_base(const uint64_t *values, uint32_t t, const uint64_t *point);
/* mle::eval (mle.rs:8-22) over base (is_ext = 0) or EF values at an EF point
 * (t coordinates, 2t u64), variable 0 first (the least-significant bit):
 * the out-of-domain answer of a WHIR round. out: one EF element. */
void or_mle_eval(const uint64_t *values, uint32_t t, int is_ext, const uint64_t *point, uint64_t out[2]);

/* ---- sumcheck of a product of two multilinear tables (common/sumcheck.rs:33-89) ---- */
/* `rounds` rounds of sumcheck::prove over sum_x f(x) h(x), 2^t entries, f base
 * (f_is_ext = 0) or EF, h EF (flattened [c0, c1]), challenges r (rounds EF).
 * Round i pairs entries (2s, 2s+1) (variable 0 = the least-significant index
 * bit), sums y_X = sum_s f(X) h(X) at X = 0, 1, 2 (f(2) = 2 f1 - f0), writes
 * c0 = y0, c1 = (4 y1 - y2 - 3 y0) / 2, c2 = (y2 - 2 y1 + y0) / 2 as 3 EF to
 * polys + 6i, then folds both tables, b[i] = a0 + r (a1 - a0). f_out and h_out
 * receive the folded EF tables (2^(t-rounds) entries each). */
void or_sumcheck_prove(const uint64_t *f, int f_is_ext, const uint64_t *h, uint32_t t, uint32_t rounds,
                       const uint64_t *r, uint64_t *polys, uint64_t *f_out, uint64_t *h_out);

/* eq(p, x) = prod_b (x_b ? p_b : 1 - p_b) for x < 2^t, bit 0 first (mle.rs:44-56),
 * EF point (t coordinates), out: 2^t EF entries. */
void or_eq_table(const uint64_t *point, uint32_t t, uint64_t *out);
/* Batched constraint weights of a WHIR round (p3-whir prover/mod.rs:228-314):
 * out[x] = sum_{j<m} gamma^j eq(p_j, x) + sum_{k<q} gamma^(m+k) z_k^x, x < 2^n
 * (EF). eq_points: m points of n EF coordinates (variable 0 first); sel: q EF. */
void or_constraint_weights(const uint64_t *eq_points, uint32_t m, const uint64_t *sel, uint32_t q,
                           const uint64_t gamma[2], uint32_t n, uint64_t *out);

/* ---- inputs (field.rs:17-36, fixed_point.rs:11-38) ---- */
uint64_t or_xorshift_next(uint64_t *state);
void or_xorshift_init(uint64_t *state, uint64_t seed);
/* n uniform field elements, next_u64() mod p */
void or_gen_uniform(uint64_t seed, uint64_t n, uint64_t *out);
/* n int16 values (next_u64() % 65536) as i16, embedded p + v for v < 0 */
void or_gen_i16(uint64_t seed, uint64_t n, uint64_t *out);
/* n int8 values (next_u64() % 255) - 127, embedded */
void or_gen_i8(uint64_t seed, uint64_t n, uint64_t *out);
/* n Irwin-Hall gaussian int16 values: round_half_up(g * std * 2^frac_bits), std = num/den */
void or_gen_gauss_i16(uint64_t seed, uint64_t n, uint64_t std_num, uint64_t std_den,
                      uint32_t frac_bits, uint64_t *out);

/* ---- thread control for the CPU baseline ---- */
void or_set_threads(int n);
int or_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
