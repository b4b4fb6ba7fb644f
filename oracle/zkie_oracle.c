/*
 * zkie_oracle.c — CPU restatement of the zkIE shard-commitment path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP library and the CPU
 * baseline of bench.py. Never linked into or called from the product path.
 *
 * Plain C on canonical u64 values. Parallel loops use OpenMP so that the
 * CPU baseline can run on every host core; every loop body is independent
 * per index, so the results do not depend on the thread count.
 */
#include "zkie_oracle.h"

#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef unsigned __int128 u128;

/* ------------------------------------------------------------------------ */
/* Field F: p = 2^64 - 2^32 + 1. Restated from the field definition; p3's
 * Goldilocks (external p3-goldilocks 0.7.0, Cargo.lock:730) exposes the same
 * canonical values (field.rs:10-14). */

uint64_t or_add(uint64_t a, uint64_t b)
{
    /* canonical inputs: a + b < 2p */
    const u128 s = (u128)a + b;
    return (uint64_t)(s >= OR_P ? s - OR_P : s);
}

uint64_t or_sub(uint64_t a, uint64_t b)
{
    return a >= b ? a - b : (uint64_t)(((u128)a + OR_P) - b);
}

uint64_t or_mul(uint64_t a, uint64_t b)
{
    return (uint64_t)(((u128)a * b) % OR_P);
}

uint64_t or_pow(uint64_t a, uint64_t e)
{
    uint64_t r = 1, x = a % OR_P;
    while (e) {
        if (e & 1) r = or_mul(r, x);
        x = or_mul(x, x);
        e >>= 1;
    }
    return r;
}

uint64_t or_inv(uint64_t a) { return or_pow(a, OR_P - 2); }

/* EF = BinomialExtensionField<F, 2> (whir.rs:38), x^2 = W with W = 7. */
#define OR_W 7ULL
void or_ef_mul(const uint64_t a[2], const uint64_t b[2], uint64_t out[2])
{
    uint64_t c0 = or_add(or_mul(a[0], b[0]), or_mul(OR_W, or_mul(a[1], b[1])));
    uint64_t c1 = or_add(or_mul(a[0], b[1]), or_mul(a[1], b[0]));
    out[0] = c0;
    out[1] = c1;
}

static void ef_add(const uint64_t a[2], const uint64_t b[2], uint64_t o[2])
{
    o[0] = or_add(a[0], b[0]);
    o[1] = or_add(a[1], b[1]);
}

static void ef_sub(const uint64_t a[2], const uint64_t b[2], uint64_t o[2])
{
    o[0] = or_sub(a[0], b[0]);
    o[1] = or_sub(a[1], b[1]);
}

/* TWO_ADIC_GENERATORS[k] (dft_cuda.rs:49): the closed form 7^((p-1)/2^k),
 * 7 being the multiplicative generator of F_p^*. */
uint64_t or_two_adic_generator(uint32_t k)
{
    if (k > 32) return 0;
    return or_pow(7, (OR_P - 1) >> k);
}

/* ------------------------------------------------------------------------ */
/* DFT (TwoAdicSubgroupDft::dft_batch, contract at goldilocks_ntt.cu:3-23).
 * Iterative radix-2 decimation in time: bit-reverse the rows, then stage s
 * (1..lg) combines halves at distance 2^(s-1) with twiddles g_s^j
 * (dft_cuda.rs:44-59 builds the same per-stage tables). Row vectors of w
 * columns move together, so all columns share twiddles. */

static uint32_t bitrev(uint32_t x, uint32_t bits)
{
    uint32_t r = 0;
    for (uint32_t b = 0; b < bits; b++) {
        r = (r << 1) | (x & 1);
        x >>= 1;
    }
    return r;
}

static void dft_core(uint64_t *mat, uint32_t lg, uint64_t w, int inverse)
{
    if (lg == 0 || w == 0) return;
    const uint64_t h = 1ULL << lg;
    uint64_t *tmp = (uint64_t *)malloc(w * sizeof(uint64_t));
    for (uint64_t i = 0; i < h; i++) {
        uint64_t j = bitrev((uint32_t)i, lg);
        if (j > i) {
            memcpy(tmp, mat + i * w, w * 8);
            memcpy(mat + i * w, mat + j * w, w * 8);
            memcpy(mat + j * w, tmp, w * 8);
        }
    }
    free(tmp);
    uint64_t *tw = (uint64_t *)malloc((h / 2) * sizeof(uint64_t));
    for (uint32_t s = 1; s <= lg; s++) {
        const uint64_t half = 1ULL << (s - 1);
        uint64_t root = or_two_adic_generator(s);
        if (inverse) root = or_inv(root);
        tw[0] = 1;
        for (uint64_t j = 1; j < half; j++) tw[j] = or_mul(tw[j - 1], root);
        const int64_t pairs = (int64_t)(h / 2);
#pragma omp parallel for schedule(static)
        for (int64_t k = 0; k < pairs; k++) {
            uint64_t g = (uint64_t)k / half, j = (uint64_t)k % half;
            uint64_t i0 = g * 2 * half + j, i1 = i0 + half;
            uint64_t *a = mat + i0 * w, *b = mat + i1 * w;
            for (uint64_t c = 0; c < w; c++) {
                uint64_t u = a[c], v = or_mul(b[c], tw[j]);
                a[c] = or_add(u, v);
                b[c] = or_sub(u, v);
            }
        }
    }
    free(tw);
}

void or_dft_batch(uint64_t *mat, uint32_t lg_h, uint64_t w) { dft_core(mat, lg_h, w, 0); }

void or_idft_batch(uint64_t *mat, uint32_t lg_h, uint64_t w)
{
    dft_core(mat, lg_h, w, 1);
    const uint64_t inv_n = or_inv(1ULL << lg_h);
    const int64_t total = (int64_t)((1ULL << lg_h) * w);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < total; i++) mat[i] = or_mul(mat[i], inv_n);
}

/* Horner evaluation of column c of an h x w coefficient matrix at x. */
uint64_t or_poly_eval(const uint64_t *mat, uint64_t h, uint64_t w, uint64_t c, uint64_t x)
{
    /* Horner over chunks of 2^20 coefficients in parallel: chunk b holds
     * coefficients [b B, (b + 1) B) and contributes x^(b B) times its own
     * Horner value. */
    const uint64_t B = (uint64_t)1 << 20;
    if (h <= B) {
        uint64_t acc = 0;
        for (uint64_t j = h; j-- > 0;) acc = or_add(or_mul(acc, x), mat[j * w + c]);
        return acc;
    }
    const uint64_t nb = (h + B - 1) / B;
    const uint64_t xB = or_pow(x, B);
    uint64_t total = 0;
#pragma omp parallel
    {
        uint64_t part = 0;
#pragma omp for schedule(static)
        for (int64_t b = 0; b < (int64_t)nb; b++) {
            const uint64_t lo = (uint64_t)b * B, hi = lo + B < h ? lo + B : h;
            uint64_t acc = 0;
            for (uint64_t j = hi; j-- > lo;) acc = or_add(or_mul(acc, x), mat[j * w + c]);
            part = or_add(part, or_mul(acc, or_pow(xB, (uint64_t)b)));
        }
#pragma omp critical
        total = or_add(total, part);
    }
    return total;
}

/* Polynomial checksum sum_i v[i] z^i (Horner), a fingerprint of a vector. */
uint64_t or_checksum(const uint64_t *v, uint64_t n, uint64_t z)
{
    uint64_t acc = 0;
    for (uint64_t i = n; i-- > 0;) acc = or_add(or_mul(acc, z), v[i] % OR_P);
    return acc;
}

void or_dft_naive(const uint64_t *in, uint64_t *out, uint32_t lg_h, uint64_t w)
{
    const uint64_t h = 1ULL << lg_h;
    const uint64_t g = or_two_adic_generator(lg_h);
    for (uint64_t i = 0; i < h; i++) {
        const uint64_t gi = or_pow(g, i);
        for (uint64_t c = 0; c < w; c++) {
            uint64_t acc = 0, x = 1;
            for (uint64_t j = 0; j < h; j++) {
                acc = or_add(acc, or_mul(in[j * w + c], x));
                x = or_mul(x, gi);
            }
            out[i * w + c] = acc;
        }
    }
}

/* p3-whir writer.rs:73-81 (Suffix order): rows [0, h) hold the coefficient
 * rows, the remaining rows are zero, then dft_algebra_batch / dft_batch. A
 * shift s != 1 evaluates on the coset s*H instead (coefficient j scaled by s^j). */
void or_lde_batch(const uint64_t *in, uint64_t h, uint64_t w, uint32_t log_blowup,
                  uint64_t shift, uint64_t *out)
{
    const uint64_t n = h << log_blowup;
    memset(out, 0, n * w * sizeof(uint64_t));
    if (shift == 1) {
        memcpy(out, in, h * w * sizeof(uint64_t));
    } else {
        uint64_t sj = 1;
        for (uint64_t j = 0; j < h; j++) {
            for (uint64_t c = 0; c < w; c++) out[j * w + c] = or_mul(in[j * w + c], sj);
            sj = or_mul(sj, shift);
        }
    }
    uint32_t lg = 0;
    while ((1ULL << lg) < n) lg++;
    or_dft_batch(out, lg, w);
}

/* ------------------------------------------------------------------------ */
/* rand 0.10.3 SmallRng = Xoshiro256++ on 64-bit targets, seed_from_u64 via
 * SplitMix64 (the seeding used by merkle_cuda.rs:64 and whir.rs:316). */

uint64_t or_splitmix64_next(uint64_t *state)
{
    *state += 0x9e3779b97f4a7c15ULL;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

void or_xoshiro_seed_u64(or_xoshiro *r, uint64_t seed)
{
    uint64_t st = seed;
    for (int i = 0; i < 4; i++) r->s[i] = or_splitmix64_next(&st);
}

void or_xoshiro_from_state(or_xoshiro *r, const uint64_t s[4])
{
    for (int i = 0; i < 4; i++) r->s[i] = s[i];
}

static uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

uint64_t or_xoshiro_next(or_xoshiro *r)
{
    uint64_t *s = r->s;
    const uint64_t res = rotl64(s[0] + s[3], 23) + s[0];
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return res;
}

/* p3-goldilocks StandardUniform: rejection of u64 >= p. */
static uint64_t sample_field(or_xoshiro *r)
{
    for (;;) {
        uint64_t x = or_xoshiro_next(r);
        if (x < OR_P) return x;
    }
}

/* ------------------------------------------------------------------------ */
/* Poseidon2-Goldilocks-16, restated from poseidon2_merkle.cu:37-155:
 *  - x^7 S-box through x^2, x^3, x^4 (:43-53);
 *  - apply_mat4 [2 3 1 1; 1 2 3 1; 1 1 2 3; 3 1 1 2] (:63-76);
 *  - mds_light16: mat4 per 4-chunk, then add per-residue-class sums (:80-97);
 *  - internal layer: st0 += rc, st0 = st0^7, st_i = sum + V_i st_i with
 *    V = [-2, 1, 2, 1/2, 3, 4, -1/2, -3, -4, 1/2^3, 1/2^4, 1/2^5,
 *         -1/2^3, -1/2^4, -1/2^5, diag15] (:111-142);
 *  - permutation: mds_light16, 4 external, 22 internal, 4 external (:146-155).
 * Constants follow merkle_cuda.rs:54-85. */

static uint64_t g_rc_init[64], g_rc_final[64], g_rc_int[22], g_diag15;
static uint64_t g_V[16];
static int g_p2_ready = 0;

void or_p2_derive_constants(uint64_t rc_init[64], uint64_t rc_final[64],
                            uint64_t rc_internal[22], uint64_t *diag15)
{
    or_xoshiro r;
    or_xoshiro_seed_u64(&r, 1);
    /* ExternalLayerConstants::new_from_rng(8): 4 initial then 4 terminal [F;16]. */
    for (int i = 0; i < 64; i++) rc_init[i] = sample_field(&r);
    for (int i = 0; i < 64; i++) rc_final[i] = sample_field(&r);
    /* then 22 internal constants from StandardUniform. */
    for (int i = 0; i < 22; i++) rc_internal[i] = sample_field(&r);
    /* MATRIX_DIAG_16_GOLDILOCKS[15], documented as 1/2^32 (poseidon2_merkle.cu:34). */
    *diag15 = or_inv(or_pow(2, 32));
}

void or_p2_set_constants(const uint64_t rc_init[64], const uint64_t rc_final[64],
                         const uint64_t rc_internal[22], uint64_t diag15)
{
    memcpy(g_rc_init, rc_init, sizeof g_rc_init);
    memcpy(g_rc_final, rc_final, sizeof g_rc_final);
    memcpy(g_rc_int, rc_internal, sizeof g_rc_int);
    g_diag15 = diag15;
    const uint64_t i2 = or_inv(2), i8 = or_inv(8), i16 = or_inv(16), i32 = or_inv(32);
    const uint64_t V[16] = {OR_P - 2, 1, 2, i2, 3, 4, OR_P - i2, OR_P - 3, OR_P - 4,
                            i8, i16, i32, OR_P - i8, OR_P - i16, OR_P - i32, diag15};
    memcpy(g_V, V, sizeof V);
    g_p2_ready = 1;
}

static void p2_ensure(void)
{
    if (!g_p2_ready) {
        uint64_t a[64], b[64], c[22], d;
        or_p2_derive_constants(a, b, c, &d);
        or_p2_set_constants(a, b, c, d);
    }
}

static uint64_t sbox7(uint64_t x)
{
    uint64_t x2 = or_mul(x, x), x3 = or_mul(x2, x), x4 = or_mul(x2, x2);
    return or_mul(x3, x4);
}

static void apply_mat4(uint64_t *x)
{
    const uint64_t m[4][4] = {{2, 3, 1, 1}, {1, 2, 3, 1}, {1, 1, 2, 3}, {3, 1, 1, 2}};
    uint64_t y[4];
    for (int r = 0; r < 4; r++) {
        uint64_t acc = 0;
        for (int c = 0; c < 4; c++) acc = or_add(acc, or_mul(m[r][c], x[c]));
        y[r] = acc;
    }
    memcpy(x, y, sizeof y);
}

void or_p2_mds_light(uint64_t st[16])
{
    for (int j = 0; j < 16; j += 4) apply_mat4(st + j);
    uint64_t sums[4] = {0, 0, 0, 0};
    for (int j = 0; j < 16; j += 4)
        for (int k = 0; k < 4; k++) sums[k] = or_add(sums[k], st[j + k]);
    for (int i = 0; i < 16; i++) st[i] = or_add(st[i], sums[i % 4]);
}

void or_p2_internal_linear(uint64_t st[16])
{
    p2_ensure();
    uint64_t sum = 0;
    for (int i = 0; i < 16; i++) sum = or_add(sum, st[i]);
    for (int i = 0; i < 16; i++) st[i] = or_add(sum, or_mul(g_V[i], st[i]));
}

static void ext_round(uint64_t st[16], const uint64_t *rc)
{
    for (int i = 0; i < 16; i++) st[i] = sbox7(or_add(st[i], rc[i]));
    or_p2_mds_light(st);
}

void or_p2_permute(uint64_t st[16])
{
    p2_ensure();
    or_p2_mds_light(st);
    for (int r = 0; r < 4; r++) ext_round(st, g_rc_init + 16 * r);
    for (int r = 0; r < 22; r++) {
        st[0] = sbox7(or_add(st[0], g_rc_int[r]));
        or_p2_internal_linear(st);
    }
    for (int r = 0; r < 4; r++) ext_round(st, g_rc_final + 16 * r);
}

/* PaddingFreeSponge<Perm, 16, 8, 8> (whir.rs:40): zero state; absorb chunks of
 * up to 8 by overwriting state[0..len]; permute after every full chunk and
 * after a trailing partial chunk; squeeze state[0..8]. */
void or_leaf_hash(const uint64_t *row, uint64_t w, uint64_t out[8])
{
    uint64_t st[16] = {0};
    uint64_t pos = 0;
    while (pos < w) {
        uint64_t len = w - pos < 8 ? w - pos : 8;
        for (uint64_t i = 0; i < len; i++) st[i] = row[pos + i];
        or_p2_permute(st);
        pos += len;
    }
    memcpy(out, st, 8 * sizeof(uint64_t));
}

/* TruncatedPermutation<Perm, 2, 8, 16> (whir.rs:41): permute [left || right],
 * keep state[0..8]. */
void or_compress(const uint64_t left[8], const uint64_t right[8], uint64_t out[8])
{
    uint64_t st[16];
    memcpy(st, left, 64);
    memcpy(st + 8, right, 64);
    or_p2_permute(st);
    memcpy(out, st, 64);
}

/* ------------------------------------------------------------------------ */
/* Merkle tree (vendored p3-merkle-tree: merkle_tree.rs:95-178 `new`,
 * :372-442 first_digest_layer, :594-642 compress, :577-585 padded_len).
 * Single matrix, arity 2, cap height 0 (whir.rs:321,329-332). */

uint64_t or_padded_len(uint64_t raw, uint64_t n)
{
    if (raw <= 1) return raw;
    if (raw >= n) return (raw + n - 1) / n * n;
    return n;
}

uint32_t or_merkle_num_layers(uint64_t h)
{
    uint32_t nl = 1;
    uint64_t len = or_padded_len(h, 2);
    while (len > 1) {
        len = or_padded_len(len / 2, 2);
        nl++;
    }
    return nl;
}

void or_merkle_layer_lens(uint64_t h, uint64_t *lens)
{
    uint32_t i = 0;
    uint64_t len = or_padded_len(h, 2);
    lens[i++] = len;
    while (len > 1) {
        len = or_padded_len(len / 2, 2);
        lens[i++] = len;
    }
}

static void compress_pair(const uint64_t *l, const uint64_t *r, uint64_t *o, int compressor)
{
    if (compressor == 1) {
        for (int e = 0; e < 8; e++) o[e] = l[e] ^ r[e];
    } else {
        or_compress(l, r, o);
    }
}

/* compress() (merkle_tree.rs:594-642): next_len = prev_len / 2 digests from
 * consecutive pairs, padded with zero digests to padded_len(next_len, 2). */
uint64_t or_merkle_compress_layer(const uint64_t *prev, uint64_t prev_len, uint64_t *next,
                                  int compressor)
{
    const uint64_t next_len = prev_len / 2;
    const uint64_t padded = or_padded_len(next_len, 2);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)next_len; i++)
        compress_pair(prev + 16 * i, prev + 16 * i + 8, next + 8 * i, compressor);
    memset(next + 8 * next_len, 0, (padded - next_len) * 64);
    return padded;
}

void or_merkle_build_layers(const uint64_t *layer0_digests, uint64_t h, uint64_t *layers,
                            int compressor)
{
    uint64_t len = or_padded_len(h, 2);
    memcpy(layers, layer0_digests, h * 64);
    memset(layers + 8 * h, 0, (len - h) * 64);
    uint64_t *cur = layers;
    while (len > 1) {
        uint64_t *next = cur + 8 * len;
        len = or_merkle_compress_layer(cur, len, next, compressor);
        cur = next;
    }
}

void or_merkle_leaf_digests(const uint64_t *mat, uint64_t h, uint64_t w, uint64_t *digests)
{
    p2_ensure();
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)h; i++) or_leaf_hash(mat + (uint64_t)i * w, w, digests + 8 * i);
}

void or_merkle_commit(const uint64_t *mat, uint64_t h, uint64_t w, uint64_t *layers,
                      uint64_t root[8])
{
    p2_ensure();
    /* first_digest_layer writes the leaf digests straight into layer 0. */
    or_merkle_leaf_digests(mat, h, w, layers);
    uint64_t len = or_padded_len(h, 2);
    memset(layers + 8 * h, 0, (len - h) * 64);
    uint64_t *cur = layers;
    while (len > 1) {
        uint64_t *next = cur + 8 * len;
        len = or_merkle_compress_layer(cur, len, next, 0);
        cur = next;
    }
    memcpy(root, cur, 64);
}

/* open_batch (mmcs/batch.rs:75-121): one sibling per proof level, taken from
 * digest_layers[level][idx ^ 1]; proof_levels = num_layers - 1 (cap 0). */
void or_merkle_open(const uint64_t *layers, uint64_t h, uint64_t index, uint64_t *siblings)
{
    const uint32_t nl = or_merkle_num_layers(h);
    uint64_t lens[80];
    or_merkle_layer_lens(h, lens);
    const uint64_t *layer = layers;
    uint64_t idx = index;
    for (uint32_t l = 0; l + 1 < nl; l++) {
        memcpy(siblings + 8 * l, layer + 8 * (idx ^ 1), 64);
        layer += 8 * lens[l];
        idx >>= 1;
    }
}

static int cmp_u64(const void *a, const void *b)
{
    uint64_t x = *(const uint64_t *)a, y = *(const uint64_t *)b;
    return x < y ? -1 : (x > y ? 1 : 0);
}

/* prune_paths / walk_frontier (pruning.rs:130-232) for arity 2: sort and
 * dedup the indices; per level, per group (ascending), emit every child
 * position not covered by a frontier node. The emitted digest is the lead
 * path's sibling, i.e. digest_layers[level][group*2 + k]. */
uint64_t or_merkle_open_pruned(const uint64_t *layers, uint64_t h, const uint64_t *indices,
                               uint64_t n, uint64_t *out, uint64_t cap)
{
    const uint32_t nl = or_merkle_num_layers(h);
    uint64_t lens[80];
    or_merkle_layer_lens(h, lens);
    uint64_t *nodes = (uint64_t *)malloc((n ? n : 1) * sizeof(uint64_t));
    memcpy(nodes, indices, n * sizeof(uint64_t));
    qsort(nodes, n, sizeof(uint64_t), cmp_u64);
    uint64_t m = 0;
    for (uint64_t i = 0; i < n; i++)
        if (m == 0 || nodes[m - 1] != nodes[i]) nodes[m++] = nodes[i];
    uint64_t count = 0;
    const uint64_t *layer = layers;
    for (uint32_t l = 0; l + 1 < nl && m > 0; l++) {
        uint64_t np = 0, i = 0;
        while (i < m) {
            const uint64_t group = nodes[i] / 2, start = group * 2;
            uint64_t member = i;
            for (uint64_t k = 0; k < 2; k++) {
                if (member < m && nodes[member] == start + k) {
                    member++;
                } else {
                    if (count < cap) memcpy(out + 8 * count, layer + 8 * (start + k), 64);
                    count++;
                }
            }
            nodes[np++] = group;
            i = member;
        }
        m = np;
        layer += 8 * lens[l];
    }
    free(nodes);
    return count;
}

/* verify_batch (mmcs/batch.rs:158-296) for one matrix, arity 2, cap 0. */
int or_merkle_verify(const uint64_t root[8], uint64_t h, uint64_t index, const uint64_t *row,
                     uint64_t w, const uint64_t *siblings)
{
    if (index >= h) return 0;
    const uint32_t nl = or_merkle_num_layers(h);
    uint64_t d[8], t[8];
    or_leaf_hash(row, w, d);
    uint64_t idx = index;
    for (uint32_t l = 0; l + 1 < nl; l++) {
        if (idx & 1)
            or_compress(siblings + 8 * l, d, t);
        else
            or_compress(d, siblings + 8 * l, t);
        memcpy(d, t, 64);
        idx >>= 1;
    }
    return memcmp(d, root, 64) == 0;
}

/* ------------------------------------------------------------------------ */
/* Fold. mle::eval (mle.rs:8-22): variable 0 is the least-significant index
 * bit; each step maps buf[i] = a + p (b - a) over pairs (a, b) = (buf[2i],
 * buf[2i+1]). With EF points this is the row fold of p3-whir
 * prover/mod.rs:257-290 (Suffix order reverses the folding randomness for the
 * MSB-first p3 evaluator, which lands on the same LSB-first binding). */

uint64_t or_mle_eval_base(const uint64_t *values, uint32_t t, const uint64_t *point)
{
    uint64_t n = 1ULL << t;
    uint64_t *buf = (uint64_t *)malloc(n * sizeof(uint64_t));
    memcpy(buf, values, n * 8);
    for (uint32_t v = 0; v < t; v++) {
        uint64_t half = n / 2;
        for (uint64_t i = 0; i < half; i++) {
            uint64_t a = buf[2 * i], b = buf[2 * i + 1];
            buf[i] = or_add(a, or_mul(point[v], or_sub(b, a)));
        }
        n = half;
    }
    uint64_t r = buf[0];
    free(buf);
    return r;
}

void or_mle_eval(const uint64_t *values, uint32_t t, int is_ext, const uint64_t *point, uint64_t out[2])
{
    /* mle.rs:12-20: each round halves the table, buf[i] = a + r_v (b - a)
     * for the pair (2i, 2i + 1), in EF. */
    uint64_t n = 1ULL << t;
    uint64_t *buf = (uint64_t *)malloc(2 * n * sizeof(uint64_t));
    for (uint64_t i = 0; i < n; i++) {
        buf[2 * i] = (is_ext ? values[2 * i] : values[i]) % OR_P;
        buf[2 * i + 1] = is_ext ? values[2 * i + 1] % OR_P : 0;
    }
    for (uint32_t v = 0; v < t; v++) {
        uint64_t half = n / 2;
        for (uint64_t i = 0; i < half; i++) {
            uint64_t d[2], m[2];
            ef_sub(buf + 4 * i + 2, buf + 4 * i, d);
            or_ef_mul(point + 2 * v, d, m);
            ef_add(buf + 4 * i, m, buf + 2 * i);
        }
        n = half;
    }
    out[0] = buf[0];
    out[1] = buf[1];
    free(buf);
}

/* mle.rs:44-56 (eq_evals), coordinate b doubling the table: entries with bit b
 * set take p_b, the others 1 - p_b. */
void or_eq_table(const uint64_t *point, uint32_t t, uint64_t *out)
{
    out[0] = 1;
    out[1] = 0;
    for (uint32_t b = 0; b < t; b++) {
        const uint64_t m = 1ULL << b;
        const uint64_t z[2] = {point[2 * b] % OR_P, point[2 * b + 1] % OR_P};
        const uint64_t om[2] = {or_sub(1, z[0]), or_sub(0, z[1])};
        for (uint64_t j = 0; j < m; j++) {
            uint64_t v[2] = {out[2 * j], out[2 * j + 1]};
            or_ef_mul(v, z, out + 2 * (j + m));
            or_ef_mul(v, om, out + 2 * j);
        }
    }
}

/* The batched constraint of a WHIR round (p3-whir src/pcs/prover/mod.rs:228-314):
 * Constraint::new(gamma, n, [Statements::Eq(ood), Statements::Select(stir)])
 * as one weight table over the 2^n-entry round table,
 *   out[x] = sum_{j<m} gamma^j eq(p_j, x) + sum_{k<q} gamma^(m+k) z_k^x,
 * eq(p, x) as or_eq_table (bit b of x is variable b) and z^x the powers of a
 * univariate point (the select weight: sum_x f(x) z^x is the value at z of the
 * polynomial whose coefficients are the table). The p3-sumcheck crate that
 * defines the combination is external to the reference: the order of the
 * powers (the Eq group first, from gamma^0) is not pinned by its files. */
void or_constraint_weights(const uint64_t *eq_points, uint32_t m, const uint64_t *sel, uint32_t q,
                           const uint64_t gamma[2], uint32_t n, uint64_t *out)
{
    const uint64_t N = 1ULL << n;
    uint64_t *tab = (uint64_t *)malloc(2 * N * sizeof(uint64_t));
    uint64_t g[2] = {1, 0};
    const uint64_t gm[2] = {gamma[0] % OR_P, gamma[1] % OR_P};
    memset(out, 0, 2 * N * sizeof(uint64_t));
    for (uint32_t c = 0; c < m + q; c++) {
        if (c < m) {
            or_eq_table(eq_points + 2 * (uint64_t)c * n, n, tab);
        } else {
            const uint64_t z[2] = {sel[2 * (c - m)] % OR_P, sel[2 * (c - m) + 1] % OR_P};
            tab[0] = 1;
            tab[1] = 0;
            for (uint64_t x = 1; x < N; x++) or_ef_mul(tab + 2 * (x - 1), z, tab + 2 * x);
        }
#pragma omp parallel for schedule(static)
        for (int64_t x = 0; x < (int64_t)N; x++) {
            uint64_t t[2];
            or_ef_mul(g, tab + 2 * x, t);
            ef_add(out + 2 * x, t, out + 2 * x);
        }
        uint64_t ng[2];
        or_ef_mul(g, gm, ng);
        g[0] = ng[0];
        g[1] = ng[1];
    }
    free(tab);
}

/* common/sumcheck.rs:33-89 (prove and fold) with EF tables and challenges. */
void or_sumcheck_prove(const uint64_t *f, int f_is_ext, const uint64_t *h, uint32_t t, uint32_t rounds,
                       const uint64_t *r, uint64_t *polys, uint64_t *f_out, uint64_t *h_out)
{
    uint64_t n = 1ULL << t;
    uint64_t *fb = (uint64_t *)malloc(2 * n * sizeof(uint64_t));
    uint64_t *hb = (uint64_t *)malloc(2 * n * sizeof(uint64_t));
    for (uint64_t i = 0; i < n; i++) {
        fb[2 * i] = (f_is_ext ? f[2 * i] : f[i]) % OR_P;
        fb[2 * i + 1] = f_is_ext ? f[2 * i + 1] % OR_P : 0;
        hb[2 * i] = h[2 * i] % OR_P;
        hb[2 * i + 1] = h[2 * i + 1] % OR_P;
    }
    const uint64_t inv2 = OR_P / 2 + 1;
    for (uint32_t i = 0; i < rounds; i++) {
        const uint64_t half = n / 2;
        uint64_t y0[2] = {0, 0}, y1[2] = {0, 0}, y2[2] = {0, 0};
        for (uint64_t s2 = 0; s2 < half; s2++) {
            const uint64_t *f0 = fb + 4 * s2, *f1 = fb + 4 * s2 + 2;
            const uint64_t *h0 = hb + 4 * s2, *h1 = hb + 4 * s2 + 2;
            uint64_t f2[2], h2[2], m[2];
            f2[0] = or_sub(or_add(f1[0], f1[0]), f0[0]);
            f2[1] = or_sub(or_add(f1[1], f1[1]), f0[1]);
            h2[0] = or_sub(or_add(h1[0], h1[0]), h0[0]);
            h2[1] = or_sub(or_add(h1[1], h1[1]), h0[1]);
            or_ef_mul(f0, h0, m);
            ef_add(y0, m, y0);
            or_ef_mul(f1, h1, m);
            ef_add(y1, m, y1);
            or_ef_mul(f2, h2, m);
            ef_add(y2, m, y2);
        }
        uint64_t *c = polys + 6 * i;
        for (int e = 0; e < 2; e++) {
            c[e] = y0[e];
            c[2 + e] = or_mul(or_sub(or_sub(or_mul(4, y1[e]), y2[e]), or_mul(3, y0[e])), inv2);
            c[4 + e] = or_mul(or_add(or_sub(y2[e], or_mul(2, y1[e])), y0[e]), inv2);
        }
        for (uint64_t s2 = 0; s2 < half; s2++) {
            uint64_t d[2], m[2];
            ef_sub(fb + 4 * s2 + 2, fb + 4 * s2, d);
            or_ef_mul(r + 2 * i, d, m);
            ef_add(fb + 4 * s2, m, fb + 2 * s2);
            ef_sub(hb + 4 * s2 + 2, hb + 4 * s2, d);
            or_ef_mul(r + 2 * i, d, m);
            ef_add(hb + 4 * s2, m, hb + 2 * s2);
        }
        n = half;
    }
    memcpy(f_out, fb, 2 * n * sizeof(uint64_t));
    memcpy(h_out, hb, 2 * n * sizeof(uint64_t));
    free(fb);
    free(hb);
}

void or_fold_rows(const uint64_t *mat, uint64_t h, uint32_t k, int is_ext, const uint64_t *r,
                  uint64_t *out)
{
    const uint64_t width = 1ULL << k;
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < (int64_t)h; t++) {
        uint64_t buf[2 * 64 * 2];
        uint64_t *b = buf;
        uint64_t *heap = NULL;
        if (width > 128) {
            heap = (uint64_t *)malloc(2 * width * sizeof(uint64_t));
            b = heap;
        }
        for (uint64_t j = 0; j < width; j++) {
            if (is_ext) {
                b[2 * j] = mat[(uint64_t)t * 2 * width + 2 * j];
                b[2 * j + 1] = mat[(uint64_t)t * 2 * width + 2 * j + 1];
            } else {
                b[2 * j] = mat[(uint64_t)t * width + j];
                b[2 * j + 1] = 0;
            }
        }
        uint64_t n = width;
        for (uint32_t v = 0; v < k; v++) {
            uint64_t half = n / 2;
            for (uint64_t i = 0; i < half; i++) {
                uint64_t d[2], m[2];
                ef_sub(b + 4 * i + 2, b + 4 * i, d);
                or_ef_mul(r + 2 * v, d, m);
                ef_add(b + 4 * i, m, b + 2 * i);
            }
            n = half;
        }
        out[2 * t] = b[0];
        out[2 * t + 1] = b[1];
        free(heap);
    }
}

/* ------------------------------------------------------------------------ */
/* Inputs. XorShift64 (field.rs:17-36): state = seed + 0x9e3779b97f4a7c15;
 * x ^= x << 13; x ^= x >> 7; x ^= x << 17. Signed embedding v < 0 -> p - |v|
 * (fixed_point.rs:11-38). */

void or_xorshift_init(uint64_t *state, uint64_t seed) { *state = seed + 0x9e3779b97f4a7c15ULL; }

uint64_t or_xorshift_next(uint64_t *state)
{
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return x;
}

static uint64_t embed_i64(int64_t v) { return v >= 0 ? (uint64_t)v : OR_P - (uint64_t)(-v); }

void or_gen_uniform(uint64_t seed, uint64_t n, uint64_t *out)
{
    uint64_t s;
    or_xorshift_init(&s, seed);
    for (uint64_t i = 0; i < n; i++) out[i] = or_xorshift_next(&s) % OR_P;
}

void or_gen_i16(uint64_t seed, uint64_t n, uint64_t *out)
{
    uint64_t s;
    or_xorshift_init(&s, seed);
    for (uint64_t i = 0; i < n; i++) {
        int16_t v = (int16_t)(uint16_t)(or_xorshift_next(&s) % 65536);
        out[i] = embed_i64(v);
    }
}

void or_gen_i8(uint64_t seed, uint64_t n, uint64_t *out)
{
    uint64_t s;
    or_xorshift_init(&s, seed);
    for (uint64_t i = 0; i < n; i++) {
        int64_t v = (int64_t)(or_xorshift_next(&s) % 255) - 127;
        out[i] = embed_i64(v);
    }
}

/* Integer Irwin-Hall N(0,1) approximation: g = S * 2^-53 - 6 with S the sum of
 * 12 53-bit uniforms; value = floor(g * std * 2^frac + 1/2), clamped to int16.
 * Exact integer arithmetic, so every implementation agrees bit for bit. */
void or_gen_gauss_i16(uint64_t seed, uint64_t n, uint64_t std_num, uint64_t std_den,
                      uint32_t frac_bits, uint64_t *out)
{
    uint64_t s;
    or_xorshift_init(&s, seed);
    const __int128 two53 = (__int128)1 << 53;
    for (uint64_t i = 0; i < n; i++) {
        __int128 S = 0;
        for (int k = 0; k < 12; k++) S += (__int128)(or_xorshift_next(&s) >> 11);
        __int128 num = 2 * (S - 6 * two53) * (__int128)std_num * ((__int128)1 << frac_bits) +
                       (__int128)std_den * two53;
        __int128 den = 2 * (__int128)std_den * two53;
        __int128 q = num / den;
        if ((num % den != 0) && ((num < 0) != (den < 0))) q -= 1; /* floor */
        if (q > 32767) q = 32767;
        if (q < -32768) q = -32768;
        out[i] = embed_i64((int64_t)q);
    }
}

void or_set_threads(int n)
{
#ifdef _OPENMP
    omp_set_num_threads(n > 0 ? n : 1);
#else
    (void)n;
#endif
}

int or_get_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
