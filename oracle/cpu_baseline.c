/*
 * cpu_baseline.c — the CPU baseline of bench.py: the reference's CPU commit
 * path restated in its own class of implementation, for timing beside the
 * GPU. TEST INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg and its parity
 * test); the product path never links, loads or calls it. The checker is
 * zkie_oracle.c; this file is the fast port, and tests/test_cpu_baseline.py
 * proves it bit-identical to the oracle.
 *
 * What it restates (paths relative to the reference repository root):
 *  - the DFT of the encode, p3-dft's Radix2DftSmallBatch behind
 *    DftBackend::Cpu (crates/zkie-core/src/pcs/whir.rs:47,113-119): a radix-2
 *    decimation-in-time transform of the zero-padded row-major matrix, all
 *    columns of a row in 4-wide AVX2 vectors;
 *  - the Merkle commit of CpuMerkleTreeMmcs (merkle_cuda.rs:44-48, p3's
 *    PackedGoldilocksAVX2): Poseidon2-Goldilocks-16 on 4 rows (or 4 parents)
 *    at once, one state word per 4-lane vector, the addition chains of
 *    poseidon2_merkle.cu:63-97 for the external layer and shift forms for the
 *    powers of two of the internal diagonal (poseidon2_merkle.cu:111-142);
 *    leaf sponge and 2-to-1 compression as merkle_tree.rs:372-442,594-642;
 *  - the row fold of the WHIR prover (mle.rs:8-22, prover/mod.rs:257-290).
 * Field arithmetic uses the special form of p = 2^64 - 2^32 + 1
 * (2^64 = 2^32 - 1, 2^96 = -1) on canonical values, with 32 x 32 -> 64
 * vector products (_mm256_mul_epu32). Parallel loops use OpenMP; results do
 * not depend on the thread count.
 */
#include <immintrin.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef unsigned __int128 u128;
typedef __m256i v4;

#define CB_P 0xFFFFFFFF00000001ULL
#define CB_EPS 0xFFFFFFFFULL
#define CB_SIGN 0x8000000000000000ULL

/* ---- scalar field (canonical values) ----------------------------------- */
static inline uint64_t s_add(uint64_t a, uint64_t b)
{
    uint64_t s = a + b;
    const int ov = s < a;
    if (ov || s >= CB_P) s += CB_EPS;
    return s;
}
static inline uint64_t s_sub(uint64_t a, uint64_t b)
{
    uint64_t d = a - b;
    if (a < b) d -= CB_EPS;
    return d;
}
static inline uint64_t s_reduce128(uint64_t lo, uint64_t hi)
{
    const uint64_t hh = hi >> 32, hl = hi & CB_EPS;
    uint64_t t0 = lo - hh;
    if (lo < hh) t0 -= CB_EPS;
    const uint64_t t1 = (hl << 32) - hl;
    uint64_t r = t0 + t1;
    if (r < t1) r += CB_EPS;
    if (r >= CB_P) r -= CB_P;
    return r;
}
static inline uint64_t s_mul(uint64_t a, uint64_t b)
{
    const u128 x = (u128)a * b;
    return s_reduce128((uint64_t)x, (uint64_t)(x >> 64));
}
static uint64_t s_pow(uint64_t a, uint64_t e)
{
    uint64_t r = 1;
    while (e) {
        if (e & 1) r = s_mul(r, a);
        a = s_mul(a, a);
        e >>= 1;
    }
    return r;
}

/* ---- 4-wide AVX2 field (canonical values) ------------------------------- */
static inline v4 v_set1(uint64_t x) { return _mm256_set1_epi64x((long long)x); }
/* unsigned a < b, all-ones lanes */
static inline v4 v_ltu(v4 a, v4 b)
{
    const v4 s = v_set1(CB_SIGN);
    return _mm256_cmpgt_epi64(_mm256_xor_si256(b, s), _mm256_xor_si256(a, s));
}
static inline v4 v_add(v4 a, v4 b)
{
    const v4 s = _mm256_add_epi64(a, b);
    /* wrapped past 2^64, or at least p: subtract p (= add eps mod 2^64) */
    const v4 fix = _mm256_or_si256(v_ltu(s, a), _mm256_andnot_si256(v_ltu(s, v_set1(CB_P)), v_set1(-1LL)));
    return _mm256_add_epi64(s, _mm256_and_si256(fix, v_set1(CB_EPS)));
}
static inline v4 v_sub(v4 a, v4 b)
{
    const v4 d = _mm256_sub_epi64(a, b);
    return _mm256_sub_epi64(d, _mm256_and_si256(v_ltu(a, b), v_set1(CB_EPS)));
}
static inline v4 v_mul(v4 a, v4 b)
{
    const v4 lo32 = v_set1(CB_EPS);
    const v4 ah = _mm256_srli_epi64(a, 32), bh = _mm256_srli_epi64(b, 32);
    const v4 ll = _mm256_mul_epu32(a, b), lh = _mm256_mul_epu32(a, bh);
    const v4 hl = _mm256_mul_epu32(ah, b), hh = _mm256_mul_epu32(ah, bh);
    const v4 t = _mm256_add_epi64(hl, _mm256_srli_epi64(ll, 32));
    const v4 u = _mm256_add_epi64(lh, _mm256_and_si256(t, lo32));
    const v4 lo = _mm256_or_si256(_mm256_slli_epi64(u, 32), _mm256_and_si256(ll, lo32));
    const v4 hi = _mm256_add_epi64(_mm256_add_epi64(hh, _mm256_srli_epi64(t, 32)), _mm256_srli_epi64(u, 32));
    /* lo + hi.lo eps - hi.hi */
    const v4 hhi = _mm256_srli_epi64(hi, 32), hlo = _mm256_and_si256(hi, lo32);
    v4 t0 = _mm256_sub_epi64(lo, hhi);
    t0 = _mm256_sub_epi64(t0, _mm256_and_si256(v_ltu(lo, hhi), lo32));
    const v4 t1 = _mm256_sub_epi64(_mm256_slli_epi64(hlo, 32), hlo);
    v4 r = _mm256_add_epi64(t0, t1);
    r = _mm256_add_epi64(r, _mm256_and_si256(v_ltu(r, t1), lo32));
    /* canonical */
    return _mm256_add_epi64(r, _mm256_andnot_si256(v_ltu(r, v_set1(CB_P)), lo32));
}
static inline v4 v_double(v4 a) { return v_add(a, a); }
/* x / 2 */
static inline v4 v_halve(v4 x)
{
    const v4 odd = _mm256_sub_epi64(_mm256_setzero_si256(), _mm256_and_si256(x, v_set1(1)));
    return _mm256_add_epi64(_mm256_srli_epi64(x, 1), _mm256_and_si256(odd, v_set1(0x7FFFFFFF80000001ULL)));
}
/* x 2^-k, 1 <= k <= 32: x = q 2^k + r, r 2^-k = -(m eps) with m = r 2^(32-k),
 * and -(m eps) = (2^32 - 1 - m) 2^32 + m + 1 (mod p), below p. */
static inline v4 v_mul_inv_pow2(v4 x, int k)
{
    const v4 q = _mm256_srli_epi64(x, k);
    const v4 m = _mm256_slli_epi64(_mm256_and_si256(x, v_set1((1ULL << k) - 1)), 32 - k);
    const v4 y = _mm256_add_epi64(_mm256_slli_epi64(_mm256_sub_epi64(v_set1(CB_EPS), m), 32),
                                  _mm256_add_epi64(m, v_set1(1)));
    return v_add(q, y);
}

/* ---- Poseidon2-Goldilocks-16 ---------------------------------------------- */
static uint64_t g_ext[8][16], g_int[22], g_diag15;
static int g_diag15_inv32;

void cb_p2_set_constants(const uint64_t rc_init[64], const uint64_t rc_final[64], const uint64_t rc_internal[22],
                         uint64_t diag15)
{
    for (int k = 0; k < 4; k++)
        for (int i = 0; i < 16; i++) {
            g_ext[k][i] = rc_init[16 * k + i] % CB_P;
            g_ext[4 + k][i] = rc_final[16 * k + i] % CB_P;
        }
    for (int k = 0; k < 22; k++) g_int[k] = rc_internal[k] % CB_P;
    g_diag15 = diag15 % CB_P;
    g_diag15_inv32 = g_diag15 == 0xFFFFFFFE00000002ULL;
}

static inline v4 v_sbox7(v4 x)
{
    const v4 x2 = v_mul(x, x), x3 = v_mul(x2, x), x4 = v_mul(x2, x2);
    return v_mul(x3, x4);
}

/* mat4 = [2 3 1 1; 1 2 3 1; 1 1 2 3; 3 1 1 2] by the addition chain of
 * poseidon2_merkle.cu:63-76 */
static inline void v_mat4(v4 *x)
{
    const v4 t01 = v_add(x[0], x[1]), t23 = v_add(x[2], x[3]);
    const v4 t0123 = v_add(t01, t23);
    const v4 t01123 = v_add(t0123, x[1]), t01233 = v_add(t0123, x[3]);
    const v4 y3 = v_add(t01233, v_double(x[0]));
    const v4 y1 = v_add(t01123, v_double(x[2]));
    const v4 y0 = v_add(t01123, t01);
    const v4 y2 = v_add(t01233, t23);
    x[0] = y0;
    x[1] = y1;
    x[2] = y2;
    x[3] = y3;
}

/* mds_light16 (poseidon2_merkle.cu:80-97): mat4 per group of four, then each
 * word plus the sum of its column over the four groups */
static inline void v_mds_light16(v4 *st)
{
    for (int g = 0; g < 4; g++) v_mat4(st + 4 * g);
    for (int k = 0; k < 4; k++) {
        const v4 s = v_add(v_add(st[k], st[4 + k]), v_add(st[8 + k], st[12 + k]));
        for (int g = 0; g < 4; g++) st[4 * g + k] = v_add(st[4 * g + k], s);
    }
}

/* internal round: st0 <- (st0 + rc)^7, then st_i <- sum + V_i st_i with
 * V = [-2, 1, 2, 1/2, 3, 4, -1/2, -3, -4, 1/2^3, 1/2^4, 1/2^5, -1/2^3,
 *      -1/2^4, -1/2^5, diag15] (poseidon2_merkle.cu:111-142) */
static inline void v_internal_round(v4 *st, uint64_t rc)
{
    st[0] = v_sbox7(v_add(st[0], v_set1(rc)));
    v4 sum = st[0];
    for (int i = 1; i < 16; i++) sum = v_add(sum, st[i]);
    const v4 x0 = st[0];
    st[0] = v_sub(sum, v_double(x0));
    st[1] = v_add(sum, st[1]);
    st[2] = v_add(sum, v_double(st[2]));
    st[3] = v_add(sum, v_halve(st[3]));
    st[4] = v_add(sum, v_add(v_double(st[4]), st[4]));
    st[5] = v_add(sum, v_double(v_double(st[5])));
    st[6] = v_sub(sum, v_halve(st[6]));
    st[7] = v_sub(sum, v_add(v_double(st[7]), st[7]));
    st[8] = v_sub(sum, v_double(v_double(st[8])));
    st[9] = v_add(sum, v_mul_inv_pow2(st[9], 3));
    st[10] = v_add(sum, v_mul_inv_pow2(st[10], 4));
    st[11] = v_add(sum, v_mul_inv_pow2(st[11], 5));
    st[12] = v_sub(sum, v_mul_inv_pow2(st[12], 3));
    st[13] = v_sub(sum, v_mul_inv_pow2(st[13], 4));
    st[14] = v_sub(sum, v_mul_inv_pow2(st[14], 5));
    st[15] = v_add(sum, g_diag15_inv32 ? v_mul_inv_pow2(st[15], 32) : v_mul(st[15], v_set1(g_diag15)));
}

static void v_permute(v4 *st)
{
    v_mds_light16(st);
    for (int r = 0; r < 4; r++) {
        for (int i = 0; i < 16; i++) st[i] = v_sbox7(v_add(st[i], v_set1(g_ext[r][i])));
        v_mds_light16(st);
    }
    for (int k = 0; k < 22; k++) v_internal_round(st, g_int[k]);
    for (int r = 4; r < 8; r++) {
        for (int i = 0; i < 16; i++) st[i] = v_sbox7(v_add(st[i], v_set1(g_ext[r][i])));
        v_mds_light16(st);
    }
}

/* Word i of 4 records (stride `stride` u64 apart) into one vector, and back. */
static inline v4 v_gather4(const uint64_t *base, uint64_t stride, int i)
{
    return _mm256_set_epi64x((long long)base[3 * stride + i], (long long)base[2 * stride + i],
                             (long long)base[stride + i], (long long)base[i]);
}
static inline void v_scatter4(uint64_t *base, uint64_t stride, int i, v4 x)
{
    uint64_t t[4];
    _mm256_storeu_si256((v4 *)t, x);
    for (int l = 0; l < 4; l++) base[l * stride + i] = t[l];
}

/* Leaf digests of rows [r0, r0 + 4) of a w-wide matrix (PaddingFreeSponge<16,8,8>). */
static void leaf4(const uint64_t *mat, uint64_t w, uint64_t r0, uint64_t *digests)
{
    v4 st[16];
    for (int i = 0; i < 16; i++) st[i] = _mm256_setzero_si256();
    const uint64_t *rows = mat + r0 * w;
    for (uint64_t pos = 0; pos < w; pos += 8) {
        const uint64_t len = w - pos < 8 ? w - pos : 8;
        for (uint64_t i = 0; i < len; i++) st[i] = v_gather4(rows + pos, w, (int)i);
        v_permute(st);
    }
    for (int i = 0; i < 8; i++) v_scatter4(digests + r0 * 8, 8, i, st[i]);
}

/* One leaf digest (the tail rows). */
static void leaf1(const uint64_t *row, uint64_t w, uint64_t *out)
{
    v4 st[16];
    for (int i = 0; i < 16; i++) st[i] = _mm256_setzero_si256();
    for (uint64_t pos = 0; pos < w; pos += 8) {
        const uint64_t len = w - pos < 8 ? w - pos : 8;
        for (uint64_t i = 0; i < len; i++) st[i] = v_set1(row[pos + i]);
        v_permute(st);
    }
    uint64_t t[4];
    for (int i = 0; i < 8; i++) {
        _mm256_storeu_si256((v4 *)t, st[i]);
        out[i] = t[0];
    }
}

/* Parents [p0, p0 + cnt) (cnt <= 4) of prev (TruncatedPermutation<2,8,16>). */
static void compress4(const uint64_t *prev, uint64_t *next, uint64_t p0, int cnt)
{
    v4 st[16];
    uint64_t buf[4][16];
    for (int l = 0; l < 4; l++) {
        const uint64_t p = p0 + (uint64_t)(l < cnt ? l : 0);
        memcpy(buf[l], prev + p * 16, 128);
    }
    for (int i = 0; i < 16; i++)
        st[i] = _mm256_set_epi64x((long long)buf[3][i], (long long)buf[2][i], (long long)buf[1][i],
                                  (long long)buf[0][i]);
    v_permute(st);
    uint64_t t[4];
    for (int i = 0; i < 8; i++) {
        _mm256_storeu_si256((v4 *)t, st[i]);
        for (int l = 0; l < cnt; l++) next[(p0 + l) * 8 + i] = t[l];
    }
}

static uint64_t padded_len(uint64_t raw) { return raw <= 1 ? raw : (raw + 1) / 2 * 2; }

/* Number of layers and their lengths (merkle_tree.rs:577-585 schedule). */
uint32_t cb_merkle_layer_lens(uint64_t h, uint64_t *lens)
{
    uint32_t n = 0;
    uint64_t len = padded_len(h);
    if (lens) lens[n] = len;
    n++;
    while (len > 1) {
        len = padded_len(len / 2);
        if (lens) lens[n] = len;
        n++;
    }
    return n;
}

/* Every digest layer of the tree over the h x w matrix (concatenated, zero
 * digests in padded slots) and the root. */
void cb_merkle_commit(const uint64_t *mat, uint64_t h, uint64_t w, uint64_t *layers, uint64_t root[8])
{
    uint64_t lens[66];
    const uint32_t nl = cb_merkle_layer_lens(h, lens);
    memset(layers, 0, lens[0] * 64);
    const int64_t quads = (int64_t)(h / 4);
#pragma omp parallel for schedule(static)
    for (int64_t q = 0; q < quads; q++) leaf4(mat, w, (uint64_t)q * 4, layers);
    for (uint64_t r = (uint64_t)quads * 4; r < h; r++) leaf1(mat + r * w, w, layers + r * 8);
    uint64_t off = 0;
    for (uint32_t l = 0; l + 1 < nl; l++) {
        const uint64_t *prev = layers + off * 8;
        uint64_t *next = layers + (off + lens[l]) * 8;
        const uint64_t raw = lens[l] / 2;
        memset(next, 0, lens[l + 1] * 64);
        const int64_t blocks = (int64_t)((raw + 3) / 4);
#pragma omp parallel for schedule(static) if (blocks > 64)
        for (int64_t b = 0; b < blocks; b++) {
            const uint64_t p0 = (uint64_t)b * 4;
            compress4(prev, next, p0, (int)(raw - p0 < 4 ? raw - p0 : 4));
        }
        off += lens[l];
    }
    memcpy(root, layers + off * 8, 64);
}

/* ---- DFT (radix-2 DIT on the row-major matrix, columns in vectors) ------- */
static uint32_t bitrev(uint64_t x, uint32_t bits)
{
    uint64_t r = 0;
    for (uint32_t i = 0; i < bits; i++) r |= ((x >> i) & 1) << (bits - 1 - i);
    return (uint32_t)r;
}

/* Butterflies of stage s (span half = 2^(s-1)) over rows [b0, b1) of blocks
 * of 2^s rows: u + w v, u - w v. tw[j * tstride] = w_{2^s}^j. */
static void dit_stage(uint64_t *X, uint64_t w, uint64_t b0, uint64_t b1, uint32_t s, const uint64_t *tw,
                      uint64_t tstride)
{
    const uint64_t half = 1ULL << (s - 1), blk = half << 1;
    for (uint64_t b = b0; b < b1; b += blk)
        for (uint64_t j = 0; j < half; j++) {
            uint64_t *u = X + (b + j) * w, *v = X + (b + j + half) * w;
            const uint64_t t = tw[j * tstride];
            if ((w & 3) == 0) {
                const v4 tv = v_set1(t);
                for (uint64_t c = 0; c < w; c += 4) {
                    const v4 a = _mm256_loadu_si256((const v4 *)(u + c));
                    const v4 bb = j ? v_mul(_mm256_loadu_si256((const v4 *)(v + c)), tv)
                                    : _mm256_loadu_si256((const v4 *)(v + c));
                    _mm256_storeu_si256((v4 *)(u + c), v_add(a, bb));
                    _mm256_storeu_si256((v4 *)(v + c), v_sub(a, bb));
                }
            } else {
                for (uint64_t c = 0; c < w; c++) {
                    const uint64_t a = u[c], bb = j ? s_mul(v[c], t) : v[c];
                    u[c] = s_add(a, bb);
                    v[c] = s_sub(a, bb);
                }
            }
        }
}

/* LDE: zero-pad the h x w coefficient matrix to n = h << log_blowup rows and
 * transform every column on the subgroup of order n (natural order in and
 * out), as dft_batch of the padded matrix (writer.rs:73-81). */
void cb_lde(const uint64_t *in, uint64_t h, uint64_t w, uint32_t log_blowup, uint64_t *out)
{
    uint32_t lgh = 0;
    while ((1ULL << lgh) < h) lgh++;
    const uint32_t L = lgh + log_blowup;
    const uint64_t n = 1ULL << L;
    memset(out, 0, n * w * 8);
    if (n == 1) {
        memcpy(out, in, w * 8);
        return;
    }
    /* bit-reversed input order for the DIT transform */
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < (int64_t)h; j++) memcpy(out + (uint64_t)bitrev((uint64_t)j, L) * w, in + (uint64_t)j * w, w * 8);
    /* w_n^j for j < n/2; stage s reads it with stride n / 2^s */
    uint64_t *tw = (uint64_t *)malloc((n / 2) * 8);
    const uint64_t g = s_pow(7, (CB_P - 1) >> L); /* TWO_ADIC_GENERATORS[L] */
    const int64_t chunks = (int64_t)((n / 2 + 4095) / 4096);
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < chunks; c++) {
        const uint64_t j0 = (uint64_t)c * 4096;
        uint64_t x = s_pow(g, j0);
        for (uint64_t j = j0; j < j0 + 4096 && j < n / 2; j++) {
            tw[j] = x;
            x = s_mul(x, g);
        }
    }
    /* stages 1..k inside blocks of 2^k rows (cache resident), then the rest */
    uint32_t k = L < 10 ? L : 10;
    while (k > 1 && ((1ULL << k) * w * 8) > (256u << 10)) k--;
    const uint64_t B = 1ULL << k;
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < (int64_t)(n / B); b++)
        for (uint32_t s = 1; s <= k; s++) dit_stage(out, w, (uint64_t)b * B, (uint64_t)b * B + B, s, tw, n >> s);
    for (uint32_t s = k + 1; s <= L; s++) {
        const uint64_t half = 1ULL << (s - 1);
        /* split each stage into independent pieces: a block of 2^s rows, or
         * a range of j inside one block when blocks are few */
        const uint64_t blocks = n >> s;
        const uint64_t jparts = blocks >= 64 ? 1 : 64 / blocks;
        const uint64_t jlen = (half + jparts - 1) / jparts;
#pragma omp parallel for schedule(static)
        for (int64_t t = 0; t < (int64_t)(blocks * jparts); t++) {
            const uint64_t blk = (uint64_t)t / jparts, part = (uint64_t)t % jparts;
            const uint64_t bs = blk << s;
            const uint64_t j0 = part * jlen, j1 = j0 + jlen < half ? j0 + jlen : half;
            for (uint64_t j = j0; j < j1; j++) {
                uint64_t *u = out + (bs + j) * w, *v = out + (bs + j + half) * w;
                const uint64_t tt = tw[j * (n >> s)];
                if ((w & 3) == 0) {
                    const v4 tv = v_set1(tt);
                    for (uint64_t c = 0; c < w; c += 4) {
                        const v4 a = _mm256_loadu_si256((const v4 *)(u + c));
                        const v4 bb = v_mul(_mm256_loadu_si256((const v4 *)(v + c)), tv);
                        _mm256_storeu_si256((v4 *)(u + c), v_add(a, bb));
                        _mm256_storeu_si256((v4 *)(v + c), v_sub(a, bb));
                    }
                } else {
                    for (uint64_t c = 0; c < w; c++) {
                        const uint64_t a = u[c], bb = s_mul(v[c], tt);
                        u[c] = s_add(a, bb);
                        v[c] = s_sub(a, bb);
                    }
                }
            }
        }
    }
    free(tw);
}

/* ---- row fold (mle.rs:8-22 on each row, EF challenges, base rows) --------- */
#define CB_W 7ULL
/* out[t] = sum_j eq(r, j) row_t[j] over 2^k base entries, EF out (2 u64). */
void cb_fold_rows(const uint64_t *mat, uint64_t h, uint32_t k, const uint64_t *r, uint64_t *out)
{
    const uint64_t W = 1ULL << k;
    uint64_t *eq = (uint64_t *)malloc(2 * W * 8);
    eq[0] = 1;
    eq[1] = 0;
    for (uint32_t b = 0; b < k; b++) {
        const uint64_t r0 = r[2 * b] % CB_P, r1 = r[2 * b + 1] % CB_P;
        const uint64_t m0 = s_sub(1, r0), m1 = s_sub(0, r1);
        for (uint64_t j = (1ULL << b); j-- > 0;) {
            /* eq over b + 1 bits: j with bit b clear -> (1 - r_b), set -> r_b */
            const uint64_t e0 = eq[2 * j], e1 = eq[2 * j + 1];
            const uint64_t hi = j | (1ULL << b);
            eq[2 * hi] = s_add(s_mul(e0, r0), s_mul(CB_W, s_mul(e1, r1)));
            eq[2 * hi + 1] = s_add(s_mul(e0, r1), s_mul(e1, r0));
            eq[2 * j] = s_add(s_mul(e0, m0), s_mul(CB_W, s_mul(e1, m1)));
            eq[2 * j + 1] = s_add(s_mul(e0, m1), s_mul(e1, m0));
        }
    }
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < (int64_t)h; t++) {
        const uint64_t *row = mat + (uint64_t)t * W;
        u128 a0 = 0, a1 = 0;
        uint64_t c0 = 0, c1 = 0;
        for (uint64_t j = 0; j < W; j++) {
            /* exact sums of the 128-bit products, reduced once per output */
            const u128 p0 = (u128)eq[2 * j] * row[j], p1 = (u128)eq[2 * j + 1] * row[j];
            a0 += p0;
            c0 += a0 < p0;
            a1 += p1;
            c1 += a1 < p1;
        }
        /* value = a + c 2^128, 2^128 = -2^32 (mod p) */
        uint64_t v0 = s_reduce128((uint64_t)a0, (uint64_t)(a0 >> 64) % CB_P);
        uint64_t v1 = s_reduce128((uint64_t)a1, (uint64_t)(a1 >> 64) % CB_P);
        v0 = s_sub(v0, s_mul(c0 % CB_P, 1ULL << 32));
        v1 = s_sub(v1, s_mul(c1 % CB_P, 1ULL << 32));
        out[2 * t] = v0;
        out[2 * t + 1] = v1;
    }
    free(eq);
}

int cb_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void cb_set_threads(int n)
{
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
