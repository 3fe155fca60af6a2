/*
 * CPU oracle for the Q4_0 / Q4_K_M dequant-matvec path (C restatement of the
 * reference's Rust CPU code).  TEST INFRASTRUCTURE ONLY: the checker for the
 * HIP path, loaded by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg, never by the product library.
 *
 * Parity pins (each is a test under tests/):
 *   axo_f16_bits_to_f32      exhaustive 65,536 patterns vs numpy float16 widening
 *   axo_f32_to_f16_bits      vs numpy float32->float16 (RNE) on edge and random values
 *   axo_unpack_scale_min_k4  AT-1312 hand-verified pairs + the q[j] vs q[j-4]
 *                            discriminator, and all 8 x 4096 (j, byte-pattern) cases
 *                            vs an independent numpy bit-spread
 *   axo_q4_0_dot             Q4_0 layout KATs (-128.0, -96.0), closed forms,
 *                            pure-Python float32 loop on small inputs
 *   axo_q4k_dot              AT-1323 (determinism, n=0 -> +0.0), closed forms,
 *                            pure-Python float32 loop on small inputs
 *   axo_*_dequant            closed form (one rounding), numpy restatement
 *   axo_generate_q4km_test_data  independent Python-integer LCG restatement
 *   axo_*_f64                error bounds against the f32 paths
 * Build: -O2 -ffp-contract=off, no fast-math (see oracle/Makefile).
 */
#include "q4_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------
 * binary16 <-> binary32 (IEEE 754).  The reference decodes with half 2.7.1
 * (Cargo.lock:478-480), whose conversion is the exact IEEE widening; NaNs come
 * back quiet (quiet bit set), the other mantissa bits kept.
 * ------------------------------------------------------------------------- */
static inline float bits_to_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static inline uint32_t f32_to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

float axo_f16_bits_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0x1Fu) {
        if (m == 0) return bits_to_f32(sign | 0x7F800000u);
        return bits_to_f32(sign | 0x7FC00000u | (m << 13));
    }
    if (e == 0) {
        if (m == 0) return bits_to_f32(sign);
        /* subnormal: value m * 2^-24.  Shift until bit 10 is set; the value is
         * then (m/1024) * 2^(-14 - shift), biased f32 exponent 113 - shift. */
        int shift = 0;
        while ((m & 0x400u) == 0) {
            m <<= 1;
            ++shift;
        }
        return bits_to_f32(sign | ((uint32_t)(113 - shift) << 23) | ((m & 0x3FFu) << 13));
    }
    return bits_to_f32(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t axo_f32_to_f16_bits(float f) {
    const uint32_t u = f32_to_bits(f);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t e = (u >> 23) & 0xFFu;
    const uint32_t m = u & 0x7FFFFFu;
    if (e == 0xFFu) { /* inf / NaN (NaN kept quiet, top payload bits kept) */
        if (m == 0) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | (m >> 13));
    }
    const int exp = (int)e - 127; /* unbiased */
    if (exp > 15) return (uint16_t)(sign | 0x7C00u);
    /* Significand with hidden bit, 24 bits; f32 subnormals are far below the
     * f16 range and round to zero below. */
    uint32_t sig = (e == 0) ? m : (m | 0x800000u);
    int shift; /* right shift that aligns sig to the f16 mantissa grid */
    uint32_t base;
    if (exp >= -14) { /* normal f16 */
        shift = 13;
        base = (uint32_t)(exp + 15) << 10;
        sig &= 0x7FFFFFu; /* drop hidden bit, carried by base */
    } else {          /* subnormal f16: units of 2^-24 */
        shift = -exp - 1; /* = 13 + (-14 - exp) */
        base = 0;
        if (e == 0 || shift > 31) return sign; /* |f| < 2^-25: rounds to 0 */
    }
    uint32_t q = sig >> shift;
    const uint32_t rem = sig & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q += 1u; /* RNE; carry may bump exponent */
    return (uint16_t)(sign | (base + q));
}

/* ---------------------------------------------------------------------------
 * get_scale_min_k4 (tests/common_helpers.rs:352-371; DESIGN.md:456-470).
 * For j >= 4 the high bits of m come from scales[j], not scales[j-4].
 * ------------------------------------------------------------------------- */
void axo_unpack_scale_min_k4(const uint8_t s[12], int j, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = (uint8_t)(s[j] & 63u);
        *m = (uint8_t)(s[j + 4] & 63u);
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0Fu) | (((s[j - 4] >> 6) & 3u) << 4));
        *m = (uint8_t)(((s[j + 4] >> 4) & 0x0Fu) | (((s[j] >> 6) & 3u) << 4));
    }
}

static inline float load_f16le(const uint8_t *p) {
    return axo_f16_bits_to_f32((uint16_t)(p[0] | ((uint16_t)p[1] << 8)));
}

/* ---------------------------------------------------------------------------
 * Q4_0: q4_0_dequant_matvec_cpu (benches/common.rs:212-259).
 * acc += w_lo * x[32b+k]; acc += w_hi * x[32b+k+16], sequential f32, k = 0..15.
 * ------------------------------------------------------------------------- */
float axo_q4_0_dot(const uint8_t *q, const float *x, size_t n_blocks) {
    float acc = 0.0f;
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint8_t *blk = q + b * AXO_Q4_0_BLOCK_BYTES;
        const float scale = load_f16le(blk);
        const float *xb = x + b * AXO_Q4_0_BLOCK_ELEMS;
        for (int k = 0; k < 16; ++k) {
            const uint8_t packed = blk[2 + k];
            const float w_lo = ((float)(packed & 0x0F) - 8.0f) * scale;
            acc += w_lo * xb[k];
            const float w_hi = ((float)((packed >> 4) & 0x0F) - 8.0f) * scale;
            acc += w_hi * xb[k + 16];
        }
    }
    return acc;
}

/* ---------------------------------------------------------------------------
 * Q4_K: q4km_dequant_matvec_cpu (tests/common_helpers.rs:411-461).
 * sb -> chunk 0..3 -> l 0..31: sum += lo_f * x[..l]; sum += hi_f * x[..32+l].
 * ------------------------------------------------------------------------- */
float axo_q4k_dot(const uint8_t *q, const float *x, size_t n_superblocks) {
    float sum = 0.0f;
    for (size_t sb = 0; sb < n_superblocks; ++sb) {
        const uint8_t *base = q + sb * AXO_Q4K_SB_BYTES;
        const float d = load_f16le(base);
        const float dmin = load_f16le(base + 2);
        const uint8_t *scales = base + 4;
        for (int chunk = 0; chunk < 4; ++chunk) {
            uint8_t sc0, m0, sc1, m1;
            axo_unpack_scale_min_k4(scales, chunk * 2, &sc0, &m0);
            axo_unpack_scale_min_k4(scales, chunk * 2 + 1, &sc1, &m1);
            const float d1 = d * (float)sc0;
            const float m1f = dmin * (float)m0;
            const float d2 = d * (float)sc1;
            const float m2f = dmin * (float)m1;
            const uint8_t *qs = base + 16 + chunk * 32;
            const float *xc = x + sb * AXO_Q4K_SB_ELEMS + chunk * 64;
            for (int l = 0; l < 32; ++l) {
                const uint8_t byte = qs[l];
                const float lo = (float)(byte & 0x0F);
                const float hi = (float)((byte >> 4) & 0x0F);
                const float lo_f = d1 * lo - m1f;
                const float hi_f = d2 * hi - m2f;
                sum += lo_f * xc[l];
                sum += hi_f * xc[32 + l];
            }
        }
    }
    return sum;
}

void axo_q4_0_matvec(const uint8_t *q, const float *x, float *y, size_t n_rows,
                     size_t blocks_per_row) {
    const size_t row_bytes = blocks_per_row * AXO_Q4_0_BLOCK_BYTES;
    for (size_t r = 0; r < n_rows; ++r) y[r] = axo_q4_0_dot(q + r * row_bytes, x, blocks_per_row);
}

void axo_q4k_matvec(const uint8_t *q, const float *x, float *y, size_t n_rows,
                    size_t sb_per_row) {
    const size_t row_bytes = sb_per_row * AXO_Q4K_SB_BYTES;
    for (size_t r = 0; r < n_rows; ++r) y[r] = axo_q4k_dot(q + r * row_bytes, x, sb_per_row);
}

/* --- row-parallel variants ------------------------------------------------ */
typedef struct {
    const uint8_t *q;
    const float *x;
    float *y;
    size_t r0, r1, units;
    int kind; /* 0 = Q4_0, 1 = Q4_K */
} mv_job;

static void *mv_worker(void *arg) {
    mv_job *j = (mv_job *)arg;
    if (j->kind == 0) {
        const size_t rb = j->units * AXO_Q4_0_BLOCK_BYTES;
        for (size_t r = j->r0; r < j->r1; ++r) j->y[r] = axo_q4_0_dot(j->q + r * rb, j->x, j->units);
    } else {
        const size_t rb = j->units * AXO_Q4K_SB_BYTES;
        for (size_t r = j->r0; r < j->r1; ++r) j->y[r] = axo_q4k_dot(j->q + r * rb, j->x, j->units);
    }
    return NULL;
}

static void mv_parallel(int kind, const uint8_t *q, const float *x, float *y, size_t n_rows,
                        size_t units, int n_threads) {
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 256) n_threads = 256;
    if ((size_t)n_threads > n_rows) n_threads = n_rows ? (int)n_rows : 1;
    pthread_t th[256];
    mv_job jobs[256];
    const size_t per = (n_rows + (size_t)n_threads - 1) / (size_t)n_threads;
    int started = 0;
    for (int t = 0; t < n_threads; ++t) {
        size_t r0 = (size_t)t * per, r1 = r0 + per;
        if (r0 > n_rows) r0 = n_rows;
        if (r1 > n_rows) r1 = n_rows;
        jobs[t] = (mv_job){q, x, y, r0, r1, units, kind};
        if (t == n_threads - 1 || pthread_create(&th[t], NULL, mv_worker, &jobs[t]) != 0) {
            mv_worker(&jobs[t]); /* last slice (or a failed spawn) runs inline */
        } else {
            ++started;
            continue;
        }
    }
    for (int t = 0; t < n_threads - 1 && started > 0; ++t) {
        pthread_join(th[t], NULL);
        --started;
    }
}

void axo_q4k_matvec_mt(const uint8_t *q, const float *x, float *y, size_t n_rows,
                       size_t sb_per_row, int n_threads) {
    mv_parallel(1, q, x, y, n_rows, sb_per_row, n_threads);
}

void axo_q4_0_matvec_mt(const uint8_t *q, const float *x, float *y, size_t n_rows,
                        size_t blocks_per_row, int n_threads) {
    mv_parallel(0, q, x, y, n_rows, blocks_per_row, n_threads);
}

/* ---------------------------------------------------------------------------
 * Dequantisation in the reference's element order.
 * ------------------------------------------------------------------------- */
void axo_q4_0_dequant(const uint8_t *q, float *w, size_t n_blocks) {
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint8_t *blk = q + b * AXO_Q4_0_BLOCK_BYTES;
        const float scale = load_f16le(blk);
        float *wb = w + b * AXO_Q4_0_BLOCK_ELEMS;
        for (int k = 0; k < 16; ++k) {
            const uint8_t packed = blk[2 + k];
            wb[k] = ((float)(packed & 0x0F) - 8.0f) * scale;
            wb[k + 16] = ((float)((packed >> 4) & 0x0F) - 8.0f) * scale;
        }
    }
}

void axo_q4k_dequant(const uint8_t *q, float *w, size_t n_superblocks) {
    for (size_t sb = 0; sb < n_superblocks; ++sb) {
        const uint8_t *base = q + sb * AXO_Q4K_SB_BYTES;
        const float d = load_f16le(base);
        const float dmin = load_f16le(base + 2);
        float *ws = w + sb * AXO_Q4K_SB_ELEMS;
        for (int chunk = 0; chunk < 4; ++chunk) {
            uint8_t sc0, m0, sc1, m1;
            axo_unpack_scale_min_k4(base + 4, chunk * 2, &sc0, &m0);
            axo_unpack_scale_min_k4(base + 4, chunk * 2 + 1, &sc1, &m1);
            const float d1 = d * (float)sc0, m1f = dmin * (float)m0;
            const float d2 = d * (float)sc1, m2f = dmin * (float)m1;
            for (int l = 0; l < 32; ++l) {
                const uint8_t byte = base[16 + chunk * 32 + l];
                ws[chunk * 64 + l] = d1 * (float)(byte & 0x0F) - m1f;
                ws[chunk * 64 + 32 + l] = d2 * (float)((byte >> 4) & 0x0F) - m2f;
            }
        }
    }
}

/* ---------------------------------------------------------------------------
 * f64 references (same f32 weights, exact f64 products, f64 sums).
 * ------------------------------------------------------------------------- */
void axo_q4k_matvec_f64(const uint8_t *q, const float *x, double *y, double *absdot,
                        size_t n_rows, size_t sb_per_row) {
    float w[AXO_Q4K_SB_ELEMS];
    const size_t rb = sb_per_row * AXO_Q4K_SB_BYTES;
    for (size_t r = 0; r < n_rows; ++r) {
        double s = 0.0, a = 0.0;
        for (size_t sb = 0; sb < sb_per_row; ++sb) {
            axo_q4k_dequant(q + r * rb + sb * AXO_Q4K_SB_BYTES, w, 1);
            const float *xs = x + sb * AXO_Q4K_SB_ELEMS;
            for (int i = 0; i < (int)AXO_Q4K_SB_ELEMS; ++i) {
                const double p = (double)w[i] * (double)xs[i];
                s += p;
                a += fabs(p);
            }
        }
        y[r] = s;
        if (absdot) absdot[r] = a;
    }
}

void axo_q4_0_matvec_f64(const uint8_t *q, const float *x, double *y, double *absdot,
                         size_t n_rows, size_t blocks_per_row) {
    float w[AXO_Q4_0_BLOCK_ELEMS];
    const size_t rb = blocks_per_row * AXO_Q4_0_BLOCK_BYTES;
    for (size_t r = 0; r < n_rows; ++r) {
        double s = 0.0, a = 0.0;
        for (size_t b = 0; b < blocks_per_row; ++b) {
            axo_q4_0_dequant(q + r * rb + b * AXO_Q4_0_BLOCK_BYTES, w, 1);
            const float *xb = x + b * AXO_Q4_0_BLOCK_ELEMS;
            for (int i = 0; i < (int)AXO_Q4_0_BLOCK_ELEMS; ++i) {
                const double p = (double)w[i] * (double)xb[i];
                s += p;
                a += fabs(p);
            }
        }
        y[r] = s;
        if (absdot) absdot[r] = a;
    }
}

/* --- batched: per column, the Q4_K dot with f32(f16 activation) ----------- */
typedef struct {
    const uint8_t *q;
    const float *xf; /* batch x cols f32, column b contiguous */
    float *y;
    size_t r0, r1, sb, cols, batch;
} mm_job;

static void *mm_worker(void *arg) {
    mm_job *j = (mm_job *)arg;
    const size_t rb = j->sb * AXO_Q4K_SB_BYTES;
    for (size_t r = j->r0; r < j->r1; ++r)
        for (size_t b = 0; b < j->batch; ++b)
            j->y[r * j->batch + b] = axo_q4k_dot(j->q + r * rb, j->xf + b * j->cols, j->sb);
    return NULL;
}

void axo_q4k_matmul_f16x(const uint8_t *q, const uint16_t *x_f16, float *y, size_t n_rows,
                         size_t sb_per_row, size_t batch, int n_threads) {
    const size_t cols = sb_per_row * AXO_Q4K_SB_ELEMS;
    const size_t nx = cols * batch;
    float *xf = (float *)malloc(sizeof(float) * (nx > 0 ? nx : 1));
    if (!xf) return;
    for (size_t i = 0; i < nx; ++i) xf[i] = axo_f16_bits_to_f32(x_f16[i]);
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 256) n_threads = 256;
    if ((size_t)n_threads > n_rows) n_threads = n_rows ? (int)n_rows : 1;
    pthread_t th[256];
    mm_job jobs[256];
    const size_t per = (n_rows + (size_t)n_threads - 1) / (size_t)n_threads;
    int spawned[256] = {0};
    for (int t = 0; t < n_threads; ++t) {
        size_t r0 = (size_t)t * per, r1 = r0 + per;
        if (r0 > n_rows) r0 = n_rows;
        if (r1 > n_rows) r1 = n_rows;
        jobs[t] = (mm_job){q, xf, y, r0, r1, sb_per_row, cols, batch};
        if (t < n_threads - 1 && pthread_create(&th[t], NULL, mm_worker, &jobs[t]) == 0)
            spawned[t] = 1;
        else
            mm_worker(&jobs[t]);
    }
    for (int t = 0; t < n_threads; ++t)
        if (spawned[t]) pthread_join(th[t], NULL);
    free(xf);
}

/* ---------------------------------------------------------------------------
 * generate_q4km_test_data (tests/common_helpers.rs:476-519): Knuth MMIX LCG,
 * state = seed ^ 0x9E3779B97F4A7C15; u64 -> f32 and u64::MAX -> f32 (2^64) are
 * round-to-nearest conversions; all f32 arithmetic uncontracted.
 * ------------------------------------------------------------------------- */
static inline uint64_t lcg_next(uint64_t *s) {
    *s = *s * 6364136223846793005ull + 1442695040888963407ull;
    return *s;
}

void axo_generate_q4km_test_data(uint32_t n_superblocks, uint64_t seed, uint8_t *q, float *x) {
    uint64_t state = seed ^ 0x9E3779B97F4A7C15ull;
    const float umax = (float)UINT64_MAX;
    for (uint32_t i = 0; i < n_superblocks; ++i) {
        uint8_t *b = q + (size_t)i * AXO_Q4K_SB_BYTES;
        const float d_raw = 0.1f + ((float)lcg_next(&state) / umax) * 1.9f;
        const uint16_t d16 = axo_f32_to_f16_bits(d_raw);
        b[0] = (uint8_t)(d16 & 0xFF);
        b[1] = (uint8_t)(d16 >> 8);
        const float dmin_raw = ((float)lcg_next(&state) / umax) * 0.5f;
        const uint16_t m16 = axo_f32_to_f16_bits(dmin_raw);
        b[2] = (uint8_t)(m16 & 0xFF);
        b[3] = (uint8_t)(m16 >> 8);
        for (int k = 0; k < 12; ++k) b[4 + k] = (uint8_t)(lcg_next(&state) & 0xFF);
        for (int k = 0; k < 128; ++k) b[16 + k] = (uint8_t)(lcg_next(&state) & 0xFF);
    }
    for (size_t i = 0; i < (size_t)n_superblocks * AXO_Q4K_SB_ELEMS; ++i)
        x[i] = ((float)lcg_next(&state) / umax) * 2.0f - 1.0f;
}

/* ---------------------------------------------------------------------------
 * Benchmark-shape generators (SplitMix64, Steele/Lea/Flood 2014).
 * ------------------------------------------------------------------------- */
static inline uint64_t splitmix64(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline float unit24(uint64_t v) { return (float)(v >> 40) * (1.0f / 16777216.0f); }

void axo_gen_q4k_weights(uint64_t seed, uint8_t *q, size_t n_superblocks) {
    uint64_t s = seed;
    for (size_t i = 0; i < n_superblocks; ++i) {
        uint8_t *b = q + i * AXO_Q4K_SB_BYTES;
        const uint16_t d16 = axo_f32_to_f16_bits(0.001f + 0.049f * unit24(splitmix64(&s)));
        const uint16_t m16 = axo_f32_to_f16_bits(0.02f * unit24(splitmix64(&s)));
        b[0] = (uint8_t)(d16 & 0xFF);
        b[1] = (uint8_t)(d16 >> 8);
        b[2] = (uint8_t)(m16 & 0xFF);
        b[3] = (uint8_t)(m16 >> 8);
        for (int k = 0; k < 140; k += 8) { /* 12 scale bytes + 128 qs bytes */
            uint64_t v = splitmix64(&s);
            for (int t = 0; t < 8 && k + t < 140; ++t) b[4 + k + t] = (uint8_t)(v >> (8 * t));
        }
    }
}

void axo_gen_q4_0_weights(uint64_t seed, uint8_t *q, size_t n_blocks) {
    uint64_t s = seed;
    for (size_t i = 0; i < n_blocks; ++i) {
        uint8_t *b = q + i * AXO_Q4_0_BLOCK_BYTES;
        const uint16_t d16 = axo_f32_to_f16_bits(0.001f + 0.049f * unit24(splitmix64(&s)));
        b[0] = (uint8_t)(d16 & 0xFF);
        b[1] = (uint8_t)(d16 >> 8);
        uint64_t v0 = splitmix64(&s), v1 = splitmix64(&s);
        for (int t = 0; t < 8; ++t) {
            b[2 + t] = (uint8_t)(v0 >> (8 * t));
            b[10 + t] = (uint8_t)(v1 >> (8 * t));
        }
    }
}

void axo_gen_normal_f32(uint64_t seed, float *x, size_t n, double sigma) {
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        const double u1 = ((double)(splitmix64(&s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        const double u2 = (double)(splitmix64(&s) >> 11) * (1.0 / 9007199254740992.0);
        const double r = sqrt(-2.0 * log(u1));
        x[i] = (float)(sigma * r * cos(two_pi * u2));
        if (i + 1 < n) x[i + 1] = (float)(sigma * r * sin(two_pi * u2));
    }
}
