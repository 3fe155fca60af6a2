/*
 * CPU oracle for the ggml k-quant formats that real Q4_K_M checkpoints mix in
 * next to Q4_K: Q5_K and Q6_K.  TEST INFRASTRUCTURE ONLY (the checker for the
 * HIP path; loaded by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg, never by the product library).
 *
 * The reference has no loader or kernel for these formats ("GGUF file parsing
 * - separate", ROADMAP.md:230-234; .pipeline/milestones/M2.5-q4_0-matmul.json:24).
 * They are ggml's, the third-party library behind llama.cpp, which is not
 * vendored under the reference.  Restated from ggml's published block layouts
 * (ggml-common.h: block_q5_K, block_q6_K; ggml-quants.c: dequantize_row_q5_K,
 * dequantize_row_q6_K; QK_K = 256), unchanged since the k-quants landed in
 * llama.cpp in 2023 and as stored by GGUF v3 (ggml type ids Q5_K = 13,
 * Q6_K = 14):
 *
 *   Q5_K, 176 bytes: d f16 @0, dmin f16 @2, scales[12] @4 (get_scale_min_k4,
 *     as Q4_K), qh[32] @16, qs[128] @48.  For chunk j = 0..3 (64 weights),
 *     l = 0..31:  w[64j + l]      = d*sc(2j)   * (lo(qs[32j+l]) + 16*bit(qh[l], 2j))   - dmin*m(2j)
 *                 w[64j + 32 + l] = d*sc(2j+1) * (hi(qs[32j+l]) + 16*bit(qh[l], 2j+1)) - dmin*m(2j+1)
 *   Q6_K, 210 bytes: ql[128] @0, qh[64] @128, scales[16] (int8) @192,
 *     d f16 @208.  For half n = 0..1 (128 weights; ql += 64n, qh += 32n,
 *     sc += 8n), l = 0..31, is = l/16:
 *       w[128n + l]      = d*sc[is+0] * ((lo(ql[l])    | ((qh[l] >> 0) & 3) << 4) - 32)
 *       w[128n + 32 + l] = d*sc[is+2] * ((lo(ql[l+32]) | ((qh[l] >> 2) & 3) << 4) - 32)
 *       w[128n + 64 + l] = d*sc[is+4] * ((hi(ql[l])    | ((qh[l] >> 4) & 3) << 4) - 32)
 *       w[128n + 96 + l] = d*sc[is+6] * ((hi(ql[l+32]) | ((qh[l] >> 6) & 3) << 4) - 32)
 *
 * Arithmetic: Q5_K d*sc and dmin*m are exact in f32 (11 x 6 bits), the
 * product with q (5 bits) is exact, and the subtraction rounds once.  Q6_K
 * (d*sc)*q needs at most 11 + 7 + 5 bits: every weight is exact in f32.
 * Dot products: sequential f32 in element order, no FMA (the convention of
 * the reference's Q4_K dot, which has no Q5_K / Q6_K counterpart).
 *
 * Parity pins (tests/test_oracle_pins.py): an independent numpy restatement
 * written from the layouts above (oracle/q4_numpy.py); closed forms (one
 * non-zero field at a time: each weight index has a hand-derived byte/bit
 * source); planted mistakes (swapped qh bit pairs, the Q4_K-style q[j-4]
 * scale spread, ql halves exchanged) that the pins reject.
 * Build: -O2 -ffp-contract=off, no fast-math (see oracle/Makefile).
 */
#include "q4_oracle.h"

#include <math.h>
#include <pthread.h>
#include <string.h>

static inline float f16le(const uint8_t *p) {
    return axo_f16_bits_to_f32((uint16_t)(p[0] | ((uint16_t)p[1] << 8)));
}

void axo_q5k_dequant(const uint8_t *q, float *w, size_t n_superblocks) {
    for (size_t sb = 0; sb < n_superblocks; ++sb) {
        const uint8_t *b = q + sb * AXO_Q5K_SB_BYTES;
        const float d = f16le(b), dmin = f16le(b + 2);
        const uint8_t *qh = b + 16, *qs = b + 48;
        float *o = w + sb * 256u;
        for (int j = 0; j < 4; ++j) {
            uint8_t sc0, m0, sc1, m1;
            axo_unpack_scale_min_k4(b + 4, 2 * j, &sc0, &m0);
            axo_unpack_scale_min_k4(b + 4, 2 * j + 1, &sc1, &m1);
            const float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
            const float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
            for (int l = 0; l < 32; ++l) {
                const int lo = (qs[32 * j + l] & 0x0F) + (((qh[l] >> (2 * j)) & 1) ? 16 : 0);
                const int hi = (qs[32 * j + l] >> 4) + (((qh[l] >> (2 * j + 1)) & 1) ? 16 : 0);
                o[64 * j + l] = d1 * (float)lo - mm1;
                o[64 * j + 32 + l] = d2 * (float)hi - mm2;
            }
        }
    }
}

void axo_q6k_dequant(const uint8_t *q, float *w, size_t n_superblocks) {
    for (size_t sb = 0; sb < n_superblocks; ++sb) {
        const uint8_t *b = q + sb * AXO_Q6K_SB_BYTES;
        const float d = f16le(b + 208);
        float *o = w + sb * 256u;
        for (int n = 0; n < 2; ++n) {
            const uint8_t *ql = b + 64 * n, *qh = b + 128 + 32 * n;
            const int8_t *sc = (const int8_t *)(b + 192 + 8 * n);
            for (int l = 0; l < 32; ++l) {
                const int is = l / 16;
                const int q1 = (int)((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = (int)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                o[128 * n + l] = d * (float)sc[is + 0] * (float)q1;
                o[128 * n + 32 + l] = d * (float)sc[is + 2] * (float)q2;
                o[128 * n + 64 + l] = d * (float)sc[is + 4] * (float)q3;
                o[128 * n + 96 + l] = d * (float)sc[is + 6] * (float)q4;
            }
        }
    }
}

static void dequant_one(int type, const uint8_t *blk, float *w) {
    if (type == AXO_GGML_Q5_K)
        axo_q5k_dequant(blk, w, 1);
    else
        axo_q6k_dequant(blk, w, 1);
}

static size_t type_bytes(int type) {
    return type == AXO_GGML_Q5_K ? AXO_Q5K_SB_BYTES : AXO_Q6K_SB_BYTES;
}

float axo_kq_dot(int type, const uint8_t *q, const float *x, size_t n_superblocks) {
    float w[256];
    float sum = 0.0f;
    for (size_t sb = 0; sb < n_superblocks; ++sb) {
        dequant_one(type, q + sb * type_bytes(type), w);
        for (int i = 0; i < 256; ++i) sum += w[i] * x[sb * 256u + (size_t)i];
    }
    return sum;
}

typedef struct {
    int type;
    const uint8_t *q;
    const float *x;
    float *y;
    size_t r0, r1, sbpr;
} kq_job;

static void *kq_worker(void *arg) {
    kq_job *j = (kq_job *)arg;
    const size_t rb = j->sbpr * type_bytes(j->type);
    for (size_t r = j->r0; r < j->r1; ++r) j->y[r] = axo_kq_dot(j->type, j->q + r * rb, j->x, j->sbpr);
    return NULL;
}

void axo_kq_matvec(int type, const uint8_t *q, const float *x, float *y, size_t n_rows,
                   size_t sb_per_row, int n_threads) {
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 256) n_threads = 256;
    if ((size_t)n_threads > n_rows) n_threads = n_rows ? (int)n_rows : 1;
    pthread_t th[256];
    kq_job jobs[256];
    int spawned[256];
    const size_t per = (n_rows + (size_t)n_threads - 1) / (size_t)n_threads;
    for (int t = 0; t < n_threads; ++t) {
        size_t r0 = (size_t)t * per, r1 = r0 + per;
        if (r0 > n_rows) r0 = n_rows;
        if (r1 > n_rows) r1 = n_rows;
        jobs[t] = (kq_job){type, q, x, y, r0, r1, sb_per_row};
        spawned[t] = t < n_threads - 1 && pthread_create(&th[t], NULL, kq_worker, &jobs[t]) == 0;
        if (!spawned[t]) kq_worker(&jobs[t]);
    }
    for (int t = 0; t < n_threads; ++t)
        if (spawned[t]) pthread_join(th[t], NULL);
}

void axo_kq_matvec_f64(int type, const uint8_t *q, const float *x, double *y, double *absdot,
                       size_t n_rows, size_t sb_per_row) {
    float w[256];
    const size_t rb = sb_per_row * type_bytes(type);
    for (size_t r = 0; r < n_rows; ++r) {
        double s = 0.0, a = 0.0;
        for (size_t sb = 0; sb < sb_per_row; ++sb) {
            dequant_one(type, q + r * rb + sb * type_bytes(type), w);
            for (int i = 0; i < 256; ++i) {
                const double p = (double)w[i] * (double)x[sb * 256u + (size_t)i];
                s += p;
                a += fabs(p);
            }
        }
        y[r] = s;
        if (absdot) absdot[r] = a;
    }
}

/* Benchmark-shape generators (SplitMix64).  Q5_K: d ~ f16(U(0.001, 0.05)),
 * dmin ~ f16(U(0, 0.02)), uniform random scale / qh / qs bytes (as the Q4_K
 * generator).  Q6_K: d ~ f16(U(1e-4, 2e-3)) and uniform random ql / qh /
 * int8 scale bytes (|d * sc * q| up to about 8, the Q4_K weights' range). */
static inline uint64_t sm64(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline float u24(uint64_t v) { return (float)(v >> 40) * (1.0f / 16777216.0f); }

static void fill_random(uint64_t *s, uint8_t *p, size_t n) {
    for (size_t k = 0; k < n; k += 8) {
        const uint64_t v = sm64(s);
        for (size_t t = 0; t < 8 && k + t < n; ++t) p[k + t] = (uint8_t)(v >> (8 * t));
    }
}

void axo_gen_q5k_weights(uint64_t seed, uint8_t *q, size_t n_superblocks) {
    uint64_t s = seed;
    for (size_t i = 0; i < n_superblocks; ++i) {
        uint8_t *b = q + i * AXO_Q5K_SB_BYTES;
        const uint16_t d16 = axo_f32_to_f16_bits(0.001f + 0.049f * u24(sm64(&s)));
        const uint16_t m16 = axo_f32_to_f16_bits(0.02f * u24(sm64(&s)));
        b[0] = (uint8_t)(d16 & 0xFF);
        b[1] = (uint8_t)(d16 >> 8);
        b[2] = (uint8_t)(m16 & 0xFF);
        b[3] = (uint8_t)(m16 >> 8);
        fill_random(&s, b + 4, AXO_Q5K_SB_BYTES - 4);
    }
}

void axo_gen_q6k_weights(uint64_t seed, uint8_t *q, size_t n_superblocks) {
    uint64_t s = seed;
    for (size_t i = 0; i < n_superblocks; ++i) {
        uint8_t *b = q + i * AXO_Q6K_SB_BYTES;
        fill_random(&s, b, 208);
        const uint16_t d16 = axo_f32_to_f16_bits(1e-4f + 1.9e-3f * u24(sm64(&s)));
        b[208] = (uint8_t)(d16 & 0xFF);
        b[209] = (uint8_t)(d16 >> 8);
    }
}
