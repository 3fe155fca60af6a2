/*
 * CPU oracle for the Q4_0 / Q4_K_M dequant-matvec path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP path: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product library (axiom-compute_amd/) never links or calls it.
 *
 * Every function restates the reference's Rust CPU code (rudybear/axiom-compute)
 * in C, in the same arithmetic order.  Build with -O2 -ffp-contract=off and no
 * fast-math so each f32 operation rounds exactly once, as Rust's does.
 */
#ifndef AXH_Q4_ORACLE_H
#define AXH_Q4_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AXO_Q4_0_BLOCK_BYTES 18u
#define AXO_Q4_0_BLOCK_ELEMS 32u
#define AXO_Q4K_SB_BYTES 144u
#define AXO_Q4K_SB_ELEMS 256u

/* IEEE binary16 -> binary32, exact (subnormals, inf, NaN payload kept).
 * Restates half::f16::from_bits(..).to_f32() (half 2.7.1) as used at
 * crates/axc-driver/benches/common.rs:230-233 and tests/common_helpers.rs:427-432. */
float axo_f16_bits_to_f32(uint16_t h);

/* binary32 -> binary16, round-to-nearest-even (half::f16::from_f32, used by the
 * generators at common.rs:177 and common_helpers.rs:491,497). */
uint16_t axo_f32_to_f16_bits(float f);

/* get_scale_min_k4: tests/common_helpers.rs:352-371. */
void axo_unpack_scale_min_k4(const uint8_t scales[12], int j, uint8_t *sc, uint8_t *m);

/* Single-output dot products (the reference's kernels produce y[0] only). */
/* q4_0_dequant_matvec_cpu: benches/common.rs:212-259.  Returns 0 status via *ok. */
float axo_q4_0_dot(const uint8_t *q, const float *x, size_t n_blocks);
/* q4km_dequant_matvec_cpu: tests/common_helpers.rs:411-461. */
float axo_q4k_dot(const uint8_t *q, const float *x, size_t n_superblocks);

/* Multi-row extension: row r is the reference dot applied to row r's
 * contiguous blocks with x shared (row-major, ggml layout). */
void axo_q4_0_matvec(const uint8_t *q, const float *x, float *y, size_t n_rows,
                     size_t blocks_per_row);
void axo_q4k_matvec(const uint8_t *q, const float *x, float *y, size_t n_rows,
                    size_t sb_per_row);
/* Same rows split over n_threads pthreads; per-row arithmetic unchanged, so
 * the output is bit-identical to the single-threaded call. */
void axo_q4k_matvec_mt(const uint8_t *q, const float *x, float *y, size_t n_rows,
                       size_t sb_per_row, int n_threads);
void axo_q4_0_matvec_mt(const uint8_t *q, const float *x, float *y, size_t n_rows,
                        size_t blocks_per_row, int n_threads);

/* Dequantisation to f32 in the reference's element order. */
/* Q4_0: value = (nibble - 8) * d; byte k -> elements k (lo) and k+16 (hi). */
void axo_q4_0_dequant(const uint8_t *q, float *w, size_t n_blocks);
/* Q4_K: w[64c+l] = d*sc0*lo - dmin*m0, w[64c+32+l] = d*sc1*hi - dmin*m1. */
void axo_q4k_dequant(const uint8_t *q, float *w, size_t n_superblocks);

/* f64 matvec with |w|.|x| row sums, for error analysis of both paths. */
void axo_q4k_matvec_f64(const uint8_t *q, const float *x, double *y, double *absdot,
                        size_t n_rows, size_t sb_per_row);
void axo_q4_0_matvec_f64(const uint8_t *q, const float *x, double *y, double *absdot,
                         size_t n_rows, size_t blocks_per_row);

/* Batched case: Y[r, b] = dot(row r, f32(X[:, b])) where X is f16, stored
 * column-major as B contiguous vectors of `cols` halves. Y is row-major
 * n_rows x batch. */
void axo_q4k_matmul_f16x(const uint8_t *q, const uint16_t *x_f16, float *y, size_t n_rows,
                         size_t sb_per_row, size_t batch, int n_threads);

/* generate_q4km_test_data: tests/common_helpers.rs:476-519 (Knuth MMIX LCG).
 * q must hold n*144 bytes and x n*256 floats. */
void axo_generate_q4km_test_data(uint32_t n_superblocks, uint64_t seed, uint8_t *q, float *x);

/* Synthetic inputs for the benchmark configurations (this build's own
 * generator; the reference has none at these shapes).  SplitMix64 stream:
 *   Q4_K superblock: d = f16(0.001 + 0.049u), dmin = f16(0.02u), 12 random scale
 *   bytes, 128 random qs bytes.  Q4_0 block: d = f16(0.001 + 0.049u), 16 random
 *   qs bytes.  u = (next() >> 40) * 2^-24 in [0, 1). */
void axo_gen_q4k_weights(uint64_t seed, uint8_t *q, size_t n_superblocks);
void axo_gen_q4_0_weights(uint64_t seed, uint8_t *q, size_t n_blocks);
/* x ~ N(0, sigma^2): Box-Muller on SplitMix64 uniforms, computed in double. */
void axo_gen_normal_f32(uint64_t seed, float *x, size_t n, double sigma);

/* ---- ggml k-quants next to Q4_K in real checkpoints (kq_oracle.c) ---------
 * No reference counterpart; restated from ggml's block layouts (see
 * kq_oracle.c).  type: AXO_GGML_Q5_K or AXO_GGML_Q6_K (GGUF type ids). */
#define AXO_GGML_Q5_K 13
#define AXO_GGML_Q6_K 14
#define AXO_Q5K_SB_BYTES 176u
#define AXO_Q6K_SB_BYTES 210u
void axo_q5k_dequant(const uint8_t *q, float *w, size_t n_superblocks);
void axo_q6k_dequant(const uint8_t *q, float *w, size_t n_superblocks);
/* Sequential f32 dot in element order (no FMA). */
float axo_kq_dot(int type, const uint8_t *q, const float *x, size_t n_superblocks);
void axo_kq_matvec(int type, const uint8_t *q, const float *x, float *y, size_t n_rows,
                   size_t sb_per_row, int n_threads);
void axo_kq_matvec_f64(int type, const uint8_t *q, const float *x, double *y, double *absdot,
                       size_t n_rows, size_t sb_per_row);
void axo_gen_q5k_weights(uint64_t seed, uint8_t *q, size_t n_superblocks);
void axo_gen_q6k_weights(uint64_t seed, uint8_t *q, size_t n_superblocks);

#ifdef __cplusplus
}
#endif
#endif
