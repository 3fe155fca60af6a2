/*
 * axh_check: host-side correctness verdicts for the tuning tools.
 *
 * Counterpart of the CPU references the reference's MCP bench_variant tool
 * consults (crates/axc-driver/src/mcp/tools/bench_variant.rs:53-78,373-420),
 * which has none for the Q4 kernels and reports them "not_checked".  Each
 * function compares a device result already copied to host memory with an f64
 * accumulation of the reference's dequantised weights
 * (crates/axc-driver/tests/common_helpers.rs:437-454; benches/common.rs:229-253)
 * and never produces results for callers.
 *
 * Criterion per output (n products, s = sum|w*x| / sqrt(n)):
 *   |y - ref| <= tol*|ref| when |ref| >= 0.1*s, else |y - ref| <= tol*s,
 * and ||y - ref||_2 <= tol*||ref||_2 over all outputs.  All pointers are host
 * pointers.
 */
#ifndef AXH_CHECK_H
#define AXH_CHECK_H

#include <stdint.h>

#include "axh.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct axh_check_report {
    uint32_t ok;                /* 1 when every output and the norm pass */
    uint64_t rows_checked;      /* outputs compared */
    uint64_t rows_failed;
    uint64_t worst_row;         /* output index with the largest err / allowed */
    double worst_over_allowed;  /* that ratio (<= 1 passes) */
    double norm_rel_err;        /* ||y - ref|| / ||ref|| */
} axh_check_report;

const char *axh_check_last_error(void);

/* Q4_K_M matvec: y[r] against rows of sb_per_row superblocks and x (256 f32 per SB). */
axh_status axh_check_q4k_matvec(const void *q, const float *x, const float *y, uint32_t n_rows,
                                uint32_t sb_per_row, double rel_tol, axh_check_report *out);
/* Q4_0 matvec: rows of blocks_per_row 18-byte blocks, x holds 32 f32 per block. */
axh_status axh_check_q4_0_matvec(const void *q, const float *x, const float *y, uint32_t n_rows,
                                 uint32_t blocks_per_row, double rel_tol,
                                 axh_check_report *out);
/* Batched matmul (axh_q4k_matmul_f16 layout): y[b*n_rows + r] with RN_f16 weights and
 * f16 activations x[b*K + k]. */
axh_status axh_check_q4k_matmul_f16(const void *q, const uint16_t *x, const float *y,
                                    uint32_t n_rows, uint32_t sb_per_row, uint32_t batch,
                                    double rel_tol, axh_check_report *out);

#ifdef __cplusplus
}
#endif

#endif /* AXH_CHECK_H */
