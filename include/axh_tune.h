/*
 * axh_tune: the @strategy-hole autotuner surface of rudybear/axiom-compute
 * (crates/axc-optimize) over plain C types.  Holes are named integer
 * candidate lists; a variant is one assignment; the caller's bench and
 * correctness callbacks receive the assignment values (the HIP counterpart of
 * the reference passing resolved SPIR-V to its BenchFn/CorrectnessFn).
 */
#ifndef AXH_TUNE_H
#define AXH_TUNE_H

#include <stddef.h>
#include <stdint.h>

#include "axh.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes beyond axh_status for the autotuner (EnumerateError and
 * GridSearchError, crates/axc-optimize/src/lib.rs:35-52). */
enum {
    AXH_ERR_EMPTY_STRATEGY = 40,          /* EnumerateError::EmptyStrategy        */
    AXH_ERR_UNKNOWN_HOLE = 41,            /* EnumerateError::UnknownHole          */
    AXH_ERR_NO_STRATEGY = 42,             /* GridSearchError::NoStrategy          */
    AXH_ERR_ENUMERATE_FAILED = 43,        /* GridSearchError::EnumerateFailed     */
    AXH_ERR_NO_SUCCESSFUL_VARIANTS = 44   /* GridSearchError::NoSuccessfulVariants */
};

/* CARTESIAN_WARN_THRESHOLD (crates/axc-optimize/src/enumerator.rs:42). */
#define AXH_CARTESIAN_WARN_THRESHOLD 100u

typedef struct axh_strategy_hole {
    const char *name;          /* UTF-8 hole name                */
    const int64_t *candidates; /* source order; [0] is the baseline */
    uint32_t n_candidates;
} axh_strategy_hole;

/* XXH3 64-bit hash, seed 0 (the variant_id hash, xxhash-rust xxh3_64). */
uint64_t axh_xxh3_64(const void *data, size_t len);

/* enumerate_strategy (enumerator.rs:68-129).  Holes are ordered by name
 * (byte-wise, as a BTreeMap); variants walk the mixed-radix product with the
 * last key varying fastest; variant_id = xxh3_64 over, per key in order,
 * u32le(len(name)) || name || i64le(value).
 *   sorted_hole_index_out[k] = caller index of the k-th key (n_holes entries)
 *   values_out[v * n_holes + k] = value of key k in variant v
 *   variant_ids_out[v]
 * With capacity 0 (or NULL outputs) only *n_variants_out is filled. */
axh_status axh_enumerate_strategy(const axh_strategy_hole *holes, uint32_t n_holes,
                                  uint64_t *n_variants_out, uint32_t *sorted_hole_index_out,
                                  int64_t *values_out, uint64_t *variant_ids_out,
                                  uint64_t capacity);

/* CorrectnessPolicy (grid_search.rs:55-66). */
enum { AXH_POLICY_NONE = 0, AXH_POLICY_BIT_EXACT = 1, AXH_POLICY_EQUIV_FP_TOL = 2 };
typedef struct axh_correctness_policy {
    uint32_t kind;
    uint32_t ulp; /* EquivFpTol */
} axh_correctness_policy;

/* SampleStats (grid_search.rs:80-90). */
typedef struct axh_sample_stats {
    uint64_t median_ns, min_ns, max_ns;
    uint32_t n_samples;
} axh_sample_stats;

/* BenchOutcome (grid_search.rs:93-101). */
enum { AXH_OUTCOME_OK = 0, AXH_OUTCOME_FAILED = 1, AXH_OUTCOME_CORRECTNESS_REJECTED = 2 };

/* Callbacks: return 0 on success; on failure write a message into err. */
typedef int (*axh_bench_fn)(void *user, uint64_t ordinal, const int64_t *values, uint32_t n_holes,
                            axh_sample_stats *out, char *err, size_t err_cap);
typedef int (*axh_correctness_fn)(void *user, uint64_t ordinal, const int64_t *values,
                                  uint32_t n_holes, char *err, size_t err_cap);

typedef struct axh_variant_result {
    uint64_t ordinal;
    uint64_t variant_id;
    uint32_t outcome;     /* AXH_OUTCOME_* */
    axh_sample_stats stats; /* valid when outcome == AXH_OUTCOME_OK */
    char message[120];    /* failure reason, if any */
} axh_variant_result;

typedef struct axh_grid_search_result {
    uint64_t winner_ordinal;
    uint64_t winner_variant_id;
    uint32_t fallback_used;
    uint32_t warned_large_product; /* product > AXH_CARTESIAN_WARN_THRESHOLD */
    uint64_t n_results;
} axh_grid_search_result;

/* grid_search (grid_search.rs:158-283): for every variant in ordinal order,
 * run correctness (if policy != NONE and a callback is given), then bench.
 * Winner = minimum median_ns among OK variants (ties: lowest ordinal).  If
 * none is OK, fall back to ordinal 0 (then 1, 2, 3) with fallback_used = 1.
 * results must hold the full product (see axh_enumerate_strategy). */
axh_status axh_grid_search(const axh_strategy_hole *holes, uint32_t n_holes,
                           const axh_correctness_policy *policy, axh_correctness_fn correctness,
                           axh_bench_fn bench, void *user, axh_variant_result *results,
                           uint64_t capacity, axh_grid_search_result *out);

/* ---- Tuned-winner table ---------------------------------------------------
 * The persistent artefact of a search, one hole assignment per (op, n_rows,
 * units): the counterpart of the reference's strategy sidecar
 * (crates/axc-driver/src/optimize.rs:103-128) and, as a file a context loads
 * at creation, of its pipeline cache (crates/axc-runtime/src/pipeline_cache.rs).
 * JSON, schema "axh-winners-1".  A missing file loads as an empty table; an
 * unreadable or malformed one is AXH_ERR_CODE_OBJECT_CACHE_LOAD
 * (PipelineCacheLoadFailed).  Saving is atomic (temporary file + rename).
 * A table is not thread-safe; a context guards its own. */
typedef struct axh_winner_table axh_winner_table;
axh_winner_table *axh_winners_new(void);
void axh_winners_free(axh_winner_table *t);
uint64_t axh_winners_count(const axh_winner_table *t);
axh_status axh_winners_load(const char *path, axh_winner_table **out);
axh_status axh_winners_save(const axh_winner_table *t, const char *path);
axh_status axh_winners_put(axh_winner_table *t, const char *op, uint32_t n_rows, uint32_t units,
                           const axh_q4_variant *v, uint64_t median_ns);
/* *found = 1 and the entry, or *found = 0. */
axh_status axh_winners_get(const axh_winner_table *t, const char *op, uint32_t n_rows,
                           uint32_t units, uint32_t *found, axh_q4_variant *v,
                           uint64_t *median_ns);

/* The context's table (owned by the context).  axh_context_create loads it
 * from <code_object_cache_dir>/axh_winners.json unless the option is NULL or
 * AXH_DISABLE_CODE_OBJECT_CACHE=1; a file that fails to load is reported on
 * stderr and the context starts with an empty table (as the reference treats
 * its pipeline cache, pipeline_cache.rs:45-100).  axh_q4k_matvec called with
 * no variant uses the table's "q4k_matvec" entry for its shape, if any. */
axh_status axh_context_winner_put(axh_context *ctx, const char *op, uint32_t n_rows,
                                  uint32_t units, const axh_q4_variant *v, uint64_t median_ns);
axh_status axh_context_winner_get(axh_context *ctx, const char *op, uint32_t n_rows,
                                  uint32_t units, uint32_t *found, axh_q4_variant *v,
                                  uint64_t *median_ns);
/* Writes the context's table to its file (no-op without one). */
axh_status axh_context_winners_save(axh_context *ctx);
/* Path of the context's table file, "" when it has none. */
const char *axh_context_winners_path(const axh_context *ctx);
/* The kernel axh_q4k_matvec launches on this context for the shape and
 * variant (a NULL variant consults the context's table). */
axh_status axh_context_q4k_matvec_kernel_name(axh_context *ctx, uint32_t n_rows,
                                              uint32_t sb_per_row, const axh_q4_variant *variant,
                                              char *buf, size_t cap);

/* ---- Q4_K matvec autotuner ---------------------------------------------------
 * Grid search over the whole Q4_K matvec kernel space on resident buffers,
 * one axh_grid_search per kernel family that takes the shape (family plus that
 * family's holes; every default is among the assignments).  Each variant runs
 * once and its output is judged by axh_check_q4k_matvec (f64 accumulation of
 * the reference's dequantised weights, relative tolerance `tol`, 1e-3 when 0)
 * on host copies of q and x, then it is timed over `samples` groups of 20
 * back-to-back calls with HIP events.  Timed calls rotate through device
 * copies of q totalling more than 512 MiB (up to 64 copies), so each call
 * reads its weights from HBM rather than the 256 MiB Infinity Cache.  The
 * fastest accepted variant is then timed again against the default in 9
 * interleaved rounds of 50 calls each; unless its median is more than 2 %
 * below the default's (the run-to-run spread), the default is kept.  The
 * result is stored in the context's table (and its file, if any). */
typedef struct axh_autotune_report {
    axh_q4_variant best;          /* winner (the default when kept_default) */
    uint64_t best_median_ns;      /* its median per call in the sweep */
    axh_q4_variant dflt;          /* the shape's default assignment */
    uint64_t default_median_ns;   /* its median in the same sweep */
    uint32_t variants;            /* assignments enumerated over all families */
    uint32_t accepted;            /* passed the checker and timed */
    uint32_t rejected;            /* failed the checker */
    uint32_t failed;              /* not compiled, not valid for the shape, or launch error */
    char best_kernel[64];         /* entry point of the winner */
    uint64_t confirm_best_ns;     /* the sweep's fastest, interleaved re-timing (median) */
    uint64_t confirm_default_ns;  /* the default in the same rounds */
    uint32_t kept_default;        /* 1: the result is the default (the sweep's fastest,
                                     or a variant that did not beat it by more than 2 %) */
    uint32_t weight_copies;       /* copies of q the timing rotated through */
} axh_autotune_report;
axh_status axh_q4k_matvec_autotune(axh_context *ctx, const void *q, const float *x, float *y,
                                   uint32_t n_rows, uint32_t sb_per_row, uint32_t samples,
                                   double tol, axh_autotune_report *out);

/* The hole space the autotuner searches for one kernel family at a shape (the
 * family hole first, with the family as its one candidate, then that family's
 * holes), for callers that run their own search over the same space, such as
 * the JSON-RPC tuning tools.  names[h] (static strings) and n_candidates[h]
 * for h < *n_holes; the candidates of all holes concatenated in `candidates`.
 * With names == NULL only *n_holes is set.  InvalidArgument when the family
 * has no kernel for the shape or an array is too small.  No counterpart in
 * the reference (its holes come from the kernel source's @strategy block,
 * crates/axc-hir/src/hir.rs:62-68). */
axh_status axh_q4k_matvec_family_holes(uint32_t family, uint32_t n_rows, uint32_t sb_per_row,
                                       const char **names, uint32_t *n_candidates,
                                       int64_t *candidates, uint32_t cap_holes,
                                       uint32_t cap_candidates, uint32_t *n_holes);

#ifdef __cplusplus
}
#endif
#endif /* AXH_TUNE_H */
