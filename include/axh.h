/*
 * axh: C ABI of the MI355X (gfx950) Q4_0 / Q4_K_M dequant-matvec path.
 *
 * Drop-in boundary for rudybear/axiom-compute's runtime surface
 * (crates/axc-runtime).  Plain pointers and sizes only; every call returns an
 * axh_status and leaves a thread-local message readable with axh_last_error().
 * Device pointers are HIP device addresses (from axh_buffer_alloc or any other
 * HIP allocation on the context's device).  `stream` arguments are hipStream_t
 * values passed as void*; NULL means the context's own stream.
 */
#ifndef AXH_H
#define AXH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Layout version of the structs below, raised whenever one of them changes
 * size or field order.  2: axh_q4_variant grew from 4 to 6 fields (16 to 24
 * bytes: family, sb_per_lane appended).  3: axh_autotune_report (axh_tune.h)
 * gained confirm_best_ns, confirm_default_ns, kept_default and
 * weight_copies at its end.  A binding written against an older
 * header compares axh_abi_version() with the AXH_ABI_VERSION it was written
 * for and refuses to run on a mismatch.  No counterpart in the reference
 * (its runtime is linked as one Rust crate graph). */
#define AXH_ABI_VERSION 3u
uint32_t axh_abi_version(void);

/* One code per DispatchError variant (crates/axc-runtime/src/error.rs:27-195),
 * in the reference's order, with the HIP failure each one stands for. */
typedef enum axh_status {
    AXH_OK = 0,
    AXH_ERR_RUNTIME_LOAD = 1,                 /* VulkanEntryFailed: HIP runtime unusable        */
    AXH_ERR_NO_INSTANCE = 2,                  /* NoVulkanInstance: hipInit failed               */
    AXH_ERR_NO_SUPPORTED_DEVICE = 3,          /* NoSupportedDevice: no gfx950 device at index   */
    AXH_ERR_NO_COMPUTE_QUEUE = 4,             /* NoComputeQueue: stream creation failed         */
    AXH_ERR_DEVICE_CREATION = 5,              /* DeviceCreationFailed: hipSetDevice failed      */
    AXH_ERR_MODULE_CREATION = 6,              /* ShaderModuleCreationFailed: hipModuleLoadData  */
    AXH_ERR_DESCRIPTOR_SET_LAYOUT = 7,        /* DescriptorSetLayoutFailed: bad binding plan    */
    AXH_ERR_DESCRIPTOR_POOL = 8,              /* DescriptorPoolFailed: kernarg assembly         */
    AXH_ERR_PIPELINE_LAYOUT = 9,              /* PipelineLayoutFailed: plan/pc size disagree    */
    AXH_ERR_PIPELINE_CREATION = 10,           /* PipelineCreationFailed: entry not in module    */
    AXH_ERR_BUFFER_ALLOCATION = 11,           /* BufferAllocationFailed: hipMalloc              */
    AXH_ERR_MEMORY_MAP = 12,                  /* MemoryMapFailed: pinned host allocation        */
    AXH_ERR_NO_COMPATIBLE_MEMORY_TYPE = 13,   /* NoCompatibleMemoryType                         */
    AXH_ERR_COMMAND_RECORD = 14,              /* CommandBufferRecordFailed: launch rejected     */
    AXH_ERR_QUEUE_SUBMIT = 15,                /* QueueSubmitFailed: stream/event error          */
    AXH_ERR_FENCE_TIMEOUT = 16,               /* FenceTimeout: completion wait timed out        */
    AXH_ERR_READBACK = 17,                    /* ReadbackFailed: device-to-host copy            */
    AXH_ERR_BINDING_COUNT_MISMATCH = 18,      /* BindingCountMismatch                           */
    AXH_ERR_PUSH_CONSTANT_SIZE_MISMATCH = 19, /* PushConstantSizeMismatch                       */
    AXH_ERR_WORKGROUP_COUNT_EXCEEDS_LIMIT = 20, /* WorkgroupCountExceedsDeviceLimit             */
    AXH_ERR_METADATA_IO = 21,                 /* MetadataIoError                                */
    AXH_ERR_METADATA_PARSE = 22,              /* MetadataParseError                             */
    AXH_ERR_METADATA_SCHEMA_MISMATCH = 23,    /* MetadataSchemaMismatch                         */
    AXH_ERR_CODE_OBJECT_CACHE_LOAD = 24,      /* PipelineCacheLoadFailed                        */
    AXH_ERR_STAGING_COPY = 25,                /* StagingCopyFailed: host-to-device copy         */
    AXH_ERR_INVALID_ARGUMENT = 100            /* no counterpart: null pointer or bad shape      */
} axh_status;

typedef struct axh_context axh_context;
typedef struct axh_kernel axh_kernel;

/* Thread-local description of the last failure on this thread ("" if none). */
const char *axh_last_error(void);
const char *axh_status_name(int status);

/* ---- context ---------------------------------------------------------------
 * Replaces VulkanContextOptions / VulkanContext::new_with_options
 * (crates/axc-runtime/src/context.rs:76-109,175). */
typedef struct axh_context_options {
    /* pipeline_cache_path: directory of the tuned-winner table
     * (axh_winners.json, see axh_tune.h), loaded at creation and consulted by
     * calls that pass no variant; NULL, or AXH_DISABLE_CODE_OBJECT_CACHE=1
     * (as AXC_DISABLE_PIPELINE_CACHE, pipeline_cache.rs:153-170), = none.
     * Kernels are embedded code objects, so nothing else is cached. */
    const char *code_object_cache_dir;
    int32_t device_index;              /* physical_device_index; -1 = AXH_DEVICE_INDEX env or 0 */
    uint64_t fence_timeout_ms;         /* 0 = AXH_FENCE_TIMEOUT_MS env or 10000 (dispatch.rs:26) */
} axh_context_options;

axh_status axh_context_create(const axh_context_options *opts, axh_context **out);
/* Handles prepared on the context stay valid after this call
 * (crates/axc-runtime/tests/kernel_handle_outlives_context.rs:24): the device
 * state is released with the last handle. */
void axh_context_destroy(axh_context *ctx);
const char *axh_context_device_name(const axh_context *ctx);
void *axh_context_stream(const axh_context *ctx);
/* Device limit checked before any dispatch (dispatch.rs:85-93). */
void axh_context_max_workgroup_count(const axh_context *ctx, uint32_t out[3]);

/* ---- kernels ---------------------------------------------------------------
 * Binding plan: ParamBindingPlan (crates/axc-hir/src/param.rs:119-126) plus
 * the launch facts a HIP code object needs (KernelMetadata workgroup size,
 * crates/axc-runtime/src/metadata.rs:45-68).  Kernel arguments are one
 * pointer per buffer in binding order followed by one push-constant struct
 * of push_constant_total_bytes passed by value. */
enum { AXH_ACCESS_READ_ONLY = 0, AXH_ACCESS_WRITE_ONLY = 1, AXH_ACCESS_READ_WRITE = 2 };

typedef struct axh_binding_plan {
    uint32_t n_buffers;
    const uint8_t *access;             /* n_buffers AXH_ACCESS_* values */
    uint32_t push_constant_total_bytes;
    uint32_t workgroup_size[3];        /* @workgroup(x, y, z) */
    uint32_t dynamic_lds_bytes;        /* 0 for kernels whose LDS is static */
} axh_binding_plan;

/* prepare_kernel (context.rs:392-486): code object (HSACO/ELF or offload
 * bundle for gfx950) + plan + entry -> handle.  Handles are cached per
 * context by (code-object hash, plan, push-constant size, entry); a second
 * prepare of the same key returns the cached handle with one more reference. */
axh_status axh_prepare_kernel(axh_context *ctx, const void *code_object, size_t code_object_bytes,
                              const axh_binding_plan *plan, uint32_t push_constant_bytes,
                              const char *entry, axh_kernel **out);
void axh_kernel_retain(axh_kernel *k);
void axh_kernel_release(axh_kernel *k);
uint64_t axh_kernel_cache_key(const axh_kernel *k);
/* Bytes currently held by the handle's buffer pool for binding i (0 if none). */
uint64_t axh_kernel_pool_bytes(const axh_kernel *k, uint32_t binding);

/* dispatch_handle (context.rs:498-547): uploads each non-empty input into its
 * binding's pooled device buffer (pool size round_up_pow2(max(in, out, 4)),
 * grown only upward: kernel_handle.rs:295-393), launches workgroups, waits
 * with the fence timeout and copies output_sizes[i] bytes of every binding
 * into outputs[i] (skipped when output_sizes[i] == 0).  Validation happens
 * before any device work (dispatch.rs:56-95).  Dispatches on one handle are
 * serialised; different handles may dispatch concurrently. */
axh_status axh_dispatch_handle(axh_context *ctx, axh_kernel *k, const uint32_t workgroups[3],
                               const void *const *inputs, const size_t *input_sizes,
                               size_t n_inputs, const size_t *output_sizes, size_t n_outputs,
                               void *const *outputs, const void *push_constants,
                               size_t push_constant_bytes);

/* Legacy one-shot dispatch (DispatchRequest, dispatch.rs:33-50,109-132):
 * validate, prepare, dispatch_handle, release. */
axh_status axh_dispatch(axh_context *ctx, const void *code_object, size_t code_object_bytes,
                        const axh_binding_plan *plan, const uint32_t workgroups[3],
                        const void *const *inputs, const size_t *input_sizes, size_t n_inputs,
                        const size_t *output_sizes, size_t n_outputs, void *const *outputs,
                        const void *push_constants, size_t push_constant_bytes, const char *entry);

/* Pure request validation (dispatch.rs:56-95), usable without a device. */
axh_status axh_validate_request(const axh_binding_plan *plan, const uint32_t workgroups[3],
                                size_t n_inputs, size_t n_outputs, size_t push_constant_bytes,
                                const uint32_t max_workgroup_count[3]);

/* ---- resident buffers and asynchronous launch ------------------------------
 * The hot path: buffers stay in HBM between calls; launches are asynchronous
 * on `stream`.  Uploads/downloads go through the context's pinned staging
 * buffer with hipMemcpyAsync and return when the copy is complete. */
axh_status axh_buffer_alloc(axh_context *ctx, size_t bytes, void **device_ptr);
axh_status axh_buffer_free(axh_context *ctx, void *device_ptr);
axh_status axh_upload(axh_context *ctx, void *device_dst, const void *host_src, size_t bytes);
axh_status axh_download(axh_context *ctx, void *host_dst, const void *device_src, size_t bytes);
/* Device-to-device copy on the context stream; returns when complete. */
axh_status axh_copy_device(axh_context *ctx, void *device_dst, const void *device_src, size_t bytes);
axh_status axh_launch(axh_context *ctx, axh_kernel *k, const uint32_t workgroups[3],
                      void *const *device_buffers, size_t n_buffers, const void *push_constants,
                      size_t push_constant_bytes, void *stream);
/* Waits for `stream` with the context's fence timeout (AXH_ERR_FENCE_TIMEOUT). */
axh_status axh_synchronize(axh_context *ctx, void *stream);
/* Waits for all work on the context's device, without a timeout. */
axh_status axh_device_synchronize(axh_context *ctx);

/* ---- timing ----------------------------------------------------------------
 * HIP events on the context's runtime, for timing launches on a stream
 * (the reference times dispatches on the host only; GPU timestamps are the
 * measurement this build reports). */
typedef struct axh_event axh_event;
axh_status axh_event_create(axh_context *ctx, axh_event **out);
axh_status axh_event_record(axh_context *ctx, axh_event *ev, void *stream);
axh_status axh_event_synchronize(axh_context *ctx, axh_event *ev);
axh_status axh_event_elapsed_ms(axh_event *start, axh_event *end, float *ms);
void axh_event_destroy(axh_event *ev);

/* ---- Q4 dequant-matvec operations ------------------------------------------
 * Strategy holes of the matvec kernels (the reference's @strategy surface,
 * crates/axc-hir/src/hir.rs:62-68).  `family` picks the Q4_K kernel family
 * (AXH_Q4K_FAMILY_*); the other holes are that family's:
 *   persistent: rows_per_wave, waves_per_workgroup, prefetch (superblock
 *     iterations loaded ahead: 1 issues the next iteration's loads before the
 *     current one is computed and stages x chunk by chunk; P >= 2 keeps P
 *     iterations loaded and refills a slot after computing it) and nontemporal
 *     (weight-load cache policy);
 *   one pass (x staged chunk by chunk, or whole): sb_per_lane, the superblocks
 *     a lane walks per row (the kernel's trip count, eight superblocks per
 *     half-wave per step: from ceil(sb_per_row / 8) to 16); chunk by chunk
 *     also prefetch, the x chunks requested ahead of their staging (1, or 2
 *     from three steps: axh_q4k_matvec_onep_i*; the default is 2 from four
 *     steps up to 4096 rows);
 *   one workgroup: rows_per_wave = rows per workgroup (1, 2 or 4, at least
 *     n_rows);
 *   tiled: rows_per_wave, waves_per_workgroup, prefetch.
 * Zero fields take the shape's choice.  family = 0 selects the persistent
 * family when any of its four holes is set, else the default family for the
 * shape: one workgroup for 1-4 long rows, split-K for fewer than 32 rows of
 * 129-256 superblocks, tiled for fewer than 32 rows otherwise and for 32-512
 * rows of 13-128 superblocks and 513-1024 rows of 17-128, one pass for
 * 32-32768 rows of 1-128 superblocks otherwise (and up to
 * 65536 rows of at most 16; x staged whole from 6144 rows of at most 32
 * superblocks and from 4097 rows of at most 24), except 4097-6143 and
 * 24576-32768 rows of 25-32 superblocks and 4097-8191 rows of 74 or more,
 * which take the persistent family; persistent beyond,
 * tiled for rows of more than 128 superblocks.  Every default is a hole
 * assignment.  The gate/up operations
 * take the persistent holes, or their one-pass families (see axh_q4k_gate_up).
 * Q4_0 takes family PERSISTENT (axh_q4_0_matvec_flat_r*_w*_p*_x*: the Q4_K
 * persistent kernel over octets of 8 blocks; holes rows_per_wave,
 * waves_per_workgroup, prefetch), ONE_PASS / ONE_PASS_X
 * (axh_q4_0_matvec_one{,p,x}_i{sb_per_lane}, sb_per_lane the octets a lane
 * walks per row, each step covering 64 blocks: ceil(blocks / 64) to 16;
 * prefetch as for Q4_K), COLUMNS (axh_q4_0_matvec_cols_r1, rows
 * of 2-128 blocks) and TILED (axh_q4_0_matvec_r*_w*: rows_per_wave,
 * waves_per_workgroup; also what family 0 with a hole set selects).  The
 * octet families take rows of an even block count up to 1024 blocks, below
 * 4 GiB.  With no hole set: tiled for fewer than 32 rows, for 32-1024 rows of
 * up to 128 blocks and 32-256 rows of 193-256 blocks,
 * odd block counts and rows of more than 1024 blocks, persistent
 * for more than 16384 rows of more than 256 blocks, else one pass (x whole
 * for rows of 65-128 blocks from 6144 rows, x two chunks ahead for 14-16 steps
 * from 4096 rows).
 * Q5_K and Q6_K take the persistent holes or family =
 * AXH_Q4K_FAMILY_ONE_PASS with sb_per_lane 1-8 (rows of up to 64
 * superblocks) and prefetch (x one or two chunks ahead, two from three
 * steps); with no hole set they run one pass for rows of up to 16
 * superblocks over 768-32768 rows (Q5_K) or 256-4096 rows (Q6_K), and for
 * 2049-4096 rows of up to 64 superblocks (Q5_K) or 2049-8192 rows of up to 40
 * (Q6_K), else the persistent family (4 waves with x staged whole for up to
 * 2048 rows of 17-64 superblocks and for 14336 rows and more of 33-64). */
enum {
    AXH_Q4K_FAMILY_DEFAULT = 0,
    AXH_Q4K_FAMILY_PERSISTENT = 1, /* axh_q4k_matvec_flat_r*_w*_p*_n*[_x2]            */
    AXH_Q4K_FAMILY_ONE_PASS = 2,   /* axh_q4k_matvec_one[p]_i{sb_per_lane}           */
    AXH_Q4K_FAMILY_ONE_PASS_X = 3, /* axh_q4k_matvec_onex_i{sb_per_lane}: x whole    */
    AXH_Q4K_FAMILY_WORKGROUP = 4,  /* axh_q4k_matvec_wg_w8_x2_r{1,2,4}: 1-4 rows     */
    AXH_Q4K_FAMILY_SPLIT_K = 5,    /* axh_q4k_matvec_sk_s16: <= 32 rows, <= 256 SB   */
    AXH_Q4K_FAMILY_COLUMNS = 6,    /* axh_q4k_matvec_cols_r4_w*: rows of <= 128 SB   */
    AXH_Q4K_FAMILY_TILED = 7       /* axh_q4k_matvec_tiled_r*_w*_p*: any row length  */
};
typedef struct axh_q4_variant {
    uint32_t rows_per_wave;
    uint32_t waves_per_workgroup;
    uint32_t prefetch;
    uint32_t nontemporal; /* 1: weight loads bypass cache allocation; 2: force normal loads */
    uint32_t family;      /* AXH_Q4K_FAMILY_* */
    uint32_t sb_per_lane; /* one-pass families: superblocks a lane walks per row */
} axh_q4_variant;

/* y[r] = dot(row r of Q4_K_M matrix q, x) for r < n_rows, where each row is
 * sb_per_row contiguous 144-byte superblocks and x holds sb_per_row*256 f32.
 * Replaces prepare_kernel + dispatch_handle of examples/q4km_dequant_matvec.axc
 * (its single output is the n_rows = 1 case), compared against
 * q4km_dequant_matvec_cpu (crates/axc-driver/tests/common_helpers.rs:411-461). */
axh_status axh_q4k_matvec(axh_context *ctx, const void *q, const float *x, float *y,
                          uint32_t n_rows, uint32_t sb_per_row, const axh_q4_variant *variant,
                          void *stream);
/* Allocation-free variant of axh_q4k_matvec.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory during a
 * call (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Computes the same y for 1-32 rows of 1-256 superblocks
 * with the split-K kernel, whose workgroup counter and partial sums live in
 * a fixed 2304-byte per-device scratch array that axh_context_create sets up;
 * a call allocates nothing and calls no allocating routine.  Larger shapes
 * (and sb_per_row = 0) return AXH_ERR_INVALID_ARGUMENT.  Every call on a
 * device shares that device's scratch, which keeps the last call's partial
 * sums (the counter is back at zero after each call): calls that overlap on
 * one GPU (two streams, two host threads, two contexts) race, so order them.
 * q and x 16-byte aligned. */
axh_status axh_q4k_matvec_noalloc(axh_context *ctx, const void *q, const float *x, float *y,
                                  uint32_t n_rows, uint32_t sb_per_row, void *stream);
/* The hole assignment (family and that family's holes, no zero left to the
 * shape) that axh_q4k_matvec uses for this shape when given no variant:
 * passing it as the variant launches the same kernel.  No device work. */
axh_status axh_q4k_matvec_default_variant(uint32_t n_rows, uint32_t sb_per_row,
                                         axh_q4_variant *out);
/* Name of the kernel axh_q4k_matvec launches for this shape and variant (the
 * entry point profilers report), NUL-terminated into buf[cap].  No device
 * work.  Counterpart of the kernel name the reference's BenchFn receives in
 * place of SPIR-V (crates/axc-optimize/src/grid_search.rs:139-146). */
axh_status axh_q4k_matvec_kernel_name(uint32_t n_rows, uint32_t sb_per_row,
                                      const axh_q4_variant *variant, char *buf, size_t cap);
/* Q4_0 counterpart: rows of blocks_per_row 18-byte blocks; x holds
 * blocks_per_row*32 f32.  Replaces examples/q4_0_dequant_matvec.axc; compared
 * against q4_0_dequant_matvec_cpu (crates/axc-driver/benches/common.rs:212-259). */
axh_status axh_q4_0_matvec(axh_context *ctx, const void *q, const float *x, float *y,
                           uint32_t n_rows, uint32_t blocks_per_row,
                           const axh_q4_variant *variant, void *stream);
axh_status axh_q4_0_matvec_kernel_name(uint32_t n_rows, uint32_t blocks_per_row,
                                       const axh_q4_variant *variant, char *buf, size_t cap);
/* ---- ggml k-quants next to Q4_K, and matvec by ggml type ---------------------
 * ggml tensor type ids as stored in GGUF files (ggml.h enum ggml_type). */
enum {
    AXH_GGML_F32 = 0, AXH_GGML_F16 = 1, AXH_GGML_Q4_0 = 2, AXH_GGML_Q4_1 = 3,
    AXH_GGML_Q5_0 = 6, AXH_GGML_Q5_1 = 7, AXH_GGML_Q8_0 = 8, AXH_GGML_Q8_1 = 9,
    AXH_GGML_Q2_K = 10, AXH_GGML_Q3_K = 11, AXH_GGML_Q4_K = 12, AXH_GGML_Q5_K = 13,
    AXH_GGML_Q6_K = 14, AXH_GGML_Q8_K = 15, AXH_GGML_I8 = 24, AXH_GGML_I16 = 25,
    AXH_GGML_I32 = 26, AXH_GGML_I64 = 27, AXH_GGML_F64 = 28, AXH_GGML_BF16 = 30
};
/* Elements and bytes per block of a ggml type (error for unsized types). */
axh_status axh_ggml_type_size(uint32_t type, uint32_t *block_elems, uint32_t *block_bytes);
/* y = W x for the ggml k-quants that real Q4_K_M / Q5_K_M checkpoints mix in:
 * Q5_K (176-byte superblocks: d, dmin, the Q4_K scale field, qh[32], qs[128])
 * and Q6_K (210-byte superblocks: ql[128], qh[64], int8 scales[16], d).  No
 * counterpart in the reference (it has no loader for real checkpoints,
 * ROADMAP.md:230-234); checked against a sequential-f32 CPU restatement of
 * ggml's dequantisation with the matvec tolerance.  Limits: 1 <= sb_per_row
 * <= 128 (the row's x is staged in LDS), matrix below 4 GiB, q and x 16-byte
 * aligned.  Variant holes as for Q4_K (nontemporal 0 or 2). */
axh_status axh_q5k_matvec(axh_context *ctx, const void *q, const float *x, float *y,
                          uint32_t n_rows, uint32_t sb_per_row, const axh_q4_variant *variant,
                          void *stream);
axh_status axh_q6k_matvec(axh_context *ctx, const void *q, const float *x, float *y,
                          uint32_t n_rows, uint32_t sb_per_row, const axh_q4_variant *variant,
                          void *stream);
axh_status axh_q5k_matvec_kernel_name(uint32_t n_rows, uint32_t sb_per_row,
                                      const axh_q4_variant *variant, char *buf, size_t cap);
axh_status axh_q6k_matvec_kernel_name(uint32_t n_rows, uint32_t sb_per_row,
                                      const axh_q4_variant *variant, char *buf, size_t cap);
uint32_t axh_q5k_matvec_variant_count(void);
axh_status axh_q5k_matvec_variant_at(uint32_t i, axh_q4_variant *out);
uint32_t axh_q6k_matvec_variant_count(void);
axh_status axh_q6k_matvec_variant_at(uint32_t i, axh_q4_variant *out);
/* Matvec of a row-major ggml tensor of n_rows rows of n_cols elements
 * (GGUF ne[0] = n_cols), dispatched on its type: Q4_0, Q4_K, Q5_K or Q6_K,
 * each with its default variant. */
axh_status axh_matvec_ggml(axh_context *ctx, uint32_t ggml_type, const void *q, const float *x,
                           float *y, uint32_t n_rows, uint64_t n_cols, void *stream);

/* Fused SwiGLU gate/up projection of a decode step, one pass over x:
 *   h[r] = silu(g_r) * u_r,  g_r = dot(q_gate row r, x),  u_r = dot(q_up row r, x),
 *   silu(g) = g / (1 + exp(-g)),
 * for two Q4_K_M matrices of the same shape (n_rows rows of sb_per_row
 * superblocks).  No counterpart in the reference, whose kernels stop at one
 * matvec per dispatch (multi-row work is roadmap, ROADMAP.md:54-72); it
 * equals two axh_q4k_matvec calls followed by silu(g) * u, with each dot
 * product held to the matvec's tolerance.  Limits: 1 <= sb_per_row <= 128,
 * each matrix below 4 GiB, q_gate / q_up / x 16-byte aligned.  Variant holes
 * (the persistent kernel): rows_per_wave = output rows per lane group (each
 * reads that many gate and up rows), waves_per_workgroup, prefetch;
 * nontemporal 0 or 2.  Or family = AXH_Q4K_FAMILY_ONE_PASS / _ONE_PASS_X
 * (x chunk by chunk / whole) with sb_per_lane 1-8 (rows of up to 64
 * superblocks): the wave-paired one-pass kernels, one workgroup per 8 output
 * rows, the even wave of a pair on gate rows and the odd wave on up rows.
 * With no hole set, up to 12288 rows of up to 64 superblocks take the
 * one-pass kernel (x whole from 2049 rows), larger matrices the persistent
 * one. */
axh_status axh_q4k_gate_up(axh_context *ctx, const void *q_gate, const void *q_up,
                           const float *x, float *h, uint32_t n_rows, uint32_t sb_per_row,
                           const axh_q4_variant *variant, void *stream);
axh_status axh_q4k_gate_up_kernel_name(uint32_t n_rows, uint32_t sb_per_row,
                                       const axh_q4_variant *variant, char *buf, size_t cap);
uint32_t axh_q4k_gate_up_variant_count(void);
axh_status axh_q4k_gate_up_variant_at(uint32_t i, axh_q4_variant *out);
/* The same fusion over two Q4_0 matrices (n_rows rows of blocks_per_row
 * 18-byte blocks each; x holds blocks_per_row * 32 f32): equals two
 * axh_q4_0_matvec calls followed by silu(g) * u.  No counterpart in the
 * reference (see axh_q4k_gate_up).  Limits: blocks_per_row even, 2-1024;
 * each matrix below 4 GiB; q_gate / q_up 4-byte and x 16-byte aligned.
 * Variant holes and defaults as for axh_q4k_gate_up (the kernels over octets of
 * 8 blocks; one-pass rows of up to 512 blocks). */
axh_status axh_q4_0_gate_up(axh_context *ctx, const void *q_gate, const void *q_up,
                            const float *x, float *h, uint32_t n_rows, uint32_t blocks_per_row,
                            const axh_q4_variant *variant, void *stream);
axh_status axh_q4_0_gate_up_kernel_name(uint32_t n_rows, uint32_t blocks_per_row,
                                        const axh_q4_variant *variant, char *buf, size_t cap);
/* The same fusion over two Q5_K matrices (n_rows rows of sb_per_row 176-byte
 * superblocks; x holds sb_per_row * 256 f32): equals two axh_q5k_matvec calls
 * followed by silu(g) * u.  No counterpart in the reference.  Limits: 1 <=
 * sb_per_row <= 128, each matrix below 4 GiB, q_gate / q_up / x 16-byte
 * aligned.  Holes as for axh_q4k_gate_up; with none set, the wave-paired
 * one-pass kernel (x chunk by chunk) up to 12288 rows of up to 64
 * superblocks, else the persistent kernel. */
axh_status axh_q5k_gate_up(axh_context *ctx, const void *q_gate, const void *q_up,
                           const float *x, float *h, uint32_t n_rows, uint32_t sb_per_row,
                           const axh_q4_variant *variant, void *stream);
axh_status axh_q5k_gate_up_kernel_name(uint32_t n_rows, uint32_t sb_per_row,
                                       const axh_q4_variant *variant, char *buf, size_t cap);
/* Decode-only kernels, bit-exact with the reference's CPU dequantisation
 * (common_helpers.rs:437-454; common.rs:229-253): w receives 256 (Q4_K) or
 * 32 (Q4_0) f32 per unit in the reference's element order. */
axh_status axh_q4k_dequant(axh_context *ctx, const void *q, float *w, uint64_t n_superblocks,
                           void *stream);
axh_status axh_q4_0_dequant(axh_context *ctx, const void *q, float *w, uint64_t n_blocks,
                            void *stream);
/* Q5_K / Q6_K decode (256 f32 per superblock in ggml's element order),
 * bit-exact with the CPU restatement: Q5_K rounds once (the subtraction),
 * Q6_K weights are exact products.  Q5_K: q and w 16-byte aligned; Q6_K:
 * q 2-byte and w 4-byte aligned. */
axh_status axh_q5k_dequant(axh_context *ctx, const void *q, float *w, uint64_t n_superblocks,
                           void *stream);
axh_status axh_q6k_dequant(axh_context *ctx, const void *q, float *w, uint64_t n_superblocks,
                           void *stream);
/* IEEE binary16 -> binary32 widening of n raw patterns (the ptr_read_u16_zext +
 * f16_bits_to_f32 builtins, crates/axc-codegen/src/q4_0.rs:86-171). */
axh_status axh_f16_widen(axh_context *ctx, const uint16_t *h, float *f, uint64_t n, void *stream);

/* Measurement helpers (no counterpart in the reference): the floor that one
 * kernel launch per call puts under a matvec on this device.  Both use the
 * matvec's launch shape, one 512-thread workgroup per compute unit.
 * axh_read_floor streams `bytes` (a multiple of 16, below 4 GiB) from q with
 * 16-byte loads and writes, per wave, the XOR of every dword it read to
 * out[wave]; axh_launch_empty does nothing.  out holds out_words >= 8 *
 * axh_cu_count(ctx) words. */
axh_status axh_read_floor(axh_context *ctx, const void *q, uint64_t bytes, uint32_t *out,
                          uint32_t out_words, void *stream);
axh_status axh_launch_empty(axh_context *ctx, uint32_t *out, uint32_t out_words, void *stream);
/* The same read at another launch shape: `grid` workgroups of `threads`
 * (256, 512 or 1024) lanes with `loads` (2, 4 or 8) 16-byte loads in flight
 * per lane, walking the buffer grid-stride; out holds one word per wave.
 * For the sweep that finds the best single-launch read of a buffer. */
axh_status axh_read_floor_shape(axh_context *ctx, const void *q, uint64_t bytes, uint32_t threads,
                                uint32_t loads, uint32_t grid, uint32_t *out, uint32_t out_words,
                                void *stream);
uint32_t axh_cu_count(axh_context *ctx);
/* binary32 -> binary16, round to nearest even, of n values (NaN stays NaN,
 * values beyond the f16 range become infinities): the activation cast that
 * feeds the f16 matmul.  No counterpart in the reference.  x and h 16-byte
 * aligned; n < 2^32 - 16. */
axh_status axh_f32_to_f16(axh_context *ctx, const float *x, uint16_t *h, uint64_t n, void *stream);

/* ---- graph capture -----------------------------------------------------------
 * Records the launches issued on the context stream between begin and end
 * (axh_q4k_matvec, axh_q4_0_matvec, axh_q4k_gate_up, axh_q4k_matmul_f16/_f32,
 * axh_launch with a NULL stream) into a graph that replays them in order with no host work per
 * kernel: the HIP counterpart of recording a Vulkan command buffer once and
 * resubmitting it.  Launch each operation once before capturing it (its
 * kernel is then prepared and cached).  No event, copy or synchronisation
 * call may be made on the context stream while capturing.  A graph that holds
 * a split-K matvec (by default fewer than 32 rows of 129-256 superblocks) uses the
 * context stream's workspace and replays only on the context stream: another
 * stream gets AXH_ERR_INVALID_ARGUMENT. */
typedef struct axh_graph axh_graph;
axh_status axh_capture_begin(axh_context *ctx);
axh_status axh_capture_end(axh_context *ctx, axh_graph **out);
axh_status axh_graph_launch(axh_context *ctx, axh_graph *g, void *stream);
uint64_t axh_graph_node_count(const axh_graph *g);
void axh_graph_destroy(axh_graph *g);

/* Number of compiled matvec variants and the i-th one (for the autotuner). */
uint32_t axh_q4k_matvec_variant_count(void);
axh_status axh_q4k_matvec_variant_at(uint32_t i, axh_q4_variant *out);
uint32_t axh_q4_0_matvec_variant_count(void);
axh_status axh_q4_0_matvec_variant_at(uint32_t i, axh_q4_variant *out);

/* Batched Q4_K_M matmul on MFMA (f16 in, f32 accumulate):
 *   y[b * n_rows + r] = sum_k RN_f16(w32[r][k]) * x[b * K + k],  K = 256 * sb_per_row,
 * for b < batch, where w32 is the reference's f32 dequantisation
 * (crates/axc-driver/tests/common_helpers.rs:437-454) and x holds `batch`
 * contiguous f16 activation vectors.  Y is batch x n_rows f32.  The reference
 * has no batched kernel (its matvec, examples/q4km_dequant_matvec.axc, is the
 * batch = 1 case with f32 weights); multi-row matmul is roadmap there
 * (ROADMAP.md:54-72).  q and x 16-byte aligned, each below 4 GiB. */
typedef struct axh_q4_matmul_variant {
    uint32_t kind;                /* 3 K-split, 5 K-split tile, 7 streaming rows
                                     (K <= 4096), 8 32x32 tiles (128 columns per
                                     workgroup), 9 long rows (K < 262144, X in
                                     chunks through LDS); 0 = default, chosen by the grid
                                     each kind launches on 256 CUs.  Kinds 1, 2, 4
                                     and 6 were removed (no shape where they won) */
    uint32_t waves_per_workgroup; /* 3, 5, 7, 9: waves splitting K; 8: waves of row_tiles
                                     row tiles each */
    uint32_t col_tiles;           /* 16-column MFMA tiles per workgroup (kind 8: 8;
                                     kind 9: 4-column groups, 1, 2 or 4) */
    uint32_t prefetch;            /* K steps in flight (kinds 3, 7; kind 7 prefetch 2:
                                     8-column groups), LDS ring depth (5, 8: 4), X
                                     chunks in flight (9) */
    uint32_t row_tiles;           /* kind 3: 16-row MFMA tiles (0: 2); kind 5: 16-row
                                     MFMA tiles per wave (0: 4); kind 8: 32-row tiles
                                     per wave (0: 1); kind 9: 16-row tiles per
                                     workgroup (0: 1); 0 otherwise */
} axh_q4_matmul_variant;
axh_status axh_q4k_matmul_f16(axh_context *ctx, const void *q, const uint16_t *x, float *y,
                              uint32_t n_rows, uint32_t sb_per_row, uint32_t batch,
                              const axh_q4_matmul_variant *variant, void *stream);
/* The same product for f32 activations: x (batch x K f32) is first rounded
 * to f16 (RN, ties to even) into the caller's buffer x16 (batch x K f16) by
 * axh_f32_to_f16, then axh_q4k_matmul_f16 runs on x16; both launches go to
 * `stream` in that order.  A separate cast pass is cheaper than converting
 * inside the matmul's loads, because every row tile re-reads X.  x and x16
 * 16-byte aligned.  No counterpart in the reference (see axh_q4k_matmul_f16). */
axh_status axh_q4k_matmul_f32(axh_context *ctx, const void *q, const float *x, uint16_t *x16,
                              float *y, uint32_t n_rows, uint32_t sb_per_row, uint32_t batch,
                              const axh_q4_matmul_variant *variant, void *stream);
axh_status axh_q4k_matmul_kernel_name(uint32_t n_rows, uint32_t sb_per_row, uint32_t batch,
                                      const axh_q4_matmul_variant *variant, char *buf,
                                      size_t cap);
uint32_t axh_q4k_matmul_variant_count(void);
axh_status axh_q4k_matmul_variant_at(uint32_t i, axh_q4_matmul_variant *out);

/* ---- measurement loop ------------------------------------------------------
 * `groups` x `calls_per_group` back-to-back calls of one operation, launched
 * by this library's own loop on the context stream through the public entry
 * points above (each call a full dispatch: validation, kernel choice, one
 * kernel launch), after `warmup` untimed calls.  Call i reads the weights at
 * q + (i % n_copies) * q_stride.  The device is synchronised before the
 * warmup calls, not after them: they prime the queue, so the first timed call
 * starts behind queued work like every later one.  A HIP event is recorded
 * before the first timed call and after every group; group_ms[g] receives
 * group g's time (groups = 1 times all the calls between two events).  The
 * bench's counterpart of the reference's compiled benchmark loops
 * (crates/axc-driver/benches/dispatch_q4km.rs:101-124): no interpreter
 * between launches.  No counterpart in the reference's C surface. */
enum {
    AXH_BENCH_Q4K_MATVEC = 1, AXH_BENCH_Q4_0_MATVEC = 2, AXH_BENCH_Q5K_MATVEC = 3,
    AXH_BENCH_Q6K_MATVEC = 4, AXH_BENCH_Q4K_GATE_UP = 5, AXH_BENCH_Q4K_MATMUL_F16 = 6,
    AXH_BENCH_Q4K_MATMUL_F32 = 7, AXH_BENCH_READ_FLOOR = 8, AXH_BENCH_LAUNCH_EMPTY = 9,
    AXH_BENCH_READ_SHAPE = 10, /* axh_read_floor_shape: n_rows = workgroups, variant->
                                  waves_per_workgroup = threads / 64, variant->prefetch = loads */
    AXH_BENCH_Q4_0_GATE_UP = 11, AXH_BENCH_Q5K_GATE_UP = 12
};
typedef struct axh_bench_op {
    uint32_t op;                   /* AXH_BENCH_* */
    const void *q;                 /* first weight copy */
    uint64_t q_stride;             /* bytes between copies */
    uint32_t n_copies;             /* >= 1 */
    uint64_t q2_offset;            /* gate/up: the up matrix at q + q2_offset in a copy */
    const void *x;                 /* activations (f32, or f16 for MATMUL_F16) */
    void *x16;                     /* MATMUL_F32: the f16 staging buffer */
    void *y;                       /* output; READ_FLOOR / LAUNCH_EMPTY: the out words */
    uint32_t n_rows, units, batch; /* READ_FLOOR: units = bytes / 16; y holds batch words */
    const axh_q4_variant *variant;
    const axh_q4_matmul_variant *matmul_variant;
} axh_bench_op;
axh_status axh_bench_loop(axh_context *ctx, const axh_bench_op *op, uint32_t warmup,
                          uint32_t groups, uint32_t calls_per_group, float *group_ms);

/* The built-in code object holding every kernel above, for callers that drive
 * the generic prepare/dispatch API (e.g. the reference-contract kernels
 * "q4km_dequant_matvec" and "q4_0_dequant_matvec"). */
const void *axh_builtin_code_object(size_t *bytes);

#ifdef __cplusplus
}
#endif
#endif /* AXH_H */
