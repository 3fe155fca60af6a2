// Q4_0 / Q4_K_M operations over resident device buffers: variant selection
// (the strategy holes), LDS tile sizing, grid shape and launch of the
// builtin gfx950 kernels in q4_matvec.hip.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "axh_internal.h"

// Code objects embedded by axh_embed.S (.incbin of the gfx950 ELFs).
extern "C" const unsigned char axh_q4_matvec_co_begin[];
extern "C" const unsigned char axh_q4_matvec_co_end[];
extern "C" const unsigned char axh_q4_matmul_co_begin[];
extern "C" const unsigned char axh_q4_matmul_co_end[];

namespace axh {

namespace {

struct RowsArgs {
  uint32_t n_rows;
  uint32_t units_per_row;
  uint32_t tile_units;
  uint32_t pad;
};
struct CountArgs {
  uint32_t n_units;
};
struct MatmulArgs {
  uint32_t n_rows;
  uint32_t sb_per_row;
  uint32_t batch;
  uint32_t pad;
};

// Compiled batched-matmul kernels (keep in sync with q4_matmul.hip).  Kinds 1
// (LDS-tiled), 2 (register A), 4 (streaming) and 6 (row-split tile) were
// removed: none was the fastest variant at any shape measured; their numbers
// stay unused so that a request for one fails as an unknown variant.
//   kind 3 (K-split)    axh_q4k_matmul_ks_k{W}_n{NT}_p{PF}[_r1]: W waves split K of one tile of
//                       16 * RT rows (RT = 2, or 1 with _r1);
//   kind 5 (K-split tile) axh_q4k_matmul_kx_r{RT}_n{NT}_k{W}_p{PF}: a 16*RT x 16*NT tile per
//                       workgroup, its W waves splitting K by 64-wide superblock chunks,
//                       register A, operands through per-wave LDS rings, PF superblocks in
//                       flight.
//   kind 7 (streaming rows) axh_q4k_matmul_sr_w{W}_s2[_n2|_h]: persistent, one workgroup per
//                       CU over 16-row blocks, K <= 4096 (pf 2: 8-column groups).
//   kind 8 (32x32 tiles) axh_q4k_matmul_rm_w{W}_r{RT}_p4: W waves of RT 32-row MFMA tiles
//                       over 128 columns, a 4-deep LDS ring.
//   kind 9 (long rows)  axh_q4k_matmul_lk_c{4*NT}_x{PF}_w{WD}[_r2]: 8 waves over RT 16-row
//                       tiles and 4 * NT columns (col_tiles counts 4-column groups), K in
//                       chunks of 8 superblocks, X through an LDS ring PF chunks ahead, the
//                       weights in registers WD chunks ahead (3 for PF 1, else PF).
struct MatmulVariant {
  uint32_t kind, w, nt, pf, rt; // rt: row tiles (kinds 3, 5, 8 and 9)
};
constexpr MatmulVariant kQ4kMatmulVariants[] = {
    {3, 4, 1, 2, 2}, {3, 8, 1, 1, 2}, {3, 4, 2, 2, 2}, {3, 8, 2, 1, 2}, {3, 8, 1, 1, 1},
    {3, 8, 1, 2, 1}, {5, 4, 8, 2, 4},
    {5, 4, 8, 2, 2}, {5, 4, 4, 2, 4}, {5, 4, 4, 3, 4}, {5, 4, 4, 2, 8}, {5, 4, 2, 2, 4},
    {5, 4, 2, 3, 4}, {5, 4, 1, 3, 4}, {7, 8, 1, 1, 0}, {7, 8, 2, 1, 0}, {7, 8, 1, 2, 0},
    {8, 8, 8, 4, 1}, {8, 4, 8, 4, 2}, {8, 4, 8, 4, 1}, {8, 2, 8, 4, 2}, {9, 8, 2, 2, 1},
    {9, 8, 2, 1, 1}, {9, 8, 4, 1, 1}, {9, 8, 2, 2, 2}, {9, 8, 4, 1, 2}, {9, 8, 1, 2, 1}};
// The matmul kernels read zeros through offsets at or past 0xFFF00000 (with
// the step offsets on top), and address rows up to 16 past the matrix: q and
// x must stay below that, with 16 rows to spare.
constexpr uint64_t kMatmulOob = 0xFFF00000u;

struct MatvecVariant {
  uint32_t rpw, nw, pf, nt;
  uint32_t xp; // x sub-blocks staged per thread (1, or 2 for the _x2 kernels)
};

// Compiled instantiations of axh_q4k_matvec_flat_r{rpw}_w{nw}_p{pf}_n{0|1}[_x2]
// (persistent kernel; nt: 1 = non-temporal weight loads, 2 = normal loads).
// Keep in sync with the AXH_Q4K_MATVEC_FLAT / _X2 lists in q4_matvec.hip.
constexpr MatvecVariant kQ4kVariants[] = {
    {1, 8, 2, 2, 1}, {1, 8, 4, 2, 1}, {1, 8, 7, 2, 1}, {1, 16, 2, 2, 1}, {1, 4, 7, 2, 1},
    {2, 4, 2, 2, 1}, {2, 4, 4, 2, 1}, {2, 8, 2, 2, 1}, {2, 8, 4, 2, 1},  {4, 4, 2, 2, 1},
    {1, 8, 7, 1, 1}, {2, 4, 2, 1, 1}, {2, 4, 4, 1, 1}, {1, 4, 2, 2, 2},  {1, 4, 4, 2, 2},
    {2, 4, 2, 2, 2}, {2, 4, 4, 2, 2}, {1, 8, 1, 2, 1}, {1, 4, 1, 2, 1}, {2, 4, 1, 2, 1},
    {2, 8, 1, 2, 1},
};
// axh_q4k_gate_up_r{rpw}_w{nw}_p{pf}_x{xp}: fused SwiGLU gate/up kernels, rpw
// output rows per bundle (each lane group reads rpw gate and rpw up rows).
// Keep in sync with the AXH_Q4K_GATE_UP list in q4_matvec.hip.
constexpr MatvecVariant kGateUpVariants[] = {
    {1, 4, 2, 2, 1}, {1, 4, 4, 2, 1}, {1, 8, 2, 2, 1}, {2, 4, 2, 2, 1},
    {2, 8, 2, 2, 1}, {1, 4, 2, 2, 2}, {1, 8, 2, 2, 2}, {1, 4, 1, 2, 1},
    {1, 8, 1, 2, 1},
};
// axh_q5k_matvec_flat_r{rpw}_w{nw}_p{pf}_x{xp} and axh_q6k_... (ggml k-quants
// next to Q4_K).  Keep in sync with AXH_Q5K_MATVEC_FLAT / AXH_Q6K_MATVEC_FLAT.
constexpr MatvecVariant kQ5kVariants[] = {
    {1, 4, 2, 2, 1}, {1, 8, 2, 2, 1}, {2, 4, 2, 2, 1}, {1, 4, 2, 2, 2}, {1, 8, 2, 2, 2},
    {1, 4, 1, 2, 1}, {1, 8, 1, 2, 1},
};
constexpr MatvecVariant kQ6kVariants[] = {
    {1, 4, 2, 2, 1}, {1, 8, 2, 2, 1}, {1, 4, 4, 2, 1}, {2, 4, 2, 2, 1},
    {1, 4, 2, 2, 2}, {1, 8, 2, 2, 2}, {1, 4, 1, 2, 1}, {1, 8, 1, 2, 1},
};
// axh_q4_0_matvec_r{rpw}_w{nw} (prefetch and cache policy are not holes for Q4_0).
constexpr MatvecVariant kQ4_0Variants[] = {
    {1, 1, 1, 2, 1}, {1, 4, 1, 2, 1}, {2, 4, 1, 2, 1}, {4, 4, 1, 2, 1}};
// axh_q4_0_matvec_flat_r{rpw}_w{nw}_p{pf}_x{xp}: the Q4_K persistent kernel
// over octets of 8 Q4_0 blocks (normal loads only).  Keep in sync with the
// AXH_Q4_0_MATVEC_FLAT list in q4_matvec.hip.
constexpr MatvecVariant kQ4_0FlatVariants[] = {
    {1, 4, 1, 2, 1}, {1, 8, 1, 2, 1}, {2, 4, 1, 2, 1}, {2, 8, 1, 2, 1},
    {1, 8, 2, 2, 1}, {2, 4, 2, 2, 2}, {1, 16, 2, 2, 1}};
constexpr uint32_t kQ4_0FlatRounds = 2; // persistent Q4_0 grid: resident workgroups x 2
// axh_q4_0_gate_up_r{rpw}_w{nw}_p{pf}_x{xp}: the fused gate/up kernel over two
// Q4_0 matrices.  Keep in sync with the AXH_Q4_0_GATE_UP list in q4_matvec.hip.
constexpr MatvecVariant kQ4_0GateUpVariants[] = {
    {1, 4, 1, 2, 1}, {1, 8, 1, 2, 1}, {2, 4, 1, 2, 1},
    {1, 4, 2, 2, 1}, {1, 8, 2, 2, 1}, {1, 4, 2, 2, 2}};

constexpr uint32_t kQ4kMaxTileSb = 128;   // tiled kernel: 128 * 1088 B = 136 KiB of LDS
constexpr uint32_t kQ4kFlatMaxSb = 128;   // persistent kernel: 128 * 1120 B = 140 KiB of LDS
constexpr uint32_t kQ4kFlatRounds = 2;    // persistent Q4_K grid: resident workgroups x 2
constexpr uint32_t kQ4_0MaxTileB = 1024; // 1024 * 132 B = 132 KiB of LDS

} // namespace

bool is_builtin_code_object(const void *co, size_t bytes) {
  const unsigned char *objs[2][2] = {{axh_q4_matvec_co_begin, axh_q4_matvec_co_end},
                                     {axh_q4_matmul_co_begin, axh_q4_matmul_co_end}};
  for (const auto &o : objs) {
    const size_t n = (size_t)(o[1] - o[0]);
    if (bytes == n && (co == o[0] || std::memcmp(co, o[0], n) == 0)) return true;
  }
  return false;
}

axh_status builtin_kernel(axh_context *ctx, const char *entry, uint32_t n_buffers,
                          uint32_t pc_bytes, uint32_t wg_x, axh_kernel **out) {
  std::lock_guard<std::mutex> lk(ctx->ops_mu);
  auto it = ctx->ops.find(entry);
  if (it != ctx->ops.end()) {
    *out = it->second;
    return AXH_OK;
  }
  // Inputs are read-only; the last binding is the output.
  uint8_t access[4] = {AXH_ACCESS_READ_ONLY, AXH_ACCESS_READ_ONLY, AXH_ACCESS_READ_ONLY,
                       AXH_ACCESS_READ_ONLY};
  if (n_buffers == 0 || n_buffers > 4) return fail(AXH_ERR_INVALID_ARGUMENT, "bad binding count");
  access[n_buffers - 1] = AXH_ACCESS_READ_WRITE;
  axh_binding_plan plan{};
  plan.n_buffers = n_buffers;
  plan.access = access;
  plan.push_constant_total_bytes = pc_bytes;
  plan.workgroup_size[0] = wg_x;
  plan.workgroup_size[1] = 1;
  plan.workgroup_size[2] = 1;
  plan.dynamic_lds_bytes = 0;
  size_t n = 0;
  const void *co = axh_builtin_code_object(&n);
  if (std::strncmp(entry, "axh_q4k_matmul_", 15) == 0) {
    co = axh_q4_matmul_co_begin;
    n = (size_t)(axh_q4_matmul_co_end - axh_q4_matmul_co_begin);
  }
  axh_kernel *k = nullptr;
  axh_status s = axh_prepare_kernel(ctx, co, n, &plan, pc_bytes, entry, &k);
  if (s != AXH_OK) return s;
  ctx->ops.emplace(entry, k);
  *out = k;
  return AXH_OK;
}

// The compiled variant matching the requested holes (unset holes take the
// default's value); among staging widths, the smallest one that holds
// `min_xp` x sub-blocks per thread, else the widest.
static const MatvecVariant *find_variant(const MatvecVariant *table, size_t n,
                                         const axh_q4_variant *v, MatvecVariant dflt,
                                         uint32_t min_xp = 1) {
  MatvecVariant want = dflt;
  if (v) {
    if (v->rows_per_wave) want.rpw = v->rows_per_wave;
    if (v->waves_per_workgroup) want.nw = v->waves_per_workgroup;
    if (v->prefetch) want.pf = v->prefetch;
    if (v->nontemporal) want.nt = v->nontemporal;
  }
  const MatvecVariant *best = nullptr;
  for (size_t i = 0; i < n; ++i) {
    const MatvecVariant &t = table[i];
    if (t.rpw != want.rpw || t.nw != want.nw || t.pf != want.pf || t.nt != want.nt) continue;
    if (!best) {
      best = &t;
      continue;
    }
    const bool t_fits = t.xp >= min_xp, b_fits = best->xp >= min_xp;
    if ((t_fits && (!b_fits || t.xp < best->xp)) || (!t_fits && !b_fits && t.xp > best->xp))
      best = &t;
  }
  return best;
}

// The family and sb_per_lane holes belong to the Q4_K matvec only.
static axh_status reject_family(const axh_q4_variant *v) {
  if (v && (v->family || v->sb_per_lane))
    return fail(AXH_ERR_INVALID_ARGUMENT,
                "family and sb_per_lane are holes of the Q4_K and Q4_0 matvecs (and of the "
                "one-pass families of Q5_K / Q6_K and of the gate/up operations) only");
  return AXH_OK;
}

// Prefetch 1 (early refill) kernels stage x chunk by chunk during the first
// pass, so any row of up to 128 superblocks fits their x staging; the others
// stage XP sub-blocks per thread before the first iteration.
static bool staged_in_chunks(const MatvecVariant &v) { return v.pf == 1; }

// Default strategy per shape (chosen from on-device sweeps; any compiled
// variant can be forced through axh_q4_variant).
// Between 4097 and 6143 rows (more one-pass workgroups than CUs, fewer than
// two per CU) the one-pass kernels' default gives way: rows of up to 24
// superblocks take the whole-x kernel, rows of 25-32 the persistent kernel
// with one row per lane group.  A/B in one run each, us per call, default
// then the replacement: 4160 x 4096 5.12 vs 4.71, 5120 x 6144 6.87 vs 6.55,
// 5632 x 3072 5.10 vs 4.87 (and the autotuner's re-timed winners at
// 4352-5632 x 4096: 6-9 % faster, 4608 x 5120 6 %); 4608 x 8192 8.14 vs 7.41,
// 5120 x 8192 8.24 vs 7.54, 5632 x 8192 8.38 vs 7.66, 6000 x 7168 8.49 vs
// 7.76, 4352 x 7680 8.16 vs 7.43, where the persistent kernel with two rows
// per lane group (its default for short rows) took 9.2-9.7 and the whole-x
// kernel 8.3-8.5; 4097 x 6400 even (6.15 vs 6.25), 4608 x 2048 even.
constexpr uint32_t kOneWholeMinRows = 6144, kOneWholeMaxSb = 32; // x whole from here on
constexpr uint32_t kOneMidMinRows = 4097, kOneMidWholeMaxSb = 24;

// Rows of 74 or more superblocks leave LDS for one one-pass workgroup per CU
// (nsb * 1120 bytes each, 160 KiB per CU), so the one-pass grid balances only
// at whole multiples of 4096 rows;
// the persistent kernel's 4096 waves (16 per workgroup, one row pair each)
// balance up to 8192 rows.  Between 4097 and 8191 rows the persistent kernel
// is ahead (A/B in one run, us per call, one pass vs persistent: 4352 x
// 28672 24.17 vs 18.95, 5120 x 28672 24.25 vs 19.48, 6144 x 28672 24.78 vs
// 21.03, 7168 x 28672 25.72 vs 24.24, 5120 x 20480 18.70 vs 15.42, 6144 x
// 20480 18.66 vs 16.52, 7168 x 20480 20.06 vs 18.24, 6144 x 32768 28.00 vs
// 23.81); at 8192 rows they are even (27.34 vs 27.01) and at 10240 the one
// pass is ahead (37.38 vs 42.37).
constexpr uint32_t kLongMinSb = 74, kLongMaxRows = 8191;

// 24576-32768 rows of 25-32 superblocks too (A/B in one run, us per call,
// persistent r1 w4 p1 against x staged whole: 28672 x 8192 26.18 vs 27.48,
// 32768 x 8192 29.48 vs 31.56, 28672 x 7168 25.21 vs 26.30; even at 16384 x
// 8192, 16.72 vs 16.87 for x whole, and 20480 x 8192, 20.73 vs 20.86).
constexpr uint32_t kTallPersistMinRows = 24576, kTallPersistMaxRows = 32768;

static bool q4k_mid_band_persistent(uint32_t n_rows, uint32_t nsb) {
  if (n_rows >= kOneMidMinRows && n_rows <= kLongMaxRows && nsb >= kLongMinSb) return true;
  if (n_rows >= kTallPersistMinRows && n_rows <= kTallPersistMaxRows && nsb > kOneMidWholeMaxSb &&
      nsb <= kOneWholeMaxSb)
    return true;
  return n_rows >= kOneMidMinRows && n_rows < kOneWholeMinRows && nsb > kOneMidWholeMaxSb &&
         nsb <= kOneWholeMaxSb;
}

static MatvecVariant q4k_default(uint32_t n_rows, uint32_t nsb) {
  // The persistent kernel stages 32-element sub-blocks of x, one (or two for
  // the _x2 kernels) per thread.
  // Early refill (prefetch 1) for short rows: 14336 x 4096 9.9 vs 10.5 us,
  // neutral on 4096 x 4096.  On the 128256 x 4096 head prefetch 2 stays
  // ahead by 1-2 % (58.1-59.0 vs 59.4 us in one run).
  if (q4k_mid_band_persistent(n_rows, nsb) && nsb <= kOneWholeMaxSb) return {1, 4, 1, 2, 1};
  if (nsb * 8u <= 256u) return {2, 4, n_rows >= 65536u ? 2u : 1u, 2, 1};
  if (nsb * 8u <= 512u) return {1, 8, 2, 2, 1};
  return {1, 16, 2, 2, 1};
}

// The LDS-tiled Q4_0 kernel's rows per wave (4 waves per workgroup), for the
// rows the octet kernels do not take (odd block counts, rows of more than
// 1024 blocks, fewer than 32 rows).  A/B in one run, us per call through the
// library's launch loop (one wave per workgroup was the default below 4096
// rows): 2048 x 448 blocks r1 w4 9.68 vs r1 w1 32.27, 256 x 160 3.99 vs 4.61;
// 4096 x 160 r1 6.98 vs r2 7.31, 4096 x 448 r2 13.82 vs r1 17.70; 8192 x 128
// r2 6.34 vs r4 7.35, 8192 x 448 r4 21.77 vs r2 25.71; 14336 x 256 r4 17.57
// vs r2 20.18.
static MatvecVariant q4_0_default(uint32_t n_rows, uint32_t nb) {
  if (n_rows < 4096) return {1, 4, 1, 2, 1};
  if (n_rows < 8192 || (n_rows < 14336 && nb <= 256)) return {2, 4, 1, 2, 1};
  return {4, 4, 1, 2, 1};
}

// The register-resident column-slice kernel (family COLUMNS) splits each of
// up to kQ4kColsMaxSb superblocks across the workgroup's waves.  Fewer than
// kQ4kColsMaxRows rows of at most kQ4kColsMaxSb superblocks (the one-workgroup
// kernel's shapes aside) default to the tiled kernel, one row per wave: per
// call, interleaved in one run, 8 x 4096 3.32 vs 4.84 us for the column
// kernel, 31 x 4096 2.65 vs 4.13, 3 x 4096 3.31 vs 4.97, 8 x 14336 4.35 vs
// 6.13, 31 x 14336 4.44 vs 6.15, 24 x 8192 3.44 vs 5.17; and against split-K
// on 64-128 superblocks 16 x 32768 7.28 vs 9.64, 12 x 25600 6.36 vs 9.08, 31 x
// 16384 4.61 vs 13.66 (8 x 32768 7.26 vs 7.27).  Split-K keeps the longer
// rows (8 x 65536 9.42 vs 14.65 tiled, 16 x 51200 10.58 vs 12.00).
constexpr uint32_t kQ4kColsMaxRows = 32;
constexpr uint32_t kQ4kColsMaxSb = 128; // 4 * 128 lanes = 8 waves
constexpr uint32_t kQ4kColsRb = 4;      // rows per batch of the compiled cols kernels

// Few long rows: K split across one-wave workgroups of kSkSpw superblocks,
// reduced by the last workgroup through a per-stream workspace (counter and
// partials).  Every workgroup's device-scope release writes back its XCD's
// L2, so the split stays at 4..16 workgroups.
constexpr uint32_t kSkMinSb = 64;  // the split-K kernel's shortest rows (on request)
constexpr uint32_t kSkMaxSb = 256; // longer rows: more workgroups than pay
constexpr uint32_t kSkSpw = 16;    // superblocks per workgroup
constexpr uint32_t kSkMaxGroups = kSkMaxSb / kSkSpw;
constexpr uint32_t kSkMaxGroupRows = 32; // partial-sum rows per workgroup
constexpr size_t kSkWorkspaceBytes = (64u + kSkMaxGroups * 32u) * 4u;

static bool device_ptr_ok(const void *p) { return p != nullptr; }

// The workspace of `stream`: allocated and zeroed on first use (which must
// not be inside a graph capture); the kernels leave its counter at zero.
// Calls on one stream run in order, so they share it safely.
static axh_status stream_workspace(axh_context *ctx, hipStream_t stream, void **out) {
  std::lock_guard<std::mutex> lk(ctx->ops_mu);
  auto it = ctx->workspaces.find(stream);
  if (it != ctx->workspaces.end()) {
    *out = it->second;
    return ok();
  }
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, kSkWorkspaceBytes);
  if (e != hipSuccess) return fail(AXH_ERR_BUFFER_ALLOCATION, "workspace hipMalloc failed");
  e = hipMemset(p, 0, kSkWorkspaceBytes);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    hipFree(p);
    return fail(AXH_ERR_STAGING_COPY, "workspace initialisation failed");
  }
  ctx->workspaces.emplace(stream, p);
  *out = p;
  return ok();
}

} // namespace axh

using namespace axh;

extern "C" {

const void *axh_builtin_code_object(size_t *bytes) {
  if (bytes) *bytes = (size_t)(axh_q4_matvec_co_end - axh_q4_matvec_co_begin);
  return axh_q4_matvec_co_begin;
}

// Distinct hole assignments of a persistent-kernel table (staging width is
// derived from the shape, not a hole).
static bool first_of_holes(const MatvecVariant *t, size_t i) {
  for (size_t k = 0; k < i; ++k)
    if (t[k].rpw == t[i].rpw && t[k].nw == t[i].nw && t[k].pf == t[i].pf && t[k].nt == t[i].nt)
      return false;
  return true;
}

static uint32_t count_holes(const MatvecVariant *t, size_t n) {
  uint32_t c = 0;
  for (size_t i = 0; i < n; ++i) c += first_of_holes(t, i) ? 1u : 0u;
  return c;
}

static axh_status holes_at(const MatvecVariant *t, size_t n, uint32_t i, axh_q4_variant *out) {
  if (!out) return fail(AXH_ERR_INVALID_ARGUMENT, "out is NULL");
  uint32_t c = 0;
  for (size_t k = 0; k < n; ++k) {
    if (!first_of_holes(t, k)) continue;
    if (c++ == i) {
      out->rows_per_wave = t[k].rpw;
      out->waves_per_workgroup = t[k].nw;
      out->prefetch = t[k].pf;
      out->nontemporal = t[k].nt;
      return ok();
    }
  }
  return fail(AXH_ERR_INVALID_ARGUMENT, "variant index out of range");
}

uint32_t axh_q4k_matvec_variant_count(void) {
  return count_holes(kQ4kVariants, sizeof(kQ4kVariants) / sizeof(kQ4kVariants[0]));
}

axh_status axh_q4k_matvec_variant_at(uint32_t i, axh_q4_variant *out) {
  return holes_at(kQ4kVariants, sizeof(kQ4kVariants) / sizeof(kQ4kVariants[0]), i, out);
}

uint32_t axh_q4k_gate_up_variant_count(void) {
  return count_holes(kGateUpVariants, sizeof(kGateUpVariants) / sizeof(kGateUpVariants[0]));
}

axh_status axh_q4k_gate_up_variant_at(uint32_t i, axh_q4_variant *out) {
  return holes_at(kGateUpVariants, sizeof(kGateUpVariants) / sizeof(kGateUpVariants[0]), i, out);
}

uint32_t axh_q4_0_matvec_variant_count(void) {
  return (uint32_t)(sizeof(kQ4_0Variants) / sizeof(kQ4_0Variants[0]));
}

axh_status axh_q4_0_matvec_variant_at(uint32_t i, axh_q4_variant *out) {
  if (!out || i >= axh_q4_0_matvec_variant_count())
    return fail(AXH_ERR_INVALID_ARGUMENT, "variant index out of range");
  out->rows_per_wave = kQ4_0Variants[i].rpw;
  out->waves_per_workgroup = kQ4_0Variants[i].nw;
  out->prefetch = kQ4_0Variants[i].pf;
  out->nontemporal = kQ4_0Variants[i].nt;
  return ok();
}

// Workgroups of `k` resident per CU at `lds` bytes of dynamic LDS (cached).
static uint32_t occupancy(axh_context *ctx, axh_kernel *k, uint32_t lds) {
  const uint64_t key = ((uint64_t)(uintptr_t)k << 20) ^ lds;
  {
    std::lock_guard<std::mutex> lk(ctx->ops_mu);
    auto it = ctx->occupancy.find(key);
    if (it != ctx->occupancy.end()) return it->second;
  }
  int blocks = 0;
  const int threads = (int)(k->wg[0] * k->wg[1] * k->wg[2]);
  if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, k->fn, threads, lds) !=
          hipSuccess ||
      blocks < 1)
    blocks = 1;
  std::lock_guard<std::mutex> lk(ctx->ops_mu);
  ctx->occupancy[key] = (uint32_t)blocks;
  return (uint32_t)blocks;
}

// The kernel, LDS bytes and shape arguments for one Q4_K matvec call.
struct Q4kPlan {
  char name[64];
  uint32_t nw;      // waves per workgroup
  uint32_t lds;     // dynamic LDS bytes
  bool flat;        // persistent kernel (grid sized by occupancy)
  uint32_t units;   // flat: workgroups needed; tiled: workgroups
  RowsArgs args;
};

// One workgroup for 1-4 long rows (axh_q4k_matvec_wg_w8_x2_r{1,2,4}): all 512 lanes
// on the same rows, x staged in LDS by coalesced loads (272 + 8 floats per
// superblock), so rows of up to 128 superblocks.  Measured faster than the
// split-K and column kernels for 1-2 rows of 33+ superblocks and 3-4 rows of
// 64+ (1 x 32768: 4.6 vs 7.4 us per host-launched call).
constexpr uint32_t kWgMaxSb = 128, kWgNw = 8;

static bool q4k_use_wg(uint32_t n_rows, uint32_t nsb) {
  return nsb <= kWgMaxSb && ((n_rows <= 2u && nsb >= 33u) || (n_rows <= 4u && nsb >= 64u));
}

// One pass with one pair of rows per wave (axh_q4k_matvec_one_i{NIT}, NIT =
// ceil(nsb / 8)): one 8-wave workgroup per 16 rows, all launched, each
// staging x for its own rows.  Faster than the persistent kernels from 32 up
// to 32768 rows (A/B in one run: 4096 x 14336 8.1-8.4 vs 8.5-8.7 us, 4096 x
// 4096 4.06 vs 4.6-4.9, 14336 x 4096 8.9-9.1 vs 9.9-10.5, 32768 x 4096 17.0
// vs 18.6); on the 128256-row head (8016 workgroups) the persistent kernel
// stays ahead (53.5 vs 56.8 us).
constexpr uint32_t kOneMinRows = 32, kOneMaxRows = 32768, kOneMaxSb = 128;
// From 6144 rows of at most 32 superblocks (two or more workgroups per CU,
// and LDS for three or more) the one-pass kernel that stages x whole behind
// one barrier (axh_q4k_matvec_onex_i{NIT}) is used: A/B in one run, 6144 x
// 4096 5.31 vs 5.77 us, 8192 x 4096 5.63 vs 6.24, 11008 x 4096 7.10 vs 7.53,
// 14336 x 4096 8.39-8.47 vs 8.90-8.97, 14336 x 8192 15.7-16.0 vs 16.1-16.4,
// 32768 x 4096 even.  4096 rows (one workgroup per CU) and longer rows (LDS
// for one or two) measured slower or even: 4096 x 4096 4.21 vs 4.08, 4096 x
// 14336 8.84-8.93 vs 8.42-8.55, 8192 x 14336 even, 8192 x 32768 32.5-32.8 vs
// 31.5-32.2.  (kOneWholeMinRows and kOneWholeMaxSb are defined with the
// 4097-6143-row band above.)

// The whole-x kernel also takes 32769-65536 rows of at most 16 superblocks
// (A/B in one run against the persistent kernel: 40000 x 4096 18.5-18.8 vs
// 20.5-21.7 us, 65536 x 4096 29.1 vs 29.8-30.1), but not longer rows (50000 x
// 8192: 46.3-46.6 vs 43.4-44.1); the 128256-row head stays persistent
// (51.6-51.8 vs 53.5-54.3 us).
constexpr uint32_t kOneTallMaxRows = 65536, kOneTallMaxSb = 16;

// x two chunks ahead (axh_q4k_matvec_onep_i{NIT}) from four iterations on, up
// to one workgroup per CU (A/B in one run, GB/s at the median, one vs onep:
// 4096 rows x 8192 3411-3420 vs 3526-3531, x 14336 4114-4169 vs 4254-4277, x
// 32768 4767-4832 vs 4870-4974, 3072 x 14336 3315-3323 vs 3376-3381; even at
// 1024-2048 rows; slower at three iterations, 4096 x 6144 3008-3020 vs
// 2965-2974, and with two workgroups per CU, 6144 x 14336 3982-4015 vs
// 3912-3925).  The prefetch hole of the one-pass family picks either.
constexpr uint32_t kOnePMinIt = 4, kOnePMaxRows = 4096;

// Up to 1024 rows the one-pass kernels' 16 rows per workgroup leave CUs idle
// (64 workgroups at 1024 rows); the tiled kernel with one row per wave (4
// rows per workgroup) fills 4x as many, and from 24 superblocks per row that
// pays.  A/B in one run, us per call, one pass vs tiled r1 w4 p2: 128 x 8192
// 4.38 vs 3.41, 128 x 28672 11.94 vs 7.43, 256 x 6144 3.70 vs 3.29, 256 x
// 14336 6.88 vs 4.98, 512 x 14336 6.90 vs 5.57, 512 x 28672 12.06 vs 8.61,
// 1024 x 6144 4.00 vs 3.87, 1024 x 28672 12.13 vs 9.43 (and the autotuner's
// re-timed winners: 1024 x 8192 -12 %, 1024 x 14336 -19 %, 512 x 8192 -13 %);
// from 2048 rows the one pass is ahead (2048 x 8192 4.98 vs 5.14, 2048 x
// 28672 12.33 vs 16.91).  Shorter rows pay on fewer rows: up to 512 rows from
// 13 superblocks (512 x 3584 2.78 vs 3.02-3.15, 512 x 4096 2.84 vs 3.10-3.19,
// 256 x 3584 2.75 vs 2.91, 512 x 5120 3.61 vs 3.78-3.90), 513-1024 rows from
// 17 (1024 x 5120 3.88 vs 4.04-4.08; 1024 x 4096 3.25 vs 3.27-3.29 and 1024 x
// 3584 even), and not below 13 (512 x 3072 3.19 vs 3.24-3.30, 512 x 2048
// even).
constexpr uint32_t kTiledFewMaxRows = 1024, kTiledFewMinSb = 24;
constexpr uint32_t kTiledFewShortMaxRows = 512, kTiledFewShortMinSb = 13, kTiledFewMidMinSb = 17;

static bool q4k_tiled_few(uint32_t n_rows, uint32_t nsb) {
  if (n_rows > kTiledFewMaxRows) return false;
  if (nsb >= kTiledFewMinSb) return true;
  return nsb >= (n_rows <= kTiledFewShortMaxRows ? kTiledFewShortMinSb : kTiledFewMidMinSb);
}

static bool use_one_pass(uint32_t n_rows, uint32_t nsb) {
  if (nsb < 1 || nsb > kOneMaxSb || n_rows < kOneMinRows) return false;
  return n_rows <= kOneMaxRows || (nsb <= kOneTallMaxSb && n_rows <= kOneTallMaxRows);
}


// Tiled kernel plan (rows longer than one LDS tile, or matrices >= 4 GiB).
static void plan_tiled(uint32_t n_rows, uint32_t nsb, const MatvecVariant &tv, Q4kPlan *p) {
  std::snprintf(p->name, sizeof(p->name), "axh_q4k_matvec_tiled_r%u_w%u_p%u", tv.rpw, tv.nw, tv.pf);
  uint32_t tile = (nsb + 7u) & ~7u;
  if (tile == 0) tile = 8;
  if (tile > kQ4kMaxTileSb) tile = kQ4kMaxTileSb;
  p->nw = tv.nw;
  p->lds = tile * 1088u;
  p->flat = false;
  const uint32_t rows_per_wg = tv.rpw * tv.nw;
  p->units = (n_rows + rows_per_wg - 1) / rows_per_wg;
  p->args = RowsArgs{n_rows, nsb, tile, 0};
}

// Which holes a family reads; the others must stay zero.
static bool q4k_persistent_holes(const axh_q4_variant *v) {
  return v && (v->rows_per_wave || v->waves_per_workgroup || v->prefetch || v->nontemporal);
}

// The default family for a shape (the sweeps quoted above each kernel).
static uint32_t q4k_default_family(uint32_t n_rows, uint32_t nsb, uint64_t q_bytes) {
  if (q4k_use_wg(n_rows, nsb)) return AXH_Q4K_FAMILY_WORKGROUP;
  if (n_rows < kQ4kColsMaxRows && nsb > kQ4kColsMaxSb && nsb <= kSkMaxSb &&
      q_bytes < 0xFFFFFF00ull)
    return AXH_Q4K_FAMILY_SPLIT_K;
  if (n_rows < kQ4kColsMaxRows && nsb >= 1 && nsb <= kQ4kColsMaxSb) return AXH_Q4K_FAMILY_TILED;
  if (use_one_pass(n_rows, nsb) && q_bytes < 0xFFFFFFFFull) {
    if (q4k_tiled_few(n_rows, nsb)) return AXH_Q4K_FAMILY_TILED;
    if (q4k_mid_band_persistent(n_rows, nsb)) return AXH_Q4K_FAMILY_PERSISTENT;
    if (n_rows >= kOneWholeMinRows && nsb <= kOneWholeMaxSb) return AXH_Q4K_FAMILY_ONE_PASS_X;
    if (n_rows >= kOneMidMinRows && n_rows < kOneWholeMinRows && nsb <= kOneMidWholeMaxSb)
      return AXH_Q4K_FAMILY_ONE_PASS_X;
    return AXH_Q4K_FAMILY_ONE_PASS;
  }
  return AXH_Q4K_FAMILY_PERSISTENT; // falls back to tiled for rows it cannot stage
}

static axh_status plan_q4k(uint32_t n_rows, uint32_t sb_per_row, const axh_q4_variant *variant,
                           Q4kPlan *p) {
  const uint64_t q_bytes = (uint64_t)n_rows * sb_per_row * 144u;
  const uint32_t nsb = sb_per_row;
  uint32_t fam = variant ? variant->family : 0u;
  if (fam > AXH_Q4K_FAMILY_TILED) return fail(AXH_ERR_INVALID_ARGUMENT, "unknown kernel family");
  const bool explicit_family = fam != AXH_Q4K_FAMILY_DEFAULT;
  if (!explicit_family)
    fam = q4k_persistent_holes(variant) ? (uint32_t)AXH_Q4K_FAMILY_PERSISTENT
                                        : q4k_default_family(n_rows, nsb, q_bytes);
  if (variant && variant->sb_per_lane && fam != AXH_Q4K_FAMILY_ONE_PASS &&
      fam != AXH_Q4K_FAMILY_ONE_PASS_X)
    return fail(AXH_ERR_INVALID_ARGUMENT, "sb_per_lane is a hole of the one-pass families only");
  const bool other_holes = q4k_persistent_holes(variant);
  switch (fam) {
  case AXH_Q4K_FAMILY_WORKGROUP: {
    if (variant && (variant->waves_per_workgroup || variant->prefetch || variant->nontemporal))
      return fail(AXH_ERR_INVALID_ARGUMENT, "the one-workgroup family's only hole is rows_per_wave");
    if (n_rows > 4u || nsb < 1u || nsb > kWgMaxSb)
      return fail(AXH_ERR_INVALID_ARGUMENT,
                  "the one-workgroup family takes 1-4 rows of 1-128 superblocks");
    uint32_t rb = variant && variant->rows_per_wave ? variant->rows_per_wave
                  : n_rows == 1u                    ? 1u
                  : n_rows == 2u                    ? 2u
                                                    : 4u;
    if ((rb != 1u && rb != 2u && rb != 4u) || rb < n_rows)
      return fail(AXH_ERR_INVALID_ARGUMENT,
                  "one-workgroup rows_per_wave must be 1, 2 or 4 and cover n_rows");
    std::snprintf(p->name, sizeof(p->name), "axh_q4k_matvec_wg_w%u_x2_r%u", kWgNw, rb);
    p->nw = kWgNw;
    p->lds = nsb * (272u + 8u) * 4u + rb * kWgNw * 4u;
    p->flat = false;
    p->units = 1;
    p->args = RowsArgs{n_rows, nsb, nsb, 0};
    return ok();
  }
  case AXH_Q4K_FAMILY_SPLIT_K:
    if (other_holes) return fail(AXH_ERR_INVALID_ARGUMENT, "the split-K family has no holes");
    if (n_rows > kSkMaxGroupRows || nsb < 1u || nsb > kSkMaxSb || q_bytes >= 0xFFFFFF00ull)
      return fail(AXH_ERR_INVALID_ARGUMENT,
                  "the split-K family takes 1-32 rows of 1-256 superblocks");
    std::snprintf(p->name, sizeof(p->name), "axh_q4k_matvec_sk_s%u", kSkSpw);
    p->nw = 1;
    p->lds = 0;
    p->flat = false;
    p->units = (nsb + kSkSpw - 1) / kSkSpw;
    p->args = RowsArgs{n_rows, nsb, kSkSpw, 0};
    return ok();
  case AXH_Q4K_FAMILY_COLUMNS: {
    if (other_holes) return fail(AXH_ERR_INVALID_ARGUMENT, "the column family has no holes");
    if (nsb < 1u || nsb > kQ4kColsMaxSb || q_bytes >= 0xFFFFFF00ull)
      return fail(AXH_ERR_INVALID_ARGUMENT, "the column family takes rows of 1-128 superblocks");
    // Each row is split across NW waves (4 lanes per superblock).
    const uint32_t nw = (nsb * 4u + 63u) / 64u;
    std::snprintf(p->name, sizeof(p->name), "axh_q4k_matvec_cols_r%u_w%u_n0_x1", kQ4kColsRb, nw);
    p->nw = nw;
    p->lds = 0;
    p->flat = false;
    p->units = (n_rows + kQ4kColsRb - 1) / kQ4kColsRb;
    p->args = RowsArgs{n_rows, nsb, nsb, 0};
    return ok();
  }
  case AXH_Q4K_FAMILY_ONE_PASS:
  case AXH_Q4K_FAMILY_ONE_PASS_X: {
    const uint32_t xd = variant ? variant->prefetch : 0u;
    if (variant && (variant->rows_per_wave || variant->waves_per_workgroup || variant->nontemporal))
      return fail(AXH_ERR_INVALID_ARGUMENT,
                  "the one-pass families' holes are sb_per_lane and (one pass) prefetch");
    if (xd && (fam == AXH_Q4K_FAMILY_ONE_PASS_X || xd > 2u))
      return fail(AXH_ERR_INVALID_ARGUMENT,
                  "one-pass prefetch is 1 or 2 x chunks ahead (none for the whole-x kernel)");
    if (nsb < 1u || nsb > kOneMaxSb || q_bytes >= 0xFFFFFFFFull)
      return fail(AXH_ERR_INVALID_ARGUMENT,
                  "the one-pass families take rows of 1-128 superblocks below 4 GiB");
    const uint32_t need = (nsb + 7u) / 8u;
    const uint32_t nit = variant && variant->sb_per_lane ? variant->sb_per_lane : need;
    if (nit < need || nit > 16u)
      return fail(AXH_ERR_INVALID_ARGUMENT,
                  "sb_per_lane must cover the row (ceil(sb_per_row / 8)) and be at most 16");
    if (xd == 2u && nit < 3u)
      return fail(AXH_ERR_INVALID_ARGUMENT, "x two chunks ahead needs three or more iterations");
    const bool two_ahead = fam == AXH_Q4K_FAMILY_ONE_PASS &&
                           (xd == 2u || (xd == 0u && nit >= kOnePMinIt && n_rows <= kOnePMaxRows));
    std::snprintf(p->name, sizeof(p->name), "axh_q4k_matvec_one%s_i%u",
                  fam == AXH_Q4K_FAMILY_ONE_PASS_X ? "x" : two_ahead ? "p" : "", nit);
    p->nw = 8;
    p->lds = nsb * 1120u;
    p->flat = false; // one workgroup per 16 rows, all of them launched
    p->units = (n_rows + 15u) / 16u;
    p->args = RowsArgs{n_rows, nsb, nsb, 0};
    return ok();
  }
  case AXH_Q4K_FAMILY_TILED: {
    if (variant && variant->nontemporal)
      return fail(AXH_ERR_INVALID_ARGUMENT, "the tiled family has no nontemporal hole");
    MatvecVariant tv = n_rows >= 2048 ? MatvecVariant{2, 8, 2, 2, 1} : MatvecVariant{1, 4, 2, 2, 1};
    if (variant && variant->rows_per_wave) tv.rpw = variant->rows_per_wave;
    if (variant && variant->waves_per_workgroup) tv.nw = variant->waves_per_workgroup;
    if (variant && variant->prefetch) tv.pf = variant->prefetch;
    if (!((tv.rpw == 2 && tv.nw == 8 && tv.pf == 2) || (tv.rpw == 1 && tv.nw == 4 && tv.pf == 2)))
      return fail(AXH_ERR_INVALID_ARGUMENT, "no compiled tiled Q4_K matvec variant matches");
    plan_tiled(n_rows, nsb, tv, p);
    return ok();
  }
  default:
    break;
  }
  // Persistent family (explicitly, or from its holes, or by default).
  const MatvecVariant dflt = q4k_default(n_rows, nsb);
  const uint32_t want_nw =
      variant && variant->waves_per_workgroup ? variant->waves_per_workgroup : dflt.nw;
  const uint32_t min_xp = (nsb * 8u + want_nw * 64u - 1u) / (want_nw * 64u);
  const MatvecVariant *v = find_variant(
      kQ4kVariants, sizeof(kQ4kVariants) / sizeof(kQ4kVariants[0]), variant, dflt, min_xp);
  if (!v) return fail(AXH_ERR_INVALID_ARGUMENT, "no compiled Q4_K matvec variant matches");
  p->flat = nsb >= 1 && nsb <= kQ4kFlatMaxSb && q_bytes < 0xFFFFFFFFull &&
            (staged_in_chunks(*v) || nsb * 8u <= v->xp * v->nw * 64u);
  if (p->flat) {
    std::snprintf(p->name, sizeof(p->name), "axh_q4k_matvec_flat_r%u_w%u_p%u_n%u%s", v->rpw,
                  v->nw, v->pf, v->nt == 1 ? 1u : 0u, v->xp == 2 ? "_x2" : "");
    p->nw = v->nw;
    p->lds = nsb * 1120u; // 272 floats of x + 8 sums per superblock
    // Each wave handles pairs of RPW-row bundles; the grid is persistent.
    const uint32_t bundles = (n_rows + v->rpw - 1) / v->rpw;
    const uint32_t pairs = (bundles + 1) / 2;
    p->units = (pairs + v->nw - 1) / v->nw;
    p->args = RowsArgs{n_rows, nsb, nsb, 0};
    return ok();
  }
  if (explicit_family)
    return fail(AXH_ERR_INVALID_ARGUMENT,
                "the persistent family takes rows of 1-128 superblocks below 4 GiB whose x "
                "this variant can stage");
  // Rows longer than one LDS tile, or matrices of 4 GiB and more.
  plan_tiled(n_rows, nsb,
             n_rows >= 2048 ? MatvecVariant{2, 8, 2, 2, 1} : MatvecVariant{1, 4, 2, 2, 1}, p);
  return ok();
}

// A call with no variant takes the context's tuned winner for the shape when
// it plans (a stale entry that no longer fits falls back to the default).
static axh_status plan_q4k_ctx(axh_context *ctx, uint32_t n_rows, uint32_t sb_per_row,
                               const axh_q4_variant *variant, Q4kPlan *p) {
  axh_q4_variant tuned{};
  if (!variant && lookup_winner(ctx, "q4k_matvec", n_rows, sb_per_row, &tuned) &&
      plan_q4k(n_rows, sb_per_row, &tuned, p) == AXH_OK)
    return ok();
  return plan_q4k(n_rows, sb_per_row, variant, p);
}

axh_status axh_context_q4k_matvec_kernel_name(axh_context *ctx, uint32_t n_rows,
                                              uint32_t sb_per_row, const axh_q4_variant *variant,
                                              char *buf, size_t cap) {
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  if (!buf || cap == 0) return fail(AXH_ERR_INVALID_ARGUMENT, "buf is NULL");
  Q4kPlan p{};
  axh_status s = plan_q4k_ctx(ctx, n_rows, sb_per_row, variant, &p);
  if (s != AXH_OK) return s;
  if (std::strlen(p.name) + 1 > cap) return fail(AXH_ERR_INVALID_ARGUMENT, "buf too small");
  std::memcpy(buf, p.name, std::strlen(p.name) + 1);
  return ok();
}

axh_status axh_q4k_matvec_default_variant(uint32_t n_rows, uint32_t sb_per_row,
                                         axh_q4_variant *out) {
  if (!out) return fail(AXH_ERR_INVALID_ARGUMENT, "out is NULL");
  *out = axh_q4_variant{};
  const uint64_t q_bytes = (uint64_t)n_rows * sb_per_row * 144u;
  const uint32_t fam = q4k_default_family(n_rows, sb_per_row, q_bytes);
  Q4kPlan p{};
  axh_status s = plan_q4k(n_rows, sb_per_row, nullptr, &p);
  if (s != AXH_OK) return s;
  out->family = fam;
  unsigned a = 0, b = 0, c = 0, d = 0;
  if (fam == AXH_Q4K_FAMILY_ONE_PASS || fam == AXH_Q4K_FAMILY_ONE_PASS_X) {
    out->sb_per_lane = (sb_per_row + 7u) / 8u;
    if (fam == AXH_Q4K_FAMILY_ONE_PASS)
      out->prefetch = std::strncmp(p.name, "axh_q4k_matvec_onep_", 20) == 0 ? 2u : 1u;
  } else if (fam == AXH_Q4K_FAMILY_WORKGROUP) {
    if (std::sscanf(p.name, "axh_q4k_matvec_wg_w%u_x2_r%u", &a, &b) == 2) out->rows_per_wave = b;
  } else if (std::sscanf(p.name, "axh_q4k_matvec_flat_r%u_w%u_p%u_n%u", &a, &b, &c, &d) == 4) {
    out->rows_per_wave = a;
    out->waves_per_workgroup = b;
    out->prefetch = c;
    out->nontemporal = d == 1u ? 1u : 2u;
  } else if (std::sscanf(p.name, "axh_q4k_matvec_tiled_r%u_w%u_p%u", &a, &b, &c) == 3) {
    out->family = AXH_Q4K_FAMILY_TILED;
    out->rows_per_wave = a;
    out->waves_per_workgroup = b;
    out->prefetch = c;
  }
  return ok();
}

axh_status axh_q4k_matvec_kernel_name(uint32_t n_rows, uint32_t sb_per_row,
                                      const axh_q4_variant *variant, char *buf, size_t cap) {
  if (!buf || cap == 0) return fail(AXH_ERR_INVALID_ARGUMENT, "buf is NULL");
  Q4kPlan p{};
  axh_status s = plan_q4k(n_rows, sb_per_row, variant, &p);
  if (s != AXH_OK) return s;
  if (std::strlen(p.name) + 1 > cap) return fail(AXH_ERR_INVALID_ARGUMENT, "buf too small");
  std::memcpy(buf, p.name, std::strlen(p.name) + 1);
  return ok();
}

axh_status axh_q4k_matvec(axh_context *ctx, const void *q, const float *x, float *y,
                          uint32_t n_rows, uint32_t sb_per_row, const axh_q4_variant *variant,
                          void *stream) {
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  if (n_rows == 0) return ok();
  if (!device_ptr_ok(y) || (sb_per_row && (!device_ptr_ok(q) || !device_ptr_ok(x))))
    return fail(AXH_ERR_INVALID_ARGUMENT, "q, x and y must be device pointers");
  if ((uint64_t)sb_per_row * 256u > 0xFFFFFFFFull)
    return fail(AXH_ERR_INVALID_ARGUMENT, "sb_per_row too large");
  if (((uintptr_t)q & 15u) || ((uintptr_t)x & 15u))
    return fail(AXH_ERR_INVALID_ARGUMENT, "q and x must be 16-byte aligned");
  Q4kPlan p{};
  axh_status s = plan_q4k_ctx(ctx, n_rows, sb_per_row, variant, &p);
  if (s != AXH_OK) return s;
  if (p.lds > ctx->core->max_lds)
    return fail(AXH_ERR_PIPELINE_LAYOUT, "LDS tile exceeds the device limit");
  hipSetDevice(ctx->core->device);
  axh_kernel *k = nullptr;
  const bool split_k = std::strncmp(p.name, "axh_q4k_matvec_sk_", 18) == 0;
  s = builtin_kernel(ctx, p.name, split_k ? 4 : 3, sizeof(RowsArgs), p.nw * 64u, &k);
  if (s != AXH_OK) return s;
  uint32_t grid[3] = {p.units, 1, 1};
  if (p.flat) {
    // Two rounds of resident workgroups (the bundle loop is grid-stride):
    // the tall matrices this kernel is the default for end with less tail
    // (128256 x 4096, prefetch 2, A/B in one run: 51.3-52.7 vs 52.2-54.1 us;
    // four rounds 51.4, one workgroup per bundle pair group 57.0).  The Q5_K,
    // Q6_K and gate/up launches stay at one round, where more was slower.
    const uint32_t resident = kQ4kFlatRounds * occupancy(ctx, k, p.lds) * ctx->core->cu_count;
    if (resident < grid[0]) grid[0] = resident;
  }
  const hipStream_t st = pick_stream(ctx, stream);
  if (split_k) {
    void *ws = nullptr;
    s = stream_workspace(ctx, st, &ws);
    if (s != AXH_OK) return s;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (st == ctx->core->stream && hipStreamIsCapturing(st, &cs) == hipSuccess &&
        cs == hipStreamCaptureStatusActive)
      ctx->capture_uses_workspace = true;
    void *bufs4[4] = {const_cast<void *>(q), const_cast<float *>(x), y, ws};
    s = launch_raw(k, grid, bufs4, 4, &p.args, sizeof(p.args), 0, st);
    return s == AXH_OK ? ok() : s;
  }
  void *bufs[3] = {const_cast<void *>(q), const_cast<float *>(x), y};
  s = launch_raw(k, grid, bufs, 3, &p.args, sizeof(p.args), p.lds, st);
  return s == AXH_OK ? ok() : s;
}

// Fused gate/up: the persistent kernel only (x of a row fits LDS).
static MatvecVariant gate_up_default(uint32_t n_rows, uint32_t nsb) {
  (void)n_rows;
  // early refill: 2 x 14336 x 4096 15.1-15.6 vs 15.7-16.4 us
  if (nsb * 8u <= 256u) return {1, 4, 1, 2, 1};
  return {1, 8, 2, 2, 1};
}

// The wave-paired one-pass gate/up kernels (axh_{q4k,q4_0}_gate_up_one{,x}_i*):
// one workgroup of 8 waves per 8 output rows, the even wave of a pair on the
// gate rows and the odd wave on the same up rows, rows of up to 8 steps (64
// superblocks or 512 Q4_0 blocks).  Family ONE_PASS (x chunk by chunk) or
// ONE_PASS_X (x whole); the only hole is sb_per_lane.  The shape's limits
// are checked by the caller.
constexpr uint32_t kGateUpOneMaxIt = 8;

static axh_status plan_gate_up_one(const char *fmt, bool q40, uint32_t n_rows, uint32_t units,
                                   const axh_q4_variant *variant, Q4kPlan *p) {
  if (variant->rows_per_wave || variant->waves_per_workgroup || variant->prefetch ||
      variant->nontemporal)
    return fail(AXH_ERR_INVALID_ARGUMENT, "the gate/up one-pass families' only hole is sb_per_lane");
  const uint32_t per_step = q40 ? 64u : 8u; // blocks or superblocks per step
  const uint32_t need = (units + per_step - 1u) / per_step;
  const uint32_t nit = variant->sb_per_lane ? variant->sb_per_lane : need;
  if (nit < need || nit > kGateUpOneMaxIt)
    return fail(AXH_ERR_INVALID_ARGUMENT,
                "gate/up one pass: sb_per_lane must cover the row and be at most 8");
  std::snprintf(p->name, sizeof(p->name), "axh_%s_gate_up_one%s_i%u", fmt,
                variant->family == AXH_Q4K_FAMILY_ONE_PASS_X ? "x" : "", nit);
  const uint32_t n_units = q40 ? (units + 7u) / 8u : units;
  p->nw = 8;
  p->lds = n_units * 1120u + 32u; // x, its sums, and 2 floats per wave pair
  p->flat = false;                // one workgroup per 8 output rows, all launched
  p->units = (n_rows + 7u) / 8u;
  p->args = RowsArgs{n_rows, units, units, 0};
  return ok();
}

static bool gate_up_one_family(const axh_q4_variant *v) {
  return v && (v->family == AXH_Q4K_FAMILY_ONE_PASS || v->family == AXH_Q4K_FAMILY_ONE_PASS_X);
}

// With no hole set, up to 12288 rows of up to 8 steps take the wave-paired
// one-pass kernel (x chunk by chunk up to 2048 rows, whole beyond), larger
// matrices the persistent one.  A/B in one run, us per call, Q4_K / Q4_0
// against the persistent default: 1024 x 4096 4.02 / 3.99 vs 4.88 / 4.92,
// 4096 x 4096 (x whole) 5.95 / 5.92 vs 6.91 / 6.80, 11008 x 4096 12.85 /
// 12.49 vs 13.43 / 13.13; but 14336 x 4096 15.32 / 14.78 vs 14.82 / 14.61
// and 28672 x 8192 52.3 / 47.6 vs 46.7 / 46.3 (the pair's closing barrier
// keeps a workgroup's waves from retiring on their own).
constexpr uint32_t kGateUpOneMaxRows = 12288, kGateUpOneChunkMaxRows = 2048;

static bool gate_up_default_one(const axh_q4_variant *variant, uint32_t n_rows, uint32_t nit,
                                axh_q4_variant *out) {
  if (variant && (variant->rows_per_wave || variant->waves_per_workgroup ||
                  variant->prefetch || variant->nontemporal || variant->family ||
                  variant->sb_per_lane))
    return false;
  if (n_rows > kGateUpOneMaxRows || nit > kGateUpOneMaxIt) return false;
  *out = axh_q4_variant{};
  out->family = n_rows <= kGateUpOneChunkMaxRows ? AXH_Q4K_FAMILY_ONE_PASS
                                                 : AXH_Q4K_FAMILY_ONE_PASS_X;
  return true;
}

static axh_status plan_gate_up(uint32_t n_rows, uint32_t sb_per_row,
                               const axh_q4_variant *variant, Q4kPlan *p) {
  if (!gate_up_one_family(variant) && reject_family(variant) != AXH_OK)
    return AXH_ERR_INVALID_ARGUMENT;
  if (sb_per_row == 0 || sb_per_row > kQ4kFlatMaxSb)
    return fail(AXH_ERR_INVALID_ARGUMENT, "gate/up: sb_per_row must be 1..128");
  if ((uint64_t)n_rows * sb_per_row * 144u >= 0xFFFFFFFFull)
    return fail(AXH_ERR_INVALID_ARGUMENT, "gate/up: each matrix must be below 4 GiB");
  if (gate_up_one_family(variant))
    return plan_gate_up_one("q4k", false, n_rows, sb_per_row, variant, p);
  axh_q4_variant one{};
  if (gate_up_default_one(variant, n_rows, (sb_per_row + 7u) / 8u, &one))
    return plan_gate_up_one("q4k", false, n_rows, sb_per_row, &one, p);
  if (variant && variant->nontemporal == 1)
    return fail(AXH_ERR_INVALID_ARGUMENT, "gate/up: no non-temporal variant is compiled");
  const MatvecVariant dflt = gate_up_default(n_rows, sb_per_row);
  const uint32_t want_nw =
      variant && variant->waves_per_workgroup ? variant->waves_per_workgroup : dflt.nw;
  const uint32_t min_xp = (sb_per_row * 8u + want_nw * 64u - 1u) / (want_nw * 64u);
  const MatvecVariant *v =
      find_variant(kGateUpVariants, sizeof(kGateUpVariants) / sizeof(kGateUpVariants[0]),
                   variant, dflt, min_xp);
  if (!v) return fail(AXH_ERR_INVALID_ARGUMENT, "no compiled gate/up variant matches");
  if (!staged_in_chunks(*v) && sb_per_row * 8u > v->xp * v->nw * 64u)
    return fail(AXH_ERR_INVALID_ARGUMENT, "gate/up: row too long for this variant's x staging");
  std::snprintf(p->name, sizeof(p->name), "axh_q4k_gate_up_r%u_w%u_p%u_x%u", v->rpw, v->nw,
                v->pf, v->xp);
  p->nw = v->nw;
  p->lds = sb_per_row * 1120u;
  p->flat = true;
  const uint32_t bundles = (n_rows + v->rpw - 1) / v->rpw;
  p->units = ((bundles + 1) / 2 + v->nw - 1) / v->nw;
  p->args = RowsArgs{n_rows, sb_per_row, sb_per_row, 0};
  return ok();
}

axh_status axh_q4k_gate_up_kernel_name(uint32_t n_rows, uint32_t sb_per_row,
                                       const axh_q4_variant *variant, char *buf, size_t cap) {
  if (!buf || cap == 0) return fail(AXH_ERR_INVALID_ARGUMENT, "buf is NULL");
  Q4kPlan p{};
  axh_status s = plan_gate_up(n_rows, sb_per_row, variant, &p);
  if (s != AXH_OK) return s;
  if (std::strlen(p.name) + 1 > cap) return fail(AXH_ERR_INVALID_ARGUMENT, "buf too small");
  std::memcpy(buf, p.name, std::strlen(p.name) + 1);
  return ok();
}

axh_status axh_q4k_gate_up(axh_context *ctx, const void *q_gate, const void *q_up,
                           const float *x, float *h, uint32_t n_rows, uint32_t sb_per_row,
                           const axh_q4_variant *variant, void *stream) {
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  if (n_rows == 0) return ok();
  if (!device_ptr_ok(h) || !device_ptr_ok(q_gate) || !device_ptr_ok(q_up) || !device_ptr_ok(x))
    return fail(AXH_ERR_INVALID_ARGUMENT, "q_gate, q_up, x and h must be device pointers");
  if (((uintptr_t)q_gate & 15u) || ((uintptr_t)q_up & 15u) || ((uintptr_t)x & 15u))
    return fail(AXH_ERR_INVALID_ARGUMENT, "q_gate, q_up and x must be 16-byte aligned");
  Q4kPlan p{};
  axh_status s = plan_gate_up(n_rows, sb_per_row, variant, &p);
  if (s != AXH_OK) return s;
  if (p.lds > ctx->core->max_lds)
    return fail(AXH_ERR_PIPELINE_LAYOUT, "LDS tile exceeds the device limit");
  hipSetDevice(ctx->core->device);
  axh_kernel *k = nullptr;
  s = builtin_kernel(ctx, p.name, 4, sizeof(RowsArgs), p.nw * 64u, &k);
  if (s != AXH_OK) return s;
  uint32_t grid[3] = {p.units, 1, 1};
  if (p.flat) { // persistent: at most one resident round of workgroups
    const uint32_t resident = occupancy(ctx, k, p.lds) * ctx->core->cu_count;
    if (resident < grid[0]) grid[0] = resident;
  }
  void *bufs[4] = {const_cast<void *>(q_gate), const_cast<void *>(q_up), const_cast<float *>(x),
                   h};
  s = launch_raw(k, grid, bufs, 4, &p.args, sizeof(p.args), p.lds, pick_stream(ctx, stream));
  return s == AXH_OK ? ok() : s;
}

// Fused gate/up over two Q5_K matrices.  With no hole set: the wave-paired
// one-pass kernel with x chunk by chunk up to 12288 rows of up to 8 steps
// (ahead of x staged whole at every size measured: 14336 x 4096 18.9 vs
// 20.1 us, 11008 x 4096 16.1 vs 16.7), else the persistent kernel with 4
// waves, x whole and two iterations in flight (28672 x 8192 58.4 us against
// 81.7 for the one-pass kernel and 2 x 32.7 for two Q5_K matvec calls;
// 13824 x 5120 23.7 against 24.8 and 2 x 14.5), early refill past 64
// superblocks.  The persistent holes and the one-pass families (family,
// sb_per_lane) select the others.
constexpr MatvecVariant kQ5GateUpVariants[] = {
    {1, 4, 1, 2, 1}, {1, 8, 1, 2, 1}, {1, 4, 2, 2, 1}, {1, 4, 2, 2, 2}};

static axh_status plan_q5k_gate_up(uint32_t n_rows, uint32_t sb_per_row,
                                   const axh_q4_variant *variant, Q4kPlan *p) {
  if (!gate_up_one_family(variant) && reject_family(variant) != AXH_OK)
    return AXH_ERR_INVALID_ARGUMENT;
  if (sb_per_row == 0 || sb_per_row > kQ4kFlatMaxSb)
    return fail(AXH_ERR_INVALID_ARGUMENT, "Q5_K gate/up: sb_per_row must be 1..128");
  if ((uint64_t)n_rows * sb_per_row * 176u >= 0xFFFFFFFFull)
    return fail(AXH_ERR_INVALID_ARGUMENT, "Q5_K gate/up: each matrix must be below 4 GiB");
  if (gate_up_one_family(variant))
    return plan_gate_up_one("q5k", false, n_rows, sb_per_row, variant, p);
  axh_q4_variant one{};
  if (gate_up_default_one(variant, n_rows, (sb_per_row + 7u) / 8u, &one)) {
    one.family = AXH_Q4K_FAMILY_ONE_PASS;
    return plan_gate_up_one("q5k", false, n_rows, sb_per_row, &one, p);
  }
  if (variant && variant->nontemporal == 1)
    return fail(AXH_ERR_INVALID_ARGUMENT, "Q5_K gate/up: no non-temporal variant is compiled");
  const MatvecVariant dflt =
      sb_per_row <= 64u ? MatvecVariant{1, 4, 2, 2, 1} : MatvecVariant{1, 4, 1, 2, 1};
  const uint32_t want_nw =
      variant && variant->waves_per_workgroup ? variant->waves_per_workgroup : dflt.nw;
  const uint32_t min_xp = (sb_per_row * 8u + want_nw * 64u - 1u) / (want_nw * 64u);
  const MatvecVariant *v = find_variant(
      kQ5GateUpVariants, sizeof(kQ5GateUpVariants) / sizeof(kQ5GateUpVariants[0]), variant, dflt,
      min_xp);
  if (!v) return fail(AXH_ERR_INVALID_ARGUMENT, "no compiled Q5_K gate/up variant matches");
  if (!staged_in_chunks(*v) && sb_per_row * 8u > v->xp * v->nw * 64u)
    return fail(AXH_ERR_INVALID_ARGUMENT,
                "Q5_K gate/up: row too long for this variant's x staging");
  std::snprintf(p->name, sizeof(p->name), "axh_q5k_gate_up_r%u_w%u_p%u_x%u", v->rpw, v->nw,
                v->pf, v->xp);
  p->nw = v->nw;
  p->lds = sb_per_row * 1120u;
  p->flat = true;
  const uint32_t bundles = (n_rows + v->rpw - 1) / v->rpw;
  p->units = ((bundles + 1) / 2 + v->nw - 1) / v->nw;
  p->args = RowsArgs{n_rows, sb_per_row, sb_per_row, 0};
  return ok();
}

axh_status axh_q5k_gate_up_kernel_name(uint32_t n_rows, uint32_t sb_per_row,
                                       const axh_q4_variant *variant, char *buf, size_t cap) {
  if (!buf || cap == 0) return fail(AXH_ERR_INVALID_ARGUMENT, "buf is NULL");
  Q4kPlan p{};
  axh_status s = plan_q5k_gate_up(n_rows, sb_per_row, variant, &p);
  if (s != AXH_OK) return s;
  if (std::strlen(p.name) + 1 > cap) return fail(AXH_ERR_INVALID_ARGUMENT, "buf too small");
  std::memcpy(buf, p.name, std::strlen(p.name) + 1);
  return ok();
}

axh_status axh_q5k_gate_up(axh_context *ctx, const void *q_gate, const void *q_up,
                           const float *x, float *h, uint32_t n_rows, uint32_t sb_per_row,
                           const axh_q4_variant *variant, void *stream) {
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  if (n_rows == 0) return ok();
  if (!device_ptr_ok(h) || !device_ptr_ok(q_gate) || !device_ptr_ok(q_up) || !device_ptr_ok(x))
    return fail(AXH_ERR_INVALID_ARGUMENT, "q_gate, q_up, x and h must be device pointers");
  if (((uintptr_t)q_gate & 15u) || ((uintptr_t)q_up & 15u) || ((uintptr_t)x & 15u))
    return fail(AXH_ERR_INVALID_ARGUMENT, "q_gate, q_up and x must be 16-byte aligned");
  Q4kPlan p{};
  axh_status s = plan_q5k_gate_up(n_rows, sb_per_row, variant, &p);
  if (s != AXH_OK) return s;
  if (p.lds > ctx->core->max_lds)
    return fail(AXH_ERR_PIPELINE_LAYOUT, "LDS tile exceeds the device limit");
  hipSetDevice(ctx->core->device);
  axh_kernel *k = nullptr;
  s = builtin_kernel(ctx, p.name, 4, sizeof(RowsArgs), p.nw * 64u, &k);
  if (s != AXH_OK) return s;
  uint32_t grid[3] = {p.units, 1, 1};
  if (p.flat) { // persistent: at most one resident round of workgroups
    const uint32_t resident = occupancy(ctx, k, p.lds) * ctx->core->cu_count;
    if (resident < grid[0]) grid[0] = resident;
  }
  void *bufs[4] = {const_cast<void *>(q_gate), const_cast<void *>(q_up), const_cast<float *>(x),
                   h};
  s = launch_raw(k, grid, bufs, 4, &p.args, sizeof(p.args), p.lds, pick_stream(ctx, stream));
  return s == AXH_OK ? ok() : s;
}

// ---- Q5_K / Q6_K (persistent kernels; one-pass kernels for short rows) -----
struct KqFormat {
  const char *prefix;            // kernel name prefix
  const char *one_prefix;        // the one-pass kernels' name prefix
  const MatvecVariant *table;
  size_t n;
  uint32_t sb_bytes, lds_per_sb; // superblock bytes, LDS bytes per superblock of x
  bool chunked_early;            // prefetch-1 kernels stage x in chunks (any row fits)
};

static const KqFormat kQ5kFormat{"axh_q5k_matvec_flat", "axh_q5k_matvec_one", kQ5kVariants,
                                 sizeof(kQ5kVariants) / sizeof(kQ5kVariants[0]), 176u, 1120u,
                                 true};
static const KqFormat kQ6kFormat{"axh_q6k_matvec_flat", "axh_q6k_matvec_one", kQ6kVariants,
                                 sizeof(kQ6kVariants) / sizeof(kQ6kVariants[0]), 210u, 1152u,
                                 false};

// Early refill (prefetch 1) where the format's kernel can stage the row's x:
// Q5_K 14336 x 4096 10.6-10.9 vs 11.3-11.4 us; Q6_K 4096 x 14336 12.5 vs
// 13.4-13.9 us, 128256 x 4096 90.0-90.6 vs 90.9-92.0 us.  The Q6_K kernel
// stages x whole, one sub-block per thread with its prefetch-1 variants.
//
// Q6_K rows of 17-32 superblocks on at most 1024 rows (at most half the CUs
// get a workgroup) keep x staged whole and two iterations in flight instead:
// A/B in one run, us per call, prefetch 2 vs early refill: 512 x 8192 5.87
// vs 6.21, 1024 x 8192 (Llama-2-70B attn_v) 5.81 vs 6.13, 1024 x 6144 5.03
// vs 5.57; from 2048 rows early refill stays ahead (early refill vs
// prefetch 2: 2048 x 8192 6.39 vs 6.45, 4096 x 8192 7.87 vs 8.16).  The same
// holds for Q5_K rows of up to 32 superblocks (its one-pass kernel starts at
// 2048 rows): 1024 x 4096 3.46 vs 3.57 us, 1024 x 8192 5.10 vs 5.38.
constexpr uint32_t kKqFewRows = 1024;

// Rows of 17-64 superblocks on at most 2048 rows, and of 33-64 on 14336 rows
// and more, take 4 waves with x staged whole and two iterations in flight
// (the _x2 kernels past 32 superblocks).  A/B in one run, us per call, Q5_K /
// Q6_K, against 8 waves with early refill: 1024 x 14336 7.32 vs 9.51 / 9.10
// vs 10.71, 2048 x 10240 6.41 vs 7.60 / 7.51 vs 8.69, 2048 x 6144 4.71 vs
// 5.06 (early refill, 4 waves) / 5.39 vs 5.66, 14336 x 14336 27.7 vs 31.3 /
// 34.7 vs 37.6, 14336 x 10240 21.7 vs 23.5 / 24.8 vs 25.6; not at 4096 rows
// (Q6_K 4096 x 14336 13.1 vs 11.5) nor on 14336 rows of 24 superblocks (Q6_K
// 16.8 vs 16.3).
constexpr uint32_t kKqW4MaxRows = 2048, kKqW4TallMinRows = 14336;

static MatvecVariant kq_default(const KqFormat &f, uint32_t n_rows, uint32_t nsb) {
  const uint32_t nw = nsb * 8u <= 256u ? 4u : 8u;
  const bool early = f.chunked_early || nsb * 8u <= nw * 64u;
  const bool few = n_rows <= kKqFewRows && nsb <= 32u && (&f == &kQ5kFormat || nsb > 16u);
  const bool w4 = nsb > 16u && nsb <= 64u &&
                  (n_rows <= kKqW4MaxRows || (n_rows >= kKqW4TallMinRows && nsb > 32u));
  if (few || w4) return {1, 4, 2, 2, 1}; // the _x2 kernel where the row needs it
  return {1, nw, early ? 1u : 2u, 2, 1};
}

// Q5_K rows of up to 16 superblocks over 768 to 32768 rows take the
// one-pass kernel (axh_q5k_matvec_one_i{NIT}: one workgroup per 16 rows, x
// staged chunk by chunk, fully unrolled).  A/B in one run, 14336 x 4096:
// 10.02-10.08 vs 10.56-10.70 us (plain launches, one weight copy per call
// from 14 rotated copies), 10.71 vs 11.05 on another box, and 10.79-10.88 vs
// 10.92-10.96 through the library's launch loop on a third, and even in the
// kernel trace on a fourth (10.85-10.90 vs 10.84-10.88); 4096 x 4096 4.60 vs
// 4.70; from 768 rows in two repetitions
// in one run: 768 x 4096 3.88 / 4.01 vs 4.15 / 4.30, 1024 x 4096 4.11 / 4.13
// vs 4.30 / 4.53, 1024 x 2048 3.19 / 3.18 vs 4.14 / 4.09, 1536 x 4096 4.10 /
// 4.14 vs 4.35 / 4.28, 1900 x 4096 4.25 / 4.19 vs 4.53 / 4.55 (an earlier box
// had 1024 x 4096 at 3.95 vs 3.49); not below (512 x 4096 3.72 vs 3.57, 256
// x 4096 3.57 vs 3.36) nor for longer rows (4096 x 14336: even).  The family is also reachable as
// variant->family = AXH_Q4K_FAMILY_ONE_PASS (hole: sb_per_lane, 1 or 2).
constexpr uint32_t kQ5OneMinRows = 768, kQ5OneMaxRows = 32768, kKqOneMaxSb = 16;
constexpr uint32_t kKqOneMaxIt = 8; // one-pass kernels compiled for 1-8 steps

// Q6_K rows of up to 16 superblocks over 256 to 4096 rows (at most one
// workgroup per CU) take the one-pass kernel too (axh_q6k_matvec_one_i{NIT}).
// A/B in one run, us per call through the library's launch loop, one-pass vs
// persistent: 256 x 4096 4.05 vs 4.74, 512 x 4096 4.56 vs 4.65, 1024 x 4096
// 4.62 vs 4.85, 2048 x 4096 4.85 vs 5.00, 4096 x 4096 5.44 vs 5.90, 4096 x
// 3072 5.21 vs 5.38, 4096 x 2048 3.72 vs 4.30, 1024 x 2048 3.24 vs 4.08; but
// 6144 x 4096 7.28 vs 6.91 and 14336 x 4096 12.08 vs 11.95.
constexpr uint32_t kQ6OneMinRows = 256, kQ6OneMaxRows = 4096;

// Longer rows take the one-pass kernel past 2048 rows too: Q5_K 2049-4096
// rows of 17-64 superblocks (4096 x 6144 5.67 vs 6.49 us, 4096 x 10240 7.84 vs
// 8.18, 4096 x 14336 10.10 vs 10.46, 4096 x 16384 11.03 vs 11.55; 8192 x
// 10240 14.8 vs 14.6 stays persistent), Q6_K 2049-8192 rows of 17-40 (4096 x
// 6144 6.59 vs 7.26, 4096 x 10240 9.15 vs 9.49, 8192 x 6144 10.52 vs 11.06,
// 8192 x 10240 15.24 vs 15.71; 4096 x 14336 11.79 vs 11.52 stays persistent).
// At 2048 rows the 4-wave persistent kernel stays ahead (Q5_K 2048 x 14336
// 7.64 vs 9.18).
constexpr uint32_t kKqOneLongMinRows = 2049, kQ5OneLongMaxRows = 4096, kQ6OneLongMaxRows = 8192;
constexpr uint32_t kQ5OneLongMaxSb = 64, kQ6OneLongMaxSb = 40;

static bool kq_one_long(const KqFormat &f, uint32_t n_rows, uint32_t nsb) {
  const bool q5 = &f == &kQ5kFormat;
  return n_rows >= kKqOneLongMinRows && nsb > kKqOneMaxSb &&
         n_rows <= (q5 ? kQ5OneLongMaxRows : kQ6OneLongMaxRows) &&
         nsb <= (q5 ? kQ5OneLongMaxSb : kQ6OneLongMaxSb);
}

static axh_status plan_kq(const KqFormat &f, uint32_t n_rows, uint32_t sb_per_row,
                          const axh_q4_variant *variant, Q4kPlan *p) {
  const bool q5 = &f == &kQ5kFormat;
  const uint32_t fam = variant ? variant->family : 0u;
  const bool flat_holes = variant && (variant->rows_per_wave || variant->waves_per_workgroup ||
                                      variant->prefetch || variant->nontemporal);
  if (fam != AXH_Q4K_FAMILY_ONE_PASS && reject_family(variant) != AXH_OK)
    return AXH_ERR_INVALID_ARGUMENT;
  if (sb_per_row == 0 || sb_per_row > kQ4kFlatMaxSb)
    return fail(AXH_ERR_INVALID_ARGUMENT, "sb_per_row must be 1..128 for Q5_K / Q6_K");
  if ((uint64_t)n_rows * sb_per_row * f.sb_bytes >= 0xFFFFFFFFull)
    return fail(AXH_ERR_INVALID_ARGUMENT, "Q5_K / Q6_K matrices must be below 4 GiB");
  const uint32_t one_min = q5 ? kQ5OneMinRows : kQ6OneMinRows;
  const uint32_t one_max = q5 ? kQ5OneMaxRows : kQ6OneMaxRows;
  if (fam == AXH_Q4K_FAMILY_ONE_PASS ||
      (!flat_holes && ((n_rows >= one_min && n_rows <= one_max && sb_per_row <= kKqOneMaxSb) ||
                       kq_one_long(f, n_rows, sb_per_row)))) {
    const uint32_t xd = variant ? variant->prefetch : 0u;
    if (variant && (variant->rows_per_wave || variant->waves_per_workgroup ||
                    variant->nontemporal || xd > 2u))
      return fail(AXH_ERR_INVALID_ARGUMENT,
                  "the Q5_K / Q6_K one-pass family's holes are sb_per_lane and prefetch (x one "
                  "or two chunks ahead)");
    const uint32_t need = (sb_per_row + 7u) / 8u;
    const uint32_t nit = variant && variant->sb_per_lane ? variant->sb_per_lane : need;
    if (nit < need || nit > kKqOneMaxIt)
      return fail(AXH_ERR_INVALID_ARGUMENT,
                  "Q5_K / Q6_K one-pass: sb_per_lane must cover the row and be at most 8 (rows "
                  "of up to 64 superblocks)");
    if (xd == 2u && nit < 3u)
      return fail(AXH_ERR_INVALID_ARGUMENT, "x two chunks ahead needs three or more steps");
    std::snprintf(p->name, sizeof(p->name), "%s%s_i%u", f.one_prefix, xd == 2u ? "p" : "", nit);
    p->nw = 8;
    p->lds = sb_per_row * f.lds_per_sb;
    p->flat = false; // one workgroup per 16 rows, all of them launched
    p->units = (n_rows + 15u) / 16u;
    p->args = RowsArgs{n_rows, sb_per_row, sb_per_row, 0};
    return ok();
  }
  if (variant && variant->nontemporal == 1)
    return fail(AXH_ERR_INVALID_ARGUMENT, "no non-temporal Q5_K / Q6_K variant is compiled");
  const MatvecVariant dflt = kq_default(f, n_rows, sb_per_row);
  const uint32_t want_nw =
      variant && variant->waves_per_workgroup ? variant->waves_per_workgroup : dflt.nw;
  const uint32_t min_xp = (sb_per_row * 8u + want_nw * 64u - 1u) / (want_nw * 64u);
  const MatvecVariant *v = find_variant(f.table, f.n, variant, dflt, min_xp);
  if (!v) return fail(AXH_ERR_INVALID_ARGUMENT, "no compiled Q5_K / Q6_K variant matches");
  if (!(f.chunked_early && staged_in_chunks(*v)) && sb_per_row * 8u > v->xp * v->nw * 64u)
    return fail(AXH_ERR_INVALID_ARGUMENT, "row too long for this variant's x staging");
  std::snprintf(p->name, sizeof(p->name), "%s_r%u_w%u_p%u_x%u", f.prefix, v->rpw, v->nw, v->pf,
                v->xp);
  p->nw = v->nw;
  p->lds = sb_per_row * f.lds_per_sb;
  p->flat = true;
  const uint32_t bundles = (n_rows + v->rpw - 1) / v->rpw;
  p->units = ((bundles + 1) / 2 + v->nw - 1) / v->nw;
  p->args = RowsArgs{n_rows, sb_per_row, sb_per_row, 0};
  return ok();
}

static axh_status kq_kernel_name(const KqFormat &f, uint32_t n_rows, uint32_t sb_per_row,
                                 const axh_q4_variant *variant, char *buf, size_t cap) {
  if (!buf || cap == 0) return fail(AXH_ERR_INVALID_ARGUMENT, "buf is NULL");
  Q4kPlan p{};
  axh_status s = plan_kq(f, n_rows, sb_per_row, variant, &p);
  if (s != AXH_OK) return s;
  if (std::strlen(p.name) + 1 > cap) return fail(AXH_ERR_INVALID_ARGUMENT, "buf too small");
  std::memcpy(buf, p.name, std::strlen(p.name) + 1);
  return ok();
}

static axh_status kq_matvec(const KqFormat &f, axh_context *ctx, const void *q, const float *x,
                            float *y, uint32_t n_rows, uint32_t sb_per_row,
                            const axh_q4_variant *variant, void *stream) {
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  if (n_rows == 0) return ok();
  if (!device_ptr_ok(y) || !device_ptr_ok(q) || !device_ptr_ok(x))
    return fail(AXH_ERR_INVALID_ARGUMENT, "q, x and y must be device pointers");
  if (((uintptr_t)q & 15u) || ((uintptr_t)x & 15u))
    return fail(AXH_ERR_INVALID_ARGUMENT, "q and x must be 16-byte aligned");
  Q4kPlan p{};
  axh_status s = plan_kq(f, n_rows, sb_per_row, variant, &p);
  if (s != AXH_OK) return s;
  if (p.lds > ctx->core->max_lds)
    return fail(AXH_ERR_PIPELINE_LAYOUT, "LDS tile exceeds the device limit");
  hipSetDevice(ctx->core->device);
  axh_kernel *k = nullptr;
  s = builtin_kernel(ctx, p.name, 3, sizeof(RowsArgs), p.nw * 64u, &k);
  if (s != AXH_OK) return s;
  uint32_t grid[3] = {p.units, 1, 1};
  if (p.flat) { // persistent: at most one resident round of workgroups
    const uint32_t resident = occupancy(ctx, k, p.lds) * ctx->core->cu_count;
    if (resident < grid[0]) grid[0] = resident;
  }
  void *bufs[3] = {const_cast<void *>(q), const_cast<float *>(x), y};
  s = launch_raw(k, grid, bufs, 3, &p.args, sizeof(p.args), p.lds, pick_stream(ctx, stream));
  return s == AXH_OK ? ok() : s;
}

axh_status axh_q5k_matvec(axh_context *ctx, const void *q, const float *x, float *y,
                          uint32_t n_rows, uint32_t sb_per_row, const axh_q4_variant *variant,
                          void *stream) {
  return kq_matvec(kQ5kFormat, ctx, q, x, y, n_rows, sb_per_row, variant, stream);
}

axh_status axh_q6k_matvec(axh_context *ctx, const void *q, const float *x, float *y,
                          uint32_t n_rows, uint32_t sb_per_row, const axh_q4_variant *variant,
                          void *stream) {
  return kq_matvec(kQ6kFormat, ctx, q, x, y, n_rows, sb_per_row, variant, stream);
}

axh_status axh_q5k_matvec_kernel_name(uint32_t n_rows, uint32_t sb_per_row,
                                      const axh_q4_variant *variant, char *buf, size_t cap) {
  return kq_kernel_name(kQ5kFormat, n_rows, sb_per_row, variant, buf, cap);
}

axh_status axh_q6k_matvec_kernel_name(uint32_t n_rows, uint32_t sb_per_row,
                                      const axh_q4_variant *variant, char *buf, size_t cap) {
  return kq_kernel_name(kQ6kFormat, n_rows, sb_per_row, variant, buf, cap);
}

uint32_t axh_q5k_matvec_variant_count(void) { return count_holes(kQ5kVariants, kQ5kFormat.n); }
axh_status axh_q5k_matvec_variant_at(uint32_t i, axh_q4_variant *out) {
  return holes_at(kQ5kVariants, kQ5kFormat.n, i, out);
}
uint32_t axh_q6k_matvec_variant_count(void) { return count_holes(kQ6kVariants, kQ6kFormat.n); }
axh_status axh_q6k_matvec_variant_at(uint32_t i, axh_q4_variant *out) {
  return holes_at(kQ6kVariants, kQ6kFormat.n, i, out);
}

axh_status axh_matvec_ggml(axh_context *ctx, uint32_t ggml_type, const void *q, const float *x,
                           float *y, uint32_t n_rows, uint64_t n_cols, void *stream) {
  const uint32_t block = ggml_type == AXH_GGML_Q4_0 ? 32u : 256u;
  if (n_cols % block != 0)
    return fail(AXH_ERR_INVALID_ARGUMENT, "n_cols must be a whole number of blocks");
  if (n_cols / block > 0xFFFFFFFFull) return fail(AXH_ERR_INVALID_ARGUMENT, "n_cols too large");
  const uint32_t units = (uint32_t)(n_cols / block);
  switch (ggml_type) {
  case AXH_GGML_Q4_0:
    return axh_q4_0_matvec(ctx, q, x, y, n_rows, units, nullptr, stream);
  case AXH_GGML_Q4_K:
    return axh_q4k_matvec(ctx, q, x, y, n_rows, units, nullptr, stream);
  case AXH_GGML_Q5_K:
    return axh_q5k_matvec(ctx, q, x, y, n_rows, units, nullptr, stream);
  case AXH_GGML_Q6_K:
    return axh_q6k_matvec(ctx, q, x, y, n_rows, units, nullptr, stream);
  default:
    return fail(AXH_ERR_INVALID_ARGUMENT, "unsupported ggml type for matvec");
  }
}

// The Q4_0 column kernel takes rows of at most 128 blocks, an even count
// (lane = block pair, x in VGPRs, one row per batch: measured 2.7 us at 256 x
// 4096 against 3.3 us for two or four rows per batch).
constexpr uint32_t kQ4_0ColsMaxB = 128;
constexpr uint32_t kQ4_0ColsRb = 1;

static bool q4_0_cols_fit(uint32_t n_rows, uint32_t nb) {
  return nb >= 2 && nb <= kQ4_0ColsMaxB && (nb & 1u) == 0 &&
         (uint64_t)n_rows * nb * 18u < 0xFFFFFF00ull;
}

// The persistent and one-pass kernels read a row as octets of 8 blocks (the
// Q4_K kernels' layout, 1120 bytes of LDS per octet of x): rows of an even
// block count (every quarter-octet 4-byte aligned), at most 1024 blocks,
// matrices below 4 GiB.
constexpr uint32_t kQ4_0MaxOctets = 128;
constexpr uint32_t kQ4_0OneMaxIt = 16; // one-pass kernels: 1-16 steps of 64 blocks

static bool q4_0_octets_fit(uint32_t n_rows, uint32_t nb) {
  return nb >= 2 && (nb & 1u) == 0 && (nb + 7u) / 8u <= kQ4_0MaxOctets &&
         (uint64_t)n_rows * nb * 18u < 0xFFFFFFFFull;
}

// Persistent Q4_0 default: one row per bundle, 8 waves, early refill (A/B in
// one run, us per call: 28672 x 448 blocks 42.5 vs 47.8 for 4 waves and 42.9
// for prefetch 2; 4096 x 1024 16.1 vs 27.4 for 4 waves).
static MatvecVariant q4_0_flat_default(uint32_t n_rows, uint32_t nb) {
  (void)n_rows;
  (void)nb;
  return {1, 8, 1, 2, 1};
}

// Default Q4_0 family per shape, from A/B runs (interleaved launch loops, us
// per call, rotated weights; the LDS-tiled kernel's figures are its best row
// count):
// - fewer than 32 rows: tiled, one row per wave, ahead of the column kernel
//   on every shape it takes (interleaved in one run: 1 x 128 blocks 3.33 vs
//   4.21, 3 x 128 3.31 vs 3.91, 8 x 128 2.59 vs 2.71, 16 x 128 3.30 vs 3.87,
//   31 x 128 3.21 vs 3.93, 31 x 32 3.16 vs 3.79, 8 x 16 3.24 vs 4.08, 24 x 100
//   3.18 vs 3.97) and of the one pass on longer rows (16 x 1024 blocks 11.4
//   vs 12.3, 8 x 344 4.90 vs 4.91);
// - 32-1024 rows of at most 128 blocks: tiled, one row per wave, ahead of
//   the column kernel per call in loops of every length (interleaved in one
//   run: 256 x 128 blocks 3.11 vs 3.32 us over 1000 calls, 3.08 vs 4.07 over
//   100, 3.32 vs 3.81 over 20; 512 x 112 3.11 vs 3.34 over 1000) and of the
//   one pass (3.26 over 1000; 640 x 112 2.90 vs 3.08, 1024 x 128 3.22 vs
//   3.36, 1024 x 96 3.27 vs 3.39, 513 x 128 3.21 vs 3.24, 1024 x 64 3.10 vs
//   3.15; 2048 x 128 3.88 vs 3.69 stays one pass), though the column kernel's
//   dispatches are shorter in the kernel trace (2.76 against 3.48 us);
// - 32-256 rows of 193-256 blocks (four one-pass steps): tiled, ahead of the
//   one pass and of the one pass with x two chunks ahead (32 x 256 3.96 vs
//   4.33, 128 x 256 4.04 vs 4.39, 256 x 256 4.09 vs 4.67 and 4.77, 256 x 224
//   4.00 vs 4.60, 256 x 200 3.94 vs 5.12, 128 x 240 4.00 vs 4.37); even at 256
//   x 192 (3.85 vs 3.86), 384 x 256 and 512 x 224, behind from 1024 rows
//   (2048 x 256 5.87 vs 4.96) and at 256 x 320 (5.95 vs 5.40);
// - one pass from 32 rows (the Q4_K one-pass kernel over octets): 4096 x 448
//   8.1 vs 13.7 tiled, 14336 x 448 24.0 vs 40.8, 4096 x 128 3.9 vs 4.7 tiled
//   and 6.0 column, 1024 x 1024 13.5 vs 14.0, 256 x 160 3.8 vs 4.3; x staged
//   whole for rows of 65-128 blocks from 6144 rows (8192 x 128 5.22 vs 5.53,
//   14336 x 128 8.34 vs 8.71, 128256 x 128 49.7 vs 50.8; 4096 x 128 4.01 vs
//   3.93), x two chunks ahead for 14-16 steps from 4096 rows (4096 x 1024
//   15.9 vs 16.5, 8192 x 1024 31.3 vs 31.6; below 14 steps it runs even:
//   4096 x 14336 8.19 vs 8.21, 4096 x 12288 7.63 vs 7.39, 4096 x 26624 13.67
//   vs 13.70);
// - persistent for more than 16384 rows of more than 256 blocks (28672 x 448
//   42.5 vs 44.1-44.7 one pass; 28672 x 256 25.3 vs 24.7 stays one pass).
constexpr uint32_t kQ4_0TiledShortMaxRows = 1024, kQ4_0TiledShortMaxB = 128, kQ4_0FewRows = 32;
constexpr uint32_t kQ4_0TiledMidMaxRows = 256, kQ4_0TiledMidMinB = 193, kQ4_0TiledMidMaxB = 256;
constexpr uint32_t kQ4_0OneXMinRows = 6144;
constexpr uint32_t kQ4_0OnePMinIt = 14, kQ4_0OnePMinRows = 4096;
constexpr uint32_t kQ4_0FlatMinRows = 16385, kQ4_0FlatMinB = 257;

static uint32_t q4_0_default_family(uint32_t n_rows, uint32_t nb) {
  if (n_rows < kQ4_0FewRows) return AXH_Q4K_FAMILY_TILED;
  if (n_rows <= kQ4_0TiledShortMaxRows && nb <= kQ4_0TiledShortMaxB) return AXH_Q4K_FAMILY_TILED;
  if (n_rows <= kQ4_0TiledMidMaxRows && nb >= kQ4_0TiledMidMinB && nb <= kQ4_0TiledMidMaxB)
    return AXH_Q4K_FAMILY_TILED;
  if (!q4_0_octets_fit(n_rows, nb)) return AXH_Q4K_FAMILY_TILED;
  if (n_rows >= kQ4_0FlatMinRows && nb >= kQ4_0FlatMinB) return AXH_Q4K_FAMILY_PERSISTENT;
  if ((nb + 63u) / 64u == 2u && n_rows >= kQ4_0OneXMinRows) return AXH_Q4K_FAMILY_ONE_PASS_X;
  return AXH_Q4K_FAMILY_ONE_PASS;
}

// Kernel, LDS and grid of one Q4_0 matvec call.  family 0 with a hole set
// means the LDS-tiled kernel (axh_q4_0_matvec_r*_w*), the only family with
// holes before the others were built; with no hole set, the shape's default.
static axh_status plan_q4_0(uint32_t n_rows, uint32_t nb, const axh_q4_variant *variant,
                            Q4kPlan *p) {
  const bool holes = variant && (variant->rows_per_wave || variant->waves_per_workgroup ||
                                 variant->prefetch || variant->nontemporal);
  uint32_t fam = variant ? variant->family : 0u;
  if (variant && variant->sb_per_lane && fam != AXH_Q4K_FAMILY_ONE_PASS &&
      fam != AXH_Q4K_FAMILY_ONE_PASS_X)
    return fail(AXH_ERR_INVALID_ARGUMENT, "sb_per_lane is a hole of the one-pass families only");
  if (fam == AXH_Q4K_FAMILY_DEFAULT)
    fam = holes ? AXH_Q4K_FAMILY_TILED : q4_0_default_family(n_rows, nb);
  const uint32_t n_oct = (nb + 7u) / 8u;
  switch (fam) {
  case AXH_Q4K_FAMILY_COLUMNS: {
    if (holes) return fail(AXH_ERR_INVALID_ARGUMENT, "the column family has no holes");
    if (!q4_0_cols_fit(n_rows, nb))
      return fail(AXH_ERR_INVALID_ARGUMENT,
                  "the Q4_0 column family takes rows of 2-128 blocks, an even count");
    std::snprintf(p->name, sizeof(p->name), "axh_q4_0_matvec_cols_r%u", kQ4_0ColsRb);
    const uint32_t n_batches = (n_rows + kQ4_0ColsRb - 1) / kQ4_0ColsRb;
    p->nw = 1;
    p->lds = 0;
    p->flat = false;
    p->units = n_batches < 2048u ? n_batches : 2048u;
    p->args = RowsArgs{n_rows, nb, 0, 0};
    return ok();
  }
  case AXH_Q4K_FAMILY_PERSISTENT: {
    if (variant && variant->nontemporal == 1)
      return fail(AXH_ERR_INVALID_ARGUMENT, "no non-temporal Q4_0 variant is compiled");
    if (!q4_0_octets_fit(n_rows, nb))
      return fail(AXH_ERR_INVALID_ARGUMENT,
                  "the Q4_0 persistent family takes rows of 2-1024 blocks, an even count, "
                  "below 4 GiB");
    const MatvecVariant dflt = q4_0_flat_default(n_rows, nb);
    const uint32_t want_nw =
        variant && variant->waves_per_workgroup ? variant->waves_per_workgroup : dflt.nw;
    const uint32_t min_xp = (nb + want_nw * 64u - 1u) / (want_nw * 64u);
    const MatvecVariant *v =
        find_variant(kQ4_0FlatVariants, sizeof(kQ4_0FlatVariants) / sizeof(kQ4_0FlatVariants[0]),
                     variant, dflt, min_xp);
    if (!v) return fail(AXH_ERR_INVALID_ARGUMENT, "no compiled Q4_0 persistent variant matches");
    if (!staged_in_chunks(*v) && nb > v->xp * v->nw * 64u)
      return fail(AXH_ERR_INVALID_ARGUMENT, "row too long for this variant's x staging");
    std::snprintf(p->name, sizeof(p->name), "axh_q4_0_matvec_flat_r%u_w%u_p%u_x%u", v->rpw,
                  v->nw, v->pf, v->xp);
    p->nw = v->nw;
    p->lds = n_oct * 1120u;
    p->flat = true;
    const uint32_t bundles = (n_rows + v->rpw - 1) / v->rpw;
    p->units = ((bundles + 1) / 2 + v->nw - 1) / v->nw;
    p->args = RowsArgs{n_rows, nb, nb, 0};
    return ok();
  }
  case AXH_Q4K_FAMILY_ONE_PASS:
  case AXH_Q4K_FAMILY_ONE_PASS_X: {
    const uint32_t xd = variant ? variant->prefetch : 0u;
    if (variant && (variant->rows_per_wave || variant->waves_per_workgroup || variant->nontemporal))
      return fail(AXH_ERR_INVALID_ARGUMENT,
                  "the one-pass families' holes are sb_per_lane and (one pass) prefetch");
    if (xd && (fam == AXH_Q4K_FAMILY_ONE_PASS_X || xd > 2u))
      return fail(AXH_ERR_INVALID_ARGUMENT,
                  "one-pass prefetch is 1 or 2 x chunks ahead (none for the whole-x kernel)");
    if (!q4_0_octets_fit(n_rows, nb))
      return fail(AXH_ERR_INVALID_ARGUMENT,
                  "the Q4_0 one-pass families take rows of 2-1024 blocks, an even count, "
                  "below 4 GiB");
    const uint32_t need = (nb + 63u) / 64u;
    const uint32_t nit = variant && variant->sb_per_lane ? variant->sb_per_lane : need;
    if (nit < need || nit > kQ4_0OneMaxIt)
      return fail(AXH_ERR_INVALID_ARGUMENT,
                  "Q4_0 one pass: sb_per_lane (steps of 64 blocks) must cover the row and be at "
                  "most 16");
    if (xd == 2u && nit < 3u)
      return fail(AXH_ERR_INVALID_ARGUMENT, "x two chunks ahead needs three or more steps");
    const bool two_ahead = fam == AXH_Q4K_FAMILY_ONE_PASS &&
                           (xd == 2u || (xd == 0u && nit >= kQ4_0OnePMinIt &&
                                         n_rows >= kQ4_0OnePMinRows));
    std::snprintf(p->name, sizeof(p->name), "axh_q4_0_matvec_one%s_i%u",
                  fam == AXH_Q4K_FAMILY_ONE_PASS_X ? "x" : two_ahead ? "p" : "", nit);
    p->nw = 8;
    p->lds = n_oct * 1120u;
    p->flat = false; // one workgroup per 16 rows, all of them launched
    p->units = (n_rows + 15u) / 16u;
    p->args = RowsArgs{n_rows, nb, nb, 0};
    return ok();
  }
  case AXH_Q4K_FAMILY_TILED: {
    axh_q4_variant vv{};
    if (variant) vv = *variant;
    vv.prefetch = 1; // prefetch and cache policy are not holes of this kernel
    vv.nontemporal = 2;
    const MatvecVariant *v = find_variant(kQ4_0Variants, axh_q4_0_matvec_variant_count(), &vv,
                                          q4_0_default(n_rows, nb));
    if (!v) return fail(AXH_ERR_INVALID_ARGUMENT, "no compiled Q4_0 matvec variant matches");
    std::snprintf(p->name, sizeof(p->name), "axh_q4_0_matvec_r%u_w%u", v->rpw, v->nw);
    uint32_t tile = (nb + 127u) & ~127u;
    if (tile == 0) tile = 128;
    if (tile > kQ4_0MaxTileB) tile = kQ4_0MaxTileB;
    p->nw = v->nw;
    p->lds = tile * 132u;
    p->flat = false;
    const uint32_t rows_per_wg = v->rpw * v->nw;
    p->units = (n_rows + rows_per_wg - 1) / rows_per_wg;
    p->args = RowsArgs{n_rows, nb, tile, 0};
    return ok();
  }
  default:
    return fail(AXH_ERR_INVALID_ARGUMENT,
                "Q4_0 takes the persistent, one-pass, column and tiled families");
  }
}

axh_status axh_q4_0_matvec_kernel_name(uint32_t n_rows, uint32_t blocks_per_row,
                                       const axh_q4_variant *variant, char *buf, size_t cap) {
  if (!buf || cap == 0) return fail(AXH_ERR_INVALID_ARGUMENT, "buf is NULL");
  Q4kPlan p{};
  axh_status s = plan_q4_0(n_rows, blocks_per_row, variant, &p);
  if (s != AXH_OK) return s;
  if (std::strlen(p.name) + 1 > cap) return fail(AXH_ERR_INVALID_ARGUMENT, "buf too small");
  std::memcpy(buf, p.name, std::strlen(p.name) + 1);
  return ok();
}

axh_status axh_q4_0_matvec(axh_context *ctx, const void *q, const float *x, float *y,
                           uint32_t n_rows, uint32_t blocks_per_row,
                           const axh_q4_variant *variant, void *stream) {
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  if (n_rows == 0) return ok();
  if (!device_ptr_ok(y) || (blocks_per_row && (!device_ptr_ok(q) || !device_ptr_ok(x))))
    return fail(AXH_ERR_INVALID_ARGUMENT, "q, x and y must be device pointers");
  if ((uint64_t)blocks_per_row * 32u > 0xFFFFFFFFull)
    return fail(AXH_ERR_INVALID_ARGUMENT, "blocks_per_row too large");
  if (((uintptr_t)q & 3u) || ((uintptr_t)x & 15u))
    return fail(AXH_ERR_INVALID_ARGUMENT, "q must be 4-byte and x 16-byte aligned");
  Q4kPlan p{};
  axh_status s = plan_q4_0(n_rows, blocks_per_row, variant, &p);
  if (s != AXH_OK) return s;
  if (p.lds > ctx->core->max_lds)
    return fail(AXH_ERR_PIPELINE_LAYOUT, "LDS tile exceeds the device limit");
  hipSetDevice(ctx->core->device);
  axh_kernel *k = nullptr;
  s = builtin_kernel(ctx, p.name, 3, sizeof(RowsArgs), p.nw * 64u, &k);
  if (s != AXH_OK) return s;
  uint32_t grid[3] = {p.units, 1, 1};
  if (p.flat) { // persistent: at most kQ4_0FlatRounds rounds of resident workgroups
    const uint32_t resident = kQ4_0FlatRounds * occupancy(ctx, k, p.lds) * ctx->core->cu_count;
    if (resident < grid[0]) grid[0] = resident;
  }
  void *bufs[3] = {const_cast<void *>(q), const_cast<float *>(x), y};
  s = launch_raw(k, grid, bufs, 3, &p.args, sizeof(p.args), p.lds, pick_stream(ctx, stream));
  return s == AXH_OK ? ok() : s;
}

// Fused gate/up over two Q4_0 matrices: the persistent kernel over octets of
// 8 blocks (rows of an even block count up to 1024 blocks).
static MatvecVariant q4_0_gate_up_default(uint32_t n_rows, uint32_t nb) {
  (void)n_rows;
  (void)nb;
  return {1, 4, 1, 2, 1};
}

static axh_status plan_q4_0_gate_up(uint32_t n_rows, uint32_t nb, const axh_q4_variant *variant,
                                    Q4kPlan *p) {
  if (!gate_up_one_family(variant) && reject_family(variant) != AXH_OK)
    return AXH_ERR_INVALID_ARGUMENT;
  if (!q4_0_octets_fit(n_rows, nb))
    return fail(AXH_ERR_INVALID_ARGUMENT,
                "Q4_0 gate/up: rows of 2-1024 blocks, an even count, each matrix below 4 GiB");
  if (gate_up_one_family(variant)) return plan_gate_up_one("q4_0", true, n_rows, nb, variant, p);
  axh_q4_variant one{};
  if (gate_up_default_one(variant, n_rows, (nb + 63u) / 64u, &one))
    return plan_gate_up_one("q4_0", true, n_rows, nb, &one, p);
  if (variant && variant->nontemporal == 1)
    return fail(AXH_ERR_INVALID_ARGUMENT, "Q4_0 gate/up: no non-temporal variant is compiled");
  const MatvecVariant dflt = q4_0_gate_up_default(n_rows, nb);
  const uint32_t want_nw =
      variant && variant->waves_per_workgroup ? variant->waves_per_workgroup : dflt.nw;
  const uint32_t min_xp = (nb + want_nw * 64u - 1u) / (want_nw * 64u);
  const MatvecVariant *v = find_variant(
      kQ4_0GateUpVariants, sizeof(kQ4_0GateUpVariants) / sizeof(kQ4_0GateUpVariants[0]), variant,
      dflt, min_xp);
  if (!v) return fail(AXH_ERR_INVALID_ARGUMENT, "no compiled Q4_0 gate/up variant matches");
  if (!staged_in_chunks(*v) && nb > v->xp * v->nw * 64u)
    return fail(AXH_ERR_INVALID_ARGUMENT,
                "Q4_0 gate/up: row too long for this variant's x staging");
  std::snprintf(p->name, sizeof(p->name), "axh_q4_0_gate_up_r%u_w%u_p%u_x%u", v->rpw, v->nw,
                v->pf, v->xp);
  p->nw = v->nw;
  p->lds = (nb + 7u) / 8u * 1120u;
  p->flat = true;
  const uint32_t bundles = (n_rows + v->rpw - 1) / v->rpw;
  p->units = ((bundles + 1) / 2 + v->nw - 1) / v->nw;
  p->args = RowsArgs{n_rows, nb, nb, 0};
  return ok();
}

axh_status axh_q4_0_gate_up_kernel_name(uint32_t n_rows, uint32_t blocks_per_row,
                                        const axh_q4_variant *variant, char *buf, size_t cap) {
  if (!buf || cap == 0) return fail(AXH_ERR_INVALID_ARGUMENT, "buf is NULL");
  Q4kPlan p{};
  axh_status s = plan_q4_0_gate_up(n_rows, blocks_per_row, variant, &p);
  if (s != AXH_OK) return s;
  if (std::strlen(p.name) + 1 > cap) return fail(AXH_ERR_INVALID_ARGUMENT, "buf too small");
  std::memcpy(buf, p.name, std::strlen(p.name) + 1);
  return ok();
}

axh_status axh_q4_0_gate_up(axh_context *ctx, const void *q_gate, const void *q_up,
                            const float *x, float *h, uint32_t n_rows, uint32_t blocks_per_row,
                            const axh_q4_variant *variant, void *stream) {
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  if (n_rows == 0) return ok();
  if (!device_ptr_ok(h) || !device_ptr_ok(q_gate) || !device_ptr_ok(q_up) || !device_ptr_ok(x))
    return fail(AXH_ERR_INVALID_ARGUMENT, "q_gate, q_up, x and h must be device pointers");
  if (((uintptr_t)q_gate & 3u) || ((uintptr_t)q_up & 3u) || ((uintptr_t)x & 15u))
    return fail(AXH_ERR_INVALID_ARGUMENT,
                "q_gate and q_up must be 4-byte and x 16-byte aligned");
  Q4kPlan p{};
  axh_status s = plan_q4_0_gate_up(n_rows, blocks_per_row, variant, &p);
  if (s != AXH_OK) return s;
  if (p.lds > ctx->core->max_lds)
    return fail(AXH_ERR_PIPELINE_LAYOUT, "LDS tile exceeds the device limit");
  hipSetDevice(ctx->core->device);
  axh_kernel *k = nullptr;
  s = builtin_kernel(ctx, p.name, 4, sizeof(RowsArgs), p.nw * 64u, &k);
  if (s != AXH_OK) return s;
  uint32_t grid[3] = {p.units, 1, 1};
  if (p.flat) { // persistent: at most one resident round of workgroups
    const uint32_t resident = occupancy(ctx, k, p.lds) * ctx->core->cu_count;
    if (resident < grid[0]) grid[0] = resident;
  }
  void *bufs[4] = {const_cast<void *>(q_gate), const_cast<void *>(q_up), const_cast<float *>(x),
                   h};
  s = launch_raw(k, grid, bufs, 4, &p.args, sizeof(p.args), p.lds, pick_stream(ctx, stream));
  return s == AXH_OK ? ok() : s;
}

// Kind 5 LDS: each wave's ring of `pf` buffers, one 1 KiB slot row per
// 16-byte-per-lane load of a step (2*nt for X, ceil(48*rt/64) for the
// weights), reused at the end for the waves' partial tiles (1 KiB per tile).
static uint32_t kx_lds_bytes(const MatmulVariant &v) {
  const uint32_t ring = v.w * v.pf * (2u * v.nt + (48u * v.rt + 63u) / 64u);
  const uint32_t red = v.w * v.rt * v.nt;
  return (ring > red ? ring : red) * 1024u;
}

// Kind 8 LDS: a ring of 4 buffers, each the X tile (16 KiB) and every wave's
// weight pieces (32 * rt rows x 48 bytes, in 1 KiB load instructions).
static uint32_t rm_lds_bytes(const MatmulVariant &v) {
  return 4u * (16u + v.w * ((96u * v.rt + 63u) / 64u)) * 1024u;
}

// Kind 9 LDS: a ring of pf + 1 buffers of the X chunk (4 * nt columns x 4
// KiB), then the waves' partial tiles (1 KiB each, rt per wave).  Its loads take the
// chunk as an SGPR offset of 512 bytes per superblock (X), up to 3 chunks
// past the row, over the zero-reading offset 0xFFF00000, which leaves 1 MiB:
// rows of fewer than 1024 superblocks keep it below 2^32.
static uint32_t lk_lds_bytes(const MatmulVariant &v) {
  return (v.pf + 1u) * 4u * v.nt * 4096u + 8u * v.rt * 1024u;
}
constexpr uint32_t kLkMaxSb = 1024;

// Kind 7 (streaming rows) keeps each wave's X fragments in VGPRs after
// staging them through 128 KiB of LDS: K up to 16 superblocks (8 waves x 2).
constexpr uint32_t kSrMaxSb = 16;

// The default matmul kind follows the grid each kind would launch, counted in
// MI355X's 256 CUs (a constant, so that the choice and its kernel name do not
// depend on the device a query runs on).  Measured over 60 shapes (1024 to
// 14336 rows, K = 4096 and 14336, 8 to 512 columns, every compiled variant):
// the choice below is the fastest variant at 59 and within 2% at the last.
// A later sweep of 22 shapes (up to 28672 rows, K up to 14336) moved two
// regions: 128 columns on enough rows (32 x 32 tiles) and more than 32
// columns on few long rows (the long-rows kind).
constexpr uint64_t kMatmulCus = 256;
// Workgroups the tile kinds (5 and 8) need before their tile size matters
// less than filling the chip: 5/8 of the CUs.  Below it, more and smaller
// tiles win (4096 x 4096 x 256: 16-row x 64-column K-split tiles in 256
// workgroups 21.5 us, 32 x 32 MFMA tiles in 64 workgroups 37.6).
constexpr uint64_t kMatmulFill = 160;

static MatmulVariant q4k_matmul_default(uint32_t n_rows, uint32_t batch, uint32_t nsb) {
  const auto groups = [&](uint32_t rows_per_wg, uint32_t cols_per_wg) {
    return (uint64_t)((n_rows + rows_per_wg - 1) / rows_per_wg) *
           ((batch + cols_per_wg - 1) / cols_per_wg);
  };
  if (nsb <= kSrMaxSb) {
    // Kind 7 runs one workgroup per CU over the 16-row blocks of each column
    // group.  The narrowest group (8, 16 or 32 columns) whose grid is one
    // resident wave wins: 14336 x 4096 at B = 8 10.9 us, 16 11.8 and 32 15.0
    // against the K-split tile kind's 14.2, 14.6 and 16.0; 1024 x 4096 x 64
    // 5.5 us with 16-column groups against 6.9 with 32 and 13.2 as tiles.
    const uint64_t per_group = std::min<uint64_t>(kMatmulCus, (n_rows + 15u) / 16u);
    if (per_group * ((batch + 7u) / 8u) <= kMatmulCus) return {7, 8, 1, 2, 0};
    if (per_group * ((batch + 15u) / 16u) <= kMatmulCus) return {7, 8, 1, 1, 0};
    if (per_group * ((batch + 31u) / 32u) <= kMatmulCus) return {7, 8, 2, 1, 0};
    // Up to two blocks of 32 columns per CU it still beats the tiles (4096 x
    // 4096 x 64 13.8 us against 14.7; 2048 x 4096 x 128 13.5 against 14.9),
    // not at four (8192 x 4096 x 64 18.6 against 16.3).
    if (groups(16, 32) <= 2 * kMatmulCus) return {7, 8, 2, 1, 0};
  }
  // Long rows (K > 4096) over few of them, up to 32 columns: kind 9 (8 waves
  // over 16 or 32 rows and 8 or 16 columns, K in chunks of 8 superblocks, X
  // through an LDS ring).  Every workgroup reads all of X for its columns, so
  // the largest tile whose grid still fills the chip wins: 4096 x 14336 x 32
  // 23.4 us with 32 x 16 tiles against 28.2 with 16 x 16 and 35.7 for the
  // K-split kind; B = 16 16.5 with 16 x 16 (32 x 16: 128 workgroups, 23.5);
  // B = 8 13.6 with 16 x 8 against 19.9 for the K-split kind; 8192 x 14336 x
  // 8 22.5 with 32 x 8 against 30.5.  Only while the grid is one wave (one
  // workgroup per CU): with more, the K-split tile kind is ahead (8192 x
  // 14336 x 32 42.4 against 45.0; 14336 x 14336 x 8 40.1 against 41.5).
  // Kind 9 keeps a row's superblock offsets below kLkMaxSb; longer rows fall
  // through to the K-split kinds.
  if (nsb > kSrMaxSb && nsb < kLkMaxSb && batch <= 32) {
    // up to 4 columns: 4-column tiles (X loads halved; 56 KiB of LDS, so two
    // workgroups per CU): 4096 x 14336 x 4 10.8 us against 11.7 with 8
    // columns, 8192 x 14336 x 4 (512 workgroups) 20.0 against 21.9.  Also up
    // to 8 columns where 8-column tiles would leave half the CUs or more idle
    // (A/B in one run: 512 x 14336 x 8 8.65 vs 9.69 us, 1024 x 14336 x 8 9.53
    // vs 11.13, 2048 x 14336 x 6 9.94 vs 11.61, 1024 x 8192 x 8 6.34 vs 6.90,
    // 2048 x 8192 x 8 7.28 vs 8.46, 1024 x 8192 x 5 6.30 vs 6.71; at 4096 x
    // 14336 x 8 the 8-column tiles stay ahead).
    const bool narrow = batch <= 4 || (batch <= 8 && groups(16, 8) <= kMatmulCus / 2);
    if (narrow && groups(16, 4) <= 2 * kMatmulCus) return {9, 8, 1, 2, 1};
    constexpr uint32_t cand[4][2] = {{16, 2}, {16, 1}, {8, 2}, {8, 1}}; // columns, row tiles
    for (int i = 0; i < 4; ++i) {
      const uint32_t xc = cand[i][0], rt = cand[i][1];
      if (batch <= 8 && xc == 16) continue;
      const uint64_t g = groups(16 * rt, xc);
      if (g < kMatmulFill && i < 3) continue;
      if (g <= kMatmulCus) return xc == 16 ? MatmulVariant{9, 8, 4, 1, rt} : MatmulVariant{9, 8, 2, 2, rt};
      break;
    }
  }
  // Long rows over few of them, more than 32 columns, where one wave of
  // 16 x 16 or 32 x 16 tiles fills the chip: the long-rows kind with 16-column
  // tiles (A/B in one run, against the K-split kind with the same tiles:
  // 1024 x 8192 x 64 9.08 vs 14.79 us, 1024 x 8192 x 128 13.69 vs 20.61, 1024
  // x 14336 x 128 21.19 vs 34.85, 2048 x 14336 x 64 21.88 vs 35.04, 512 x
  // 14336 x 128 13.01 vs 24.41).  The K-split kind (K over 8 waves) keeps
  // rows the long-rows kind cannot index (kLkMaxSb superblocks and more):
  // 16-row tiles first (4096 x 14336 at B = 8 19.8 us, B = 16 24.3, against
  // 28.9 and 34.5 with 32-row tiles), then 32-row tiles (4096 x 14336 x 32
  // 35.4 against 40.2; 1024 x 14336 x 128 35.1 against 40.1).
  const bool lk_ok = nsb > kSrMaxSb && nsb < kLkMaxSb;
  if (groups(16, 16) <= kMatmulCus) return lk_ok ? MatmulVariant{9, 8, 4, 1, 1} : MatmulVariant{3, 8, 1, 1, 1};
  if (groups(32, 16) <= kMatmulCus) return lk_ok ? MatmulVariant{9, 8, 4, 1, 2} : MatmulVariant{3, 8, 1, 1, 2};
  // kind 8 (32 x 32 MFMA tiles) where its rows fill the chip: 14336 x 4096 x
  // 512 74.1 us (8 waves of 32 rows) against 83-94 for a row-split kind,
  // B = 256 49.3 (4 waves of 32 rows) against 52.1; 8192 x 4096 x 512 46.0 us
  // with 4 waves against 60.7 as K-split tiles.
  if (batch > 256 && groups(256, 128) >= kMatmulFill) return {8, 8, 8, 4, 1};
  // from 128 columns (A/B in one run against the K-split tile kind at 128
  // columns: 20480 x 4096 40.35 vs 51.0 us, 28672 x 4096 43.95 vs 53.0, 28672
  // x 8192 78.45 vs 94.92, 24576 x 14336 136.0 vs 156.2; below the fill
  // 16384 x 8192 and 11008 x 4096 stay on the K-split tile kind)
  if (batch >= 128 && groups(128, 128) >= kMatmulFill) return {8, 4, 8, 4, 1};
  // The K-split tile kind: up to 128 columns per workgroup, halved until the
  // grid fills (4096 x 14336 x 64: one column tile 41.3 us against four
  // 58.8; 4096 x 11008 x 128: two 37.9 against eight 76.5).  Two column
  // tiles prefetch 3 steps at K > 4096 (4096 x 14336 x 128 45.8 us against
  // 47.6), 2 at K <= 4096 (4096 x 4096 x 128 16.0 against 16.3).
  uint32_t nt = batch <= 16 ? 1u : batch <= 32 ? 2u : batch <= 64 ? 4u : 8u;
  while (nt > 1 && groups(64, 16 * nt) < kMatmulFill) nt /= 2;
  return {5, 4, nt, nt == 1 || (nt == 2 && nsb > kSrMaxSb) ? 3u : 2u, 4};
}

uint32_t axh_q4k_matmul_variant_count(void) {
  return (uint32_t)(sizeof(kQ4kMatmulVariants) / sizeof(kQ4kMatmulVariants[0]));
}

axh_status axh_q4k_matmul_variant_at(uint32_t i, axh_q4_matmul_variant *out) {
  if (!out || i >= axh_q4k_matmul_variant_count())
    return fail(AXH_ERR_INVALID_ARGUMENT, "variant index out of range");
  out->kind = kQ4kMatmulVariants[i].kind;
  out->waves_per_workgroup = kQ4kMatmulVariants[i].w;
  out->col_tiles = kQ4kMatmulVariants[i].nt;
  out->prefetch = kQ4kMatmulVariants[i].pf;
  out->row_tiles = kQ4kMatmulVariants[i].rt;
  return ok();
}

static axh_status plan_q4k_matmul(uint32_t n_rows, uint32_t sb_per_row, uint32_t batch,
                                  const axh_q4_matmul_variant *variant, MatmulVariant *out,
                                  char *name, size_t cap) {
  MatmulVariant want = q4k_matmul_default(n_rows, batch, sb_per_row);
  if (variant) {
    if (variant->kind && variant->kind != want.kind) {
      want.kind = variant->kind;
      want.rt = 0; // the row tiles of the requested kind's default
    }
    if (variant->waves_per_workgroup) want.w = variant->waves_per_workgroup;
    if (variant->col_tiles) want.nt = variant->col_tiles;
    if (variant->prefetch) want.pf = variant->prefetch;
    if (variant->row_tiles) {
      if (want.kind != 3 && want.kind != 5 && want.kind != 8 && want.kind != 9)
        return fail(AXH_ERR_INVALID_ARGUMENT,
                    "row_tiles is a hole of matmul kinds 3, 5, 8 and 9 only");
      want.rt = variant->row_tiles;
    }
  }
  if (want.kind != 3 && want.kind != 5 && want.kind != 8 && want.kind != 9) want.rt = 0;
  else if (want.rt == 0)
    want.rt = want.kind == 5 ? 4u : want.kind == 3 ? 2u : 1u;
  for (const MatmulVariant &v : kQ4kMatmulVariants)
    if (v.kind == want.kind && v.w == want.w && v.nt == want.nt && v.pf == want.pf &&
        v.rt == want.rt) {
      *out = v;
      if (v.kind == 3)
        std::snprintf(name, cap, "axh_q4k_matmul_ks_k%u_n%u_p%u%s", v.w, v.nt, v.pf,
                      v.rt == 1 ? "_r1" : "");
      else if (v.kind == 5)
        std::snprintf(name, cap, "axh_q4k_matmul_kx_r%u_n%u_k%u_p%u", v.rt, v.nt, v.w, v.pf);
      else if (v.kind == 8)
        std::snprintf(name, cap, "axh_q4k_matmul_rm_w%u_r%u_p4", v.w, v.rt);
      else if (v.kind == 9) {
        if (sb_per_row >= kLkMaxSb)
          return fail(AXH_ERR_INVALID_ARGUMENT,
                      "matmul kind 9 takes rows of fewer than 1024 superblocks");
        std::snprintf(name, cap, "axh_q4k_matmul_lk_c%u_x%u_w%u%s", 4u * v.nt, v.pf,
                      v.pf == 1u ? 3u : v.pf, v.rt == 2u ? "_r2" : "");
      }
      else {
        if (sb_per_row > kSrMaxSb)
          return fail(AXH_ERR_INVALID_ARGUMENT,
                      "matmul kind 7 takes rows of at most 16 superblocks (K <= 4096)");
        // prefetch 2: 8-column groups, X staged through 64 KiB
        std::snprintf(name, cap, "axh_q4k_matmul_sr_w%u_s2%s%s", v.w, v.nt == 2 ? "_n2" : "",
                      v.pf == 2 ? "_h" : "");
      }
      return ok();
    }
  return fail(AXH_ERR_INVALID_ARGUMENT, "no compiled Q4_K matmul variant matches");
}

axh_status axh_q4k_matmul_kernel_name(uint32_t n_rows, uint32_t sb_per_row, uint32_t batch,
                                      const axh_q4_matmul_variant *variant, char *buf,
                                      size_t cap) {
  if (!buf || cap == 0) return fail(AXH_ERR_INVALID_ARGUMENT, "buf is NULL");
  MatmulVariant v{};
  char name[64];
  axh_status s = plan_q4k_matmul(n_rows, sb_per_row, batch, variant, &v, name, sizeof(name));
  if (s != AXH_OK) return s;
  if (std::strlen(name) + 1 > cap) return fail(AXH_ERR_INVALID_ARGUMENT, "buf too small");
  std::memcpy(buf, name, std::strlen(name) + 1);
  return ok();
}

// Argument checks shared by the f16 and f32 entry points.
static axh_status q4k_matmul_check(axh_context *ctx, const void *q, const void *x, const float *y,
                                   uint32_t n_rows, uint32_t sb_per_row, uint32_t batch) {
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  if (n_rows == 0 || batch == 0) return ok();
  if (sb_per_row == 0)
    return fail(AXH_ERR_INVALID_ARGUMENT, "sb_per_row must be at least 1 for the matmul");
  if (!device_ptr_ok(q) || !device_ptr_ok(x) || !device_ptr_ok(y))
    return fail(AXH_ERR_INVALID_ARGUMENT, "q, x and y must be device pointers");
  if (((uintptr_t)q & 15u) || ((uintptr_t)x & 15u) || ((uintptr_t)y & 3u))
    return fail(AXH_ERR_INVALID_ARGUMENT, "q and x must be 16-byte and y 4-byte aligned");
  const uint64_t q_bytes = (uint64_t)n_rows * sb_per_row * 144u;
  const uint64_t x_f16_bytes = (uint64_t)batch * sb_per_row * 256u * 2u;
  if (q_bytes + 16ull * sb_per_row * 144u >= kMatmulOob || x_f16_bytes >= kMatmulOob)
    return fail(AXH_ERR_INVALID_ARGUMENT, "q (with 16 rows to spare) and f16 x must each be below 4 GiB - 1 MiB");
  return ok();
}

axh_status axh_q4k_matmul_f16(axh_context *ctx, const void *q, const uint16_t *x, float *y,
                              uint32_t n_rows, uint32_t sb_per_row, uint32_t batch,
                              const axh_q4_matmul_variant *variant, void *stream) {
  axh_status s = q4k_matmul_check(ctx, q, x, y, n_rows, sb_per_row, batch);
  if (s != AXH_OK || n_rows == 0 || batch == 0) return s;
  MatmulVariant v{};
  char name[64];
  s = plan_q4k_matmul(n_rows, sb_per_row, batch, variant, &v, name, sizeof(name));
  if (s != AXH_OK) return s;
  // kind 5 sums the partial tiles of its waves in LDS (one 16x16 f32 tile =
  // 1 KiB per wave); kind 7: 128 KiB of X staging (64 KiB with 8-column
  // groups), whose wave regions then hold the waves' partial tiles
  const uint32_t lds = v.kind == 5   ? kx_lds_bytes(v)
                       : v.kind == 7 ? (v.pf == 2 ? 65536u : 131072u)
                       : v.kind == 8 ? rm_lds_bytes(v)
                       : v.kind == 9 ? lk_lds_bytes(v)
                                     : 0u;
  if (lds > ctx->core->max_lds)
    return fail(AXH_ERR_INVALID_ARGUMENT, "matmul variant needs more LDS than the device has");
  const uint32_t tm = v.kind == 3   ? 16u * v.rt
                      : v.kind == 5 ? 16u * v.rt
                      : v.kind == 7 ? 16u
                      : v.kind == 9 ? 16u * v.rt
                                    : 32u * v.rt * v.w;
  const uint32_t tn = v.kind == 9 ? 4u * v.nt : (v.kind == 7 && v.pf == 2 ? 8u : 16u) * v.nt;
  uint64_t gx = (n_rows + tm - 1) / tm;
  const uint64_t gy = (batch + tn - 1) / tn;
  if (gx > ctx->core->max_wg[0] || gy > ctx->core->max_wg[1])
    return fail(AXH_ERR_WORKGROUP_COUNT_EXCEEDS_LIMIT, "matmul grid exceeds the device limit");
  hipSetDevice(ctx->core->device);
  axh_kernel *k = nullptr;
  s = builtin_kernel(ctx, name, 3, sizeof(MatmulArgs), v.w * 64u, &k);
  if (s != AXH_OK) return s;
  // kind 7 is persistent: one workgroup per CU per column group, even where two would fit
  if (v.kind == 7 && ctx->core->cu_count < gx) gx = ctx->core->cu_count;
  const uint32_t grid[3] = {(uint32_t)gx, (uint32_t)gy, 1};
  void *bufs[3] = {const_cast<void *>(q), const_cast<uint16_t *>(x), y};
  MatmulArgs a{n_rows, sb_per_row, batch, 0};
  s = launch_raw(k, grid, bufs, 3, &a, sizeof(a), (uint32_t)lds, pick_stream(ctx, stream));
  return s == AXH_OK ? ok() : s;
}

axh_status axh_q4k_matmul_f32(axh_context *ctx, const void *q, const float *x, uint16_t *x16,
                              float *y, uint32_t n_rows, uint32_t sb_per_row, uint32_t batch,
                              const axh_q4_matmul_variant *variant, void *stream) {
  axh_status s = q4k_matmul_check(ctx, q, x, y, n_rows, sb_per_row, batch);
  if (s != AXH_OK || n_rows == 0 || batch == 0) return s;
  if (!device_ptr_ok(x16) || ((uintptr_t)x16 & 15u))
    return fail(AXH_ERR_INVALID_ARGUMENT, "x16 must be a 16-byte aligned device pointer");
  MatmulVariant v{};
  char name[64];
  s = plan_q4k_matmul(n_rows, sb_per_row, batch, variant, &v, name, sizeof(name));
  if (s != AXH_OK) return s; // reject a bad variant before any device work
  s = axh_f32_to_f16(ctx, x, x16, (uint64_t)batch * sb_per_row * 256u, stream);
  if (s != AXH_OK) return s;
  return axh_q4k_matmul_f16(ctx, q, x16, y, n_rows, sb_per_row, batch, variant, stream);
}

static axh_status count_launch(axh_context *ctx, const char *name, const void *in, void *out,
                               uint64_t n_threads, uint64_t n_units, void *stream) {
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  if (n_units == 0) return ok();
  if (!in || !out) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL device pointer");
  if (n_units > 0xFFFFFFFFull || n_threads > (uint64_t)0xFFFFFFFFull * 256ull)
    return fail(AXH_ERR_INVALID_ARGUMENT, "too many units for one launch");
  axh_kernel *k = nullptr;
  axh_status s = builtin_kernel(ctx, name, 2, sizeof(CountArgs), 256, &k);
  if (s != AXH_OK) return s;
  CountArgs a{(uint32_t)n_units};
  const uint32_t grid[3] = {(uint32_t)((n_threads + 255u) / 256u), 1, 1};
  void *bufs[2] = {const_cast<void *>(in), out};
  hipSetDevice(ctx->core->device);
  s = launch_raw(k, grid, bufs, 2, &a, sizeof(a), 0, pick_stream(ctx, stream));
  return s == AXH_OK ? ok() : s;
}

axh_status axh_q5k_dequant(axh_context *ctx, const void *q, float *w, uint64_t n_sb, void *stream) {
  if (n_sb > (1ull << 28)) return fail(AXH_ERR_INVALID_ARGUMENT, "too many superblocks");
  if (((uintptr_t)q & 15u) || ((uintptr_t)w & 15u))
    return fail(AXH_ERR_INVALID_ARGUMENT, "q and w must be 16-byte aligned");
  return count_launch(ctx, "axh_q5k_dequant", q, w, n_sb * 8u, n_sb, stream);
}

axh_status axh_q6k_dequant(axh_context *ctx, const void *q, float *w, uint64_t n_sb, void *stream) {
  if (n_sb > (1ull << 28)) return fail(AXH_ERR_INVALID_ARGUMENT, "too many superblocks");
  if ((uintptr_t)q & 1u) return fail(AXH_ERR_INVALID_ARGUMENT, "q must be 2-byte aligned");
  if ((uintptr_t)w & 3u) return fail(AXH_ERR_INVALID_ARGUMENT, "w must be 4-byte aligned");
  return count_launch(ctx, "axh_q6k_dequant", q, w, n_sb * 8u, n_sb, stream);
}

axh_status axh_q4k_dequant(axh_context *ctx, const void *q, float *w, uint64_t n_sb, void *stream) {
  if (n_sb > (1ull << 28)) return fail(AXH_ERR_INVALID_ARGUMENT, "too many superblocks");
  if (((uintptr_t)q & 15u) || ((uintptr_t)w & 15u))
    return fail(AXH_ERR_INVALID_ARGUMENT, "q and w must be 16-byte aligned");
  return count_launch(ctx, "axh_q4k_dequant", q, w, n_sb * 8u, n_sb, stream);
}

axh_status axh_q4_0_dequant(axh_context *ctx, const void *q, float *w, uint64_t n_blocks,
                            void *stream) {
  if (((uintptr_t)q & 1u) || ((uintptr_t)w & 3u))
    return fail(AXH_ERR_INVALID_ARGUMENT, "q must be 2-byte and w 4-byte aligned");
  return count_launch(ctx, "axh_q4_0_dequant", q, w, n_blocks, n_blocks, stream);
}

// Measurement helpers: the matvec's launch shape (one 512-thread workgroup
// per CU) reading `bytes` or doing nothing.
static axh_status floor_launch(axh_context *ctx, const char *name, const void *q, uint64_t pieces,
                               uint32_t *out, uint32_t out_words, void *stream) {
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  if (!device_ptr_ok(out) || (pieces && !device_ptr_ok(q)))
    return fail(AXH_ERR_INVALID_ARGUMENT, "q and out must be device pointers");
  const uint32_t grid[3] = {ctx->core->cu_count, 1, 1};
  // The kernel's 32-bit byte offsets reach (pieces + 4 * threads in the grid) * 16.
  if (((uintptr_t)q & 15u) || pieces + 4ull * 512u * grid[0] > 0xFFFFFFFFull / 16u)
    return fail(AXH_ERR_INVALID_ARGUMENT, "q must be 16-byte aligned and below 4 GiB");
  if (out_words < 8u * grid[0])
    return fail(AXH_ERR_INVALID_ARGUMENT, "out needs 8 words per compute unit");
  hipSetDevice(ctx->core->device);
  axh_kernel *k = nullptr;
  axh_status s = builtin_kernel(ctx, name, 2, sizeof(CountArgs), 512, &k);
  if (s != AXH_OK) return s;
  CountArgs a{(uint32_t)pieces};
  void *bufs[2] = {const_cast<void *>(q), out};
  s = launch_raw(k, grid, bufs, 2, &a, sizeof(a), 0, pick_stream(ctx, stream));
  return s == AXH_OK ? ok() : s;
}

axh_status axh_read_floor(axh_context *ctx, const void *q, uint64_t bytes, uint32_t *out,
                          uint32_t out_words, void *stream) {
  if (bytes % 16u) return fail(AXH_ERR_INVALID_ARGUMENT, "bytes must be a multiple of 16");
  return floor_launch(ctx, "axh_read_floor", q, bytes / 16u, out, out_words, stream);
}

axh_status axh_read_floor_shape(axh_context *ctx, const void *q, uint64_t bytes, uint32_t threads,
                                uint32_t loads, uint32_t grid, uint32_t *out, uint32_t out_words,
                                void *stream) {
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  if ((threads != 256 && threads != 512 && threads != 1024) ||
      (loads != 2 && loads != 4 && loads != 8) || grid == 0 || grid > 65536)
    return fail(AXH_ERR_INVALID_ARGUMENT,
                "read floor shapes: 256/512/1024 threads, 2/4/8 loads, 1..65536 workgroups");
  // The kernel's 32-bit byte offsets reach (pieces + loads * threads in the grid) * 16.
  if (bytes % 16u || bytes / 16u + (uint64_t)loads * threads * grid > 0xFFFFFFFFull / 16u)
    return fail(AXH_ERR_INVALID_ARGUMENT, "bytes must be a multiple of 16 below 4 GiB");
  if (!device_ptr_ok(out) || (bytes && !device_ptr_ok(q)) || ((uintptr_t)q & 15u))
    return fail(AXH_ERR_INVALID_ARGUMENT, "q (16-byte aligned) and out must be device pointers");
  if ((uint64_t)out_words < (uint64_t)grid * threads / 64u)
    return fail(AXH_ERR_INVALID_ARGUMENT, "out needs one word per wave of the grid");
  char name[48];
  std::snprintf(name, sizeof(name), "axh_read_floor_t%u_u%u", threads, loads);
  hipSetDevice(ctx->core->device);
  axh_kernel *k = nullptr;
  axh_status s = builtin_kernel(ctx, name, 2, sizeof(CountArgs), threads, &k);
  if (s != AXH_OK) return s;
  CountArgs a{(uint32_t)(bytes / 16u)};
  const uint32_t g[3] = {grid, 1, 1};
  void *bufs[2] = {const_cast<void *>(q), out};
  s = launch_raw(k, g, bufs, 2, &a, sizeof(a), 0, pick_stream(ctx, stream));
  return s == AXH_OK ? ok() : s;
}

axh_status axh_launch_empty(axh_context *ctx, uint32_t *out, uint32_t out_words, void *stream) {
  return floor_launch(ctx, "axh_launch_empty", out, 0, out, out_words, stream);
}

uint32_t axh_cu_count(axh_context *ctx) { return ctx ? ctx->core->cu_count : 0u; }

axh_status axh_f16_widen(axh_context *ctx, const uint16_t *h, float *f, uint64_t n, void *stream) {
  return count_launch(ctx, "axh_f16_widen", h, f, n, n, stream);
}

axh_status axh_f32_to_f16(axh_context *ctx, const float *x, uint16_t *h, uint64_t n, void *stream) {
  if (n > 0xFFFFFFF0ull) return fail(AXH_ERR_INVALID_ARGUMENT, "n too large for one launch");
  if (((uintptr_t)x & 15u) || ((uintptr_t)h & 15u))
    return fail(AXH_ERR_INVALID_ARGUMENT, "x and h must be 16-byte aligned");
  return count_launch(ctx, "axh_f32_to_f16", x, h, (n + 7u) / 8u, n, stream);
}

} // extern "C"

// ---- measurement loop ---------------------------------------------------------
static axh_status bench_call(axh_context *ctx, const axh_bench_op *o, uint32_t i) {
  const uint8_t *q = static_cast<const uint8_t *>(o->q) + (uint64_t)(i % o->n_copies) * o->q_stride;
  switch (o->op) {
  case AXH_BENCH_Q4K_MATVEC:
    return axh_q4k_matvec(ctx, q, static_cast<const float *>(o->x), static_cast<float *>(o->y),
                          o->n_rows, o->units, o->variant, nullptr);
  case AXH_BENCH_Q4_0_MATVEC:
    return axh_q4_0_matvec(ctx, q, static_cast<const float *>(o->x), static_cast<float *>(o->y),
                           o->n_rows, o->units, o->variant, nullptr);
  case AXH_BENCH_Q5K_MATVEC:
    return axh_q5k_matvec(ctx, q, static_cast<const float *>(o->x), static_cast<float *>(o->y),
                          o->n_rows, o->units, o->variant, nullptr);
  case AXH_BENCH_Q6K_MATVEC:
    return axh_q6k_matvec(ctx, q, static_cast<const float *>(o->x), static_cast<float *>(o->y),
                          o->n_rows, o->units, o->variant, nullptr);
  case AXH_BENCH_Q4K_GATE_UP:
    return axh_q4k_gate_up(ctx, q, q + o->q2_offset, static_cast<const float *>(o->x),
                           static_cast<float *>(o->y), o->n_rows, o->units, o->variant, nullptr);
  case AXH_BENCH_Q4_0_GATE_UP:
    return axh_q4_0_gate_up(ctx, q, q + o->q2_offset, static_cast<const float *>(o->x),
                            static_cast<float *>(o->y), o->n_rows, o->units, o->variant, nullptr);
  case AXH_BENCH_Q5K_GATE_UP:
    return axh_q5k_gate_up(ctx, q, q + o->q2_offset, static_cast<const float *>(o->x),
                           static_cast<float *>(o->y), o->n_rows, o->units, o->variant, nullptr);
  case AXH_BENCH_Q4K_MATMUL_F16:
    return axh_q4k_matmul_f16(ctx, q, static_cast<const uint16_t *>(o->x),
                              static_cast<float *>(o->y), o->n_rows, o->units, o->batch,
                              o->matmul_variant, nullptr);
  case AXH_BENCH_Q4K_MATMUL_F32:
    return axh_q4k_matmul_f32(ctx, q, static_cast<const float *>(o->x),
                              static_cast<uint16_t *>(o->x16), static_cast<float *>(o->y),
                              o->n_rows, o->units, o->batch, o->matmul_variant, nullptr);
  case AXH_BENCH_READ_FLOOR:
    return axh_read_floor(ctx, q, (uint64_t)o->units * 16u, static_cast<uint32_t *>(o->y),
                          o->batch, nullptr);
  case AXH_BENCH_LAUNCH_EMPTY:
    return axh_launch_empty(ctx, static_cast<uint32_t *>(o->y), o->batch, nullptr);
  case AXH_BENCH_READ_SHAPE:
    if (!o->variant) return fail(AXH_ERR_INVALID_ARGUMENT, "read shape needs a variant");
    return axh_read_floor_shape(ctx, q, (uint64_t)o->units * 16u, o->variant->waves_per_workgroup * 64u,
                                o->variant->prefetch, o->n_rows, static_cast<uint32_t *>(o->y),
                                o->batch, nullptr);
  default:
    return fail(AXH_ERR_INVALID_ARGUMENT, "unknown bench operation");
  }
}

extern "C" axh_status axh_bench_loop(axh_context *ctx, const axh_bench_op *op, uint32_t warmup,
                                     uint32_t groups, uint32_t calls_per_group, float *group_ms) {
  if (!ctx || !op || !group_ms || groups == 0 || calls_per_group == 0 || op->n_copies == 0)
    return fail(AXH_ERR_INVALID_ARGUMENT, "bench loop: bad arguments");
  if (groups > 100000) return fail(AXH_ERR_INVALID_ARGUMENT, "bench loop: too many groups");
  hipSetDevice(ctx->core->device);
  const hipStream_t st = ctx->core->stream;
  axh_status s = axh_device_synchronize(ctx);
  if (s != AXH_OK) return s;
  std::vector<hipEvent_t> ev(groups + 1u, nullptr);
  for (auto &e : ev)
    if (hipEventCreate(&e) != hipSuccess) {
      for (auto &f : ev)
        if (f) hipEventDestroy(f);
      return fail(AXH_ERR_QUEUE_SUBMIT, "hipEventCreate failed");
    }
  // The warmup calls prime the queue: the first event follows them with no
  // synchronisation in between, so the first timed call starts behind queued
  // work, as every later one does, instead of on an idle device.
  uint32_t i = 0;
  for (; i < warmup && s == AXH_OK; ++i) s = bench_call(ctx, op, i);
  if (s != AXH_OK) {
    for (auto &e : ev) hipEventDestroy(e);
    return s;
  }
  hipEventRecord(ev[0], st);
  for (uint32_t g = 0; g < groups && s == AXH_OK; ++g) {
    for (uint32_t c = 0; c < calls_per_group && s == AXH_OK; ++c) s = bench_call(ctx, op, i++);
    hipEventRecord(ev[g + 1u], st);
  }
  if (s == AXH_OK) s = axh_synchronize(ctx, nullptr);
  for (uint32_t g = 0; g < groups && s == AXH_OK; ++g)
    if (hipEventElapsedTime(&group_ms[g], ev[g], ev[g + 1u]) != hipSuccess)
      s = fail(AXH_ERR_QUEUE_SUBMIT, "hipEventElapsedTime failed");
  for (auto &e : ev) hipEventDestroy(e);
  return s == AXH_OK ? ok() : s;
}
