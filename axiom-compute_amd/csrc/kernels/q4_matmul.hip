// gfx950 batched Q4_K_M matmul on MFMA: Y[b][r] = sum_k W[r][k] * X[b][k]
// for a Q4_K_M weight matrix W (n_rows x K, K = 256 * sb_per_row, rows of
// contiguous 144-byte superblocks) and `batch` f16 activation vectors X
// (batch x K, each vector contiguous).  Y is f32, batch x n_rows (each
// output vector contiguous).
//
// The reference has no batched kernel (its matvec produces one output); per
// column b this is the reference dot product (q4km_dequant_matvec_cpu,
// crates/axc-driver/tests/common_helpers.rs:411-461) with x_b widened from
// f16, computed here with f16 weights: every weight is dequantised exactly as
// the reference does it in f32 (w32 = RN_f32(d*sc*q - dmin*m),
// common_helpers.rs:437-454) and then rounded once to f16 (RN_f16(w32)).
// f16 x f16 products are exact in the f32 accumulators of the MFMA.
//
// Four kernel kinds; the runtime picks one by the grid each would launch
// (the others stay reachable as strategy variants):
//   * streaming rows (axh_q4k_matmul_sr_..., kind 7; K <= 4096): persistent,
//     K split across the waves, X fragments kept in VGPRs, weights streamed
//     like the matvec; see q4k_matmul_sr;
//   * K-split (axh_q4k_matmul_ks_..., kind 3): the waves of a workgroup share
//     one 32-row tile and split K, summing in LDS; see q4k_matmul_ks;
//   * K-split tile (axh_q4k_matmul_kx_..., kind 5): the waves of a workgroup
//     split K, each streaming raw weight bytes and X through a private LDS
//     ring filled by coalesced direct-to-LDS loads; see q4k_matmul_kx;
//   * 32 x 32 tiles (axh_q4k_matmul_rm_..., kind 8): waves of 32-row MFMA
//     tiles over 128 columns, X and weights through a 4-deep LDS ring; see
//     q4k_matmul_rm.
#include "q4_common.h"

using namespace axh;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

struct MatmulArgs {
  uint32_t n_rows;
  uint32_t sb_per_row;
  uint32_t batch;
  uint32_t pad;
};
// The shape as separate 32-bit kernel arguments (the struct's kernarg
// layout), so that all arguments are preloaded into SGPRs at wave launch.
#define AXH_MATMUL_ARGS uint32_t a_n_rows, uint32_t a_sb_per_row, uint32_t a_batch, uint32_t a_pad
#define AXH_MATMUL_UNPACK const MatmulArgs a{a_n_rows, a_sb_per_row, a_batch, a_pad}

namespace {

constexpr uint32_t kOob = 0xFFFFFF00u; // out-of-range buffer offset: loads return zeros

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                           0x00020000);
}

__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// RN_f16 of two f32 values, packed (lo = a).
__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
  const half2_t h = __builtin_convertvector((f32x2_t){a, b}, half2_t);
  return __builtin_bit_cast(uint32_t, h);
}

// Four qs bytes (one dword) of a quarter: low nibbles are weights 4t..4t+3 of
// the quarter's first sub-block, high nibbles the same of its second.  Each
// weight is w32 = RN_f32(q * d1 - m1) through v_fma_mix_f32 with the nibble
// as an f16 subnormal (q * 2^-24 or q * 2^-20) against d1 pre-scaled by 2^24
// or 2^20, then RN_f16.  Outputs: lo = 4 f16 (2 dwords), hi = 4 f16.
__device__ __forceinline__ void dequant_dword(uint32_t w, float d1s, float m1, float d2s, float m2,
                                              uint32_t &lo01, uint32_t &lo23, uint32_t &hi01,
                                              uint32_t &hi23) {
  const uint32_t w8 = w >> 8;
  const uint32_t a = w & 0x000F000Fu;   // bytes 0, 2 low nibbles
  const uint32_t b = w8 & 0x000F000Fu;  // bytes 1, 3 low nibbles
  const uint32_t ch = w & 0x00F000F0u;  // bytes 0, 2 high nibbles
  const uint32_t dh = w8 & 0x00F000F0u; // bytes 1, 3 high nibbles
  const float l0 = __builtin_fmaf(lo_half_f16(a), d1s, -m1);
  const float l1 = __builtin_fmaf(lo_half_f16(b), d1s, -m1);
  const float l2 = __builtin_fmaf(hi_half_f16(a), d1s, -m1);
  const float l3 = __builtin_fmaf(hi_half_f16(b), d1s, -m1);
  const float h0 = __builtin_fmaf(lo_half_f16(ch), d2s, -m2);
  const float h1 = __builtin_fmaf(lo_half_f16(dh), d2s, -m2);
  const float h2 = __builtin_fmaf(hi_half_f16(ch), d2s, -m2);
  const float h3 = __builtin_fmaf(hi_half_f16(dh), d2s, -m2);
  lo01 = pack_f16(l0, l1);
  lo23 = pack_f16(l2, l3);
  hi01 = pack_f16(h0, h1);
  hi23 = pack_f16(h2, h3);
}

// Four consecutive rows r0..r0+3 of one output column (the lane's part of a
// 16x16 MFMA tile): one 16-byte store when all four exist and the address is
// aligned (y is only required to be 4-byte aligned), else scalar stores.
// Scalar stores put every lane of a store on its own 4-byte word, 4x the
// store instructions.
__device__ __forceinline__ void store_col4(float *ycol, uint32_t r0, uint32_t n_rows, f32x4_t v) {
  float *dst = ycol + r0;
  if (r0 + 4u <= n_rows && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0u) {
    *reinterpret_cast<f32x4_t *>(dst) = v;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (r0 + (uint32_t)e < n_rows) dst[e] = v[e];
  }
}

__device__ __forceinline__ uint2 bload8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
  const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b32(r, (int)off + 4, 0, 0);
  return make_uint2(lo, hi);
}

// ---------------------------------------------------------------------------
// K-split variant for small batches (memory- and dequant-bound): the KS waves
// of a workgroup share one 16*RT x TN output tile and take interleaved 128-wide
// K steps (half a superblock; wave w: steps w, w + KS, ...).  Each lane
// dequantises exactly the A fragments it feeds to v_mfma_f32_16x16x32_f16
// (row lane%16 of a 16-row tile, k = 32*kk + 8*(lane/16) + 0..7), so A never
// goes through LDS: in step ks of superblock sb (half h = ks%2) the lane
// reads, per 16-row tile, the row's 16-byte header and the 8 qs bytes
// [32c + 8g, 32c + 8g + 8) for c = 2h and 2h+1, whose low nibbles feed the
// fragments of sub-block 2c and high nibbles those of 2c+1.  X fragments
// come straight from global memory.  Loads run PF steps ahead in a register
// ring.  The KS partial tiles are summed in LDS in wave order
// (deterministic) by wave 0.
// ---------------------------------------------------------------------------
template <int NT, int RT>
struct KsStep {
  uint4 hd[RT];
  uint2 qlo[RT], qhi[RT];
  uint4 xv[4 * NT];
};

template <int KS, int NT, int PF, int RT>
__device__ __forceinline__ void q4k_matmul_ks(const uint8_t *__restrict__ q,
                                              const uint16_t *__restrict__ x,
                                              float *__restrict__ y, const MatmulArgs a) {
  constexpr int TN = 16 * NT;
  __shared__ __attribute__((aligned(16))) f32x4_t red[KS > 1 ? (KS - 1) * RT * NT * 64 : 1];

  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t n_rows = a.n_rows, nsb = a.sb_per_row, batch = a.batch;
  const uint32_t m0 = blockIdx.x * (16u * RT), n0 = blockIdx.y * TN;
  const uint32_t K = nsb * 256u;
  const uint32_t row_bytes = nsb * (uint32_t)kQ4kSbBytes;
  const __amdgpu_buffer_rsrc_t qr = rsrc(q, n_rows * row_bytes);
  const __amdgpu_buffer_rsrc_t xr = rsrc(x, batch * K * 2u);
  const uint32_t fr = lane & 15u, g = lane >> 4;
  const uint32_t n_steps = 2u * nsb;

  uint32_t row_off[RT];
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    const uint32_t row = m0 + 16u * (uint32_t)i + fr;
    row_off[i] = row < n_rows ? row * row_bytes : kOob;
  }
  uint32_t xoff0[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const uint32_t b = n0 + 16u * (uint32_t)j + fr;
    xoff0[j] = b < batch ? (b * K + 8u * g) * 2u : kOob;
  }

  auto load_step = [&](KsStep<NT, RT> &S, uint32_t ks) {
    const uint32_t sb = ks >> 1, h = ks & 1u;
    const bool live = ks < n_steps;
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const uint32_t base = (row_off[i] == kOob || !live) ? kOob : row_off[i] + sb * 144u;
      S.hd[i] = bload16(qr, base);
      const uint32_t qo = 16u + 64u * h + 8u * g;
      S.qlo[i] = bload8(qr, base == kOob ? kOob : base + qo);
      S.qhi[i] = bload8(qr, base == kOob ? kOob : base + qo + 32u);
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int j = 0; j < NT; ++j)
        S.xv[kk * NT + j] =
            bload16(xr, (xoff0[j] == kOob || !live) ? kOob : xoff0[j] + ks * 256u + 64u * kk);
  };

  f32x4_t acc[RT][NT];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};

  KsStep<NT, RT> S[PF];
#pragma unroll
  for (int p = 0; p < PF; ++p) load_step(S[p], wave + (uint32_t)(p * KS));

  const uint32_t my_steps = (n_steps + KS - 1u) / KS;
  const uint32_t n_iter = (my_steps + PF - 1u) / PF * PF;
  for (uint32_t j0 = 0; j0 < n_iter; j0 += PF) {
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      const uint32_t ks = wave + (j0 + (uint32_t)p) * KS;
      const uint32_t h = ks & 1u;
      half8_t af[RT][4];
#pragma unroll
      for (int i = 0; i < RT; ++i) {
        const uint4 hd = S[p].hd[i];
        const float d = f16_to_f32(hd.x & 0xFFFFu), dmin = f16_to_f32(hd.x >> 16);
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
          const uint32_t c = 2u * h + (uint32_t)cc;
          uint32_t scp, mp;
          q4k_scale_min_pair(hd.y, hd.z, hd.w, c, &scp, &mp);
          const float d1s = d * (float)(scp & 0xFFu) * 16777216.0f;
          const float d2s = d * (float)(scp >> 8) * 1048576.0f;
          const float m1 = dmin * (float)(mp & 0xFFu), m2 = dmin * (float)(mp >> 8);
          const uint2 qw = cc == 0 ? S[p].qlo[i] : S[p].qhi[i];
          uint32_t l0, l1, h0, h1, l2, l3, h2, h3;
          dequant_dword(qw.x, d1s, m1, d2s, m2, l0, l1, h0, h1);
          dequant_dword(qw.y, d1s, m1, d2s, m2, l2, l3, h2, h3);
          af[i][2 * cc] = __builtin_bit_cast(half8_t, make_uint4(l0, l1, l2, l3));
          af[i][2 * cc + 1] = __builtin_bit_cast(half8_t, make_uint4(h0, h1, h2, h3));
        }
      }
      half8_t bfr[4][NT];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int j = 0; j < NT; ++j) bfr[kk][j] = __builtin_bit_cast(half8_t, S[p].xv[kk * NT + j]);
      load_step(S[p], ks + (uint32_t)(PF * KS));
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
          for (int j = 0; j < NT; ++j)
            acc[i][j] =
                __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i][kk], bfr[kk][j], acc[i][j], 0, 0, 0);
    }
  }

  if constexpr (KS > 1) {
    if (wave > 0) {
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) red[(((wave - 1u) * RT + i) * NT + j) * 64u + lane] = acc[i][j];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (uint32_t w = 1; w < (uint32_t)KS; ++w)
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] += red[(((w - 1u) * RT + i) * NT + j) * 64u + lane];
  }
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const uint32_t b = n0 + 16u * j + fr;
      const uint32_t r0 = m0 + 16u * i + 4u * g;
      if (b >= batch) continue;
      store_col4(y + (size_t)b * n_rows, r0, n_rows, acc[i][j]);
    }
}


// ---------------------------------------------------------------------------
// K-split tile variant (kind 5): a workgroup of KS waves owns a TM = 16*RT
// by TN = 16*NT tile of Y, and every wave runs the whole tile over its share
// of K: wave w takes the 64-wide chunk c = w % 4 of superblocks w/4, w/4 +
// KS/4, ... (from a per-workgroup start, see below).  Each lane dequantises
// exactly the A fragments it feeds (row lane%16 of each of the RT row tiles;
// the 8 qs bytes [32c + 8g, 32c + 8g + 8), g = lane/16, hold the fragment of
// sub-block 2c in their low nibbles and that of 2c+1 in their high nibbles),
// so one dequantised fragment feeds NT MFMAs.
//
// Operands reach the wave through a private ring of PF LDS buffers filled by
// direct-to-LDS buffer loads (16 bytes per lane, no VGPRs), laid out so that
// the global reads are coalesced: a fragment's 16 lanes read 16 different
// rows (weights) or columns (X), which as direct loads would touch 4 cache
// lines per 4 lanes.  X instruction u covers columns 8u..8u+7 and the whole
// 64-k chunk, one 128-byte line per column: lane 8b + s loads 16-byte piece
// s ^ f of column 8u + b, f = (b >> 1) | ((u & 1) << 2), so that the fragment
// reads (16 lanes: columns 16t..16t+15, one piece) hit 16 distinct 16-byte
// bank groups.  (Two instructions per line, 64 bytes of 16 columns each,
// measured 3 % slower, A/B in one run at 14336 x 4096: B = 128 28.97 vs
// 28.09 us, B = 64 20.86 vs 20.45, B = 32 16.17 vs 15.78.)  Weight piece
// 3r + {0, 1, 2} is row r's header or its two 16-byte halves of the chunk's
// 32 qs bytes.  A wave waits only for its own loads
// (the load counter), so there is no barrier until the end, when all KS
// partial tiles go to LDS and wave w sums tiles w, w + KS, ... in wave order
// (deterministic) and stores them.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void_t;

template <int RT, int NT>
struct KxLayout {
  static constexpr int kX = 2 * NT;                  // X instructions per superblock step
  static constexpr int kW = (48 * RT + 63) / 64;     // weight instructions per step
  static constexpr int kPerStep = kX + kW;           // 16-byte-per-lane loads (1 KiB each)
};

// The slot of X piece p (0..7, 8 k each) of tile column n in a ring buffer.
__device__ __forceinline__ uint32_t kx_xslot(uint32_t n, uint32_t p) {
  const uint32_t b = n & 7u, f = (b >> 1) | (((n >> 3) & 1u) << 2);
  return 64u * (n >> 3) + 8u * b + (p ^ f);
}

template <int RT, int NT, int KS, int PF>
__device__ __forceinline__ void q4k_matmul_kx(const uint8_t *__restrict__ q,
                                              const uint16_t *__restrict__ x,
                                              float *__restrict__ y, const MatmulArgs a,
                                              f32x4_t *lds) {
  static_assert(KS % 4 == 0, "each wave keeps one 64-wide chunk of the superblocks it visits");
  using L = KxLayout<RT, NT>;
  static_assert(L::kPerStep * (PF - 1) <= 63, "loads in flight must fit the load counter");
  constexpr uint32_t kSbStride = KS / 4;
  constexpr int kTiles = RT * NT;
  constexpr uint32_t kBufSlots = 64u * L::kPerStep; // 16-byte slots per ring buffer
  constexpr bool kTileOuter = NT == 4;
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t c = wave & 3u, sb0 = wave >> 2;
  const uint32_t fr = lane & 15u, g = lane >> 4;
  const uint32_t n_rows = a.n_rows, nsb = a.sb_per_row, batch = a.batch;
  const uint32_t K = nsb * 256u;
  const uint32_t row_bytes = nsb * (uint32_t)kQ4kSbBytes;
  const __amdgpu_buffer_rsrc_t qr = rsrc(q, n_rows * row_bytes);
  const __amdgpu_buffer_rsrc_t xr = rsrc(x, batch * K * 2u);
  const uint32_t m0 = blockIdx.x * (16u * RT), n0 = blockIdx.y * (16u * NT);
  f32x4_t *ring = lds + wave * (uint32_t)PF * kBufSlots;

  // The wave's superblocks sb0 + kSbStride * t, t < n_my, are visited from a
  // per-workgroup start, so that the workgroups of an XCD (dealt round-robin
  // to the 8 XCDs) do not all read the same stretch of X at once.
  const uint32_t n_my = sb0 < nsb ? (nsb - sb0 + kSbStride - 1u) / kSbStride : 0u;
  const uint32_t rot = n_my ? ((blockIdx.x >> 3) + blockIdx.y) % n_my : 0u;

  // Load roles (fixed per lane).  X instruction u: lane l takes the piece
  // whose slot is 64u + l (kx_xslot).  Weights: piece P = 64m + lane
  // -> row P / 3, part P % 3 (0 header, 1-2 qs halves of the chunk).  The
  // step's superblock enters as an SGPR offset (X: 512 bytes, weights: 144
  // per superblock) over these per-lane offsets; lanes past the matrix or the
  // batch start far past any buffer, so they read zeros whatever the step.
  // (A/B in one run, 14336 x 4096: B = 128 28.8-29.4 vs 30.5-31.2 us, B = 64
  // 22.2 vs 23.6, against per-lane offsets recomputed every step.)
  constexpr uint32_t kFar = 0xFFF00000u;
  uint32_t xoff0[2 * NT];
#pragma unroll
  for (int u = 0; u < 2 * NT; ++u) {
    const uint32_t b = n0 + 8u * (uint32_t)u + (lane >> 3);
    const uint32_t p = (lane & 7u) ^ ((lane >> 4) | (((uint32_t)u & 1u) << 2));
    xoff0[u] = b < batch ? (b * K + 64u * c + 8u * p) * 2u : kFar;
  }
  uint32_t woff0[L::kW];
#pragma unroll
  for (int m = 0; m < L::kW; ++m) {
    const uint32_t P = 64u * (uint32_t)m + lane, r = P / 3u, part = P - 3u * r;
    const uint32_t row = m0 + r;
    woff0[m] = (r < 16u * RT && row < n_rows)
                   ? row * row_bytes + (part == 0u ? 0u : 16u + 32u * c + 16u * (part - 1u))
                   : kFar;
  }

  // step j -> ring buffer j % PF (steps are issued in order); past the wave's
  // last step the loads read superblocks of its own range again, never used
  uint32_t it = rot; // the wave's superblock index of the next step issued
  auto issue = [&](uint32_t j) {
    const uint32_t sb = sb0 + kSbStride * it;
    it = it + 1u == n_my ? 0u : it + 1u;
    f32x4_t *buf = ring + (j % (uint32_t)PF) * kBufSlots;
#pragma unroll
    for (int u = 0; u < 2 * NT; ++u)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void_t *)(buf + u * 64), 16, xoff0[u],
                                               sb * 512u, 0, 0);
#pragma unroll
    for (int m = 0; m < L::kW; ++m)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(qr, (lds_void_t *)(buf + (L::kX + m) * 64), 16,
                                               woff0[m], sb * 144u, 0, 0);
  };

  f32x4_t acc[RT][NT];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};

#pragma unroll
  for (int p = 0; p < PF; ++p) issue((uint32_t)p);

  // Fragment read slots (fixed per lane).
  const uint32_t xs0 = kx_xslot(fr, g), xs1 = kx_xslot(fr, 4u + g);
  for (uint32_t j = 0; j < n_my; ++j) {
    // this step's loads are done when at most (PF - 1) steps' loads remain
    if constexpr (PF == 2)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(L::kPerStep) : "memory");
    else if constexpr (PF == 3)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * L::kPerStep) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const f32x4_t *buf = ring + (j % (uint32_t)PF) * kBufSlots;
    uint4 hd[RT];
    uint2 qw[RT];
    half8_t xf[2][NT];
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const uint32_t r3 = 3u * (16u * (uint32_t)i + fr);
      const f32x4_t *wp = buf + L::kX * 64 + r3;
      hd[i] = __builtin_bit_cast(uint4, wp[0]);
      qw[i] = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint8_t *>(wp + 1 + (g >> 1)) +
                                               8u * (g & 1u));
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      xf[0][t] = __builtin_bit_cast(half8_t, buf[128 * t + xs0]);
      xf[1][t] = __builtin_bit_cast(half8_t, buf[128 * t + xs1]);
    }
    // the buffer is refilled only after every read of it has returned
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    half8_t af[RT][2];
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const float d = f16_to_f32(hd[i].x & 0xFFFFu), dmin = f16_to_f32(hd[i].x >> 16);
      uint32_t scp, mp;
      q4k_scale_min_pair(hd[i].y, hd[i].z, hd[i].w, c, &scp, &mp);
      const float d1s = d * (float)(scp & 0xFFu) * 16777216.0f;
      const float d2s = d * (float)(scp >> 8) * 1048576.0f;
      const float m1 = dmin * (float)(mp & 0xFFu), m2 = dmin * (float)(mp >> 8);
      uint32_t l0, l1, h0, h1, l2, l3, h2, h3;
      dequant_dword(qw[i].x, d1s, m1, d2s, m2, l0, l1, h0, h1);
      dequant_dword(qw[i].y, d1s, m1, d2s, m2, l2, l3, h2, h3);
      af[i][0] = __builtin_bit_cast(half8_t, make_uint4(l0, l1, l2, l3));
      af[i][1] = __builtin_bit_cast(half8_t, make_uint4(h0, h1, h2, h3));
    }
    // The refill loads go out among the MFMAs instead of as one burst, which
    // filled the load unit's queue and held the wave.  With 4 column tiles
    // the MFMAs run tile by tile, so that row tile i + 1's dequantisation
    // sits among row tile i's MFMAs (a first tile's worth of VALU, then
    // MFMA, 3 VALU, MFMA, 3 VALU, load, MFMA per load); otherwise the
    // dequantisation comes first and every load sits between MFMAs.
    if constexpr (kTileOuter) {
      issue(j + (uint32_t)PF);
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
          for (int t = 0; t < NT; ++t)
            acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i][kk], xf[kk][t], acc[i][t], 0, 0, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 40, 0);
#pragma unroll
      for (int k = 0; k < L::kPerStep; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
    } else {
      __builtin_amdgcn_sched_barrier(0);
      issue(j + (uint32_t)PF);
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
          for (int t = 0; t < NT; ++t)
            acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i][kk], xf[kk][t], acc[i][t], 0, 0, 0);
      constexpr int kPer = (2 * RT * NT) / L::kPerStep > 0 ? (2 * RT * NT) / L::kPerStep : 1;
#pragma unroll
      for (int k = 0; k < L::kPerStep; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, kPer, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  // Ring loads past the wave's last step are still landing: drain them, and
  // let every wave finish with its ring before the LDS is reused.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  // Partial tiles -> LDS as red[wave][tile][lane]; wave w then owns tiles w, w + KS, ...
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int t = 0; t < NT; ++t) lds[(wave * kTiles + (uint32_t)(i * NT + t)) * 64u + lane] = acc[i][t];
  __syncthreads();
  for (uint32_t tt = wave; tt < (uint32_t)kTiles; tt += KS) {
    f32x4_t s = lds[tt * 64u + lane];
#pragma unroll
    for (uint32_t w = 1; w < (uint32_t)KS; ++w) s += lds[(w * kTiles + tt) * 64u + lane];
    const uint32_t i = tt / NT, t = tt - i * NT;
    const uint32_t b = n0 + 16u * t + fr;
    const uint32_t r0 = m0 + 16u * i + 4u * g;
    if (b >= batch) continue;
    store_col4(y + (size_t)b * n_rows, r0, n_rows, s);
  }
}

// ---------------------------------------------------------------------------
// Long rows over few of them (kind 9, axh_q4k_matmul_lk_c{XC}_x{XD}_w{WD}[_r2]):
// a workgroup of 8 waves owns 16 * RT rows (RT = 1, or 2 with _r2: each wave
// then works on two 16-row tiles) and XC = 8 or 16 columns and
// walks K in chunks of 8 superblocks, wave w taking superblock w of every
// chunk.  A lane (row r = lane % 16, k-block g = lane / 16) loads the row's
// header and the 32 qs bytes of chunk g of that superblock into registers,
// WD chunks ahead, and dequantises them into the A fragments of 8 MFMA steps,
// as q4k_matmul_sr does.  X for a chunk (XC columns x 2048 k, 4 KiB per
// column) is staged in a ring of XD + 1 LDS buffers by coalesced direct-to-LDS
// loads shared by the waves, XD chunks ahead: instruction (n, pc) copies 1 KiB
// of column n (superblocks 2pc and 2pc + 1 of the chunk), lane l taking
// 16-byte piece l ^ n, so that the 16 lanes of a fragment read (columns
// 0..15, same piece) hit distinct banks.  One barrier per chunk.  Unlike
// q4k_matmul_sr, which keeps X fragments in VGPRs and so stops at K = 4096,
// any K fits; each workgroup reads X once, from L2.  At the end the 8 partial
// 16x16 tiles are summed in LDS in wave order (deterministic).  For XC = 8
// the lanes of MFMA columns 8..15 hold zero X fragments and store nothing.
// ---------------------------------------------------------------------------
template <int XC, int XD, int WD, int RT = 1>
__device__ __forceinline__ void q4k_matmul_lk(const uint8_t *__restrict__ q,
                                              const uint16_t *__restrict__ x,
                                              float *__restrict__ y, const MatmulArgs a,
                                              f32x4_t *lds) {
  static_assert(XC == 4 || XC == 8 || XC == 16, "4, 8 or 16 columns per workgroup");
  static_assert(RT == 1 || RT == 2, "16 or 32 rows per workgroup");
  constexpr int NW = 8, XR = XD + 1, WR = WD + 1; // ring slots of X (LDS) and weights (VGPRs)
  static_assert(XD >= 1 && WD >= XD && WR % XR == 0 && WR <= 8,
                "the weights run at least as far ahead as X, in a ring of whole X rings");
  constexpr uint32_t kColB = 4096u;            // staged bytes of one column per chunk
  constexpr uint32_t kSlot = XC * kColB / 16u; // f32x4 slots of an X buffer
  constexpr int kXL = XC * 4 / NW;             // X instructions per wave per chunk
  constexpr int kPer = kXL + 3 * RT;           // loads per wave per chunk
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t r = lane & 15u, g = lane >> 4;
  const uint32_t n_rows = a.n_rows, nsb = a.sb_per_row, batch = a.batch;
  const uint32_t K = nsb * 256u;
  const uint32_t row_bytes = nsb * (uint32_t)kQ4kSbBytes;
  const __amdgpu_buffer_rsrc_t qr = rsrc(q, n_rows * row_bytes);
  const __amdgpu_buffer_rsrc_t xr = rsrc(x, batch * K * 2u);
  const uint32_t n_ch = (nsb + 7u) >> 3;
  const uint32_t m0 = 16u * RT * blockIdx.x, n0 = XC * blockIdx.y;
  const uint32_t rr = r & (uint32_t)(XC - 1); // the lane's column within the group

  // Per-lane offsets are prepared once and the chunk enters as an SGPR
  // offset; loads past the last superblock or column read zeros (kFar, with
  // room for the SGPR offset on top).
  constexpr uint32_t kFar = 0xFFF00000u;
  uint32_t xv0[kXL];
#pragma unroll
  for (int m = 0; m < kXL; ++m) {
    const uint32_t qi = wave + (uint32_t)(NW * m), n = qi >> 2, col = n0 + n;
    xv0[m] = col < batch ? col * K * 2u + 16u * (lane ^ n) : kFar;
  }
  const uint32_t xhalf = lane >> 5; // superblock of the lane's piece within the pair
  uint32_t wv0[RT];
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    const uint32_t row = m0 + 16u * (uint32_t)i + r;
    wv0[i] = row < n_rows ? row * row_bytes : kFar;
  }
  // X of chunk c into X slot xs (this wave's instructions)
  auto issue_x = [&](uint32_t c, auto xs_c) {
    constexpr int xs = decltype(xs_c)::value;
    f32x4_t *buf = lds + xs * kSlot;
#pragma unroll
    for (int m = 0; m < kXL; ++m) {
      const uint32_t qi = wave + (uint32_t)(NW * m), n = qi >> 2, pc = qi & 3u;
      const uint32_t s0 = 8u * c + 2u * pc;
      const uint32_t v = s0 + xhalf < nsb ? xv0[m] : kFar;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void_t *)(buf + n * (kColB / 16u) + pc * 64u),
                                               16, v, 512u * s0, 0, 0);
    }
  };
  // weights of superblock 8c + wave (each row tile) into register slot ws
  uint4 H[WR][RT], QA[WR][RT], QB[WR][RT];
  auto issue_w = [&](uint32_t c, auto ws_c) {
    constexpr int ws = decltype(ws_c)::value;
    const uint32_t sb = 8u * c + wave;
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const uint32_t v = sb < nsb ? wv0[i] : kFar;
      const u32x4_t h = __builtin_amdgcn_raw_buffer_load_b128(qr, (int)v, (int)(sb * 144u), 0);
      const u32x4_t qa =
          __builtin_amdgcn_raw_buffer_load_b128(qr, (int)(v + 16u + 32u * g), (int)(sb * 144u), 0);
      const u32x4_t qb =
          __builtin_amdgcn_raw_buffer_load_b128(qr, (int)(v + 32u + 32u * g), (int)(sb * 144u), 0);
      H[ws][i] = make_uint4(h.x, h.y, h.z, h.w);
      QA[ws][i] = make_uint4(qa.x, qa.y, qa.z, qa.w);
      QB[ws][i] = make_uint4(qb.x, qb.y, qb.z, qb.w);
    }
  };
  // X fragment of step t: piece P = 32 (wave & 1) + 8g + t of the wave's
  // superblock pair wave >> 1 in column rr.
  uint32_t xa[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const uint32_t P = 32u * (wave & 1u) + 8u * g + (uint32_t)t;
    xa[t] = rr * (kColB / 16u) + 64u * (wave >> 1) + (P ^ rr);
  }
  f32x4_t acc[RT];
#pragma unroll
  for (int i = 0; i < RT; ++i) acc[i] = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};
  // Chunk c (c % WR = e) issues X of chunk c + XD after its barrier, then
  // the weights of chunk c + WD halfway through its MFMAs (issued with the X
  // loads, the burst filled the load unit's queue and held the waves: A/B in
  // one run at 4096 x 14336, B = 8 13.31 vs 12.39 us, B = 16 15.92 vs 15.32,
  // B = 32 23.21 vs 22.17; at the end of the step, B = 32 took 23.05).  The
  // issue order is fixed, so the loads issued after X of chunk c are always
  // the 3 * RT weight loads of its group and the XD - 1 groups in between:
  // waiting for that many leaves the weights ahead in flight.
  auto step = [&](uint32_t c, auto e_c) {
    constexpr int e = decltype(e_c)::value;
    // own X of chunk c landed; after the barrier every wave's X of chunk c is
    // in LDS and chunk c - 1's X buffer is free
    static_assert((XD - 1) * kPer + 3 * RT <= 63, "vmcnt holds 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((XD - 1) * kPer + 3 * RT) : "memory");
    __builtin_amdgcn_sched_barrier(0);
    issue_x(c + (uint32_t)XD, std::integral_constant<int, (e + XD) % XR>{});
    __builtin_amdgcn_sched_barrier(0);
    const f32x4_t *buf = lds + (e % XR) * kSlot;
    half8_t xf[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const half8_t v = __builtin_bit_cast(half8_t, buf[xa[t]]);
      xf[t] = r < (uint32_t)XC ? v : (half8_t){};
    }
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const uint4 hd = H[e][i];
      const float d = f16_to_f32(hd.x & 0xFFFFu), dmin = f16_to_f32(hd.x >> 16);
      uint32_t scp, mp;
      q4k_scale_min_pair(hd.y, hd.z, hd.w, g, &scp, &mp);
      const float d1s = d * (float)(scp & 0xFFu) * 16777216.0f;
      const float d2s = d * (float)(scp >> 8) * 1048576.0f;
      const float m1 = dmin * (float)(mp & 0xFFu), m2 = dmin * (float)(mp >> 8);
      const uint32_t w[8] = {QA[e][i].x, QA[e][i].y, QA[e][i].z, QA[e][i].w,
                             QB[e][i].x, QB[e][i].y, QB[e][i].z, QB[e][i].w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        uint32_t l0, l1, h0, h1, l2, l3, h2, h3;
        dequant_dword(w[2 * t], d1s, m1, d2s, m2, l0, l1, h0, h1);
        dequant_dword(w[2 * t + 1], d1s, m1, d2s, m2, l2, l3, h2, h3);
        const half8_t alo = __builtin_bit_cast(half8_t, make_uint4(l0, l1, l2, l3));
        const half8_t ahi = __builtin_bit_cast(half8_t, make_uint4(h0, h1, h2, h3));
        acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, xf[t], acc[i], 0, 0, 0);
        acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, xf[t + 4], acc[i], 0, 0, 0);
        if (4 * i + t == 2 * RT - 1) { // halfway
          __builtin_amdgcn_sched_barrier(0);
          issue_w(c + (uint32_t)WD, std::integral_constant<int, (e + WD) % WR>{});
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  };
  // Prologue: the groups chunks -WD .. -1 would have issued (weights of
  // chunks 0 .. WD - 1, X of chunks 0 .. XD - 1), in the same order.
  auto pro = [&](auto i_c) {
    constexpr int i = decltype(i_c)::value; // the group of chunk i - WD
    if constexpr (i < WD) {
      if constexpr (i - WD + XD >= 0)
        issue_x((uint32_t)(i - WD + XD), std::integral_constant<int, (i - WD + XD) % XR>{});
      issue_w((uint32_t)i, std::integral_constant<int, i>{});
    }
  };
  pro(std::integral_constant<int, 0>{});
  pro(std::integral_constant<int, 1>{});
  pro(std::integral_constant<int, 2>{});
  pro(std::integral_constant<int, 3>{});
  pro(std::integral_constant<int, 4>{});
  pro(std::integral_constant<int, 5>{});
  pro(std::integral_constant<int, 6>{});
  // Whole rounds of WR chunks, then the rest: no step of the loop body is
  // conditional, so no load is left in flight on a path around the back edge
  // (which made the compiler wait for every load at the loop head).
  auto round = [&](uint32_t c0, auto e_c, bool guard) {
    constexpr int e = decltype(e_c)::value;
    if constexpr (e < WR)
      if (!guard || c0 + (uint32_t)e < n_ch) step(c0 + (uint32_t)e, e_c);
  };
  uint32_t c0 = 0;
  for (; c0 + (uint32_t)WR <= n_ch; c0 += (uint32_t)WR) {
    round(c0, std::integral_constant<int, 0>{}, false);
    round(c0, std::integral_constant<int, 1>{}, false);
    round(c0, std::integral_constant<int, 2>{}, false);
    round(c0, std::integral_constant<int, 3>{}, false);
    round(c0, std::integral_constant<int, 4>{}, false);
    round(c0, std::integral_constant<int, 5>{}, false);
    round(c0, std::integral_constant<int, 6>{}, false);
    round(c0, std::integral_constant<int, 7>{}, false);
  }
  round(c0, std::integral_constant<int, 0>{}, true);
  round(c0, std::integral_constant<int, 1>{}, true);
  round(c0, std::integral_constant<int, 2>{}, true);
  round(c0, std::integral_constant<int, 3>{}, true);
  round(c0, std::integral_constant<int, 4>{}, true);
  round(c0, std::integral_constant<int, 5>{}, true);
  round(c0, std::integral_constant<int, 6>{}, true);
  // every load (the ones past the last chunk too) has landed before the LDS
  // is reused and before the waves end
  f32x4_t *red = lds + XR * kSlot;
#pragma unroll
  for (int i = 0; i < RT; ++i) red[(wave * RT + (uint32_t)i) * 64u + lane] = acc[i];
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if (wave < (uint32_t)RT) { // wave i sums and stores row tile i
    f32x4_t sum = red[wave * 64u + lane];
#pragma unroll
    for (uint32_t w2 = 1; w2 < (uint32_t)NW; ++w2) sum += red[(w2 * RT + wave) * 64u + lane];
    const uint32_t col = n0 + r;
    if (r < (uint32_t)XC && col < batch)
      store_col4(y + (size_t)col * n_rows, m0 + 16u * wave + 4u * g, n_rows, sum);
  }
}

// ---------------------------------------------------------------------------
// 32 x 32 tiles with wide waves (kind 8, axh_q4k_matmul_rm_w{W}_r{RT}_p4): a
// workgroup of W waves owns 32 * RT * W rows x 128 columns of Y; wave w owns
// 32 * RT rows (RT 32-row MFMA tiles) x 128 columns (four 32-column tiles) and
// walks all of K in 64-wide steps (one chunk of a superblock) with
// v_mfma_f32_32x32x16_f16, so each X fragment read from LDS feeds RT MFMAs of
// 32 rows (16x16 tiles: 16 rows) and each dequantised A
// fragment four (128 columns).  A ring of 4 LDS buffers, each the step's X
// tile (128 columns x 64 k, 16 KiB) and every wave's weight pieces (per row:
// header and the chunk's 32 qs bytes), is filled by direct-to-LDS loads three
// steps ahead; each step's fragments (X read from LDS, A dequantised) are
// prepared during the previous step's MFMAs.  Lane l (row l % 32 of a row
// tile, half h = l / 32) dequantises the qs bytes [16h, 16h + 16) of the
// chunk: their low nibbles are the A fragments of k-steps 0-1 (k = 16h +
// 0..15), their high nibbles those of k-steps 2-3 (k = 32 + 16h + ..), each 8
// consecutive k, so the X fragment of the same (k-step, half) is one 16-byte
// piece.  X piece p of column n sits in slot p ^ ((n >> 1) & 7) of the
// column's 128 bytes: columns n and n + 1 lie in the two 128-byte halves of
// the 64 banks, so 16 lanes reading one piece of 16 consecutive columns hit
// 16 distinct 16-byte bank groups (with p ^ (n & 7), columns n and n + 8
// collided).  One barrier per step makes every wave's X of step j + 1 visible and
// frees the buffer the next loads refill.
// The step loop is unrolled by the ring depth, so a step's ring slot and
// chunk are compile-time constants: the LDS addresses of the fragment reads
// are a per-lane base plus immediates, the scale decode of a chunk is
// specialised, and the direct-to-LDS loads take the step's offset in an SGPR
// (X: 128 bytes per step, weights: 144 bytes per superblock) over per-lane
// offsets prepared once.  Each X fragment is refilled for the next step right
// after the step's last MFMA that reads it, and the next step's
// dequantisation is written between the MFMAs.  That takes the VALU work per
// step from 111 to 86 instructions (32 rows) and measured, A/B in one run at
// 14336 x 4096: B = 256 (4 waves) 44.8 vs 52.8 us, B = 512 (8 waves) 78.5 vs
// 79.1.  (The compiler's own schedule is kept: a fixed MFMA / LDS read / VALU
// pattern through sched_group_barrier put dependent MFMAs back to back, and
// sched_barrier fences between the groups measured even.)
typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <int W, int RT>
__device__ __forceinline__ void q4k_matmul_rm(const uint8_t *__restrict__ q,
                                              const uint16_t *__restrict__ x,
                                              float *__restrict__ y, const MatmulArgs a,
                                              f32x4_t *lds) {
  static_assert(W == 1 || W == 2 || W == 4 || W == 8, "16 X instructions per step over the waves");
  static_assert(RT == 1 || RT == 2, "32 or 64 rows per wave");
  constexpr int kXPer = 16 / W;                   // X instructions per wave per step
  constexpr int kWI = (96 * RT + 63) / 64;        // weight instructions (32 RT rows x 48 B)
  constexpr int kPerStep = kXPer + kWI;
  constexpr uint32_t kWs = 64u * kWI;             // f32x4 slots of a wave's weight pieces
  constexpr uint32_t kBuf = 16u * 64u + W * kWs;  // f32x4 slots per ring buffer
  // Offset of loads that must read zeros: past any buffer the runtime passes
  // (below 4 GiB - 1 MiB), with room for the SGPR step offsets on top.
  constexpr uint32_t kFar = 0xFFF00000u;
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t r = lane & 31u, h = lane >> 5;
  const uint32_t n_rows = a.n_rows, nsb = a.sb_per_row, batch = a.batch;
  const uint32_t K = nsb * 256u, n_steps = 4u * nsb;
  const uint32_t row_bytes = nsb * (uint32_t)kQ4kSbBytes;
  const __amdgpu_buffer_rsrc_t qr = rsrc(q, n_rows * row_bytes);
  const __amdgpu_buffer_rsrc_t xr = rsrc(x, batch * K * 2u);
  const uint32_t m0 = blockIdx.x * (32u * RT * W) + 32u * RT * wave, n0 = blockIdx.y * 128u;

  // X load role: instruction i = wave + W * u covers columns 8i .. 8i + 7;
  // lane L loads piece (L & 7) ^ ((col >> 1) & 7) of column 8i + L / 8.  Step j
  // adds 128 j bytes (SGPR offset).
  uint32_t xv0[kXPer];
#pragma unroll
  for (int u = 0; u < kXPer; ++u) {
    const uint32_t i = wave + (uint32_t)(W * u), col = 8u * i + (lane >> 3);
    const uint32_t p = (lane & 7u) ^ ((col >> 1) & 7u), b = n0 + col;
    xv0[u] = b < batch ? (b * K + 8u * p) * 2u : kFar;
  }
  // Weight load role: piece P = 64m + lane -> row P / 3 of the wave's 32 RT,
  // part P % 3 (0 the header, 1-2 the 16-byte halves of the chunk's qs), one
  // per-lane offset for each chunk c; superblock j / 4 adds 144 (j / 4) bytes.
  uint32_t wv0[kWI][4];
#pragma unroll
  for (int m = 0; m < kWI; ++m) {
    const uint32_t P = 64u * (uint32_t)m + lane, rr = P / 3u, part = P - 3u * rr, row = m0 + rr;
    const uint32_t base = (rr < 32u * RT && row < n_rows) ? row * row_bytes : kFar;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      wv0[m][c] = base == kFar ? kFar : base + (part == 0u ? 0u : 16u * part + 32u * (uint32_t)c);
  }
  // step j -> ring buffer j % 4 (a compile-time slot); past the last step the
  // loads read bytes that are never used, or zeros past the buffers
  auto issue = [&](uint32_t j, auto slot_c) {
    constexpr int sl = decltype(slot_c)::value;
    f32x4_t *buf = lds + sl * kBuf;
#pragma unroll
    for (int u = 0; u < kXPer; ++u) {
      const uint32_t i = wave + (uint32_t)(W * u);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void_t *)(buf + i * 64u), 16, xv0[u],
                                               128u * j, 0, 0);
    }
    f32x4_t *wb = buf + 16u * 64u + wave * kWs;
#pragma unroll
    for (int m = 0; m < kWI; ++m)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(qr, (lds_void_t *)(wb + m * 64), 16, wv0[m][sl],
                                               (j >> 2) * 144u, 0, 0);
  };
  // A fragments of a step from its ring buffer: af[i][s], s the k-step.
  auto dequant = [&](const f32x4_t *buf, uint32_t c, half8_t (&af)[RT][4]) {
    const f32x4_t *wb = buf + 16u * 64u + wave * kWs;
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const uint32_t pr = 3u * (32u * (uint32_t)i + r); // the row's three pieces
      const uint4 hd = __builtin_bit_cast(uint4, wb[pr]);
      const uint4 qv = __builtin_bit_cast(uint4, wb[pr + 1u + h]);
      const float d = f16_to_f32(hd.x & 0xFFFFu), dmin = f16_to_f32(hd.x >> 16);
      uint32_t scp, mp;
      q4k_scale_min_pair(hd.y, hd.z, hd.w, c, &scp, &mp);
      const float d1s = d * (float)(scp & 0xFFu) * 16777216.0f;
      const float d2s = d * (float)(scp >> 8) * 1048576.0f;
      const float m1 = dmin * (float)(mp & 0xFFu), m2 = dmin * (float)(mp >> 8);
      uint32_t l[4][2], hh[4][2];
      dequant_dword(qv.x, d1s, m1, d2s, m2, l[0][0], l[0][1], hh[0][0], hh[0][1]);
      dequant_dword(qv.y, d1s, m1, d2s, m2, l[1][0], l[1][1], hh[1][0], hh[1][1]);
      dequant_dword(qv.z, d1s, m1, d2s, m2, l[2][0], l[2][1], hh[2][0], hh[2][1]);
      dequant_dword(qv.w, d1s, m1, d2s, m2, l[3][0], l[3][1], hh[3][0], hh[3][1]);
      af[i][0] = __builtin_bit_cast(half8_t, make_uint4(l[0][0], l[0][1], l[1][0], l[1][1]));
      af[i][1] = __builtin_bit_cast(half8_t, make_uint4(l[2][0], l[2][1], l[3][0], l[3][1]));
      af[i][2] = __builtin_bit_cast(half8_t, make_uint4(hh[0][0], hh[0][1], hh[1][0], hh[1][1]));
      af[i][3] = __builtin_bit_cast(half8_t, make_uint4(hh[2][0], hh[2][1], hh[3][0], hh[3][1]));
    }
  };
  // X fragment (k-step s, column tile t) of this lane: piece p(s) = (s & 1) +
  // 2h + 4 (s >> 1) of column 32t + r, at f32x4 slot xl[s] + 256 t of a buffer.
  uint32_t xl[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const uint32_t p = ((uint32_t)s & 1u) + 2u * h + 4u * ((uint32_t)s >> 1);
    xl[s] = 8u * r + (p ^ ((r >> 1) & 7u));
  }
  f32x16_t acc[RT][4];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[i][t] = (f32x16_t){};
  issue(0u, std::integral_constant<int, 0>{});
  issue(1u, std::integral_constant<int, 1>{});
  issue(2u, std::integral_constant<int, 2>{});
  half8_t af[2][RT][4]; // A fragments of steps jj and jj + 1
  half8_t bf[4][4];     // X fragments, each refilled for step jj + 1 once step jj's MFMAs read it
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(2 * kPerStep) : "memory"); // step 0 landed
  dequant(lds, 0u, af[0]);
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int t = 0; t < 4; ++t) bf[s][t] = __builtin_bit_cast(half8_t, lds[xl[s] + 256u * (uint32_t)t]);
  // Step jj's MFMAs, with step jj + 1's X fragments read and its A fragments
  // dequantised between them (per row tile: the scale decode, then the four
  // qs dwords in low and high halves).
  auto step = [&](uint32_t jj, auto e_c) {
    constexpr int e = decltype(e_c)::value; // jj % 4: the ring slot
    constexpr int sn = (e + 1) & 3;         // slot and chunk of step jj + 1
    // own loads of step jj + 1 landed (jj + 2 in flight); after the barrier
    // every wave's X of step jj + 1 is in LDS and step jj - 1's buffer is free
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kPerStep) : "memory");
    issue(jj + 3u, std::integral_constant<int, (e + 3) & 3>{});
    const f32x4_t *bufn = lds + sn * kBuf; // past the last step: read, never used
    const f32x4_t *wb = bufn + 16u * 64u + wave * kWs;
    uint4 hd[RT], qv[RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const uint32_t pr = 3u * (32u * (uint32_t)i + r); // the row's three pieces
      hd[i] = __builtin_bit_cast(uint4, wb[pr]);
      qv[i] = __builtin_bit_cast(uint4, wb[pr + 1u + h]);
    }
    float dd[RT], dm[RT], d1s[RT], d2s[RT], m1[RT], m2[RT];
    uint32_t scp[RT], mp[RT], lo[RT][4][2], hi[RT][4][2];
#pragma unroll
    for (int k = 0; k < 16 * RT; ++k) {
      const int s = k / (4 * RT), i = (k >> 2) % RT, t = k & 3;
      acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[e & 1][i][s], bf[s][t], acc[i][t], 0, 0, 0);
      if (i == RT - 1)
        bf[s][t] = __builtin_bit_cast(half8_t, bufn[xl[s] + 256u * (uint32_t)t]);
      const int ii = k >> 4, kk = k & 15; // dequantisation work of row tile ii
      if (kk == 2) {
        dd[ii] = f16_to_f32(hd[ii].x & 0xFFFFu);
        dm[ii] = f16_to_f32(hd[ii].x >> 16);
        q4k_scale_min_pair(hd[ii].y, hd[ii].z, hd[ii].w, (uint32_t)sn, &scp[ii], &mp[ii]);
      } else if (kk == 3) {
        d1s[ii] = dd[ii] * (float)(scp[ii] & 0xFFu) * 16777216.0f;
        d2s[ii] = dd[ii] * (float)(scp[ii] >> 8) * 1048576.0f;
        m1[ii] = dm[ii] * (float)(mp[ii] & 0xFFu);
        m2[ii] = dm[ii] * (float)(mp[ii] >> 8);
      } else if (kk >= 4 && kk < 12) {
        const int dw = (kk - 4) >> 1;
        const uint32_t w = dw == 0 ? qv[ii].x : dw == 1 ? qv[ii].y : dw == 2 ? qv[ii].z : qv[ii].w;
        const uint32_t w8 = w >> 8;
        if (((kk - 4) & 1) == 0) { // low nibbles: bytes 0, 2 and 1, 3 of the dword
          const uint32_t lb = w & 0x000F000Fu, hb = w8 & 0x000F000Fu;
          lo[ii][dw][0] = pack_f16(__builtin_fmaf(lo_half_f16(lb), d1s[ii], -m1[ii]),
                                   __builtin_fmaf(lo_half_f16(hb), d1s[ii], -m1[ii]));
          lo[ii][dw][1] = pack_f16(__builtin_fmaf(hi_half_f16(lb), d1s[ii], -m1[ii]),
                                   __builtin_fmaf(hi_half_f16(hb), d1s[ii], -m1[ii]));
        } else { // high nibbles
          const uint32_t lb = w & 0x00F000F0u, hb = w8 & 0x00F000F0u;
          hi[ii][dw][0] = pack_f16(__builtin_fmaf(lo_half_f16(lb), d2s[ii], -m2[ii]),
                                   __builtin_fmaf(lo_half_f16(hb), d2s[ii], -m2[ii]));
          hi[ii][dw][1] = pack_f16(__builtin_fmaf(hi_half_f16(lb), d2s[ii], -m2[ii]),
                                   __builtin_fmaf(hi_half_f16(hb), d2s[ii], -m2[ii]));
        }
      }
    }
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      half8_t(&o)[4] = af[(e & 1) ^ 1][i];
      o[0] = __builtin_bit_cast(half8_t, make_uint4(lo[i][0][0], lo[i][0][1], lo[i][1][0], lo[i][1][1]));
      o[1] = __builtin_bit_cast(half8_t, make_uint4(lo[i][2][0], lo[i][2][1], lo[i][3][0], lo[i][3][1]));
      o[2] = __builtin_bit_cast(half8_t, make_uint4(hi[i][0][0], hi[i][0][1], hi[i][1][0], hi[i][1][1]));
      o[3] = __builtin_bit_cast(half8_t, make_uint4(hi[i][2][0], hi[i][2][1], hi[i][3][0], hi[i][3][1]));
    }
  };
  for (uint32_t j = 0; j < n_steps; j += 4) { // n_steps is a multiple of 4
    step(j, std::integral_constant<int, 0>{});
    step(j + 1u, std::integral_constant<int, 1>{});
    step(j + 2u, std::integral_constant<int, 2>{});
    step(j + 3u, std::integral_constant<int, 3>{});
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); // ring loads past the last step

#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t b = n0 + 32u * (uint32_t)t + r;
      if (b >= batch) continue;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const f32x4_t v = {acc[i][t][4 * q4], acc[i][t][4 * q4 + 1], acc[i][t][4 * q4 + 2],
                           acc[i][t][4 * q4 + 3]};
        store_col4(y + (size_t)b * n_rows, m0 + 32u * (uint32_t)i + 8u * (uint32_t)q4 + 4u * h,
                   n_rows, v);
      }
    }
}

// ---------------------------------------------------------------------------
// Streaming rows (kind 7, the default up to 32 columns and K <= 4096): a
// persistent workgroup of NW waves walks 16-row blocks b = blockIdx.x +
// k * gridDim.x for the 16 * NC columns n0 = 16 * NC * blockIdx.y ..; wave w owns
// superblocks [w*SPW, w*SPW + SPW) of every row (K split NW ways), so its X
// fragments for those superblocks stay in VGPRs for the whole kernel and
// only weights stream.  Per superblock a lane (row r = lane % 16, k-block
// g = lane / 16) loads the row's header and the 32 qs bytes of chunk g (three
// 16-byte loads, the next superblock's issued before this one is computed)
// and dequantises them into the A fragments of 8 MFMA steps: step t < 4 takes
// the low nibbles of qs bytes [32g + 8t, 32g + 8t + 8) (weights 64g + 8t ..
// of the superblock, sub-block 2g), step t + 4 their high nibbles (64g + 32 +
// 8t .., sub-block 2g + 1); the X fragment of step t holds the same k.  Each
// wave writes its partial 16x16 tiles of every block into its own X staging
// region, free once its fragments are in VGPRs, and after one barrier at the
// end (or when the regions fill: 16 blocks, 8 with two column groups or
// 8-column groups) the waves sum the blocks' tiles in wave order
// (deterministic) and store them.  A barrier and a sum after every block cost
// 6-10 %, A/B in one run at 14336 x 4096: B = 8 11.01 vs 10.35 us, B = 16
// 12.00 vs 11.21, B = 32 14.68 vs 13.23.  Against the K-split
// tile kind at 14336 x 4096: 11.2 vs 14.2 us at 8 columns, 11.8 vs 14.6 at 16,
// 15.0 vs 16.0 at 32 (NC = 2: every A fragment feeds two MFMAs).
// XH (axh_q4k_matmul_sr_w*_s*_h): column groups of 8 (lanes of MFMA columns
// 8..15 hold zero X fragments and store nothing), staged through 64 KiB, so
// the kernel needs 80 KiB of LDS and two workgroups share a CU; for at most 8
// columns, where a 16-column group would carry 8 empty ones.
template <int NW, int SPW, int NC, bool XH = false>
__device__ __forceinline__ void q4k_matmul_sr(const uint8_t *__restrict__ q,
                                              const uint16_t *__restrict__ x,
                                              float *__restrict__ y, const MatmulArgs a,
                                              f32x4_t *red) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t r = lane & 15u, g = lane >> 4;
  const uint32_t n_rows = a.n_rows, nsb = a.sb_per_row, batch = a.batch;
  const uint32_t K = nsb * 256u;
  const uint32_t row_bytes = nsb * (uint32_t)kQ4kSbBytes;
  const __amdgpu_buffer_rsrc_t qr = rsrc(q, n_rows * row_bytes);
  const __amdgpu_buffer_rsrc_t xr = rsrc(x, batch * K * 2u);
  // 16-row blocks b = blockIdx.x + k * gridDim.x.  When the last round's T
  // blocks would leave half the grid idle (2T <= grid), they are split into
  // 2T half blocks of 8 rows, one per workgroup: a half block's lane (r, g)
  // takes row r & 7 and superblock wave * SPW + (r >> 3), so every lane
  // dequantises one superblock instead of two, and the MFMAs against the X
  // fragments of the wave's first and second superblock give rows 0..7 and
  // 8..15 of two tiles whose matching halves are the row's two parts.  At
  // 14336 rows (896 blocks over 256 workgroups) every workgroup then does 3.5
  // blocks of work instead of 4 or 3: A/B in one run, 14336 x 4096 x 8 10.23-
  // 10.30 vs 10.56-10.64 us, x 16 11.43-11.61 vs 11.57-11.64, x 32 13.84-14.03
  // vs 14.06-14.37.  (Contiguous row ranges per workgroup, and 8-row halves
  // that kept two superblocks per lane, both measured slower.)
  const uint32_t n_blocks = (n_rows + 15u) >> 4, G = gridDim.x;
  const uint32_t n_full = n_blocks / G, n_tail = n_blocks - n_full * G;
  const bool split = SPW == 2 && n_tail != 0u && 2u * n_tail <= G;
  const uint32_t n_myb =
      split ? n_full : (blockIdx.x < n_blocks ? (n_blocks - 1u - blockIdx.x) / G + 1u : 0u);
  const bool half = split && blockIdx.x < 2u * n_tail;
  const uint32_t hrow0 = 16u * n_full * G + 8u * blockIdx.x; // the half block's first row
  constexpr uint32_t kXc = XH ? 8u : 16u;    // columns of a group
  const uint32_t n0 = kXc * NC * blockIdx.y; // this workgroup's kXc * NC columns
  // A wave's X staging region (f32x4 slots), free once its fragments are in
  // VGPRs; it then holds the wave's partial tiles of up to kGroup blocks.
  constexpr uint32_t kRegion = kXc * 512u * SPW / 16u;
  constexpr uint32_t kGroup = kRegion / 64u / NC;

  // Weight loads of step (k, j): row 16 b + r, superblock wave*SPW + j: header
  // and the 32 qs bytes of chunk g.  k == n_myb is the half block (one step).
  uint4 H[2], QA[2], QB[2];
  auto issue = [&](uint32_t k, int j, int slot) {
    uint32_t row, s;
    bool ok;
    if (k < n_myb) {
      row = 16u * (blockIdx.x + k * G) + r;
      s = wave * SPW + (uint32_t)j;
      ok = s < nsb;
    } else {
      row = hrow0 + (r & 7u);
      s = wave * SPW + (r >> 3);
      ok = half && k == n_myb && j == 0 && s < nsb;
    }
    const uint32_t off = ok ? row * row_bytes + s * 144u : kOob;
    H[slot] = bload16(qr, off);
    QA[slot] = bload16(qr, off == kOob ? kOob : off + 16u + 32u * g);
    QB[slot] = bload16(qr, off == kOob ? kOob : off + 32u + 32u * g);
  };
  // X fragments of the wave's superblocks (column group c, column r, k-block g
  // of step t), staged one superblock at a time through the wave-private LDS
  // region (all regions within the first 128 KiB of LDS) by coalesced
  // direct-to-LDS loads: instruction (c, m) copies superblock j's 512 bytes of
  // columns n = 2m and 2m + 1 of group c, lane l taking 16-byte piece
  // (l & 31) ^ n of column 2m + l / 32, so that the 16 lanes of a fragment
  // (columns 0..15, same piece) hit 16 different bank groups.  Superblock 0's
  // X is requested first and the first step's weights after it, so that the
  // X wait does not queue behind the weights (loads return in order); its
  // fragments go to VGPRs, then superblock 1's X is requested and lands
  // during the first step, and its fragments are read before the first step
  // that needs them (the half block reads them too).
  static_assert(SPW == 2, "X staged one superblock at a time, two per wave");
  static_assert(NW * NC * kXc * 512u <= 131072u, "X staging fits 128 KiB");
  half8_t xf[NC][SPW][8];
  typedef __attribute__((address_space(3))) void lds_void_t;
  uint8_t *const xs = reinterpret_cast<uint8_t *>(red) + wave * (kRegion * 16u);
  const uint32_t rr = r & (kXc - 1u); // the lane's column within its group
  auto stage = [&](int j) {
    const uint32_t sj = wave * SPW + (uint32_t)j;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int m = 0; m < (int)kXc / 2; ++m) {
        const uint32_t n = 2u * (uint32_t)m + (lane >> 5), col = n0 + kXc * (uint32_t)c + n;
        const uint32_t piece = (lane & 31u) ^ n;
        const uint32_t off = (col < batch && sj < nsb) ? (col * K + 256u * sj) * 2u + 16u * piece : kOob;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            xr, (lds_void_t *)(xs + (kXc * (uint32_t)c + 2u * (uint32_t)m) * 512u), 16, off, 0, 0, 0);
      }
  };
  auto read_frags = [&](int j) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const uint32_t P = 8u * g + (uint32_t)t; // 16-byte piece of the superblock
        const uint32_t addr = (kXc * (uint32_t)c + rr) * 512u + 16u * (P ^ rr);
        const half8_t v = *reinterpret_cast<const half8_t *>(xs + addr);
        xf[c][j][t] = (!XH || r < 8u) ? v : (half8_t){};
      }
  };
  stage(0);
  __builtin_amdgcn_sched_barrier(0);
  issue(0u, 0, 0); // the first step's weights
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); // superblock 0's X is in LDS
  read_frags(0);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); // read before the region is refilled
  stage(1);
  bool x1_pending = true; // superblock 1's fragments not yet in VGPRs
  // Sums the partial tiles of blocks kb .. kb + nb - 1 (and of the half
  // block after them) over the waves, in wave order, and stores them; slot tt
  // of every region (block kb + tt / NC, column group tt % NC) is summed by
  // wave tt % NW.  Lanes 0..31 of a half block's slot hold rows 0..7 against
  // the first superblock's X, lanes 32..63 the same rows against the second.
  auto flush = [&](uint32_t kb, uint32_t nb, bool with_half) {
    const uint32_t n_t = (nb + (with_half ? 1u : 0u)) * NC;
    for (uint32_t tt = wave; tt < n_t; tt += NW) {
      const uint32_t sblk = tt / NC, c = tt - sblk * NC;
      const f32x4_t *sl = red + tt * 64u;
      const uint32_t col = n0 + kXc * c + r;
      const bool ok = (!XH || r < 8u) && col < batch;
      if (sblk < nb) {
        f32x4_t sum = sl[lane];
#pragma unroll
        for (int w2 = 1; w2 < NW; ++w2) sum += sl[(uint32_t)w2 * kRegion + lane];
        const uint32_t b = blockIdx.x + (kb + sblk) * G;
        if (ok) store_col4(y + (size_t)col * n_rows, 16u * b + 4u * g, n_rows, sum);
      } else if (lane < 32u) {
        f32x4_t sum = sl[lane] + sl[lane + 32u];
#pragma unroll
        for (int w2 = 1; w2 < NW; ++w2)
          sum += sl[(uint32_t)w2 * kRegion + lane] + sl[(uint32_t)w2 * kRegion + lane + 32u];
        if (ok) store_col4(y + (size_t)col * n_rows, hrow0 + 4u * g, n_rows, sum);
      }
    }
  };
  f32x4_t acc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) acc[c] = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};
  uint32_t kb = 0; // first block whose partial tiles are not yet summed
  for (uint32_t k = 0; k < n_myb; ++k) {
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      const int slot = j & 1;  // SPW even: slot parity follows j
      __builtin_amdgcn_sched_barrier(0);
      if (j + 1 < SPW) issue(k, j + 1, slot ^ 1);
      else issue(k + 1u, 0, slot ^ 1);
      __builtin_amdgcn_sched_barrier(0);
      if (j == 1 && x1_pending) {
        // superblock 1's X landed: at most the 3 weight loads just issued
        // remain (this step's own weights, issued before them, are needed now)
        asm volatile("s_waitcnt vmcnt(3)" ::: "memory");
        read_frags(1);
        x1_pending = false;
      }
      const uint4 hd = H[slot];
      const float d = f16_to_f32(hd.x & 0xFFFFu), dmin = f16_to_f32(hd.x >> 16);
      uint32_t scp, mp;
      q4k_scale_min_pair(hd.y, hd.z, hd.w, g, &scp, &mp);
      const float d1s = d * (float)(scp & 0xFFu) * 16777216.0f;
      const float d2s = d * (float)(scp >> 8) * 1048576.0f;
      const float m1 = dmin * (float)(mp & 0xFFu), m2 = dmin * (float)(mp >> 8);
      const uint32_t w[8] = {QA[slot].x, QA[slot].y, QA[slot].z, QA[slot].w,
                             QB[slot].x, QB[slot].y, QB[slot].z, QB[slot].w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        uint32_t l0, l1, h0, h1, l2, l3, h2, h3;
        dequant_dword(w[2 * t], d1s, m1, d2s, m2, l0, l1, h0, h1);
        dequant_dword(w[2 * t + 1], d1s, m1, d2s, m2, l2, l3, h2, h3);
        const half8_t alo = __builtin_bit_cast(half8_t, make_uint4(l0, l1, l2, l3));
        const half8_t ahi = __builtin_bit_cast(half8_t, make_uint4(h0, h1, h2, h3));
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, xf[c][j][t], acc[c], 0, 0, 0);
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, xf[c][j][t + 4], acc[c], 0, 0, 0);
        }
      }
    }
    // partial tiles of block k -> the wave's region, slot (k - kb) * NC + c
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      red[wave * kRegion + ((k - kb) * NC + (uint32_t)c) * 64u + lane] = acc[c];
      acc[c] = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};
    }
    if (k + 1u - kb == kGroup && (k + 1u < n_myb || half)) { // the regions are full
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      flush(kb, kGroup, false);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); // slots read before reuse
      kb = k + 1u;
    }
  }
  if (x1_pending) { // no full block: superblock 1's X for the half block (or nothing)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    read_frags(1);
  }
  if (half) { // its loads were issued into slot 0 with the last full block's
    const uint32_t k = n_myb;
    f32x4_t acc1[NC]; // tiles against the second superblock's X (rows 8..15 valid)
#pragma unroll
    for (int c = 0; c < NC; ++c) acc1[c] = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};
    const uint4 hd = H[0];
    const float d = f16_to_f32(hd.x & 0xFFFFu), dmin = f16_to_f32(hd.x >> 16);
    uint32_t scp, mp;
    q4k_scale_min_pair(hd.y, hd.z, hd.w, g, &scp, &mp);
    const float d1s = d * (float)(scp & 0xFFu) * 16777216.0f;
    const float d2s = d * (float)(scp >> 8) * 1048576.0f;
    const float m1 = dmin * (float)(mp & 0xFFu), m2 = dmin * (float)(mp >> 8);
    const uint32_t w[8] = {QA[0].x, QA[0].y, QA[0].z, QA[0].w, QB[0].x, QB[0].y, QB[0].z, QB[0].w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      uint32_t l0, l1, h0, h1, l2, l3, h2, h3;
      dequant_dword(w[2 * t], d1s, m1, d2s, m2, l0, l1, h0, h1);
      dequant_dword(w[2 * t + 1], d1s, m1, d2s, m2, l2, l3, h2, h3);
      const half8_t alo = __builtin_bit_cast(half8_t, make_uint4(l0, l1, l2, l3));
      const half8_t ahi = __builtin_bit_cast(half8_t, make_uint4(h0, h1, h2, h3));
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, xf[c][0][t], acc[c], 0, 0, 0);
        acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, xf[c][0][t + 4], acc[c], 0, 0, 0);
        acc1[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, xf[c][1][t], acc1[c], 0, 0, 0);
        acc1[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, xf[c][1][t + 4], acc1[c], 0, 0, 0);
      }
    }
    // lanes 0..31 hold rows 0..7 of the first tile, lanes 32..63 rows 8..15
    // of the second: the same output rows, the row's two superblock parts
#pragma unroll
    for (int c = 0; c < NC; ++c)
      red[wave * kRegion + ((k - kb) * NC + (uint32_t)c) * 64u + lane] = lane < 32u ? acc[c] : acc1[c];
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  flush(kb, n_myb - kb, half);
}

} // namespace

#define AXH_Q4K_MATMUL_KS(KS, NT, PF, RT, SUFFIX)                                                \
  extern "C" __global__ void __launch_bounds__(KS * 64)                                          \
      axh_q4k_matmul_ks_k##KS##_n##NT##_p##PF##SUFFIX(const uint8_t *__restrict__ q,             \
                                                      const uint16_t *__restrict__ x,            \
                                                      float *__restrict__ y, AXH_MATMUL_ARGS) { AXH_MATMUL_UNPACK; \
    q4k_matmul_ks<KS, NT, PF, RT>(q, x, y, a);                                                   \
  }

AXH_Q4K_MATMUL_KS(4, 1, 2, 2, )
AXH_Q4K_MATMUL_KS(8, 1, 1, 2, )
AXH_Q4K_MATMUL_KS(4, 2, 2, 2, )
AXH_Q4K_MATMUL_KS(8, 2, 1, 2, )
AXH_Q4K_MATMUL_KS(8, 1, 1, 1, _r1)
AXH_Q4K_MATMUL_KS(8, 1, 2, 1, _r1)

#define AXH_Q4K_MATMUL_KX(RT, NT, KS, PF)                                                        \
  extern "C" __global__ void __launch_bounds__(KS * 64)                                          \
      axh_q4k_matmul_kx_r##RT##_n##NT##_k##KS##_p##PF(const uint8_t *__restrict__ q,             \
                                                      const uint16_t *__restrict__ x,            \
                                                      float *__restrict__ y, AXH_MATMUL_ARGS) { AXH_MATMUL_UNPACK; \
    extern __shared__ f32x4_t axh_red_dyn[];                                                     \
    q4k_matmul_kx<RT, NT, KS, PF>(q, x, y, a, axh_red_dyn);                                      \
  }

AXH_Q4K_MATMUL_KX(4, 8, 4, 2)
AXH_Q4K_MATMUL_KX(2, 8, 4, 2)
AXH_Q4K_MATMUL_KX(4, 4, 4, 2)
AXH_Q4K_MATMUL_KX(4, 4, 4, 3)
AXH_Q4K_MATMUL_KX(8, 4, 4, 2)
AXH_Q4K_MATMUL_KX(4, 2, 4, 2)
AXH_Q4K_MATMUL_KX(4, 2, 4, 3)
AXH_Q4K_MATMUL_KX(4, 1, 4, 3)

#define AXH_Q4K_MATMUL_RM(W, RT)                                                                 \
  extern "C" __global__ void __launch_bounds__(W * 64)                                           \
      axh_q4k_matmul_rm_w##W##_r##RT##_p4(const uint8_t *__restrict__ q,                         \
                                          const uint16_t *__restrict__ x, float *__restrict__ y,  \
                                          AXH_MATMUL_ARGS) { AXH_MATMUL_UNPACK;                   \
    extern __shared__ f32x4_t axh_rm_dyn[];                                                      \
    q4k_matmul_rm<W, RT>(q, x, y, a, axh_rm_dyn);                                                \
  }

AXH_Q4K_MATMUL_RM(4, 2)
AXH_Q4K_MATMUL_RM(8, 1)
AXH_Q4K_MATMUL_RM(4, 1)
AXH_Q4K_MATMUL_RM(2, 2)

#define AXH_Q4K_MATMUL_SR(NW, SPW, NC, XH, SUFFIX)                                               \
  extern "C" __global__ void __launch_bounds__(NW * 64)                                          \
      axh_q4k_matmul_sr_w##NW##_s##SPW##SUFFIX(const uint8_t *__restrict__ q,                    \
                                               const uint16_t *__restrict__ x,                   \
                                               float *__restrict__ y, AXH_MATMUL_ARGS) { AXH_MATMUL_UNPACK; \
    extern __shared__ f32x4_t axh_sr_dyn[];                                                      \
    q4k_matmul_sr<NW, SPW, NC, XH>(q, x, y, a, axh_sr_dyn);                                      \
  }

AXH_Q4K_MATMUL_SR(8, 2, 1, false, )
AXH_Q4K_MATMUL_SR(8, 2, 2, false, _n2)
AXH_Q4K_MATMUL_SR(8, 2, 1, true, _h)

#define AXH_Q4K_MATMUL_LK(XC, XD, WD, RT, SUFFIX)                                               \
  extern "C" __global__ void __launch_bounds__(512)                                              \
      axh_q4k_matmul_lk_c##XC##_x##XD##_w##WD##SUFFIX(const uint8_t *__restrict__ q,             \
                                                      const uint16_t *__restrict__ x,            \
                                                      float *__restrict__ y, AXH_MATMUL_ARGS) {  \
    AXH_MATMUL_UNPACK;                                                                           \
    extern __shared__ f32x4_t axh_lk_dyn[];                                                      \
    q4k_matmul_lk<XC, XD, WD, RT>(q, x, y, a, axh_lk_dyn);                                       \
  }

AXH_Q4K_MATMUL_LK(8, 2, 2, 1, )
AXH_Q4K_MATMUL_LK(8, 1, 3, 1, )
AXH_Q4K_MATMUL_LK(16, 1, 3, 1, )
AXH_Q4K_MATMUL_LK(8, 2, 2, 2, _r2)
AXH_Q4K_MATMUL_LK(4, 2, 2, 1, )
AXH_Q4K_MATMUL_LK(16, 1, 3, 2, _r2)
