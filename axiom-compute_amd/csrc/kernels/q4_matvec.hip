// gfx950 Q4_K_M and Q4_0 dequant-matvec kernels, plus the decode-only kernels
// used by the bit-exact checks.  Built into one code object (q4_matvec.hsaco)
// that the runtime loads with hipModuleLoadData.
//
// Kernel argument convention (matches the runtime's binding plans): one
// pointer per buffer binding in binding order, then one push-constant struct
// passed by value.
//
// Reference kernels: examples/q4km_dequant_matvec.axc:7-117 and
// examples/q4_0_dequant_matvec.axc:7-51 (one output, one active lane).  The
// multi-row kernels apply that dot product to each row of a row-major matrix
// of contiguous blocks.
#include "q4_common.h"

using namespace axh;

struct RowsArgs {
  uint32_t n_rows;
  uint32_t units_per_row; // superblocks (Q4_K) or blocks (Q4_0) per row
  uint32_t tile_units;    // units staged in LDS per tile (multiple of the wave step)
  uint32_t pad;
};

struct CountArgs {
  uint32_t n_units; // n_superblocks (Q4_K) or n_blocks (Q4_0)
};

// Kernels take the shape as separate 32-bit arguments (the same kernarg
// layout as the structs above) so that every argument is preloaded into
// SGPRs at wave launch (-amdgpu-kernarg-preload-count): no wave waits for a
// kernarg load before its first memory request (north star 8.44 -> 8.07 us
// per call, A/B in one run).
#define AXH_ROWS_ARGS uint32_t a_n_rows, uint32_t a_units_per_row, uint32_t a_tile_units, uint32_t a_pad
#define AXH_ROWS_UNPACK const RowsArgs a{a_n_rows, a_units_per_row, a_tile_units, a_pad}
#define AXH_COUNT_ARGS uint32_t a_n_units
#define AXH_COUNT_UNPACK const CountArgs a{a_n_units}

// ===========================================================================
// Q4_K_M matvec
// ===========================================================================
// Wave mapping: lane = 8*g + k.  Group g (0..7) owns superblock it*8 + g of
// the current iteration; lane k (0..7) owns qs bytes [16k, 16k+16), i.e. chunk
// c = k/2, half h = k%2: its low nibbles are weights 64c + 16h + i of
// sub-block 2c and its high nibbles weights 64c + 32 + 16h + i of sub-block
// 2c+1 (i = 0..15).  Each lane loads the 16-byte header and its 16-byte qs
// slice: two 16-byte loads per lane, 1152 contiguous bytes per wave.
//
// LDS tile of x for `tile` superblocks (slot = superblock within the tile):
//   xs[slot*256 + part*128 + ((t*32) ^ ((slot&1)*32)) + 4k + e]
//       = x[sb*256 + 64c + 32*part + 16h + 4t + e]
//   hs[slot*16 + 2k + part] = sum over (t, e) of the same 16 values
// so that the 8 lanes of a group read 32 consecutive dwords and neighbouring
// groups land on the other half of a 64-bank LDS: ds_read_b128 is conflict-free.
//
// Per row the lane accumulates
//   alo = sum_i lo_i * 2^-24 * x_lo[i],  ahi = sum_i hi_i * 2^-20 * x_hi[i]
// through v_fma_mix_f32 (nibbles as f16 subnormals), and adds
//   d * (sc0 * 2^24 * alo + sc1 * 2^20 * ahi) - dmin * (m0 * hs_lo + m1 * hs_hi)
// which is sum_i (d*sc*q_i - dmin*m) * x_i regrouped per sub-block.

// One 16-element group of x (group gi of a tile: superblock slot gi/16,
// r = gi%16 -> x[slot*256 + 16r .. +16], i.e. c = r/4, part = (r/2)%2, h = r%2).
struct XGroup {
  float4 v[4];
};

__device__ __forceinline__ void q4k_load_group(const float *__restrict__ x, uint32_t sb0,
                                               uint32_t gi, XGroup &g) {
  const float4 *src =
      reinterpret_cast<const float4 *>(x + (size_t)(sb0 + (gi >> 4)) * 256u + 16u * (gi & 15u));
  g.v[0] = src[0];
  g.v[1] = src[1];
  g.v[2] = src[2];
  g.v[3] = src[3];
}

__device__ __forceinline__ void q4k_store_group(float *xs, float *hs, uint32_t gi,
                                                const XGroup &g) {
  const uint32_t slot = gi >> 4, r = gi & 15u;
  const uint32_t c = r >> 2, part = (r >> 1) & 1u, h = r & 1u, k = 2u * c + h;
  float *dst = xs + slot * 256u + part * 128u + 4u * k;
  const uint32_t sw = (slot & 1u) * 32u;
  *reinterpret_cast<float4 *>(dst + (0u ^ sw)) = g.v[0];
  *reinterpret_cast<float4 *>(dst + (32u ^ sw)) = g.v[1];
  *reinterpret_cast<float4 *>(dst + (64u ^ sw)) = g.v[2];
  *reinterpret_cast<float4 *>(dst + (96u ^ sw)) = g.v[3];
  const float4 a = g.v[0], b = g.v[1], cc = g.v[2], d = g.v[3];
  const float s = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w)) +
                  (((cc.x + cc.y) + (cc.z + cc.w)) + ((d.x + d.y) + (d.z + d.w)));
  hs[slot * 16u + 2u * k + part] = s;
}

__device__ __forceinline__ void q4k_stage_tile(const float *__restrict__ x, float *xs, float *hs,
                                               uint32_t sb0, uint32_t n_sb, uint32_t tid,
                                               uint32_t nthreads) {
  const uint32_t ngroups = n_sb * 16u;
  for (uint32_t gi = tid; gi < ngroups; gi += nthreads) {
    XGroup g;
    q4k_load_group(x, sb0, gi, g);
    q4k_store_group(xs, hs, gi, g);
  }
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte weight load; kNT marks it non-temporal (streamed once per call).
template <bool kNT>
__device__ __forceinline__ uint4 load16(const uint8_t *p) {
  if constexpr (kNT) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return *reinterpret_cast<const uint4 *>(p);
  }
}

// Raw buffer access (MUBUF) through a resource descriptor: 32-bit byte
// offsets, and offsets past num_records read as zero in hardware.  The
// compiler keeps these loads in program order relative to barriers.
constexpr int kBufferFlags = 0x00020000; // dword3 of the V# for gfx9 (32-bit data)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                           kBufferFlags);
}

template <bool kNT>
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kNT ? 2 : 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 buf_loadf4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  // Bit-cast the whole vector: a bit-cast of a single vector element drops
  // the other three loaded dwords with this compiler.
  const f32x4_t f =
      __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
  return make_float4(f.x, f.y, f.z, f.w);
}

// Four qs bytes (one dword) of a lane's slice against four x values of each part.
__device__ __forceinline__ void q4k_dword(uint32_t w, float4 xl, float4 xh, float &alo, float &ahi) {
  const uint32_t w8 = w >> 8;
  const uint32_t a = w & 0x000F000Fu;   // bytes 0,2 low nibbles  (x 2^-24)
  const uint32_t b = w8 & 0x000F000Fu;  // bytes 1,3 low nibbles  (x 2^-24)
  const uint32_t ch = w & 0x00F000F0u;  // bytes 0,2 high nibbles (x 2^-20)
  const uint32_t dh = w8 & 0x00F000F0u; // bytes 1,3 high nibbles (x 2^-20)
  alo = __builtin_fmaf(lo_half_f16(a), xl.x, alo);
  alo = __builtin_fmaf(lo_half_f16(b), xl.y, alo);
  alo = __builtin_fmaf(hi_half_f16(a), xl.z, alo);
  alo = __builtin_fmaf(hi_half_f16(b), xl.w, alo);
  ahi = __builtin_fmaf(lo_half_f16(ch), xh.x, ahi);
  ahi = __builtin_fmaf(lo_half_f16(dh), xh.y, ahi);
  ahi = __builtin_fmaf(hi_half_f16(ch), xh.z, ahi);
  ahi = __builtin_fmaf(hi_half_f16(dh), xh.w, ahi);
}

// All global loads of this kernel are unconditional, with addresses clamped
// into the row (the results for out-of-range slots are simply not used), so
// the hardware's in-order load counter lets each iteration wait for exactly
// its own data while later iterations' loads stay in flight.
template <int RPW, int PF, bool kNT>
__device__ __forceinline__ void q4k_load_iter(uint4 (&H)[PF][RPW], uint4 (&Qv)[PF][RPW], int p,
                                              const uint8_t *const (&rowp)[RPW], uint32_t it,
                                              uint32_t g, uint32_t k, uint32_t nsb) {
  const uint32_t sb = min(it * 8u + g, nsb - 1u);
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const uint8_t *b = rowp[r] + (size_t)sb * kQ4kSbBytes;
    H[p][r] = load16<kNT>(b - 16u * k);
    Qv[p][r] = load16<kNT>(b + 16u);
  }
}

template <int RPW, int NW, int PF, bool kNT, bool kMultiTile>
__device__ __forceinline__ void q4k_matvec_body(const uint8_t *__restrict__ q,
                                                const float *__restrict__ x, float *__restrict__ y,
                                                uint32_t n_rows, uint32_t nsb, uint32_t tile_sb,
                                                uint32_t block, float *lds) {
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t g = lane >> 3, k = lane & 7u, c = k >> 1;
  const uint32_t row0 = (block * NW + wave) * RPW;
  if (nsb == 0) { // empty rows: the reference returns +0.0 (AT-1323)
#pragma unroll
    for (int r = 0; r < RPW; ++r)
      if (lane == 0 && row0 + r < n_rows) y[row0 + r] = 0.0f;
    return;
  }
  const size_t row_bytes = (size_t)nsb * kQ4kSbBytes;
  const uint8_t *rowp[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const uint32_t row = min(row0 + r, n_rows - 1u); // clamp: loads stay in bounds
    rowp[r] = q + (size_t)row * row_bytes + 16u * k;
  }
  // iterations padded to a multiple of PF: the extra ones hold no superblock
  const uint32_t n_it = (((nsb + 7u) >> 3) + (PF - 1)) / PF * PF;
  const uint32_t it_per_tile = tile_sb >> 3;
  float *xs = lds;
  float *hs = lds + tile_sb * 256u;

  uint4 H[PF][RPW], Qv[PF][RPW];
  float acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;

  // Prologue: x for the first tile is requested before the weight prefetch so
  // that waiting for x never waits on weights.
  constexpr int kXR = 2; // x groups per thread loaded ahead of the weights
  const uint32_t ngroups0 = min(tile_sb, nsb) * 16u;
  XGroup xg[kXR];
#pragma unroll
  for (int i = 0; i < kXR; ++i)
    q4k_load_group(x, 0u, min(tid + (uint32_t)i * (NW * 64u), ngroups0 - 1u), xg[i]);
  __builtin_amdgcn_sched_barrier(0); // keep the x requests ahead of the weight requests
#pragma unroll
  for (int p = 0; p < PF; ++p) q4k_load_iter<RPW, PF, kNT>(H, Qv, p, rowp, (uint32_t)p, g, k, nsb);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < kXR; ++i) {
    const uint32_t gi = tid + (uint32_t)i * (NW * 64u);
    if (gi < ngroups0) q4k_store_group(xs, hs, gi, xg[i]);
  }
  for (uint32_t gi = tid + kXR * (NW * 64u); gi < ngroups0; gi += NW * 64u) {
    XGroup gx;
    q4k_load_group(x, 0u, gi, gx);
    q4k_store_group(xs, hs, gi, gx);
  }
  __syncthreads();

  uint32_t tile = 0;
  for (uint32_t it0 = 0; it0 < n_it; it0 += PF) {
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      const uint32_t it = it0 + (uint32_t)p;
      if constexpr (kMultiTile) {
        const uint32_t t_it = it / it_per_tile;
        if (t_it != tile && t_it * tile_sb < nsb) { // uniform across the workgroup
          __syncthreads();
          tile = t_it;
          const uint32_t sb0 = t_it * tile_sb;
          q4k_stage_tile(x, xs, hs, sb0, min(tile_sb, nsb - sb0), tid, NW * 64u);
          __syncthreads();
        }
      }
      const uint32_t sb = it * 8u + g;
      if (sb < nsb) {
        const uint32_t slot = sb - tile * tile_sb;
        const float *xb = xs + slot * 256u + 4u * k;
        const uint32_t sw = (slot & 1u) * 32u;
        float4 xl[4], xh[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          xl[t] = *reinterpret_cast<const float4 *>(xb + ((uint32_t)(t * 32) ^ sw));
          xh[t] = *reinterpret_cast<const float4 *>(xb + 128u + ((uint32_t)(t * 32) ^ sw));
        }
        const float2 hsum = *reinterpret_cast<const float2 *>(hs + slot * 16u + 2u * k);
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          const uint4 hd = H[p][r];
          const uint4 qv = Qv[p][r];
          uint32_t scp, mp;
          q4k_scale_min_pair(hd.y, hd.z, hd.w, c, &scp, &mp);
          const float d = f16_to_f32(hd.x & 0xFFFFu);
          const float dmin = f16_to_f32(hd.x >> 16);
          float alo = 0.0f, ahi = 0.0f;
          q4k_dword(qv.x, xl[0], xh[0], alo, ahi);
          q4k_dword(qv.y, xl[1], xh[1], alo, ahi);
          q4k_dword(qv.z, xl[2], xh[2], alo, ahi);
          q4k_dword(qv.w, xl[3], xh[3], alo, ahi);
          const float sc0 = (float)(scp & 0xFFu) * 16777216.0f; // 2^24
          const float sc1 = (float)(scp >> 8) * 1048576.0f;     // 2^20
          const float m0 = (float)(mp & 0xFFu), m1 = (float)(mp >> 8);
          const float dot = __builtin_fmaf(sc0, alo, sc1 * ahi);
          const float mins = __builtin_fmaf(m0, hsum.x, m1 * hsum.y);
          acc[r] = __builtin_fmaf(d, dot, __builtin_fmaf(-dmin, mins, acc[r]));
        }
      }
      // refill this prefetch slot with iteration it + PF (clamped, unconditional)
      q4k_load_iter<RPW, PF, kNT>(H, Qv, p, rowp, it + PF, g, k, nsb);
    }
  }

#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const float s = wave_sum(acc[r]);
    if (lane == 0 && row0 + r < n_rows) y[row0 + r] = s;
  }
}

// Tiled kernel: rows longer than one LDS tile (x is re-staged per tile).
#define AXH_Q4K_MATVEC_TILED(RPW, NW, PF)                                                        \
  extern "C" __global__ void __launch_bounds__(NW * 64)                                          \
      axh_q4k_matvec_tiled_r##RPW##_w##NW##_p##PF(const uint8_t *__restrict__ q,                 \
                                                  const float *__restrict__ x,                   \
                                                  float *__restrict__ y, AXH_ROWS_ARGS) { AXH_ROWS_UNPACK; \
    extern __shared__ float axh_lds_dyn[];                                                       \
    if (a.units_per_row <= a.tile_units)                                                         \
      q4k_matvec_body<RPW, NW, PF, false, false>(q, x, y, a.n_rows, a.units_per_row,             \
                                                 a.tile_units, blockIdx.x, axh_lds_dyn);         \
    else                                                                                         \
      q4k_matvec_body<RPW, NW, PF, false, true>(q, x, y, a.n_rows, a.units_per_row,              \
                                                a.tile_units, blockIdx.x, axh_lds_dyn);          \
  }

AXH_Q4K_MATVEC_TILED(1, 4, 2)
AXH_Q4K_MATVEC_TILED(2, 8, 2)

// ---------------------------------------------------------------------------
// Persistent Q4_K matvec for rows that fit one LDS tile (<= 128 superblocks).
//
// Lane mapping: lane = 4*G + c with G = 8*half + s.  The two half-waves work
// on two different row bundles (RPW consecutive rows each); in one iteration
// half-wave `half` covers superblocks it*8 + s (s = 0..7) of its bundle, and
// lane c (0..3) owns qs bytes [32c, 32c+32) of that superblock: its low
// nibbles are sub-block 2c (weights 64c + i), its high nibbles sub-block 2c+1
// (weights 64c + 32 + i), i = 0..31.  Per superblock a lane loads the 16-byte
// header and two 16-byte qs slices.
//
// Each wave walks a flattened sequence (bundle pair, iteration): loads run PF
// iterations ahead across bundle boundaries, so the load pipeline only
// drains at the end of the wave's work.  x is staged once per workgroup.
//
// LDS: xs[sb*272 + part*128 + 16t + 4c + e]
//        = x[sb*256 + 64c + 32*part + 4t + e] * (part ? 2^20 : 2^24)
//      ss[sb*8 + j] = sum of the 32 (unscaled) x of sub-block j
// The 16-float pad per superblock puts superblocks s = 0..3 of an iteration on
// different bank quarters: for fixed (t, part), 16 consecutive lanes read 64
// distinct banks, and every read is the lane's base address plus an
// immediate offset.  The
// 2^24 / 2^20 factors cancel the f16-subnormal encoding of the nibbles, so
//   sum_i (d*sc*q_i - dmin*m) * x_i = d*sc*sum_i q_i x_i - dmin*m*ss
// needs no further scaling.
// ---------------------------------------------------------------------------
constexpr uint32_t kQ4kFlatSbFloats = 272; // LDS floats per superblock of x (256 + pad)
constexpr uint32_t kWaitXMinSb = 32;       // rows this long wait for x before prefetching

// Coalesced x staging for the persistent kernels: float4 f = tid + i * NT
// (NT threads, i < 8 * XP) of x, so consecutive lanes read consecutive 16
// bytes.  (One 32-float sub-block per thread instead puts every lane of a
// load on its own cache line, 4x the address-unit work of a coalesced load,
// and the 8 loads of a lane revisit each line after the wave's other lanes
// have filled L1.)  Float4 f is element 4w of superblock f / 64, w = f % 64:
// chunk c = w / 16, part (high nibbles) = (w / 8) & 1, group t = w & 7, and
// the 8 lanes 8m..8m+7 of a load hold one whole sub-block (f / 8), whose sum
// they form with DPP inside their half-row.
template <int NT, int XP>
__device__ __forceinline__ void q4k_flat_load_xc(__amdgpu_buffer_rsrc_t xr, uint32_t tid,
                                                 float4 (&v)[8 * XP]) {
#pragma unroll
  for (int i = 0; i < 8 * XP; ++i) v[i] = buf_loadf4(xr, (tid + (uint32_t)i * NT) * 16u);
}

// kQ40: `units` is the row's Q4_0 block count (8 float4 each), else its
// superblock count (64 float4 each).  Q4_0 layout: the 256 elements of a unit
// are an octet of 8 blocks, quarter c = w / 16 holds blocks 2c and 2c + 1, and
// float4 i = w & 15 of the quarter (natural order: block 2c's low-nibble
// elements, its high-nibble elements, then block 2c + 1's) goes to 16i + 4c
// of the octet's slot; it meets high nibbles (scale 2^20) where i & 4.
template <int NT, int XP, bool kQ40 = false>
__device__ __forceinline__ void q4k_flat_stage_xc(float *xs, float *ss, uint32_t tid,
                                                  uint32_t units, const float4 (&v)[8 * XP]) {
#pragma unroll
  for (int i = 0; i < 8 * XP; ++i) {
    const uint32_t f = tid + (uint32_t)i * NT;
    const float4 a = v[i];
    float s = (a.x + a.y) + (a.z + a.w);
    s += dpp_mov<0xB1>(s);  // quad_perm [1,0,3,2]
    s += dpp_mov<0x4E>(s);  // quad_perm [2,3,0,1]
    s += dpp_mov<0x141>(s); // row_half_mirror: the 8-lane sum in every lane
    // whole 8-lane groups: NT and the row's float4 count are multiples of 8
    if (f < (kQ40 ? units * 8u : units * 64u)) {
      if constexpr (kQ40) {
        const uint32_t sb = f >> 6, w = f & 63u, c = w >> 4, i4 = w & 15u;
        const float scale = (i4 & 4u) ? 1048576.0f : 16777216.0f;
        *reinterpret_cast<float4 *>(xs + sb * kQ4kFlatSbFloats + 16u * i4 + 4u * c) =
            make_float4(a.x * scale, a.y * scale, a.z * scale, a.w * scale);
      } else {
        const uint32_t sb = f >> 6, w = f & 63u, c = w >> 4, part = (w >> 3) & 1u, t = w & 7u;
        const float scale = part ? 1048576.0f : 16777216.0f;
        *reinterpret_cast<float4 *>(xs + sb * kQ4kFlatSbFloats + part * 128u + 16u * t + 4u * c) =
            make_float4(a.x * scale, a.y * scale, a.z * scale, a.w * scale);
      }
      if ((f & 7u) == 0u) ss[f >> 3] = s;
    }
  }
}

// kQ5: Q5_K superblocks (the qh runs are loaded too).
template <int RPW, int PF, bool kQ5 = false>
struct Q4kFlatBuf {
  uint4 h[PF][RPW], a[PF][RPW], b[PF][RPW];
  uint4 q0[kQ5 ? PF : 1][kQ5 ? RPW : 1], q1[kQ5 ? PF : 1][kQ5 ? RPW : 1];
};

// Q5_K (ggml k-quant, 176 bytes; no reference counterpart): Q4_K's header
// and scale field, then qh[32] @16 and qs[128] @48.  Weight 64c + l (low
// nibble of qs[32c + l]) gains 16 * bit 2c of qh[l], weight 64c + 32 + l
// (high nibble) gains 16 * bit 2c+1.  Sub-block sums and scales are Q4_K's.
constexpr uint32_t kQ5kSbBytes = 176;

// Q4_K dword step with the fifth bits: the low-nibble value q + 16b keeps
// its f16-subnormal encoding with b in mantissa bit 4 (16 * 2^-24), the
// high-nibble value with b in bit 8 (16 * 2^-20).  qhs = qh dword >> 2c.
__device__ __forceinline__ void q5k_dword(uint32_t w, uint32_t qhs, float4 xl, float4 xh,
                                          float &alo, float &ahi) {
  const uint32_t w8 = w >> 8, q8 = qhs >> 8;
  const uint32_t a = (w & 0x000F000Fu) | ((qhs & 0x00010001u) << 4);
  const uint32_t b = (w8 & 0x000F000Fu) | ((q8 & 0x00010001u) << 4);
  const uint32_t ch = (w & 0x00F000F0u) | ((qhs & 0x00020002u) << 7);
  const uint32_t dh = (w8 & 0x00F000F0u) | ((q8 & 0x00020002u) << 7);
  alo = __builtin_fmaf(lo_half_f16(a), xl.x, alo);
  alo = __builtin_fmaf(lo_half_f16(b), xl.y, alo);
  alo = __builtin_fmaf(hi_half_f16(a), xl.z, alo);
  alo = __builtin_fmaf(hi_half_f16(b), xl.w, alo);
  ahi = __builtin_fmaf(lo_half_f16(ch), xh.x, ahi);
  ahi = __builtin_fmaf(lo_half_f16(dh), xh.y, ahi);
  ahi = __builtin_fmaf(hi_half_f16(ch), xh.z, ahi);
  ahi = __builtin_fmaf(hi_half_f16(dh), xh.w, ahi);
}

// Loads of one iteration for the RPW rows of `bundle`.  Rows past the matrix
// read zeros (buffer range check); superblocks past the row are never used.
// kDual (fused gate/up): a bundle is RPW/2 output rows, slots r < RPW/2 read
// row bundle*RPW/2 + r of the first matrix and slots r >= RPW/2 the same row
// of the second.
template <int RPW, int PF, bool kNT, bool kDual, bool kQ5>
__device__ __forceinline__ void q4k_flat_load(Q4kFlatBuf<RPW, PF, kQ5> &B, int p,
                                              __amdgpu_buffer_rsrc_t qr,
                                              __amdgpu_buffer_rsrc_t qr2, uint32_t row_bytes,
                                              uint32_t bundle, uint32_t it, uint32_t s,
                                              uint32_t c) {
  constexpr int kRb = kDual ? RPW / 2 : RPW;
  constexpr uint32_t kQs = kQ5 ? 48u : 16u; // offset of qs in the superblock
  const uint32_t sb_off = (it * 8u + s) * (kQ5 ? kQ5kSbBytes : (uint32_t)kQ4kSbBytes);
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const __amdgpu_buffer_rsrc_t src = (kDual && r >= kRb) ? qr2 : qr;
    const uint32_t off = (bundle * kRb + (uint32_t)(r % kRb)) * row_bytes + sb_off;
    B.h[p][r] = buf_load16<kNT>(src, off);
    if constexpr (kQ5) {
      B.q0[p][r] = buf_load16<kNT>(src, off + 16u);
      B.q1[p][r] = buf_load16<kNT>(src, off + 32u);
    }
    B.a[p][r] = buf_load16<kNT>(src, off + kQs + 32u * c);
    B.b[p][r] = buf_load16<kNT>(src, off + kQs + 16u + 32u * c);
  }
}

// SiLU(g) * u, the SwiGLU combination of a gate and an up projection.
__device__ __forceinline__ float silu_mul(float g, float u) {
  return g / (1.0f + expf(-g)) * u;
}

// One iteration of the flat kernels for the RPW rows of slot p: lane group s
// holds superblock sb, quarter c.  acc[r] += this quarter's share of row r.
template <int RPW, int NS, bool kQ5>
__device__ __forceinline__ void q4k_flat_compute(const Q4kFlatBuf<RPW, NS, kQ5> &B, int p,
                                                 const float *xs, const float *ss, uint32_t sb,
                                                 uint32_t c, float (&acc)[RPW]) {
  const float *xb = xs + sb * kQ4kFlatSbFloats + 4u * c;
  float4 xl[8], xh[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    xl[t] = *reinterpret_cast<const float4 *>(xb + (uint32_t)t * 16u);
    xh[t] = *reinterpret_cast<const float4 *>(xb + 128u + (uint32_t)t * 16u);
  }
  const float2 sub = *reinterpret_cast<const float2 *>(ss + sb * 8u + 2u * c);
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const uint4 hd = B.h[p][r];
    uint32_t scp, mp;
    q4k_scale_min_pair(hd.y, hd.z, hd.w, c, &scp, &mp);
    float alo = 0.0f, ahi = 0.0f;
    if constexpr (kQ5) {
      const uint4 h0 = B.q0[p][r], h1 = B.q1[p][r];
      const uint32_t sh = 2u * c;
      q5k_dword(B.a[p][r].x, h0.x >> sh, xl[0], xh[0], alo, ahi);
      q5k_dword(B.a[p][r].y, h0.y >> sh, xl[1], xh[1], alo, ahi);
      q5k_dword(B.a[p][r].z, h0.z >> sh, xl[2], xh[2], alo, ahi);
      q5k_dword(B.a[p][r].w, h0.w >> sh, xl[3], xh[3], alo, ahi);
      q5k_dword(B.b[p][r].x, h1.x >> sh, xl[4], xh[4], alo, ahi);
      q5k_dword(B.b[p][r].y, h1.y >> sh, xl[5], xh[5], alo, ahi);
      q5k_dword(B.b[p][r].z, h1.z >> sh, xl[6], xh[6], alo, ahi);
      q5k_dword(B.b[p][r].w, h1.w >> sh, xl[7], xh[7], alo, ahi);
    } else {
      q4k_dword(B.a[p][r].x, xl[0], xh[0], alo, ahi);
      q4k_dword(B.a[p][r].y, xl[1], xh[1], alo, ahi);
      q4k_dword(B.a[p][r].z, xl[2], xh[2], alo, ahi);
      q4k_dword(B.a[p][r].w, xl[3], xh[3], alo, ahi);
      q4k_dword(B.b[p][r].x, xl[4], xh[4], alo, ahi);
      q4k_dword(B.b[p][r].y, xl[5], xh[5], alo, ahi);
      q4k_dword(B.b[p][r].z, xl[6], xh[6], alo, ahi);
      q4k_dword(B.b[p][r].w, xl[7], xh[7], alo, ahi);
    }
    const float dot = __builtin_fmaf((float)(scp & 0xFFu), alo, (float)(scp >> 8) * ahi);
    const float mins = __builtin_fmaf((float)(mp & 0xFFu), sub.x, (float)(mp >> 8) * sub.y);
    acc[r] = __builtin_fmaf(f16_to_f32(hd.x & 0xFFFFu), dot,
                            __builtin_fmaf(-f16_to_f32(hd.x >> 16), mins, acc[r]));
  }
}

// Q4_0 rows in the persistent and one-pass kernels: a row is read as octets
// of 8 blocks (144 bytes and 256 weights, a Q4_K superblock's footprint), one
// octet per lane group s, and quarter c of the group owns blocks 2c and
// 2c + 1 (36 bytes at 36c: two 16-byte loads and a dword).  Rows of an even
// block count keep every quarter 4-byte aligned; a quarter past the row's
// last block computes nothing.
template <int RPW, int PF>
struct Q40FlatBuf {
  uint4 a[PF][RPW], b[PF][RPW];
  uint32_t c[PF][RPW];
};

// kDual (fused gate/up): slots r < RPW/2 read row bundle*RPW/2 + r of the
// first matrix, slots r >= RPW/2 the same row of the second.
template <int RPW, int PF, bool kNT, bool kDual>
__device__ __forceinline__ void q4_0_flat_load(Q40FlatBuf<RPW, PF> &B, int p,
                                               __amdgpu_buffer_rsrc_t qr,
                                               __amdgpu_buffer_rsrc_t qr2, uint32_t row_bytes,
                                               uint32_t bundle, uint32_t it, uint32_t s,
                                               uint32_t c) {
  constexpr int kRb = kDual ? RPW / 2 : RPW;
  const uint32_t q_off = (it * 8u + s) * (uint32_t)kQ4kSbBytes + 36u * c;
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const __amdgpu_buffer_rsrc_t src = (kDual && r >= kRb) ? qr2 : qr;
    const uint32_t off = (bundle * kRb + (uint32_t)(r % kRb)) * row_bytes + q_off;
    B.a[p][r] = buf_load16<kNT>(src, off);
    B.b[p][r] = buf_load16<kNT>(src, off + 16u);
    B.c[p][r] = __builtin_amdgcn_raw_buffer_load_b32(src, (int)(off + 32u), 0, kNT ? 2 : 0);
  }
}

// Blocks 2c and 2c + 1 of octet sb for the RPW rows of slot p (live: the
// quarter lies inside the row).  Block A is d = bytes 0-1 and qs = bytes
// 2-17, block B d = bytes 18-19 and qs = bytes 20-35; each block adds
// d * (sum q * x - 8 * sum x), its x staged pre-scaled for the
// f16-subnormal nibbles and its plain sum in ss.
template <int RPW, int NS>
__device__ __forceinline__ void q4_0_flat_compute(const Q40FlatBuf<RPW, NS> &B, int p,
                                                  const float *xs, const float *ss, uint32_t sb,
                                                  uint32_t c, bool live, float (&acc)[RPW]) {
  const float *xb = xs + sb * kQ4kFlatSbFloats + 4u * c;
  float4 xv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) xv[i] = *reinterpret_cast<const float4 *>(xb + 16u * (uint32_t)i);
  const float2 bsum = *reinterpret_cast<const float2 *>(ss + sb * 8u + 2u * c);
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const uint4 a = B.a[p][r], b = B.b[p][r];
    const uint32_t qa[4] = {__builtin_amdgcn_alignbit(a.y, a.x, 16),
                            __builtin_amdgcn_alignbit(a.z, a.y, 16),
                            __builtin_amdgcn_alignbit(a.w, a.z, 16),
                            __builtin_amdgcn_alignbit(b.x, a.w, 16)};
    const uint32_t qb[4] = {b.y, b.z, b.w, B.c[p][r]};
    float alo = 0.0f, ahi = 0.0f, blo = 0.0f, bhi = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      q4k_dword(qa[t], xv[t], xv[4 + t], alo, ahi);
      q4k_dword(qb[t], xv[8 + t], xv[12 + t], blo, bhi);
    }
    const float v = __builtin_fmaf(f16_to_f32(a.x & 0xFFFFu), __builtin_fmaf(-8.0f, bsum.x, alo + ahi),
                                   f16_to_f32(b.x >> 16) * __builtin_fmaf(-8.0f, bsum.y, blo + bhi));
    acc[r] = live ? acc[r] + v : acc[r];
  }
}

// The register slots, loads and compute of the flat layouts: Q4_K / Q5_K
// superblocks, or Q4_0 octets (kQ40; `units` is then the row's block count).
template <int RPW, int PF, bool kQ5, bool kQ40>
struct FlatBufSel {
  using type = Q4kFlatBuf<RPW, PF, kQ5>;
};
template <int RPW, int PF, bool kQ5>
struct FlatBufSel<RPW, PF, kQ5, true> {
  using type = Q40FlatBuf<RPW, PF>;
};

template <int RPW, int PF, bool kNT, bool kDual, bool kQ5, bool kQ40>
__device__ __forceinline__ void flat_load(typename FlatBufSel<RPW, PF, kQ5, kQ40>::type &B, int p,
                                          __amdgpu_buffer_rsrc_t qr, __amdgpu_buffer_rsrc_t qr2,
                                          uint32_t row_bytes, uint32_t bundle, uint32_t it,
                                          uint32_t s, uint32_t c) {
  if constexpr (kQ40)
    q4_0_flat_load<RPW, PF, kNT, kDual>(B, p, qr, qr2, row_bytes, bundle, it, s, c);
  else
    q4k_flat_load<RPW, PF, kNT, kDual, kQ5>(B, p, qr, qr2, row_bytes, bundle, it, s, c);
}

template <int RPW, int PF, bool kQ5, bool kQ40>
__device__ __forceinline__ void flat_compute(const typename FlatBufSel<RPW, PF, kQ5, kQ40>::type &B,
                                             int p, const float *xs, const float *ss, uint32_t sb,
                                             uint32_t c, uint32_t units, float (&acc)[RPW]) {
  if constexpr (kQ40)
    q4_0_flat_compute<RPW, PF>(B, p, xs, ss, sb, c, sb * 8u + 2u * c < units, acc);
  else
    q4k_flat_compute<RPW, PF, kQ5>(B, p, xs, ss, sb, c, acc);
}

// Reduce the pair of bundles (bundle0, bundle0 + 1) that a wave finished and
// store it: each half-wave's lanes hold one bundle's partial sums.
template <int RPW, bool kDual>
__device__ __forceinline__ void q4k_flat_store(float (&acc)[RPW], uint32_t bundle0, uint32_t lane,
                                               uint32_t n_rows, float *__restrict__ y) {
  constexpr int kRb = kDual ? RPW / 2 : RPW;
  float h0[RPW], h1[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    float v = acc[r];
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    v += dpp_mov<0x141>(v);
    v += dpp_mov<0x140>(v);
    const int vi = __builtin_bit_cast(int, v);
    h0[r] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 0)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 16));
    h1[r] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 32)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 48));
    acc[r] = 0.0f;
  }
#pragma unroll
  for (int r = 0; r < kRb; ++r) {
    const uint32_t r0 = bundle0 * kRb + (uint32_t)r;
    const uint32_t r1 = (bundle0 + 1u) * kRb + (uint32_t)r;
    const float o0 = kDual ? silu_mul(h0[r], h0[(r + kRb) % RPW]) : h0[r];
    const float o1 = kDual ? silu_mul(h1[r], h1[(r + kRb) % RPW]) : h1[r];
    if (lane == 0 && r0 < n_rows) y[r0] = o0;
    if (lane == 0 && r1 < n_rows) y[r1] = o1;
  }
}

// x chunk j of the early-refill kernels: superblocks [8j, 8j + 8), 512
// float4 staged by NT threads with the coalesced mapping and layout of
// q4k_flat_stage_xc (float4 f = 512j + tid + i*NT).  Chunks past the row read
// zeros and stage nothing.
template <int NT>
__device__ __forceinline__ void q4k_flat_load_chunk(__amdgpu_buffer_rsrc_t xr, uint32_t tid,
                                                    uint32_t j, float4 (&v)[512 / NT]) {
#pragma unroll
  for (int i = 0; i < 512 / NT; ++i)
    v[i] = buf_loadf4(xr, (j * 512u + tid + (uint32_t)i * NT) * 16u);
}

template <int NT, bool kQ40 = false>
__device__ __forceinline__ void q4k_flat_stage_chunk(float *xs, float *ss, uint32_t tid, uint32_t j,
                                                     uint32_t units, const float4 (&v)[512 / NT]) {
#pragma unroll
  for (int i = 0; i < 512 / NT; ++i) {
    const uint32_t f = j * 512u + tid + (uint32_t)i * NT;
    const float4 a = v[i];
    float sm = (a.x + a.y) + (a.z + a.w);
    sm += dpp_mov<0xB1>(sm);
    sm += dpp_mov<0x4E>(sm);
    sm += dpp_mov<0x141>(sm);
    if (f < (kQ40 ? units * 8u : units * 64u)) {
      if constexpr (kQ40) {
        const uint32_t sb = f >> 6, w = f & 63u, c = w >> 4, i4 = w & 15u;
        const float scale = (i4 & 4u) ? 1048576.0f : 16777216.0f;
        *reinterpret_cast<float4 *>(xs + sb * kQ4kFlatSbFloats + 16u * i4 + 4u * c) =
            make_float4(a.x * scale, a.y * scale, a.z * scale, a.w * scale);
      } else {
        const uint32_t sb = f >> 6, w = f & 63u, c = w >> 4, part = (w >> 3) & 1u, t = w & 7u;
        const float scale = part ? 1048576.0f : 16777216.0f;
        *reinterpret_cast<float4 *>(xs + sb * kQ4kFlatSbFloats + part * 128u + 16u * t + 4u * c) =
            make_float4(a.x * scale, a.y * scale, a.z * scale, a.w * scale);
      }
      if ((f & 7u) == 0u) ss[f >> 3] = sm;
    }
  }
}

// kDual: y[r] = silu(W1[r].x) * (W2[r].x) for q = W1, q2 = W2 (same shape);
// otherwise y = W1 x and q2 is unused.  kQ5: Q5_K superblocks instead of Q4_K.
//
// PF >= 2: x is staged whole first; PF register slots, slot p refilled PF
// iterations ahead right after it is computed.
// PF == 1 (early refill): two slots, and the next iteration's loads are
// issued before the current one is computed, so one iteration is in flight
// at every point of the loop.  x is staged chunk by chunk during the first
// pass over a row (chunk j right before iteration j, requested with the
// weights of iteration j), so the weight stream starts with the first 8 KiB
// of x instead of after all of it.  Every variant with more loads in flight
// was slower on this machine, while a refill that waits for the compute
// leaves the memory pipe idle during it (A/B in one run, 14336 x 4096: 9.9
// vs 10.5 us; Q6_K 4096 x 14336: 12.5 vs 13.4-13.9 us).  The one-pass kernel
// below is this order unrolled over a compile-time trip count.
template <int RPW, int NW, int PF, bool kNT, int XP, bool kDual = false, bool kQ5 = false,
          bool kQ40 = false>
__device__ __forceinline__ void q4k_matvec_flat(const uint8_t *__restrict__ q,
                                                const uint8_t *__restrict__ q2,
                                                const float *__restrict__ x,
                                                float *__restrict__ y, uint32_t n_rows,
                                                uint32_t nsb, float *lds) {
  constexpr int kRb = kDual ? RPW / 2 : RPW; // output rows per bundle
  static_assert(!kDual || RPW % 2 == 0, "the fused kernel pairs gate and up rows");
  static_assert(!(kQ40 && kQ5), "Q4_0 rows are a layout of their own");
  constexpr bool kEarly = PF == 1;        // refill before the compute, chunked x
  constexpr int kSlots = kEarly ? 2 : PF; // register slots
  constexpr int NT = NW * 64;
  static_assert(!kEarly || NT <= 512, "an x chunk is 512 float4");
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  // wave index as a scalar: every loop bound below is then wave-uniform
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t G = lane >> 2, half = G >> 3, s = G & 7u, c = lane & 3u;
  const uint32_t total_waves = gridDim.x * NW;
  const uint32_t W = blockIdx.x * NW + wave;
  const uint32_t n_bundles = (n_rows + kRb - 1) / kRb;
  const uint32_t n_pairs = (n_bundles + 1u) >> 1;
  if (nsb == 0) { // empty rows: the reference returns +0.0 (AT-1323)
    for (uint32_t r = W * 64u + lane; r < n_rows; r += total_waves * 64u) y[r] = 0.0f;
    return;
  }
  const uint32_t n_my = W < n_pairs ? (n_pairs - 1u - W) / total_waves + 1u : 0u;
  // kQ40: nsb is the row's Q4_0 block count and the 256-weight units are
  // its octets of 8 blocks.
  const uint32_t n_units = kQ40 ? (nsb + 7u) >> 3 : nsb;
  const uint32_t n_it = (n_units + 7u) >> 3;
  const uint32_t total = (n_my * n_it + (kSlots - 1)) / kSlots * kSlots;
  // The host guarantees n_rows * row_bytes < 2^32 for this kernel.
  const uint32_t row_bytes =
      nsb * (kQ40 ? (uint32_t)kQ4_0BlockBytes : kQ5 ? kQ5kSbBytes : (uint32_t)kQ4kSbBytes);
  const __amdgpu_buffer_rsrc_t qr = make_rsrc(q, n_rows * row_bytes);
  const __amdgpu_buffer_rsrc_t qr2 = kDual ? make_rsrc(q2, n_rows * row_bytes) : qr;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, nsb * (kQ40 ? 128u : 1024u));
  float *xs = lds;
  float *ss = lds + n_units * kQ4kFlatSbFloats;

  typename FlatBufSel<RPW, kSlots, kQ5, kQ40>::type B;
  uint32_t l_pi = 0, l_it = 0; // load cursor: pair index (of this wave) and iteration
  uint32_t c_pi = 0, c_it = 0; // compute cursor
  float acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
  // Loads of the next iteration into slot p (unconditional: past the last
  // pair they read zeros or bytes whose results are never used).
  auto load_next = [&](int p) {
    const uint32_t bundle = 2u * (W + l_pi * total_waves) + half;
    flat_load<RPW, kSlots, kNT, kDual, kQ5, kQ40>(B, p, qr, qr2, row_bytes, bundle, l_it, s, c);
    if (++l_it == n_it) { l_it = 0; ++l_pi; }
  };
  // Compute the current iteration from slot p and advance the compute cursor.
  auto compute = [&](int p) {
    const uint32_t sb = c_it * 8u + s;
    if (c_pi < n_my && sb < n_units)
      flat_compute<RPW, kSlots, kQ5, kQ40>(B, p, xs, ss, sb, c, nsb, acc);
    if (++c_it == n_it) { // a bundle pair is complete: reduce and store
      if (c_pi < n_my)
        q4k_flat_store<RPW, kDual>(acc, 2u * (W + c_pi * total_waves), lane, n_rows, y);
      c_it = 0;
      ++c_pi;
    }
  };

  if constexpr (kEarly) {
    // First pass: the wave's first bundle pair, iteration j with x chunk j
    // staged right before it (every wave, uniform trip count padded to even).
    // Loads past the row go through an empty resource (zero records): they
    // return zeros without a memory request.
    const uint32_t bundle0 = 2u * W + half;
    const __amdgpu_buffer_rsrc_t none = make_rsrc(q, 0u);
    auto load_first = [&](int p, uint32_t it) {
      const bool in = it < n_it;
      flat_load<RPW, kSlots, kNT, kDual, kQ5, kQ40>(B, p, in ? qr : none, in ? qr2 : none,
                                                    row_bytes, bundle0, it, s, c);
    };
    float4 xv[2][512 / NT];
    q4k_flat_load_chunk<NT>(xr, tid, 0u, xv[0]);
    load_first(0, 0u);
    const uint32_t n1 = (n_it + 1u) & ~1u;
    uint32_t j = 0;
    do {
      q4k_flat_stage_chunk<NT, kQ40>(xs, ss, tid, j, nsb, xv[0]);
      q4k_flat_load_chunk<NT>(xr, tid, j + 1u, xv[1]);
      load_first(1, j + 1u);
      __syncthreads();
      if (n_my > 0 && j * 8u + s < n_units)
        flat_compute<RPW, kSlots, kQ5, kQ40>(B, 0, xs, ss, j * 8u + s, c, nsb, acc);
      q4k_flat_stage_chunk<NT, kQ40>(xs, ss, tid, j + 1u, nsb, xv[1]);
      q4k_flat_load_chunk<NT>(xr, tid, j + 2u, xv[0]);
      load_first(0, j + 2u);
      __syncthreads();
      if (n_my > 0 && (j + 1u) * 8u + s < n_units)
        flat_compute<RPW, kSlots, kQ5, kQ40>(B, 1, xs, ss, (j + 1u) * 8u + s, c, nsb, acc);
      j += 2u;
    } while (j < n1);
    if (n_my > 0) q4k_flat_store<RPW, kDual>(acc, 2u * W, lane, n_rows, y);
    // The wave's other pairs: x is resident, no barriers.
    if (n_my > 1) {
      l_pi = 1;
      c_pi = 1;
      const uint32_t total2 = ((n_my - 1u) * n_it + 1u) & ~1u;
      load_next(0);
      for (uint32_t k = 0; k < total2; k += 2u) {
        load_next(1);
        compute(0);
        load_next(0);
        compute(1);
      }
    }
  } else {
    // Prologue: x requests first, then (for long rows once x has arrived) the
    // weight prefetch, then the LDS writes.  8 * XP float4 of x per thread (a
    // sub-block's worth per XP): the host launches this kernel only when
    // nsb * 8 <= XP * NW * 64 (Q4_0: nsb <= XP * NW * 64 blocks).
    float4 xv[8 * XP];
    q4k_flat_load_xc<NT, XP>(xr, tid, xv);
    // For long rows, let x arrive before the weight prefetch goes out: every
    // wave of the grid issues its prefetch at once, and x requests queued
    // behind that traffic arrive later than the first weights would (measured:
    // 0.3 us less per launch on 4096 x 14336, 0.2 us more on 4096 x 4096,
    // where x is 16 KiB).
    __builtin_amdgcn_sched_barrier(0);
    if (n_units >= kWaitXMinSb) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < PF; ++p) load_next(p);
    __builtin_amdgcn_sched_barrier(0);
    q4k_flat_stage_xc<NT, XP, kQ40>(xs, ss, tid, nsb, xv);
    __syncthreads();
    for (uint32_t j0 = 0; j0 < total; j0 += PF) {
#pragma unroll
      for (int p = 0; p < PF; ++p) {
        compute(p);
        load_next(p); // refill this slot PF iterations ahead
      }
    }
  }
}

// One pass, one bundle pair per wave (axh_q4k_matvec_one_i{NIT}): rows of
// 8 * (NIT - 1) < nsb <= 8 * NIT superblocks, 8 waves per workgroup, wave W
// takes rows 2W and 2W + 1 and the grid covers all of them, one workgroup per
// 16 rows.  The persistent kernel's early-refill order (one iteration in
// flight, x staged chunk by chunk with the weights), fully unrolled over the
// NIT iterations, so no load, barrier or bookkeeping is spent past the row.
// Every row group stages x itself (nsb KiB per 16 rows), which costs more
// than it saves only for very tall matrices.  Measured against the persistent
// kernels (A/B in one run): 4096 x 14336 8.13-8.36 vs 8.62-8.76 us, 4096 x
// 4096 4.06 vs 4.62-4.92, 14336 x 4096 8.9-9.1 vs 9.9-10.5, 32768 x 4096 17.0
// vs 18.6; the 128256-row head 56.8 vs 53.5 (persistent prefetch 2) stays
// persistent.  The template also covers the fused gate/up (kDual) and Q5_K
// (kQ5) layouts.  The fused gate/up measured slower than its persistent
// kernel (2 x 14336 x 4096, A/B in one run, alternating order: x chunk by
// chunk 15.12 us, x whole 14.97, persistent 14.53; identical output) and is
// not built; the Q5_K
// instances for rows of up to 16 superblocks are (axh_q5k_matvec_one_i{NIT},
// see the runtime's Q5_K kernel choice).
//
// kWhole (axh_q4k_matvec_onex_i{NIT}): x is staged whole first, behind one
// barrier, with the first iteration's weights already requested, and the
// early-refill loop then runs without barriers, so the waves of a workgroup
// drift apart and one wave's dot overlaps another's loads.  It pays where
// several workgroups share a CU and the staging of one overlaps the weight
// stream of another (A/B in one run, 14336 x 4096: 8.27-8.40 vs 8.78-9.00
// us), and costs where one workgroup per CU waits for all of x (4096 x 14336:
// 8.64-8.70 vs 8.12-8.22 us).
// The store of the wave-paired gate/up kernels: each wave reduces its two
// rows (lanes 0-31 and 32-63); the odd wave of a pair (the second matrix)
// leaves its sums in LDS, and after a barrier of the whole workgroup the even
// wave stores silu(g) * u for both rows.  xch holds 2 floats per wave pair.
__device__ __forceinline__ void gate_up_pair_store(float v, uint32_t pair, uint32_t wave,
                                                   uint32_t lane, bool mine, uint32_t n_rows,
                                                   float *__restrict__ y, float *xch) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x141>(v);
  v += dpp_mov<0x140>(v);
  const int vi = __builtin_bit_cast(int, v);
  const float h0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 0)) +
                   __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 16));
  const float h1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 32)) +
                   __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 48));
  float *slot = xch + 2u * (wave >> 1);
  if ((wave & 1u) && lane == 0) {
    slot[0] = h0;
    slot[1] = h1;
  }
  __syncthreads();
  if (!(wave & 1u) && mine && lane == 0) {
    const uint32_t r0 = 2u * pair, r1 = r0 + 1u;
    if (r0 < n_rows) y[r0] = silu_mul(h0, slot[0]);
    if (r1 < n_rows) y[r1] = silu_mul(h1, slot[1]);
  }
}

template <int NIT, bool kDual = false, bool kQ5 = false, bool kWhole = false, int XD = 1,
          bool kQ40 = false, bool kPair = false>
__device__ __forceinline__ void q4k_matvec_one(const uint8_t *__restrict__ q,
                                               const uint8_t *__restrict__ q2,
                                               const float *__restrict__ x, float *__restrict__ y,
                                               uint32_t n_rows, uint32_t nsb, float *lds) {
  constexpr int NW = 8, NT = NW * 64;
  constexpr int RPW = kDual ? 2 : 1; // row slots per lane: (gate, up) or one row
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t G = lane >> 2, half = G >> 3, s = G & 7u, c = lane & 3u;
  // kPair (fused gate/up): waves 2P and 2P + 1 take rows 2P and 2P + 1 of
  // the first and of the second matrix, one row per lane slot, so the pair's
  // loads go through one wave-uniform resource each; W is the pair index.
  static_assert(!(kPair && kDual), "one pairing of gate and up rows");
  const uint32_t W = kPair ? (blockIdx.x * NW + wave) >> 1 : blockIdx.x * NW + wave;
  const bool mine = W < (n_rows + 1u) >> 1; // this wave has a pair of rows
  static_assert(!(kQ40 && (kDual || kQ5)), "Q4_0 rows are a layout of their own");
  // kQ40: nsb is the row's Q4_0 block count, read as octets of 8 blocks.
  const uint32_t n_units = kQ40 ? (nsb + 7u) >> 3 : nsb;
  const uint32_t row_bytes =
      nsb * (kQ40 ? (uint32_t)kQ4_0BlockBytes : kQ5 ? kQ5kSbBytes : (uint32_t)kQ4kSbBytes);
  const __amdgpu_buffer_rsrc_t q1r = make_rsrc(q, n_rows * row_bytes);
  const __amdgpu_buffer_rsrc_t q2r = (kDual || kPair) ? make_rsrc(q2, n_rows * row_bytes) : q1r;
  const __amdgpu_buffer_rsrc_t qr = (kPair && (wave & 1u)) ? q2r : q1r;
  const __amdgpu_buffer_rsrc_t qr2 = kPair ? qr : q2r;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, nsb * (kQ40 ? 128u : 1024u));
  float *xs = lds;
  float *ss = lds + n_units * kQ4kFlatSbFloats;
  const uint32_t bundle = 2u * W + half;
  typename FlatBufSel<RPW, 2, kQ5, kQ40>::type B;
  float acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
  if constexpr (kWhole) {
    flat_load<RPW, 2, false, kDual, kQ5, kQ40>(B, 0, qr, qr2, row_bytes, bundle, 0u, s, c);
#pragma unroll
    for (int g = 0; g < NIT; g += 4) { // x chunks in groups of 4 (16 VGPRs)
      float4 xg[4][512 / NT];
#pragma unroll
      for (int j = g; j < g + 4 && j < NIT; ++j)
        q4k_flat_load_chunk<NT>(xr, tid, (uint32_t)j, xg[j - g]);
#pragma unroll
      for (int j = g; j < g + 4 && j < NIT; ++j)
        q4k_flat_stage_chunk<NT, kQ40>(xs, ss, tid, (uint32_t)j, nsb, xg[j - g]);
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NIT; ++j) {
      const int p = j & 1;
      if (j + 1 < NIT)
        flat_load<RPW, 2, false, kDual, kQ5, kQ40>(B, p ^ 1, qr, qr2, row_bytes, bundle,
                                                   (uint32_t)(j + 1), s, c);
      const uint32_t sb = (uint32_t)j * 8u + s;
      if (mine && sb < n_units) flat_compute<RPW, 2, kQ5, kQ40>(B, p, xs, ss, sb, c, nsb, acc);
    }
    if constexpr (kPair)
      gate_up_pair_store(acc[0], W, wave, lane, mine, n_rows, y, ss + n_units * 8u);
    else if (mine)
      q4k_flat_store<RPW, kDual>(acc, 2u * W, lane, n_rows, y);
    return;
  }
  // x chunks are requested XD iterations ahead of their staging (issued
  // before the weights of the next iteration), the weights one iteration
  // ahead.  The load counter is in order, so with XD = 1 the staging of chunk
  // j + 1 waits behind the weights requested with it; XD = 2
  // (axh_q4k_matvec_onep_i{NIT}) takes that wait off the critical path where
  // nothing else on the CU hides it: one workgroup per CU (A/B in one run,
  // 4096 x 14336: 7.55-7.87 vs 7.88-8.01 us, 4096 x 8192 5.42 vs 5.58), but
  // not with two (8192 x 14336: 14.7 vs 13.8) or at three iterations (4096 x
  // 6144: 4.78 vs 4.70).  Three weight slots, or x three ahead, were slower.
  static_assert(XD == 1 || XD == 2, "x one or two chunks ahead");
  constexpr int XB = XD + 1;
  float4 xq[XB][512 / NT];
  q4k_flat_load_chunk<NT>(xr, tid, 0u, xq[0]);
  flat_load<RPW, 2, false, kDual, kQ5, kQ40>(B, 0, qr, qr2, row_bytes, bundle, 0u, s, c);
#pragma unroll
  for (int k = 1; k < XD; ++k) q4k_flat_load_chunk<NT>(xr, tid, (uint32_t)k, xq[k]);
#pragma unroll
  for (int j = 0; j < NIT; ++j) {
    const int p = j & 1;
    q4k_flat_stage_chunk<NT, kQ40>(xs, ss, tid, (uint32_t)j, nsb, xq[j % XB]);
    if (j + XD < NIT) q4k_flat_load_chunk<NT>(xr, tid, (uint32_t)(j + XD), xq[(j + XD) % XB]);
    if (j + 1 < NIT) // next iteration's weights, before the compute
      flat_load<RPW, 2, false, kDual, kQ5, kQ40>(B, p ^ 1, qr, qr2, row_bytes, bundle,
                                                 (uint32_t)(j + 1), s, c);
    __syncthreads();
    const uint32_t sb = (uint32_t)j * 8u + s;
    if (mine && sb < n_units) flat_compute<RPW, 2, kQ5, kQ40>(B, p, xs, ss, sb, c, nsb, acc);
  }
  if constexpr (kPair)
    gate_up_pair_store(acc[0], W, wave, lane, mine, n_rows, y, ss + n_units * 8u);
  else if (mine)
    q4k_flat_store<RPW, kDual>(acc, 2u * W, lane, n_rows, y);
}

#define AXH_Q4K_MATVEC_ONE(NIT)                                                                  \
  extern "C" __global__ void __launch_bounds__(512)                                              \
      axh_q4k_matvec_one_i##NIT(const uint8_t *__restrict__ q, const float *__restrict__ x,      \
                                float *__restrict__ y, AXH_ROWS_ARGS) { AXH_ROWS_UNPACK; \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4k_matvec_one<NIT>(q, q, x, y, a.n_rows, a.units_per_row, axh_lds_dyn);                     \
  }                                                                                              \
  extern "C" __global__ void __launch_bounds__(512)                                              \
      axh_q4k_matvec_onex_i##NIT(const uint8_t *__restrict__ q, const float *__restrict__ x,     \
                                 float *__restrict__ y, AXH_ROWS_ARGS) { AXH_ROWS_UNPACK; \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4k_matvec_one<NIT, false, false, true>(q, q, x, y, a.n_rows, a.units_per_row, axh_lds_dyn); \
  }
AXH_Q4K_MATVEC_ONE(1)
AXH_Q4K_MATVEC_ONE(2)
AXH_Q4K_MATVEC_ONE(3)
AXH_Q4K_MATVEC_ONE(4)
AXH_Q4K_MATVEC_ONE(5)
AXH_Q4K_MATVEC_ONE(6)
AXH_Q4K_MATVEC_ONE(7)
AXH_Q4K_MATVEC_ONE(8)
AXH_Q4K_MATVEC_ONE(9)
AXH_Q4K_MATVEC_ONE(10)
AXH_Q4K_MATVEC_ONE(11)
AXH_Q4K_MATVEC_ONE(12)
AXH_Q4K_MATVEC_ONE(13)
AXH_Q4K_MATVEC_ONE(14)
AXH_Q4K_MATVEC_ONE(15)
AXH_Q4K_MATVEC_ONE(16)

#define AXH_Q5K_MATVEC_ONE(NIT)                                                                  \
  extern "C" __global__ void __launch_bounds__(512)                                              \
      axh_q5k_matvec_one_i##NIT(const uint8_t *__restrict__ q, const float *__restrict__ x,      \
                                float *__restrict__ y, AXH_ROWS_ARGS) { AXH_ROWS_UNPACK; \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4k_matvec_one<NIT, false, true>(q, q, x, y, a.n_rows, a.units_per_row, axh_lds_dyn);        \
  }
#define AXH_Q5K_MATVEC_ONEP(NIT)                                                                 \
  extern "C" __global__ void __launch_bounds__(512)                                              \
      axh_q5k_matvec_onep_i##NIT(const uint8_t *__restrict__ q, const float *__restrict__ x,     \
                                 float *__restrict__ y, AXH_ROWS_ARGS) { AXH_ROWS_UNPACK;        \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4k_matvec_one<NIT, false, true, false, 2>(q, q, x, y, a.n_rows, a.units_per_row,            \
                                               axh_lds_dyn);                                     \
  }
AXH_Q5K_MATVEC_ONE(1)
AXH_Q5K_MATVEC_ONE(2)
AXH_Q5K_MATVEC_ONE(3)
AXH_Q5K_MATVEC_ONEP(3)
AXH_Q5K_MATVEC_ONE(4)
AXH_Q5K_MATVEC_ONEP(4)
AXH_Q5K_MATVEC_ONE(5)
AXH_Q5K_MATVEC_ONEP(5)
AXH_Q5K_MATVEC_ONE(6)
AXH_Q5K_MATVEC_ONEP(6)
AXH_Q5K_MATVEC_ONE(7)
AXH_Q5K_MATVEC_ONEP(7)
AXH_Q5K_MATVEC_ONE(8)
AXH_Q5K_MATVEC_ONEP(8)

#define AXH_Q4K_MATVEC_ONEP(NIT)                                                                 \
  extern "C" __global__ void __launch_bounds__(512)                                              \
      axh_q4k_matvec_onep_i##NIT(const uint8_t *__restrict__ q, const float *__restrict__ x,     \
                                 float *__restrict__ y, AXH_ROWS_ARGS) { AXH_ROWS_UNPACK; \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4k_matvec_one<NIT, false, false, false, 2>(q, q, x, y, a.n_rows, a.units_per_row,           \
                                                axh_lds_dyn);                                    \
  }
AXH_Q4K_MATVEC_ONEP(3)
AXH_Q4K_MATVEC_ONEP(4)
AXH_Q4K_MATVEC_ONEP(5)
AXH_Q4K_MATVEC_ONEP(6)
AXH_Q4K_MATVEC_ONEP(7)
AXH_Q4K_MATVEC_ONEP(8)
AXH_Q4K_MATVEC_ONEP(9)
AXH_Q4K_MATVEC_ONEP(10)
AXH_Q4K_MATVEC_ONEP(11)
AXH_Q4K_MATVEC_ONEP(12)
AXH_Q4K_MATVEC_ONEP(13)
AXH_Q4K_MATVEC_ONEP(14)
AXH_Q4K_MATVEC_ONEP(15)
AXH_Q4K_MATVEC_ONEP(16)

#define AXH_Q4K_MATVEC_FLAT(RPW, NW, PF, NT)                                                     \
  extern "C" __global__ void __launch_bounds__(NW * 64)                                          \
      axh_q4k_matvec_flat_r##RPW##_w##NW##_p##PF##_n##NT(const uint8_t *__restrict__ q,          \
                                                         const float *__restrict__ x,            \
                                                         float *__restrict__ y, AXH_ROWS_ARGS) { AXH_ROWS_UNPACK; \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4k_matvec_flat<RPW, NW, PF, NT != 0, 1>(q, q, x, y, a.n_rows, a.units_per_row,             \
                                               axh_lds_dyn);                                     \
  }
// Two staged x sub-blocks per thread (rows of up to 2 * NW * 8 superblocks).
#define AXH_Q4K_MATVEC_FLAT_X2(RPW, NW, PF, NT)                                                  \
  extern "C" __global__ void __launch_bounds__(NW * 64)                                          \
      axh_q4k_matvec_flat_r##RPW##_w##NW##_p##PF##_n##NT##_x2(const uint8_t *__restrict__ q,     \
                                                              const float *__restrict__ x,       \
                                                              float *__restrict__ y,             \
                                                              AXH_ROWS_ARGS) { AXH_ROWS_UNPACK; \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4k_matvec_flat<RPW, NW, PF, NT != 0, 2>(q, q, x, y, a.n_rows, a.units_per_row,             \
                                               axh_lds_dyn);                                     \
  }

// ===========================================================================
// Q6_K matvec (ggml k-quant, 210-byte superblocks; no reference counterpart).
// Superblock: ql[128] @0, qh[64] @128, int8 scales[16] @192, f16 d @208.
// Weight 128n + 32p + l (half n, part p = 0..3, l = 0..31) has the 6-bit
// value q = nibble | (2 bits of qh[32n + l] at 2p) << 4, the nibble being the
// low (p = 0, 1) or high (p = 2, 3) half of ql[64n + l + 32(p & 1)], and
// w = d * scales[8n + 2p + l/16] * (q - 32) (exact in f32).
//
// Same persistent skeleton as the Q4_K flat kernel (pairs of RPW-row
// bundles per wave, 16 superblocks per wave iteration, 4 lanes each, loads PF
// iterations ahead).  Lane c of a superblock takes half n = c/2 and
// l in [16(c&1), 16(c&1) + 16): 64 weights, 4 parts of 16.  Its bytes are
// three 16-byte runs (ql for parts 0/2, ql for parts 1/3, qh), the 16 scale
// bytes and d.  Superblocks start at 2-byte boundaries (210 = 2 mod 4); each
// 16-byte run is one 16-byte load at its own (possibly 2-byte-aligned)
// address, and every read lies inside the superblock.
//
// LDS: xs[sb*272 + 64p + 16i + 4c + e] = x[sb*256 + 128n + 32p + 16h + 4i + e] * 2^24
//      (c = 2n + h), and ss[sb*16 + 4c + p] = sum of those 16 x (unscaled), so
//      sum_l (q_l - 32) x_l = sum_l q_l x_l - 32 * ss.
// ===========================================================================
constexpr uint32_t kQ6kSbBytes = 210;
constexpr uint32_t kQ6kSbFloats = 272;

// Coalesced as q4k_flat_stage_xc: float4 f holds elements 4w..4w+3 of
// superblock f / 64 (w = f % 64), i.e. 128n + 32p + 16h + 4i with n = w / 32,
// p = (w / 8) & 3, h = (w / 4) & 1, i = w & 3; a lane quad holds one
// 16-element group (n, p, h), summed with DPP.
template <int NT, int XP>
__device__ __forceinline__ void q6k_stage_xc(float *xs, float *ss, uint32_t tid, uint32_t nsb,
                                             const float4 (&v)[8 * XP]) {
#pragma unroll
  for (int k = 0; k < 8 * XP; ++k) {
    const uint32_t f = tid + (uint32_t)k * NT;
    const float4 a = v[k];
    float s = (a.x + a.y) + (a.z + a.w);
    s += dpp_mov<0xB1>(s); // quad_perm [1,0,3,2]
    s += dpp_mov<0x4E>(s); // quad_perm [2,3,0,1]: the quad's sum in every lane
    if (f < nsb * 64u) {
      const uint32_t sb = f >> 6, w = f & 63u;
      const uint32_t n = w >> 5, p = (w >> 3) & 3u, h = (w >> 2) & 1u, i = w & 3u;
      const uint32_t c = 2u * n + h;
      *reinterpret_cast<float4 *>(xs + sb * kQ6kSbFloats + 64u * p + 4u * c + 16u * i) =
          make_float4(a.x * 16777216.0f, a.y * 16777216.0f, a.z * 16777216.0f,
                      a.w * 16777216.0f);
      if (i == 0u) ss[sb * 16u + 4u * c + p] = s;
    }
  }
}

// Dword-aligned loads of a superblock's runs.  A superblock starts at 0 or 2
// mod 4 (210 = 2 mod 4), and every run starts at a multiple of 16 from it,
// so all of a superblock's runs share one misalignment sh = start & 3 (0 or
// 2).  A 16-byte load at a 2-mod-4 address is split by the memory pipeline:
// with the decode and x reads taken out (timing-only copies), the 128256 x
// 4096 head took 78.0 us with the runs loaded as they lie and 71.0 us with
// their addresses rounded down to 4 bytes.  So each lane loads its three
// 16-byte runs (ql low, ql high, qh) from run start - sh, and the dword that
// completes a run is the first dword of another run of the same superblock:
// with lane c = 2n + h of a lane quad holding half n, l in [16h, 16h + 16),
//   ql low  (n, 0) <- ql low  (n, 1);  ql low  (n, 1) <- ql high (n, 0)
//   ql high (n, 0) <- ql high (n, 1);  ql high (0, 1) <- ql low (1, 0);
//   ql high (1, 1) <- qh (0, 0);       qh (n, h) <- qh of the next lane,
//   qh (1, 1) <- the scale run's first dword (bytes 190..193),
// fetched with a quad permute, and v_alignbyte shifts each run into place.
// The lanes of half 0 load the 16 scale bytes from 192 - sh; the lanes of
// half 1 need scale bytes 200..207, loaded from 192 (sh = 0) or 194 (sh = 2),
// so that no load leaves the superblock (the d load stays a 2-byte load at
// 208: a dword there would reach past the last superblock of the matrix).
template <int RPW, int PF>
struct Q6kFlatBuf {
  uint4 lo[PF][RPW], hi[PF][RPW], qh[PF][RPW], sc[PF][RPW];
  uint32_t d[PF][RPW], sh[PF][RPW]; // sh: the superblock's start & 3
};

template <int RPW, int PF>
__device__ __forceinline__ void q6k_flat_load(Q6kFlatBuf<RPW, PF> &B, int p,
                                              __amdgpu_buffer_rsrc_t qr, uint32_t row_bytes,
                                              uint32_t bundle, uint32_t it, uint32_t s,
                                              uint32_t c) {
  const uint32_t n = c >> 1, h = c & 1u;
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const uint32_t o = (bundle * RPW + (uint32_t)r) * row_bytes + (it * 8u + s) * kQ6kSbBytes;
    const uint32_t sh = o & 3u, a = o - sh; // a: the dword-aligned start
    const uint32_t sc_off = a + 192u + (n != 0u && sh != 0u ? 4u : 0u);
    const u32x4_t lo = __builtin_amdgcn_raw_buffer_load_b128(qr, (int)(a + 64u * n + 16u * h), 0, 0);
    const u32x4_t hi =
        __builtin_amdgcn_raw_buffer_load_b128(qr, (int)(a + 64u * n + 32u + 16u * h), 0, 0);
    const u32x4_t qh =
        __builtin_amdgcn_raw_buffer_load_b128(qr, (int)(a + 128u + 32u * n + 16u * h), 0, 0);
    const u32x4_t sc = __builtin_amdgcn_raw_buffer_load_b128(qr, (int)sc_off, 0, 0);
    B.lo[p][r] = make_uint4(lo.x, lo.y, lo.z, lo.w);
    B.hi[p][r] = make_uint4(hi.x, hi.y, hi.z, hi.w);
    B.qh[p][r] = make_uint4(qh.x, qh.y, qh.z, qh.w);
    B.sc[p][r] = make_uint4(sc.x, sc.y, sc.z, sc.w);
    B.d[p][r] = __builtin_amdgcn_raw_buffer_load_b16(qr, (int)(o + 208u), 0, 0);
    B.sh[p][r] = sh;
  }
}

__device__ __forceinline__ uint32_t quad_perm_u32_b1(uint32_t v) { // quad_perm [1,0,3,2]
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t quad_perm_u32_39(uint32_t v) { // quad_perm [1,2,3,0]
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x39, 0xF, 0xF, false);
}

// A run's four dwords from its dword-aligned load v and the next dword e,
// shifted by sh bytes (sh = 0 returns v).
__device__ __forceinline__ void q6k_align_run(uint4 v, uint32_t e, uint32_t sh, uint32_t (&w)[4]) {
  w[0] = __builtin_amdgcn_alignbyte(v.y, v.x, sh);
  w[1] = __builtin_amdgcn_alignbyte(v.z, v.y, sh);
  w[2] = __builtin_amdgcn_alignbyte(v.w, v.z, sh);
  w[3] = __builtin_amdgcn_alignbyte(e, v.w, sh);
}

// (a & m) | c as one v_and_or_b32 whose result the caller then masks and
// permutes: written out, the compiler forms the masked half with a v_bitop3
// of a & m and c, and the full value with a separate v_or for the permute.
__device__ __forceinline__ uint32_t q6k_and_or(uint32_t a, uint32_t m, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(c));
  return r;
}

// Four bytes of 6-bit values (bits 6-7 clear) against four x (pre-scaled by
// 2^24): bytes 0 and 2 are the f16 halves of v & 0x00FF00FF, and one byte
// permute (v_perm_b32, selector 0x0C030C01: byte 1, zero, byte 3, zero) puts
// bytes 1 and 3 in the same places, where a shift and a mask took two.
__device__ __forceinline__ float q6k_bytes(uint32_t v, float4 x, float acc) {
  const uint32_t a = v & 0x00FF00FFu, b = __builtin_amdgcn_perm(v, v, 0x0C030C01u);
  acc = __builtin_fmaf(lo_half_f16(a), x.x, acc);
  acc = __builtin_fmaf(lo_half_f16(b), x.y, acc);
  acc = __builtin_fmaf(hi_half_f16(a), x.z, acc);
  acc = __builtin_fmaf(hi_half_f16(b), x.w, acc);
  return acc;
}

// One iteration of the Q6_K kernels for the RPW rows of slot p: lane quad s
// holds superblock sb, lane c of it half n = c / 2 and l in [16(c & 1),
// 16(c & 1) + 16).  acc[r] += this lane's share of row r.  The quad permutes
// read the other lanes of the quad, which take the same branch (same sb).
template <int RPW, int NS>
__device__ __forceinline__ void q6k_flat_compute(const Q6kFlatBuf<RPW, NS> &B, int p,
                                                 const float *xs, const float *ss, uint32_t sb,
                                                 uint32_t c, float (&acc)[RPW]) {
  const uint32_t n = c >> 1, hsel = (c & 1u) * 8u; // scale byte of (n, h): 8n + 2p + h
  const float *xb = xs + sb * kQ6kSbFloats + 4u * c;
  const float4 sums = *reinterpret_cast<const float4 *>(ss + sb * 16u + 4u * c);
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const uint4 lo = B.lo[p][r], hi = B.hi[p][r], qh = B.qh[p][r], sc = B.sc[p][r];
    const uint32_t sh = B.sh[p][r];
    // the dword after each run, from the lane of the quad that loaded it
    const uint32_t lo_e = quad_perm_u32_b1((c & 1u) ? lo.x : hi.x);
    const uint32_t hi_e = quad_perm_u32_39(c == 0u ? qh.x : c == 2u ? lo.x : hi.x);
    const uint32_t qh_e = quad_perm_u32_39(c == 0u ? sc.x : qh.x);
    uint32_t lw[4], hw[4], qw[4];
    q6k_align_run(lo, lo_e, sh, lw);
    q6k_align_run(hi, hi_e, sh, hw);
    q6k_align_run(qh, qh_e, sh, qw);
    float d0 = 0.0f, d1 = 0.0f, d2 = 0.0f, d3 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v0 = q6k_and_or(lw[i], 0x0F0F0F0Fu, (qw[i] << 4) & 0x30303030u);
      const uint32_t v1 = q6k_and_or(hw[i], 0x0F0F0F0Fu, (qw[i] << 2) & 0x30303030u);
      const uint32_t v2 = q6k_and_or(lw[i] >> 4, 0x0F0F0F0Fu, qw[i] & 0x30303030u);
      const uint32_t v3 = q6k_and_or(hw[i] >> 4, 0x0F0F0F0Fu, (qw[i] >> 2) & 0x30303030u);
      d0 = q6k_bytes(v0, *reinterpret_cast<const float4 *>(xb + 16u * i), d0);
      d1 = q6k_bytes(v1, *reinterpret_cast<const float4 *>(xb + 64u + 16u * i), d1);
      d2 = q6k_bytes(v2, *reinterpret_cast<const float4 *>(xb + 128u + 16u * i), d2);
      d3 = q6k_bytes(v3, *reinterpret_cast<const float4 *>(xb + 192u + 16u * i), d3);
    }
    // scale bytes 8n + h + {0, 2} (dword 2n) and 8n + h + {4, 6} (dword 2n + 1):
    // dwords k, k + 1 of the scale load shifted by sh, k = 0 for half 0,
    // 2 for half 1 at sh = 0 (loaded from 192), 1 at sh = 2 (from 194)
    const uint32_t k0 = n ? (sh ? sc.y : sc.z) : sc.x;
    const uint32_t k1 = n ? (sh ? sc.z : sc.w) : sc.y;
    const uint32_t k2 = n ? sc.w : sc.z;
    const uint32_t s0 = __builtin_amdgcn_alignbyte(k1, k0, sh);
    const uint32_t s1 = __builtin_amdgcn_alignbyte(k2, k1, sh);
    // int8 scales (the sign-extending byte extract; a bit-field builtin
    // returning an unsigned type would turn -1 into 2^32 - 1 here)
    const float c0 = (float)(int8_t)(s0 >> hsel);
    const float c1 = (float)(int8_t)(s0 >> (hsel + 16u));
    const float c2 = (float)(int8_t)(s1 >> hsel);
    const float c3 = (float)(int8_t)(s1 >> (hsel + 16u));
    float t = c0 * __builtin_fmaf(-32.0f, sums.x, d0);
    t = __builtin_fmaf(c1, __builtin_fmaf(-32.0f, sums.y, d1), t);
    t = __builtin_fmaf(c2, __builtin_fmaf(-32.0f, sums.z, d2), t);
    t = __builtin_fmaf(c3, __builtin_fmaf(-32.0f, sums.w, d3), t);
    acc[r] = __builtin_fmaf(f16_to_f32(B.d[p][r]), t, acc[r]);
  }
}

// Reduce the pair of bundles (bundle0, bundle0 + 1) a wave finished (each
// half-wave's lanes hold one bundle's partial sums) and store it.
template <int RPW>
__device__ __forceinline__ void q6k_flat_store(float (&acc)[RPW], uint32_t bundle0, uint32_t lane,
                                               uint32_t n_rows, float *__restrict__ y) {
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    float v = acc[r];
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    v += dpp_mov<0x141>(v);
    v += dpp_mov<0x140>(v);
    const int vi = __builtin_bit_cast(int, v);
    const float h0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 0)) +
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 16));
    const float h1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 32)) +
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 48));
    const uint32_t r0 = bundle0 * RPW + (uint32_t)r;
    const uint32_t r1 = (bundle0 + 1u) * RPW + (uint32_t)r;
    if (lane == 0 && r0 < n_rows) y[r0] = h0;
    if (lane == 0 && r1 < n_rows) y[r1] = h1;
    acc[r] = 0.0f;
  }
}

template <int RPW, int NW, int PF, int XP>
__device__ __forceinline__ void q6k_matvec_flat(const uint8_t *__restrict__ q,
                                                const float *__restrict__ x,
                                                float *__restrict__ y, uint32_t n_rows,
                                                uint32_t nsb, float *lds) {
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t G = lane >> 2, half = G >> 3, s = G & 7u, c = lane & 3u;
  const uint32_t total_waves = gridDim.x * NW;
  const uint32_t W = blockIdx.x * NW + wave;
  const uint32_t n_bundles = (n_rows + RPW - 1) / RPW;
  const uint32_t n_pairs = (n_bundles + 1u) >> 1;
  if (nsb == 0) {
    for (uint32_t r = W * 64u + lane; r < n_rows; r += total_waves * 64u) y[r] = 0.0f;
    return;
  }
  const uint32_t n_my = W < n_pairs ? (n_pairs - 1u - W) / total_waves + 1u : 0u;
  constexpr bool kEarly = PF == 1;        // refill before the compute
  constexpr int kSlots = kEarly ? 2 : PF; // register slots
  const uint32_t n_it = (nsb + 7u) >> 3;
  const uint32_t total = (n_my * n_it + (kSlots - 1)) / kSlots * kSlots;
  // The host guarantees n_rows * row_bytes < 2^32 for this kernel.
  const uint32_t row_bytes = nsb * kQ6kSbBytes;
  const __amdgpu_buffer_rsrc_t qr = make_rsrc(q, n_rows * row_bytes);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, nsb * 1024u);
  float *xs = lds;
  float *ss = lds + nsb * kQ6kSbFloats;

  // Prologue as in the Q4_K flat kernel: x first, then (for long rows once x
  // has arrived) the weight prefetch, then the LDS writes.
  float4 xv[8 * XP];
  q4k_flat_load_xc<NW * 64, XP>(xr, tid, xv);
  __builtin_amdgcn_sched_barrier(0);
  if (nsb >= kWaitXMinSb) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);

  Q6kFlatBuf<RPW, kSlots> B;
  uint32_t l_pi = 0, l_it = 0;
#pragma unroll
  for (int p = 0; p < PF; ++p) {
    const uint32_t bundle = 2u * (W + l_pi * total_waves) + half;
    q6k_flat_load<RPW, kSlots>(B, p, qr, row_bytes, bundle, l_it, s, c);
    if (++l_it == n_it) { l_it = 0; ++l_pi; }
  }
  __builtin_amdgcn_sched_barrier(0);
  q6k_stage_xc<NW * 64, XP>(xs, ss, tid, nsb, xv);
  __syncthreads();

  float acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
  uint32_t c_pi = 0, c_it = 0;
  for (uint32_t j0 = 0; j0 < total; j0 += kSlots) {
#pragma unroll
    for (int p = 0; p < kSlots; ++p) {
      if constexpr (kEarly) { // the other slot: the next iteration (unconditional)
        const uint32_t bundle = 2u * (W + l_pi * total_waves) + half;
        q6k_flat_load<RPW, kSlots>(B, (p + 1) % kSlots, qr, row_bytes, bundle, l_it, s, c);
        if (++l_it == n_it) { l_it = 0; ++l_pi; }
      }
      const uint32_t sb = c_it * 8u + s;
      if (c_pi < n_my && sb < nsb) q6k_flat_compute<RPW, kSlots>(B, p, xs, ss, sb, c, acc);
      if constexpr (!kEarly) {
        const uint32_t bundle = 2u * (W + l_pi * total_waves) + half;
        q6k_flat_load<RPW, kSlots>(B, p, qr, row_bytes, bundle, l_it, s, c);
        if (++l_it == n_it) { l_it = 0; ++l_pi; }
      }
      if (++c_it == n_it) {
        if (c_pi < n_my) q6k_flat_store<RPW>(acc, 2u * (W + c_pi * total_waves), lane, n_rows, y);
        c_it = 0;
        ++c_pi;
      }
    }
  }
}

#define AXH_Q6K_MATVEC_FLAT(RPW, NW, PF, XP)                                                     \
  extern "C" __global__ void __launch_bounds__(NW * 64)                                          \
      axh_q6k_matvec_flat_r##RPW##_w##NW##_p##PF##_x##XP(const uint8_t *__restrict__ q,          \
                                                         const float *__restrict__ x,            \
                                                         float *__restrict__ y, AXH_ROWS_ARGS) { AXH_ROWS_UNPACK; \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q6k_matvec_flat<RPW, NW, PF, XP>(q, x, y, a.n_rows, a.units_per_row, axh_lds_dyn);          \
  }

#define AXH_Q5K_MATVEC_FLAT(RPW, NW, PF, XP)                                                     \
  extern "C" __global__ void __launch_bounds__(NW * 64)                                          \
      axh_q5k_matvec_flat_r##RPW##_w##NW##_p##PF##_x##XP(const uint8_t *__restrict__ q,          \
                                                         const float *__restrict__ x,            \
                                                         float *__restrict__ y, AXH_ROWS_ARGS) { AXH_ROWS_UNPACK; \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4k_matvec_flat<RPW, NW, PF, false, XP, false, true>(q, q, x, y, a.n_rows,                   \
                                                         a.units_per_row, axh_lds_dyn);          \
  }

AXH_Q5K_MATVEC_FLAT(1, 4, 2, 1)
AXH_Q5K_MATVEC_FLAT(1, 4, 1, 1)
AXH_Q5K_MATVEC_FLAT(1, 8, 1, 1)
AXH_Q5K_MATVEC_FLAT(1, 8, 2, 1)
AXH_Q5K_MATVEC_FLAT(2, 4, 2, 1)
AXH_Q5K_MATVEC_FLAT(1, 4, 2, 2)
AXH_Q5K_MATVEC_FLAT(1, 8, 2, 2)

AXH_Q6K_MATVEC_FLAT(1, 4, 2, 1)
AXH_Q6K_MATVEC_FLAT(1, 4, 1, 1)
AXH_Q6K_MATVEC_FLAT(1, 8, 1, 1)
AXH_Q6K_MATVEC_FLAT(1, 8, 2, 1)
AXH_Q6K_MATVEC_FLAT(1, 4, 4, 1)
AXH_Q6K_MATVEC_FLAT(2, 4, 2, 1)
AXH_Q6K_MATVEC_FLAT(1, 4, 2, 2)
AXH_Q6K_MATVEC_FLAT(1, 8, 2, 2)

// x chunk j of the Q6_K one-pass kernel: superblocks [8j, 8j + 8), float4 f
// = 512j + tid + i*NT, staged with the mapping and layout of q6k_stage_xc.
// Chunks past the row read zeros (buffer range) and stage nothing.
template <int NT>
__device__ __forceinline__ void q6k_stage_chunk(float *xs, float *ss, uint32_t tid, uint32_t j,
                                                uint32_t nsb, const float4 (&v)[512 / NT]) {
#pragma unroll
  for (int i = 0; i < 512 / NT; ++i) {
    const uint32_t f = j * 512u + tid + (uint32_t)i * NT;
    const float4 a = v[i];
    float sm = (a.x + a.y) + (a.z + a.w);
    sm += dpp_mov<0xB1>(sm);
    sm += dpp_mov<0x4E>(sm);
    if (f < nsb * 64u) {
      const uint32_t sb = f >> 6, w = f & 63u;
      const uint32_t n = w >> 5, p = (w >> 3) & 3u, h = (w >> 2) & 1u, i4 = w & 3u;
      const uint32_t c = 2u * n + h;
      *reinterpret_cast<float4 *>(xs + sb * kQ6kSbFloats + 64u * p + 4u * c + 16u * i4) =
          make_float4(a.x * 16777216.0f, a.y * 16777216.0f, a.z * 16777216.0f,
                      a.w * 16777216.0f);
      if (i4 == 0u) ss[sb * 16u + 4u * c + p] = sm;
    }
  }
}

// Q6_K one pass, one pair of rows per wave (axh_q6k_matvec_one_i{NIT}): rows
// of 8 * (NIT - 1) < nsb <= 8 * NIT superblocks, 8 waves per workgroup, wave
// W takes rows 2W and 2W + 1, one workgroup per 16 rows, all launched.  The
// Q4_K one-pass order (q4k_matvec_one) with the Q6_K loads and decode of the
// persistent kernel, so its output equals the persistent kernel's bit for
// bit: x staged chunk by chunk (8 superblocks, 8 KiB) with the next
// iteration's weights in flight, fully unrolled, one barrier per iteration.
// Every chunk has its own LDS region (nsb * 1152 bytes in all), so a chunk is
// never overwritten while a wave still reads it.  XD = 2 (x two chunks
// ahead) and longer rows measured even with the persistent kernel (4096 x
// 14336, seven iterations: 11.80-11.85 vs 11.87 us) and are not built.
template <int NIT, int XD>
__device__ __forceinline__ void q6k_matvec_one(const uint8_t *__restrict__ q,
                                               const float *__restrict__ x, float *__restrict__ y,
                                               uint32_t n_rows, uint32_t nsb, float *lds) {
  constexpr int NW = 8, NT = NW * 64;
  static_assert(XD == 1 || XD == 2, "x one or two chunks ahead");
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t G = lane >> 2, half = G >> 3, s = G & 7u, c = lane & 3u;
  const uint32_t W = blockIdx.x * NW + wave;
  const bool mine = W < (n_rows + 1u) >> 1; // this wave has a pair of rows
  // The host guarantees n_rows * row_bytes < 2^32 for this kernel.
  const uint32_t row_bytes = nsb * kQ6kSbBytes;
  const __amdgpu_buffer_rsrc_t qr = make_rsrc(q, n_rows * row_bytes);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, nsb * 1024u);
  float *xs = lds;
  float *ss = lds + nsb * kQ6kSbFloats;
  const uint32_t bundle = 2u * W + half;
  Q6kFlatBuf<1, 2> B;
  float acc[1] = {0.0f};
  constexpr int XB = XD + 1;
  float4 xq[XB][512 / NT];
  q4k_flat_load_chunk<NT>(xr, tid, 0u, xq[0]);
  q6k_flat_load<1, 2>(B, 0, qr, row_bytes, bundle, 0u, s, c);
#pragma unroll
  for (int k = 1; k < XD; ++k) q4k_flat_load_chunk<NT>(xr, tid, (uint32_t)k, xq[k]);
#pragma unroll
  for (int j = 0; j < NIT; ++j) {
    const int p = j & 1;
    q6k_stage_chunk<NT>(xs, ss, tid, (uint32_t)j, nsb, xq[j % XB]);
    if (j + XD < NIT) q4k_flat_load_chunk<NT>(xr, tid, (uint32_t)(j + XD), xq[(j + XD) % XB]);
    if (j + 1 < NIT) // next iteration's weights, before the compute
      q6k_flat_load<1, 2>(B, p ^ 1, qr, row_bytes, bundle, (uint32_t)(j + 1), s, c);
    __syncthreads();
    const uint32_t sb = (uint32_t)j * 8u + s;
    if (mine && sb < nsb) q6k_flat_compute<1, 2>(B, p, xs, ss, sb, c, acc);
  }
  if (mine) q6k_flat_store<1>(acc, 2u * W, lane, n_rows, y);
}

#define AXH_Q6K_MATVEC_ONE(NIT, XD, TAG)                                                         \
  extern "C" __global__ void __launch_bounds__(512)                                              \
      axh_q6k_matvec_one##TAG##_i##NIT(const uint8_t *__restrict__ q,                            \
                                       const float *__restrict__ x, float *__restrict__ y,       \
                                       AXH_ROWS_ARGS) { AXH_ROWS_UNPACK;                         \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q6k_matvec_one<NIT, XD>(q, x, y, a.n_rows, a.units_per_row, axh_lds_dyn);                    \
  }
AXH_Q6K_MATVEC_ONE(1, 1, )
AXH_Q6K_MATVEC_ONE(2, 1, )
AXH_Q6K_MATVEC_ONE(3, 1, )
AXH_Q6K_MATVEC_ONE(3, 2, p)
AXH_Q6K_MATVEC_ONE(4, 1, )
AXH_Q6K_MATVEC_ONE(4, 2, p)
AXH_Q6K_MATVEC_ONE(5, 1, )
AXH_Q6K_MATVEC_ONE(5, 2, p)
AXH_Q6K_MATVEC_ONE(6, 1, )
AXH_Q6K_MATVEC_ONE(6, 2, p)
AXH_Q6K_MATVEC_ONE(7, 1, )
AXH_Q6K_MATVEC_ONE(7, 2, p)
AXH_Q6K_MATVEC_ONE(8, 1, )
AXH_Q6K_MATVEC_ONE(8, 2, p)

// Fused SwiGLU gate/up projection: y[r] = silu(Wg[r].x) * (Wu[r].x), ROWS
// output rows per bundle (2 * ROWS weight rows per lane group).
#define AXH_Q4K_GATE_UP(ROWS, NW, PF, XP)                                                        \
  extern "C" __global__ void __launch_bounds__(NW * 64)                                          \
      axh_q4k_gate_up_r##ROWS##_w##NW##_p##PF##_x##XP(                                           \
          const uint8_t *__restrict__ qg, const uint8_t *__restrict__ qu,                        \
          const float *__restrict__ x, float *__restrict__ y, AXH_ROWS_ARGS) { AXH_ROWS_UNPACK; \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4k_matvec_flat<2 * ROWS, NW, PF, false, XP, true>(qg, qu, x, y, a.n_rows, a.units_per_row,  \
                                                       axh_lds_dyn);                             \
  }

// The same fusion over two Q4_0 matrices (rows read as octets of 8 blocks).
#define AXH_Q4_0_GATE_UP(ROWS, NW, PF, XP)                                                       \
  extern "C" __global__ void __launch_bounds__(NW * 64)                                          \
      axh_q4_0_gate_up_r##ROWS##_w##NW##_p##PF##_x##XP(                                          \
          const uint8_t *__restrict__ qg, const uint8_t *__restrict__ qu,                        \
          const float *__restrict__ x, float *__restrict__ y, AXH_ROWS_ARGS) { AXH_ROWS_UNPACK; \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4k_matvec_flat<2 * ROWS, NW, PF, false, XP, true, false, true>(                             \
        qg, qu, x, y, a.n_rows, a.units_per_row, axh_lds_dyn);                                   \
  }

// Wave-paired one-pass gate/up (axh_q4k_gate_up_one{,x}_i{NIT} and the Q4_0
// and Q5_K axh_{q4_0,q5k}_gate_up_one{,x}_i{NIT}): one workgroup of 8 waves
// per 8 output rows, the even wave of a pair reading gate rows and the odd
// wave the same up rows, x staged chunk by chunk (one) or whole (onex).
#define AXH_GATE_UP_ONE(FMT, Q5, Q40, NIT)                                                       \
  extern "C" __global__ void __launch_bounds__(512)                                              \
      axh_##FMT##_gate_up_one_i##NIT(const uint8_t *__restrict__ qg,                             \
                                     const uint8_t *__restrict__ qu,                             \
                                     const float *__restrict__ x, float *__restrict__ y,         \
                                     AXH_ROWS_ARGS) { AXH_ROWS_UNPACK;                           \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4k_matvec_one<NIT, false, Q5, false, 1, Q40, true>(qg, qu, x, y, a.n_rows,                  \
                                                        a.units_per_row, axh_lds_dyn);          \
  }                                                                                              \
  extern "C" __global__ void __launch_bounds__(512)                                              \
      axh_##FMT##_gate_up_onex_i##NIT(const uint8_t *__restrict__ qg,                            \
                                      const uint8_t *__restrict__ qu,                            \
                                      const float *__restrict__ x, float *__restrict__ y,        \
                                      AXH_ROWS_ARGS) { AXH_ROWS_UNPACK;                          \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4k_matvec_one<NIT, false, Q5, true, 1, Q40, true>(qg, qu, x, y, a.n_rows,                   \
                                                       a.units_per_row, axh_lds_dyn);           \
  }
AXH_GATE_UP_ONE(q4k, false, false, 1)
AXH_GATE_UP_ONE(q4_0, false, true, 1)
AXH_GATE_UP_ONE(q5k, true, false, 1)
AXH_GATE_UP_ONE(q4k, false, false, 2)
AXH_GATE_UP_ONE(q4_0, false, true, 2)
AXH_GATE_UP_ONE(q5k, true, false, 2)
AXH_GATE_UP_ONE(q4k, false, false, 3)
AXH_GATE_UP_ONE(q4_0, false, true, 3)
AXH_GATE_UP_ONE(q5k, true, false, 3)
AXH_GATE_UP_ONE(q4k, false, false, 4)
AXH_GATE_UP_ONE(q4_0, false, true, 4)
AXH_GATE_UP_ONE(q5k, true, false, 4)
AXH_GATE_UP_ONE(q4k, false, false, 5)
AXH_GATE_UP_ONE(q4_0, false, true, 5)
AXH_GATE_UP_ONE(q5k, true, false, 5)
AXH_GATE_UP_ONE(q4k, false, false, 6)
AXH_GATE_UP_ONE(q4_0, false, true, 6)
AXH_GATE_UP_ONE(q5k, true, false, 6)
AXH_GATE_UP_ONE(q4k, false, false, 7)
AXH_GATE_UP_ONE(q4_0, false, true, 7)
AXH_GATE_UP_ONE(q5k, true, false, 7)
AXH_GATE_UP_ONE(q4k, false, false, 8)
AXH_GATE_UP_ONE(q4_0, false, true, 8)
AXH_GATE_UP_ONE(q5k, true, false, 8)

AXH_Q4K_GATE_UP(1, 4, 2, 1)
AXH_Q4K_GATE_UP(1, 4, 1, 1)
AXH_Q4K_GATE_UP(1, 8, 1, 1)
AXH_Q4K_GATE_UP(1, 4, 4, 1)
AXH_Q4K_GATE_UP(1, 8, 2, 1)
AXH_Q4K_GATE_UP(2, 4, 2, 1)
AXH_Q4K_GATE_UP(2, 8, 2, 1)
AXH_Q4K_GATE_UP(1, 4, 2, 2)
AXH_Q4K_GATE_UP(1, 8, 2, 2)
// ... and over two Q5_K matrices (the persistent kernel with both flags).
#define AXH_Q5K_GATE_UP(ROWS, NW, PF, XP)                                                        \
  extern "C" __global__ void __launch_bounds__(NW * 64)                                          \
      axh_q5k_gate_up_r##ROWS##_w##NW##_p##PF##_x##XP(                                           \
          const uint8_t *__restrict__ qg, const uint8_t *__restrict__ qu,                        \
          const float *__restrict__ x, float *__restrict__ y, AXH_ROWS_ARGS) { AXH_ROWS_UNPACK; \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4k_matvec_flat<2 * ROWS, NW, PF, false, XP, true, true>(qg, qu, x, y, a.n_rows,             \
                                                             a.units_per_row, axh_lds_dyn);      \
  }
AXH_Q5K_GATE_UP(1, 4, 1, 1)
AXH_Q5K_GATE_UP(1, 8, 1, 1)
AXH_Q5K_GATE_UP(1, 4, 2, 1)
AXH_Q5K_GATE_UP(1, 4, 2, 2)
AXH_Q4_0_GATE_UP(1, 4, 1, 1)
AXH_Q4_0_GATE_UP(1, 8, 1, 1)
AXH_Q4_0_GATE_UP(2, 4, 1, 1)
AXH_Q4_0_GATE_UP(1, 4, 2, 1)
AXH_Q4_0_GATE_UP(1, 8, 2, 1)
AXH_Q4_0_GATE_UP(1, 4, 2, 2)

AXH_Q4K_MATVEC_FLAT(1, 8, 2, 0)
AXH_Q4K_MATVEC_FLAT(1, 8, 1, 0)
AXH_Q4K_MATVEC_FLAT(1, 4, 1, 0)
AXH_Q4K_MATVEC_FLAT(2, 4, 1, 0)
AXH_Q4K_MATVEC_FLAT(2, 8, 1, 0)
AXH_Q4K_MATVEC_FLAT(1, 8, 4, 0)
AXH_Q4K_MATVEC_FLAT(1, 8, 7, 0)
AXH_Q4K_MATVEC_FLAT(1, 16, 2, 0)
AXH_Q4K_MATVEC_FLAT(1, 4, 7, 0)
AXH_Q4K_MATVEC_FLAT(2, 4, 2, 0)
AXH_Q4K_MATVEC_FLAT(2, 4, 4, 0)
AXH_Q4K_MATVEC_FLAT(2, 8, 2, 0)
AXH_Q4K_MATVEC_FLAT(2, 8, 4, 0)
AXH_Q4K_MATVEC_FLAT(4, 4, 2, 0)
AXH_Q4K_MATVEC_FLAT(1, 8, 7, 1)
AXH_Q4K_MATVEC_FLAT(2, 4, 2, 1)
AXH_Q4K_MATVEC_FLAT(2, 4, 4, 1)
AXH_Q4K_MATVEC_FLAT_X2(1, 4, 2, 0)
AXH_Q4K_MATVEC_FLAT_X2(1, 4, 4, 0)
AXH_Q4K_MATVEC_FLAT_X2(2, 4, 2, 0)
AXH_Q4K_MATVEC_FLAT_X2(2, 4, 4, 0)

// ---------------------------------------------------------------------------
// Column-slice Q4_K matvec: x held in VGPRs, rows streamed in batches.
//
// Thread t of the workgroup owns quarter t of every row: superblock sb = t/4,
// c = t%4, i.e. qs bytes [32c, 32c+32) of that superblock, whose low nibbles
// are weights 64c + i of sub-block 2c and high nibbles weights 64c + 32 + i of
// sub-block 2c+1 (i = 0..31).  The workgroup has NW*64 >= 4*nsb threads;
// threads past 4*nsb read zeros (buffer range check) and add 0.
//
// Each thread loads its 64 x values once, keeps them in VGPRs pre-scaled by
// 2^24 (sub-block 2c) and 2^20 (sub-block 2c+1) for the f16-subnormal nibble
// encoding, with the two unscaled sub-block sums for the dmin term.  No LDS
// staging of x and no barrier before the first row.
//
// Rows go in batches of RB: workgroup g handles batches g, g + G, g + 2G, ...
// (G = gridDim.x) and keeps the next batch's weights in flight while it
// computes the current one.  Per row the 64 lane partials are summed with
// DPP (all 16-lane rows, then row_bcast15/31 into lane 63); with NW > 1 the
// wave sums meet in LDS (double-buffered by batch parity, one barrier per
// batch).
// ---------------------------------------------------------------------------
template <int RB>
struct Q4kColsBuf {
  uint4 h[RB], a[RB], b[RB];
};

// Out-of-range offset for idle lanes and rows past the matrix: the buffer
// range check returns zeros (the host keeps n_rows * row_bytes below it).
constexpr uint32_t kQ4kColsOob = 0xFFFFFF00u;

// `lane_off` is this lane's header offset within a row, or kQ4kColsOob for
// an idle lane.
template <int RB, bool kNT>
__device__ __forceinline__ void q4k_cols_load(Q4kColsBuf<RB> &B, __amdgpu_buffer_rsrc_t qr,
                                              uint32_t batch, uint32_t n_rows,
                                              uint32_t row_bytes, uint32_t lane_off,
                                              uint32_t c) {
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const uint32_t row = batch * RB + (uint32_t)r;
    const uint32_t off =
        (row < n_rows && lane_off != kQ4kColsOob) ? row * row_bytes + lane_off : kQ4kColsOob;
    B.h[r] = buf_load16<kNT>(qr, off);
    B.a[r] = buf_load16<kNT>(qr, off + 16u + 32u * c);
    B.b[r] = buf_load16<kNT>(qr, off + 32u + 32u * c);
  }
}

// Sum over the wave, valid in lane 63.
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
  v += dpp_mov<0xB1>(v);  // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);  // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v); // row_half_mirror
  v += dpp_mov<0x140>(v); // row_mirror: every lane holds its 16-lane row sum
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142,
                                                             0xA, 0xF, false)); // row_bcast15
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143,
                                                             0xC, 0xF, false)); // row_bcast31
  return v;
}

template <int RB>
__device__ __forceinline__ void q4k_cols_compute(const Q4kColsBuf<RB> &B, const float4 (&xl)[8],
                                                 const float4 (&xh)[8], float s0, float s1,
                                                 uint32_t c, float (&v)[RB]) {
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const uint4 hd = B.h[r];
    uint32_t scp, mp;
    q4k_scale_min_pair(hd.y, hd.z, hd.w, c, &scp, &mp);
    float alo = 0.0f, ahi = 0.0f;
    q4k_dword(B.a[r].x, xl[0], xh[0], alo, ahi);
    q4k_dword(B.a[r].y, xl[1], xh[1], alo, ahi);
    q4k_dword(B.a[r].z, xl[2], xh[2], alo, ahi);
    q4k_dword(B.a[r].w, xl[3], xh[3], alo, ahi);
    q4k_dword(B.b[r].x, xl[4], xh[4], alo, ahi);
    q4k_dword(B.b[r].y, xl[5], xh[5], alo, ahi);
    q4k_dword(B.b[r].z, xl[6], xh[6], alo, ahi);
    q4k_dword(B.b[r].w, xl[7], xh[7], alo, ahi);
    const float dot = __builtin_fmaf((float)(scp & 0xFFu), alo, (float)(scp >> 8) * ahi);
    const float mins = __builtin_fmaf((float)(mp & 0xFFu), s0, (float)(mp >> 8) * s1);
    v[r] = __builtin_fmaf(f16_to_f32(hd.x & 0xFFFFu), dot, -f16_to_f32(hd.x >> 16) * mins);
  }
}

// Wave sums of the batch's rows -> y (through LDS when NW > 1).
template <int RB, int NW>
__device__ __forceinline__ void q4k_cols_finish(float (&v)[RB], float *red, uint32_t parity,
                                                uint32_t batch, uint32_t n_rows, uint32_t tid,
                                                uint32_t wave, float *__restrict__ y) {
#pragma unroll
  for (int r = 0; r < RB; ++r) v[r] = wave_sum_to_lane63(v[r]);
  const uint32_t lane = tid & 63u;
  if constexpr (NW == 1) {
    if (lane == 63u) {
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const uint32_t row = batch * RB + (uint32_t)r;
        if (row < n_rows) y[row] = v[r];
      }
    }
  } else {
    float *buf = red + parity * (RB * NW);
    if (lane == 63u) {
#pragma unroll
      for (int r = 0; r < RB; ++r) buf[r * NW + wave] = v[r];
    }
    __syncthreads();
    if (tid < (uint32_t)RB) {
      float s = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) s += buf[tid * NW + w];
      const uint32_t row = batch * RB + tid;
      if (row < n_rows) y[row] = s;
    }
  }
}

template <int RB, int NW, bool kNT, bool kXFirst>
__device__ __forceinline__ void q4k_matvec_cols(const uint8_t *__restrict__ q,
                                                const float *__restrict__ x,
                                                float *__restrict__ y, uint32_t n_rows,
                                                uint32_t nsb, float *red) {
  const uint32_t tid = threadIdx.x;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t G = gridDim.x;
  const uint32_t n_batches = (n_rows + RB - 1) / RB;
  uint32_t b = blockIdx.x;
  if (nsb == 0) { // empty rows: the reference returns +0.0 (AT-1323)
    for (uint32_t r = b * (NW * 64u) + tid; r < n_rows; r += G * (NW * 64u)) y[r] = 0.0f;
    return;
  }
  if (b >= n_batches) return; // whole workgroup
  const uint32_t row_bytes = nsb * (uint32_t)kQ4kSbBytes;
  const __amdgpu_buffer_rsrc_t qr = make_rsrc(q, n_rows * row_bytes);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, nsb * 1024u);
  const uint32_t nq = nsb * 4u;
  const uint32_t c = tid & 3u;
  // header offset of this lane's superblock within a row (idle lanes: out of range)
  const uint32_t lane_off = tid < nq ? (tid >> 2) * (uint32_t)kQ4kSbBytes : kQ4kColsOob;
  const uint32_t x_off = tid < nq ? tid * 256u : nsb * 1024u; // idle lanes read zeros

  float4 xl[8], xh[8];
  Q4kColsBuf<RB> B0, B1;
  if constexpr (kXFirst) {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      xl[t] = buf_loadf4(xr, x_off + 16u * (uint32_t)t);
      xh[t] = buf_loadf4(xr, x_off + 128u + 16u * (uint32_t)t);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  // B0 strictly before B1: the loop waits on B0 with B1 still in flight
  q4k_cols_load<RB, kNT>(B0, qr, b, n_rows, row_bytes, lane_off, c);
  __builtin_amdgcn_sched_barrier(0);
  q4k_cols_load<RB, kNT>(B1, qr, b + G, n_rows, row_bytes, lane_off, c);
  if constexpr (!kXFirst) {
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      xl[t] = buf_loadf4(xr, x_off + 16u * (uint32_t)t);
      xh[t] = buf_loadf4(xr, x_off + 128u + 16u * (uint32_t)t);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    s0 += (xl[t].x + xl[t].y) + (xl[t].z + xl[t].w);
    s1 += (xh[t].x + xh[t].y) + (xh[t].z + xh[t].w);
    xl[t] = make_float4(xl[t].x * 16777216.0f, xl[t].y * 16777216.0f, xl[t].z * 16777216.0f,
                        xl[t].w * 16777216.0f);
    xh[t] = make_float4(xh[t].x * 1048576.0f, xh[t].y * 1048576.0f, xh[t].z * 1048576.0f,
                        xh[t].w * 1048576.0f);
  }

  // Batches of this workgroup, padded to an even count: a padding batch has
  // only out-of-range rows (zero loads, nothing stored).
  const uint32_t n_mine = (n_batches - b + G - 1u) / G;
  const uint32_t n_pad = (n_mine + 1u) & ~1u;
  float v[RB];
  uint32_t i = 0;
  do { // n_pad >= 2: this workgroup has at least one batch
    q4k_cols_compute<RB>(B0, xl, xh, s0, s1, c, v);
    q4k_cols_load<RB, kNT>(B0, qr, b + 2u * G, n_rows, row_bytes, lane_off, c);
    q4k_cols_finish<RB, NW>(v, red, 0u, b, n_rows, tid, wave, y);
    q4k_cols_compute<RB>(B1, xl, xh, s0, s1, c, v);
    q4k_cols_load<RB, kNT>(B1, qr, b + 3u * G, n_rows, row_bytes, lane_off, c);
    q4k_cols_finish<RB, NW>(v, red, 1u, b + G, n_rows, tid, wave, y);
    b += 2u * G;
    i += 2u;
  } while (i < n_pad);
}

// ---------------------------------------------------------------------------
// One workgroup for up to RB long rows (the single row of config 2): all
// NW*64 lanes work on the same rows, four lanes per superblock (lane t:
// superblock t / 4, quarter t % 4, as the column kernel), with x staged once
// in LDS by the coalesced loads of the persistent kernel (the same layout,
// pre-scaled, with sub-block sums) instead of 64 contiguous floats per lane.
// All rows are requested at once; each lane's partial sums are reduced with
// DPP and the NW wave sums are added in wave order in LDS: no atomics and
// no ordering between workgroups.
// ---------------------------------------------------------------------------
template <int NW, int XP, int RB>
__device__ __forceinline__ void q4k_matvec_wg(const uint8_t *__restrict__ q,
                                              const float *__restrict__ x,
                                              float *__restrict__ y, uint32_t n_rows,
                                              uint32_t nsb, float *lds) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t row_bytes = nsb * (uint32_t)kQ4kSbBytes;
  const __amdgpu_buffer_rsrc_t qr = make_rsrc(q, n_rows * row_bytes);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, nsb * 1024u);
  float *xs = lds, *ss = lds + nsb * kQ4kFlatSbFloats, *red = ss + nsb * 8u;
  float4 xv[8 * XP];
  q4k_flat_load_xc<NW * 64, XP>(xr, tid, xv);
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t sbi = tid >> 2, c = tid & 3u;
  const uint32_t lane_off = sbi < nsb ? sbi * (uint32_t)kQ4kSbBytes : kQ4kColsOob;
  Q4kColsBuf<RB> B;
  q4k_cols_load<RB, false>(B, qr, 0u, n_rows, row_bytes, lane_off, c);
  __builtin_amdgcn_sched_barrier(0);
  q4k_flat_stage_xc<NW * 64, XP>(xs, ss, tid, nsb, xv);
  __syncthreads();
  // idle lanes (superblock past the row) read superblock 0's x; their weights are zero
  const uint32_t sbx = sbi < nsb ? sbi : 0u;
  const float *xb = xs + sbx * kQ4kFlatSbFloats + 4u * c;
  float4 xl[8], xh[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    xl[t] = *reinterpret_cast<const float4 *>(xb + (uint32_t)t * 16u);
    xh[t] = *reinterpret_cast<const float4 *>(xb + 128u + (uint32_t)t * 16u);
  }
  const float2 sub = *reinterpret_cast<const float2 *>(ss + sbx * 8u + 2u * c);
  float v[RB];
  q4k_cols_compute<RB>(B, xl, xh, sub.x, sub.y, c, v);
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    v[r] = wave_sum_to_lane63(v[r]);
    if (lane == 63u) red[r * NW + wave] = v[r];
  }
  __syncthreads();
  if (tid < (uint32_t)RB && tid < n_rows) {
    float sum = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) sum += red[tid * NW + (uint32_t)w];
    y[tid] = sum;
  }
}

#define AXH_Q4K_MATVEC_WG(NW, XP, RB)                                                            \
  extern "C" __global__ void __launch_bounds__(NW * 64)                                          \
      axh_q4k_matvec_wg_w##NW##_x##XP##_r##RB(const uint8_t *__restrict__ q,                     \
                                              const float *__restrict__ x,                       \
                                              float *__restrict__ y, AXH_ROWS_ARGS) { AXH_ROWS_UNPACK; \
    extern __shared__ float axh_wg_dyn[];                                                        \
    q4k_matvec_wg<NW, XP, RB>(q, x, y, a.n_rows, a.units_per_row, axh_wg_dyn);                   \
  }

AXH_Q4K_MATVEC_WG(8, 2, 1)
AXH_Q4K_MATVEC_WG(8, 2, 2)
AXH_Q4K_MATVEC_WG(8, 2, 4)

// ---------------------------------------------------------------------------
// Split-K for few long rows (fewer than 32 rows of 64..256 superblocks that
// the one-workgroup kernel does not take):
// workgroup g (one wave) takes superblocks [g*SPW, g*SPW + SPW) of every row,
// four lanes per superblock (as the column kernel), with its x slice in
// VGPRs.  Lane 63 stores the per-row partial sums to
// ws[kSkPartials + g*32 + row] and counts the workgroup with a device-scope
// release increment of ws[0]; the workgroup that sees G - 1 (all others
// done) takes an acquire fence, adds the partials in workgroup order
// (deterministic), writes y and resets the counter to zero for the next
// call.  The host allocates the workspace once per stream (counter zeroed
// then); calls on one stream never overlap.  Each release writes back the
// L2 of its XCD, so the split is kept to at most 16 workgroups (measured:
// 8 workgroups 7.2 us, 32 workgroups 14 us for 1 x 32768).
// ---------------------------------------------------------------------------
constexpr uint32_t kSkPartials = 64; // floats before the partials (the counter is word 0)
constexpr uint32_t kSkMaxRows = 32;

template <int SPW>
__device__ __forceinline__ void q4k_matvec_sk(const uint8_t *__restrict__ q,
                                              const float *__restrict__ x,
                                              float *__restrict__ y, float *ws, uint32_t n_rows,
                                              uint32_t nsb) {
  constexpr int RB = 4;
  const uint32_t tid = threadIdx.x, g = blockIdx.x, G = gridDim.x;
  const uint32_t row_bytes = nsb * (uint32_t)kQ4kSbBytes;
  const __amdgpu_buffer_rsrc_t qr = make_rsrc(q, n_rows * row_bytes);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, nsb * 1024u);
  const uint32_t sb = g * SPW + (tid >> 2), c = tid & 3u;
  const bool live = tid < 4u * SPW && sb < nsb;
  const uint32_t lane_off = live ? sb * (uint32_t)kQ4kSbBytes : kQ4kColsOob;
  const uint32_t x_off = live ? (sb * 4u + c) * 256u : nsb * 1024u; // idle lanes read zeros
  const uint32_t n_batches = (n_rows + RB - 1) / RB;

  float4 xl[8], xh[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    xl[t] = buf_loadf4(xr, x_off + 16u * (uint32_t)t);
    xh[t] = buf_loadf4(xr, x_off + 128u + 16u * (uint32_t)t);
  }
  __builtin_amdgcn_sched_barrier(0);
  Q4kColsBuf<RB> B0, B1;
  q4k_cols_load<RB, false>(B0, qr, 0u, n_rows, row_bytes, lane_off, c);
  __builtin_amdgcn_sched_barrier(0);
  q4k_cols_load<RB, false>(B1, qr, 1u, n_rows, row_bytes, lane_off, c);
  __builtin_amdgcn_sched_barrier(0);
  float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    s0 += (xl[t].x + xl[t].y) + (xl[t].z + xl[t].w);
    s1 += (xh[t].x + xh[t].y) + (xh[t].z + xh[t].w);
    xl[t] = make_float4(xl[t].x * 16777216.0f, xl[t].y * 16777216.0f, xl[t].z * 16777216.0f,
                        xl[t].w * 16777216.0f);
    xh[t] = make_float4(xh[t].x * 1048576.0f, xh[t].y * 1048576.0f, xh[t].z * 1048576.0f,
                        xh[t].w * 1048576.0f);
  }
  float *part = ws + kSkPartials + g * kSkMaxRows;
  const uint32_t n_pad = (n_batches + 1u) & ~1u; // >= 2; padding batches store nothing
  float v[RB];
  uint32_t b = 0;
  do {
    q4k_cols_compute<RB>(B0, xl, xh, s0, s1, c, v);
    q4k_cols_load<RB, false>(B0, qr, b + 2u, n_rows, row_bytes, lane_off, c);
#pragma unroll
    for (int r = 0; r < RB; ++r) v[r] = wave_sum_to_lane63(v[r]);
    if (tid == 63u) {
#pragma unroll
      for (int r = 0; r < RB; ++r)
        if (b * RB + r < n_rows) part[b * RB + r] = v[r];
    }
    q4k_cols_compute<RB>(B1, xl, xh, s0, s1, c, v);
    q4k_cols_load<RB, false>(B1, qr, b + 3u, n_rows, row_bytes, lane_off, c);
#pragma unroll
    for (int r = 0; r < RB; ++r) v[r] = wave_sum_to_lane63(v[r]);
    if (tid == 63u) {
#pragma unroll
      for (int r = 0; r < RB; ++r)
        if ((b + 1u) * RB + r < n_rows) part[(b + 1u) * RB + r] = v[r];
    }
    b += 2u;
  } while (b < n_pad);

  // Lane 63 stored the partials: its release increment orders them before the count.
  uint32_t last = 0;
  if (tid == 63u) {
    const uint32_t prev = __hip_atomic_fetch_add(reinterpret_cast<uint32_t *>(ws), 1u,
                                                 __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    last = prev == G - 1u ? 1u : 0u;
  }
  last = __builtin_amdgcn_readlane(last, 63);
  if (!last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  if (tid < n_rows) {
    float s = 0.0f;
    for (uint32_t k = 0; k < G; ++k)
      s += __hip_atomic_load(ws + kSkPartials + k * kSkMaxRows + tid, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    y[tid] = s;
  }
  if (tid == 0u)
    __hip_atomic_store(reinterpret_cast<uint32_t *>(ws), 0u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

#define AXH_Q4K_MATVEC_SK(SPW)                                                                   \
  extern "C" __global__ void __launch_bounds__(64)                                               \
      axh_q4k_matvec_sk_s##SPW(const uint8_t *__restrict__ q, const float *__restrict__ x,      \
                               float *__restrict__ y, float *ws, AXH_ROWS_ARGS) { AXH_ROWS_UNPACK; \
    q4k_matvec_sk<SPW>(q, x, y, ws, a.n_rows, a.units_per_row);                                  \
  }

AXH_Q4K_MATVEC_SK(16)

#define AXH_Q4K_MATVEC_COLS(RB, NW, NT, XF)                                                       \
  extern "C" __global__ void __launch_bounds__(NW * 64)                                          \
      axh_q4k_matvec_cols_r##RB##_w##NW##_n##NT##_x##XF(const uint8_t *__restrict__ q,           \
                                                         const float *__restrict__ x,            \
                                                         float *__restrict__ y, AXH_ROWS_ARGS) { AXH_ROWS_UNPACK; \
    __shared__ float red[2 * RB * NW];                                                           \
    q4k_matvec_cols<RB, NW, NT != 0, XF != 0>(q, x, y, a.n_rows, a.units_per_row, red);         \
  }

AXH_Q4K_MATVEC_COLS(4, 1, 0, 1)
AXH_Q4K_MATVEC_COLS(4, 2, 0, 1)
AXH_Q4K_MATVEC_COLS(4, 3, 0, 1)
AXH_Q4K_MATVEC_COLS(4, 4, 0, 1)
AXH_Q4K_MATVEC_COLS(4, 5, 0, 1)
AXH_Q4K_MATVEC_COLS(4, 6, 0, 1)
AXH_Q4K_MATVEC_COLS(4, 7, 0, 1)
AXH_Q4K_MATVEC_COLS(4, 8, 0, 1)

// Reference-compatible entry point: the contract of
// examples/q4km_dequant_matvec.axc (bindings q=0, x=1, y=2; push constant
// n_superblocks: u32 @0; @workgroup(64,1,1); dispatched as 1x1x1).  One wave
// computes y[0]; workgroups other than 0 return, like the reference's
// `if gid(0) >= 1 { return; }`.
constexpr uint32_t kRefTileSb = 16; // 17 KiB static LDS tile
extern "C" __global__ void __launch_bounds__(64)
    q4km_dequant_matvec(const uint8_t *__restrict__ q, const float *__restrict__ x,
                        float *__restrict__ y, AXH_COUNT_ARGS) { AXH_COUNT_UNPACK;
  __shared__ float lds[kRefTileSb * 256 + kRefTileSb * 16];
  if (blockIdx.x != 0 || blockIdx.y != 0 || blockIdx.z != 0) return;
  if (a.n_units <= kRefTileSb)
    q4k_matvec_body<1, 1, 2, false, false>(q, x, y, 1u, a.n_units, kRefTileSb, 0u, lds);
  else
    q4k_matvec_body<1, 1, 2, false, true>(q, x, y, 1u, a.n_units, kRefTileSb, 0u, lds);
}

// ===========================================================================
// Q4_0 matvec
// ===========================================================================
// Lane mapping: each lane owns a pair of consecutive blocks (36 bytes); one
// wave iteration covers 64 pairs = 128 blocks = 4096 weights of a row.  With
// an even number of blocks per row every pair starts 4-byte aligned and is
// read as nine dwords; otherwise the lane reads 2-byte halves.
//
// LDS tile for `tile` blocks (pair slot s = block/2 within the tile):
//   xs[s*64 + ((f ^ (s & 15)) * 4) + e] = x[(2s + f/8)*32 + (f%8)*4 + e],
//     f = float4 index 0..15 within the pair (block A lo, A hi, B lo, B hi)
//   bs[block] = sum of that block's 32 x values
// Per block: sum_k (q_k - 8) * d * x_k = d * (sum_k q_k x_k - 8 * bs).

__device__ __forceinline__ void q4_0_stage_tile(const float *__restrict__ x, float *xs, float *bs,
                                                uint32_t b0, uint32_t n_b, uint32_t tid,
                                                uint32_t nthreads) {
  for (uint32_t bi = tid; bi < n_b; bi += nthreads) {
    const float4 *src = reinterpret_cast<const float4 *>(x + (size_t)(b0 + bi) * 32u);
    const uint32_t s = bi >> 1, fb = (bi & 1u) * 8u;
    float sum = 0.0f;
#pragma unroll
    for (int f = 0; f < 8; ++f) {
      const float4 v = src[f];
      *reinterpret_cast<float4 *>(xs + s * 64u + ((((uint32_t)f + fb) ^ (s & 15u)) * 4u)) = v;
      sum += (v.x + v.y) + (v.z + v.w);
    }
    bs[bi] = sum;
  }
}

// One block: d and 16 qs bytes (as 4 dwords) against its 8 staged float4 of x.
__device__ __forceinline__ float q4_0_block(uint32_t dbits, const uint32_t qs[4], const float *xp,
                                            uint32_t s, uint32_t fb, float bsum) {
  float alo = 0.0f, ahi = 0.0f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const float4 xl = *reinterpret_cast<const float4 *>(xp + ((((uint32_t)t + fb) ^ (s & 15u)) * 4u));
    const float4 xh =
        *reinterpret_cast<const float4 *>(xp + ((((uint32_t)t + 4u + fb) ^ (s & 15u)) * 4u));
    q4k_dword(qs[t], xl, xh, alo, ahi);
  }
  const float dot = __builtin_fmaf(16777216.0f, alo, 1048576.0f * ahi);
  return f16_to_f32(dbits) * __builtin_fmaf(-8.0f, bsum, dot);
}

template <int RPW, int NW>
__device__ __forceinline__ void q4_0_matvec_body(const uint8_t *__restrict__ q,
                                                 const float *__restrict__ x,
                                                 float *__restrict__ y, uint32_t n_rows,
                                                 uint32_t nb, uint32_t tile_b, uint32_t block,
                                                 float *lds) {
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u, wave = tid >> 6;
  const uint32_t row0 = (block * NW + wave) * RPW;
  const size_t row_bytes = (size_t)nb * kQ4_0BlockBytes;
  const bool aligned = (nb & 1u) == 0u;
  const uint32_t n_pairs = (nb + 1u) >> 1;
  const uint32_t n_it = (n_pairs + 63u) >> 6;
  const uint32_t it_per_tile = tile_b >> 7; // 128 blocks per iteration
  float *xs = lds;
  float *bs = lds + (tile_b >> 1) * 64u;

  float acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;

  uint32_t tile = 0xFFFFFFFFu;
  for (uint32_t it = 0; it < n_it; ++it) {
    const uint32_t t_it = it / it_per_tile;
    if (t_it != tile) {
      if (tile != 0xFFFFFFFFu) __syncthreads();
      tile = t_it;
      const uint32_t b0 = t_it * tile_b;
      q4_0_stage_tile(x, xs, bs, b0, min(tile_b, nb - b0), tid, NW * 64u);
      __syncthreads();
    }
    const uint32_t pr = it * 64u + lane;
    if (pr < n_pairs) {
      const bool has_b = 2u * pr + 1u < nb;
      const uint32_t s = pr - tile * (tile_b >> 1);
      const float *xp = xs + s * 64u;
      const float2 bsum = *reinterpret_cast<const float2 *>(bs + 2u * s);
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        const uint32_t row = min(row0 + r, n_rows - 1u);
        const uint8_t *pp = q + (size_t)row * row_bytes + (size_t)pr * 36u;
        uint32_t D[9];
        if (aligned) {
          const uint32_t *p32 = reinterpret_cast<const uint32_t *>(pp);
#pragma unroll
          for (int i = 0; i < 9; ++i) D[i] = p32[i];
        } else {
          // halves 0..8 are block A, 9..17 block B (only read when it exists)
          const uint16_t *p16 = reinterpret_cast<const uint16_t *>(pp);
#pragma unroll
          for (int i = 0; i < 4; ++i) D[i] = (uint32_t)p16[2 * i] | ((uint32_t)p16[2 * i + 1] << 16);
          D[4] = (uint32_t)p16[8];
          D[5] = D[6] = D[7] = D[8] = 0u;
          if (has_b) {
            D[4] |= (uint32_t)p16[9] << 16;
#pragma unroll
            for (int i = 5; i < 9; ++i)
              D[i] = (uint32_t)p16[2 * i] | ((uint32_t)p16[2 * i + 1] << 16);
          }
        }
        const uint32_t qa[4] = {__builtin_amdgcn_alignbit(D[1], D[0], 16),
                                __builtin_amdgcn_alignbit(D[2], D[1], 16),
                                __builtin_amdgcn_alignbit(D[3], D[2], 16),
                                __builtin_amdgcn_alignbit(D[4], D[3], 16)};
        float v = q4_0_block(D[0] & 0xFFFFu, qa, xp, s, 0u, bsum.x);
        if (has_b) {
          const uint32_t qb[4] = {D[5], D[6], D[7], D[8]};
          v += q4_0_block(D[4] >> 16, qb, xp, s, 8u, bsum.y);
        }
        acc[r] += v;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const float sres = wave_sum(acc[r]);
    if (lane == 0 && row0 + r < n_rows) y[row0 + r] = sres;
  }
}

// ---------------------------------------------------------------------------
// Q4_0 rows of at most 128 blocks (an even count, so every block pair starts
// 4-byte aligned): lane l owns the block pair [2l, 2l + 2) of every row, with
// its 64 x values in VGPRs (no LDS staging, no barrier).  A wave takes RB
// rows at a time (batches strided over the grid), with the next batch's nine
// dwords per row in flight, and reduces each row with DPP.  Rows past the
// matrix and idle lanes read zeros through the buffer range check.
// ---------------------------------------------------------------------------
template <int RB>
struct Q4_0ColsBuf {
  uint4 a[RB], b[RB];
  uint32_t c[RB];
};

template <int RB>
__device__ __forceinline__ void q4_0_cols_load(Q4_0ColsBuf<RB> &B, __amdgpu_buffer_rsrc_t qr,
                                               uint32_t batch, uint32_t n_rows,
                                               uint32_t row_bytes, uint32_t lane_off) {
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const uint32_t row = batch * RB + (uint32_t)r;
    const uint32_t off =
        (row < n_rows && lane_off != kQ4kColsOob) ? row * row_bytes + lane_off : kQ4kColsOob;
    B.a[r] = buf_load16<false>(qr, off);
    B.b[r] = buf_load16<false>(qr, off + 16u);
    B.c[r] = __builtin_amdgcn_raw_buffer_load_b32(qr, (int)(off + 32u), 0, 0);
  }
}

template <int RB>
__device__ __forceinline__ void q4_0_cols_compute(const Q4_0ColsBuf<RB> &B,
                                                  const float4 (&x)[2][8], float sa, float sb,
                                                  float (&v)[RB]) {
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const uint32_t D[9] = {B.a[r].x, B.a[r].y, B.a[r].z, B.a[r].w, B.b[r].x,
                           B.b[r].y, B.b[r].z, B.b[r].w, B.c[r]};
    // block A: d = bytes 0-1, qs = bytes 2-17; block B: d = bytes 18-19, qs = bytes 20-35
    const uint32_t qa[4] = {__builtin_amdgcn_alignbit(D[1], D[0], 16),
                            __builtin_amdgcn_alignbit(D[2], D[1], 16),
                            __builtin_amdgcn_alignbit(D[3], D[2], 16),
                            __builtin_amdgcn_alignbit(D[4], D[3], 16)};
    float alo = 0.0f, ahi = 0.0f, blo = 0.0f, bhi = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      q4k_dword(qa[t], x[0][t], x[0][4 + t], alo, ahi);
      q4k_dword(D[5 + t], x[1][t], x[1][4 + t], blo, bhi);
    }
    v[r] = __builtin_fmaf(f16_to_f32(D[0] & 0xFFFFu), __builtin_fmaf(-8.0f, sa, alo + ahi),
                          f16_to_f32(D[4] >> 16) * __builtin_fmaf(-8.0f, sb, blo + bhi));
  }
}

template <int RB>
__device__ __forceinline__ void q4_0_matvec_cols(const uint8_t *__restrict__ q,
                                                 const float *__restrict__ x,
                                                 float *__restrict__ y, uint32_t n_rows,
                                                 uint32_t nb) {
  const uint32_t lane = threadIdx.x, G = gridDim.x;
  const uint32_t n_batches = (n_rows + RB - 1) / RB;
  uint32_t b = blockIdx.x;
  if (b >= n_batches) return;
  // The host guarantees n_rows * row_bytes < 2^32 - 256 for this kernel.
  const uint32_t row_bytes = nb * (uint32_t)kQ4_0BlockBytes;
  const __amdgpu_buffer_rsrc_t qr = make_rsrc(q, n_rows * row_bytes);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, nb * 128u);
  const bool live = 2u * lane < nb;
  const uint32_t lane_off = live ? lane * 36u : kQ4kColsOob;
  const uint32_t x_off = live ? lane * 256u : nb * 128u; // idle lanes read zeros

  float4 xv[2][8];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int t = 0; t < 8; ++t) xv[h][t] = buf_loadf4(xr, x_off + 128u * h + 16u * (uint32_t)t);
  __builtin_amdgcn_sched_barrier(0);
  Q4_0ColsBuf<RB> B0, B1;
  q4_0_cols_load<RB>(B0, qr, b, n_rows, row_bytes, lane_off);
  __builtin_amdgcn_sched_barrier(0);
  q4_0_cols_load<RB>(B1, qr, b + G, n_rows, row_bytes, lane_off);
  __builtin_amdgcn_sched_barrier(0);
  // low nibbles (elements 0..15 of a block) against x * 2^24, high against x * 2^20
  float sa = 0.0f, sb = 0.0f;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const float f = t < 4 ? 16777216.0f : 1048576.0f;
    sa += (xv[0][t].x + xv[0][t].y) + (xv[0][t].z + xv[0][t].w);
    sb += (xv[1][t].x + xv[1][t].y) + (xv[1][t].z + xv[1][t].w);
#pragma unroll
    for (int h = 0; h < 2; ++h)
      xv[h][t] = make_float4(xv[h][t].x * f, xv[h][t].y * f, xv[h][t].z * f, xv[h][t].w * f);
  }
  const uint32_t n_mine = (n_batches - b + G - 1u) / G;
  const uint32_t n_pad = (n_mine + 1u) & ~1u;
  float v[RB];
  uint32_t i = 0;
  do { // n_pad >= 2: this workgroup has at least one batch
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      Q4_0ColsBuf<RB> &B = half ? B1 : B0;
      q4_0_cols_compute<RB>(B, xv, sa, sb, v);
      const uint32_t cur = b + (uint32_t)half * G;
      q4_0_cols_load<RB>(B, qr, b + (2u + (uint32_t)half) * G, n_rows, row_bytes, lane_off);
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const float sres = wave_sum_to_lane63(v[r]);
        const uint32_t row = cur * RB + (uint32_t)r;
        if (lane == 63u && row < n_rows) y[row] = sres;
      }
    }
    b += 2u * G;
    i += 2u;
  } while (i < n_pad);
}

#define AXH_Q4_0_MATVEC_COLS(RB)                                                                 \
  extern "C" __global__ void __launch_bounds__(64)                                               \
      axh_q4_0_matvec_cols_r##RB(const uint8_t *__restrict__ q, const float *__restrict__ x,     \
                                 float *__restrict__ y, AXH_ROWS_ARGS) { AXH_ROWS_UNPACK; \
    q4_0_matvec_cols<RB>(q, x, y, a.n_rows, a.units_per_row);                                    \
  }

AXH_Q4_0_MATVEC_COLS(1)

#define AXH_Q4_0_MATVEC(RPW, NW)                                                                 \
  extern "C" __global__ void __launch_bounds__(NW * 64)                                          \
      axh_q4_0_matvec_r##RPW##_w##NW(const uint8_t *__restrict__ q,                              \
                                     const float *__restrict__ x, float *__restrict__ y,         \
                                     AXH_ROWS_ARGS) { AXH_ROWS_UNPACK;                   \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4_0_matvec_body<RPW, NW>(q, x, y, a.n_rows, a.units_per_row, a.tile_units, blockIdx.x,      \
                              axh_lds_dyn);                                                      \
  }

AXH_Q4_0_MATVEC(1, 1)
AXH_Q4_0_MATVEC(1, 4)
AXH_Q4_0_MATVEC(2, 4)
AXH_Q4_0_MATVEC(4, 4)

// Q4_0 through the Q4_K persistent and one-pass kernels (kQ40: octets of 8
// blocks in place of superblocks, 64 blocks per iteration).
// axh_q4_0_matvec_flat_r{RPW}_w{NW}_p{PF}: persistent, grid-strided pairs of
// RPW-row bundles; PF 1 stages x chunk by chunk with early refill, PF 2 stages
// it whole first (XP * NW * 64 blocks at most).
#define AXH_Q4_0_MATVEC_FLAT(RPW, NW, PF, XP)                                                    \
  extern "C" __global__ void __launch_bounds__(NW * 64)                                          \
      axh_q4_0_matvec_flat_r##RPW##_w##NW##_p##PF##_x##XP(const uint8_t *__restrict__ q,         \
                                                          const float *__restrict__ x,           \
                                                          float *__restrict__ y,                 \
                                                          AXH_ROWS_ARGS) { AXH_ROWS_UNPACK;      \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4k_matvec_flat<RPW, NW, PF, false, XP, false, false, true>(q, q, x, y, a.n_rows,            \
                                                                a.units_per_row, axh_lds_dyn);   \
  }
AXH_Q4_0_MATVEC_FLAT(1, 4, 1, 1)
AXH_Q4_0_MATVEC_FLAT(1, 8, 1, 1)
AXH_Q4_0_MATVEC_FLAT(2, 4, 1, 1)
AXH_Q4_0_MATVEC_FLAT(2, 8, 1, 1)
AXH_Q4_0_MATVEC_FLAT(1, 8, 2, 1)
AXH_Q4_0_MATVEC_FLAT(2, 4, 2, 2)
AXH_Q4_0_MATVEC_FLAT(1, 16, 2, 1)

// axh_q4_0_matvec_one{,x,p}_i{NIT}: one workgroup of 8 waves per 16 rows of
// 64 * (NIT - 1) < nb <= 64 * NIT blocks (x chunk by chunk, x whole, x two
// chunks ahead).
#define AXH_Q4_0_MATVEC_ONE(NIT)                                                                 \
  extern "C" __global__ void __launch_bounds__(512)                                              \
      axh_q4_0_matvec_one_i##NIT(const uint8_t *__restrict__ q, const float *__restrict__ x,     \
                                 float *__restrict__ y, AXH_ROWS_ARGS) { AXH_ROWS_UNPACK;        \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4k_matvec_one<NIT, false, false, false, 1, true>(q, q, x, y, a.n_rows, a.units_per_row,     \
                                                      axh_lds_dyn);                              \
  }                                                                                              \
  extern "C" __global__ void __launch_bounds__(512)                                              \
      axh_q4_0_matvec_onex_i##NIT(const uint8_t *__restrict__ q, const float *__restrict__ x,    \
                                  float *__restrict__ y, AXH_ROWS_ARGS) { AXH_ROWS_UNPACK;       \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4k_matvec_one<NIT, false, false, true, 1, true>(q, q, x, y, a.n_rows, a.units_per_row,      \
                                                     axh_lds_dyn);                               \
  }
#define AXH_Q4_0_MATVEC_ONEP(NIT)                                                                \
  extern "C" __global__ void __launch_bounds__(512)                                              \
      axh_q4_0_matvec_onep_i##NIT(const uint8_t *__restrict__ q, const float *__restrict__ x,    \
                                  float *__restrict__ y, AXH_ROWS_ARGS) { AXH_ROWS_UNPACK;       \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4k_matvec_one<NIT, false, false, false, 2, true>(q, q, x, y, a.n_rows, a.units_per_row,     \
                                                      axh_lds_dyn);                              \
  }
AXH_Q4_0_MATVEC_ONE(1)
AXH_Q4_0_MATVEC_ONE(2)
AXH_Q4_0_MATVEC_ONE(3)
AXH_Q4_0_MATVEC_ONE(4)
AXH_Q4_0_MATVEC_ONE(5)
AXH_Q4_0_MATVEC_ONE(6)
AXH_Q4_0_MATVEC_ONE(7)
AXH_Q4_0_MATVEC_ONE(8)
AXH_Q4_0_MATVEC_ONE(9)
AXH_Q4_0_MATVEC_ONE(10)
AXH_Q4_0_MATVEC_ONE(11)
AXH_Q4_0_MATVEC_ONE(12)
AXH_Q4_0_MATVEC_ONE(13)
AXH_Q4_0_MATVEC_ONE(14)
AXH_Q4_0_MATVEC_ONE(15)
AXH_Q4_0_MATVEC_ONE(16)
AXH_Q4_0_MATVEC_ONEP(3)
AXH_Q4_0_MATVEC_ONEP(4)
AXH_Q4_0_MATVEC_ONEP(5)
AXH_Q4_0_MATVEC_ONEP(6)
AXH_Q4_0_MATVEC_ONEP(7)
AXH_Q4_0_MATVEC_ONEP(8)
AXH_Q4_0_MATVEC_ONEP(9)
AXH_Q4_0_MATVEC_ONEP(10)
AXH_Q4_0_MATVEC_ONEP(11)
AXH_Q4_0_MATVEC_ONEP(12)
AXH_Q4_0_MATVEC_ONEP(13)
AXH_Q4_0_MATVEC_ONEP(14)
AXH_Q4_0_MATVEC_ONEP(15)
AXH_Q4_0_MATVEC_ONEP(16)

// Reference-compatible entry point for examples/q4_0_dequant_matvec.axc
// (bindings q=0, x=1, y=2; push constant n_blocks: u32 @0; 1x1x1 of 64).
constexpr uint32_t kRefTileB = 128; // 17 KiB static LDS tile
extern "C" __global__ void __launch_bounds__(64)
    q4_0_dequant_matvec(const uint8_t *__restrict__ q, const float *__restrict__ x,
                        float *__restrict__ y, AXH_COUNT_ARGS) { AXH_COUNT_UNPACK;
  __shared__ float lds[(kRefTileB / 2) * 64 + kRefTileB];
  if (blockIdx.x != 0 || blockIdx.y != 0 || blockIdx.z != 0) return;
  if (a.n_units == 0) {
    if (threadIdx.x == 0) y[0] = 0.0f;
    return;
  }
  q4_0_matvec_body<1, 1>(q, x, y, 1u, a.n_units, kRefTileB, 0u, lds);
}

// ===========================================================================
// Decode-only kernels (bit-exact checks of the dequantised weights)
// ===========================================================================
// Q5_K: one thread per (superblock, 16-byte qs slice), as Q4_K plus the
// fifth bit from qh: fma(d*sc, q, -(dmin*m)) with d*sc, dmin*m and (d*sc)*q
// exact in f32 (q <= 31), so the one rounding is the subtraction's.
extern "C" __global__ void __launch_bounds__(256)
    axh_q5k_dequant(const uint8_t *__restrict__ q, float *__restrict__ w, AXH_COUNT_ARGS) { AXH_COUNT_UNPACK;
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  const uint32_t sb = gid >> 3, k = gid & 7u, c = k >> 1, h = k & 1u;
  if (sb >= a.n_units) return;
  const uint8_t *b = q + (size_t)sb * kQ5kSbBytes;
  const uint4 hd = *reinterpret_cast<const uint4 *>(b);
  const uint4 qv = *reinterpret_cast<const uint4 *>(b + 48u + 16u * k);
  const uint4 hv = *reinterpret_cast<const uint4 *>(b + 16u + 16u * h);
  uint32_t scp, mp;
  q4k_scale_min_pair(hd.y, hd.z, hd.w, c, &scp, &mp);
  const float d = f16_to_f32(hd.x & 0xFFFFu), dmin = f16_to_f32(hd.x >> 16);
  const float d1 = d * (float)(scp & 0xFFu), m1f = dmin * (float)(mp & 0xFFu);
  const float d2 = d * (float)(scp >> 8), m2f = dmin * (float)(mp >> 8);
  float *wl = w + (size_t)sb * kQ4kSbElems + 64u * c + 16u * h;
  float *wh = wl + 32;
  const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w};
  const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    float lo[4], hi[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t byte = (qw[t] >> (8 * e)) & 0xFFu, bits = (hw[t] >> (8 * e + 2 * c)) & 3u;
      lo[e] = __builtin_fmaf(d1, (float)((byte & 15u) + 16u * (bits & 1u)), -m1f);
      hi[e] = __builtin_fmaf(d2, (float)((byte >> 4) + 16u * (bits >> 1)), -m2f);
    }
    *reinterpret_cast<float4 *>(wl + 4 * t) = make_float4(lo[0], lo[1], lo[2], lo[3]);
    *reinterpret_cast<float4 *>(wh + 4 * t) = make_float4(hi[0], hi[1], hi[2], hi[3]);
  }
}

// Q6_K: one thread per (superblock, half n, part p): 32 weights
// d * sc * (q - 32), exact in f32.  Byte reads (superblocks are 2-byte aligned).
extern "C" __global__ void __launch_bounds__(256)
    axh_q6k_dequant(const uint8_t *__restrict__ q, float *__restrict__ w, AXH_COUNT_ARGS) { AXH_COUNT_UNPACK;
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  const uint32_t sb = gid >> 3, n = (gid >> 2) & 1u, p = gid & 3u;
  if (sb >= a.n_units) return;
  const uint8_t *b = q + (size_t)sb * kQ6kSbBytes;
  const float d = f16_to_f32((uint32_t)b[208] | ((uint32_t)b[209] << 8));
  const float s0 = d * (float)(int8_t)b[192u + 8u * n + 2u * p];
  const float s1 = d * (float)(int8_t)b[192u + 8u * n + 2u * p + 1u];
  const uint8_t *ql = b + 64u * n + 32u * (p & 1u), *qh = b + 128u + 32u * n;
  float *o = w + (size_t)sb * kQ4kSbElems + 128u * n + 32u * p;
  for (uint32_t l = 0; l < 32; ++l) {
    const uint32_t v = ((ql[l] >> (4u * (p >> 1))) & 15u) | (((qh[l] >> (2u * p)) & 3u) << 4);
    o[l] = (l < 16 ? s0 : s1) * (float)((int)v - 32);
  }
}

// Q4_K: one thread per (superblock, 16-byte qs slice).  Each value is
// fma(d*sc, nibble, -(dmin*m)): d*sc, dmin*m and (d*sc)*nibble are exact in
// f32, so the single rounding equals the reference's d1*lo - m1f.
extern "C" __global__ void __launch_bounds__(256)
    axh_q4k_dequant(const uint8_t *__restrict__ q, float *__restrict__ w, AXH_COUNT_ARGS) { AXH_COUNT_UNPACK;
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  const uint32_t sb = gid >> 3, k = gid & 7u, c = k >> 1, h = k & 1u;
  if (sb >= a.n_units) return;
  const uint8_t *b = q + (size_t)sb * kQ4kSbBytes;
  const uint4 hd = *reinterpret_cast<const uint4 *>(b);
  const uint4 qv = *reinterpret_cast<const uint4 *>(b + 16u + 16u * k);
  uint32_t scp, mp;
  q4k_scale_min_pair(hd.y, hd.z, hd.w, c, &scp, &mp);
  const float d = f16_to_f32(hd.x & 0xFFFFu), dmin = f16_to_f32(hd.x >> 16);
  const float d1 = d * (float)(scp & 0xFFu), m1f = dmin * (float)(mp & 0xFFu);
  const float d2 = d * (float)(scp >> 8), m2f = dmin * (float)(mp >> 8);
  float *wl = w + (size_t)sb * kQ4kSbElems + 64u * c + 16u * h;
  float *wh = wl + 32;
  const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    float4 lo, hi;
    lo.x = __builtin_fmaf(d1, (float)((qw[t] >> 0) & 15u), -m1f);
    lo.y = __builtin_fmaf(d1, (float)((qw[t] >> 8) & 15u), -m1f);
    lo.z = __builtin_fmaf(d1, (float)((qw[t] >> 16) & 15u), -m1f);
    lo.w = __builtin_fmaf(d1, (float)((qw[t] >> 24) & 15u), -m1f);
    hi.x = __builtin_fmaf(d2, (float)((qw[t] >> 4) & 15u), -m2f);
    hi.y = __builtin_fmaf(d2, (float)((qw[t] >> 12) & 15u), -m2f);
    hi.z = __builtin_fmaf(d2, (float)((qw[t] >> 20) & 15u), -m2f);
    hi.w = __builtin_fmaf(d2, (float)((qw[t] >> 28) & 15u), -m2f);
    *reinterpret_cast<float4 *>(wl + 4 * t) = lo;
    *reinterpret_cast<float4 *>(wh + 4 * t) = hi;
  }
}

// Q4_0: one thread per block; (nibble - 8) * d is exact in f32.
extern "C" __global__ void __launch_bounds__(256)
    axh_q4_0_dequant(const uint8_t *__restrict__ q, float *__restrict__ w, AXH_COUNT_ARGS) { AXH_COUNT_UNPACK;
  const uint32_t blk = blockIdx.x * 256u + threadIdx.x;
  if (blk >= a.n_units) return;
  const uint16_t *p16 = reinterpret_cast<const uint16_t *>(q + (size_t)blk * kQ4_0BlockBytes);
  const float d = f16_to_f32(p16[0]);
  float *wb = w + (size_t)blk * kQ4_0BlockElems;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t two = p16[1 + i]; // qs bytes 2i, 2i+1
    wb[2 * i] = ((float)(two & 15u) - 8.0f) * d;
    wb[2 * i + 1] = ((float)((two >> 8) & 15u) - 8.0f) * d;
    wb[16 + 2 * i] = ((float)((two >> 4) & 15u) - 8.0f) * d;
    wb[16 + 2 * i + 1] = ((float)((two >> 12) & 15u) - 8.0f) * d;
  }
}

// f16 -> f32 widening of raw 16-bit patterns (pins v_cvt_f32_f16 against the
// oracle's exhaustive table).
extern "C" __global__ void __launch_bounds__(256)
    axh_f16_widen(const uint16_t *__restrict__ h, float *__restrict__ f, AXH_COUNT_ARGS) { AXH_COUNT_UNPACK;
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i < a.n_units) f[i] = f16_to_f32(h[i]);
}

// f32 -> f16, round to nearest even, of n values: the activation cast that
// feeds the batched matmul (one pass: 6 bytes of HBM traffic per value).
// Eight values per thread (two 16-byte loads, one 16-byte store); the thread
// holding the last n % 8 values converts them one at a time.  The host
// guarantees 16-byte aligned x and h and n <= 2^32 - 16.
typedef _Float16 axh_half2_t __attribute__((ext_vector_type(2)));
typedef float axh_float2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_rn_f16(float a, float b) {
  return __builtin_bit_cast(uint32_t,
                            __builtin_convertvector((axh_float2_t){a, b}, axh_half2_t));
}

extern "C" __global__ void __launch_bounds__(256)
    axh_f32_to_f16(const float *__restrict__ x, uint16_t *__restrict__ h, AXH_COUNT_ARGS) { AXH_COUNT_UNPACK;
  const uint32_t i = (blockIdx.x * 256u + threadIdx.x) * 8u;
  if (i + 8u <= a.n_units) {
    const float4 lo = *reinterpret_cast<const float4 *>(x + i);
    const float4 hi = *reinterpret_cast<const float4 *>(x + i + 4u);
    *reinterpret_cast<uint4 *>(h + i) =
        make_uint4(pack_rn_f16(lo.x, lo.y), pack_rn_f16(lo.z, lo.w), pack_rn_f16(hi.x, hi.y),
                   pack_rn_f16(hi.z, hi.w));
  } else {
    for (uint32_t k = i; k < a.n_units; ++k)
      h[k] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(x[k]));
  }
}

// Measurement helpers for the floor that one launch per call puts under a
// matvec (no counterpart in the reference).  axh_read_floor streams
// a.n_units 16-byte pieces of q with the matvec's launch shape (one 8-wave
// workgroup per CU, 16-byte buffer loads, four in flight per lane) and
// writes, per wave, the XOR of every dword it read to out[wave], so the loads
// cannot be dropped and each wave ends with one store, as a matvec wave does.
// T threads per workgroup, U loads of 16 bytes in flight per lane, a
// grid-stride walk over the whole buffer (consecutive lanes read consecutive
// pieces); the grid is the caller's.
template <int T, int U>
__device__ __forceinline__ void read_floor(const uint8_t *__restrict__ q, uint32_t *__restrict__ out,
                                           uint32_t n) {
  const uint32_t nt = gridDim.x * (uint32_t)T;
  const uint32_t gtid = blockIdx.x * (uint32_t)T + threadIdx.x;
  const __amdgpu_buffer_rsrc_t r = make_rsrc(q, n * 16u);
  uint32_t acc = 0;
  for (uint32_t i = gtid; i < n; i += (uint32_t)U * nt) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = buf_load16<false>(r, (i + (uint32_t)u * nt) * 16u);
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (int off = 32; off >= 1; off >>= 1) // XOR across the wave
    acc ^= (uint32_t)__shfl_xor((int)acc, off, 64);
  if ((threadIdx.x & 63u) == 0u) out[gtid >> 6] = acc;
}

extern "C" __global__ void __launch_bounds__(512) axh_read_floor(const uint8_t *__restrict__ q,
                                                                 uint32_t *__restrict__ out,
                                                                 AXH_COUNT_ARGS) { AXH_COUNT_UNPACK;
  read_floor<512, 4>(q, out, a.n_units);
}

// The same read at other launch shapes (axh_read_floor_shape: the sweep for
// the best single-launch read of a buffer).
#define AXH_READ_FLOOR_SHAPE(T, U)                                                               \
  extern "C" __global__ void __launch_bounds__(T) axh_read_floor_t##T##_u##U(                    \
      const uint8_t *__restrict__ q, uint32_t *__restrict__ out, AXH_COUNT_ARGS) {               \
    AXH_COUNT_UNPACK;                                                                            \
    read_floor<T, U>(q, out, a.n_units);                                                         \
  }
AXH_READ_FLOOR_SHAPE(256, 2)
AXH_READ_FLOOR_SHAPE(256, 4)
AXH_READ_FLOOR_SHAPE(256, 8)
AXH_READ_FLOOR_SHAPE(512, 2)
AXH_READ_FLOOR_SHAPE(512, 4)
AXH_READ_FLOOR_SHAPE(512, 8)
AXH_READ_FLOOR_SHAPE(1024, 2)
AXH_READ_FLOOR_SHAPE(1024, 4)
AXH_READ_FLOOR_SHAPE(1024, 8)

// The same launch shape doing nothing: the per-launch cost alone.
extern "C" __global__ void __launch_bounds__(512) axh_launch_empty(const uint8_t *__restrict__ q,
                                                                   uint32_t *__restrict__ out,
                                                                   AXH_COUNT_ARGS) { AXH_COUNT_UNPACK;
  if (a.n_units == 0xFFFFFFFFu && threadIdx.x == 0) out[0] = (uint32_t)(uintptr_t)q;
}

// Bounded busy wait (runtime tests of the completion timeout): sleeps
// a.n_units times (about 3 us each) and then writes the count.  Always ends.
extern "C" __global__ void __launch_bounds__(64) axh_spin(uint32_t *__restrict__ out,
                                                          AXH_COUNT_ARGS) { AXH_COUNT_UNPACK;
  for (uint32_t i = 0; i < a.n_units; ++i) __builtin_amdgcn_s_sleep(127);
  if (threadIdx.x == 0 && blockIdx.x == 0) out[0] = a.n_units;
}
