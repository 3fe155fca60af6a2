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

__device__ __forceinline__ void q4k_stage_tile(const float *__restrict__ x, float *xs, float *hs,
                                               uint32_t sb0, uint32_t n_sb, uint32_t tid,
                                               uint32_t nthreads) {
  const uint32_t ngroups = n_sb * 16u;
  for (uint32_t gi = tid; gi < ngroups; gi += nthreads) {
    const uint32_t slot = gi >> 4, r = gi & 15u;
    const uint32_t c = r >> 2, part = (r >> 1) & 1u, h = r & 1u, k = 2u * c + h;
    const float4 *src = reinterpret_cast<const float4 *>(x + (size_t)(sb0 + slot) * 256u + 16u * r);
    const float4 v0 = src[0], v1 = src[1], v2 = src[2], v3 = src[3];
    float *dst = xs + slot * 256u + part * 128u + 4u * k;
    const uint32_t sw = (slot & 1u) * 32u;
    *reinterpret_cast<float4 *>(dst + (0u ^ sw)) = v0;
    *reinterpret_cast<float4 *>(dst + (32u ^ sw)) = v1;
    *reinterpret_cast<float4 *>(dst + (64u ^ sw)) = v2;
    *reinterpret_cast<float4 *>(dst + (96u ^ sw)) = v3;
    const float s = ((v0.x + v0.y) + (v0.z + v0.w)) + ((v1.x + v1.y) + (v1.z + v1.w)) +
                    (((v2.x + v2.y) + (v2.z + v2.w)) + ((v3.x + v3.y) + (v3.z + v3.w)));
    hs[slot * 16u + 2u * k + part] = s;
  }
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

template <int RPW, int NW, int PF>
__device__ __forceinline__ void q4k_matvec_body(const uint8_t *__restrict__ q,
                                                const float *__restrict__ x, float *__restrict__ y,
                                                uint32_t n_rows, uint32_t nsb, uint32_t tile_sb,
                                                uint32_t block, float *lds) {
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u, wave = tid >> 6;
  const uint32_t g = lane >> 3, k = lane & 7u, c = k >> 1;
  const uint32_t row0 = (block * NW + wave) * RPW;
  const size_t row_bytes = (size_t)nsb * kQ4kSbBytes;

  const uint8_t *rowp[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const uint32_t row = min(row0 + r, n_rows - 1u); // clamp: loads stay in bounds
    rowp[r] = q + (size_t)row * row_bytes + 16u * k;
  }
  const uint32_t n_it = (nsb + 7u) >> 3;
  const uint32_t it_per_tile = tile_sb >> 3;
  float *xs = lds;
  float *hs = lds + tile_sb * 256u;

  uint4 H[PF][RPW], Qv[PF][RPW];
  float acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;

#pragma unroll
  for (int p = 0; p < PF; ++p) {
    const uint32_t sb = (uint32_t)p * 8u + g;
    if ((uint32_t)p < n_it && sb < nsb) {
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        const uint8_t *b = rowp[r] + (size_t)sb * kQ4kSbBytes;
        H[p][r] = *reinterpret_cast<const uint4 *>(b - 16u * k);
        Qv[p][r] = *reinterpret_cast<const uint4 *>(b + 16u);
      }
    }
  }

  uint32_t tile = 0xFFFFFFFFu;
  for (uint32_t it0 = 0; it0 < n_it; it0 += PF) {
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      const uint32_t it = it0 + (uint32_t)p;
      if (it < n_it) {
        const uint32_t t_it = it / it_per_tile;
        if (t_it != tile) { // uniform across the workgroup
          if (tile != 0xFFFFFFFFu) __syncthreads();
          tile = t_it;
          const uint32_t sb0 = t_it * tile_sb;
          q4k_stage_tile(x, xs, hs, sb0, min(tile_sb, nsb - sb0), tid, NW * 64u);
          __syncthreads();
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
        // refill this prefetch slot with iteration it + PF
        const uint32_t nit = it + PF;
        const uint32_t nsb_i = nit * 8u + g;
        if (nit < n_it && nsb_i < nsb) {
#pragma unroll
          for (int r = 0; r < RPW; ++r) {
            const uint8_t *b = rowp[r] + (size_t)nsb_i * kQ4kSbBytes;
            H[p][r] = *reinterpret_cast<const uint4 *>(b - 16u * k);
            Qv[p][r] = *reinterpret_cast<const uint4 *>(b + 16u);
          }
        }
      }
    }
  }

#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const float s = wave_sum(acc[r]);
    if (lane == 0 && row0 + r < n_rows) y[row0 + r] = s;
  }
}

#define AXH_Q4K_MATVEC(RPW, NW, PF)                                                              \
  extern "C" __global__ void __launch_bounds__(NW * 64)                                          \
      axh_q4k_matvec_r##RPW##_w##NW##_p##PF(const uint8_t *__restrict__ q,                       \
                                            const float *__restrict__ x, float *__restrict__ y,  \
                                            RowsArgs a) {                                        \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4k_matvec_body<RPW, NW, PF>(q, x, y, a.n_rows, a.units_per_row, a.tile_units, blockIdx.x,   \
                                 axh_lds_dyn);                                                   \
  }

AXH_Q4K_MATVEC(1, 4, 2)
AXH_Q4K_MATVEC(1, 4, 4)
AXH_Q4K_MATVEC(1, 8, 4)
AXH_Q4K_MATVEC(1, 8, 8)
AXH_Q4K_MATVEC(1, 16, 4)
AXH_Q4K_MATVEC(2, 4, 2)
AXH_Q4K_MATVEC(2, 4, 4)
AXH_Q4K_MATVEC(2, 8, 2)
AXH_Q4K_MATVEC(2, 8, 4)
AXH_Q4K_MATVEC(2, 8, 7)
AXH_Q4K_MATVEC(4, 4, 2)
AXH_Q4K_MATVEC(4, 4, 4)
AXH_Q4K_MATVEC(4, 8, 2)

// Reference-compatible entry point: the contract of
// examples/q4km_dequant_matvec.axc (bindings q=0, x=1, y=2; push constant
// n_superblocks: u32 @0; @workgroup(64,1,1); dispatched as 1x1x1).  One wave
// computes y[0]; workgroups other than 0 return, like the reference's
// `if gid(0) >= 1 { return; }`.
constexpr uint32_t kRefTileSb = 16; // 17 KiB static LDS tile
extern "C" __global__ void __launch_bounds__(64)
    q4km_dequant_matvec(const uint8_t *__restrict__ q, const float *__restrict__ x,
                        float *__restrict__ y, CountArgs a) {
  __shared__ float lds[kRefTileSb * 256 + kRefTileSb * 16];
  if (blockIdx.x != 0 || blockIdx.y != 0 || blockIdx.z != 0) return;
  if (a.n_units == 0) {
    if (threadIdx.x == 0) y[0] = 0.0f;
    return;
  }
  q4k_matvec_body<1, 1, 2>(q, x, y, 1u, a.n_units, kRefTileSb, 0u, lds);
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

#define AXH_Q4_0_MATVEC(RPW, NW)                                                                 \
  extern "C" __global__ void __launch_bounds__(NW * 64)                                          \
      axh_q4_0_matvec_r##RPW##_w##NW(const uint8_t *__restrict__ q,                              \
                                     const float *__restrict__ x, float *__restrict__ y,         \
                                     RowsArgs a) {                                               \
    extern __shared__ float axh_lds_dyn[];                                                       \
    q4_0_matvec_body<RPW, NW>(q, x, y, a.n_rows, a.units_per_row, a.tile_units, blockIdx.x,      \
                              axh_lds_dyn);                                                      \
  }

AXH_Q4_0_MATVEC(1, 1)
AXH_Q4_0_MATVEC(1, 4)
AXH_Q4_0_MATVEC(2, 4)
AXH_Q4_0_MATVEC(4, 4)

// Reference-compatible entry point for examples/q4_0_dequant_matvec.axc
// (bindings q=0, x=1, y=2; push constant n_blocks: u32 @0; 1x1x1 of 64).
constexpr uint32_t kRefTileB = 128; // 17 KiB static LDS tile
extern "C" __global__ void __launch_bounds__(64)
    q4_0_dequant_matvec(const uint8_t *__restrict__ q, const float *__restrict__ x,
                        float *__restrict__ y, CountArgs a) {
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
// Q4_K: one thread per (superblock, 16-byte qs slice).  Each value is
// fma(d*sc, nibble, -(dmin*m)): d*sc, dmin*m and (d*sc)*nibble are exact in
// f32, so the single rounding equals the reference's d1*lo - m1f.
extern "C" __global__ void __launch_bounds__(256)
    axh_q4k_dequant(const uint8_t *__restrict__ q, float *__restrict__ w, CountArgs a) {
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
    axh_q4_0_dequant(const uint8_t *__restrict__ q, float *__restrict__ w, CountArgs a) {
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
    axh_f16_widen(const uint16_t *__restrict__ h, float *__restrict__ f, CountArgs a) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i < a.n_units) f[i] = f16_to_f32(h[i]);
}
