// Shared device helpers for the gfx950 Q4_0 / Q4_K_M kernels.
//
// Formats (reference: DESIGN.md:322-380 and 436-520 of rudybear/axiom-compute):
//   Q4_0 block, 18 B / 32 weights: f16 LE d @0, qs[16] @2.  Byte k -> weight k
//        (low nibble) and weight k+16 (high nibble); value = (nibble - 8) * d.
//   Q4_K superblock, 144 B / 256 weights: f16 LE d @0, f16 LE dmin @2,
//        scales[12] @4, qs[128] @16.  Chunk c (0..3) uses sub-blocks 2c, 2c+1;
//        qs byte 32c+l -> weight 64c+l (low nibble, sub-block 2c) and weight
//        64c+32+l (high nibble, sub-block 2c+1); value = d*sc*nibble - dmin*m.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace axh {

constexpr int kQ4kSbBytes = 144;
constexpr int kQ4kSbElems = 256;
constexpr int kQ4_0BlockBytes = 18;
constexpr int kQ4_0BlockElems = 32;
constexpr int kWave = 64;

// IEEE binary16 bits -> f32.  v_cvt_f32_f16 is exact for every input, f16
// subnormals included (f16 denormals are kept by the default FP mode).
__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}

// A 4-bit nibble sitting in bits 0..3 (or 4..7) of a 16-bit half, with all
// other bits clear, is the f16 subnormal nibble * 2^-24 (or nibble * 2^-20).
// Feeding it to an f32 FMA through the f16 -> f32 operand conversion
// (v_fma_mix_f32) multiplies by the exact nibble value with no separate
// integer -> float conversion.  The 2^24 / 2^20 factors are folded into the
// per-sub-block scales, so every product stays exact.
__device__ __forceinline__ float lo_half_f16(uint32_t v) { return f16_to_f32(v & 0xFFFFu); }
__device__ __forceinline__ float hi_half_f16(uint32_t v) { return f16_to_f32(v >> 16); }

// The per-sub-block (scale, min) pairs for sub-blocks j0 = 2c and j1 = 2c + 1
// of a Q4_K superblock, unpacked from the 12-byte scales field held in header
// words s03 (scales[0..3]), s47 (scales[4..7]) and s811 (scales[8..11]).
// get_scale_min_k4 (reference tests/common_helpers.rs:352-371):
//   j < 4 : sc = s[j] & 63;                          m = s[j+4] & 63
//   j >= 4: sc = (s[j+4] & 15) | ((s[j-4] >> 6) << 4); m = (s[j+4] >> 4) | ((s[j] >> 6) << 4)
// Both j of a chunk share byte lane (j & 3) pairs, so the two decodes run as
// one 16-bit SWAR decode.  Returns sc0 | sc1 << 8 in *sc and m0 | m1 << 8 in *m.
__device__ __forceinline__ void q4k_scale_min_pair(uint32_t s03, uint32_t s47, uint32_t s811,
                                                   uint32_t c, uint32_t *sc, uint32_t *m) {
  const uint32_t sh = (c & 1u) * 16u;
  const uint32_t a = (s03 >> sh) & 0xFFFFu;   // s[j & 3] pair
  const uint32_t b = (s47 >> sh) & 0xFFFFu;   // s[(j & 3) + 4] pair
  const uint32_t cc = (s811 >> sh) & 0xFFFFu; // s[(j & 3) + 8] pair
  const uint32_t sc_lo = a & 0x3F3Fu;
  const uint32_t m_lo = b & 0x3F3Fu;
  const uint32_t sc_hi = (cc & 0x0F0Fu) | ((a >> 2) & 0x3030u);
  const uint32_t m_hi = ((cc >> 4) & 0x0F0Fu) | ((b >> 2) & 0x3030u);
  const bool high = c >= 2u;
  *sc = high ? sc_hi : sc_lo;
  *m = high ? m_hi : m_lo;
}

// Sum across the 64 lanes of a wave: DPP butterflies inside each 16-lane row,
// then the four row sums are read out with v_readlane.  Result is uniform.
template <int kCtrl>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, false));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov<0xB1>(v);  // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);  // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v); // row_half_mirror
  v += dpp_mov<0x140>(v); // row_mirror
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (r0 + r1) + (r2 + r3);
}

} // namespace axh
