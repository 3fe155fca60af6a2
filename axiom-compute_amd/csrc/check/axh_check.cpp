// Host-side correctness verdicts for the tuning tools (the counterpart of the
// reference's CPU references in crates/axc-driver/src/mcp/tools/
// bench_variant.rs:53-78,373-420, which left Q4_0 / Q4_K as "not checked").
// A verdict compares a device result, copied to the host, with an f64
// accumulation of the exact weights; it never produces results for callers.
//
// Weights: Q4_K_M w = RN_f32(d*sc*q - dmin*m) and Q4_0 w = (q - 8)*d, the
// reference's dequantisation (crates/axc-driver/tests/common_helpers.rs:
// 437-454; crates/axc-driver/benches/common.rs:229-253); for the batched
// matmul the weight is RN_f16 of that value.
//
// Criterion per row (n products, s = sum|w*x| / sqrt(n)): |y - ref| <= tol*|ref|
// when |ref| >= 0.1*s, else |y - ref| <= tol*s; plus ||y - ref|| <= tol*||ref||.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "axh.h"
#include "axh_check.h"

namespace {

thread_local char g_err[256];

float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31;
  const uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { // subnormal: man * 2^-24, exact in f32
      float v = (float)man * 5.9604644775390625e-8f;
      std::memcpy(&bits, &v, 4);
      bits |= sign;
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (man << 13) | (man ? 0x00400000u : 0u);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

uint16_t f32_to_f16_rne(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); // rounds to infinity
  if (ax < 0x38800000u) {                                    // f16 subnormal or zero
    const float a = std::fabs(f) * 16777216.0f;              // exact scaling into integer range
    const float r = std::nearbyint(a);                       // default mode: ties to even
    return (uint16_t)(sign | (uint32_t)r);
  }
  const uint32_t mant = ax & 0x7FFFFFu, e = (ax >> 23) - 112u;
  uint32_t h = (e << 10) | (mant >> 13);
  const uint32_t rem = mant & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  return (uint16_t)(sign | h);
}

void scale_min(const uint8_t *s, int j, int *sc, int *m) {
  if (j < 4) {
    *sc = s[j] & 63;
    *m = s[j + 4] & 63;
  } else {
    *sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
    *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

// 256 dequantised weights of one superblock.
void q4k_weights(const uint8_t *sb, float *w) {
  uint16_t dh, mh;
  std::memcpy(&dh, sb, 2);
  std::memcpy(&mh, sb + 2, 2);
  const float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
  const uint8_t *scales = sb + 4, *qs = sb + 16;
  for (int c = 0; c < 4; ++c) {
    int sc0, m0, sc1, m1;
    scale_min(scales, 2 * c, &sc0, &m0);
    scale_min(scales, 2 * c + 1, &sc1, &m1);
    const float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
    const float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
    for (int l = 0; l < 32; ++l) {
      const uint8_t b = qs[32 * c + l];
      w[64 * c + l] = std::fma(d1, (float)(b & 0x0F), -mm1);
      w[64 * c + 32 + l] = std::fma(d2, (float)(b >> 4), -mm2);
    }
  }
}

void q4_0_weights(const uint8_t *blk, float *w) {
  uint16_t dh;
  std::memcpy(&dh, blk, 2);
  const float d = f16_to_f32(dh);
  for (int k = 0; k < 16; ++k) {
    const uint8_t b = blk[2 + k];
    w[k] = (float)((int)(b & 0x0F) - 8) * d;
    w[k + 16] = (float)((int)(b >> 4) - 8) * d;
  }
}

struct Acc {
  double num2 = 0.0, den2 = 0.0;
  double worst = 0.0;
  uint64_t worst_row = 0, failed = 0, rows = 0;
};

void judge_row(Acc &a, uint64_t row, double got, double ref, double absdot, double n, double tol) {
  const double s = absdot / std::sqrt(n > 0 ? n : 1.0);
  const double err = std::fabs(got - ref);
  const bool cancelling = std::fabs(ref) < 0.1 * s;
  const double allowed = tol * (cancelling ? s : std::fabs(ref));
  const double scaled = allowed > 0 ? err / allowed : (err > 0 ? INFINITY : 0.0);
  if (!(err <= allowed) || std::isnan(got)) ++a.failed;
  if (scaled > a.worst || std::isnan(got)) {
    a.worst = std::isnan(got) ? INFINITY : scaled;
    a.worst_row = row;
  }
  a.num2 += (got - ref) * (got - ref);
  a.den2 += ref * ref;
  ++a.rows;
}

axh_status finish(const Acc &a, double tol, axh_check_report *out) {
  out->rows_checked = a.rows;
  out->rows_failed = a.failed;
  out->worst_row = a.worst_row;
  out->worst_over_allowed = a.worst;
  out->norm_rel_err = a.den2 > 0 ? std::sqrt(a.num2 / a.den2) : std::sqrt(a.num2);
  out->ok = (a.failed == 0 && out->norm_rel_err <= tol) ? 1u : 0u;
  return AXH_OK;
}

axh_status bad(const char *msg) {
  std::snprintf(g_err, sizeof(g_err), "%s", msg);
  return AXH_ERR_INVALID_ARGUMENT;
}

} // namespace

extern "C" {

const char *axh_check_last_error(void) { return g_err; }

axh_status axh_check_q4k_matvec(const void *q, const float *x, const float *y, uint32_t n_rows,
                                uint32_t sb_per_row, double rel_tol, axh_check_report *out) {
  if (!out || (n_rows && (!y || (sb_per_row && (!q || !x))))) return bad("NULL argument");
  Acc a;
  std::vector<float> w(256);
  const uint8_t *qb = static_cast<const uint8_t *>(q);
  for (uint64_t r = 0; r < n_rows; ++r) {
    double ref = 0.0, absdot = 0.0;
    for (uint32_t s = 0; s < sb_per_row; ++s) {
      q4k_weights(qb + (r * sb_per_row + s) * 144u, w.data());
      for (int k = 0; k < 256; ++k) {
        const double p = (double)w[k] * (double)x[s * 256u + k];
        ref += p;
        absdot += std::fabs(p);
      }
    }
    judge_row(a, r, y[r], ref, absdot, 256.0 * sb_per_row, rel_tol);
  }
  return finish(a, rel_tol, out);
}

axh_status axh_check_q4_0_matvec(const void *q, const float *x, const float *y, uint32_t n_rows,
                                 uint32_t blocks_per_row, double rel_tol,
                                 axh_check_report *out) {
  if (!out || (n_rows && (!y || (blocks_per_row && (!q || !x))))) return bad("NULL argument");
  Acc a;
  float w[32];
  const uint8_t *qb = static_cast<const uint8_t *>(q);
  for (uint64_t r = 0; r < n_rows; ++r) {
    double ref = 0.0, absdot = 0.0;
    for (uint32_t b = 0; b < blocks_per_row; ++b) {
      q4_0_weights(qb + (r * blocks_per_row + b) * 18u, w);
      for (int k = 0; k < 32; ++k) {
        const double p = (double)w[k] * (double)x[b * 32u + k];
        ref += p;
        absdot += std::fabs(p);
      }
    }
    judge_row(a, r, y[r], ref, absdot, 32.0 * blocks_per_row, rel_tol);
  }
  return finish(a, rel_tol, out);
}

axh_status axh_check_q4k_matmul_f16(const void *q, const uint16_t *x, const float *y,
                                    uint32_t n_rows, uint32_t sb_per_row, uint32_t batch,
                                    double rel_tol, axh_check_report *out) {
  if (!out || (n_rows && batch && (!y || !q || !x))) return bad("NULL argument");
  if (sb_per_row == 0) return bad("sb_per_row must be at least 1");
  Acc a;
  const uint64_t K = 256ull * sb_per_row;
  std::vector<float> w(K), w32(256), xf(K * batch);
  for (uint64_t i = 0; i < K * batch; ++i) xf[i] = f16_to_f32(x[i]);
  const uint8_t *qb = static_cast<const uint8_t *>(q);
  for (uint64_t r = 0; r < n_rows; ++r) {
    for (uint32_t s = 0; s < sb_per_row; ++s) {
      q4k_weights(qb + (r * sb_per_row + s) * 144u, w32.data());
      for (int k = 0; k < 256; ++k) w[s * 256u + k] = f16_to_f32(f32_to_f16_rne(w32[k]));
    }
    for (uint32_t b = 0; b < batch; ++b) {
      double ref = 0.0, absdot = 0.0;
      const float *xb = xf.data() + (uint64_t)b * K;
      for (uint64_t k = 0; k < K; ++k) {
        const double p = (double)w[k] * (double)xb[k];
        ref += p;
        absdot += std::fabs(p);
      }
      judge_row(a, (uint64_t)b * n_rows + r, y[(uint64_t)b * n_rows + r], ref, absdot,
                (double)K, rel_tol);
    }
  }
  return finish(a, rel_tol, out);
}

} // extern "C"
