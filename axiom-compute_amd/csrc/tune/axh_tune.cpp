// Strategy-hole autotuner: XXH3-64 variant ids, mixed-radix enumeration and
// grid search with caller callbacks (crates/axc-optimize of
// rudybear/axiom-compute), plus a HIP-timed sweep of the Q4_K matvec
// variants built on the same grid search.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <numeric>
#include <string>
#include <vector>

#include "axh_check.h"
#include "axh_internal.h"
#include "axh_tune.h"

namespace axh {
namespace {

// ---------------------------------------------------------------------------
// XXH3 64-bit, seed 0, default 192-byte secret (the published XXH3 algorithm;
// variant ids must equal the reference's xxhash-rust xxh3_64).
// ---------------------------------------------------------------------------
constexpr uint64_t kP32_1 = 0x9E3779B1u, kP32_2 = 0x85EBCA77u, kP32_3 = 0xC2B2AE3Du;
constexpr uint64_t kP64_1 = 0x9E3779B185EBCA87ull, kP64_2 = 0xC2B2AE3D27D4EB4Full,
                   kP64_3 = 0x165667B19E3779F9ull, kP64_4 = 0x85EBCA77C2B2AE63ull,
                   kP64_5 = 0x27D4EB2F165667C5ull;
constexpr uint64_t kMx1 = 0x165667919E3779F9ull, kMx2 = 0x9FB21C651E98DF25ull;

const uint8_t kSecret[192] = {
    0xb8, 0xfe, 0x6c, 0x39, 0x23, 0xa4, 0x4b, 0xbe, 0x7c, 0x01, 0x81, 0x2c, 0xf7, 0x21, 0xad, 0x1c,
    0xde, 0xd4, 0x6d, 0xe9, 0x83, 0x90, 0x97, 0xdb, 0x72, 0x40, 0xa4, 0xa4, 0xb7, 0xb3, 0x67, 0x1f,
    0xcb, 0x79, 0xe6, 0x4e, 0xcc, 0xc0, 0xe5, 0x78, 0x82, 0x5a, 0xd0, 0x7d, 0xcc, 0xff, 0x72, 0x21,
    0xb8, 0x08, 0x46, 0x74, 0xf7, 0x43, 0x24, 0x8e, 0xe0, 0x35, 0x90, 0xe6, 0x81, 0x3a, 0x26, 0x4c,
    0x3c, 0x28, 0x52, 0xbb, 0x91, 0xc3, 0x00, 0xcb, 0x88, 0xd0, 0x65, 0x8b, 0x1b, 0x53, 0x2e, 0xa3,
    0x71, 0x64, 0x48, 0x97, 0xa2, 0x0d, 0xf9, 0x4e, 0x38, 0x19, 0xef, 0x46, 0xa9, 0xde, 0xac, 0xd8,
    0xa8, 0xfa, 0x76, 0x3f, 0xe3, 0x9c, 0x34, 0x3f, 0xf9, 0xdc, 0xbb, 0xc7, 0xc7, 0x0b, 0x4f, 0x1d,
    0x8a, 0x51, 0xe0, 0x4b, 0xcd, 0xb4, 0x59, 0x31, 0xc8, 0x9f, 0x7e, 0xc9, 0xd9, 0x78, 0x73, 0x64,
    0xea, 0xc5, 0xac, 0x83, 0x34, 0xd3, 0xeb, 0xc3, 0xc5, 0x81, 0xa0, 0xff, 0xfa, 0x13, 0x63, 0xeb,
    0x17, 0x0d, 0xdd, 0x51, 0xb7, 0xf0, 0xda, 0x49, 0xd3, 0x16, 0x55, 0x26, 0x29, 0xd4, 0x68, 0x9e,
    0x2b, 0x16, 0xbe, 0x58, 0x7d, 0x47, 0xa1, 0xfc, 0x8f, 0xf8, 0xb8, 0xd1, 0x7a, 0xd0, 0x31, 0xce,
    0x45, 0xcb, 0x3a, 0x8f, 0x95, 0x16, 0x04, 0x28, 0xaf, 0xd7, 0xfb, 0xca, 0xbb, 0x4b, 0x40, 0x7e,
};
constexpr size_t kSecretLen = sizeof(kSecret);

inline uint64_t rd64(const uint8_t *p) {
  uint64_t v;
  std::memcpy(&v, p, 8); // little-endian host (x86-64)
  return v;
}
inline uint32_t rd32(const uint8_t *p) {
  uint32_t v;
  std::memcpy(&v, p, 4);
  return v;
}
inline uint64_t rotl64(uint64_t v, int r) { return (v << r) | (v >> (64 - r)); }
inline uint64_t bswap64(uint64_t v) { return __builtin_bswap64(v); }

// low 64 bits XOR high 64 bits of the 128-bit product
inline uint64_t mul_fold(uint64_t a, uint64_t b) {
  const unsigned __int128 p = (unsigned __int128)a * b;
  return (uint64_t)p ^ (uint64_t)(p >> 64);
}

inline uint64_t avalanche_xxh64(uint64_t h) {
  h ^= h >> 33;
  h *= kP64_2;
  h ^= h >> 29;
  h *= kP64_3;
  h ^= h >> 32;
  return h;
}

inline uint64_t avalanche_xxh3(uint64_t h) {
  h ^= h >> 37;
  h *= kMx1;
  h ^= h >> 32;
  return h;
}

inline uint64_t rrmxmx(uint64_t h, uint64_t len) {
  h ^= rotl64(h, 49) ^ rotl64(h, 24);
  h *= kMx2;
  h ^= (h >> 35) + len;
  h *= kMx2;
  return h ^ (h >> 28);
}

inline uint64_t mix16(const uint8_t *in, const uint8_t *sec) {
  return mul_fold(rd64(in) ^ rd64(sec), rd64(in + 8) ^ rd64(sec + 8));
}

inline void acc512(uint64_t acc[8], const uint8_t *in, const uint8_t *sec) {
  for (int i = 0; i < 8; ++i) {
    const uint64_t v = rd64(in + 8 * i);
    const uint64_t k = v ^ rd64(sec + 8 * i);
    acc[i ^ 1] += v;
    acc[i] += (uint64_t)(uint32_t)k * (k >> 32);
  }
}

uint64_t xxh3_long(const uint8_t *in, size_t len) {
  uint64_t acc[8] = {kP32_3, kP64_1, kP64_2, kP64_3, kP64_4, kP32_2, kP64_5, kP32_1};
  const size_t stripes_per_block = (kSecretLen - 64) / 8;
  const size_t block = 64 * stripes_per_block;
  const size_t n_blocks = (len - 1) / block;
  for (size_t b = 0; b < n_blocks; ++b) {
    for (size_t s = 0; s < stripes_per_block; ++s) acc512(acc, in + b * block + 64 * s, kSecret + 8 * s);
    for (int i = 0; i < 8; ++i) { // scramble
      uint64_t a = acc[i];
      a ^= a >> 47;
      a ^= rd64(kSecret + kSecretLen - 64 + 8 * i);
      acc[i] = a * kP32_1;
    }
  }
  const size_t stripes = ((len - 1) - block * n_blocks) / 64;
  for (size_t s = 0; s < stripes; ++s) acc512(acc, in + n_blocks * block + 64 * s, kSecret + 8 * s);
  acc512(acc, in + len - 64, kSecret + kSecretLen - 64 - 7);
  uint64_t r = (uint64_t)len * kP64_1;
  for (int i = 0; i < 4; ++i)
    r += mul_fold(acc[2 * i] ^ rd64(kSecret + 11 + 16 * i), acc[2 * i + 1] ^ rd64(kSecret + 11 + 16 * i + 8));
  return avalanche_xxh3(r);
}

uint64_t xxh3_64(const uint8_t *in, size_t len) {
  if (len == 0) return avalanche_xxh64(rd64(kSecret + 56) ^ rd64(kSecret + 64));
  if (len <= 3) {
    const uint32_t combined = ((uint32_t)in[0] << 16) | ((uint32_t)in[len >> 1] << 24) |
                              (uint32_t)in[len - 1] | ((uint32_t)len << 8);
    const uint64_t flip = (uint64_t)(rd32(kSecret) ^ rd32(kSecret + 4));
    return avalanche_xxh64((uint64_t)combined ^ flip);
  }
  if (len <= 8) {
    const uint64_t flip = rd64(kSecret + 8) ^ rd64(kSecret + 16);
    const uint64_t v = (uint64_t)rd32(in + len - 4) + ((uint64_t)rd32(in) << 32);
    return rrmxmx(v ^ flip, len);
  }
  if (len <= 16) {
    const uint64_t lo = rd64(in) ^ (rd64(kSecret + 24) ^ rd64(kSecret + 32));
    const uint64_t hi = rd64(in + len - 8) ^ (rd64(kSecret + 40) ^ rd64(kSecret + 48));
    return avalanche_xxh3((uint64_t)len + bswap64(lo) + hi + mul_fold(lo, hi));
  }
  if (len <= 128) {
    uint64_t acc = (uint64_t)len * kP64_1;
    if (len > 32) {
      if (len > 64) {
        if (len > 96) {
          acc += mix16(in + 48, kSecret + 96);
          acc += mix16(in + len - 64, kSecret + 112);
        }
        acc += mix16(in + 32, kSecret + 64);
        acc += mix16(in + len - 48, kSecret + 80);
      }
      acc += mix16(in + 16, kSecret + 32);
      acc += mix16(in + len - 32, kSecret + 48);
    }
    acc += mix16(in, kSecret);
    acc += mix16(in + len - 16, kSecret + 16);
    return avalanche_xxh3(acc);
  }
  if (len <= 240) {
    uint64_t acc = (uint64_t)len * kP64_1;
    const size_t rounds = len / 16;
    for (size_t i = 0; i < 8; ++i) acc += mix16(in + 16 * i, kSecret + 16 * i);
    acc = avalanche_xxh3(acc);
    for (size_t i = 8; i < rounds; ++i) acc += mix16(in + 16 * i, kSecret + 16 * (i - 8) + 3);
    acc += mix16(in + len - 16, kSecret + 136 - 17);
    return avalanche_xxh3(acc);
  }
  return xxh3_long(in, len);
}

struct Sorted {
  std::vector<uint32_t> order; // caller indices, by name
  std::vector<uint64_t> radix;
  uint64_t total = 0;
};

axh_status sort_holes(const axh_strategy_hole *holes, uint32_t n, Sorted &s) {
  if (n == 0) return fail((axh_status)AXH_ERR_EMPTY_STRATEGY,
                          "strategy map is empty (no holes to enumerate)");
  if (!holes) return fail(AXH_ERR_INVALID_ARGUMENT, "holes is NULL");
  s.order.resize(n);
  std::iota(s.order.begin(), s.order.end(), 0u);
  for (uint32_t i = 0; i < n; ++i)
    if (!holes[i].name || !holes[i].candidates || holes[i].n_candidates == 0)
      return fail(AXH_ERR_INVALID_ARGUMENT, "hole " + std::to_string(i) + " has no candidates");
  std::sort(s.order.begin(), s.order.end(), [&](uint32_t a, uint32_t b) {
    return std::strcmp(holes[a].name, holes[b].name) < 0;
  });
  for (uint32_t i = 1; i < n; ++i)
    if (std::strcmp(holes[s.order[i - 1]].name, holes[s.order[i]].name) == 0)
      return fail(AXH_ERR_INVALID_ARGUMENT,
                  std::string("duplicate hole name '") + holes[s.order[i]].name + "'");
  s.radix.resize(n);
  s.total = 1;
  for (uint32_t k = 0; k < n; ++k) {
    s.radix[k] = holes[s.order[k]].n_candidates;
    s.total = (s.total > UINT64_MAX / s.radix[k]) ? UINT64_MAX : s.total * s.radix[k];
  }
  return AXH_OK;
}

// Values (sorted-key order) and id of variant `ordinal`: the last key varies fastest.
uint64_t variant_at(const axh_strategy_hole *holes, const Sorted &s, uint64_t ordinal,
                    int64_t *values, std::vector<uint8_t> &enc) {
  const uint32_t n = (uint32_t)s.order.size();
  uint64_t rem = ordinal;
  for (uint32_t k = n; k-- > 0;) {
    const uint64_t idx = rem % s.radix[k];
    rem /= s.radix[k];
    values[k] = holes[s.order[k]].candidates[idx];
  }
  enc.clear();
  for (uint32_t k = 0; k < n; ++k) {
    const char *name = holes[s.order[k]].name;
    const uint32_t len = (uint32_t)std::strlen(name);
    uint8_t b[8];
    std::memcpy(b, &len, 4);
    enc.insert(enc.end(), b, b + 4);
    enc.insert(enc.end(), name, name + len);
    std::memcpy(b, &values[k], 8);
    enc.insert(enc.end(), b, b + 8);
  }
  return xxh3_64(enc.data(), enc.size());
}

} // namespace
} // namespace axh

using namespace axh;

extern "C" {

uint64_t axh_xxh3_64(const void *data, size_t len) {
  return xxh3_64(static_cast<const uint8_t *>(data), data ? len : 0);
}

axh_status axh_enumerate_strategy(const axh_strategy_hole *holes, uint32_t n_holes,
                                  uint64_t *n_variants_out, uint32_t *sorted_hole_index_out,
                                  int64_t *values_out, uint64_t *variant_ids_out,
                                  uint64_t capacity) {
  Sorted s;
  axh_status st = sort_holes(holes, n_holes, s);
  if (st != AXH_OK) return st;
  if (n_variants_out) *n_variants_out = s.total;
  if (sorted_hole_index_out)
    for (uint32_t k = 0; k < n_holes; ++k) sorted_hole_index_out[k] = s.order[k];
  if (capacity == 0 || (!values_out && !variant_ids_out)) return ok();
  if (capacity < s.total)
    return fail(AXH_ERR_INVALID_ARGUMENT, "capacity " + std::to_string(capacity) + " < " +
                                              std::to_string(s.total) + " variants");
  std::vector<int64_t> vals(n_holes);
  std::vector<uint8_t> enc;
  for (uint64_t v = 0; v < s.total; ++v) {
    const uint64_t id = variant_at(holes, s, v, vals.data(), enc);
    if (values_out) std::memcpy(values_out + v * n_holes, vals.data(), 8 * n_holes);
    if (variant_ids_out) variant_ids_out[v] = id;
  }
  return ok();
}

axh_status axh_grid_search(const axh_strategy_hole *holes, uint32_t n_holes,
                           const axh_correctness_policy *policy, axh_correctness_fn correctness,
                           axh_bench_fn bench, void *user, axh_variant_result *results,
                           uint64_t capacity, axh_grid_search_result *out) {
  if (n_holes == 0)
    return fail((axh_status)AXH_ERR_NO_STRATEGY, "kernel has no @strategy annotation");
  if (!bench || !out) return fail(AXH_ERR_INVALID_ARGUMENT, "bench and out are required");
  Sorted s;
  axh_status st = sort_holes(holes, n_holes, s);
  if (st != AXH_OK)
    return fail((axh_status)AXH_ERR_ENUMERATE_FAILED,
                std::string("strategy enumeration failed: ") + axh_last_error());
  if (!results || capacity < s.total)
    return fail(AXH_ERR_INVALID_ARGUMENT, "results must hold " + std::to_string(s.total) +
                                              " variants");
  const bool check = policy && policy->kind != AXH_POLICY_NONE && correctness;
  std::vector<int64_t> vals(n_holes);
  std::vector<uint8_t> enc;
  char err[120];
  for (uint64_t v = 0; v < s.total; ++v) {
    axh_variant_result &r = results[v];
    std::memset(&r, 0, sizeof(r));
    r.ordinal = v;
    r.variant_id = variant_at(holes, s, v, vals.data(), enc);
    err[0] = 0;
    if (check && correctness(user, v, vals.data(), n_holes, err, sizeof(err)) != 0) {
      r.outcome = AXH_OUTCOME_CORRECTNESS_REJECTED;
      std::snprintf(r.message, sizeof(r.message), "%s", err);
      continue;
    }
    err[0] = 0;
    if (bench(user, v, vals.data(), n_holes, &r.stats, err, sizeof(err)) != 0) {
      r.outcome = AXH_OUTCOME_FAILED;
      std::snprintf(r.message, sizeof(r.message), "%s", err);
      continue;
    }
    r.outcome = AXH_OUTCOME_OK;
  }
  std::memset(out, 0, sizeof(*out));
  out->n_results = s.total;
  out->warned_large_product = s.total > AXH_CARTESIAN_WARN_THRESHOLD;
  const axh_variant_result *best = nullptr;
  for (uint64_t v = 0; v < s.total; ++v) // strict < keeps the lowest ordinal on ties
    if (results[v].outcome == AXH_OUTCOME_OK &&
        (!best || results[v].stats.median_ns < best->stats.median_ns))
      best = &results[v];
  if (!best) {
    for (uint64_t fo = 0; fo < 4 && fo < s.total; ++fo) { // R3 fallback chain
      out->winner_ordinal = fo;
      out->winner_variant_id = results[fo].variant_id;
      out->fallback_used = 1;
      return ok();
    }
    return fail((axh_status)AXH_ERR_NO_SUCCESSFUL_VARIANTS, "no variant benchmarked successfully");
  }
  out->winner_ordinal = best->ordinal;
  out->winner_variant_id = best->variant_id;
  return ok();
}

// ---- Q4_K matvec autotuner: every kernel family, judged by the checker ------
namespace {
// Weight copies the timing rotates through: more bytes than the 256 MiB
// Infinity Cache, so every timed call streams its weights from HBM, as the
// bench and a model's decode step do (a single 33 MB matrix stays cache-hot).
constexpr uint64_t kRotateBytes = 512ull << 20;
constexpr uint32_t kMaxCopies = 64;
// Interleaved confirmation of the sweep's winner against the default: rounds
// of calls of each, alternating; the default is kept unless the winner's
// median is below it by more than the run-to-run spread of these boxes.
constexpr uint32_t kConfirmRounds = 9, kConfirmCalls = 50;
constexpr double kConfirmSpread = 0.02;

struct Q4kTuneCtx {
  axh_context *ctx;
  const void *q;
  const float *x;
  float *y;
  uint32_t n_rows, sb;
  uint32_t samples;
  double tol;
  std::vector<uint8_t> q_host; // checker inputs
  std::vector<float> x_host, y_host;
  // hole names of the current family's search, in the enumerator's key order
  std::vector<std::string> keys;
  // rotated weight copies (copy 0 is the caller's q)
  uint8_t *copies = nullptr;
  uint64_t stride = 0;
  uint32_t n_copies = 1;
  uint32_t next = 0;
  const void *weights() {
    const uint32_t i = next++ % n_copies;
    return i == 0 ? q : copies + (uint64_t)(i - 1) * stride;
  }
};

// Median ns per call of `calls` back-to-back calls of v over the rotated
// copies (one group between two events).
axh_status time_calls(Q4kTuneCtx &t, const axh_q4_variant &v, uint32_t calls, hipEvent_t e0,
                      hipEvent_t e1, uint64_t *ns) {
  hipStream_t s = t.ctx->core->stream;
  for (uint32_t i = 0; i < 3; ++i) {
    const axh_status st = axh_q4k_matvec(t.ctx, t.weights(), t.x, t.y, t.n_rows, t.sb, &v, s);
    if (st != AXH_OK) return st;
  }
  hipEventRecord(e0, s);
  for (uint32_t i = 0; i < calls; ++i) {
    const axh_status st = axh_q4k_matvec(t.ctx, t.weights(), t.x, t.y, t.n_rows, t.sb, &v, s);
    if (st != AXH_OK) return st;
  }
  hipEventRecord(e1, s);
  const axh_status st = axh_synchronize(t.ctx, nullptr);
  if (st != AXH_OK) return st;
  float ms = 0;
  if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
    return fail(AXH_ERR_QUEUE_SUBMIT, "hipEventElapsedTime failed");
  *ns = (uint64_t)((double)ms * 1e6 / calls);
  return AXH_OK;
}

// The assignment of one enumerated variant (values in sorted key order).
axh_q4_variant assignment(const Q4kTuneCtx &t, const int64_t *v) {
  axh_q4_variant r{};
  for (size_t k = 0; k < t.keys.size(); ++k) {
    const uint32_t val = (uint32_t)v[k];
    const std::string &n = t.keys[k];
    if (n == "family") r.family = val;
    else if (n == "nontemporal") r.nontemporal = val;
    else if (n == "prefetch") r.prefetch = val;
    else if (n == "rows_per_wave") r.rows_per_wave = val;
    else if (n == "sb_per_lane") r.sb_per_lane = val;
    else if (n == "waves_per_workgroup") r.waves_per_workgroup = val;
  }
  return r;
}

// A variant is valid for the shape when it plans to a compiled kernel.
bool plans(const Q4kTuneCtx &t, const axh_q4_variant &v, char *err, size_t cap) {
  char name[64];
  if (axh_q4k_matvec_kernel_name(t.n_rows, t.sb, &v, name, sizeof(name)) != AXH_OK) {
    std::snprintf(err, cap, "%s", axh_last_error());
    return false;
  }
  return true;
}

int tune_correct(void *user, uint64_t, const int64_t *vals, uint32_t, char *err, size_t cap) {
  Q4kTuneCtx &t = *static_cast<Q4kTuneCtx *>(user);
  const axh_q4_variant v = assignment(t, vals);
  // An assignment with no kernel for the shape is not judged here: the bench
  // then reports it Failed (grid_search.rs:93-101), not CorrectnessRejected.
  if (!plans(t, v, err, cap)) return 0;
  if (axh_q4k_matvec(t.ctx, t.q, t.x, t.y, t.n_rows, t.sb, &v, nullptr) != AXH_OK ||
      axh_synchronize(t.ctx, nullptr) != AXH_OK ||
      axh_download(t.ctx, t.y_host.data(), t.y, 4u * t.n_rows) != AXH_OK) {
    std::snprintf(err, cap, "%s", axh_last_error());
    return 1;
  }
  axh_check_report rep{};
  if (axh_check_q4k_matvec(t.q_host.data(), t.x_host.data(), t.y_host.data(), t.n_rows, t.sb,
                           t.tol, &rep) != AXH_OK) {
    std::snprintf(err, cap, "%s", axh_check_last_error());
    return 1;
  }
  if (!rep.ok) {
    std::snprintf(err, cap, "checker: %llu of %llu rows beyond %.3g (worst %.3g x allowed)",
                  (unsigned long long)rep.rows_failed, (unsigned long long)rep.rows_checked,
                  t.tol, rep.worst_over_allowed);
    return 1;
  }
  return 0;
}

int tune_bench(void *user, uint64_t, const int64_t *vals, uint32_t, axh_sample_stats *out,
               char *err, size_t cap) {
  Q4kTuneCtx &t = *static_cast<Q4kTuneCtx *>(user);
  const axh_q4_variant v = assignment(t, vals);
  if (!plans(t, v, err, cap)) return 1;
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
    std::snprintf(err, cap, "hipEventCreate failed");
    return 1;
  }
  std::vector<uint64_t> ns(t.samples);
  axh_status st = AXH_OK;
  for (uint32_t smp = 0; smp < t.samples && st == AXH_OK; ++smp)
    st = time_calls(t, v, 20, e0, e1, &ns[smp]);
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  if (st != AXH_OK) {
    std::snprintf(err, cap, "%s", axh_last_error());
    return 1;
  }
  std::sort(ns.begin(), ns.end());
  out->median_ns = ns[ns.size() / 2];
  out->min_ns = ns.front();
  out->max_ns = ns.back();
  out->n_samples = (uint32_t)ns.size();
  return 0;
}

// One family's hole space (candidate lists; the family itself is a
// one-candidate hole so every variant id names its family).
struct Hole {
  const char *name;
  std::vector<int64_t> cand;
};

std::vector<Hole> family_holes(uint32_t fam, uint32_t n_rows, uint32_t nsb) {
  std::vector<Hole> h{{"family", {(int64_t)fam}}};
  switch (fam) {
  case AXH_Q4K_FAMILY_PERSISTENT:
    h.push_back({"nontemporal", {2, 1}});
    h.push_back({"prefetch", {1, 2, 4, 7}});
    h.push_back({"rows_per_wave", {1, 2, 4}});
    h.push_back({"waves_per_workgroup", {4, 8, 16}});
    break;
  case AXH_Q4K_FAMILY_ONE_PASS:
  case AXH_Q4K_FAMILY_ONE_PASS_X: {
    const int64_t need = (nsb + 7) / 8;
    std::vector<int64_t> c{need};
    if (need < 16) c.push_back(need + 1); // a longer trip count than the row needs
    h.push_back({"sb_per_lane", c});
    // x one or two chunks ahead (variants that cannot take it fail to plan)
    if (fam == AXH_Q4K_FAMILY_ONE_PASS) h.push_back({"prefetch", {1, 2}});
    break;
  }
  case AXH_Q4K_FAMILY_WORKGROUP:
    h.push_back({"rows_per_wave", {1, 2, 4}});
    break;
  case AXH_Q4K_FAMILY_TILED:
    h.push_back({"prefetch", {2}});
    h.push_back({"rows_per_wave", {1, 2}});
    h.push_back({"waves_per_workgroup", {4, 8}});
    break;
  default: // split-K, columns: no holes beyond the family
    break;
  }
  (void)n_rows;
  return h;
}
} // namespace

// A family takes the shape when its probe assignment plans to a kernel (the
// persistent family takes every shape).
static bool family_takes(uint32_t fam, uint32_t n_rows, uint32_t nsb) {
  axh_q4_variant probe{};
  probe.family = fam;
  char name[64];
  return fam == AXH_Q4K_FAMILY_PERSISTENT ||
         axh_q4k_matvec_kernel_name(n_rows, nsb, &probe, name, sizeof(name)) == AXH_OK;
}

axh_status axh_q4k_matvec_family_holes(uint32_t family, uint32_t n_rows, uint32_t sb_per_row,
                                       const char **names, uint32_t *n_candidates,
                                       int64_t *candidates, uint32_t cap_holes,
                                       uint32_t cap_candidates, uint32_t *n_holes) {
  if (!n_holes || n_rows == 0 || sb_per_row == 0 || family < AXH_Q4K_FAMILY_PERSISTENT ||
      family > AXH_Q4K_FAMILY_TILED)
    return fail(AXH_ERR_INVALID_ARGUMENT, "family holes: a family 1-7, a shape and n_holes");
  if (!family_takes(family, n_rows, sb_per_row))
    return fail(AXH_ERR_INVALID_ARGUMENT, "the family has no kernel for this shape");
  const std::vector<Hole> hs = family_holes(family, n_rows, sb_per_row);
  *n_holes = (uint32_t)hs.size();
  if (!names) return ok(); // size query
  uint32_t used = 0;
  if (hs.size() > cap_holes || !n_candidates || !candidates)
    return fail(AXH_ERR_INVALID_ARGUMENT, "family holes: arrays too small");
  for (size_t h = 0; h < hs.size(); ++h) {
    if (used + hs[h].cand.size() > cap_candidates)
      return fail(AXH_ERR_INVALID_ARGUMENT, "family holes: candidate array too small");
    names[h] = hs[h].name;
    n_candidates[h] = (uint32_t)hs[h].cand.size();
    for (int64_t c : hs[h].cand) candidates[used++] = c;
  }
  return ok();
}

axh_status axh_q4k_matvec_autotune(axh_context *ctx, const void *q, const float *x, float *y,
                                   uint32_t n_rows, uint32_t sb_per_row, uint32_t samples,
                                   double tol, axh_autotune_report *out) {
  if (!ctx || !out || n_rows == 0 || sb_per_row == 0)
    return fail(AXH_ERR_INVALID_ARGUMENT, "autotune needs a context, a shape and an output");
  std::memset(out, 0, sizeof(*out));
  Q4kTuneCtx t{ctx, q, x, y, n_rows, sb_per_row, samples ? samples : 5, tol > 0 ? tol : 1e-3,
               {}, {}, {}, {}};
  const uint64_t q_bytes = (uint64_t)n_rows * sb_per_row * 144u;
  if (q_bytes > (uint64_t)4 << 30)
    return fail(AXH_ERR_INVALID_ARGUMENT, "autotune: the checker copy is limited to 4 GiB");
  t.q_host.resize(q_bytes);
  t.x_host.resize((size_t)sb_per_row * 256u);
  t.y_host.resize(n_rows);
  axh_status st = axh_download(ctx, t.q_host.data(), q, q_bytes);
  if (st == AXH_OK) st = axh_download(ctx, t.x_host.data(), x, 4u * t.x_host.size());
  if (st != AXH_OK) return st;
  if ((st = axh_q4k_matvec_default_variant(n_rows, sb_per_row, &out->dflt)) != AXH_OK) return st;
  // Rotated copies of q (device to device), released on every return below.
  t.stride = (q_bytes + 255u) / 256u * 256u;
  t.n_copies = (uint32_t)std::min<uint64_t>(kMaxCopies, std::max<uint64_t>(
                                                            1, (kRotateBytes + t.stride - 1) / t.stride));
  if (t.n_copies > 1) {
    void *p = nullptr;
    if ((st = axh_buffer_alloc(ctx, t.stride * (t.n_copies - 1), &p)) != AXH_OK) return st;
    t.copies = static_cast<uint8_t *>(p);
    for (uint32_t c = 1; c < t.n_copies && st == AXH_OK; ++c)
      st = axh_copy_device(ctx, t.copies + (uint64_t)(c - 1) * t.stride, q, q_bytes);
    if (st == AXH_OK) st = axh_synchronize(ctx, nullptr);
  }
  struct Release {
    Q4kTuneCtx &t;
    ~Release() {
      if (t.copies) axh_buffer_free(t.ctx, t.copies);
    }
  } release{t};
  if (st != AXH_OK) return st;
  out->weight_copies = t.n_copies;

  bool have = false;
  for (uint32_t fam = AXH_Q4K_FAMILY_PERSISTENT; fam <= AXH_Q4K_FAMILY_TILED; ++fam) {
    if (!family_takes(fam, n_rows, sb_per_row)) continue; // families without a kernel: skipped
    const std::vector<Hole> hs = family_holes(fam, n_rows, sb_per_row);
    std::vector<axh_strategy_hole> holes;
    for (const Hole &h : hs)
      holes.push_back({h.name, h.cand.data(), (uint32_t)h.cand.size()});
    uint64_t n = 0;
    std::vector<uint32_t> order(holes.size());
    if ((st = axh_enumerate_strategy(holes.data(), (uint32_t)holes.size(), &n, order.data(),
                                     nullptr, nullptr, 0)) != AXH_OK)
      return st;
    t.keys.clear();
    for (uint32_t k : order) t.keys.push_back(holes[k].name);
    std::vector<axh_variant_result> res(n);
    axh_correctness_policy pol{AXH_POLICY_EQUIV_FP_TOL, 0};
    axh_grid_search_result gs{};
    if ((st = axh_grid_search(holes.data(), (uint32_t)holes.size(), &pol, tune_correct,
                              tune_bench, &t, res.data(), n, &gs)) != AXH_OK)
      return st;
    std::vector<int64_t> vals(holes.size() * n);
    axh_enumerate_strategy(holes.data(), (uint32_t)holes.size(), &n, nullptr, vals.data(),
                           nullptr, n);
    out->variants += (uint32_t)n;
    for (uint64_t v = 0; v < n; ++v) {
      const axh_variant_result &r = res[v];
      if (r.outcome == AXH_OUTCOME_OK) ++out->accepted;
      else if (r.outcome == AXH_OUTCOME_CORRECTNESS_REJECTED) ++out->rejected;
      else ++out->failed;
      if (r.outcome != AXH_OUTCOME_OK) continue;
      const axh_q4_variant a = assignment(t, &vals[holes.size() * v]);
      if (std::memcmp(&a, &out->dflt, sizeof(a)) == 0) out->default_median_ns = r.stats.median_ns;
      if (!have || r.stats.median_ns < out->best_median_ns) {
        have = true;
        out->best = a;
        out->best_median_ns = r.stats.median_ns;
      }
    }
  }
  if (!have) return fail((axh_status)AXH_ERR_NO_SUCCESSFUL_VARIANTS, "no variant ran");
  // Confirmation: the sweep's winner against the default in interleaved
  // rounds; a winner that does not beat the default by more than the spread
  // leaves the default in place.
  if (std::memcmp(&out->best, &out->dflt, sizeof(out->best)) != 0 && out->default_median_ns) {
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)
      return fail(AXH_ERR_QUEUE_SUBMIT, "hipEventCreate failed");
    std::vector<uint64_t> tb(kConfirmRounds), td(kConfirmRounds);
    for (uint32_t r = 0; r < kConfirmRounds && st == AXH_OK; ++r) {
      st = time_calls(t, out->best, kConfirmCalls, e0, e1, &tb[r]);
      if (st == AXH_OK) st = time_calls(t, out->dflt, kConfirmCalls, e0, e1, &td[r]);
    }
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (st != AXH_OK) return st;
    std::sort(tb.begin(), tb.end());
    std::sort(td.begin(), td.end());
    out->confirm_best_ns = tb[kConfirmRounds / 2];
    out->confirm_default_ns = td[kConfirmRounds / 2];
    if ((double)out->confirm_best_ns > (1.0 - kConfirmSpread) * (double)out->confirm_default_ns) {
      out->kept_default = 1;
      out->best = out->dflt;
      out->best_median_ns = out->default_median_ns;
    }
  } else {
    out->confirm_best_ns = out->confirm_default_ns = out->best_median_ns;
    out->kept_default = std::memcmp(&out->best, &out->dflt, sizeof(out->best)) == 0;
  }
  if ((st = axh_q4k_matvec_kernel_name(n_rows, sb_per_row, &out->best, out->best_kernel,
                                       sizeof(out->best_kernel))) != AXH_OK)
    return st;
  if ((st = axh_context_winner_put(ctx, "q4k_matvec", n_rows, sb_per_row, &out->best,
                                   out->best_median_ns)) != AXH_OK)
    return st;
  return axh_context_winners_save(ctx);
}

} // extern "C"
