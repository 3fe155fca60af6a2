// Per-shape tuned-winner table: the persistent artefact of an autotune run,
// the counterpart of the reference's strategy sidecar
// (crates/axc-driver/src/optimize.rs:103-128, `<output>.axc.strategy.json`)
// and of its on-disk pipeline cache, which a context loads at creation
// (crates/axc-runtime/src/pipeline_cache.rs:45-100; a file that cannot be
// read is PipelineCacheLoadFailed, pipeline_cache.rs:153-170).
//
// File format (JSON, one object):
//   {"schema": "axh-winners-1",
//    "entries": [{"op": "q4k_matvec", "n_rows": R, "units": U, "family": F,
//                 "rows_per_wave": .., "waves_per_workgroup": .., "prefetch": ..,
//                 "nontemporal": .., "sb_per_lane": .., "median_ns": N}, ...]}
// Every entry field is required and every number a non-negative integer
// below 2^32 (median_ns below 2^63).  Saving writes a temporary file in the
// same directory and renames it over the table.
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <tuple>
#include <vector>

#include <sys/stat.h>
#include <unistd.h>

#include "axh_internal.h"
#include "axh_tune.h"

struct axh_winner_table {
  // (op, n_rows, units) -> (variant, median_ns)
  std::map<std::tuple<std::string, uint32_t, uint32_t>, std::pair<axh_q4_variant, uint64_t>> m;
};

namespace axh {
namespace {

constexpr const char *kSchema = "axh-winners-1";

// Minimal JSON reader for the table's shape: objects, arrays, strings
// without escapes other than \" and \\, and non-negative integers.
struct Reader {
  const char *p, *end;
  bool ok = true;
  void ws() {
    while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
  }
  bool eat(char c) {
    ws();
    if (p < end && *p == c) {
      ++p;
      return true;
    }
    return false;
  }
  bool expect(char c) {
    if (!eat(c)) ok = false;
    return ok;
  }
  bool str(std::string *out) {
    ws();
    if (p >= end || *p != '"') return ok = false;
    ++p;
    out->clear();
    while (p < end && *p != '"') {
      char c = *p++;
      if (c == '\\') {
        if (p >= end || (*p != '"' && *p != '\\')) return ok = false;
        c = *p++;
      } else if ((unsigned char)c < 0x20) {
        return ok = false;
      }
      out->push_back(c);
    }
    if (p >= end) return ok = false;
    ++p;
    return true;
  }
  bool num(uint64_t *out, uint64_t max) {
    ws();
    if (p >= end || *p < '0' || *p > '9') return ok = false;
    uint64_t v = 0;
    while (p < end && *p >= '0' && *p <= '9') {
      const uint64_t d = (uint64_t)(*p++ - '0');
      if (v > (max - d) / 10u) return ok = false;
      v = v * 10u + d;
    }
    *out = v;
    return true;
  }
};

bool parse_entry(Reader &r, axh_winner_table *t) {
  if (!r.expect('{')) return false;
  std::string op;
  uint64_t vals[8] = {};
  bool seen[9] = {};
  static const char *kNum[8] = {"n_rows",  "units",       "family",    "rows_per_wave",
                                "waves_per_workgroup", "prefetch", "nontemporal", "sb_per_lane"};
  uint64_t median = 0;
  bool have_median = false, first = true;
  while (!r.eat('}')) {
    if (!first && !r.expect(',')) return false;
    first = false;
    std::string key;
    if (!r.str(&key) || !r.expect(':')) return false;
    if (key == "op") {
      if (seen[8] || !r.str(&op)) return r.ok = false;
      seen[8] = true;
      continue;
    }
    if (key == "median_ns") {
      if (have_median || !r.num(&median, (uint64_t)INT64_MAX)) return r.ok = false;
      have_median = true;
      continue;
    }
    int k = -1;
    for (int i = 0; i < 8; ++i)
      if (key == kNum[i]) k = i;
    if (k < 0 || seen[k] || !r.num(&vals[k], 0xFFFFFFFFull)) return r.ok = false;
    seen[k] = true;
  }
  for (bool s : seen)
    if (!s) return r.ok = false;
  if (!have_median) return r.ok = false;
  axh_q4_variant v{};
  v.family = (uint32_t)vals[2];
  v.rows_per_wave = (uint32_t)vals[3];
  v.waves_per_workgroup = (uint32_t)vals[4];
  v.prefetch = (uint32_t)vals[5];
  v.nontemporal = (uint32_t)vals[6];
  v.sb_per_lane = (uint32_t)vals[7];
  t->m[std::make_tuple(op, (uint32_t)vals[0], (uint32_t)vals[1])] = {v, median};
  return true;
}

axh_status parse_table(const std::string &text, axh_winner_table *t, std::string *why) {
  Reader r{text.data(), text.data() + text.size()};
  bool have_schema = false, have_entries = false, first = true;
  if (!r.expect('{')) {
    *why = "not a JSON object";
    return AXH_ERR_CODE_OBJECT_CACHE_LOAD;
  }
  while (r.ok && !r.eat('}')) {
    if (!first && !r.expect(',')) break;
    first = false;
    std::string key;
    if (!r.str(&key) || !r.expect(':')) break;
    if (key == "schema") {
      std::string s;
      if (!r.str(&s)) break;
      if (s != kSchema) {
        *why = "schema '" + s + "' is not " + kSchema;
        return AXH_ERR_CODE_OBJECT_CACHE_LOAD;
      }
      have_schema = true;
    } else if (key == "entries") {
      if (!r.expect('[')) break;
      bool f2 = true;
      while (r.ok && !r.eat(']')) {
        if (!f2 && !r.expect(',')) break;
        f2 = false;
        if (!parse_entry(r, t)) break;
      }
      have_entries = r.ok;
    } else {
      r.ok = false;
    }
  }
  r.ws();
  if (!r.ok || r.p != r.end || !have_schema || !have_entries) {
    *why = "malformed winner table at byte " + std::to_string(r.p - text.data());
    t->m.clear();
    return AXH_ERR_CODE_OBJECT_CACHE_LOAD;
  }
  return AXH_OK;
}

std::string quote(const std::string &s) {
  std::string o = "\"";
  for (char c : s) {
    if (c == '"' || c == '\\') o.push_back('\\');
    o.push_back(c);
  }
  return o + "\"";
}

bool valid_op(const char *op) {
  if (!op || !*op) return false;
  for (const char *c = op; *c; ++c)
    if ((unsigned char)*c < 0x20) return false;
  return true;
}

} // namespace
} // namespace axh

using namespace axh;

extern "C" {

axh_winner_table *axh_winners_new(void) { return new axh_winner_table(); }

void axh_winners_free(axh_winner_table *t) { delete t; }

uint64_t axh_winners_count(const axh_winner_table *t) { return t ? t->m.size() : 0u; }

axh_status axh_winners_load(const char *path, axh_winner_table **out) {
  if (!path || !out) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  *out = nullptr;
  FILE *f = std::fopen(path, "rb");
  if (!f) {
    if (errno == ENOENT) { // first run: an empty table
      *out = new axh_winner_table();
      return ok();
    }
    return fail(AXH_ERR_CODE_OBJECT_CACHE_LOAD,
                std::string("cannot read winner table ") + path + ": " + std::strerror(errno));
  }
  std::string text;
  char buf[4096];
  size_t n;
  while ((n = std::fread(buf, 1, sizeof(buf), f)) > 0) {
    text.append(buf, n);
    if (text.size() > (64u << 20)) break;
  }
  const bool err = std::ferror(f) != 0;
  std::fclose(f);
  if (err || text.size() > (64u << 20))
    return fail(AXH_ERR_CODE_OBJECT_CACHE_LOAD, std::string("cannot read winner table ") + path);
  auto *t = new axh_winner_table();
  std::string why;
  const axh_status s = parse_table(text, t, &why);
  if (s != AXH_OK) {
    delete t;
    return fail(s, std::string("winner table ") + path + ": " + why);
  }
  *out = t;
  return ok();
}

axh_status axh_winners_save(const axh_winner_table *t, const char *path) {
  if (!t || !path) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  std::string o = std::string("{\"schema\": \"") + kSchema + "\",\n \"entries\": [";
  bool first = true;
  for (const auto &kv : t->m) {
    const axh_q4_variant &v = kv.second.first;
    char line[512];
    std::snprintf(line, sizeof(line),
                  "\"n_rows\": %u, \"units\": %u, \"family\": %u, \"rows_per_wave\": %u, "
                  "\"waves_per_workgroup\": %u, \"prefetch\": %u, \"nontemporal\": %u, "
                  "\"sb_per_lane\": %u, \"median_ns\": %llu}",
                  std::get<1>(kv.first), std::get<2>(kv.first), v.family, v.rows_per_wave,
                  v.waves_per_workgroup, v.prefetch, v.nontemporal, v.sb_per_lane,
                  (unsigned long long)kv.second.second);
    o += first ? "\n  {\"op\": " : ",\n  {\"op\": ";
    o += quote(std::get<0>(kv.first)) + ", " + line;
    first = false;
  }
  o += "\n ]}\n";
  const std::string tmp = std::string(path) + ".tmp." + std::to_string((long)getpid());
  FILE *f = std::fopen(tmp.c_str(), "wb");
  if (!f)
    return fail(AXH_ERR_CODE_OBJECT_CACHE_LOAD,
                "cannot write " + tmp + ": " + std::strerror(errno));
  const bool wrote = std::fwrite(o.data(), 1, o.size(), f) == o.size();
  const bool closed = std::fclose(f) == 0;
  if (!wrote || !closed || std::rename(tmp.c_str(), path) != 0) {
    std::remove(tmp.c_str());
    return fail(AXH_ERR_CODE_OBJECT_CACHE_LOAD, std::string("cannot save winner table ") + path);
  }
  return ok();
}

axh_status axh_winners_put(axh_winner_table *t, const char *op, uint32_t n_rows, uint32_t units,
                           const axh_q4_variant *v, uint64_t median_ns) {
  if (!t || !v || !valid_op(op)) return fail(AXH_ERR_INVALID_ARGUMENT, "bad winner entry");
  t->m[std::make_tuple(std::string(op), n_rows, units)] = {*v, median_ns};
  return ok();
}

axh_status axh_winners_get(const axh_winner_table *t, const char *op, uint32_t n_rows,
                           uint32_t units, uint32_t *found, axh_q4_variant *v,
                           uint64_t *median_ns) {
  if (!t || !op || !found) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  auto it = t->m.find(std::make_tuple(std::string(op), n_rows, units));
  *found = it != t->m.end() ? 1u : 0u;
  if (*found) {
    if (v) *v = it->second.first;
    if (median_ns) *median_ns = it->second.second;
  }
  return ok();
}

} // extern "C"

// ---- the context's table ------------------------------------------------------
namespace axh {

bool lookup_winner(axh_context *ctx, const char *op, uint32_t n_rows, uint32_t units,
                   axh_q4_variant *out) {
  if (!ctx || !ctx->has_winners.load(std::memory_order_acquire)) return false;
  std::lock_guard<std::mutex> lk(ctx->winners_mu);
  auto it = ctx->winners->m.find(std::make_tuple(std::string(op), n_rows, units));
  if (it == ctx->winners->m.end()) return false;
  *out = it->second.first;
  return true;
}

// Called by axh_context_create: the table of `dir`, or an empty one.
void winners_attach(axh_context *ctx, const std::string &dir) {
  const char *dis = std::getenv("AXH_DISABLE_CODE_OBJECT_CACHE");
  const bool disabled = dis && std::strcmp(dis, "1") == 0;
  axh_winner_table *t = nullptr;
  if (!dir.empty() && !disabled) {
    ctx->winners_path = dir + "/axh_winners.json";
    if (axh_winners_load(ctx->winners_path.c_str(), &t) != AXH_OK) {
      std::fprintf(stderr, "axh: %s; starting with an empty winner table\n", axh_last_error());
      t = nullptr;
    }
  }
  ctx->winners = t ? t : new axh_winner_table();
  ctx->has_winners = !ctx->winners->m.empty();
}

void winners_detach(axh_context *ctx) {
  delete ctx->winners;
  ctx->winners = nullptr;
}

} // namespace axh

extern "C" {

axh_status axh_context_winner_put(axh_context *ctx, const char *op, uint32_t n_rows,
                                  uint32_t units, const axh_q4_variant *v, uint64_t median_ns) {
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  std::lock_guard<std::mutex> lk(ctx->winners_mu);
  const axh_status s = axh_winners_put(ctx->winners, op, n_rows, units, v, median_ns);
  if (s == AXH_OK) ctx->has_winners.store(true, std::memory_order_release);
  return s;
}

axh_status axh_context_winner_get(axh_context *ctx, const char *op, uint32_t n_rows,
                                  uint32_t units, uint32_t *found, axh_q4_variant *v,
                                  uint64_t *median_ns) {
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  std::lock_guard<std::mutex> lk(ctx->winners_mu);
  return axh_winners_get(ctx->winners, op, n_rows, units, found, v, median_ns);
}

axh_status axh_context_winners_save(axh_context *ctx) {
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  if (ctx->winners_path.empty()) return ok();
  const std::string dir = ctx->winners_path.substr(0, ctx->winners_path.rfind('/'));
  if (mkdir(dir.c_str(), 0755) != 0 && errno != EEXIST)
    return fail(AXH_ERR_CODE_OBJECT_CACHE_LOAD, "cannot create " + dir + ": " + std::strerror(errno));
  std::lock_guard<std::mutex> lk(ctx->winners_mu);
  return axh_winners_save(ctx->winners, ctx->winners_path.c_str());
}

const char *axh_context_winners_path(const axh_context *ctx) {
  return ctx ? ctx->winners_path.c_str() : "";
}

} // extern "C"
