// Per-op profiler and its JSON report (src/profiler/profiler.cc:25-176).
//
//  - percentile(): linear interpolation between the closest ranks, numpy's
//    default ("type 7"; profiler.cc:25-37).
//  - stats_from(): mean, p50, p95, min, max of a sample (profiler.cc:39-49).
//  - Per-op-type statistics are taken over per-iteration sums of that type's
//    op times (profiler.cc:104-118); op counts come from the first iteration
//    (:120-125); the activation peak is the largest activation_bytes_after
//    of any op (:60-65, 127-133).
//  - to_json() writes the report's schema (profiler.cc:138-176): keys
//    sorted, two-space indent, non-finite numbers as null.
//  - Peak RSS is the process's maximum resident set (getrusage ru_maxrss),
//    the Linux counterpart of mach resident_size_max (profiler.cc:94-101).
#include <sys/resource.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <sstream>

#include "common.h"
#include "profiler.h"

namespace ih {
namespace prof {

double percentile(std::vector<double> v, double p) {
  if (v.empty()) return 0.0;
  std::sort(v.begin(), v.end());
  if (v.size() == 1) return v[0];
  const double rank = (p / 100.0) * double(v.size() - 1);
  const size_t lo = size_t(std::floor(rank));
  const size_t hi = size_t(std::ceil(rank));
  if (lo == hi) return v[lo];
  return v[lo] + (rank - double(lo)) * (v[hi] - v[lo]);
}

inferc_profiler::Stats stats_from(const std::vector<double>& v) {
  inferc_profiler::Stats s;
  if (v.empty()) return s;
  double sum = 0.0;
  s.min = s.max = v[0];
  for (double x : v) {
    sum += x;
    s.min = std::min(s.min, x);
    s.max = std::max(s.max, x);
  }
  s.mean = sum / double(v.size());
  s.p50 = percentile(v, 50.0);
  s.p95 = percentile(v, 95.0);
  return s;
}

}  // namespace prof

namespace {

double ms_between(inferc_profiler::clock::time_point a, inferc_profiler::clock::time_point b) {
  return std::chrono::duration<double, std::milli>(b - a).count();
}

// Shortest decimal form that reads back to the same double; integral values
// keep a ".0" so that readers see a floating-point field.
std::string json_number(double x) {
  if (!std::isfinite(x)) return "null";
  char b[40];
  for (int prec = 1; prec <= 17; ++prec) {
    std::snprintf(b, sizeof b, "%.*g", prec, x);
    if (std::strtod(b, nullptr) == x) break;
  }
  std::string s(b);
  if (s.find_first_of(".eE") == std::string::npos) s += ".0";
  return s;
}

std::string json_string(const std::string& s) {
  std::string o = "\"";
  for (unsigned char c : s) {
    switch (c) {
      case '"': o += "\\\""; break;
      case '\\': o += "\\\\"; break;
      case '\b': o += "\\b"; break;
      case '\f': o += "\\f"; break;
      case '\n': o += "\\n"; break;
      case '\r': o += "\\r"; break;
      case '\t': o += "\\t"; break;
      default:
        if (c < 0x20) {
          char u[8];
          std::snprintf(u, sizeof u, "\\u%04x", c);
          o += u;
        } else {
          o += char(c);
        }
    }
  }
  return o + "\"";
}

// A JSON object whose members are already-serialised values, printed with
// sorted keys and a two-space indent.
struct JObj {
  std::map<std::string, std::string> m;
  void put(const std::string& k, std::string v) { m[k] = std::move(v); }
  std::string dump(int depth) const {
    if (m.empty()) return "{}";
    const std::string pad(size_t(2 * (depth + 1)), ' ');
    std::string o = "{\n";
    size_t i = 0;
    for (const auto& kv : m) {
      o += pad + json_string(kv.first) + ": " + kv.second;
      o += (++i < m.size()) ? ",\n" : "\n";
    }
    return o + std::string(size_t(2 * depth), ' ') + "}";
  }
};

std::string stats_json(const inferc_profiler::Stats& s, int depth) {
  JObj o;
  o.put("mean_ms", json_number(s.mean));
  o.put("p50_ms", json_number(s.p50));
  o.put("p95_ms", json_number(s.p95));
  o.put("min_ms", json_number(s.min));
  o.put("max_ms", json_number(s.max));
  return o.dump(depth);
}

}  // namespace
}  // namespace ih

void inferc_profiler::begin_iteration() {
  cur = Iter{};
  in_iteration = true;
  op_in_flight = false;
  iter_t0 = clock::now();
}

void inferc_profiler::end_iteration(double total_ms) {
  const auto t1 = clock::now();
  IH_REQUIRE(in_iteration, INFERC_ERR_STATE, "Profiler: EndIteration without BeginIteration");
  IH_REQUIRE(!op_in_flight, INFERC_ERR_STATE, "Profiler: EndIteration while an op is in flight");
  cur.total_ms = total_ms >= 0.0 ? total_ms : ih::ms_between(iter_t0, t1);
  for (const auto& r : cur.ops) cur.activation_peak = std::max(cur.activation_peak, r.activation_bytes_after);
  iters.push_back(std::move(cur));
  cur = Iter{};
  in_iteration = false;
}

void inferc_profiler::begin_op(std::string op_type, std::string node_name) {
  IH_REQUIRE(!op_in_flight, INFERC_ERR_STATE,
             "Profiler: BeginOp called while another op is in flight");
  pending = Op{};
  pending.op_type = std::move(op_type);
  pending.node_name = std::move(node_name);
  op_in_flight = true;
  op_t0 = clock::now();
}

void inferc_profiler::end_op(int64_t activation_bytes_after) {
  const auto t1 = clock::now();
  IH_REQUIRE(op_in_flight, INFERC_ERR_STATE, "Profiler: EndOp called without BeginOp");
  pending.ms = ih::ms_between(op_t0, t1);
  pending.activation_bytes_after = activation_bytes_after;
  cur.ops.push_back(std::move(pending));
  op_in_flight = false;
}

void inferc_profiler::add_op(std::string op_type, std::string node_name, double ms,
                             int64_t activation_bytes_after) {
  IH_REQUIRE(!op_in_flight, INFERC_ERR_STATE, "Profiler: an op is in flight");
  Op r;
  r.op_type = std::move(op_type);
  r.node_name = std::move(node_name);
  r.ms = ms;
  r.activation_bytes_after = activation_bytes_after;
  cur.ops.push_back(std::move(r));
}

void inferc_profiler::snapshot_peak_rss() {
  struct rusage ru {};
  if (getrusage(RUSAGE_SELF, &ru) == 0) peak_rss_bytes = int64_t(ru.ru_maxrss) * 1024;
}

inferc_profiler::Stats inferc_profiler::total_stats() const {
  std::vector<double> v;
  v.reserve(iters.size());
  for (const auto& it : iters) v.push_back(it.total_ms);
  return ih::prof::stats_from(v);
}

std::map<std::string, inferc_profiler::Stats> inferc_profiler::per_op_type_stats() const {
  std::map<std::string, std::vector<double>> by_op;
  for (const auto& it : iters) {
    std::map<std::string, double> sums;
    for (const auto& r : it.ops) sums[r.op_type] += r.ms;
    for (const auto& kv : sums) by_op[kv.first].push_back(kv.second);
  }
  std::map<std::string, Stats> out;
  for (const auto& kv : by_op) out[kv.first] = ih::prof::stats_from(kv.second);
  return out;
}

std::map<std::string, int64_t> inferc_profiler::op_counts_per_iter() const {
  std::map<std::string, int64_t> out;
  if (iters.empty()) return out;
  for (const auto& r : iters.front().ops) ++out[r.op_type];
  return out;
}

int64_t inferc_profiler::activation_peak_bytes() const {
  int64_t peak = 0;
  for (const auto& it : iters) peak = std::max(peak, it.activation_peak);
  return peak;
}

std::string inferc_profiler::to_json(const std::string& backend, const std::string& model) const {
  using ih::JObj;
  JObj j;
  j.put("backend", ih::json_string(backend));
  j.put("model", ih::json_string(model));
  j.put("iterations", std::to_string(iters.size()));
  j.put("total", ih::stats_json(total_stats(), 1));
  const auto counts = op_counts_per_iter();
  JObj per_op;
  for (const auto& kv : per_op_type_stats()) {
    JObj e;
    auto c = counts.find(kv.first);
    e.put("calls_per_iter", std::to_string(c == counts.end() ? 0 : c->second));
    e.put("total_ms", ih::stats_json(kv.second, 3));
    per_op.put(kv.first, e.dump(2));
  }
  j.put("per_op_type", per_op.dump(1));
  JObj oc;
  for (const auto& kv : counts) oc.put(kv.first, std::to_string(kv.second));
  j.put("op_counts", oc.dump(1));
  j.put("peak_rss_bytes", std::to_string(peak_rss_bytes));
  j.put("activation_bytes_peak", std::to_string(activation_peak_bytes()));
  return j.dump(0);
}

namespace {

inferc_profiler* check_prof(inferc_profiler* p) {
  IH_REQUIRE(p != nullptr, INFERC_ERR_ARG, "null profiler");
  return p;
}

std::vector<double> read_sample(const double* v, int64_t n) {
  IH_REQUIRE(n >= 0, INFERC_ERR_ARG, "negative sample size");
  IH_REQUIRE(n == 0 || v != nullptr, INFERC_ERR_ARG, "null sample");
  return std::vector<double>(v, v + n);
}

void put_stats(const inferc_profiler::Stats& s, double* out5) {
  IH_REQUIRE(out5 != nullptr, INFERC_ERR_ARG, "null output");
  out5[0] = s.mean;
  out5[1] = s.p50;
  out5[2] = s.p95;
  out5[3] = s.min;
  out5[4] = s.max;
}

}  // namespace

extern "C" {

int inferc_profile_percentile(const double* v, int64_t n, double p, double* out) {
  return ih::guard([&] {
    IH_REQUIRE(out != nullptr, INFERC_ERR_ARG, "null output");
    *out = ih::prof::percentile(read_sample(v, n), p);
  });
}

int inferc_profile_stats(const double* v, int64_t n, double* out5) {
  return ih::guard([&] { put_stats(ih::prof::stats_from(read_sample(v, n)), out5); });
}

int inferc_profiler_create(inferc_profiler** out) {
  return ih::guard([&] {
    IH_REQUIRE(out != nullptr, INFERC_ERR_ARG, "null output pointer");
    *out = new inferc_profiler();
  });
}

int inferc_profiler_destroy(inferc_profiler* p) {
  return ih::guard([&] { delete p; });
}

int inferc_profiler_begin_iteration(inferc_profiler* p) {
  return ih::guard([&] { check_prof(p)->begin_iteration(); });
}

int inferc_profiler_end_iteration(inferc_profiler* p) {
  return ih::guard([&] { check_prof(p)->end_iteration(); });
}

int inferc_profiler_begin_op(inferc_profiler* p, const char* op_type, const char* node_name) {
  return ih::guard([&] {
    IH_REQUIRE(op_type != nullptr, INFERC_ERR_ARG, "null op type");
    check_prof(p)->begin_op(op_type, node_name ? node_name : "");
  });
}

int inferc_profiler_end_op(inferc_profiler* p, int64_t activation_bytes_after) {
  return ih::guard([&] { check_prof(p)->end_op(activation_bytes_after); });
}

int inferc_profiler_record_op(inferc_profiler* p, const char* op_type, const char* node_name,
                              double ms, int64_t activation_bytes_after) {
  return ih::guard([&] {
    IH_REQUIRE(op_type != nullptr, INFERC_ERR_ARG, "null op type");
    check_prof(p)->add_op(op_type, node_name ? node_name : "", ms, activation_bytes_after);
  });
}

int inferc_profiler_set_track_activation_bytes(inferc_profiler* p, int on) {
  return ih::guard([&] { check_prof(p)->track_activation_bytes = on != 0; });
}

int inferc_profiler_snapshot_peak_rss(inferc_profiler* p) {
  return ih::guard([&] { check_prof(p)->snapshot_peak_rss(); });
}

int inferc_profiler_iteration_count(inferc_profiler* p, int64_t* n) {
  return ih::guard([&] {
    IH_REQUIRE(n != nullptr, INFERC_ERR_ARG, "null output");
    *n = int64_t(check_prof(p)->iters.size());
  });
}

int inferc_profiler_total_stats(inferc_profiler* p, double* out5) {
  return ih::guard([&] { put_stats(check_prof(p)->total_stats(), out5); });
}

int inferc_profiler_to_json(inferc_profiler* p, const char* backend, const char* model,
                            char* buf, size_t capacity, size_t* len) {
  return ih::guard([&] {
    IH_REQUIRE(len != nullptr, INFERC_ERR_ARG, "null length pointer");
    const std::string s =
        check_prof(p)->to_json(backend ? backend : "", model ? model : "");
    *len = s.size();
    if (buf == nullptr) return;
    IH_REQUIRE(capacity > s.size(), INFERC_ERR_ARG,
               "JSON buffer too small: need " + std::to_string(s.size() + 1) + " bytes");
    std::memcpy(buf, s.c_str(), s.size() + 1);
  });
}

}  // extern "C"
