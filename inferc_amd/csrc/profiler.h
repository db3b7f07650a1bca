// Per-op profiler behind the inferc_profiler_* entry points: the records,
// statistics and JSON report of prof::Profiler (src/profiler/profiler.h:14-89,
// profiler.cc:25-176), with one addition for a device executor: an op's time
// may be given directly (measured between two HIP events on the stream)
// instead of by the host clock between begin_op and end_op.
//
// Host-only code; not part of the C-ABI.
#pragma once

#include <chrono>
#include <cstdint>
#include <map>
#include <string>
#include <vector>

struct inferc_profiler {
  using clock = std::chrono::steady_clock;

  struct Op {  // prof::OpRecord (profiler.h:15-20)
    std::string op_type, node_name;
    double ms = 0.0;
    int64_t activation_bytes_after = 0;
  };
  struct Iter {  // prof::IterRecord (profiler.h:23-27)
    double total_ms = 0.0;
    std::vector<Op> ops;
    int64_t activation_peak = 0;
  };
  struct Stats {  // prof::Stats (profiler.h:29-35)
    double mean = 0.0, p50 = 0.0, p95 = 0.0, min = 0.0, max = 0.0;
  };

  std::vector<Iter> iters;
  Iter cur;
  bool in_iteration = false;
  bool op_in_flight = false;
  Op pending;
  clock::time_point iter_t0{}, op_t0{};
  int64_t peak_rss_bytes = 0;
  bool track_activation_bytes = true;

  void begin_iteration();
  // Ends the iteration; its total is the host time since begin_iteration
  // unless `total_ms` is given (>= 0).
  void end_iteration(double total_ms = -1.0);
  void begin_op(std::string op_type, std::string node_name);
  void end_op(int64_t activation_bytes_after);
  // A finished op whose time was measured elsewhere (device events).
  void add_op(std::string op_type, std::string node_name, double ms,
              int64_t activation_bytes_after);
  void snapshot_peak_rss();

  Stats total_stats() const;
  std::map<std::string, Stats> per_op_type_stats() const;
  std::map<std::string, int64_t> op_counts_per_iter() const;
  int64_t activation_peak_bytes() const;
  std::string to_json(const std::string& backend, const std::string& model) const;
};

namespace ih {
namespace prof {

double percentile(std::vector<double> v, double p);
inferc_profiler::Stats stats_from(const std::vector<double>& v);

}  // namespace prof
}  // namespace ih
