// Graph executor: the device counterpart of rt::Executor
// (src/runtime/executor.h:24-41, executor.cc:89-366).
//
//  - The constructor uploads every initializer to the device once
//    (executor.cc:89-96) and keeps a host copy for shape plumbing.
//  - run() walks the nodes in order and dispatches each op_type to a kernel
//    (executor.cc:123-352); multi-output ops (Split, FusedQKV) bind every
//    output. Unsupported ops fail with INFERC_ERR_UNSUPPORTED
//    (executor.cc:340-343); missing tensors with INFERC_ERR_STATE (:104-110).
//  - Integer shape plumbing (Shape, Gather/Range/Slice/Unsqueeze/Concat on
//    int64 data known on the host) is evaluated on the host; its results are
//    uploaded only if a device kernel consumes them.
//  - Peephole fusion at construction: MatMul -> Add(bias) -> Add(residual)
//    with single-use intermediates becomes one GEMM with a bias+residual
//    epilogue, and Gemm -> Relu one GEMM with a ReLU epilogue. The arithmetic
//    is the unfused sequence's, (acc + b) + r, in the same order.
//  - Activation buffers live in a per-executor arena keyed by tensor name, so
//    repeated runs with the same input shapes touch no allocator; the second
//    such run is captured into a HIP graph that later runs replay.
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <set>
#include <unordered_set>
#include <sstream>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.h"
#include "ew.h"
#include "graph.h"
#include "profiler.h"


namespace ih {
namespace {

size_t dtype_size(int dt) {
  switch (dt) {
    case INFERC_DT_F32: return 4;
    case INFERC_DT_U8: return 1;
    case INFERC_DT_BOOL: return 1;
    case INFERC_DT_I32: return 4;
    case INFERC_DT_I64: return 8;
    default: fail(INFERC_ERR_UNSUPPORTED, "unsupported dtype code " + std::to_string(dt));
  }
}

int64_t numel_of(const std::vector<int64_t>& s) {
  int64_t n = 1;
  for (int64_t d : s) n *= d;
  return n;
}

// A tensor during a run: device data and/or a host copy (initializers and
// host-evaluated shape math).
struct Value {
  int dtype = 0;
  std::vector<int64_t> shape;
  void* dev = nullptr;
  std::shared_ptr<std::vector<uint8_t>> host;  // set when known on the host
  int64_t numel() const { return numel_of(shape); }
  size_t bytes() const { return size_t(numel()) * dtype_size(dtype); }
  const float* f32() const { return static_cast<const float*>(dev); }
  template <class T>
  T host_at(int64_t i) const {
    return reinterpret_cast<const T*>(host->data())[i];
  }
};

int64_t attr_int(const inferc_graph::Node& n, const char* key, int64_t def) {
  auto it = n.attrs.find(key);
  if (it == n.attrs.end()) return def;
  return std::stoll(it->second);
}

// A float as attribute text that reads back to the same float.
std::string float_text(float f) {
  char b[32];
  std::snprintf(b, sizeof b, "%.9g", double(f));
  return b;
}

float attr_float(const inferc_graph::Node& n, const char* key, float def) {
  auto it = n.attrs.find(key);
  if (it == n.attrs.end()) return def;
  return std::stof(it->second);
}

std::vector<int64_t> attr_ints(const inferc_graph::Node& n, const char* key) {
  std::vector<int64_t> v;
  auto it = n.attrs.find(key);
  if (it == n.attrs.end() || it->second.empty()) return v;
  std::stringstream ss(it->second);
  std::string tok;
  while (std::getline(ss, tok, ',')) v.push_back(std::stoll(tok));
  return v;
}

// Mask strides of `in_shape` right-aligned against [B,nH,S,S], 0 on
// broadcast axes (src/kernels/attention.cc:17-29).
void mask_strides(const std::vector<int64_t>& in_shape, int64_t s[4]) {
  s[0] = s[1] = s[2] = s[3] = 0;
  int64_t st = 1;
  const int r = int(in_shape.size());
  for (int i = r - 1; i >= 0; --i) {
    const int od = 4 - (r - i);
    if (od >= 0) s[od] = (in_shape[size_t(i)] == 1) ? 0 : st;
    st *= in_shape[size_t(i)];
  }
}

}  // namespace
}  // namespace ih

struct inferc_executor {
  inferc_hip_ctx* ctx = nullptr;
  std::vector<inferc_graph::Node> nodes;
  std::vector<std::string> outputs;
  std::unordered_map<std::string, ih::Value> inits;
  std::vector<void*> init_allocs;
  struct Input {
    ih::Value v;
    bool from_host = false;
    std::vector<uint8_t> staged;  // host bytes, uploaded when set (dirty)
    bool dirty = false;
    size_t cap = 0;               // bytes of the device buffer of a host input
  };
  std::unordered_map<std::string, Input> inputs;
  std::unordered_map<std::string, ih::Value> vals;  // the "tape" of the last run
  // Outputs of Constant nodes, computed by the first unprofiled run and kept:
  // later runs skip those nodes (const_done[i] for node i).
  std::unordered_map<std::string, ih::Value> consts;
  std::vector<char> const_done;
  struct Buf {
    void* p = nullptr;
    size_t bytes = 0;
  };
  std::unordered_map<std::string, Buf> arena;
  std::unordered_map<std::string, int> fused_act;  // Gemm name -> folded activation
  bool graph_mode = true;
  // Dry run: shape inference and peephole only, no device (host-logic tests).
  bool dry = false;
  uintptr_t dry_next = 0x10000;
  std::string last_key;  // run_key() of the last unrecorded (planning) pass
  // Recorded runs by run_key(), the most recently used last. A recording is
  // replayed only while the workspace, the GEMV route and every executor
  // buffer it names are still the ones it was recorded with: input buffers
  // through the key (their addresses are part of it), the arena and the KV
  // caches through buf_gen.
  // With each recording, the value table its pass left (shapes and buffers of
  // every tensor), which outputs are read through after a replay.
  struct CacheView {
    const float* base = nullptr;
    int64_t rows = 0, T = 0, dh = 0, max_t = 0;
  };
  struct Recorded {
    std::string key;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    uint64_t ws_gen = 0, route_gen = 0, buf_gen = 0;
    std::unordered_map<std::string, ih::Value> vals;
    std::map<std::string, CacheView> views;
  };
  static constexpr size_t kMaxRecorded = 4;
  std::vector<Recorded> recorded;
  uint64_t buf_gen = 0;         // bumped before an arena or KV-cache buffer is freed
  uint64_t plan_route_gen = 0;  // the GEMV route the last planning pass saw
  // A LayerNorm whose input h comes from a FusedGemmEpilogue and whose
  // readers are all GEMM operands (A of FusedQKV / FusedMatMulAddGELU /
  // FusedGemmEpilogue, the residual of a FusedGemmEpilogue): peephole lists
  // the readers by h, and
  // each run decides at the producer whether they read h through the
  // LayerNorm (the small-M GEMM path for every product involved) instead of
  // the LayerNorm kernel writing its output.
  struct LnRead {
    std::string out;  // the LayerNorm's output
    std::string gamma, beta;
    float eps = 1e-5f;
    std::vector<std::pair<size_t, char>> readers;  // node index, 'a' (A) or 'r' (R)
  };
  std::unordered_map<std::string, LnRead> ln_reads;  // by h
  std::unordered_map<std::string, bool> ln_on;       // this run, by h
  // Sticky device flag of the gathers whose indices live on the device: set
  // by the kernel on an out-of-range index, read (and cleared) by the calls
  // that wait for the stream, which then fail as Gather does on the host
  // (embedding.cc:63). dev_gather: the last walk launched such a gather.
  int32_t* gather_err = nullptr;
  bool dev_gather = false;
  // Gathers of embedding rows whose one reader is a LayerNorm (its rows or
  // its residual): the LayerNorm kernel gathers the rows itself, so no
  // [rows, feat] copy is written (decided when planning; the indices must
  // turn out to live on the device, else the Gather runs).
  std::unordered_set<std::string> gather_ln;
  struct PendingGather {
    const float* table;
    const int64_t* ids;
    int64_t vocab, feat, n;
  };
  std::unordered_map<std::string, PendingGather> pending_gather;  // this walk
  // Decode mode: the Add of a token-embedding Gather (device ids) and the
  // position-embedding Gather runs as one kernel; the two gathers leave
  // their rows pending for it (embed_gather_at / embed_add_at, by node).
  struct PendingEmbed {
    const float* table;
    int64_t rows, feat, n;
    const int64_t* ids;  // token rows by these device ids; null: rows at the device position
  };
  std::unordered_map<std::string, PendingEmbed> pending_embed;  // this walk
  std::vector<char> embed_gather_at, embed_add_at;
  void materialize_gather(const std::string& name);
  void materialize_embed(const std::string& name);
  // Equals on graph inputs and initializers, each computed by the launch of
  // a LayerNorm before it (by that LayerNorm's output; decided when
  // planning), and the ones done so in this walk.
  std::unordered_map<std::string, size_t> eq_side;
  std::unordered_set<std::string> eq_done;
  // Gather outputs (this walk) whose Gather applied the LayerNorm the
  // peephole had moved into their Gemm reader (a feature-axis gather).
  std::set<std::string> ln_gemm_off;
  void check_gather_err();
  std::vector<hipEvent_t> prof_ev;  // one per node boundary of a profiled pass
  // Device KV caches of FusedAttentionPast nodes (bind_kv_cache): per node,
  // K and V as [B, nH, kv_max_t, dh] and the number of positions held.
  int64_t kv_max_t = 0;
  struct KvCache {
    float* k = nullptr;
    float* v = nullptr;
    int64_t B = 0, nH = 0, dh = 0, len = 0;
  };
  std::map<std::string, KvCache> kv;  // keyed by the node's name
  // present.* outputs that live in a KV cache: name -> (cache, rows held)
  std::map<std::string, CacheView> cache_views;
  std::string vals_key;  // the run_key() of the pass that left vals
  // Decode mode (inferc_executor_set_decode_position): the KV caches hold
  // decode_len positions, a count also kept on the device (decode_pos). A
  // run walks the graph as if the past were empty, with an attention mask of
  // the new positions alone: the attention nodes take the past length from
  // the device (and ignore the mask: all ones), the position-embedding
  // gathers (pos_gathers) add it to their rows, and the walk ends by
  // advancing it. Every step then walks the same graph, and the second one
  // on records the HIP graph that the rest replay.
  bool decode = false;
  int64_t decode_len = 0;
  int64_t decode_step = 0;  // new positions per run (from the last walk)
  int64_t* decode_pos = nullptr;
  // Per node (by index; node names may be empty or repeated): a position
  // gather, and a node whose results decode mode never reads (the attention
  // mask's own arithmetic: the attention nodes ignore the mask there).
  std::vector<char> pos_gather_at, decode_skip_at;
  size_t node_index(const inferc_graph::Node& n) const { return size_t(&n - nodes.data()); }
  void plan_decode(const std::string& mask_input);
  // Decode feedback (inferc_executor_set_decode_feedback): every decode-mode
  // run ends with the arg-max of fb_logits' last row, which becomes input
  // fb_ids' value for the next run (fb_buf[0]) and is recorded at its
  // position (fb_buf[1 + position]), so the steps replay back to back with
  // no host copy between them.
  std::string fb_logits, fb_ids;
  std::string decode_mask;  // decode mode's attention-mask input
  int64_t* fb_buf = nullptr;
  // This walk's LM-head arg-max partials, when its GEMV wrote them.
  const ih::ValIdxPart* fb_parts = nullptr;
  int64_t fb_parts_n = 0;
  std::vector<hipEvent_t> step_ev;  // inferc_executor_run_steps' step timing

  void free_kv() {
    for (auto& c : kv) {
      if (c.second.k) (void)hipFree(c.second.k);
      if (c.second.v) (void)hipFree(c.second.v);
    }
    kv.clear();
  }

  ~inferc_executor() {
    if (dry) return;
    drop_graph();
    free_kv();
    for (hipEvent_t e : prof_ev) (void)hipEventDestroy(e);
    for (auto& kv : arena) (void)hipFree(kv.second.p);
    for (auto& kv : inputs)
      if (kv.second.from_host && kv.second.v.dev) (void)hipFree(kv.second.v.dev);
    for (void* p : init_allocs) (void)hipFree(p);
    if (gather_err) (void)hipFree(gather_err);
    if (decode_pos) (void)hipFree(decode_pos);
    if (fb_buf) (void)hipFree(fb_buf);
    for (hipEvent_t e : step_ev) (void)hipEventDestroy(e);
  }

  static void destroy(Recorded& r) {
    if (r.exec) (void)hipGraphExecDestroy(r.exec);
    if (r.graph) (void)hipGraphDestroy(r.graph);
    r.exec = nullptr;
    r.graph = nullptr;
  }
  // Drops every recording (the caller has drained the stream where a
  // recording may still run).
  void drop_graph() {
    for (Recorded& r : recorded) destroy(r);
    recorded.clear();
  }

  // Device buffer for tensor `name` of at least `bytes`, reused across runs.
  void* fake_ptr(size_t bytes) {
    void* p = reinterpret_cast<void*>(dry_next);
    dry_next += (bytes + 255) / 256 * 256 + 256;
    return p;
  }

  void* buf(const std::string& name, size_t bytes) {
    Buf& b = arena[name];
    if (b.p && b.bytes >= bytes) return b.p;
    if (dry) {
      b.p = fake_ptr(bytes);
      b.bytes = bytes;
      return b.p;
    }
    IH_REQUIRE(!ctx->capturing, INFERC_ERR_STATE, "executor: allocation during graph capture");
    // A buffer that has to grow (a tensor whose shape grows run by run, as
    // the with-past decode's do by one position per step) grows by half
    // again at least, so it is reallocated, with the stream drained, a few
    // times rather than on every run.
    size_t want = bytes;
    if (b.p) {
      IH_HIP(hipStreamSynchronize(ctx->stream));
      ++buf_gen;  // recordings naming this buffer are stale
      IH_HIP(hipFree(b.p));
      b.p = nullptr;
      const size_t grown = b.bytes + b.bytes / 2;
      want = ((grown > bytes ? grown : bytes) + 255) & ~size_t(255);
    }
    IH_HIP(hipMalloc(&b.p, want > 0 ? want : 4));
    b.bytes = want;
    return b.p;
  }

  // A value by name: this run's tape, then the Constant outputs folded by an
  // earlier run, then the initializers (which the tape does not copy).
  const ih::Value* find_val(const std::string& name) const {
    auto it = vals.find(name);
    if (it != vals.end()) return &it->second;
    auto ic = consts.find(name);
    if (ic != consts.end()) return &ic->second;
    auto ii = inits.find(name);
    return ii != inits.end() ? &ii->second : nullptr;
  }
  ih::Value* find_val(const std::string& name) {
    return const_cast<ih::Value*>(static_cast<const inferc_executor*>(this)->find_val(name));
  }
  const ih::Value& get(const std::string& name) const {
    const ih::Value* v = find_val(name);
    if (!v) ih::fail(INFERC_ERR_STATE, "Executor: missing tensor '" + name + "'");
    return *v;
  }

  // Device pointer of a value. Host-only values (shape math consumed by a
  // kernel) are uploaded into the arena once and reused while their bytes
  // stay the same, so a captured run needs no copy. New bytes make the
  // recordings stale (one may read the old ones).
  struct Upload {
    std::vector<uint8_t> bytes;
    void* p = nullptr;
  };
  std::unordered_map<std::string, Upload> uploads;
  void* dev_of(const std::string& name) {
    if (!pending_embed.empty()) materialize_embed(name);  // (a reader the plan did not expect)
    ih::Value* vp = find_val(name);
    if (!vp) ih::fail(INFERC_ERR_STATE, "Executor: missing tensor '" + name + "'");
    ih::Value& v = *vp;
    if (v.dev) return v.dev;
    IH_REQUIRE(v.host != nullptr, INFERC_ERR_STATE, "tensor '" + name + "' has no data");
    Upload& up = uploads[name];
    if (up.p && up.bytes == *v.host) {
      v.dev = up.p;
      return up.p;
    }
    IH_REQUIRE(dry || !ctx->capturing, INFERC_ERR_STATE, "host constant changed inside capture");
    if (up.p) ++buf_gen;
    up.bytes = *v.host;
    up.p = buf("__h2d__" + name, v.bytes());
    if (dry) {
      v.dev = up.p;
      return up.p;
    }
    IH_HIP(hipMemcpyAsync(up.p, up.bytes.data(), up.bytes.size(), hipMemcpyHostToDevice,
                          ctx->stream));
    v.dev = up.p;
    return up.p;
  }

  // [N, K] copies of [K, N] weight initializers, for products with one row
  // of A: as transB operands they take the GEMV route of gemm() (the M == 1
  // sgemv of src/kernels/matmul.cc:207-216), whose rows are coalesced reads
  // of W, instead of a tiled GEMM with 1 of its 16..128 rows live. Made on
  // first use, outside any capture, and kept with the initializers.
  std::unordered_map<std::string, float*> wt_cache;
  size_t wt_cache_bytes = 0;  // device bytes of those copies
  const float* transposed_init(const std::string& name) {
    auto it = wt_cache.find(name);
    if (it != wt_cache.end()) return it->second;
    if (dry || ctx->capturing) return nullptr;
    auto ii = inits.find(name);
    if (ii == inits.end() || !ii->second.host || ii->second.dtype != INFERC_DT_F32 ||
        ii->second.shape.size() != 2 || ii->second.host->size() != ii->second.bytes())
      return nullptr;
    const int64_t K = ii->second.shape[0], N = ii->second.shape[1];
    const float* src = reinterpret_cast<const float*>(ii->second.host->data());
    std::vector<float> t(size_t(N) * size_t(K));
    for (int64_t k = 0; k < K; ++k)
      for (int64_t c = 0; c < N; ++c) t[size_t(c) * size_t(K) + size_t(k)] = src[k * N + c];
    void* d = nullptr;
    IH_HIP(hipMalloc(&d, t.size() * sizeof(float)));
    init_allocs.push_back(d);
    IH_HIP(hipMemcpy(d, t.data(), t.size() * sizeof(float), hipMemcpyHostToDevice));
    wt_cache_bytes += t.size() * sizeof(float);
    return wt_cache[name] = static_cast<float*>(d);
  }
  // Points g at the transposed copy of its B when the product has one row,
  // B is a [K, N] initializer that no input, tape value or folded constant
  // of the same name shadows, and the GEMV route (switched on in the
  // context, as the reference's SetGemvDecodeEnabled) takes the result.
  void batch1_route(ih::GemmArgs& g, const std::string& b_name) {
    if (dry || g.M != 1 || g.batch != 1 || g.trans_a || g.trans_b || g.ldb != g.N) return;
    auto ii = inits.find(b_name);
    if (ii == inits.end() || find_val(b_name) != &ii->second) return;
    ih::GemmArgs t = g;
    t.trans_b = 1;
    t.ldb = g.K;
    if (!ih::gemm_gemv_route(ctx, t)) return;
    const float* wt = transposed_init(b_name);
    if (!wt) return;
    t.B = wt;
    g = t;
  }

  ih::Value& make_dev(const std::string& name, int dtype, std::vector<int64_t> shape) {
    ih::Value v;
    v.dtype = dtype;
    v.shape = std::move(shape);
    v.dev = buf(name, v.bytes());
    vals[name] = v;
    return vals[name];
  }

  ih::Value& make_host(const std::string& name, int dtype, std::vector<int64_t> shape,
                       const void* data) {
    ih::Value v;
    v.dtype = dtype;
    v.shape = std::move(shape);
    v.host = std::make_shared<std::vector<uint8_t>>(v.bytes());
    if (v.bytes()) std::memcpy(v.host->data(), data, v.bytes());
    vals[name] = v;
    return vals[name];
  }

  // A host value of the given shape, zero-filled; returns its bytes.
  void* make_host_buf(const std::string& name, int dtype, std::vector<int64_t> shape) {
    ih::Value v;
    v.dtype = dtype;
    v.shape = std::move(shape);
    v.host = std::make_shared<std::vector<uint8_t>>(v.bytes());
    vals[name] = v;
    return vals[name].host->data();
  }

  // Every input of `n` is known on the host and the result is small: the
  // node is folded on the host (values derived from shapes and constants
  // only; graph inputs are always on the device).
  bool host_foldable(const inferc_graph::Node& n, int64_t out_numel) const {
    if (out_numel > (int64_t(1) << 16)) return false;
    for (const auto& i : n.in) {
      if (i.empty()) continue;
      const ih::Value* v = find_val(i);
      if (!v || !v->host) return false;
    }
    return true;
  }
  const void* host_of(const std::string& name) const { return get(name).host->data(); }

  void alias(const std::string& out, const ih::Value& in, std::vector<int64_t> shape) {
    ih::Value v = in;
    IH_REQUIRE(ih::numel_of(shape) == in.numel(), INFERC_ERR_SHAPE,
               "reshape: element count changes " + ih::shape_str(in.shape) + " -> " +
                   ih::shape_str(shape));
    v.shape = std::move(shape);
    vals[out] = v;
  }

  // Bytes of every non-initializer tensor on the tape (inputs and node
  // outputs, views counted at their logical size), the reference's
  // live_activation_bytes (src/runtime/executor.cc:112-119).
  int64_t live_activation_bytes() const {
    int64_t b = 0;
    for (const auto& kv : vals)
      if (!inits.count(kv.first)) b += int64_t(kv.second.bytes());
    return b;
  }

  void peephole();
  void exec_node(const inferc_graph::Node& n);
  bool ln_read_ok(const std::string& h, int64_t M, int64_t N, int64_t K);
  bool ln_read_of(const inferc_graph::Node& n, char role, std::string* h, ih::RowNorm* rn,
                  size_t* reader = nullptr);
  void fold_ln_weights();
  static std::string ln_fold_name(size_t reader, char what, int slice) {
    return "__lnfold:" + std::to_string(reader) + ":" + what + std::to_string(slice);
  }
  void generic_binary(const inferc_graph::Node& n, int ewop);
  void exec_attention_past(const inferc_graph::Node& n);
  void ln_prologue(const inferc_graph::Node& n, ih::GemmArgs& g);
  bool exec_generic(const inferc_graph::Node& n);
  // With `act`, records an event before each node and after the last on the
  // stream, and appends each node's activation bytes (0 unless `track`).
  void walk(std::vector<int64_t>* act = nullptr, bool track = false);
  std::string signature() const;
  std::string run_key() const;
  void stage_inputs();
  void run();
  void run_profiled(inferc_profiler* p);
};

namespace ih {
namespace {

using Node = inferc_graph::Node;

std::vector<int64_t> host_i64(const Value& v, const std::string& what) {
  IH_REQUIRE(v.host != nullptr, INFERC_ERR_UNSUPPORTED,
             what + ": needs host-known int64 data (constant shape plumbing)");
  IH_REQUIRE(v.dtype == INFERC_DT_I64 || v.dtype == INFERC_DT_I32, INFERC_ERR_ARG,
             what + ": expected an integer tensor");
  std::vector<int64_t> r(size_t(v.numel()));
  for (int64_t i = 0; i < v.numel(); ++i)
    r[size_t(i)] = v.dtype == INFERC_DT_I64 ? v.host_at<int64_t>(i) : v.host_at<int32_t>(i);
  return r;
}

// Right-aligned numpy broadcast test: b broadcasts into a as a repeated
// suffix (every leading dim of b is 1 or absent).
bool suffix_broadcast(const std::vector<int64_t>& a, const std::vector<int64_t>& b) {
  size_t lead = 0;
  while (lead < b.size() && b[lead] == 1) ++lead;
  const size_t r = b.size() - lead;
  if (r > a.size()) return false;
  for (size_t i = 0; i < r; ++i)
    if (b[lead + i] != a[a.size() - r + i]) return false;
  return true;
}

std::vector<int64_t> broadcast_shape(const std::vector<int64_t>& a, const std::vector<int64_t>& b) {
  const size_t r = a.size() > b.size() ? a.size() : b.size();
  std::vector<int64_t> out(r);
  for (size_t i = 0; i < r; ++i) {
    const int64_t da = i < a.size() ? a[a.size() - 1 - i] : 1;
    const int64_t db = i < b.size() ? b[b.size() - 1 - i] : 1;
    IH_REQUIRE(da == db || da == 1 || db == 1, INFERC_ERR_SHAPE, "incompatible broadcast");
    out[r - 1 - i] = da == 1 ? db : da;
  }
  return out;
}

}  // namespace
}  // namespace ih

void inferc_executor::peephole() {
  // consumer counts (graph outputs count as consumers)
  std::unordered_map<std::string, int> uses;
  for (const auto& n : nodes)
    for (const auto& i : n.in) ++uses[i];
  for (const auto& o : outputs) ++uses[o];
  auto producer = [&](const std::string& t) -> int {
    for (size_t i = 0; i < nodes.size(); ++i)
      for (const auto& o : nodes[i].out)
        if (o == t) return int(i);
    return -1;
  };
  std::vector<bool> dead(nodes.size(), false);
  for (size_t i = 0; i < nodes.size(); ++i) {
    inferc_graph::Node& n = nodes[i];
    if (dead[i]) continue;
    // MatMul(x, W) -> Add(., b) [-> Add(., r)]  ==>  FusedGemmEpilogue
    if (n.op == "MatMul" && n.in.size() == 2 && inits.count(n.in[1]) &&
        inits.at(n.in[1]).shape.size() == 2 && uses[n.out[0]] == 1) {
      const std::string mm_out = n.out[0];
      int a1 = -1;
      for (size_t j = i + 1; j < nodes.size(); ++j)
        if (!dead[j] && nodes[j].op == "Add" &&
            (nodes[j].in[0] == mm_out || nodes[j].in[1] == mm_out)) {
          a1 = int(j);
          break;
        }
      if (a1 < 0) continue;
      inferc_graph::Node& add1 = nodes[size_t(a1)];
      const std::string bias = add1.in[0] == mm_out ? add1.in[1] : add1.in[0];
      auto bit = inits.find(bias);
      if (bit == inits.end() || bit->second.shape.size() != 1 ||
          bit->second.shape[0] != inits.at(n.in[1]).shape[1])
        continue;
      inferc_graph::Node fused;
      fused.op = "FusedGemmEpilogue";
      fused.name = n.name + "+bias";
      fused.in = {n.in[0], n.in[1], bias};
      fused.out = add1.out;
      // optional residual add consuming the biased output once
      if (uses[add1.out[0]] == 1) {
        const std::string t = add1.out[0];
        for (size_t j = size_t(a1) + 1; j < nodes.size(); ++j) {
          if (dead[j] || nodes[j].op != "Add") continue;
          if (nodes[j].in[0] != t && nodes[j].in[1] != t) continue;
          const std::string res = nodes[j].in[0] == t ? nodes[j].in[1] : nodes[j].in[0];
          if (inits.count(res)) break;  // a second bias is not a residual
          // the residual must be produced before the MatMul runs
          const int pr = producer(res);
          if (pr >= int(i)) break;
          fused.in.push_back(res);
          fused.out = nodes[j].out;
          fused.name += "+residual";
          dead[j] = true;
          break;
        }
      }
      dead[size_t(a1)] = true;
      n = fused;
      continue;
    }
    // Gemm -> Relu  ==>  Gemm with a ReLU epilogue
    if (n.op == "Gemm" && uses[n.out[0]] == 1) {
      for (size_t j = i + 1; j < nodes.size(); ++j) {
        if (dead[j] || nodes[j].op != "Relu" || nodes[j].in[0] != n.out[0]) continue;
        n.out = nodes[j].out;
        n.attrs["__act"] = std::to_string(INFERC_ACT_RELU);
        dead[j] = true;
        break;
      }
    }
  }
  // Gemm chains of exported transformer layers, where views (Reshape) sit
  // between the ops:
  //  - Gemm -> [Reshape] -> Relu / Gelu / GeluTanh  ==>  Gemm with that
  //    activation as its epilogue (the activation acts elementwise, so it
  //    commutes with the view);
  //  - Gemm -> [Reshape] -> Add(., r)  ==>  Gemm with r as its residual,
  //    when r is no initializer and exists before the Gemm runs (the
  //    residual stream of a pre-LN layer);
  //  - FusedLayerNorm(x) -> [Reshape] -> Gemm or MatMul (as A, a 2-D
  //    initializer as B: the LM head)  ==>  the product normalizing its A
  //    rows, the view taking x (LayerNorm acts on rows over the last axis,
  //    which the view must keep: checked when the product runs).
  // Each intermediate must have the one reader. On the one-row GEMV route
  // all three become the GEMV's prologue and epilogue.
  auto sole_reader = [&](const std::string& t, size_t from) -> int {
    if (uses[t] != 1) return -1;
    for (size_t j = from; j < nodes.size(); ++j) {
      if (dead[j]) continue;
      if (std::find(nodes[j].in.begin(), nodes[j].in.end(), t) != nodes[j].in.end())
        return int(j);
    }
    return -1;
  };
  static const std::map<std::string, int> gemm_acts = {
      {"Relu", INFERC_ACT_RELU}, {"Gelu", INFERC_ACT_GELU_ERF},
      {"GeluTanh", INFERC_ACT_GELU_TANH}};
  for (size_t i = 0; i < nodes.size(); ++i) {
    inferc_graph::Node& n = nodes[i];
    if (dead[i] || n.op != "Gemm" || n.out.size() != 1 || n.attrs.count("__act") ||
        ih::attr_int(n, "transA", 0) != 0)
      continue;
    int c = sole_reader(n.out[0], i + 1);
    if (c < 0) continue;
    int view = -1;  // a Reshape between the Gemm and its reader
    if (nodes[size_t(c)].op == "Reshape" && nodes[size_t(c)].in[0] == n.out[0] &&
        nodes[size_t(c)].out.size() == 1) {
      view = c;
      c = sole_reader(nodes[size_t(c)].out[0], size_t(c) + 1);
      if (c < 0) continue;
    }
    inferc_graph::Node& d = nodes[size_t(c)];
    const std::string t = view >= 0 ? nodes[size_t(view)].out[0] : n.out[0];
    auto act = gemm_acts.find(d.op);
    if (act != gemm_acts.end() && d.in.size() == 1 && d.in[0] == t && d.out.size() == 1) {
      n.attrs["__act"] = std::to_string(act->second);
    } else if (d.op == "Add" && d.in.size() == 2 && d.out.size() == 1 &&
               (d.in[0] == t) != (d.in[1] == t)) {
      const std::string res = d.in[0] == t ? d.in[1] : d.in[0];
      const int pr = producer(res);
      if (inits.count(res) || pr >= int(i) || n.in.size() < 2) continue;
      n.attrs["__res"] = res;
    } else {
      continue;
    }
    // the reader's output is now the Gemm's (through the view, if any)
    if (view >= 0)
      nodes[size_t(view)].out = d.out;
    else
      n.out = d.out;
    dead[size_t(c)] = true;
  }
  for (size_t i = 0; i < nodes.size(); ++i) {
    inferc_graph::Node& ln = nodes[i];
    if (dead[i] || ln.op != "FusedLayerNorm" || ln.in.size() != 3 || ln.out.size() != 1 ||
        !inits.count(ln.in[1]) || !inits.count(ln.in[2]) ||
        std::find(outputs.begin(), outputs.end(), ln.out[0]) != outputs.end())
      continue;
    // readers of the LayerNorm's output; Shape nodes only need its shape,
    // which is its input's
    std::vector<size_t> shapes;
    int c = -1, others = 0;
    for (size_t j = i + 1; j < nodes.size(); ++j) {
      if (dead[j]) continue;
      const auto& in = nodes[j].in;
      if (std::find(in.begin(), in.end(), ln.out[0]) == in.end()) continue;
      if (nodes[j].op == "Shape") {
        shapes.push_back(j);
      } else {
        c = int(j);
        ++others;
      }
    }
    if (others != 1 || c < 0) continue;
    int view = -1;
    if (nodes[size_t(c)].op == "Reshape" && nodes[size_t(c)].in[0] == ln.out[0] &&
        nodes[size_t(c)].out.size() == 1) {
      view = c;
      c = sole_reader(nodes[size_t(c)].out[0], size_t(c) + 1);
      if (c < 0) continue;
    }
    inferc_graph::Node& g = nodes[size_t(c)];
    const std::string t = view >= 0 ? nodes[size_t(view)].out[0] : ln.out[0];
    const bool mm = g.op == "MatMul" && g.in.size() == 2 && inits.count(g.in[1]) &&
                    inits.at(g.in[1]).shape.size() == 2;
    if ((g.op != "Gemm" && !mm) || g.in.empty() || g.in[0] != t ||
        ih::attr_int(g, "transA", 0) != 0 || g.attrs.count("__ln_g"))
      continue;
    g.attrs["__ln_g"] = ln.in[1];
    g.attrs["__ln_b"] = ln.in[2];
    g.attrs["__ln_eps"] = ih::float_text(ih::attr_float(ln, "epsilon", 1e-5f));
    g.attrs["__ln_x"] = ln.in[0];  // the rows normalized, for the last-axis check
    if (view >= 0)
      nodes[size_t(view)].in[0] = ln.in[0];
    else
      g.in[0] = ln.in[0];
    for (size_t j : shapes) nodes[j].in[0] = ln.in[0];
    dead[i] = true;
  }
  // Add(a, b) -> FusedLayerNorm (its only reader)  ==>  LayerNorm with a
  // residual input: the embedding sum word + position goes straight into
  // the LayerNorm kernel (activation.cc:103-150 on the summed rows).
  for (size_t i = 0; i < nodes.size(); ++i) {
    inferc_graph::Node& n = nodes[i];
    if (dead[i] || n.op != "Add" || n.in.size() != 2 || n.out.size() != 1 ||
        uses[n.out[0]] != 1 || inits.count(n.in[0]) || inits.count(n.in[1]))
      continue;
    for (size_t j = i + 1; j < nodes.size(); ++j) {
      if (dead[j]) continue;
      inferc_graph::Node& ln = nodes[j];
      if (std::find(ln.in.begin(), ln.in.end(), n.out[0]) == ln.in.end()) continue;
      if (ln.op == "FusedLayerNorm" && ln.in.size() == 3 && ln.in[0] == n.out[0]) {
        ln.in = {n.in[0], ln.in[1], ln.in[2], n.in[1]};
        ln.name = n.name + "+" + ln.name;
        dead[i] = true;
      }
      break;
    }
  }
  // FusedLayerNorm (x) -> Gather(x, constant indices) -> Gemm(transB), each
  // result read once: the Gather takes the LayerNorm's input and the Gemm
  // normalizes its A rows (LayerNorm acts row by row, so the two commute; the
  // classifier head of an encoder). On the one-row GEMV route the GEMV's
  // LayerNorm prologue does it, else a LayerNorm of the gathered rows.
  for (size_t i = 0; i < nodes.size(); ++i) {
    inferc_graph::Node& gt = nodes[i];
    if (dead[i] || gt.op != "Gather" || gt.in.size() != 2 || !inits.count(gt.in[1]) ||
        uses[gt.in[0]] != 1 || uses[gt.out[0]] != 1)
      continue;
    const int li = producer(gt.in[0]);
    if (li < 0 || dead[size_t(li)]) continue;
    const inferc_graph::Node& ln = nodes[size_t(li)];
    if (ln.op != "FusedLayerNorm" || ln.in.size() != 3 || !inits.count(ln.in[1]) ||
        !inits.count(ln.in[2]))
      continue;
    for (size_t j = i + 1; j < nodes.size(); ++j) {
      inferc_graph::Node& c = nodes[j];
      if (dead[j] || c.in.empty() || c.in[0] != gt.out[0]) continue;
      if (c.op == "Gemm" && ih::attr_int(c, "transB", 0) == 1 && ih::attr_int(c, "transA", 0) == 0) {
        // both carry the LayerNorm: the Gather applies it itself when it
        // selects along the feature axis (where the two do not commute)
        for (inferc_graph::Node* t : {&c, &gt}) {
          t->attrs["__ln_g"] = ln.in[1];
          t->attrs["__ln_b"] = ln.in[2];
          t->attrs["__ln_eps"] = ih::float_text(ih::attr_float(ln, "epsilon", 1e-5f));
        }
        gt.in[0] = ln.in[0];
        dead[size_t(li)] = true;
      }
      break;
    }
  }
  std::vector<inferc_graph::Node> kept;
  for (size_t i = 0; i < nodes.size(); ++i)
    if (!dead[i]) kept.push_back(std::move(nodes[i]));
  nodes = std::move(kept);
  // Nodes none of whose outputs is read or returned are not run (e.g. the
  // float mask an attention fusion left behind). A graph that declares no
  // outputs keeps every node.
  for (bool changed = !outputs.empty(); changed;) {
    changed = false;
    std::unordered_map<std::string, int> used;
    for (const auto& n : nodes)
      for (const auto& i : n.in) ++used[i];
    for (const auto& o : outputs) ++used[o];
    std::vector<inferc_graph::Node> live;
    for (auto& n : nodes) {
      bool read = n.out.empty();
      for (const auto& o : n.out) read = read || used.count(o) > 0;
      if (read) live.push_back(std::move(n));
      else changed = true;
    }
    nodes = std::move(live);
  }
  // LayerNorms that their readers can apply as they read (final node
  // order, so the reader indices stay valid)
  ln_reads.clear();
  std::unordered_map<std::string, int> ln_of;  // LayerNorms per input
  for (const auto& n : nodes)
    if (n.op == "FusedLayerNorm" && !n.in.empty()) ++ln_of[n.in[0]];
  for (size_t i = 0; i < nodes.size(); ++i) {
    const inferc_graph::Node& ln = nodes[i];
    if (ln.op != "FusedLayerNorm" || ln.in.size() != 3 || ln.out.size() != 1) continue;
    const std::string& h = ln.in[0];
    const std::string& x = ln.out[0];
    // (an h with two LayerNorms keeps both as kernels)
    if (!inits.count(ln.in[1]) || !inits.count(ln.in[2]) || inits.count(h) || ln_of[h] != 1 ||
        std::find(outputs.begin(), outputs.end(), x) != outputs.end())
      continue;
    int pi = -1;
    for (size_t j = 0; j < i; ++j)
      if (std::find(nodes[j].out.begin(), nodes[j].out.end(), h) != nodes[j].out.end())
        pi = int(j);
    if (pi < 0 || nodes[size_t(pi)].op != "FusedGemmEpilogue") continue;
    LnRead lr;
    lr.out = x;
    lr.gamma = ln.in[1];
    lr.beta = ln.in[2];
    lr.eps = ih::attr_float(ln, "epsilon", 1e-5f);
    bool ok = true;
    for (size_t j = i + 1; j < nodes.size() && ok; ++j) {
      const inferc_graph::Node& c = nodes[j];
      for (size_t k = 0; k < c.in.size(); ++k) {
        if (c.in[k] != x) continue;
        const bool a = k == 0 && (c.op == "FusedQKV" || c.op == "FusedMatMulAddGELU" ||
                                  c.op == "FusedGemmEpilogue");
        const bool r = k == 3 && c.op == "FusedGemmEpilogue";
        if (!(a || r) || !inits.count(c.in[1])) ok = false;
        else lr.readers.emplace_back(j, a ? 'a' : 'r');
      }
    }
    if (ok && !lr.readers.empty()) ln_reads[h] = std::move(lr);
  }
  // Row gathers from an initializer table read by one FusedLayerNorm only
  gather_ln.clear();
  std::unordered_map<std::string, int> reads;
  for (const auto& n : nodes)
    for (const auto& t : n.in) ++reads[t];
  for (const auto& g : nodes) {
    if (g.op != "Gather" || g.in.size() != 2 || g.out.size() != 1 || !inits.count(g.in[0]) ||
        inits.count(g.in[1]) || ih::attr_int(g, "axis", 0) != 0 || g.attrs.count("__ln_g") ||
        reads[g.out[0]] != 1 ||
        std::find(outputs.begin(), outputs.end(), g.out[0]) != outputs.end())
      continue;
    const ih::Value& t = inits.at(g.in[0]);
    if (t.dtype != INFERC_DT_F32 || t.shape.size() != 2) continue;
    for (const auto& n : nodes)
      if (n.op == "FusedLayerNorm" && n.in.size() >= 3 &&
          (n.in[0] == g.out[0] || (n.in.size() >= 4 && n.in[3] == g.out[0])))
        gather_ln.insert(g.out[0]);
  }
  // An Equal whose operands exist before any node runs (a graph input and an
  // initializer) rides along with the launch of the nearest FusedLayerNorm
  // before it: one launch fewer (an encoder's padding mask).
  eq_side.clear();
  std::unordered_set<std::string> produced;
  for (const auto& n : nodes)
    for (const auto& o : n.out) produced.insert(o);
  for (size_t i = 0; i < nodes.size(); ++i) {
    const inferc_graph::Node& e = nodes[i];
    if (e.op != "Equal" || e.in.size() != 2 || e.out.size() != 1 || inits.count(e.in[0]) ||
        produced.count(e.in[0]) || !inits.count(e.in[1]))
      continue;
    for (size_t j = i; j-- > 0;)
      if (nodes[j].op == "FusedLayerNorm" && nodes[j].out.size() == 1) {
        if (!eq_side.count(nodes[j].out[0])) eq_side[nodes[j].out[0]] = i;
        break;
      }
  }
}

// Whether this run's readers of h apply its LayerNorm as they read (decided
// at h's producer, which then writes h's row statistics): every product
// involved takes the small-M GEMM path, and the operands are 16-byte aligned.
bool inferc_executor::ln_read_ok(const std::string& h, int64_t M, int64_t N, int64_t K) {
  auto it = ln_reads.find(h);
  if (it == ln_reads.end() || dry || N % 16 != 0 || N > 1024) return false;
  if (!ih::gemm_small_m_path(ctx, M, N, K, 1)) return false;
  const LnRead& lr = it->second;
  auto aligned = [&](const std::string& t) {
    return (reinterpret_cast<uintptr_t>(inits.at(t).dev) & 15) == 0;
  };
  if (inits.at(lr.gamma).numel() != N || inits.at(lr.beta).numel() != N || !aligned(lr.gamma) ||
      !aligned(lr.beta))
    return false;
  for (const auto& rd : lr.readers) {
    const inferc_graph::Node& c = nodes[rd.first];
    const ih::Value& w = inits.at(c.in[1]);
    if (w.shape.size() != 2 || !aligned(c.in[1])) return false;
    if (rd.second == 'a') {
      const int64_t slices = c.op == "FusedQKV" ? 3 : 1;
      if (w.shape[0] != N || !ih::gemm_small_m_path(ctx, M, w.shape[1], N, slices)) return false;
      for (int i = 0; i < int(slices); ++i)
        if (!inits.count(ln_fold_name(rd.first, 'w', i))) return false;
    } else if (w.shape[1] != N || !ih::gemm_small_m_path(ctx, M, N, w.shape[0], 1)) {
      return false;
    }
  }
  return true;
}

// The LayerNorm a reader applies to operand `role` ('a' or 'r') of node n
// this run, if any: the tensor h it reads instead of the LayerNorm output,
// and the normalization.
bool inferc_executor::ln_read_of(const inferc_graph::Node& n, char role, std::string* h,
                                 ih::RowNorm* rn, size_t* reader) {
  const size_t k = role == 'a' ? 0 : 3;
  if (n.in.size() <= k) return false;
  for (const auto& kv : ln_reads) {
    auto on = ln_on.find(kv.first);
    if (on == ln_on.end() || !on->second) continue;
    for (const auto& rd : kv.second.readers) {
      if (rd.second != role || &nodes[rd.first] != &n) continue;
      *h = kv.first;
      if (reader) *reader = rd.first;
      rn->stats = static_cast<const float*>(arena.at("__lnstats:" + kv.first).p);
      rn->eps = kv.second.eps;
      if (role == 'r') {
        rn->gamma = static_cast<const float*>(dev_of(kv.second.gamma));
        rn->beta = static_cast<const float*>(dev_of(kv.second.beta));
      } else {
        const int slices = n.op == "FusedQKV" ? 3 : 1;
        for (int i = 0; i < slices; ++i)
          rn->colsum[i] = static_cast<const float*>(dev_of(ln_fold_name(rd.first, 'c', i)));
      }
      return true;
    }
  }
  return false;
}

// For every reader that takes a LayerNorm's output as its A operand: the
// folded operands that let it read the LayerNorm's input instead,
// B'_kn = gamma_k B_kn, colsum_n = sum_k B'_kn and C'_n = C_n + sum_k
// beta_k B_kn (sums in double), kept as device initializers beside the
// originals, which the LayerNorm-kernel path still uses. A LayerNorm whose
// readers' operands cannot be folded (not float32 initializers of the
// expected shapes) is left to the kernel.
void inferc_executor::fold_ln_weights() {
  for (auto it = ln_reads.begin(); it != ln_reads.end();) {
    const LnRead& lr = it->second;
    const ih::Value& gv = inits.at(lr.gamma);
    const ih::Value& bv = inits.at(lr.beta);
    const int64_t D = gv.numel();
    bool ok = gv.dtype == INFERC_DT_F32 && bv.dtype == INFERC_DT_F32 && gv.host && bv.host &&
              bv.numel() == D;
    struct Fold {
      std::string name;
      std::vector<int64_t> shape;
      std::vector<float> v;
    };
    std::vector<Fold> folds;
    for (const auto& rd : lr.readers) {
      if (!ok || rd.second != 'a') continue;
      const inferc_graph::Node& c = nodes[rd.first];
      const int slices = c.op == "FusedQKV" ? 3 : 1;
      for (int i = 0; i < slices && ok; ++i) {
        const size_t wi = size_t(1 + 2 * i), bi = size_t(2 + 2 * i);
        if (c.in.size() <= bi || !inits.count(c.in[wi]) || !inits.count(c.in[bi])) {
          ok = false;
          break;
        }
        const ih::Value& W = inits.at(c.in[wi]);
        const ih::Value& B = inits.at(c.in[bi]);
        if (W.dtype != INFERC_DT_F32 || B.dtype != INFERC_DT_F32 || !W.host || !B.host ||
            W.shape.size() != 2 || W.shape[0] != D || B.numel() != W.shape[1]) {
          ok = false;
          break;
        }
        const int64_t N = W.shape[1];
        const float* w = reinterpret_cast<const float*>(W.host->data());
        const float* b = reinterpret_cast<const float*>(B.host->data());
        const float* gam = reinterpret_cast<const float*>(gv.host->data());
        const float* bet = reinterpret_cast<const float*>(bv.host->data());
        Fold fw{ln_fold_name(rd.first, 'w', i), {D, N}, std::vector<float>(size_t(D * N))};
        std::vector<double> cs(size_t(N), 0.0), ds(size_t(N), 0.0);
        for (int64_t k = 0; k < D; ++k)
          for (int64_t n = 0; n < N; ++n) {
            const float wk = gam[k] * w[k * N + n];
            fw.v[size_t(k * N + n)] = wk;
            cs[size_t(n)] += double(wk);
            ds[size_t(n)] += double(bet[k]) * double(w[k * N + n]);
          }
        Fold fc{ln_fold_name(rd.first, 'c', i), {N}, std::vector<float>(size_t(N))};
        Fold fb{ln_fold_name(rd.first, 'b', i), {N}, std::vector<float>(size_t(N))};
        for (int64_t n = 0; n < N; ++n) {
          fc.v[size_t(n)] = float(cs[size_t(n)]);
          fb.v[size_t(n)] = float(double(b[n]) + ds[size_t(n)]);
        }
        folds.push_back(std::move(fw));
        folds.push_back(std::move(fc));
        folds.push_back(std::move(fb));
      }
    }
    if (!ok) {
      it = ln_reads.erase(it);
      continue;
    }
    for (Fold& f : folds) {
      ih::Value v;
      v.dtype = INFERC_DT_F32;
      v.shape = f.shape;
      const size_t bytes = f.v.size() * sizeof(float);
      IH_HIP(hipMalloc(&v.dev, bytes));
      init_allocs.push_back(v.dev);
      IH_HIP(hipMemcpy(v.dev, f.v.data(), bytes, hipMemcpyHostToDevice));
      inits[f.name] = v;
    }
    ++it;
  }
}

void inferc_executor::exec_node(const inferc_graph::Node& n) {
  using namespace ih;
  const std::string& op = n.op;
  auto in = [&](size_t i) -> const Value& {
    IH_REQUIRE(i < n.in.size(), INFERC_ERR_ARG, op + ": missing input " + std::to_string(i));
    return get(n.in[i]);
  };
  auto require_f32 = [&](const Value& v, const char* what) {
    IH_REQUIRE(v.dtype == INFERC_DT_F32, INFERC_ERR_UNSUPPORTED,
               op + ": " + what + " must be float32");
  };
  IH_REQUIRE(!n.out.empty(), INFERC_ERR_ARG, op + ": node has no outputs");

  if (op == "FusedQKV") {
    std::string ha;
    RowNorm rna;
    size_t rdr = 0;
    const bool lna = ln_read_of(n, 'a', &ha, &rna, &rdr);
    const Value x = lna ? get(ha) : in(0);
    require_f32(x, "X");
    const int64_t K = x.shape.back(), M = x.numel() / K;
    const Value& wq = in(1);
    IH_REQUIRE(wq.shape.size() == 2 && wq.shape[0] == K, INFERC_ERR_SHAPE, "FusedQKV: W shape");
    const int64_t N = wq.shape[1];
    std::vector<int64_t> os = x.shape;
    os.back() = N;
    const float* w[3];
    const float* b[3];
    float* y[3];
    for (int i = 0; i < 3; ++i) {
      const Value& wi = in(size_t(1 + 2 * i));
      const Value& bi = in(size_t(2 + 2 * i));
      IH_REQUIRE(wi.shape == wq.shape && bi.numel() == N, INFERC_ERR_SHAPE,
                 "FusedQKV: projections must share shapes");
      w[i] = static_cast<const float*>(
          dev_of(lna ? ln_fold_name(rdr, 'w', i) : n.in[size_t(1 + 2 * i)]));
      b[i] = static_cast<const float*>(
          dev_of(lna ? ln_fold_name(rdr, 'b', i) : n.in[size_t(2 + 2 * i)]));
      IH_REQUIRE(i < int(n.out.size()), INFERC_ERR_ARG, "FusedQKV: needs three outputs");
      y[i] = static_cast<float*>(make_dev(n.out[size_t(i)], INFERC_DT_F32, os).dev);
    }
    if (!dry) {
      gemm_qkv(ctx, M, K, N, static_cast<const float*>(dev_of(lna ? ha : n.in[0])), w, b, y, N,
               lna ? &rna : nullptr);
    }
    return;
  }
  if (op == "FusedAttention") {
    const Value& q = in(0);
    require_f32(q, "Q");
    IH_REQUIRE(q.shape.size() == 3, INFERC_ERR_SHAPE, "FusedAttention: expect [B,S,H]");
    IH_REQUIRE(in(1).shape == q.shape && in(2).shape == q.shape, INFERC_ERR_SHAPE,
               "FusedAttention: Q/K/V shapes differ");
    AttnArgs a;
    a.B = q.shape[0]; a.S = q.shape[1]; a.H = q.shape[2];
    a.head_dim = attr_int(n, "head_dim", 64);
    a.fill = attr_float(n, "fill", -3.0e38f);
    a.q = static_cast<const float*>(dev_of(n.in[0]));
    a.k = static_cast<const float*>(dev_of(n.in[1]));
    a.v = static_cast<const float*>(dev_of(n.in[2]));
    a.ldq = a.ldk = a.ldv = a.ldo = a.H;
    if (n.in.size() >= 4 && !n.in[3].empty()) {
      const Value& m = in(3);
      IH_REQUIRE(m.dtype == INFERC_DT_BOOL || m.dtype == INFERC_DT_U8, INFERC_ERR_UNSUPPORTED,
                 "FusedAttention: mask must be bool");
      IH_REQUIRE(m.shape.size() <= 4, INFERC_ERR_SHAPE, "FusedAttention: mask rank > 4");
      a.mask = static_cast<const uint8_t*>(dev_of(n.in[3]));
      mask_strides(m.shape, a.ms);
    }
    a.out = static_cast<float*>(make_dev(n.out[0], INFERC_DT_F32, q.shape).dev);
    if (!dry) {
      attention(ctx, a);
    }
    return;
  }
  if (op == "FusedAttentionPast") {
    exec_attention_past(n);
    return;
  }
  if (op == "FusedMatMulAddGELU" || op == "FusedGemmEpilogue" || op == "MatMul") {
    std::string ha, hr;
    RowNorm rna, rnr;
    size_t rdr = 0;
    const bool lna = op != "MatMul" && ln_read_of(n, 'a', &ha, &rna, &rdr);
    const bool lnr = op == "FusedGemmEpilogue" && ln_read_of(n, 'r', &hr, &rnr);
    const Value x = lna ? get(ha) : in(0);
    const Value& w = in(1);
    require_f32(x, "A");
    require_f32(w, "B");
    if (op == "MatMul" && (w.shape.size() != 2 || x.shape.size() < 2)) {
      // numpy-batched MatMul with broadcast batch dims (matmul.cc:63-159)
      IH_REQUIRE(x.shape.size() >= 2 && w.shape.size() >= 2, INFERC_ERR_UNSUPPORTED,
                 "MatMul: 1-D operands are not supported");
      const int64_t M = x.shape[x.shape.size() - 2], K = x.shape.back();
      const int64_t N = w.shape.back();
      IH_REQUIRE(w.shape[w.shape.size() - 2] == K, INFERC_ERR_SHAPE,
                 "MatMul: inner dim mismatch (K!=K)");
      std::vector<int64_t> ab(x.shape.begin(), x.shape.end() - 2);
      std::vector<int64_t> bb(w.shape.begin(), w.shape.end() - 2);
      std::vector<int64_t> ob = broadcast_shape(ab, bb);
      const int64_t batch = numel_of(ob);
      const int64_t na = numel_of(ab), nb = numel_of(bb);
      IH_REQUIRE((na == batch || na == 1) && (nb == batch || nb == 1), INFERC_ERR_UNSUPPORTED,
                 "MatMul: partial batch broadcast is not supported");
      std::vector<int64_t> os = ob;
      os.push_back(M);
      os.push_back(N);
      GemmArgs g;
      g.M = M; g.N = N; g.K = K;
      g.A = static_cast<const float*>(dev_of(n.in[0])); g.lda = K;
      g.B = static_cast<const float*>(dev_of(n.in[1])); g.ldb = N;
      g.batch = batch;
      g.stride_a = na == 1 ? 0 : M * K;
      g.stride_b = nb == 1 ? 0 : K * N;
      g.Y = static_cast<float*>(make_dev(n.out[0], INFERC_DT_F32, os).dev);
      g.ldy = N; g.stride_y = M * N;
      if (!dry) {
        gemm(ctx, g);
      }
      return;
    }
    IH_REQUIRE(w.shape.size() == 2, INFERC_ERR_SHAPE, op + ": W must be 2D [K,N]");
    const int64_t K = w.shape[0], N = w.shape[1];
    IH_REQUIRE(!x.shape.empty() && x.shape.back() == K, INFERC_ERR_SHAPE,
               op + ": K mismatch between X and W");
    const int64_t M = x.numel() / K;
    std::vector<int64_t> os = x.shape;
    os.back() = N;
    GemmArgs g;
    g.M = M; g.N = N; g.K = K;
    g.A = static_cast<const float*>(dev_of(lna ? ha : n.in[0])); g.lda = K;
    g.B = static_cast<const float*>(dev_of(lna ? ln_fold_name(rdr, 'w', 0) : n.in[1]));
    g.ldb = N;
    g.ldy = N;
    if (lna) g.norm_a = rna;
    if (op != "MatMul") {
      IH_REQUIRE(in(2).numel() == N, INFERC_ERR_SHAPE, op + ": bias size must equal N");
      g.beta = 1.0f;
      g.C = static_cast<const float*>(dev_of(lna ? ln_fold_name(rdr, 'b', 0) : n.in[2]));
      g.c_kind = INFERC_C_ROW;
    }
    if (op == "FusedMatMulAddGELU") g.act = INFERC_ACT_GELU_ERF;
    if (op == "FusedGemmEpilogue" && n.in.size() >= 4) {
      const Value r = lnr ? get(hr) : in(3);
      IH_REQUIRE(r.numel() == M * N, INFERC_ERR_UNSUPPORTED,
                 "fused residual must match the product's shape");
      g.R = static_cast<const float*>(dev_of(lnr ? hr : n.in[3]));
      g.ldr = N;
      if (lnr) g.norm_r = rnr;
    }
    g.Y = static_cast<float*>(make_dev(n.out[0], INFERC_DT_F32, os).dev);
    if (op == "FusedGemmEpilogue" && ln_reads.count(n.out[0])) {
      // the producer of a LayerNorm read by its readers: decide for this
      // run, and write the row statistics they combine
      const bool on = ln_read_ok(n.out[0], M, N, K);
      ln_on[n.out[0]] = on;
      // (an arena buffer, not a tensor of the graph)
      if (on)
        g.stats_out = static_cast<float*>(
            buf("__lnstats:" + n.out[0], size_t(M) * size_t(N / 16) * 2 * sizeof(float)));
    }
    // (after the row statistics are decided: a product that writes them
    // stays off the GEMV route)
    if (!lna) batch1_route(g, n.in[1]);
    if (op == "MatMul") ln_prologue(n, g);
    if (!dry && decode && !fb_logits.empty() && n.out[0] == fb_logits &&
        gemm_gemv_route(ctx, g) && gemv2_supported(g.K) && aligned16(g.B) && aligned16(g.A) &&
        (!g.gemv_ln_g || (aligned16(g.gemv_ln_g) && aligned16(g.gemv_ln_b))) &&
        g.c_kind == INFERC_C_NONE && g.R == nullptr) {
      // the fed-back logits' GEMV also leaves its blocks' (max, first index)
      // for the step's feedback to reduce
      Gemv2Args a;
      a.N = g.N; a.K = g.K; a.W = g.B; a.x = g.A;
      a.ln_g = g.gemv_ln_g; a.ln_b = g.gemv_ln_b; a.ln_eps = g.gemv_ln_eps;
      a.act = g.act; a.y = g.Y;
      fb_parts_n = gemv2_blocks(ctx, g.N, g.K, true);
      a.amax = static_cast<ValIdxPart*>(
          buf("__fbparts__", size_t(fb_parts_n) * sizeof(ValIdxPart)));
      fb_parts = a.amax;
      gemv2(ctx, a);
      return;
    }
    if (!dry) {
      gemm(ctx, g);
    }
    return;
  }
  if (op == "Gemm") {
    const Value& a = in(0);
    const Value& b = in(1);
    require_f32(a, "A");
    require_f32(b, "B");
    IH_REQUIRE(a.shape.size() == 2 && b.shape.size() == 2, INFERC_ERR_SHAPE,
               "Gemm: 2D inputs only, got " + shape_str(a.shape) + " and " + shape_str(b.shape));
    GemmArgs g;
    g.trans_a = int(attr_int(n, "transA", 0));
    g.trans_b = int(attr_int(n, "transB", 0));
    g.alpha = attr_float(n, "alpha", 1.0f);
    g.beta = attr_float(n, "beta", 1.0f);
    g.M = g.trans_a ? a.shape[1] : a.shape[0];
    g.K = g.trans_a ? a.shape[0] : a.shape[1];
    const int64_t Kb = g.trans_b ? b.shape[1] : b.shape[0];
    g.N = g.trans_b ? b.shape[0] : b.shape[1];
    IH_REQUIRE(g.K == Kb, INFERC_ERR_SHAPE, "Gemm: K mismatch");
    g.A = static_cast<const float*>(dev_of(n.in[0]));
    g.lda = a.shape[1];
    g.B = static_cast<const float*>(dev_of(n.in[1]));
    g.ldb = b.shape[1];
    if (n.in.size() >= 3 && !n.in[2].empty() && g.beta != 0.0f) {
      const Value& c = in(2);
      if (c.numel() == g.M * g.N) {
        g.c_kind = INFERC_C_FULL;
        g.ldc = g.N;
      } else if (c.shape.size() == 1 && c.shape[0] == g.N) {
        g.c_kind = INFERC_C_ROW;
      } else if (c.numel() == 1) {
        g.c_kind = INFERC_C_SCALAR;
      } else {
        fail(INFERC_ERR_SHAPE, "Gemm: unsupported C shape for broadcast");
      }
      g.C = static_cast<const float*>(dev_of(n.in[2]));
    }
    g.act = int(attr_int(n, "__act", INFERC_ACT_NONE));
    auto rs = n.attrs.find("__res");
    if (rs != n.attrs.end()) {
      // the residual Add folded in by the peephole (through a view)
      const Value& rv = get(rs->second);
      IH_REQUIRE(rv.dtype == INFERC_DT_F32 && rv.numel() == g.M * g.N, INFERC_ERR_UNSUPPORTED,
                 "Gemm: the residual added to its result must match it element for element");
      g.R = static_cast<const float*>(dev_of(rs->second));
      g.ldr = g.N;
    }
    g.Y = static_cast<float*>(make_dev(n.out[0], INFERC_DT_F32, {g.M, g.N}).dev);
    g.ldy = g.N;
    batch1_route(g, n.in[1]);
    if (!ln_gemm_off.count(n.in[0])) ln_prologue(n, g);
    if (!dry) {
      gemm(ctx, g);
    }
    return;
  }
  if (op == "FusedLayerNorm") {
    if (n.in.size() == 3) {
      auto on = ln_on.find(n.in[0]);
      auto lr = ln_reads.find(n.in[0]);
      if (on != ln_on.end() && on->second && lr != ln_reads.end() && lr->second.out == n.out[0]) {
        // its readers apply it: the output is a tensor of the tape at its
        // logical size with no data (a non-reader asking for it fails)
        ih::Value v;
        v.dtype = INFERC_DT_F32;
        v.shape = get(n.in[0]).shape;
        vals[n.out[0]] = v;
        return;
      }
    }
    // optional 4th input: the other operand of an Add folded in front
    // (y = LN(x + r), r repeated over leading dims as the Add broadcast it)
    size_t xi = 0, ri = 3;
    if (n.in.size() >= 4 && in(3).numel() > in(0).numel()) std::swap(xi, ri);
    if (n.in.size() >= 4 && pending_gather.count(n.in[ri])) materialize_gather(n.in[ri]);
    const auto pg = pending_gather.find(n.in[xi]);
    const Value& x = in(xi);
    require_f32(x, "X");
    const int64_t feat = x.shape.back();
    IH_REQUIRE(in(1).numel() == feat && in(2).numel() == feat, INFERC_ERR_SHAPE,
               "LayerNorm: scale/bias size mismatch with feature dim");
    const float eps = attr_float(n, "epsilon", 1e-5f);
    const float* res = nullptr;
    int64_t res_rows = 1;
    if (n.in.size() >= 4) {
      const Value& rv = in(ri);
      require_f32(rv, "residual");
      IH_REQUIRE(rv.numel() > 0 && rv.numel() % feat == 0 && x.numel() % rv.numel() == 0 &&
                     (rv.shape.empty() || rv.shape.back() == feat),
                 INFERC_ERR_UNSUPPORTED, "Add before LayerNorm: unsupported broadcast");
      res = static_cast<const float*>(dev_of(n.in[ri]));
      res_rows = rv.numel() / feat;
    }
    float* y = static_cast<float*>(make_dev(n.out[0], INFERC_DT_F32, x.shape).dev);
    ih::EqSide side;
    const auto es = eq_side.find(n.out[0]);
    if (es != eq_side.end()) {
      // the Equal's own fast-path conditions (below), else it runs itself
      const inferc_graph::Node& e = nodes[es->second];
      const Value& ea = get(e.in[0]);
      const Value& eb = get(e.in[1]);
      if (ea.dtype == INFERC_DT_I64 && eb.dtype == INFERC_DT_I64 && !(ea.host && eb.host) &&
          eb.numel() > 0 &&
          (eb.numel() == ea.numel() || eb.numel() == 1 || suffix_broadcast(ea.shape, eb.shape)) &&
          eb.numel() <= ea.numel()) {
        side.a = static_cast<const int64_t*>(dev_of(e.in[0]));
        side.b = static_cast<const int64_t*>(dev_of(e.in[1]));
        side.n = ea.numel();
        side.b_n = eb.numel();
        side.out = static_cast<uint8_t*>(make_dev(e.out[0], INFERC_DT_BOOL, ea.shape).dev);
        eq_done.insert(e.out[0]);
      }
    }
    if (pg != pending_gather.end()) {
      // x is a row gather from an embedding table: the kernel gathers
      const PendingGather g = pg->second;
      pending_gather.erase(pg);
      IH_REQUIRE(g.feat == feat && g.n == x.numel() / feat, INFERC_ERR_SHAPE,
                 "LayerNorm: gathered rows do not match the feature dim");
      if (!dry) {
        layernorm_gather(ctx, g.n, feat, g.table, g.vocab, g.ids, gather_err, res, res_rows,
                         static_cast<const float*>(dev_of(n.in[1])),
                         static_cast<const float*>(dev_of(n.in[2])), eps, y, side);
        dev_gather = true;
      }
      return;
    }
    if (!dry) {
      layernorm_res_period(ctx, x.numel() / feat, feat, static_cast<const float*>(dev_of(n.in[xi])),
                           res, res_rows, static_cast<const float*>(dev_of(n.in[1])),
                           static_cast<const float*>(dev_of(n.in[2])), eps, y, side);
    }
    return;
  }
  if (op == "Gelu" || op == "GeluTanh" || op == "Relu") {
    const Value& x = in(0);
    require_f32(x, "X");
    const int act = op == "Gelu" ? INFERC_ACT_GELU_ERF
                    : op == "GeluTanh" ? INFERC_ACT_GELU_TANH
                                       : INFERC_ACT_RELU;
    float* y = static_cast<float*>(make_dev(n.out[0], INFERC_DT_F32, x.shape).dev);
    if (!dry) {
      activation(ctx, x.numel(), static_cast<const float*>(dev_of(n.in[0])), act, y);
    }
    return;
  }
  if (op == "Softmax") {
    const Value& x = in(0);
    require_f32(x, "X");
    int64_t axis = attr_int(n, "axis", -1);
    const int64_t r = int64_t(x.shape.size());
    if (axis < 0) axis += r;
    IH_REQUIRE(axis >= 0 && axis < r, INFERC_ERR_ARG, "Softmax: axis out of range");
    int64_t outer = 1, inner = 1;
    for (int64_t i = 0; i < axis; ++i) outer *= x.shape[size_t(i)];
    for (int64_t i = axis + 1; i < r; ++i) inner *= x.shape[size_t(i)];
    float* y = static_cast<float*>(make_dev(n.out[0], INFERC_DT_F32, x.shape).dev);
    if (!dry) {
      IH_REQUIRE(inferc_hip_softmax_f32(ctx, outer, x.shape[size_t(axis)], inner,
                                        static_cast<const float*>(dev_of(n.in[0])), y) == 0,
                 INFERC_ERR_HIP, inferc_hip_last_error());
    }
    return;
  }
  if (op == "Add") {
    if (decode && embed_add_at[node_index(n)] && n.in.size() == 2) {
      auto e0 = pending_embed.find(n.in[0]), e1 = pending_embed.find(n.in[1]);
      if (e0 != pending_embed.end() && e1 != pending_embed.end() &&
          (e0->second.ids == nullptr) != (e1->second.ids == nullptr) &&
          get(n.in[0]).shape == get(n.in[1]).shape && e0->second.feat == e1->second.feat &&
          e0->second.n == e1->second.n) {
        const PendingEmbed& tok = e0->second.ids ? e0->second : e1->second;
        const PendingEmbed& pos = e0->second.ids ? e1->second : e0->second;
        float* y = static_cast<float*>(make_dev(n.out[0], INFERC_DT_F32, get(n.in[0]).shape).dev);
        if (!dry) {
          ih::embed_add_at(ctx, tok.table, tok.rows, tok.ids, pos.table, pos.rows, decode_pos,
                           tok.n, tok.feat, y, gather_err);
          dev_gather = true;
        }
        pending_embed.erase(n.in[0]);
        pending_embed.erase(n.in[1]);
        return;
      }
      for (int k = 0; k < 2; ++k) materialize_embed(n.in[size_t(k)]);
    }
    const Value& a0 = in(0);
    const Value& b0 = in(1);
    if (a0.host && b0.host && a0.dtype == INFERC_DT_I64 && b0.dtype == INFERC_DT_I64 &&
        b0.numel() == 1) {
      std::vector<int64_t> r = host_i64(a0, "Add");
      const int64_t s = b0.host_at<int64_t>(0);
      for (auto& e : r) e += s;
      make_host(n.out[0], INFERC_DT_I64, a0.shape, r.data());
      return;
    }
    if (a0.dtype != INFERC_DT_F32 || b0.dtype != INFERC_DT_F32 ||
        (a0.host && b0.host && a0.numel() <= 65536 && b0.numel() <= 65536) ||
        !(a0.numel() == b0.numel() || suffix_broadcast(a0.shape, b0.shape) ||
          suffix_broadcast(b0.shape, a0.shape))) {
      generic_binary(n, kEwAdd);
      return;
    }
    // the larger operand carries the output shape; the other broadcasts as a suffix
    const bool swap = b0.numel() > a0.numel();
    const std::string& an = swap ? n.in[1] : n.in[0];
    const std::string& bn = swap ? n.in[0] : n.in[1];
    const Value& a = get(an);
    const Value& b = get(bn);
    IH_REQUIRE(b.numel() == a.numel() || suffix_broadcast(a.shape, b.shape), INFERC_ERR_UNSUPPORTED,
               "Add: only suffix broadcasts are supported, got " + shape_str(a.shape) + " + " +
                   shape_str(b.shape));
    std::vector<int64_t> os = a.shape;
    if (b.numel() == a.numel() && b.shape.size() > a.shape.size()) os = b.shape;
    const float* ap = static_cast<const float*>(dev_of(an));
    const float* bp = static_cast<const float*>(dev_of(bn));
    float* y = static_cast<float*>(make_dev(n.out[0], INFERC_DT_F32, os).dev);
    // y = a + b elementwise is commutative in IEEE arithmetic, so swapping the
    // operands for the broadcast does not change any result bit.
    if (!dry) {
      add_bcast(ctx, a.numel(), ap, bp, b.numel(), y);
    }
    return;
  }
  if (op == "Equal") {
    if (eq_done.count(n.out[0])) return;  // computed by a LayerNorm launch
    const Value& a = in(0);
    const Value& b = in(1);
    if (a.dtype != INFERC_DT_I64 || b.dtype != INFERC_DT_I64 || (a.host && b.host) ||
        !(b.numel() == a.numel() || b.numel() == 1 || suffix_broadcast(a.shape, b.shape)) ||
        b.numel() > a.numel()) {
      generic_binary(n, kEwEqual);
      return;
    }
    uint8_t* y = static_cast<uint8_t*>(make_dev(n.out[0], INFERC_DT_BOOL, a.shape).dev);
    if (!dry) {
      equal_i64(ctx, a.numel(), static_cast<const int64_t*>(dev_of(n.in[0])),
                static_cast<const int64_t*>(dev_of(n.in[1])), b.numel(), y);
    }
    return;
  }
  if (op == "Gather") {
    const Value& data = in(0);
    const Value& idx = in(1);
    int64_t axis = attr_int(n, "axis", 0);
    const int64_t r = int64_t(data.shape.size());
    if (axis < 0) axis += r;
    IH_REQUIRE(axis >= 0 && axis < r, INFERC_ERR_ARG, "Gather: axis out of range");
    auto lnf = n.attrs.find("__ln_g");
    if (lnf != n.attrs.end() && axis == r - 1) {
      // The peephole moved the LayerNorm of the data into the Gemm reading
      // this result, but a gather along the feature axis does not commute
      // with it: normalize the data here, gather from that, and let the
      // Gemm read plain rows.
      require_f32(data, "data");
      const int64_t feat = data.shape.back();
      IH_REQUIRE(inits.at(lnf->second).numel() == feat, INFERC_ERR_SHAPE,
                 "LayerNorm: scale/bias size mismatch with feature dim");
      inferc_graph::Node m = n;
      m.attrs.erase("__ln_g");
      m.in[0] = "__lnfull:" + n.out[0];
      float* t = static_cast<float*>(make_dev(m.in[0], INFERC_DT_F32, data.shape).dev);
      if (!dry && feat > 0) {
        layernorm_res_period(ctx, data.numel() / feat, feat,
                             static_cast<const float*>(dev_of(n.in[0])), nullptr, 1,
                             static_cast<const float*>(dev_of(lnf->second)),
                             static_cast<const float*>(dev_of(n.attrs.at("__ln_b"))),
                             std::stof(n.attrs.at("__ln_eps")), t);
      }
      ln_gemm_off.insert(n.out[0]);
      exec_node(m);
      return;
    }
    std::vector<int64_t> os(data.shape.begin(), data.shape.begin() + axis);
    for (int64_t d : idx.shape) os.push_back(d);
    for (int64_t i = axis + 1; i < r; ++i) os.push_back(data.shape[size_t(i)]);
    const size_t ni = node_index(n);
    if (decode && embed_gather_at[ni] && axis == 0 && r == 2 && data.dtype == INFERC_DT_F32 &&
        idx.dtype == INFERC_DT_I64 && (pos_gather_at[ni] || !idx.host)) {
      // rows for the embedding Add that reads this output (one kernel there)
      PendingEmbed pe{static_cast<const float*>(dev_of(n.in[0])), data.shape[0], data.shape[1],
                      idx.numel(), nullptr};
      if (pos_gather_at[ni]) {
        const std::vector<int64_t> ix = host_i64(idx, "Gather");
        for (size_t i = 0; i < ix.size(); ++i)
          IH_REQUIRE(ix[i] == int64_t(i), INFERC_ERR_UNSUPPORTED,
                     "Gather: decode mode needs the positions of the new tokens in order");
        IH_REQUIRE(decode_len + int64_t(ix.size()) <= data.shape[0], INFERC_ERR_SHAPE,
                   "Gather: position past the end of the embedding table");
      } else {
        pe.ids = static_cast<const int64_t*>(dev_of(n.in[1]));
      }
      ih::Value v;
      v.dtype = INFERC_DT_F32;
      v.shape = os;
      vals[n.out[0]] = v;
      pending_embed[n.out[0]] = pe;
      return;
    }
    if (decode && pos_gather_at[ni]) {
      // decode mode: the indices, walked for an empty past, are the new
      // positions 0 .. n-1; the rows are those past the device's past length
      IH_REQUIRE(idx.host && idx.dtype == INFERC_DT_I64, INFERC_ERR_UNSUPPORTED,
                 "Gather: decode mode needs host-known position indices");
      const std::vector<int64_t> ix = host_i64(idx, "Gather");
      for (size_t i = 0; i < ix.size(); ++i)
        IH_REQUIRE(ix[i] == int64_t(i), INFERC_ERR_UNSUPPORTED,
                   "Gather: decode mode needs the positions of the new tokens in order");
      require_f32(data, "data");
      int64_t inner = 1;
      for (int64_t i = axis + 1; i < r; ++i) inner *= data.shape[size_t(i)];
      const int64_t ad = data.shape[size_t(axis)];
      IH_REQUIRE(axis == 0, INFERC_ERR_UNSUPPORTED, "Gather: decode mode gathers rows (axis 0)");
      IH_REQUIRE(decode_len + int64_t(ix.size()) <= ad, INFERC_ERR_SHAPE,
                 "Gather: position past the end of the embedding table");
      const float* dp = static_cast<const float*>(dev_of(n.in[0]));
      float* y = static_cast<float*>(make_dev(n.out[0], INFERC_DT_F32, os).dev);
      if (!dry) gather_rows_at(ctx, ad, inner, dp, decode_pos, idx.numel(), y);
      return;
    }
    if (data.host && idx.host && (data.dtype == INFERC_DT_I64 || data.dtype == INFERC_DT_I32) &&
        axis == 0 && r == 1) {
      // host shape plumbing (e.g. Gather(Shape(x), 1))
      std::vector<int64_t> d = host_i64(data, "Gather"), ix = host_i64(idx, "Gather");
      std::vector<int64_t> res;
      for (int64_t i : ix) {
        if (i < 0) i += int64_t(d.size());
        IH_REQUIRE(i >= 0 && i < int64_t(d.size()), INFERC_ERR_ARG, "Gather: index out of range");
        res.push_back(d[size_t(i)]);
      }
      make_host(n.out[0], INFERC_DT_I64, os, res.data());
      return;
    }
    if (data.dtype != INFERC_DT_F32 || host_foldable(n, numel_of(os))) {
      // any element type: on the host when everything is known there, else
      // on the device with host-validated or device indices
      int64_t outer = 1, inner = 1;
      for (int64_t i = 0; i < axis; ++i) outer *= data.shape[size_t(i)];
      for (int64_t i = axis + 1; i < r; ++i) inner *= data.shape[size_t(i)];
      const int64_t ad = data.shape[size_t(axis)];
      IH_REQUIRE(idx.dtype == INFERC_DT_I64 || idx.dtype == INFERC_DT_I32, INFERC_ERR_UNSUPPORTED,
                 "Gather: integer indices only");
      if (host_foldable(n, numel_of(os))) {
        const std::vector<int64_t> ix = host_i64(idx, "Gather");
        void* y = make_host_buf(n.out[0], data.dtype, os);
        ew_gather(nullptr, data.dtype, outer, ad, inner, host_of(n.in[0]), ix.data(),
                  int64_t(ix.size()), y);
        return;
      }
      if (idx.host) {
        for (int64_t i : host_i64(idx, "Gather"))
          IH_REQUIRE(i >= -ad && i < ad, INFERC_ERR_ARG, "Gather: index out of range");
      }
      IH_REQUIRE(idx.dtype == INFERC_DT_I64, INFERC_ERR_UNSUPPORTED,
                 "Gather: device indices must be int64");
      const void* xp = dev_of(n.in[0]);
      const int64_t* ip = static_cast<const int64_t*>(dev_of(n.in[1]));
      void* y = make_dev(n.out[0], data.dtype, os).dev;
      if (!dry) {
        ew_gather(ctx, data.dtype, outer, ad, inner, xp, ip, idx.numel(), y,
                  idx.host ? nullptr : gather_err);
        dev_gather = dev_gather || !idx.host;
      }
      return;
    }
    require_f32(data, "data");
    int64_t outer = 1, inner = 1;
    for (int64_t i = 0; i < axis; ++i) outer *= data.shape[size_t(i)];
    for (int64_t i = axis + 1; i < r; ++i) inner *= data.shape[size_t(i)];
    const int64_t ad = data.shape[size_t(axis)];
    const float* dp = static_cast<const float*>(dev_of(n.in[0]));
    if (idx.host && outer == 1 && idx.dtype == INFERC_DT_I64 && idx.numel() > 0) {
      // Host-known consecutive indices k, k+1, ... with nothing outside the
      // axis select one contiguous range (position ids from Range, the CLS
      // row of a single sequence): the output is a view, no kernel runs.
      const std::vector<int64_t> ix = host_i64(idx, "Gather");
      const int64_t k0 = ix[0] < 0 ? ix[0] + ad : ix[0];
      bool run = true;
      for (size_t i = 0; i < ix.size() && run; ++i) {
        const int64_t v = ix[i] < 0 ? ix[i] + ad : ix[i];
        run = v >= 0 && v < ad && v == k0 + int64_t(i);
      }
      if (run) {
        ih::Value v;
        v.dtype = INFERC_DT_F32;
        v.shape = os;
        v.dev = const_cast<float*>(dp) + k0 * inner;
        vals[n.out[0]] = v;
        return;
      }
    }
    if (gather_ln.count(n.out[0]) && !idx.host && idx.dtype == INFERC_DT_I64 && outer == 1) {
      // rows for the one LayerNorm reading this output, which gathers them
      ih::Value v;
      v.dtype = INFERC_DT_F32;
      v.shape = os;
      vals[n.out[0]] = v;
      pending_gather[n.out[0]] = PendingGather{
          dp, static_cast<const int64_t*>(dev_of(n.in[1])), ad, inner, idx.numel()};
      return;
    }
    float* y = static_cast<float*>(make_dev(n.out[0], INFERC_DT_F32, os).dev);
    // one device gather for any axis; host-known indices are validated here
    // and uploaded once, device indices set the executor's sticky flag
    if (idx.host) {
      for (int64_t i : host_i64(idx, "Gather"))
        IH_REQUIRE(i >= -ad && i < ad, INFERC_ERR_ARG, "Gather: index out of range");
    } else {
      IH_REQUIRE(idx.dtype == INFERC_DT_I64, INFERC_ERR_UNSUPPORTED,
                 "Gather: device indices must be int64");
    }
    IH_REQUIRE(idx.dtype == INFERC_DT_I64, INFERC_ERR_UNSUPPORTED, "Gather: int64 indices only");
    const int64_t* ip = static_cast<const int64_t*>(dev_of(n.in[1]));
    if (!dry) {
      gather_axis(ctx, outer, ad, inner, dp, ip, idx.numel(), y, idx.host ? nullptr : gather_err);
      dev_gather = dev_gather || !idx.host;
    }
    return;
  }
  if (op == "Shape") {
    const Value& x = in(0);
    std::vector<int64_t> s = x.shape;
    make_host(n.out[0], INFERC_DT_I64, {int64_t(s.size())}, s.data());
    return;
  }
  if (op == "Range") {
    const int64_t s = host_i64(in(0), "Range")[0], l = host_i64(in(1), "Range")[0],
                  d = host_i64(in(2), "Range")[0];
    IH_REQUIRE(d != 0, INFERC_ERR_ARG, "Range: delta must be non-zero");
    std::vector<int64_t> r;
    for (int64_t v = s; d > 0 ? v < l : v > l; v += d) r.push_back(v);
    make_host(n.out[0], INFERC_DT_I64, {int64_t(r.size())}, r.data());
    return;
  }
  if (op == "Unsqueeze" || op == "Squeeze" || op == "Reshape" || op == "Identity" ||
      op == "Flatten") {
    const Value& x = in(0);
    std::vector<int64_t> s = x.shape;
    if (op == "Unsqueeze" || op == "Squeeze") {
      std::vector<int64_t> axes =
          n.in.size() >= 2 ? host_i64(in(1), op) : attr_ints(n, "axes");
      if (op == "Unsqueeze") {
        const int64_t out_r = int64_t(s.size() + axes.size());
        for (auto& a : axes) if (a < 0) a += out_r;
        std::vector<int64_t> os;
        size_t k = 0;
        for (int64_t i = 0; i < out_r; ++i) {
          bool ins = false;
          for (int64_t a : axes) ins = ins || a == i;
          if (ins) os.push_back(1);
          else os.push_back(s[k++]);
        }
        s = os;
      } else {
        const int64_t r = int64_t(s.size());
        for (auto& a : axes) if (a < 0) a += r;
        std::vector<int64_t> os;
        for (int64_t i = 0; i < r; ++i) {
          bool drop = axes.empty() ? s[size_t(i)] == 1 : false;
          for (int64_t a : axes) drop = drop || a == i;
          if (!drop) os.push_back(s[size_t(i)]);
        }
        s = os;
      }
    } else if (op == "Reshape") {
      std::vector<int64_t> t = host_i64(in(1), "Reshape");
      int64_t known = 1, neg = -1;
      for (size_t i = 0; i < t.size(); ++i) {
        if (t[i] == 0) t[i] = s[i];
        if (t[i] == -1) neg = int64_t(i);
        else known *= t[i];
      }
      if (neg >= 0) t[size_t(neg)] = known ? x.numel() / known : 0;
      s = t;
    } else if (op == "Flatten") {
      int64_t axis = attr_int(n, "axis", 1);
      if (axis < 0) axis += int64_t(s.size());
      int64_t a = 1;
      for (int64_t i = 0; i < axis; ++i) a *= s[size_t(i)];
      s = {a, x.numel() / (a ? a : 1)};
    }
    alias(n.out[0], x, s);
    return;
  }
  if (op == "Split") {
    const Value& x = in(0);
    require_f32(x, "X");
    int64_t axis = attr_int(n, "axis", 0);
    const int64_t r = int64_t(x.shape.size());
    if (axis < 0) axis += r;
    IH_REQUIRE(axis >= 0 && axis < r, INFERC_ERR_ARG, "Split: axis out of range");
    std::vector<int64_t> sizes =
        n.in.size() >= 2 && !n.in[1].empty() ? host_i64(in(1), "Split") : attr_ints(n, "split");
    if (sizes.empty()) {
      const int64_t total = x.shape[size_t(axis)], k = int64_t(n.out.size());
      IH_REQUIRE(k > 0 && total % k == 0, INFERC_ERR_SHAPE, "Split: cannot infer split sizes");
      sizes.assign(size_t(k), total / k);
    }
    int64_t outer = 1, inner = 1;
    for (int64_t i = 0; i < axis; ++i) outer *= x.shape[size_t(i)];
    for (int64_t i = axis + 1; i < r; ++i) inner *= x.shape[size_t(i)];
    IH_REQUIRE(int64_t(sizes.size()) <= int64_t(n.out.size()), INFERC_ERR_ARG,
               "Split: more parts than outputs");
    if (outer == 1) {
      // nothing before the axis: each part is a contiguous range of X, read
      // in place (one decode row split into q, k, v)
      int64_t off = 0;
      for (int64_t sz : sizes) off += sz;
      IH_REQUIRE(off == x.shape[size_t(axis)], INFERC_ERR_SHAPE, "Split: sizes do not add up");
      const float* xp = static_cast<const float*>(dev_of(n.in[0]));
      off = 0;
      for (size_t i = 0; i < sizes.size(); ++i) {
        Value v;
        v.dtype = INFERC_DT_F32;
        v.shape = x.shape;
        v.shape[size_t(axis)] = sizes[i];
        v.dev = const_cast<float*>(xp) + off * inner;
        vals[n.out[i]] = v;
        off += sizes[i];
      }
      return;
    }
    std::vector<float*> outs;
    for (size_t i = 0; i < sizes.size() && i < n.out.size(); ++i) {
      std::vector<int64_t> s = x.shape;
      s[size_t(axis)] = sizes[i];
      outs.push_back(static_cast<float*>(make_dev(n.out[i], INFERC_DT_F32, s).dev));
    }
    IH_REQUIRE(outs.size() == sizes.size(), INFERC_ERR_ARG, "Split: fewer outputs than parts");
    if (!dry) {
      IH_REQUIRE(inferc_hip_split_f32(ctx, outer, x.shape[size_t(axis)], inner,
                                      int64_t(sizes.size()), sizes.data(),
                                      static_cast<const float*>(dev_of(n.in[0])), outs.data()) == 0,
                 INFERC_ERR_SHAPE, inferc_hip_last_error());
    }
    return;
  }
  if (op == "Concat" && n.in.size() == 1) {
    const Value& x0 = in(0);
    alias(n.out[0], x0, x0.shape);
    return;
  }
  if (op == "Concat") {
    int64_t axis = attr_int(n, "axis", 0);
    const Value& x0 = in(0);
    const int64_t r = int64_t(x0.shape.size());
    if (axis < 0) axis += r;
    IH_REQUIRE(axis >= 0 && axis < r, INFERC_ERR_ARG, "Concat: axis out of range");
    std::vector<int64_t> os = x0.shape;
    os[size_t(axis)] = 0;
    std::vector<int64_t> sizes;
    for (size_t i = 0; i < n.in.size(); ++i) {
      const Value& p = in(i);
      IH_REQUIRE(p.shape.size() == x0.shape.size() && p.dtype == x0.dtype, INFERC_ERR_SHAPE,
                 "Concat: rank/dtype mismatch");
      for (int64_t d = 0; d < r; ++d)
        IH_REQUIRE(d == axis || p.shape[size_t(d)] == x0.shape[size_t(d)], INFERC_ERR_SHAPE,
                   "Concat: dim mismatch outside axis");
      sizes.push_back(p.shape[size_t(axis)]);
      os[size_t(axis)] += p.shape[size_t(axis)];
    }
    if (host_foldable(n, numel_of(os)) && (x0.dtype != INFERC_DT_I64 || r != 1)) {
      // any element type on the host: parts laid side by side along `axis`
      const size_t eb = dtype_size(x0.dtype);
      int64_t outer = 1, inner = 1;
      for (int64_t i = 0; i < axis; ++i) outer *= os[size_t(i)];
      for (int64_t i = axis + 1; i < r; ++i) inner *= os[size_t(i)];
      uint8_t* y = static_cast<uint8_t*>(make_host_buf(n.out[0], x0.dtype, os));
      int64_t at = 0;
      for (size_t i = 0; i < n.in.size(); ++i) {
        const uint8_t* src = static_cast<const uint8_t*>(host_of(n.in[i]));
        const int64_t w = sizes[i] * inner;
        for (int64_t o = 0; o < outer; ++o)
          std::memcpy(y + size_t((o * os[size_t(axis)] * inner + at * inner)) * eb,
                      src + size_t(o * w) * eb, size_t(w) * eb);
        at += sizes[i];
      }
      return;
    }
    if (x0.dtype == INFERC_DT_I64) {
      bool all_host = true;
      for (size_t i = 0; i < n.in.size(); ++i) all_host = all_host && in(i).host != nullptr;
      IH_REQUIRE(all_host && r == 1, INFERC_ERR_UNSUPPORTED, "Concat: int64 only as shape math");
      std::vector<int64_t> res;
      for (size_t i = 0; i < n.in.size(); ++i) {
        auto v = host_i64(in(i), "Concat");
        res.insert(res.end(), v.begin(), v.end());
      }
      make_host(n.out[0], INFERC_DT_I64, os, res.data());
      return;
    }
    require_f32(x0, "inputs");
    int64_t outer = 1, inner = 1;
    for (int64_t i = 0; i < axis; ++i) outer *= os[size_t(i)];
    for (int64_t i = axis + 1; i < r; ++i) inner *= os[size_t(i)];
    std::vector<const float*> parts;
    for (size_t i = 0; i < n.in.size(); ++i) parts.push_back(static_cast<const float*>(dev_of(n.in[i])));
    float* y = static_cast<float*>(make_dev(n.out[0], INFERC_DT_F32, os).dev);
    if (!dry) {
      IH_REQUIRE(inferc_hip_concat_f32(ctx, outer, inner, int64_t(parts.size()), sizes.data(),
                                       parts.data(), y) == 0,
                 INFERC_ERR_SHAPE, inferc_hip_last_error());
    }
    return;
  }
  if (exec_generic(n)) return;
  fail(INFERC_ERR_UNSUPPORTED, "Executor: unsupported op '" + op + "' (node: " + n.name + ")");
}

// Binary op with numpy broadcasting: folded on the host when every input is
// host-known and the result small, else one device kernel.
void inferc_executor::generic_binary(const inferc_graph::Node& n, int ewop) {
  using namespace ih;
  IH_REQUIRE(n.in.size() == 2, INFERC_ERR_ARG, n.op + ": needs two inputs");
  Value a = get(n.in[0]);
  Value b = get(n.in[1]);
  std::string bn = n.in[1];
  if (ewop == kEwPow && b.dtype != a.dtype) {
    // a float base with an integer exponent: the exponent as float32
    IH_REQUIRE(b.host != nullptr, INFERC_ERR_UNSUPPORTED, "Pow: exponent type differs");
    std::vector<float> e(size_t(b.numel()));
    ew_cast(nullptr, b.dtype, INFERC_DT_F32, b.numel(), b.host->data(), e.data());
    bn = n.out[0] + "__exp";
    make_host(bn, INFERC_DT_F32, b.shape, e.data());
    b = get(bn);
  }
  IH_REQUIRE(a.dtype == b.dtype, INFERC_ERR_UNSUPPORTED,
             n.op + ": operand types differ (" + std::to_string(a.dtype) + " vs " +
                 std::to_string(b.dtype) + ")");
  const std::vector<int64_t> os = ew_broadcast_shape({a.shape, b.shape});
  const int odt = ew_binary_out_dtype(ewop, a.dtype);
  if (a.host && b.host && numel_of(os) <= (int64_t(1) << 16)) {
    void* y = make_host_buf(n.out[0], odt, os);
    ew_binary(nullptr, ewop, a.dtype, os, a.host->data(), a.shape, b.host->data(), b.shape, y);
    return;
  }
  const void* ap = dev_of(n.in[0]);
  const void* bp = dev_of(bn);
  void* y = make_dev(n.out[0], odt, os).dev;
  if (!dry) ew_binary(ctx, ewop, a.dtype, os, ap, a.shape, bp, b.shape, y);
}

// FusedAttentionPast(q, k, v, past_k, past_v, mask) -> (ctx, present_k,
// present_v): q/k/v [B,S,H] new rows, past_* [B,nH,P,dh], present_* =
// Concat(past, heads of k/v) along the position axis, ctx = attention of
// the S new rows over the T = P + S present keys.
//  - Unbound: present_* are materialised (past rows copied, new rows
//    written) and attention reads them.
//  - Bound to a KV cache (bind_kv_cache): the node keeps K/V in a
//    persistent [B, nH, max_t, dh] cache. A past input with data seeds rows
//    [0, P); a shape-only past input says the cache already holds them. The
//    new rows are appended at P, attention reads the cache, and present_*
//    are views of its first T rows, copied out only when asked for.
// A's rows through a LayerNorm that the peephole moved onto a Gemm or
// MatMul (it preceded A directly, through a view, or through a Gather): on
// the one-row GEMV route the GEMV's LayerNorm prologue applies it, else a
// LayerNorm of A's rows into a buffer that becomes A.
void inferc_executor::ln_prologue(const inferc_graph::Node& n, ih::GemmArgs& g) {
  using namespace ih;
  auto ln = n.attrs.find("__ln_g");
  if (ln == n.attrs.end()) return;
  const float* lg = static_cast<const float*>(dev_of(ln->second));
  const float* lb = static_cast<const float*>(dev_of(n.attrs.at("__ln_b")));
  const float eps = std::stof(n.attrs.at("__ln_eps"));
  IH_REQUIRE(!g.trans_a && inits.at(ln->second).numel() == g.K, INFERC_ERR_SHAPE,
             n.op + ": LayerNorm of A: scale size must equal K");
  auto lx = n.attrs.find("__ln_x");
  IH_REQUIRE(lx == n.attrs.end() || get(lx->second).shape.back() == g.K, INFERC_ERR_UNSUPPORTED,
             n.op + ": the view between a LayerNorm and A must keep the feature axis");
  if (gemm_gemv_route(ctx, g)) {
    g.gemv_ln_g = lg;
    g.gemv_ln_b = lb;
    g.gemv_ln_eps = eps;
  } else {
    float* t = static_cast<float*>(buf("__lnrows:" + n.out[0], size_t(g.M * g.K) * 4));
    IH_REQUIRE(g.lda == g.K && g.batch == 1, INFERC_ERR_SHAPE,
               n.op + ": LayerNorm of A needs dense rows");
    if (!dry) layernorm_res_period(ctx, g.M, g.K, g.A, nullptr, 1, lg, lb, eps, t);
    g.A = t;
  }
}

void inferc_executor::exec_attention_past(const inferc_graph::Node& n) {
  using namespace ih;
  IH_REQUIRE(n.in.size() >= 5 && n.out.size() == 3, INFERC_ERR_ARG,
             "FusedAttentionPast: needs q, k, v, past_k, past_v[, mask] and three outputs");
  const Value& q = get(n.in[0]);
  IH_REQUIRE(q.dtype == INFERC_DT_F32 && q.shape.size() == 3, INFERC_ERR_SHAPE,
             "FusedAttentionPast: q must be float32 [B,S,H]");
  IH_REQUIRE(get(n.in[1]).shape == q.shape && get(n.in[2]).shape == q.shape, INFERC_ERR_SHAPE,
             "FusedAttentionPast: q/k/v shapes differ");
  const int64_t B = q.shape[0], S = q.shape[1], H = q.shape[2];
  const int64_t dh = attr_int(n, "head_dim", 64);
  IH_REQUIRE(dh > 0 && H % dh == 0, INFERC_ERR_SHAPE, "FusedAttentionPast: H % head_dim != 0");
  const int64_t nH = H / dh;
  const bool has_past = !n.in[3].empty() && !n.in[4].empty();
  Value pk, pv;
  if (has_past) {
    pk = get(n.in[3]);
    pv = get(n.in[4]);
  } else {
    pk.dtype = pv.dtype = INFERC_DT_F32;
    pk.shape = pv.shape = {B, nH, 0, dh};
  }
  IH_REQUIRE(pk.shape.size() == 4 && pk.shape[0] == B && pk.shape[1] == nH && pk.shape[3] == dh &&
                 pv.shape == pk.shape,
             INFERC_ERR_SHAPE, "FusedAttentionPast: past must be [B, nH, P, head_dim]");
  const int64_t P = pk.shape[2], T = P + S;
  CacheAttnArgs a;
  a.B = B; a.S = S; a.nH = nH; a.dh = dh; a.T = T;
  a.fill = attr_float(n, "fill", -3.0e38f);
  a.q = static_cast<const float*>(dev_of(n.in[0]));
  a.ldq = a.ldo = H;
  // (decode mode ignores the mask: it holds only the new positions, all kept)
  if (!decode && n.in.size() >= 6 && !n.in[5].empty()) {
    const Value& m = get(n.in[5]);
    IH_REQUIRE(m.dtype == INFERC_DT_BOOL || m.dtype == INFERC_DT_U8, INFERC_ERR_UNSUPPORTED,
               "FusedAttentionPast: mask must be bool");
    IH_REQUIRE(m.shape.size() <= 4, INFERC_ERR_SHAPE, "FusedAttentionPast: mask rank > 4");
    const std::vector<int64_t> full = {B, nH, S, T};
    for (size_t i = 0; i < m.shape.size(); ++i) {
      const int64_t d = m.shape[i], f = full[4 - m.shape.size() + i];
      IH_REQUIRE(d == f || d == 1, INFERC_ERR_SHAPE,
                 "FusedAttentionPast: mask " + shape_str(m.shape) + " does not broadcast to " +
                     shape_str(full));
    }
    a.mask = static_cast<const uint8_t*>(dev_of(n.in[5]));
    mask_strides(m.shape, a.ms);
  }
  const float* kn = static_cast<const float*>(dev_of(n.in[1]));
  const float* vn = static_cast<const float*>(dev_of(n.in[2]));
  // the attention kernel appends the new rows itself
  a.kn = kn;
  a.vn = vn;
  a.ldn = H;
  a.out = static_cast<float*>(make_dev(n.out[0], INFERC_DT_F32, q.shape).dev);
  const std::vector<int64_t> present = {B, nH, T, dh};
  auto has_data = [&](const Value& v) { return v.dev != nullptr || v.host != nullptr; };
  if (kv_max_t == 0) {
    IH_REQUIRE(P == 0 || (has_data(pk) && has_data(pv)), INFERC_ERR_STATE,
               "FusedAttentionPast: past has no data and no KV cache is bound");
    float* ko = static_cast<float*>(make_dev(n.out[1], INFERC_DT_F32, present).dev);
    float* vo = static_cast<float*>(make_dev(n.out[2], INFERC_DT_F32, present).dev);
    const float* pkp = P ? static_cast<const float*>(dev_of(n.in[3])) : nullptr;
    const float* pvp = P ? static_cast<const float*>(dev_of(n.in[4])) : nullptr;
    a.kc = ko;
    a.vc = vo;
    a.max_t = T;
    if (!dry) {
      if (P) {
        copy2d(ctx, ko, T * dh, pkp, P * dh, P * dh, B * nH);
        copy2d(ctx, vo, T * dh, pvp, P * dh, P * dh, B * nH);
      }
      cache_attention(ctx, a);
    }
    return;
  }
  if (decode) {
    IH_REQUIRE(P == 0, INFERC_ERR_STATE,
               "FusedAttentionPast: in decode mode the past inputs carry no positions (length 0)");
    a.mask = nullptr;  // all ones: every cached key and the new ones (one row a step)
    a.pos = decode_pos;
    a.T = decode_len + S;
    decode_step = S;
  }
  const int64_t Tc = decode ? decode_len + S : T;  // positions held after this run
  IH_REQUIRE(Tc <= kv_max_t, INFERC_ERR_SHAPE,
             "FusedAttentionPast: " + std::to_string(Tc) + " positions exceed the KV cache (" +
                 std::to_string(kv_max_t) + ")");
  KvCache& c = kv[n.name];
  if (c.k == nullptr || c.B != B || c.nH != nH || c.dh != dh) {
    IH_REQUIRE(!dry, INFERC_ERR_STATE, "a dry-run executor has no KV cache");
    IH_REQUIRE(!ctx->capturing, INFERC_ERR_STATE, "KV cache allocation during graph capture");
    if (c.k) {
      IH_HIP(hipStreamSynchronize(ctx->stream));
      ++buf_gen;
      (void)hipFree(c.k);
      (void)hipFree(c.v);
    }
    c = KvCache{};
    const size_t bytes = size_t(B * nH * kv_max_t * dh) * sizeof(float);
    IH_HIP(hipMalloc(&c.k, bytes));
    IH_HIP(hipMalloc(&c.v, bytes));
    c.B = B; c.nH = nH; c.dh = dh;
  }
  const bool seed = !decode && P > 0 && has_data(pk) && has_data(pv);
  IH_REQUIRE(decode || seed || P <= c.len, INFERC_ERR_STATE,
             "FusedAttentionPast: the KV cache holds " + std::to_string(c.len) +
                 " positions, the past says " + std::to_string(P));
  a.kc = c.k;
  a.vc = c.v;
  a.max_t = kv_max_t;
  if (seed) {
    const float* pkp = static_cast<const float*>(dev_of(n.in[3]));
    const float* pvp = static_cast<const float*>(dev_of(n.in[4]));
    copy2d(ctx, c.k, kv_max_t * dh, pkp, P * dh, P * dh, B * nH);
    copy2d(ctx, c.v, kv_max_t * dh, pvp, P * dh, P * dh, B * nH);
  }
  if (!dry) {
    // A decode step of one sequence at head_dim 64 takes the native
    // decoder's kernel (one 8-wave block per head over the [nH, max_t, 64]
    // cache, appending the step's K/V row at the device position): 4.8 us
    // per launch traced, against 5.7 for the general one. The scale
    // 1/sqrt(64) is a power of two, so its division there equals the
    // multiplication here.
    if (decode && B == 1 && S == 1 && dh == 64 && aligned16(a.q) && aligned16(kn) &&
        aligned16(vn) && aligned16(c.k) && aligned16(c.v))
      kv_append_attend(ctx, nH, dh, kv_max_t, decode_pos, a.q, kn, vn, c.k, c.v, a.out);
    else
      cache_attention(ctx, a);
  }
  c.len = Tc;
  for (int o = 1; o <= 2; ++o) {
    Value v;
    v.dtype = INFERC_DT_F32;
    v.shape = {B, nH, Tc, dh};
    vals[n.out[size_t(o)]] = v;  // no contiguous data: read through the view
    cache_views[n.out[size_t(o)]] = CacheView{o == 1 ? c.k : c.v, B * nH, Tc, dh, kv_max_t};
  }
}

// The ops of exported graphs outside the fused set: Constant,
// ConstantOfShape, Cast, unary math, binary arithmetic / comparison /
// logic, Where, Expand, Transpose, Slice and ReduceMean
// (src/runtime/executor.cc:226-339). Returns false for an op it does not
// know.
bool inferc_executor::exec_generic(const inferc_graph::Node& n) {
  using namespace ih;
  const std::string& op = n.op;
  static const std::map<std::string, int> binary = {
      {"Sub", kEwSub}, {"Mul", kEwMul}, {"Div", kEwDiv}, {"Pow", kEwPow}, {"Max", kEwMax},
      {"Min", kEwMin}, {"Less", kEwLess}, {"LessOrEqual", kEwLessOrEqual},
      {"Greater", kEwGreater}, {"GreaterOrEqual", kEwGreaterOrEqual}, {"And", kEwAnd},
      {"Or", kEwOr}, {"Xor", kEwXor}};
  static const std::map<std::string, int> unary = {
      {"Sqrt", kEwSqrt}, {"Erf", kEwErf}, {"Tanh", kEwTanh}, {"Neg", kEwNeg},
      {"Abs", kEwAbs}, {"Exp", kEwExp}, {"Log", kEwLog}, {"Reciprocal", kEwReciprocal},
      {"Sigmoid", kEwSigmoid}, {"Floor", kEwFloor}, {"Ceil", kEwCeil}, {"Not", kEwNot}};
  auto bi = binary.find(op);
  if (bi != binary.end()) {
    generic_binary(n, bi->second);
    return true;
  }
  auto ui = unary.find(op);
  if (ui != unary.end()) {
    const Value& x = get(n.in.at(0));
    if (host_foldable(n, x.numel())) {
      void* y = make_host_buf(n.out[0], x.dtype, x.shape);
      ew_unary(nullptr, ui->second, x.dtype, x.numel(), x.host->data(), y);
    } else {
      const void* xp = dev_of(n.in[0]);
      void* y = make_dev(n.out[0], x.dtype, x.shape).dev;
      if (!dry) ew_unary(ctx, ui->second, x.dtype, x.numel(), xp, y);
    }
    return true;
  }
  if (op == "Constant") {
    auto tv = n.tattrs.find("value");
    if (tv != n.tattrs.end()) {
      (void)dtype_size(tv->second.dtype);
      make_host(n.out[0], tv->second.dtype, tv->second.shape, tv->second.data.data());
      return true;
    }
    if (n.attrs.count("value_float")) {
      const float f = attr_float(n, "value_float", 0.0f);
      make_host(n.out[0], INFERC_DT_F32, {}, &f);
    } else if (n.attrs.count("value_int")) {
      const int64_t i = attr_int(n, "value_int", 0);
      make_host(n.out[0], INFERC_DT_I64, {}, &i);
    } else if (n.attrs.count("value_ints")) {
      const std::vector<int64_t> v = attr_ints(n, "value_ints");
      make_host(n.out[0], INFERC_DT_I64, {int64_t(v.size())}, v.data());
    } else {
      fail(INFERC_ERR_UNSUPPORTED, "Constant '" + n.name + "': unsupported value attribute");
    }
    return true;
  }
  if (op == "ConstantOfShape") {
    const std::vector<int64_t> shape = host_i64(get(n.in.at(0)), "ConstantOfShape");
    int dt = INFERC_DT_F32;
    std::vector<uint8_t> one(4, 0);
    auto tv = n.tattrs.find("value");
    if (tv != n.tattrs.end()) {
      dt = tv->second.dtype;
      one = tv->second.data;
      IH_REQUIRE(one.size() == dtype_size(dt), INFERC_ERR_ARG,
                 "ConstantOfShape: value must hold one element");
    }
    const int64_t cnt = numel_of(shape);
    IH_REQUIRE(cnt <= (int64_t(1) << 24), INFERC_ERR_UNSUPPORTED, "ConstantOfShape: too large");
    uint8_t* y = static_cast<uint8_t*>(make_host_buf(n.out[0], dt, shape));
    for (int64_t i = 0; i < cnt; ++i) std::memcpy(y + size_t(i) * one.size(), one.data(), one.size());
    return true;
  }
  if (op == "Cast") {
    const Value& x = get(n.in.at(0));
    const int to = int(attr_int(n, "to", 0));
    (void)dtype_size(to);
    if (to == x.dtype) {
      alias(n.out[0], x, x.shape);
      auto pe = pending_embed.find(n.in[0]);  // rows pending for an embedding Add
      if (pe != pending_embed.end()) {
        const PendingEmbed e = pe->second;
        pending_embed.erase(pe);
        pending_embed[n.out[0]] = e;
      }
      return true;
    }
    if (host_foldable(n, x.numel())) {
      void* y = make_host_buf(n.out[0], to, x.shape);
      ew_cast(nullptr, x.dtype, to, x.numel(), x.host->data(), y);
    } else {
      const void* xp = dev_of(n.in[0]);
      void* y = make_dev(n.out[0], to, x.shape).dev;
      if (!dry) ew_cast(ctx, x.dtype, to, x.numel(), xp, y);
    }
    return true;
  }
  if (op == "Where") {
    const Value& c = get(n.in.at(0)), a = get(n.in.at(1)), b = get(n.in.at(2));
    IH_REQUIRE(c.dtype == INFERC_DT_BOOL || c.dtype == INFERC_DT_U8, INFERC_ERR_UNSUPPORTED,
               "Where: condition must be bool");
    IH_REQUIRE(a.dtype == b.dtype, INFERC_ERR_UNSUPPORTED, "Where: branch types differ");
    const std::vector<int64_t> os = ew_broadcast_shape({c.shape, a.shape, b.shape});
    if (host_foldable(n, numel_of(os))) {
      void* y = make_host_buf(n.out[0], a.dtype, os);
      ew_where(nullptr, a.dtype, os, c.host->data(), c.shape, a.host->data(), a.shape,
               b.host->data(), b.shape, y);
    } else {
      const void* cp = dev_of(n.in[0]);
      const void* ap = dev_of(n.in[1]);
      const void* bp = dev_of(n.in[2]);
      void* y = make_dev(n.out[0], a.dtype, os).dev;
      if (!dry) ew_where(ctx, a.dtype, os, cp, c.shape, ap, a.shape, bp, b.shape, y);
    }
    return true;
  }
  if (op == "Expand") {
    const Value& x = get(n.in.at(0));
    const std::vector<int64_t> target = host_i64(get(n.in.at(1)), "Expand");
    const std::vector<int64_t> os = ew_broadcast_shape({x.shape, target});
    if (os == x.shape) {
      alias(n.out[0], x, os);
      return true;
    }
    if (host_foldable(n, numel_of(os))) {
      void* y = make_host_buf(n.out[0], x.dtype, os);
      ew_expand(nullptr, x.dtype, os, x.host->data(), x.shape, y);
    } else {
      const void* xp = dev_of(n.in[0]);
      void* y = make_dev(n.out[0], x.dtype, os).dev;
      if (!dry) ew_expand(ctx, x.dtype, os, xp, x.shape, y);
    }
    return true;
  }
  if (op == "Transpose") {
    const Value& x = get(n.in.at(0));
    std::vector<int64_t> perm = attr_ints(n, "perm");
    const int64_t r = int64_t(x.shape.size());
    if (perm.empty())
      for (int64_t k = r - 1; k >= 0; --k) perm.push_back(k);
    IH_REQUIRE(int64_t(perm.size()) == r, INFERC_ERR_SHAPE, "Transpose: perm rank mismatch");
    std::vector<int64_t> os;
    for (int64_t p : perm) {
      IH_REQUIRE(p >= 0 && p < r, INFERC_ERR_SHAPE, "Transpose: perm out of range");
      os.push_back(x.shape[size_t(p)]);
    }
    if (host_foldable(n, x.numel())) {
      void* y = make_host_buf(n.out[0], x.dtype, os);
      ew_transpose(nullptr, x.dtype, x.shape, perm, x.host->data(), y);
    } else {
      const void* xp = dev_of(n.in[0]);
      void* y = make_dev(n.out[0], x.dtype, os).dev;
      if (!dry) ew_transpose(ctx, x.dtype, x.shape, perm, xp, y);
    }
    return true;
  }
  if (op == "Slice") {
    // opset 10+: data, starts, ends[, axes[, steps]]; clamping as ONNX
    // specifies (start to [0, d] / [0, d-1] for negative steps, end to
    // [0, d] / [-1, d-1])
    const Value& x = get(n.in.at(0));
    const int64_t r = int64_t(x.shape.size());
    const std::vector<int64_t> starts = host_i64(get(n.in.at(1)), "Slice");
    const std::vector<int64_t> ends = host_i64(get(n.in.at(2)), "Slice");
    std::vector<int64_t> axes, steps;
    if (n.in.size() > 3 && !n.in[3].empty()) axes = host_i64(get(n.in[3]), "Slice");
    if (n.in.size() > 4 && !n.in[4].empty()) steps = host_i64(get(n.in[4]), "Slice");
    if (axes.empty())
      for (size_t i = 0; i < starts.size(); ++i) axes.push_back(int64_t(i));
    if (steps.empty()) steps.assign(starts.size(), 1);
    IH_REQUIRE(ends.size() == starts.size() && axes.size() == starts.size() &&
                   steps.size() == starts.size(),
               INFERC_ERR_SHAPE, "Slice: starts/ends/axes/steps lengths differ");
    std::vector<int64_t> st(size_t(r), 0), sp(size_t(r), 1), os = x.shape;
    for (size_t k = 0; k < starts.size(); ++k) {
      int64_t a = axes[k] < 0 ? axes[k] + r : axes[k];
      IH_REQUIRE(a >= 0 && a < r, INFERC_ERR_ARG, "Slice: axis out of range");
      const int64_t d = x.shape[size_t(a)], step = steps[k];
      IH_REQUIRE(step != 0, INFERC_ERR_ARG, "Slice: step must be non-zero");
      int64_t b = starts[k] < 0 ? starts[k] + d : starts[k];
      int64_t e = ends[k] < 0 ? ends[k] + d : ends[k];
      if (step > 0) {
        b = b < 0 ? 0 : (b > d ? d : b);
        e = e < 0 ? 0 : (e > d ? d : e);
      } else {
        b = b < 0 ? 0 : (b > d - 1 ? d - 1 : b);
        e = e < -1 ? -1 : (e > d - 1 ? d - 1 : e);
      }
      const int64_t len = step > 0 ? (e - b + step - 1) / step : (b - e + (-step) - 1) / (-step);
      st[size_t(a)] = b;
      sp[size_t(a)] = step;
      os[size_t(a)] = len > 0 ? len : 0;
    }
    if (host_foldable(n, numel_of(os))) {
      void* y = make_host_buf(n.out[0], x.dtype, os);
      ew_slice(nullptr, x.dtype, x.shape, st, sp, os, x.host->data(), y);
    } else {
      const void* xp = dev_of(n.in[0]);
      void* y = make_dev(n.out[0], x.dtype, os).dev;
      if (!dry) ew_slice(ctx, x.dtype, x.shape, st, sp, os, xp, y);
    }
    return true;
  }
  if (op == "ReduceMean") {
    const Value& x = get(n.in.at(0));
    IH_REQUIRE(x.dtype == INFERC_DT_F32, INFERC_ERR_UNSUPPORTED, "ReduceMean: float32 only");
    const int64_t r = int64_t(x.shape.size());
    std::vector<int64_t> axes = attr_ints(n, "axes");
    if (n.in.size() > 1 && !n.in[1].empty()) axes = host_i64(get(n.in[1]), "ReduceMean");
    const bool keep = attr_int(n, "keepdims", 1) != 0;
    std::vector<bool> red(size_t(r), axes.empty());
    for (int64_t a : axes) {
      const int64_t aa = a < 0 ? a + r : a;
      IH_REQUIRE(aa >= 0 && aa < r, INFERC_ERR_ARG, "ReduceMean: axis out of range");
      red[size_t(aa)] = true;
    }
    std::vector<int64_t> os;
    for (int64_t d = 0; d < r; ++d) {
      if (!red[size_t(d)]) os.push_back(x.shape[size_t(d)]);
      else if (keep) os.push_back(1);
    }
    if (host_foldable(n, numel_of(os))) {
      float* y = static_cast<float*>(make_host_buf(n.out[0], INFERC_DT_F32, os));
      ew_reduce_mean(nullptr, x.shape, red, reinterpret_cast<const float*>(x.host->data()), y);
    } else {
      const float* xp = static_cast<const float*>(dev_of(n.in[0]));
      float* y = static_cast<float*>(make_dev(n.out[0], INFERC_DT_F32, os).dev);
      if (!dry) ew_reduce_mean(ctx, x.shape, red, xp, y);
    }
    return true;
  }
  return false;
}

void inferc_executor::walk(std::vector<int64_t>* act, bool track) {
  vals.clear();
  dev_gather = false;
  fb_parts = nullptr;
  fb_parts_n = 0;
  ln_gemm_off.clear();
  pending_gather.clear();
  pending_embed.clear();
  eq_done.clear();
  cache_views.clear();
  for (auto& kv : inputs) vals[kv.first] = kv.second.v;
  const bool events = act != nullptr && !dry;
  // A profiled run executes every node, so the tape (and the activation
  // bytes it reports) is the same as without the folded constants.
  const bool fold = act == nullptr;
  const_done.resize(nodes.size(), 0);
  for (size_t i = 0; i < nodes.size(); ++i) {
    const inferc_graph::Node& n = nodes[i];
    if (fold && const_done[i]) continue;
    if (events) IH_HIP(hipEventRecord(prof_ev[i], ctx->stream));
    if (decode && decode_skip_at[i]) {
      if (act) act->push_back(track ? live_activation_bytes() : 0);
      continue;
    }
    try {
      exec_node(n);
      if (fold && n.op == "Constant" && n.out.size() == 1) {
        auto it = vals.find(n.out[0]);
        if (it != vals.end() && it->second.host) {
          consts[n.out[0]] = std::move(it->second);
          vals.erase(it);
          const_done[i] = 1;
        }
      }
    } catch (ih::Error& e) {
      e.msg += " [node '" + n.name + "', op " + n.op + "]";
      throw;
    }
    if (act) act->push_back(track ? live_activation_bytes() : 0);
  }
  if (decode && !dry) {
    if (fb_parts) {
      ih::decode_feedback_parts(ctx, fb_parts, fb_parts_n, decode_pos, decode_step, fb_buf,
                                fb_buf + 1);
    } else if (!fb_logits.empty()) {
      const ih::Value& v = get(fb_logits);
      IH_REQUIRE(v.dtype == INFERC_DT_F32 && v.dev && !v.shape.empty() && v.shape.back() > 0,
                 INFERC_ERR_ARG, "decode feedback: '" + fb_logits + "' is not a float32 device output");
      const int64_t n = v.shape.back();
      int64_t* d = static_cast<int64_t*>(buf("__argmax__", sizeof(int64_t)));
      ih::argmax(ctx, n, static_cast<const float*>(v.dev) + (v.numel() - n), d, nullptr);
      ih::decode_feedback(ctx, decode_pos, decode_step, d, fb_buf, fb_buf + 1);
    } else {
      ih::advance_position(ctx, decode_pos, decode_step);
    }
  }
  if (events) IH_HIP(hipEventRecord(prof_ev[nodes.size()], ctx->stream));
  for (const auto& o : outputs) get(o);  // every graph output must exist
}

std::string inferc_executor::signature() const {
  std::ostringstream o;
  std::map<std::string, const Input*> sorted;
  for (const auto& kv : inputs) sorted[kv.first] = &kv.second;
  for (const auto& kv : sorted)
    o << kv.first << ":" << kv.second->v.dtype << ih::shape_str(kv.second->v.shape) << "@"
      << kv.second->v.dev << ";";
  return o.str();
}

// The key of a run's recording: the input signature and, in decode mode, the
// mode's mask input and the decode feedback's logits and ids names, which
// change what a step launches.
std::string inferc_executor::run_key() const {
  std::string k = signature();
  if (decode) k += "|decode:" + decode_mask + "|feedback:" + fb_logits + "," + fb_ids;
  return k;
}

// Host inputs are copied into their device buffers outside any graph.
void inferc_executor::stage_inputs() {
  for (auto& kv : inputs) {
    Input& in = kv.second;
    if (!in.from_host || !in.dirty) continue;  // (the graph reads inputs, never writes them)
    const size_t bytes = in.v.bytes();
    IH_HIP(hipMemcpyAsync(in.v.dev, in.staged.data(), bytes, hipMemcpyHostToDevice, ctx->stream));
    in.dirty = false;
  }
}

void inferc_executor::run() {
  if (dry) {
    walk();
    return;
  }
  ctx->make_current();
  if (decode)
    IH_REQUIRE(decode_len + std::max<int64_t>(decode_step, 1) <= kv_max_t, INFERC_ERR_SHAPE,
               "decode: the KV cache (" + std::to_string(kv_max_t) + " positions) is full");
  stage_inputs();
  const std::string key = run_key();
  if (graph_mode) {
    for (size_t i = 0; i < recorded.size(); ++i) {
      if (recorded[i].key != key) continue;
      const Recorded& r = recorded[i];
      if (r.ws_gen == ctx->ws_generation && r.route_gen == ctx->route_generation &&
          r.buf_gen == buf_gen) {
        IH_HIP(hipGraphLaunch(r.exec, ctx->stream));
        if (vals_key != key) {  // another key's pass ran since: its tape is not this one's
          vals = r.vals;
          cache_views = r.views;
          vals_key = key;
        }
        std::rotate(recorded.begin() + long(i), recorded.begin() + long(i) + 1, recorded.end());
        if (decode) decode_len += decode_step;
        return;
      }
      IH_HIP(hipStreamSynchronize(ctx->stream));  // stale: drop it
      destroy(recorded[i]);
      recorded.erase(recorded.begin() + long(i));
      break;
    }
  }
  // a changed GEMV route is planned by an eager pass, as a new signature is
  if (plan_route_gen != ctx->route_generation) last_key.clear();
  if (!graph_mode || key != last_key) {
    // first run for this key: eager, unrecorded (allocates the arena)
    walk();
    vals_key = key;
    last_key = key;
    plan_route_gen = ctx->route_generation;
    if (decode) decode_len += decode_step;
    return;
  }
  // second run with the same key: record it, then replay
  if (recorded.size() >= kMaxRecorded) {
    IH_HIP(hipStreamSynchronize(ctx->stream));
    destroy(recorded.front());
    recorded.erase(recorded.begin());
  }
  Recorded r;
  r.key = key;
  r.ws_gen = ctx->ws_generation;
  r.route_gen = ctx->route_generation;
  r.buf_gen = buf_gen;
  IH_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
  ctx->capturing = true;
  try {
    walk();
  } catch (...) {
    ctx->capturing = false;
    hipGraph_t g = nullptr;
    (void)hipStreamEndCapture(ctx->stream, &g);
    if (g) (void)hipGraphDestroy(g);
    throw;
  }
  ctx->capturing = false;
  IH_HIP(hipStreamEndCapture(ctx->stream, &r.graph));
  if (hipGraphInstantiate(&r.exec, r.graph, nullptr, nullptr, 0) != hipSuccess) {
    destroy(r);
    ih::fail(INFERC_ERR_HIP, "executor: graph instantiation failed");
  }
  vals_key = key;
  r.vals = vals;
  r.views = cache_views;
  recorded.push_back(std::move(r));
  IH_HIP(hipGraphLaunch(recorded.back().exec, ctx->stream));
  if (decode) decode_len += decode_step;
}

// Decode mode's plan: the values computed from the attention nodes' past
// inputs and from the attention-mask input carry the past length. They may
// reach the attention nodes only as their past or mask inputs, which decode
// mode replaces by the cache and the device length, and the indices of
// Gathers from an initializer (the position embeddings), which decode mode
// offsets by the device length; no graph output may depend on them.
void inferc_executor::plan_decode(const std::string& mask_input) {
  // the graph inputs the attention nodes' past inputs are computed from
  std::map<std::string, const inferc_graph::Node*> producer;
  for (const auto& n : nodes)
    for (const auto& o : n.out) producer[o] = &n;
  std::set<std::string> mark, seen;
  std::vector<std::string> todo;
  for (const auto& n : nodes)
    if (n.op == "FusedAttentionPast" && n.in.size() >= 5)
      for (size_t k = 3; k <= 4; ++k)
        if (!n.in[k].empty()) todo.push_back(n.in[k]);
  IH_REQUIRE(!todo.empty(), INFERC_ERR_UNSUPPORTED,
             "decode mode: the graph has no attention over a past");
  while (!todo.empty()) {
    const std::string v = todo.back();
    todo.pop_back();
    if (!seen.insert(v).second) continue;
    auto pr = producer.find(v);
    if (pr == producer.end()) {
      if (!inits.count(v)) mark.insert(v);  // a graph input
      continue;
    }
    for (const auto& i : pr->second->in)
      if (!i.empty()) todo.push_back(i);
  }
  if (!mask_input.empty()) mark.insert(mask_input);
  pos_gather_at.assign(nodes.size(), 0);
  for (const auto& n : nodes) {  // (in order: producers come first)
    if (n.op == "FusedAttentionPast") {
      for (size_t k = 0; k < 3 && k < n.in.size(); ++k)
        IH_REQUIRE(!mark.count(n.in[k]), INFERC_ERR_UNSUPPORTED,
                   "decode mode: attention input '" + n.in[k] + "' depends on the past length");
      continue;
    }
    bool any = false;
    for (const auto& i : n.in) any = any || mark.count(i) != 0;
    if (!any) continue;
    if (n.op == "Gather" && n.in.size() >= 2 && mark.count(n.in[1]) && !mark.count(n.in[0]) &&
        inits.count(n.in[0])) {
      pos_gather_at[node_index(n)] = 1;
      continue;
    }
    for (const auto& o : n.out) mark.insert(o);
  }
  for (const auto& o : outputs)
    IH_REQUIRE(!mark.count(o), INFERC_ERR_UNSUPPORTED,
               "decode mode: graph output '" + o + "' depends on the past length");
  // Nodes decode mode need not run: every output depends on the past or the
  // mask and is read only as an attention node's mask or by other such nodes
  // (readers come later in the order, so one backward pass decides).
  std::map<std::string, std::vector<std::pair<size_t, size_t>>> readers;  // (node, slot)
  for (size_t i = 0; i < nodes.size(); ++i)
    for (size_t k = 0; k < nodes[i].in.size(); ++k)
      if (!nodes[i].in[k].empty()) readers[nodes[i].in[k]].push_back({i, k});
  const std::set<std::string> outs(outputs.begin(), outputs.end());
  decode_skip_at.assign(nodes.size(), 0);
  for (size_t i = nodes.size(); i-- > 0;) {
    const inferc_graph::Node& n = nodes[i];
    if (n.op == "FusedAttentionPast" || pos_gather_at[i] || n.out.empty()) continue;
    bool dead = true;
    for (const auto& o : n.out) {
      if (o.empty()) continue;
      if (!mark.count(o) || outs.count(o)) {
        dead = false;
        break;
      }
      for (const auto& r : readers[o]) {
        const bool mask_slot = nodes[r.first].op == "FusedAttentionPast" && r.second == 5;
        if (!mask_slot && !decode_skip_at[r.first]) {
          dead = false;
          break;
        }
      }
      if (!dead) break;
    }
    decode_skip_at[i] = dead ? 1 : 0;
  }
  // Add(token rows, position rows): the Add of a row Gather from an
  // initializer table (the token embedding) and the position gather, each
  // read by the Add alone (through at most one same-type Cast; Shape nodes
  // read only the shape, which a pending value has), runs as one
  // kernel. Whether the token ids are on the device is decided at run time
  // (host-known ids leave the gathers as they are).
  embed_gather_at.assign(nodes.size(), 0);
  embed_add_at.assign(nodes.size(), 0);
  auto sole = [&](const std::string& v) {  // one reader of the data (Shape reads no data)
    auto it = readers.find(v);
    if (outs.count(v) || it == readers.end()) return false;
    size_t data_readers = 0;
    for (const auto& r : it->second) data_readers += nodes[r.first].op != "Shape";
    return data_readers == 1;
  };
  for (size_t i = 0; i < nodes.size(); ++i) {
    const inferc_graph::Node& n = nodes[i];
    if (n.op != "Add" || n.in.size() != 2 || n.out.size() != 1 || decode_skip_at[i]) continue;
    size_t g[2] = {0, 0};
    int n_pos = 0;
    bool ok = true;
    for (size_t k = 0; k < 2 && ok; ++k) {
      std::string v = n.in[k];
      auto pr = producer.find(v);
      ok = pr != producer.end() && sole(v);
      if (ok && pr->second->op == "Cast" && !pr->second->in.empty()) {
        v = pr->second->in[0];
        pr = producer.find(v);
        ok = pr != producer.end() && sole(v);
      }
      if (!ok) break;
      g[k] = node_index(*pr->second);
      const inferc_graph::Node& gn = nodes[g[k]];
      auto t = inits.find(gn.in.empty() ? std::string() : gn.in[0]);
      ok = gn.op == "Gather" && gn.in.size() == 2 && gn.out.size() == 1 && t != inits.end() &&
           t->second.shape.size() == 2 && ih::attr_int(gn, "axis", 0) == 0 &&
           !gn.attrs.count("__ln_g");
      if (ok && pos_gather_at[g[k]]) ++n_pos;
    }
    if (!ok || n_pos != 1) continue;
    embed_add_at[i] = 1;
    embed_gather_at[g[0]] = embed_gather_at[g[1]] = 1;
  }
}

// Waits for the stream, then fails if a device-index gather of the passes
// enqueued so far met an out-of-range index; the flag is cleared first, so
// the next pass starts clean.
// A row gather left pending for a LayerNorm that turned out to read it as
// its residual: written out after all.
void inferc_executor::materialize_gather(const std::string& name) {
  const PendingGather g = pending_gather.at(name);
  pending_gather.erase(name);
  const std::vector<int64_t> shape = get(name).shape;
  float* y = static_cast<float*>(make_dev(name, INFERC_DT_F32, shape).dev);
  if (!dry) {
    ih::gather_axis(ctx, 1, g.vocab, g.feat, g.table, g.ids, g.n, y, gather_err);
    dev_gather = true;
  }
}

// Rows left pending for an embedding Add that cannot take them as one kernel
// after all: written out on their own.
void inferc_executor::materialize_embed(const std::string& name) {
  auto it = pending_embed.find(name);
  if (it == pending_embed.end()) return;
  const PendingEmbed e = it->second;
  pending_embed.erase(it);
  const std::vector<int64_t> shape = get(name).shape;
  float* y = static_cast<float*>(make_dev(name, INFERC_DT_F32, shape).dev);
  if (dry) return;
  if (e.ids) {
    ih::gather_axis(ctx, 1, e.rows, e.feat, e.table, e.ids, e.n, y, gather_err);
    dev_gather = true;
  } else {
    ih::gather_rows_at(ctx, e.rows, e.feat, e.table, decode_pos, e.n, y);
  }
}

void inferc_executor::check_gather_err() {
  if (dry || !dev_gather || !gather_err) return;
  int32_t flag = 0;
  IH_HIP(hipStreamSynchronize(ctx->stream));
  IH_HIP(hipMemcpy(&flag, gather_err, sizeof(flag), hipMemcpyDeviceToHost));
  if (flag == 0) return;
  IH_HIP(hipMemset(gather_err, 0, sizeof(int32_t)));
  ih::fail(INFERC_ERR_ARG, "Gather: index out of range");
}

// One eager pass recorded as a profiler iteration (executor.cc:121-125,
// 145-160, 349-354): each node's time is the device time between HIP events
// recorded on the stream before and after it (host-only shape nodes read
// about 0 ms); the iteration total is the host wall clock from the first
// node's enqueue until the stream has drained, so it includes launch and
// host work. A dry executor records 0 ms per node. The recordings stay
// valid: the pass reuses their buffers (a buffer it has to grow makes those
// naming it stale).
void inferc_executor::run_profiled(inferc_profiler* p) {
  std::vector<int64_t> act;
  act.reserve(nodes.size());
  if (dry) {
    p->begin_iteration();
    walk(&act, p->track_activation_bytes);
    for (size_t i = 0; i < nodes.size(); ++i) p->add_op(nodes[i].op, nodes[i].name, 0.0, act[i]);
    p->end_iteration();
    return;
  }
  ctx->make_current();
  IH_REQUIRE(!ctx->capturing, INFERC_ERR_STATE, "executor: profiled run during graph capture");
  while (prof_ev.size() < nodes.size() + 1) {
    hipEvent_t e;
    IH_HIP(hipEventCreate(&e));
    prof_ev.push_back(e);
  }
  stage_inputs();
  const std::string key = run_key();
  if (key != last_key) {
    // a new key: one unrecorded eager pass first, so that the arena
    // allocations and the one-row products' transposed weight copies
    // (blocking allocations and uploads) fall outside the timed pass
    walk();
    last_key = key;
    if (decode) {
      // that pass advanced the device position: rewind it; the recorded pass
      // then writes the same cache rows again
      IH_HIP(hipStreamSynchronize(ctx->stream));
      IH_HIP(hipMemcpy(decode_pos, &decode_len, sizeof(int64_t), hipMemcpyHostToDevice));
    }
  }
  IH_HIP(hipStreamSynchronize(ctx->stream));
  p->begin_iteration();
  walk(&act, p->track_activation_bytes);
  vals_key = key;
  if (decode) decode_len += decode_step;
  IH_HIP(hipEventSynchronize(prof_ev[nodes.size()]));
  check_gather_err();
  for (size_t i = 0; i < nodes.size(); ++i) {
    float ms = 0.0f;
    IH_HIP(hipEventElapsedTime(&ms, prof_ev[i], prof_ev[i + 1]));
    p->add_op(nodes[i].op, nodes[i].name, double(ms), act[i]);
  }
  p->end_iteration();
}

namespace {

inferc_graph* check_graph(inferc_graph* g) {
  IH_REQUIRE(g != nullptr, INFERC_ERR_ARG, "null graph");
  return g;
}

inferc_executor* check_ex(inferc_executor* ex) {
  IH_REQUIRE(ex != nullptr && (ex->dry || ex->ctx != nullptr), INFERC_ERR_ARG, "null executor");
  if (!ex->dry) ex->ctx->make_current();
  return ex;
}

std::vector<int64_t> read_shape(int rank, const int64_t* shape) {
  IH_REQUIRE(rank >= 0 && rank <= 8, INFERC_ERR_SHAPE, "rank must be in [0, 8]");
  IH_REQUIRE(rank == 0 || shape != nullptr, INFERC_ERR_ARG, "null shape");
  std::vector<int64_t> s(shape, shape + rank);
  for (int64_t d : s) IH_REQUIRE(d >= 0, INFERC_ERR_SHAPE, "negative dimension");
  return s;
}

}  // namespace

extern "C" {

int inferc_graph_create(inferc_graph** out) {
  return ih::guard([&] {
    IH_REQUIRE(out != nullptr, INFERC_ERR_ARG, "null output pointer");
    *out = new inferc_graph();
  });
}

int inferc_graph_destroy(inferc_graph* g) {
  return ih::guard([&] { delete g; });
}

int inferc_graph_add_initializer(inferc_graph* g, const char* name, int dtype, int rank,
                                 const int64_t* shape, const void* host_data) {
  return ih::guard([&] {
    check_graph(g);
    IH_REQUIRE(name != nullptr && *name, INFERC_ERR_ARG, "initializer needs a name");
    inferc_graph::Init in;
    in.name = name;
    in.dtype = dtype;
    in.shape = read_shape(rank, shape);
    const size_t bytes = size_t(ih::numel_of(in.shape)) * ih::dtype_size(dtype);
    IH_REQUIRE(bytes == 0 || host_data != nullptr, INFERC_ERR_ARG, "null initializer data");
    in.data.assign(static_cast<const uint8_t*>(host_data),
                   static_cast<const uint8_t*>(host_data) + bytes);
    g->inits.push_back(std::move(in));
  });
}

int inferc_graph_add_node(inferc_graph* g, const char* op_type, const char* name, int n_inputs,
                          const char* const* inputs, int n_outputs, const char* const* outputs,
                          const char* attrs) {
  return ih::guard([&] {
    check_graph(g);
    IH_REQUIRE(op_type != nullptr && n_inputs >= 0 && n_outputs >= 0, INFERC_ERR_ARG,
               "bad node arguments");
    inferc_graph::Node n;
    n.op = op_type;
    n.name = name ? name : "";
    for (int i = 0; i < n_inputs; ++i) n.in.push_back(inputs[i] ? inputs[i] : "");
    for (int i = 0; i < n_outputs; ++i) n.out.push_back(outputs[i] ? outputs[i] : "");
    if (attrs) {
      std::stringstream ss(attrs);
      std::string kv;
      while (std::getline(ss, kv, ';')) {
        if (kv.empty()) continue;
        const size_t eq = kv.find('=');
        IH_REQUIRE(eq != std::string::npos, INFERC_ERR_ARG, "attribute without '=': " + kv);
        n.attrs[kv.substr(0, eq)] = kv.substr(eq + 1);
      }
    }
    g->nodes.push_back(std::move(n));
  });
}

int inferc_graph_add_output(inferc_graph* g, const char* name) {
  return ih::guard([&] {
    check_graph(g);
    IH_REQUIRE(name != nullptr, INFERC_ERR_ARG, "null output name");
    g->outputs.push_back(name);
  });
}

int inferc_graph_add_input(inferc_graph* g, const char* name, int dtype, int rank,
                           const int64_t* shape) {
  return ih::guard([&] {
    check_graph(g);
    IH_REQUIRE(name != nullptr && *name, INFERC_ERR_ARG, "input needs a name");
    IH_REQUIRE(rank >= 0 && rank <= 8 && (rank == 0 || shape != nullptr), INFERC_ERR_SHAPE,
               "rank must be in [0, 8]");
    inferc_graph::IO io;
    io.name = name;
    io.dtype = dtype;
    io.shape.assign(shape, shape + rank);  // -1 marks a symbolic dim
    g->inputs.push_back(io);
  });
}

int inferc_graph_add_tensor_attr(inferc_graph* g, const char* attr, int dtype, int rank,
                                 const int64_t* shape, const void* host_data) {
  return ih::guard([&] {
    check_graph(g);
    IH_REQUIRE(!g->nodes.empty(), INFERC_ERR_STATE, "no node to attach the attribute to");
    IH_REQUIRE(attr != nullptr && *attr, INFERC_ERR_ARG, "attribute needs a name");
    inferc_graph::Init t;
    t.name = attr;
    t.dtype = dtype;
    t.shape = read_shape(rank, shape);
    const size_t bytes = size_t(ih::numel_of(t.shape)) * ih::dtype_size(dtype);
    IH_REQUIRE(bytes == 0 || host_data != nullptr, INFERC_ERR_ARG, "null attribute data");
    t.data.assign(static_cast<const uint8_t*>(host_data),
                  static_cast<const uint8_t*>(host_data) + bytes);
    g->nodes.back().tattrs[attr] = std::move(t);
  });
}

int inferc_graph_to_json(const inferc_graph* g, char* buf, size_t capacity, size_t* len) {
  return ih::guard([&] {
    IH_REQUIRE(g != nullptr && len != nullptr, INFERC_ERR_ARG, "null argument");
    auto q = [](const std::string& s) {
      std::string o = "\"";
      for (unsigned char c : s) {
        if (c == '"' || c == '\\') {
          o += '\\';
          o += char(c);
        } else if (c < 0x20) {
          char u[8];
          std::snprintf(u, sizeof u, "\\u%04x", c);
          o += u;
        } else {
          o += char(c);
        }
      }
      return o + "\"";
    };
    auto shape = [](const std::vector<int64_t>& s) {
      std::string o = "[";
      for (size_t i = 0; i < s.size(); ++i) o += (i ? ", " : "") + std::to_string(s[i]);
      return o + "]";
    };
    auto names = [&](const std::vector<std::string>& v) {
      std::string o = "[";
      for (size_t i = 0; i < v.size(); ++i) o += (i ? ", " : "") + q(v[i]);
      return o + "]";
    };
    std::string o = "{\"name\": " + q(g->name) + ", \"inputs\": [";
    for (size_t i = 0; i < g->inputs.size(); ++i)
      o += std::string(i ? ", " : "") + "{\"name\": " + q(g->inputs[i].name) +
           ", \"dtype\": " + std::to_string(g->inputs[i].dtype) +
           ", \"shape\": " + shape(g->inputs[i].shape) + "}";
    o += "], \"outputs\": " + names(g->outputs) + ", \"initializers\": [";
    for (size_t i = 0; i < g->inits.size(); ++i)
      o += std::string(i ? ", " : "") + "{\"name\": " + q(g->inits[i].name) +
           ", \"dtype\": " + std::to_string(g->inits[i].dtype) +
           ", \"shape\": " + shape(g->inits[i].shape) +
           ", \"bytes\": " + std::to_string(g->inits[i].data.size()) + "}";
    o += "], \"nodes\": [";
    for (size_t i = 0; i < g->nodes.size(); ++i) {
      const inferc_graph::Node& n = g->nodes[i];
      o += std::string(i ? ", " : "") + "{\"op\": " + q(n.op) + ", \"name\": " + q(n.name) +
           ", \"domain\": " + q(n.domain) + ", \"inputs\": " + names(n.in) +
           ", \"outputs\": " + names(n.out) + ", \"attrs\": {";
      size_t k = 0;
      for (const auto& kv : n.attrs) o += std::string(k++ ? ", " : "") + q(kv.first) + ": " + q(kv.second);
      o += "}, \"tensor_attrs\": {";
      k = 0;
      for (const auto& kv : n.tattrs)
        o += std::string(k++ ? ", " : "") + q(kv.first) + ": {\"dtype\": " +
             std::to_string(kv.second.dtype) + ", \"shape\": " + shape(kv.second.shape) + "}";
      o += "}}";
    }
    o += "]}";
    *len = o.size();
    if (buf == nullptr) return;
    IH_REQUIRE(capacity > o.size(), INFERC_ERR_ARG,
               "buffer too small: need " + std::to_string(o.size() + 1) + " bytes");
    std::memcpy(buf, o.c_str(), o.size() + 1);
  });
}

int inferc_graph_get_initializer(const inferc_graph* g, const char* name, int* dtype, int* rank,
                                 int64_t* shape, void* host_dst, size_t capacity_bytes) {
  return ih::guard([&] {
    IH_REQUIRE(g != nullptr && name != nullptr && dtype && rank && shape, INFERC_ERR_ARG,
               "null argument");
    for (const auto& t : g->inits) {
      if (t.name != name) continue;
      IH_REQUIRE(t.shape.size() <= 8, INFERC_ERR_SHAPE, "initializer rank > 8");
      *dtype = t.dtype;
      *rank = int(t.shape.size());
      for (size_t i = 0; i < t.shape.size(); ++i) shape[i] = t.shape[i];
      if (host_dst) {
        IH_REQUIRE(capacity_bytes >= t.data.size(), INFERC_ERR_ARG, "buffer too small");
        if (!t.data.empty()) std::memcpy(host_dst, t.data.data(), t.data.size());
      }
      return;
    }
    ih::fail(INFERC_ERR_ARG, std::string("no initializer '") + name + "'");
  });
}

int inferc_executor_create(inferc_hip_ctx* ctx, const inferc_graph* g, inferc_executor** out) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    IH_REQUIRE(g != nullptr && out != nullptr, INFERC_ERR_ARG, "null argument");
    *out = nullptr;
    auto ex = std::make_unique<inferc_executor>();
    ex->ctx = ctx;
    ex->nodes = g->nodes;
    ex->outputs = g->outputs;
    for (const auto& in : g->inits) {
      ih::Value v;
      v.dtype = in.dtype;
      v.shape = in.shape;
      v.host = std::make_shared<std::vector<uint8_t>>(in.data);
      if (!in.data.empty()) {
        IH_HIP(hipMalloc(&v.dev, in.data.size()));
        ex->init_allocs.push_back(v.dev);
        IH_HIP(hipMemcpy(v.dev, in.data.data(), in.data.size(), hipMemcpyHostToDevice));
      }
      ex->inits[in.name] = v;
    }
    IH_HIP(hipMalloc(&ex->gather_err, sizeof(int32_t)));
    IH_HIP(hipMemset(ex->gather_err, 0, sizeof(int32_t)));
    ex->peephole();
    ex->fold_ln_weights();
    *out = ex.release();
  });
}

int inferc_executor_create_dry(const inferc_graph* g, inferc_executor** out) {
  return ih::guard([&] {
    IH_REQUIRE(g != nullptr && out != nullptr, INFERC_ERR_ARG, "null argument");
    *out = nullptr;
    auto ex = std::make_unique<inferc_executor>();
    ex->dry = true;
    ex->graph_mode = false;
    ex->nodes = g->nodes;
    ex->outputs = g->outputs;
    for (const auto& in : g->inits) {
      ih::Value v;
      v.dtype = in.dtype;
      v.shape = in.shape;
      v.host = std::make_shared<std::vector<uint8_t>>(in.data);
      v.dev = ex->fake_ptr(in.data.size());
      ex->inits[in.name] = v;
    }
    ex->peephole();
    *out = ex.release();
  });
}

int inferc_executor_node_count(inferc_executor* ex, int* count) {
  return ih::guard([&] {
    IH_REQUIRE(ex != nullptr && count != nullptr, INFERC_ERR_ARG, "null argument");
    *count = int(ex->nodes.size());
  });
}

int inferc_executor_destroy(inferc_executor* ex) {
  return ih::guard([&] {
    if (!ex) return;
    if (ex->ctx && !ex->dry) {
      ex->ctx->make_current();
      (void)hipStreamSynchronize(ex->ctx->stream);
    }
    delete ex;
  });
}

int inferc_executor_set_input(inferc_executor* ex, const char* name, int dtype, int rank,
                              const int64_t* shape, const void* host_data) {
  return ih::guard([&] {
    check_ex(ex);
    IH_REQUIRE(name != nullptr, INFERC_ERR_ARG, "null input name");
    inferc_executor::Input& in = ex->inputs[name];
    std::vector<int64_t> s = read_shape(rank, shape);
    const size_t bytes = size_t(ih::numel_of(s)) * ih::dtype_size(dtype);
    IH_REQUIRE(bytes == 0 || host_data != nullptr, INFERC_ERR_ARG, "null input data");
    if (ex->dry) {
      in.v.dev = ex->fake_ptr(bytes);
    } else if (!in.from_host || bytes > in.cap) {
      // an input that grows (the with-past decode's attention mask, one
      // position per step) grows its buffer by half again at least
      size_t want = bytes > 0 ? bytes : 8;
      if (in.from_host && in.v.dev) {
        IH_HIP(hipStreamSynchronize(ex->ctx->stream));
        IH_HIP(hipFree(in.v.dev));
        const size_t grown = in.cap + in.cap / 2;
        want = ((grown > want ? grown : want) + 255) & ~size_t(255);
      }
      in.v.dev = nullptr;
      IH_HIP(hipMalloc(&in.v.dev, want));
      in.cap = want;
    }
    in.from_host = true;
    in.v.dtype = dtype;
    in.v.shape = s;
    in.v.host.reset();
    in.staged.assign(static_cast<const uint8_t*>(host_data),
                     static_cast<const uint8_t*>(host_data) + bytes);
    in.dirty = true;
  });
}

int inferc_executor_set_input_device(inferc_executor* ex, const char* name, int dtype, int rank,
                                     const int64_t* shape, const void* dev_data) {
  return ih::guard([&] {
    check_ex(ex);
    IH_REQUIRE(name != nullptr, INFERC_ERR_ARG, "null input name");
    inferc_executor::Input& in = ex->inputs[name];
    if (in.from_host && in.v.dev && !ex->dry) {
      IH_HIP(hipStreamSynchronize(ex->ctx->stream));
      IH_HIP(hipFree(in.v.dev));
    }
    in.from_host = false;
    in.staged.clear();
    in.v.dtype = dtype;
    in.v.shape = read_shape(rank, shape);
    (void)ih::dtype_size(dtype);
    IH_REQUIRE(in.v.numel() == 0 || dev_data != nullptr, INFERC_ERR_ARG, "null device input");
    in.v.dev = const_cast<void*>(dev_data);
    in.v.host.reset();
  });
}

int inferc_executor_run(inferc_executor* ex) {
  return ih::guard([&] { check_ex(ex)->run(); });
}

int inferc_executor_run_profiled(inferc_executor* ex, inferc_profiler* p) {
  return ih::guard([&] {
    IH_REQUIRE(p != nullptr, INFERC_ERR_ARG, "null profiler");
    check_ex(ex)->run_profiled(p);
  });
}

int inferc_executor_output_info(inferc_executor* ex, const char* name, int* dtype, int* rank,
                                int64_t* shape) {
  return ih::guard([&] {
    check_ex(ex);
    IH_REQUIRE(name && dtype && rank && shape, INFERC_ERR_ARG, "null argument");
    const ih::Value& v = ex->get(name);
    IH_REQUIRE(v.shape.size() <= 8, INFERC_ERR_SHAPE, "output rank > 8");
    *dtype = v.dtype;
    *rank = int(v.shape.size());
    for (size_t i = 0; i < v.shape.size(); ++i) shape[i] = v.shape[i];
    // a present view in decode mode holds the positions of the last run
    if (ex->decode && ex->cache_views.count(name) && v.shape.size() == 4)
      shape[2] = ex->decode_len;
  });
}

int inferc_executor_get_output(inferc_executor* ex, const char* name, void* host_dst,
                               size_t capacity_bytes) {
  return ih::guard([&] {
    check_ex(ex);
    IH_REQUIRE(name && host_dst, INFERC_ERR_ARG, "null argument");
    const ih::Value& v = ex->get(name);
    IH_REQUIRE(!ex->dry || v.host, INFERC_ERR_STATE,
               "a dry-run executor has no output data (only host-known values)");
    IH_REQUIRE(capacity_bytes >= v.bytes(), INFERC_ERR_ARG, "output buffer too small");
    if (ex->dry) {
      std::memcpy(host_dst, v.host->data(), v.bytes());
      return;
    }
    IH_HIP(hipStreamSynchronize(ex->ctx->stream));
    ex->check_gather_err();
    auto cv = ex->cache_views.find(name);
    if (!v.dev && !v.host && cv != ex->cache_views.end()) {
      const auto& w = cv->second;
      const int64_t T = ex->decode ? ex->decode_len : w.T;
      IH_REQUIRE(capacity_bytes >= size_t(w.rows * T * w.dh) * sizeof(float), INFERC_ERR_ARG,
                 "output buffer too small");
      const size_t row = size_t(T * w.dh) * sizeof(float);
      IH_HIP(hipMemcpy2D(host_dst, row, w.base, size_t(w.max_t * w.dh) * sizeof(float), row,
                         size_t(w.rows), hipMemcpyDeviceToHost));
      return;
    }
    IH_REQUIRE(v.dev || v.host, INFERC_ERR_STATE, std::string("tensor '") + name + "' has no data");
    if (v.dev) {
      IH_HIP(hipMemcpy(host_dst, v.dev, v.bytes(), hipMemcpyDeviceToHost));
    } else if (v.host) {
      std::memcpy(host_dst, v.host->data(), v.bytes());
    }
  });
}

int inferc_executor_set_graph_mode(inferc_executor* ex, int enabled) {
  return ih::guard([&] {
    check_ex(ex);
    ex->graph_mode = enabled != 0;
    if (!ex->graph_mode && !ex->dry) {
      IH_HIP(hipStreamSynchronize(ex->ctx->stream));
      ex->drop_graph();
    }
  });
}

int inferc_executor_bind_kv_cache(inferc_executor* ex, int64_t max_t) {
  return ih::guard([&] {
    check_ex(ex);
    IH_REQUIRE(max_t >= 0, INFERC_ERR_ARG, "max_t must be >= 0");
    IH_REQUIRE(!ex->dry, INFERC_ERR_STATE, "a dry-run executor has no KV cache");
    IH_HIP(hipStreamSynchronize(ex->ctx->stream));
    ex->drop_graph();
    ex->free_kv();
    ex->kv_max_t = max_t;
    ex->last_key.clear();
    ex->decode = false;
  });
}

int inferc_executor_set_decode_position(inferc_executor* ex, int64_t len,
                                        const char* mask_input) {
  return ih::guard([&] {
    check_ex(ex);
    if (ex->dry) {
      // planning only (no cache, no device): the plan's checks
      ex->decode = len >= 0;
      ex->decode_len = len;
      ex->decode_mask = ex->decode && mask_input ? mask_input : "";
      if (ex->decode) ex->plan_decode(mask_input ? mask_input : "");
      return;
    }
    IH_HIP(hipStreamSynchronize(ex->ctx->stream));
    ex->last_key.clear();  // (recordings stay: the mode is part of their key)
    if (len < 0) {
      if (ex->decode)
        for (auto& kv : ex->kv) kv.second.len = ex->decode_len;
      ex->decode = false;
      ex->decode_mask.clear();
      ex->fb_logits.clear();  // (the fed-back input stays bound, holding the last token)
      return;
    }
    IH_REQUIRE(ex->kv_max_t > 0, INFERC_ERR_STATE, "decode mode needs a bound KV cache");
    IH_REQUIRE(len <= ex->kv_max_t, INFERC_ERR_SHAPE, "decode: position past the KV cache");
    for (const auto& kv : ex->kv)
      IH_REQUIRE(kv.second.len >= len, INFERC_ERR_STATE,
                 "decode: the KV cache holds fewer positions than the decode position");
    ex->plan_decode(mask_input ? mask_input : "");
    if (!ex->decode_pos) IH_HIP(hipMalloc(&ex->decode_pos, sizeof(int64_t)));
    IH_HIP(hipMemcpy(ex->decode_pos, &len, sizeof(int64_t), hipMemcpyHostToDevice));
    ex->decode = true;
    ex->decode_len = len;
    ex->decode_mask = mask_input ? mask_input : "";
  });
}

int inferc_executor_decode_position(inferc_executor* ex, int64_t* len) {
  return ih::guard([&] {
    check_ex(ex);
    IH_REQUIRE(len != nullptr, INFERC_ERR_ARG, "null argument");
    *len = ex->decode ? ex->decode_len : -1;
  });
}

int inferc_executor_set_decode_feedback(inferc_executor* ex, const char* logits,
                                        const char* ids, int64_t first_token) {
  return ih::guard([&] {
    check_ex(ex);
    IH_REQUIRE(!ex->dry, INFERC_ERR_STATE, "decode feedback needs a device");
    IH_HIP(hipStreamSynchronize(ex->ctx->stream));
    ex->last_key.clear();  // (recordings stay: the feedback is part of their key)
    if (logits == nullptr) {
      ex->fb_logits.clear();
      ex->fb_ids.clear();
      return;
    }
    IH_REQUIRE(ids != nullptr, INFERC_ERR_ARG, "null input name");
    IH_REQUIRE(ex->decode, INFERC_ERR_STATE, "decode feedback needs decode mode");
    IH_REQUIRE(first_token >= 0, INFERC_ERR_ARG, "decode feedback: negative token");
    if (!ex->fb_buf) {
      IH_HIP(hipMalloc(&ex->fb_buf, sizeof(int64_t) * size_t(ex->kv_max_t + 2)));
      IH_HIP(hipMemset(ex->fb_buf, 0, sizeof(int64_t) * size_t(ex->kv_max_t + 2)));
    }
    IH_HIP(hipMemcpy(ex->fb_buf, &first_token, sizeof(int64_t), hipMemcpyHostToDevice));
    IH_HIP(hipMemcpy(ex->fb_buf + 1 + ex->decode_len, &first_token, sizeof(int64_t),
                     hipMemcpyHostToDevice));
    inferc_executor::Input& in = ex->inputs[ids];
    if (in.from_host && in.v.dev) IH_HIP(hipFree(in.v.dev));
    in = inferc_executor::Input{};
    in.v.dtype = INFERC_DT_I64;
    in.v.shape = {1, 1};
    in.v.dev = ex->fb_buf;
    ex->fb_logits = logits;
    ex->fb_ids = ids;
  });
}

int inferc_executor_run_steps(inferc_executor* ex, int64_t steps, float* step_ms) {
  return ih::guard([&] {
    check_ex(ex);
    IH_REQUIRE(steps >= 0, INFERC_ERR_ARG, "run_steps: negative count");
    if (ex->dry || step_ms == nullptr) {
      for (int64_t i = 0; i < steps; ++i) ex->run();
      return;
    }
    ex->ctx->make_current();
    while (int64_t(ex->step_ev.size()) < steps + 1) {
      hipEvent_t e;
      IH_HIP(hipEventCreate(&e));
      ex->step_ev.push_back(e);
    }
    IH_HIP(hipEventRecord(ex->step_ev[0], ex->ctx->stream));
    for (int64_t i = 0; i < steps; ++i) {
      ex->run();
      IH_HIP(hipEventRecord(ex->step_ev[size_t(i + 1)], ex->ctx->stream));
    }
    IH_HIP(hipEventSynchronize(ex->step_ev[size_t(steps)]));
    for (int64_t i = 0; i < steps; ++i)
      IH_HIP(hipEventElapsedTime(&step_ms[i], ex->step_ev[size_t(i)], ex->step_ev[size_t(i + 1)]));
  });
}

int inferc_executor_decode_tokens(inferc_executor* ex, int64_t first_pos, int64_t n,
                                  int64_t* tokens) {
  return ih::guard([&] {
    check_ex(ex);
    IH_REQUIRE(tokens != nullptr || n == 0, INFERC_ERR_ARG, "null argument");
    IH_REQUIRE(ex->fb_buf != nullptr, INFERC_ERR_STATE, "no decode feedback has run");
    IH_REQUIRE(first_pos >= 0 && n >= 0 && first_pos + n <= ex->kv_max_t + 1, INFERC_ERR_SHAPE,
               "decode tokens: positions past the KV cache");
    IH_HIP(hipStreamSynchronize(ex->ctx->stream));
    if (n) IH_HIP(hipMemcpy(tokens, ex->fb_buf + 1 + first_pos, sizeof(int64_t) * size_t(n),
                            hipMemcpyDeviceToHost));
    ex->check_gather_err();
  });
}

int inferc_executor_set_input_shape(inferc_executor* ex, const char* name, int dtype, int rank,
                                    const int64_t* shape) {
  return ih::guard([&] {
    check_ex(ex);
    IH_REQUIRE(name != nullptr, INFERC_ERR_ARG, "null input name");
    inferc_executor::Input& in = ex->inputs[name];
    if (in.from_host && in.v.dev && !ex->dry) {
      IH_HIP(hipStreamSynchronize(ex->ctx->stream));
      IH_HIP(hipFree(in.v.dev));
    }
    in.from_host = false;
    in.staged.clear();
    in.v.dtype = dtype;
    (void)ih::dtype_size(dtype);
    in.v.shape = read_shape(rank, shape);
    in.v.dev = nullptr;
    in.v.host.reset();
  });
}

int inferc_executor_output_device(inferc_executor* ex, const char* name, const void** ptr) {
  return ih::guard([&] {
    check_ex(ex);
    IH_REQUIRE(name != nullptr && ptr != nullptr, INFERC_ERR_ARG, "null argument");
    const ih::Value& v = ex->get(name);
    IH_REQUIRE(v.dev != nullptr, INFERC_ERR_STATE,
               std::string("output '") + name + "' has no contiguous device buffer");
    ex->check_gather_err();
    *ptr = v.dev;
  });
}

int inferc_executor_device_bytes(inferc_executor* ex, int64_t* initializers,
                                 int64_t* transposed_copies, int64_t* arena) {
  return ih::guard([&] {
    IH_REQUIRE(ex != nullptr, INFERC_ERR_ARG, "null executor");
    int64_t w = 0, a = 0;
    for (const auto& kv : ex->inits)
      if (kv.second.dev) w += int64_t(kv.second.bytes());
    if (!ex->dry)
      for (const auto& kv : ex->arena) a += int64_t(kv.second.bytes);
    if (initializers) *initializers = w;
    if (transposed_copies) *transposed_copies = int64_t(ex->wt_cache_bytes);
    if (arena) *arena = a;
  });
}

int inferc_executor_output_argmax(inferc_executor* ex, const char* name, int64_t* index) {
  return ih::guard([&] {
    check_ex(ex);
    IH_REQUIRE(name != nullptr && index != nullptr, INFERC_ERR_ARG, "null argument");
    IH_REQUIRE(!ex->dry, INFERC_ERR_STATE, "a dry-run executor has no output data");
    const ih::Value& v = ex->get(name);
    IH_REQUIRE(v.dtype == INFERC_DT_F32 && v.dev && !v.shape.empty() && v.shape.back() > 0,
               INFERC_ERR_ARG, "argmax: needs a float32 device output");
    const int64_t n = v.shape.back();
    const float* last = static_cast<const float*>(v.dev) + (v.numel() - n);
    int64_t* d = static_cast<int64_t*>(ex->buf("__argmax__", sizeof(int64_t)));
    ih::argmax(ex->ctx, n, last, d, nullptr);
    IH_HIP(hipMemcpyAsync(index, d, sizeof(int64_t), hipMemcpyDeviceToHost, ex->ctx->stream));
    IH_HIP(hipStreamSynchronize(ex->ctx->stream));
    ex->check_gather_err();
  });
}

}  // extern "C"
