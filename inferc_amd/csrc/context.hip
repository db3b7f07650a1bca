// Context, memory and error entry points of the C-ABI.
#include <cstring>
#include <string>

#include "common.h"

namespace ih {

namespace {
thread_local std::string g_last_error;
}

void set_last_error(const std::string& msg) { g_last_error = msg; }

inferc_hip_ctx* check_ctx(inferc_hip_ctx* ctx) {
  IH_REQUIRE(ctx != nullptr, INFERC_ERR_ARG, "null context");
  return ctx;
}

}  // namespace ih

void inferc_hip_ctx::make_current() const { IH_HIP(hipSetDevice(device)); }

void* inferc_hip_ctx::ws(size_t bytes) {
  if (bytes <= workspace_bytes) return workspace;
  IH_REQUIRE(!capturing, INFERC_ERR_STATE,
             "workspace must be reserved before HIP graph capture");
  if (workspace) {
    IH_HIP(hipStreamSynchronize(stream));
    IH_HIP(hipFree(workspace));
    workspace = nullptr;
    workspace_bytes = 0;
  }
  size_t want = bytes < (size_t(4) << 20) ? (size_t(4) << 20) : bytes;
  IH_HIP(hipMalloc(&workspace, want));
  workspace_bytes = want;
  ++ws_generation;
  return workspace;
}

void inferc_hip_ctx::free_tables() {
  if (tables.empty()) return;
  IH_HIP(hipStreamSynchronize(stream));
  for (Table& t : tables) (void)hipFree(t.dev);
  tables.clear();
  ++ws_generation;
}

void inferc_hip_ctx::reserve_tables(size_t n) {
  IH_REQUIRE(n <= kMaxTables, INFERC_ERR_SHAPE, "launch needs too many descriptor tables");
  if (tables.size() + n <= kMaxTables || capturing) return;
  free_tables();
}

const void* inferc_hip_ctx::table(const void* bytes, size_t len) {
  for (const Table& t : tables)
    if (t.key.size() == len && std::memcmp(t.key.data(), bytes, len) == 0) return t.dev;
  IH_REQUIRE(!capturing, INFERC_ERR_STATE,
             "descriptor table must be uploaded before graph capture");
  IH_REQUIRE(tables.size() < kMaxTables, INFERC_ERR_STATE,
             "descriptor table cache full (reserve_tables was not called)");
  Table t;
  t.key.assign(static_cast<const char*>(bytes), len);
  IH_HIP(hipMalloc(&t.dev, len));
  try {
    IH_HIP(hipMemcpy(t.dev, bytes, len, hipMemcpyHostToDevice));
  } catch (...) {
    (void)hipFree(t.dev);
    throw;
  }
  tables.push_back(std::move(t));
  return tables.back().dev;
}

extern "C" {

const char* inferc_hip_last_error(void) { return ih::g_last_error.c_str(); }

int inferc_hip_abi_version(void) { return INFERC_HIP_ABI_VERSION; }

int inferc_hip_device_count(int* count) {
  return ih::guard([&] {
    IH_REQUIRE(count != nullptr, INFERC_ERR_ARG, "null count");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    *count = (e == hipSuccess) ? n : 0;
  });
}

int inferc_hip_create(int device, inferc_hip_ctx** out) {
  return ih::guard([&] {
    IH_REQUIRE(out != nullptr, INFERC_ERR_ARG, "null output pointer");
    *out = nullptr;
    int n = 0;
    IH_HIP(hipGetDeviceCount(&n));
    IH_REQUIRE(device >= 0 && device < n, INFERC_ERR_ARG,
               "device index " + std::to_string(device) + " out of range (" +
                   std::to_string(n) + " devices)");
    auto* c = new inferc_hip_ctx();
    c->device = device;
    try {
      IH_HIP(hipSetDevice(device));
      hipDeviceProp_t prop;
      IH_HIP(hipGetDeviceProperties(&prop, device));
      c->num_cus = prop.multiProcessorCount;
      // Default-priority, non-blocking stream: the context's only queue.
      IH_HIP(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
      IH_HIP(hipEventCreate(&c->ev_start));
      IH_HIP(hipEventCreate(&c->ev_stop));
      c->ws(size_t(16) << 20);
      IH_HIP(hipMalloc(&c->ks_count, sizeof(unsigned) * inferc_hip_ctx::kKsCounters));
      IH_HIP(hipMemset(c->ks_count, 0, sizeof(unsigned) * inferc_hip_ctx::kKsCounters));
      ih::init_gemm_scratch(device);
    } catch (...) {
      if (c->ks_count) (void)hipFree(c->ks_count);
      if (c->workspace) (void)hipFree(c->workspace);
      if (c->stream) (void)hipStreamDestroy(c->stream);
      delete c;
      throw;
    }
    *out = c;
  });
}

int inferc_hip_destroy(inferc_hip_ctx* ctx) {
  return ih::guard([&] {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    for (auto& t : ctx->tables) (void)hipFree(t.dev);
    ctx->tables.clear();
    if (ctx->workspace) (void)hipFree(ctx->workspace);
    if (ctx->ks_count) (void)hipFree(ctx->ks_count);
    if (ctx->ev_start) (void)hipEventDestroy(ctx->ev_start);
    if (ctx->ev_stop) (void)hipEventDestroy(ctx->ev_stop);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
  });
}

int inferc_hip_reserve_workspace(inferc_hip_ctx* ctx, size_t bytes) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    ctx->ws(bytes);
  });
}

int inferc_hip_set_gemv_decode(inferc_hip_ctx* ctx, int enabled) {
  return ih::guard([&] {
    ih::check_ctx(ctx);
    if (ctx->gemv_decode != (enabled != 0)) {
      ctx->gemv_decode = enabled != 0;
      // executors' captured graphs baked in the old route: they record again
      ++ctx->route_generation;
    }
  });
}

int inferc_hip_gemv_decode_enabled(inferc_hip_ctx* ctx, int* enabled) {
  return ih::guard([&] {
    ih::check_ctx(ctx);
    IH_REQUIRE(enabled != nullptr, INFERC_ERR_ARG, "null argument");
    *enabled = ctx->gemv_decode ? 1 : 0;
  });
}

int inferc_hip_malloc(inferc_hip_ctx* ctx, size_t bytes, void** dptr) {
  return ih::guard([&] {
    ih::check_ctx(ctx);
    IH_REQUIRE(dptr != nullptr, INFERC_ERR_ARG, "null output pointer");
    *dptr = nullptr;
    ctx->make_current();
    if (bytes == 0) return;
    IH_HIP(hipMalloc(dptr, bytes));
  });
}

int inferc_hip_free(inferc_hip_ctx* ctx, void* dptr) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    if (!dptr) return;
    IH_HIP(hipStreamSynchronize(ctx->stream));
    IH_HIP(hipFree(dptr));
  });
}

int inferc_hip_h2d(inferc_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    if (bytes == 0) return;
    IH_REQUIRE(dst && src, INFERC_ERR_ARG, "null pointer");
    IH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    IH_HIP(hipStreamSynchronize(ctx->stream));
  });
}

int inferc_hip_d2h(inferc_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    if (bytes == 0) return;
    IH_REQUIRE(dst && src, INFERC_ERR_ARG, "null pointer");
    IH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    IH_HIP(hipStreamSynchronize(ctx->stream));
  });
}

int inferc_hip_d2d(inferc_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    if (bytes == 0) return;
    IH_REQUIRE(dst && src, INFERC_ERR_ARG, "null pointer");
    IH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
  });
}

int inferc_hip_sync(inferc_hip_ctx* ctx) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    IH_HIP(hipStreamSynchronize(ctx->stream));
  });
}

}  // extern "C"

struct inferc_hip_capture {
  inferc_hip_ctx* ctx = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  uint64_t ws_generation = 0;
};

extern "C" {

int inferc_hip_capture_begin(inferc_hip_ctx* ctx) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    IH_REQUIRE(!ctx->capturing, INFERC_ERR_STATE, "a capture is already in progress");
    IH_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = true;
  });
}

int inferc_hip_capture_end(inferc_hip_ctx* ctx, inferc_hip_capture** out) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    IH_REQUIRE(out != nullptr, INFERC_ERR_ARG, "null output pointer");
    *out = nullptr;
    IH_REQUIRE(ctx->capturing, INFERC_ERR_STATE, "no capture in progress");
    ctx->capturing = false;
    auto* c = new inferc_hip_capture();
    c->ctx = ctx;
    c->ws_generation = ctx->ws_generation;
    hipError_t e = hipStreamEndCapture(ctx->stream, &c->graph);
    if (e == hipSuccess) e = hipGraphInstantiate(&c->exec, c->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
      if (c->graph) (void)hipGraphDestroy(c->graph);
      delete c;
      ih::fail(INFERC_ERR_HIP, std::string("capture: ") + hipGetErrorString(e));
    }
    *out = c;
  });
}

int inferc_hip_capture_replay(inferc_hip_capture* cap) {
  return ih::guard([&] {
    IH_REQUIRE(cap != nullptr && cap->exec != nullptr, INFERC_ERR_ARG, "null capture");
    cap->ctx->make_current();
    IH_REQUIRE(cap->ws_generation == cap->ctx->ws_generation, INFERC_ERR_STATE,
               "the context workspace was reallocated after this capture; capture again");
    IH_HIP(hipGraphLaunch(cap->exec, cap->ctx->stream));
  });
}

int inferc_hip_capture_destroy(inferc_hip_capture* cap) {
  return ih::guard([&] {
    if (!cap) return;
    cap->ctx->make_current();
    (void)hipStreamSynchronize(cap->ctx->stream);
    if (cap->exec) (void)hipGraphExecDestroy(cap->exec);
    if (cap->graph) (void)hipGraphDestroy(cap->graph);
    delete cap;
  });
}

int inferc_hip_timer_start(inferc_hip_ctx* ctx) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    IH_HIP(hipEventRecord(ctx->ev_start, ctx->stream));
  });
}

int inferc_hip_timer_stop(inferc_hip_ctx* ctx, float* ms) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    IH_REQUIRE(ms != nullptr, INFERC_ERR_ARG, "null output pointer");
    IH_HIP(hipEventRecord(ctx->ev_stop, ctx->stream));
    IH_HIP(hipEventSynchronize(ctx->ev_stop));
    IH_HIP(hipEventElapsedTime(ms, ctx->ev_start, ctx->ev_stop));
  });
}

}  // extern "C"
