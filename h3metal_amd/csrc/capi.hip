// The C ABI of include/h3hip.h: device context, zero-filled buffers, a table
// of precompiled kernel specialisations, dispatch on one HIP stream, and HIP
// event timing.
//
// Reference behaviour mirrored (src/capi.mm): thread-local last error
// (:15-17,75), zero-filled buffers (src/metal_rt.mm:80-83), a pipeline cache
// keyed by (file, fn, macros) that owns its entries (:185-195), dispatch
// returning 0/-1 (:202-225), wait returning GPU seconds or -1 (:229-244),
// per-dispatch profiling (:246-257).
#include "h3hip_internal.h"
#include "../../include/h3hip.h"

#include <algorithm>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <vector>

namespace {

thread_local std::string g_error;

void set_error(const std::string &msg) { g_error = msg; }

h3::Macros parse_macros(const char *s) {
  h3::Macros m;
  if (!s) return m;
  std::string all(s);
  size_t pos = 0;
  while (pos <= all.size()) {
    size_t end = all.find(';', pos);
    if (end == std::string::npos) end = all.size();
    std::string item = all.substr(pos, end - pos);
    if (!item.empty()) {
      size_t eq = item.find('=');
      if (eq == std::string::npos) m[item] = "1";
      else m[item.substr(0, eq)] = item.substr(eq + 1);
    }
    pos = end + 1;
  }
  return m;
}

struct Buffer {
  void *dev = nullptr;
  uint64_t bytes = 0;
};

std::string module_name(const std::string &file) {
  std::string f = file;
  const char *sfx[] = {".metal", ".hip"};
  for (const char *s : sfx) {
    size_t n = strlen(s);
    if (f.size() > n && f.compare(f.size() - n, n, s) == 0) f = f.substr(0, f.size() - n);
  }
  return f;
}

}  // namespace

namespace h3 {

bool macro_int(const Macros &m, const char *key, int def, int *out, std::string *err) {
  auto it = m.find(key);
  if (it == m.end()) {
    *out = def;
    return true;
  }
  char *end = nullptr;
  long v = strtol(it->second.c_str(), &end, 10);
  if (it->second.empty() || *end) {
    *err = std::string("macro ") + key + "=" + it->second + " is not an integer";
    return false;
  }
  *out = (int)v;
  return true;
}

std::string macro_str(const Macros &m, const char *key, const char *def) {
  auto it = m.find(key);
  return it == m.end() ? std::string(def) : it->second;
}


// CUs of the current device (the tail splits size themselves to them), cached per device.
int cu_count() {
  static int cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!cache[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cache[dev] = n;
  }
  return cache[dev];
}

}  // namespace h3

// Scratch memory of h3_dispatch_static (the entry point that allocates nothing): a fixed array in the code
// object's device memory, one copy per GPU, kept until the process ends. Host code must never pass the array's
// name to a kernel (it is a host-side stand-in, not a device address): h3_open looks up each device's address
// with hipGetSymbolAddress once, with that device current, and only that address is used.
static __device__ __align__(256) char scratch[h3::STATIC_SCRATCH_BYTES_VALUE];

namespace {
std::mutex g_scratch_mu;
void *g_scratch_ptr[64] = {};  // per device id

// The device address of `scratch` on `device` (current), looked up on the first call; NULL with a message.
void *static_scratch(int device, std::string *err) {
  if (device < 0 || device >= 64) {
    *err = "device id out of range";
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      *err = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
      return nullptr;
    }
    g_scratch_ptr[device] = ptr;
  }
  return g_scratch_ptr[device];
}
}  // namespace

struct h3_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string name;
  uint64_t free_at_open = 0, total = 0;
  std::map<std::string, std::unique_ptr<h3::Pipeline>> pipelines;
  // scratch memory of the launches on this context's stream (work on one stream is ordered, so one buffer
  // serves every launch); sized at open for the attention split, grown only by h3_reserve_workspace
  void *ws = nullptr;
  size_t ws_bytes = 0;
  void *static_ws = nullptr;  // this device's copy of `scratch` (h3_dispatch_static)
  // timing of the work since the last wait
  hipEvent_t t0 = nullptr, t1 = nullptr;
  bool timing = false;
  // profiling: one event pair per dispatch
  bool profile = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> prof_events;
  std::vector<double> prof;
};

static bool hip_ok(hipError_t e, const char *what) {
  if (e == hipSuccess) return true;
  set_error(std::string(what) + ": " + hipGetErrorString(e));
  return false;
}

static void drain_profile(h3_ctx *ctx) {
  for (auto &pr : ctx->prof_events) {
    float ms = 0;
    if (hipEventElapsedTime(&ms, pr.first, pr.second) == hipSuccess) ctx->prof.push_back(ms * 1e-3);
    hipEventDestroy(pr.first);
    hipEventDestroy(pr.second);
  }
  ctx->prof_events.clear();
}

extern "C" {

const char *h3_last_error(void) { return g_error.c_str(); }

h3_ctx *h3_open(const char *kernel_dir) {
  (void)kernel_dir;
  int n = 0;
  if (!hip_ok(hipGetDeviceCount(&n), "hipGetDeviceCount")) return nullptr;
  if (n < 1) {
    set_error("no HIP device");
    return nullptr;
  }
  auto *ctx = new h3_ctx;
  if (!hip_ok(hipGetDevice(&ctx->device), "hipGetDevice")) {
    delete ctx;
    return nullptr;
  }
  hipDeviceProp_t prop;
  if (!hip_ok(hipGetDeviceProperties(&prop, ctx->device), "hipGetDeviceProperties")) {
    delete ctx;
    return nullptr;
  }
  if (std::string(prop.gcnArchName).rfind("gfx950", 0) != 0) {
    set_error(std::string("h3hip kernels are built for gfx950; this device is ") + prop.gcnArchName);
    delete ctx;
    return nullptr;
  }
  ctx->name = std::string(prop.name) + " (" + prop.gcnArchName + ")";
  size_t fr = 0, tot = 0;
  hipMemGetInfo(&fr, &tot);
  ctx->free_at_open = fr;
  ctx->total = tot;
  if (!hip_ok(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking), "hipStreamCreate") ||
      !hip_ok(hipEventCreate(&ctx->t0), "hipEventCreate") || !hip_ok(hipEventCreate(&ctx->t1), "hipEventCreate")) {
    delete ctx;
    return nullptr;
  }
  const size_t ws = h3::attention_workspace_max(h3::cu_count());
  if (!hip_ok(hipMalloc(&ctx->ws, ws), "cannot allocate the dispatch scratch memory")) {
    h3_close(ctx);
    return nullptr;
  }
  ctx->ws_bytes = ws;
  std::string err;
  ctx->static_ws = static_scratch(ctx->device, &err);
  if (!ctx->static_ws) {
    set_error(err);
    h3_close(ctx);
    return nullptr;
  }
  return ctx;
}

void h3_close(h3_ctx *ctx) {
  if (!ctx) return;
  if (ctx->stream) hipStreamSynchronize(ctx->stream);
  drain_profile(ctx);
  if (ctx->ws) hipFree(ctx->ws);
  if (ctx->t0) hipEventDestroy(ctx->t0);
  if (ctx->t1) hipEventDestroy(ctx->t1);
  if (ctx->stream) hipStreamDestroy(ctx->stream);
  delete ctx;
}

int h3_reserve_workspace(h3_ctx *ctx, uint64_t bytes) {
  if (!ctx) {
    set_error("h3_reserve_workspace: no context");
    return -1;
  }
  if (bytes <= ctx->ws_bytes) return 0;
  // queued work may still use the old buffer
  if (!hip_ok(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize")) return -1;
  void *p = nullptr;
  if (!hip_ok(hipMalloc(&p, bytes), ("cannot allocate " + std::to_string(bytes) + " bytes of scratch").c_str()))
    return -1;
  hipFree(ctx->ws);
  ctx->ws = p;
  ctx->ws_bytes = bytes;
  return 0;
}

uint64_t h3_workspace_bytes(h3_ctx *ctx) { return ctx ? ctx->ws_bytes : 0; }

const char *h3_device_name(h3_ctx *ctx) { return ctx ? ctx->name.c_str() : ""; }
uint64_t h3_recommended_working_set(h3_ctx *ctx) { return ctx ? ctx->free_at_open : 0; }
uint64_t h3_max_buffer_length(h3_ctx *ctx) { return ctx ? ctx->total : 0; }

void *h3_buffer(h3_ctx *ctx, uint64_t bytes) {
  if (!ctx) {
    set_error("h3_buffer: no context");
    return nullptr;
  }
  auto *b = new Buffer;
  b->bytes = bytes;
  if (!hip_ok(hipMalloc(&b->dev, std::max<uint64_t>(bytes, 1)),
              ("cannot allocate a buffer of " + std::to_string(bytes) + " bytes").c_str())) {
    delete b;
    return nullptr;
  }
  // zero-filled, like the reference's buffers; ordered before any later work on the stream
  if (!hip_ok(hipMemsetAsync(b->dev, 0, std::max<uint64_t>(bytes, 1), ctx->stream), "hipMemsetAsync") ||
      !hip_ok(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize")) {
    hipFree(b->dev);
    delete b;
    return nullptr;
  }
  return b;
}

void *h3_buffer_contents(void *buf) {
  (void)buf;
  set_error("device buffers have no CPU view: use h3_buffer_read / h3_buffer_write");
  return nullptr;
}

uint64_t h3_buffer_length(void *buf) { return buf ? static_cast<Buffer *>(buf)->bytes : 0; }
void *h3_buffer_device(void *buf) { return buf ? static_cast<Buffer *>(buf)->dev : nullptr; }

void h3_buffer_release(void *buf) {
  if (!buf) return;
  auto *b = static_cast<Buffer *>(buf);
  // hipFree synchronises the device, so work still reading the buffer finishes first
  hipFree(b->dev);
  delete b;
}

static int copy_check(h3_ctx *ctx, void *buf, uint64_t offset, uint64_t bytes, const char *what) {
  if (!ctx || !buf) {
    set_error(std::string(what) + ": no context or buffer");
    return -1;
  }
  auto *b = static_cast<Buffer *>(buf);
  if (offset > b->bytes || bytes > b->bytes - offset) {
    set_error(std::string(what) + ": range [" + std::to_string(offset) + ", " + std::to_string(offset + bytes) +
              ") outside a buffer of " + std::to_string(b->bytes) + " bytes");
    return -1;
  }
  return 0;
}

int h3_buffer_write(h3_ctx *ctx, void *buf, uint64_t offset, const void *src, uint64_t bytes) {
  if (copy_check(ctx, buf, offset, bytes, "h3_buffer_write")) return -1;
  if (!bytes) return 0;
  auto *b = static_cast<Buffer *>(buf);
  if (!hip_ok(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize") ||
      !hip_ok(hipMemcpy(static_cast<char *>(b->dev) + offset, src, bytes, hipMemcpyHostToDevice), "hipMemcpy"))
    return -1;
  return 0;
}

int h3_buffer_read(h3_ctx *ctx, void *buf, uint64_t offset, void *dst, uint64_t bytes) {
  if (copy_check(ctx, buf, offset, bytes, "h3_buffer_read")) return -1;
  if (!bytes) return 0;
  auto *b = static_cast<Buffer *>(buf);
  if (!hip_ok(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize") ||
      !hip_ok(hipMemcpy(dst, static_cast<char *>(b->dev) + offset, bytes, hipMemcpyDeviceToHost), "hipMemcpy"))
    return -1;
  return 0;
}

// Stream work is timed from the first operation after a wait (t0) to the next h3_wait; in profile mode each
// operation also gets its own pair of events.
static bool op_begin(h3_ctx *ctx, bool prof, hipEvent_t *e0, hipEvent_t *e1) {
  if (!ctx->timing) {
    if (!hip_ok(hipEventRecord(ctx->t0, ctx->stream), "hipEventRecord")) return false;
    ctx->timing = true;
  }
  if (prof && (!hip_ok(hipEventCreate(e0), "hipEventCreate") || !hip_ok(hipEventCreate(e1), "hipEventCreate") ||
               !hip_ok(hipEventRecord(*e0, ctx->stream), "hipEventRecord")))
    return false;
  return true;
}
static void op_end(h3_ctx *ctx, hipEvent_t e0, hipEvent_t e1) {
  if (!e0) return;
  hipEventRecord(e1, ctx->stream);
  ctx->prof_events.emplace_back(e0, e1);
}

int h3_buffer_copy(h3_ctx *ctx, void *dst, uint64_t dst_offset, void *src, uint64_t src_offset, uint64_t bytes) {
  if (copy_check(ctx, dst, dst_offset, bytes, "h3_buffer_copy (destination)") ||
      copy_check(ctx, src, src_offset, bytes, "h3_buffer_copy (source)"))
    return -1;
  if (!bytes) return 0;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (!op_begin(ctx, ctx->profile, &e0, &e1)) return -1;
  char *d = static_cast<char *>(static_cast<Buffer *>(dst)->dev) + dst_offset;
  const char *sp = static_cast<const char *>(static_cast<Buffer *>(src)->dev) + src_offset;
  if (!hip_ok(hipMemcpyAsync(d, sp, bytes, hipMemcpyDeviceToDevice, ctx->stream), "hipMemcpyAsync")) {
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    return -1;
  }
  op_end(ctx, e0, e1);
  return 0;
}

void *h3_pipeline(h3_ctx *ctx, const char *file, const char *fn, const char *macros) {
  if (!ctx || !file || !fn) {
    set_error("h3_pipeline: missing context, file or function name");
    return nullptr;
  }
  h3::Macros m = parse_macros(macros);
  std::string mod = module_name(file);
  std::string key = mod + ":" + fn + "(";
  bool first = true;
  for (auto &kv : m) {  // std::map: sorted, so equal macro sets give equal keys
    key += (first ? "" : ";") + kv.first + "=" + kv.second;
    first = false;
  }
  key += ")";
  auto it = ctx->pipelines.find(key);
  if (it != ctx->pipelines.end()) return it->second.get();
  auto pl = std::make_unique<h3::Pipeline>();
  pl->name = key;
  std::string err;
  bool ok;
  if (mod == "attention") ok = h3::make_attention(fn, m, pl.get(), &err);
  else if (mod == "ops") ok = h3::make_ops(fn, m, pl.get(), &err);
  else if (mod == "gemm") ok = h3::make_gemm(fn, m, pl.get(), &err);
  else {
    ok = false;
    err = "unknown kernel module '" + std::string(file) + "' (have: attention, ops, gemm)";
  }
  if (!ok) {
    set_error(key + ": " + err);
    return nullptr;
  }
  h3::Pipeline *raw = pl.get();
  ctx->pipelines[key] = std::move(pl);
  return raw;
}

int h3_pipeline_max_threads(void *pso) { return pso ? static_cast<h3::Pipeline *>(pso)->threads : 0; }

static int dispatch(h3_ctx *ctx, void *pso, const h3_arg *bufs, int nbufs, const void *params,
                    uint32_t params_len, bool no_alloc) {
  if (!ctx) {
    set_error("dispatch without a context");
    return -1;
  }
  if (!pso) {
    set_error("dispatch without a pipeline");
    return -1;
  }
  if (nbufs < 0 || nbufs > 32) {
    set_error("dispatch: buffer count " + std::to_string(nbufs) + " outside 0..32");
    return -1;
  }
  auto *pl = static_cast<h3::Pipeline *>(pso);
  h3::Arg args[32];
  for (int i = 0; i < nbufs; i++) {
    auto *b = static_cast<Buffer *>(bufs[i].buf);
    if (!b) continue;
    if (bufs[i].offset > b->bytes) {
      set_error("dispatch: buffer " + std::to_string(i) + " offset beyond its end");
      return -1;
    }
    args[i].ptr = static_cast<char *>(b->dev) + bufs[i].offset;
    args[i].avail = b->bytes - bufs[i].offset;
  }
  // per-dispatch profiling creates events; the allocation-free entry point does not profile
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (!op_begin(ctx, ctx->profile && !no_alloc, &e0, &e1)) return -1;
  std::string err;
  h3::Exec ex;
  ex.stream = ctx->stream;
  ex.ws = no_alloc ? ctx->static_ws : ctx->ws;
  ex.ws_bytes = no_alloc ? h3::STATIC_SCRATCH_BYTES_VALUE : ctx->ws_bytes;
  int rc = pl->launch(*pl, ex, args, nbufs, params, params_len, &err);
  if (rc) {
    set_error(pl->name + ": " + err);
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    return -1;
  }
  hipError_t le = hipGetLastError();
  if (le != hipSuccess) {
    set_error(pl->name + ": launch failed: " + hipGetErrorString(le));
    return -1;
  }
  op_end(ctx, e0, e1);
  return 0;
}

int h3_dispatch(h3_ctx *ctx, void *pso, const uint32_t grid[3], const uint32_t tg[3], const h3_arg *bufs,
                int nbufs, const void *params, uint32_t params_len, int params_index, uint32_t tg_mem_bytes) {
  (void)grid;
  (void)tg;
  (void)params_index;
  (void)tg_mem_bytes;
  return dispatch(ctx, pso, bufs, nbufs, params, params_len, false);
}

int h3_dispatch_static(h3_ctx *ctx, void *pso, const uint32_t grid[3], const uint32_t tg[3], const h3_arg *bufs,
                       int nbufs, const void *params, uint32_t params_len, int params_index, uint32_t tg_mem_bytes) {
  (void)grid;
  (void)tg;
  (void)params_index;
  (void)tg_mem_bytes;
  return dispatch(ctx, pso, bufs, nbufs, params, params_len, true);
}

void h3_commit(h3_ctx *ctx) { (void)ctx; }

double h3_wait(h3_ctx *ctx) {
  if (!ctx) {
    set_error("h3_wait: no context");
    return -1.0;
  }
  double secs = 0;
  if (ctx->timing) {
    hipEventRecord(ctx->t1, ctx->stream);
    if (!hip_ok(hipEventSynchronize(ctx->t1), "GPU work failed")) {
      ctx->timing = false;
      return -1.0;
    }
    float ms = 0;
    hipEventElapsedTime(&ms, ctx->t0, ctx->t1);
    secs = ms * 1e-3;
    ctx->timing = false;
  }
  if (!hip_ok(hipStreamSynchronize(ctx->stream), "GPU work failed")) return -1.0;
  drain_profile(ctx);
  return secs;
}

void h3_set_profile(h3_ctx *ctx, int on) {
  if (!ctx) return;
  h3_wait(ctx);
  ctx->profile = on != 0;
  ctx->prof.clear();
}

int h3_profile_take(h3_ctx *ctx, double *seconds, int max) {
  if (!ctx) return 0;
  hipStreamSynchronize(ctx->stream);
  drain_profile(ctx);
  int n = std::min<int>(max, (int)ctx->prof.size());
  for (int i = 0; i < n; i++) seconds[i] = ctx->prof[i];
  ctx->prof.erase(ctx->prof.begin(), ctx->prof.begin() + n);
  return n;
}

}  // extern "C"
