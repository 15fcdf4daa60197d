// obs_context.hip — context, buffers, stream, timing: the HIP replacement of
// ObsidianExecutor (src/executor.rs:39-70) and the Model buffer helpers
// (src/forward.rs:264-286).
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "obs_internal.hpp"

namespace {
thread_local std::string g_create_error;

// The scratch of obs_moe_decode_static (the fused decode's exchange area and
// the 4-launch path's intermediates), a file-scope device array: every GPU the
// library runs on holds its own copy until the process ends. Host code never
// passes `scratch` itself to a kernel (on the host it is only a stand-in for
// the symbol): obs_create looks up each device's address once, with that
// device current, and the contexts carry that address.
static __device__ __align__(256) unsigned char scratch[obs::STATIC_SCRATCH_BYTES];

constexpr int MAX_SCRATCH_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_SCRATCH_DEVICES] = {};

// The current device's scratch address, looked up (and zeroed) on the first
// call for that device; null with a message if the lookup fails.
void* device_scratch(int device, std::string* err) {
  if (device < 0 || device >= MAX_SCRATCH_DEVICES) {
    *err = "device index beyond the static scratch table";
    return nullptr;
  }
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      *err = std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e);
      return nullptr;
    }
    // the exchange area must start at zero (epoch 0 in every slot, count 0)
    e = hipMemset(p, 0, obs::STATIC_SCRATCH_BYTES);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
      *err = std::string("clearing the static scratch failed: ") + hipGetErrorString(e);
      return nullptr;
    }
    g_scratch_ptr[device] = p;
  }
  return g_scratch_ptr[device];
}

// Busy-waits `ticks` of the 100 MHz constant clock on one lane; always ends.
__global__ void hold_kernel(uint64_t ticks) {
  if (threadIdx.x != 0) return;
  const uint64_t t0 = wall_clock64();
  while (wall_clock64() - t0 < ticks) __builtin_amdgcn_s_sleep(64);
}
}  // namespace

namespace obs {

int set_error(obs_ctx* ctx, int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (ctx) ctx->err = buf;
  return code;
}

int prof_begin(obs_ctx* ctx, const char* name) {
  if (!ctx->prof_on) return OBS_OK;
  obs_prof_pair p{name, nullptr, nullptr};
  OBS_HIP_TRY(ctx, hipEventCreate(&p.e0));
  OBS_HIP_TRY(ctx, hipEventCreate(&p.e1));
  OBS_HIP_TRY(ctx, hipEventRecord(p.e0, ctx->stream));
  ctx->prof_pairs.push_back(p);
  return OBS_OK;
}

int prof_end(obs_ctx* ctx) {
  if (!ctx->prof_on || ctx->prof_pairs.empty()) return OBS_OK;
  OBS_HIP_TRY(ctx, hipEventRecord(ctx->prof_pairs.back().e1, ctx->stream));
  return OBS_OK;
}

int ensure_decode_ws(obs_ctx* ctx, size_t bytes, void** out) {
  if (ctx->decode_ws_bytes < bytes) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    OBS_HIP_TRY(ctx, hipStreamIsCapturing(ctx->stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
      return set_error(ctx, OBS_E_INVALID, "decode workspace: run this shape once before capturing (%zu bytes)", bytes);
    if (ctx->decode_ws) {  // kept: graphs captured with it may still run
      ctx->retired.push_back(ctx->decode_ws);
      ctx->decode_ws = nullptr;
      ctx->decode_ws_bytes = 0;
    }
    size_t sz = (bytes + 4095) & ~size_t(4095);
    OBS_HIP_TRY(ctx, hipMalloc(&ctx->decode_ws, sz));
    OBS_HIP_TRY(ctx, hipMemset(ctx->decode_ws, 0, sz));
    ctx->decode_ws_bytes = sz;
  }
  *out = ctx->decode_ws;
  return OBS_OK;
}

}  // namespace obs

extern "C" {

const char* obs_create_error(void) { return g_create_error.c_str(); }

int obs_create(int device, obs_ctx** out) {
  g_create_error.clear();
  if (!out) { g_create_error = "out is NULL"; return OBS_E_INVALID; }
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= 0) {
    g_create_error = std::string("no HIP device: ") + (e != hipSuccess ? hipGetErrorString(e) : "count 0");
    return OBS_E_UNSUPPORTED;
  }
  if (device < 0 || device >= n) { g_create_error = "device index out of range"; return OBS_E_INVALID; }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) { g_create_error = "hipGetDeviceProperties failed"; return OBS_E_HIP; }
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    g_create_error = std::string("device is ") + prop.gcnArchName + ", this library is built for gfx950 only";
    return OBS_E_UNSUPPORTED;
  }
  if (hipSetDevice(device) != hipSuccess) { g_create_error = "hipSetDevice failed"; return OBS_E_HIP; }
  obs_ctx* ctx = new obs_ctx();
  ctx->device = device;
  ctx->num_cus = prop.multiProcessorCount;
  if (hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreate(&ctx->ev_start) != hipSuccess || hipEventCreate(&ctx->ev_stop) != hipSuccess) {
    g_create_error = "stream/event creation failed";
    delete ctx;
    return OBS_E_HIP;
  }
  ctx->stream = ctx->own_stream;
  std::string serr;
  ctx->scratch = device_scratch(device, &serr);
  if (!ctx->scratch) {
    g_create_error = serr;
    (void)hipEventDestroy(ctx->ev_start);
    (void)hipEventDestroy(ctx->ev_stop);
    (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
    return OBS_E_HIP;
  }
  *out = ctx;
  return OBS_OK;
}

void obs_destroy(obs_ctx* ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  (void)obs_profile_clear(ctx);
  if (ctx->decode_ws) (void)hipFree(ctx->decode_ws);
  if (ctx->fused_ws) (void)hipFree(ctx->fused_ws);
  if (ctx->attn_ws) (void)hipFree(ctx->attn_ws);
  for (const auto& r : ctx->rope_tables) (void)hipFree(r.table);
  for (void* p : ctx->retired) (void)hipFree(p);
  if (ctx->ev_start) (void)hipEventDestroy(ctx->ev_start);
  if (ctx->ev_stop) (void)hipEventDestroy(ctx->ev_stop);
  if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
  delete ctx;
}

const char* obs_last_error(const obs_ctx* ctx) { return ctx ? ctx->err.c_str() : "null context"; }

int obs_set_stream(obs_ctx* ctx, void* hip_stream) {
  if (!ctx) return OBS_E_INVALID;
  ctx->stream = hip_stream ? static_cast<hipStream_t>(hip_stream) : ctx->own_stream;
  return OBS_OK;
}

void* obs_get_stream(const obs_ctx* ctx) { return ctx ? ctx->stream : nullptr; }

int obs_alloc(obs_ctx* ctx, size_t bytes, void** dptr) {
  if (!ctx || !dptr) return OBS_E_INVALID;
  *dptr = nullptr;
  if (bytes == 0) return obs::set_error(ctx, OBS_E_INVALID, "obs_alloc: zero bytes");
  hipError_t e = hipMalloc(dptr, bytes);
  if (e != hipSuccess) return obs::set_error(ctx, OBS_E_NOMEM, "hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
  return OBS_OK;
}

int obs_free(obs_ctx* ctx, void* dptr) {
  if (!ctx) return OBS_E_INVALID;
  if (!dptr) return OBS_OK;
  OBS_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  OBS_HIP_TRY(ctx, hipFree(dptr));
  return OBS_OK;
}

int obs_upload(obs_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return OBS_E_INVALID;
  if (!bytes) return OBS_OK;
  OBS_HIP_TRY(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  // pageable host memory: make the call safe to reuse the host buffer at once
  OBS_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  return OBS_OK;
}

int obs_download(obs_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return OBS_E_INVALID;
  if (!bytes) return OBS_OK;
  OBS_HIP_TRY(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  OBS_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  return OBS_OK;
}

int obs_memset(obs_ctx* ctx, void* dst, int value, size_t bytes) {
  if (!ctx || (!dst && bytes)) return OBS_E_INVALID;
  if (!bytes) return OBS_OK;
  OBS_HIP_TRY(ctx, hipMemsetAsync(dst, value, bytes, ctx->stream));
  return OBS_OK;
}

int obs_sync(obs_ctx* ctx) {
  if (!ctx) return OBS_E_INVALID;
  OBS_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  return OBS_OK;
}

int obs_timer_start(obs_ctx* ctx) {
  if (!ctx) return OBS_E_INVALID;
  OBS_HIP_TRY(ctx, hipEventRecord(ctx->ev_start, ctx->stream));
  return OBS_OK;
}

int obs_timer_stop(obs_ctx* ctx, float* ms) {
  if (!ctx || !ms) return OBS_E_INVALID;
  OBS_HIP_TRY(ctx, hipEventRecord(ctx->ev_stop, ctx->stream));
  OBS_HIP_TRY(ctx, hipEventSynchronize(ctx->ev_stop));
  OBS_HIP_TRY(ctx, hipEventElapsedTime(ms, ctx->ev_start, ctx->ev_stop));
  return OBS_OK;
}

int obs_capture_begin(obs_ctx* ctx) {
  if (!ctx) return OBS_E_INVALID;
  OBS_HIP_TRY(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
  return OBS_OK;
}

int obs_capture_end(obs_ctx* ctx, obs_graph** out) {
  if (!ctx || !out) return OBS_E_INVALID;
  *out = nullptr;
  obs_graph* g = new obs_graph();
  hipError_t e = hipStreamEndCapture(ctx->stream, &g->graph);
  if (e != hipSuccess) {
    delete g;
    return obs::set_error(ctx, OBS_E_HIP, "hipStreamEndCapture failed: %s", hipGetErrorString(e));
  }
  e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(g->graph);
    delete g;
    return obs::set_error(ctx, OBS_E_HIP, "hipGraphInstantiate failed: %s", hipGetErrorString(e));
  }
  *out = g;
  return OBS_OK;
}

int obs_graph_launch(obs_ctx* ctx, obs_graph* g) {
  if (!ctx || !g || !g->exec) return OBS_E_INVALID;
  OBS_HIP_TRY(ctx, hipGraphLaunch(g->exec, ctx->stream));
  return OBS_OK;
}

void obs_graph_destroy(obs_graph* g) {
  if (!g) return;
  if (g->exec) (void)hipGraphExecDestroy(g->exec);
  if (g->graph) (void)hipGraphDestroy(g->graph);
  delete g;
}

int obs_stream_hold(obs_ctx* ctx, uint32_t us) {
  if (!ctx) return OBS_E_INVALID;
  if (us > 1000000u) us = 1000000u;
  int rate_khz = 0;
  OBS_HIP_TRY(ctx, hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, ctx->device));
  if (rate_khz <= 0) rate_khz = 100000;
  const uint64_t ticks = static_cast<uint64_t>(us) * static_cast<uint64_t>(rate_khz) / 1000u;
  hold_kernel<<<1, 64, 0, ctx->stream>>>(ticks);
  OBS_LAUNCH_CHECK(ctx);
  return OBS_OK;
}

int obs_profile_enable(obs_ctx* ctx, int on) {
  if (!ctx) return OBS_E_INVALID;
  ctx->prof_on = on != 0;
  return OBS_OK;
}

int obs_profile_accumulate(obs_ctx* ctx) {
  if (!ctx) return OBS_E_INVALID;
  OBS_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  for (const obs_prof_pair& p : ctx->prof_pairs) {
    float ms = 0.0f;
    OBS_HIP_TRY(ctx, hipEventElapsedTime(&ms, p.e0, p.e1));
    obs_prof_stat* st = nullptr;
    for (obs_prof_stat& s : ctx->prof_stats)
      if (std::strcmp(s.name, p.name) == 0) st = &s;
    if (!st) {
      ctx->prof_stats.push_back({p.name, 0.0, 0});
      st = &ctx->prof_stats.back();
    }
    st->total_ms += ms;
    st->launches += 1;
  }
  return OBS_OK;
}

int obs_profile_count(const obs_ctx* ctx) { return ctx ? static_cast<int>(ctx->prof_stats.size()) : 0; }

int obs_profile_stat(const obs_ctx* ctx, int i, const char** name, double* total_ms, int64_t* launches) {
  if (!ctx || i < 0 || i >= static_cast<int>(ctx->prof_stats.size())) return OBS_E_INVALID;
  const obs_prof_stat& s = ctx->prof_stats[static_cast<size_t>(i)];
  if (name) *name = s.name;
  if (total_ms) *total_ms = s.total_ms;
  if (launches) *launches = s.launches;
  return OBS_OK;
}

int obs_profile_clear(obs_ctx* ctx) {
  if (!ctx) return OBS_E_INVALID;
  for (obs_prof_pair& p : ctx->prof_pairs) {
    (void)hipEventDestroy(p.e0);
    (void)hipEventDestroy(p.e1);
  }
  ctx->prof_pairs.clear();
  ctx->prof_stats.clear();
  return OBS_OK;
}

}  // extern "C"
