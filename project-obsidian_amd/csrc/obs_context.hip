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

// Dispatch probes (obs_create). xcd_probe_kernel: workgroup b of a grid shaped
// like the fused kernels' (256 workgroups of 256 threads, one per CU) records
// the XCD it runs on (the hardware XCC_ID register, an index below 32).
constexpr uint32_t PROBE_XCD_GRID = 256;
__global__ void __launch_bounds__(256, 1) xcd_probe_kernel(uint32_t* xcc) {
  if (threadIdx.x != 0) return;
  uint32_t id;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(id));
  xcc[blockIdx.x] = id & 0xfu;
}

// order_probe_kernel: a grid of many more workgroups than can be resident at
// once. Workgroup b marks itself started, then waits (bounded) until
// workgroup b - 8, the previous one of its XCD under the round-robin deal, has
// started. When the dispatcher starts each XCD's workgroups in index order the
// predecessor is always running or done and every wait ends at once; when a
// workgroup could hold a slot its predecessor needs, the wait runs out and the
// grid reports it.
constexpr uint32_t PROBE_ORDER_GRID = 8192;
constexpr uint64_t PROBE_WAIT_TICKS = 1000000ull;  // 10 ms of the 100 MHz clock
__global__ void __launch_bounds__(256) order_probe_kernel(uint32_t* started, uint32_t* late) {
  if (threadIdx.x != 0) return;
  const uint32_t b = blockIdx.x;
  __hip_atomic_store(started + b, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  if (b < 8u) return;
  const uint64_t t0 = wall_clock64();
  while (__hip_atomic_load(started + b - 8u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u) {
    if (wall_clock64() - t0 > PROBE_WAIT_TICKS) {
      __hip_atomic_store(late, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      break;
    }
  }
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

uint32_t dispatch_gate(int num_cus, bool xcd_map_ok, bool inorder_ok) {
  uint32_t paths = 0;
  if (num_cus >= static_cast<int>(fused_decode_workgroups()) && xcd_map_ok) paths |= OBS_PATH_FUSED_DECODE;
  if (num_cus >= static_cast<int>(fused_attn_workgroups()) && xcd_map_ok) paths |= OBS_PATH_FUSED_ATTN;
  if (xcd_map_ok && inorder_ok) paths |= OBS_PATH_FFN_ONE_LAUNCH;
  return paths;
}

int probe_dispatch(obs_ctx* ctx) {
  ctx->xcd_map_ok = ctx->inorder_ok = false;
  uint32_t* d = nullptr;
  const size_t words = PROBE_XCD_GRID + PROBE_ORDER_GRID + 64;
  OBS_HIP_TRY(ctx, hipMalloc(&d, words * sizeof(uint32_t)));
  uint32_t* xcc = d;
  uint32_t* started = d + PROBE_XCD_GRID;
  uint32_t* late = started + PROBE_ORDER_GRID;
  std::vector<uint32_t> h(PROBE_XCD_GRID + 1);
  hipError_t e = hipMemsetAsync(d, 0, words * sizeof(uint32_t), ctx->stream);
  if (e == hipSuccess) {
    xcd_probe_kernel<<<PROBE_XCD_GRID, 256, 0, ctx->stream>>>(xcc);
    order_probe_kernel<<<PROBE_ORDER_GRID, 256, 0, ctx->stream>>>(started, late);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipMemcpyAsync(h.data(), xcc, PROBE_XCD_GRID * sizeof(uint32_t), hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(h.data() + PROBE_XCD_GRID, late, sizeof(uint32_t), hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  (void)hipFree(d);
  if (e != hipSuccess) return set_error(ctx, OBS_E_HIP, "dispatch probe failed: %s", hipGetErrorString(e));
  // The fused kernels need each group (workgroups b with one b % 8) inside one
  // XCD, and the 8 groups on 8 different XCDs. Which XCD takes group 0 may
  // change from launch to launch (the dispatcher's round-robin continues from
  // the previous dispatch), so only that structure is checked.
  bool map = true;
  uint32_t seen = 0;
  for (uint32_t b = 0; b < PROBE_XCD_GRID; ++b) map = map && h[b] == h[b % 8u] && h[b] < 32u;
  for (uint32_t g = 0; g < 8u && map; ++g) seen |= 1u << h[g];
  map = map && __builtin_popcount(seen) == 8;
  ctx->xcd_map_ok = map;
  ctx->inorder_ok = h[PROBE_XCD_GRID] == 0u;
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
  int rc = ctx->scratch ? OBS_OK : OBS_E_HIP;
  if (rc == OBS_OK) {
    if (hipMalloc(&ctx->status_dev, obs::CTX_ST_WORDS * sizeof(uint32_t)) != hipSuccess ||
        hipMemset(ctx->status_dev, 0, obs::CTX_ST_WORDS * sizeof(uint32_t)) != hipSuccess) {
      serr = "status words: hipMalloc/hipMemset failed";
      rc = OBS_E_HIP;
    }
  }
  if (rc == OBS_OK) {
    if (hipMalloc(&ctx->route_cnt, obs::ROUTE_CNT_WORDS * sizeof(uint32_t)) != hipSuccess ||
        hipMemsetAsync(ctx->route_cnt, 0, obs::ROUTE_CNT_WORDS * sizeof(uint32_t), ctx->stream) != hipSuccess ||
        hipStreamSynchronize(ctx->stream) != hipSuccess) {
      serr = "router counters: hipMalloc/hipMemset failed";
      rc = OBS_E_HIP;
    }
  }
  if (rc == OBS_OK) rc = obs::probe_dispatch(ctx);
  if (rc == OBS_OK) rc = obs::prefill_init(ctx);
  if (rc != OBS_OK) {
    g_create_error = serr.empty() ? ctx->err : serr;
    obs_destroy(ctx);
    return rc;
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
  if (ctx->layer_ws) (void)hipFree(ctx->layer_ws);
  if (ctx->status_dev) (void)hipFree(ctx->status_dev);
  if (ctx->route_cnt) (void)hipFree(ctx->route_cnt);
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

uint32_t obs_dispatch_gate(int num_cus, int xcd_map_ok, int inorder_ok) {
  return obs::dispatch_gate(num_cus, xcd_map_ok != 0, inorder_ok != 0);
}

int obs_dispatch_info(const obs_ctx* ctx, int* num_cus, int* xcd_map_ok, int* inorder_ok) {
  if (!ctx) return OBS_E_INVALID;
  if (num_cus) *num_cus = ctx->num_cus;
  if (xcd_map_ok) *xcd_map_ok = ctx->xcd_map_ok ? 1 : 0;
  if (inorder_ok) *inorder_ok = ctx->inorder_ok ? 1 : 0;
  return OBS_OK;
}

int obs_set_dispatch_facts(obs_ctx* ctx, int xcd_map_ok, int inorder_ok) {
  if (!ctx) return OBS_E_INVALID;
  ctx->xcd_map_ok = xcd_map_ok != 0;
  ctx->inorder_ok = inorder_ok != 0;
  return OBS_OK;
}

int obs_debug_ffn_wait(obs_ctx* ctx, uint32_t extra_count, uint32_t wait_us) {
  if (!ctx) return OBS_E_INVALID;
  if (wait_us == 0u || wait_us > 100000u)
    return obs::set_error(ctx, OBS_E_INVALID, "obs_debug_ffn_wait: wait_us must be 1..100000 (got %u)", wait_us);
  ctx->ffn_extra_count = extra_count;
  ctx->ffn_wait_ticks = static_cast<uint64_t>(wait_us) * 100u;  // the constant clock runs at 100 MHz
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
