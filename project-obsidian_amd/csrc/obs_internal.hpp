// obs_internal.hpp — shared internals of libobsidian_hip (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/obsidian_hip.h"

// ---------------------------------------------------------------------------
// Context
// ---------------------------------------------------------------------------
struct obs_prof_pair {
  const char* name;
  hipEvent_t e0, e1;
};
struct obs_prof_stat {
  const char* name;
  double total_ms;
  int64_t launches;
};

struct obs_ctx {
  int device = 0;
  int num_cus = 0;
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;  // own_stream or a caller stream
  hipEvent_t ev_start = nullptr, ev_stop = nullptr;
  std::string err;
  // decode workspace (logits, ids, weights, h, sync counters), grown on demand
  void* decode_ws = nullptr;
  size_t decode_ws_bytes = 0;
  // in-stream kernel timing
  bool prof_on = false;
  std::vector<obs_prof_pair> prof_pairs;
  std::vector<obs_prof_stat> prof_stats;
};

struct obs_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

namespace obs {

int set_error(obs_ctx* ctx, int code, const char* fmt, ...);

// Kernel bracketing for obs_profile_*: call prof_begin before a launch and
// prof_end after it; both are no-ops unless profiling is enabled.
int prof_begin(obs_ctx* ctx, const char* name);
int prof_end(obs_ctx* ctx);

#define OBS_HIP_TRY(ctx, call)                                                   \
  do {                                                                           \
    hipError_t e_ = (call);                                                      \
    if (e_ != hipSuccess)                                                        \
      return ::obs::set_error((ctx), OBS_E_HIP, "%s failed: %s", #call,          \
                              hipGetErrorString(e_));                            \
  } while (0)

// Checks the launch just issued (invalid configuration and the like).
#define OBS_LAUNCH_CHECK(ctx) OBS_HIP_TRY(ctx, hipGetLastError())

// Launch statement bracketed for in-stream timing, then checked.
#define OBS_LAUNCH(ctx, name, ...)                         \
  do {                                                     \
    int rc_ = ::obs::prof_begin((ctx), (name));            \
    if (rc_) return rc_;                                   \
    __VA_ARGS__;                                           \
    OBS_LAUNCH_CHECK(ctx);                                 \
    rc_ = ::obs::prof_end(ctx);                            \
    if (rc_) return rc_;                                   \
  } while (0)

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Workspace for decode: returns device pointer of at least `bytes`.
int ensure_decode_ws(obs_ctx* ctx, size_t bytes, void** out);

}  // namespace obs

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
namespace obsd {

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
// low / high bf16 of a packed pair
__device__ __forceinline__ float bf16lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

// fp32 -> bf16, round to nearest even, NaN kept quiet.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}

// exp(x) by Cody-Waite reduction with ln2 = HI + LO and a degree-7 Taylor
// polynomial (|r| <= ln2/2, truncation error < 6e-9 relative); every step is a
// correctly rounded fp32 operation, so the result is reproducible bit for bit
// on any IEEE fp32 machine that evaluates the same sequence. x < -86 -> +0,
// x > 88.5 -> +inf, NaN -> NaN.
__device__ __forceinline__ float exp_det(float x) {
  if (x != x) return x;
  if (x < -86.0f) return 0.0f;
  if (x > 88.5f) return __builtin_huge_valf();
  const float LOG2E = 1.44269502162933349609375f;
  const float LN2_HI = 0.693145751953125f;
  const float LN2_LO = 1.428606765330187045e-06f;
  const float n = __builtin_rintf(x * LOG2E);
  float r = __builtin_fmaf(-n, LN2_HI, x);
  r = __builtin_fmaf(-n, LN2_LO, r);
  float p = 1.98412698e-04f;
  p = __builtin_fmaf(p, r, 1.38888889e-03f);
  p = __builtin_fmaf(p, r, 8.33333333e-03f);
  p = __builtin_fmaf(p, r, 4.16666667e-02f);
  p = __builtin_fmaf(p, r, 1.66666667e-01f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int ni = static_cast<int>(n);
  if (ni > 127) { p = p * 2.0f; ni -= 1; }
  return p * __uint_as_float(static_cast<uint32_t>(ni + 127) << 23);
}

// silu(g) * u with the deterministic exp (ops.metal:21 form).
__device__ __forceinline__ float silu_mul(float g, float u) { return (g / (1.0f + exp_det(-g))) * u; }

// Wave-wide xor butterfly sum (64 lanes); identical result on every lane.
__device__ __forceinline__ float wave_sum_xor(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off, 64);
  return v;
}

}  // namespace obsd
