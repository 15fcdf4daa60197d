// obs_elementwise.hip — ew_swiglu / ew_scaled_add (shaders/ops.metal:18-29,
// Model::swiglu / Model::scaled_add, src/forward.rs:370-380), bf16 storage,
// fp32 math. Inside the fused decode and prefill paths these are epilogues;
// the standalone entry points serve callers that compose the path themselves.
#include "obs_internal.hpp"

namespace {
using namespace obsd;

__global__ void __launch_bounds__(256) swiglu_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                                                     uint16_t* __restrict__ h, uint32_t n) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) h[i] = f32_to_bf16(silu_mul(bf16_to_f32(g[i]), bf16_to_f32(u[i])));
}

__global__ void __launch_bounds__(256) scaled_add_kernel(uint16_t* __restrict__ acc, const uint16_t* __restrict__ y,
                                                         float scale, uint32_t n) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) acc[i] = f32_to_bf16(__builtin_fmaf(scale, bf16_to_f32(y[i]), bf16_to_f32(acc[i])));
}
}  // namespace

extern "C" {

int obs_swiglu(obs_ctx* ctx, const uint16_t* g, const uint16_t* u, uint16_t* h, uint32_t n) {
  if (!ctx) return OBS_E_INVALID;
  if (!g || !u || !h) return obs::set_error(ctx, OBS_E_INVALID, "obs_swiglu: null pointer");
  if (n == 0) return OBS_OK;
  OBS_LAUNCH(ctx, "swiglu", swiglu_kernel<<<(n + 255) / 256, 256, 0, ctx->stream>>>(g, u, h, n));
  return OBS_OK;
}

int obs_scaled_add(obs_ctx* ctx, uint16_t* acc, const uint16_t* y, float scale, uint32_t n) {
  if (!ctx) return OBS_E_INVALID;
  if (!acc || !y) return obs::set_error(ctx, OBS_E_INVALID, "obs_scaled_add: null pointer");
  if (n == 0) return OBS_OK;
  OBS_LAUNCH(ctx, "scaled_add", scaled_add_kernel<<<(n + 255) / 256, 256, 0, ctx->stream>>>(acc, y, scale, n));
  return OBS_OK;
}

}  // extern "C"
