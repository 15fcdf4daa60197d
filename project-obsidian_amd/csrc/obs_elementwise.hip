// obs_elementwise.hip — ew_swiglu / ew_scaled_add (shaders/ops.metal:18-29,
// Model::swiglu / Model::scaled_add, src/forward.rs:370-380) and RMSNorm
// (shaders/rmsnorm.metal:17-35, Model::rmsnorm forward.rs:345-357), bf16
// storage, fp32 math. Inside the fused decode and prefill paths the first two
// are epilogues and the norm a prologue; the standalone entry points serve
// callers that compose the path themselves.
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
// The same, 8 elements (16 bytes) per thread: both arrays 16-byte aligned, n8 = n / 8.
__global__ void __launch_bounds__(256) scaled_add8_kernel(uint16_t* __restrict__ acc, const uint16_t* __restrict__ y,
                                                          float scale, uint32_t n8) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const uint4 a = reinterpret_cast<const uint4*>(acc)[i], b = reinterpret_cast<const uint4*>(y)[i];
  const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    o[j] = pack_bf16x2(__builtin_fmaf(scale, bf16lo(bw[j]), bf16lo(aw[j])),
                       __builtin_fmaf(scale, bf16hi(bw[j]), bf16hi(aw[j])));
  reinterpret_cast<uint4*>(acc)[i] = make_uint4(o[0], o[1], o[2], o[3]);
}
// One wave per row; lane l owns the dim/64 contiguous columns [l*c, (l+1)*c).
// sum(x^2): serial fma over the lane's columns, then wave_sum_asc (the xor
// butterfly 1..32); inv = 1/sqrt(sum/dim + eps) with IEEE sqrt and division
// once per row; out = (x * inv) * w — the fused decode kernel computes the
// same sequence.
// C = dim/64 when it is a multiple of 8 (16-byte loads), else 0 (any dim).
template <uint32_t C>
__global__ void __launch_bounds__(256) rmsnorm_kernel(const uint16_t* x, const uint16_t* __restrict__ w,
                                                      uint16_t* out, uint32_t rows, uint32_t dim, float eps) {
  const uint32_t lane = threadIdx.x & 63u, row = blockIdx.x * 4u + (threadIdx.x >> 6);
  if (row >= rows) return;  // wave-uniform: the butterfly below needs the whole wave
  const uint32_t chunk = C ? C : dim / 64u, c0 = lane * chunk;
  const uint16_t* xr = x + static_cast<size_t>(row) * dim + c0;
  uint16_t* orow = out + static_cast<size_t>(row) * dim + c0;
  if constexpr (C != 0) {
    uint4 xv[C / 8], wv[C / 8];  // the weights load with x: no second round trip after the reduction
#pragma unroll
    for (uint32_t i = 0; i < C / 8; ++i) xv[i] = reinterpret_cast<const uint4*>(xr)[i];
#pragma unroll
    for (uint32_t i = 0; i < C / 8; ++i) wv[i] = reinterpret_cast<const uint4*>(w + c0)[i];
    float acc = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < C / 8; ++i) {
      const uint32_t wd[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
#pragma unroll
      for (uint32_t j = 0; j < 4; ++j) {
        const float a = bf16lo(wd[j]), b = bf16hi(wd[j]);
        acc = __builtin_fmaf(a, a, acc);
        acc = __builtin_fmaf(b, b, acc);
      }
    }
    const float inv = 1.0f / __builtin_sqrtf(wave_sum_asc(acc) / static_cast<float>(dim) + eps);
#pragma unroll
    for (uint32_t i = 0; i < C / 8; ++i) {
      const uint32_t xd[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w}, wdd[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
      uint32_t o[4];
#pragma unroll
      for (uint32_t j = 0; j < 4; ++j)
        o[j] = pack_bf16x2((bf16lo(xd[j]) * inv) * bf16lo(wdd[j]), (bf16hi(xd[j]) * inv) * bf16hi(wdd[j]));
      reinterpret_cast<uint4*>(orow)[i] = make_uint4(o[0], o[1], o[2], o[3]);
    }
  } else {
    float acc = 0.0f;
    for (uint32_t c = 0; c < chunk; ++c) {
      const float v = bf16_to_f32(xr[c]);
      acc = __builtin_fmaf(v, v, acc);
    }
    const float inv = 1.0f / __builtin_sqrtf(wave_sum_asc(acc) / static_cast<float>(dim) + eps);
    float nv[128];  // chunk <= 128 (dim <= 8192): read all before writing (x and out may alias)
    for (uint32_t c = 0; c < chunk; ++c) nv[c] = (bf16_to_f32(xr[c]) * inv) * bf16_to_f32(w[c0 + c]);
    for (uint32_t c = 0; c < chunk; ++c) orow[c] = f32_to_bf16(nv[c]);
  }
}
}  // namespace

namespace obs {
int launch_rmsnorm(obs_ctx* ctx, const uint16_t* x, const uint16_t* w, uint16_t* out, uint32_t rows, uint32_t dim,
                   float eps) {
  const uint32_t grid = (rows + 3u) / 4u;
  const bool vec = obs::aligned(x, 16) && obs::aligned(w, 16) && obs::aligned(out, 16);
  if (vec && dim == 2048)
    OBS_LAUNCH(ctx, "rmsnorm", rmsnorm_kernel<32><<<grid, 256, 0, ctx->stream>>>(x, w, out, rows, dim, eps));
  else if (vec && dim == 4096)
    OBS_LAUNCH(ctx, "rmsnorm", rmsnorm_kernel<64><<<grid, 256, 0, ctx->stream>>>(x, w, out, rows, dim, eps));
  else if (vec && dim == 1024)
    OBS_LAUNCH(ctx, "rmsnorm", rmsnorm_kernel<16><<<grid, 256, 0, ctx->stream>>>(x, w, out, rows, dim, eps));
  else
    OBS_LAUNCH(ctx, "rmsnorm", rmsnorm_kernel<0><<<grid, 256, 0, ctx->stream>>>(x, w, out, rows, dim, eps));
  return OBS_OK;
}
}  // namespace obs

extern "C" {

int obs_swiglu(obs_ctx* ctx, const uint16_t* g, const uint16_t* u, uint16_t* h, uint32_t n) {
  if (!ctx) return OBS_E_INVALID;
  if (!g || !u || !h) return obs::set_error(ctx, OBS_E_INVALID, "obs_swiglu: null pointer");
  if (n == 0) return OBS_OK;
  OBS_LAUNCH(ctx, "swiglu", swiglu_kernel<<<(n + 255) / 256, 256, 0, ctx->stream>>>(g, u, h, n));
  return OBS_OK;
}

int obs_rmsnorm(obs_ctx* ctx, const uint16_t* x, const uint16_t* weight, uint16_t* out, uint32_t rows, uint32_t dim,
                float eps) {
  if (!ctx) return OBS_E_INVALID;
  if (!x || !weight || !out) return obs::set_error(ctx, OBS_E_INVALID, "obs_rmsnorm: null pointer");
  if (dim == 0 || dim % 64u != 0 || dim > 8192u)
    return obs::set_error(ctx, OBS_E_SHAPE, "obs_rmsnorm: dim must be a multiple of 64 in [64, 8192] (got %u)", dim);
  if (rows == 0) return OBS_OK;
  return obs::launch_rmsnorm(ctx, x, weight, out, rows, dim, eps);
}

int obs_scaled_add(obs_ctx* ctx, uint16_t* acc, const uint16_t* y, float scale, uint32_t n) {
  if (!ctx) return OBS_E_INVALID;
  if (!acc || !y) return obs::set_error(ctx, OBS_E_INVALID, "obs_scaled_add: null pointer");
  if (n == 0) return OBS_OK;
  if (n % 8u == 0 && obs::aligned(acc, 16) && obs::aligned(y, 16)) {
    const uint32_t n8 = n / 8u;
    OBS_LAUNCH(ctx, "scaled_add", scaled_add8_kernel<<<(n8 + 255) / 256, 256, 0, ctx->stream>>>(acc, y, scale, n8));
  } else {
    OBS_LAUNCH(ctx, "scaled_add", scaled_add_kernel<<<(n + 255) / 256, 256, 0, ctx->stream>>>(acc, y, scale, n));
  }
  return OBS_OK;
}

}  // extern "C"
