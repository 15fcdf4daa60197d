// obs_router.hip — MoE router: 8-bit gate logits and softmax/top-k.
//
// Replaces Model::gate_gpu (src/forward.rs:386-397) + dequant_matvec_8bit.metal
// and MoeRouter::route/route_dispatch (src/router.rs:25-83) + moe_routing_topk.metal.
//
// Logit reduction order (documented, reproduced by the CPU oracle): for each
// (token, expert row) one wave of 64 lanes; lane l owns the in/64 contiguous
// columns [l*in/64, (l+1)*in/64) and accumulates acc = fma(w_c, x_c, acc) in
// column order from 0; the lanes are combined by an xor butterfly with
// offsets 32, 16, 8, 4, 2, 1.
//
// Selection (moe_routing_topk.metal:31-56): m = max logit; e_i = exp(l_i - m)
// with the deterministic exp; S = sum e_i where lane l adds e_l, e_{l+64},
// e_{l+128}, e_{l+192} in that order and the lanes are combined by the xor
// butterfly; p_i = e_i / S; k rounds of argmax over p (lower id wins ties);
// wsum = serial sum of the selected p; if norm_topk and wsum > 0 the weights
// are p / wsum. All steps are correctly rounded fp32 operations, so the ids
// and weights are bit-identical to the oracle given the same logits.
#include "obs_internal.hpp"

namespace {

using namespace obsd;

constexpr int ROUTER_TOKENS_PER_WAVE = 8;

// grid: x = ceil(n_exp / 4) (4 waves per block, one expert row each),
//       y = ceil(T / ROUTER_TOKENS_PER_WAVE)
// WPL = packed words per lane (in = 64 lanes * 4 cols * WPL).
template <int WPL>
__global__ void __launch_bounds__(256) q8_gate_logits_kernel(const uint32_t* __restrict__ w8,
                                                             const uint16_t* __restrict__ s,
                                                             const uint16_t* __restrict__ b,
                                                             const uint16_t* __restrict__ x,
                                                             float* __restrict__ logits, uint32_t T,
                                                             uint32_t in, uint32_t n_exp,
                                                             uint32_t group) {
  constexpr int C = 4 * WPL;  // columns per lane
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t e = blockIdx.x * 4 + threadIdx.x / 64;
  if (e >= n_exp) return;
  const uint32_t words = in / 4, groups = in / group;
  const uint32_t* wr = w8 + static_cast<uint64_t>(e) * words + lane * WPL;
  const uint16_t* sr = s + static_cast<uint64_t>(e) * groups;
  const uint16_t* br = b + static_cast<uint64_t>(e) * groups;
  // dequantize this lane's C weights once (exact: byte*scale has <= 16 bits)
  float wv[C];
#pragma unroll
  for (int j = 0; j < WPL; ++j) {
    const uint32_t word = wr[j];
    const uint32_t g = (lane * C + 4 * j) / group;
    const float sc = bf16_to_f32(sr[g]), bi = bf16_to_f32(br[g]);
#pragma unroll
    for (int q = 0; q < 4; ++q) wv[4 * j + q] = __builtin_fmaf(static_cast<float>((word >> (8 * q)) & 0xffu), sc, bi);
  }
  const uint32_t t0 = blockIdx.y * ROUTER_TOKENS_PER_WAVE;
  for (uint32_t t = t0; t < t0 + ROUTER_TOKENS_PER_WAVE && t < T; ++t) {
    const uint16_t* xr = x + static_cast<uint64_t>(t) * in + lane * C;
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < C; c += 8) {
      const uint4 xv = *reinterpret_cast<const uint4*>(xr + c);
      acc = __builtin_fmaf(wv[c + 0], bf16lo(xv.x), acc);
      acc = __builtin_fmaf(wv[c + 1], bf16hi(xv.x), acc);
      acc = __builtin_fmaf(wv[c + 2], bf16lo(xv.y), acc);
      acc = __builtin_fmaf(wv[c + 3], bf16hi(xv.y), acc);
      acc = __builtin_fmaf(wv[c + 4], bf16lo(xv.z), acc);
      acc = __builtin_fmaf(wv[c + 5], bf16hi(xv.z), acc);
      acc = __builtin_fmaf(wv[c + 6], bf16lo(xv.w), acc);
      acc = __builtin_fmaf(wv[c + 7], bf16hi(xv.w), acc);
    }
    acc = wave_sum_xor(acc);
    if (lane == 0) logits[static_cast<uint64_t>(t) * n_exp + e] = acc;
  }
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const unsigned long long o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// One wave per token; n_exp <= 256, k <= 64. Result written by lanes 0..k-1.
__device__ __forceinline__ void route_one_wave(const float* __restrict__ lg, uint32_t n_exp, uint32_t k,
                                               int norm_topk, uint32_t lane, int32_t* my_id, float* my_w) {
  float l[4], e[4];
  int key[4];
  float m = -__builtin_huge_valf();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t i = lane + 64u * j;
    l[j] = i < n_exp ? lg[i] : 0.0f;
    if (i < n_exp) m = __builtin_fmaxf(m, l[j]);
  }
  m = wave_max_f32(m);
  float a = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t i = lane + 64u * j;
    e[j] = 0.0f;
    if (i < n_exp) {
      e[j] = exp_det(l[j] - m);
      a = a + e[j];
    }
  }
  const float S = wave_sum_xor(a);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t i = lane + 64u * j;
    if (i < n_exp) {
      const float p = e[j] / S;
      key[j] = (p != p) ? -2 : __float_as_int(p);
    } else {
      key[j] = -1;
    }
  }
  float wsum = 0.0f;
  int32_t sel_id = -1;
  float sel_p = 0.0f;
  for (uint32_t kk = 0; kk < k; ++kk) {
    // lane-local best: first maximum over j (ids increase with j)
    int bk = key[0];
    uint32_t bi = lane;
#pragma unroll
    for (int j = 1; j < 4; ++j)
      if (key[j] > bk) { bk = key[j]; bi = lane + 64u * j; }
    const unsigned long long packed =
        (static_cast<unsigned long long>(static_cast<uint32_t>(bk + 2)) << 32) | static_cast<uint32_t>(~bi);
    const unsigned long long best = wave_max_u64(packed);
    const int bkey = static_cast<int>(static_cast<uint32_t>(best >> 32)) - 2;
    const uint32_t bidx = ~static_cast<uint32_t>(best & 0xffffffffull);
    if (bkey < 0) continue;  // nothing selectable: slot keeps id -1, weight 0
    const float p = __int_as_float(bkey);
    if (lane == kk) { sel_id = static_cast<int32_t>(bidx); sel_p = p; }
    wsum = wsum + p;
    if ((bidx & 63u) == lane) key[bidx >> 6] = -1;
  }
  float wout = sel_p;
  if (norm_topk && wsum > 0.0f && sel_id >= 0) wout = sel_p / wsum;
  *my_id = sel_id;
  *my_w = sel_id >= 0 ? wout : 0.0f;
}

__global__ void __launch_bounds__(256) route_topk_kernel(const float* __restrict__ logits, int32_t* __restrict__ ids,
                                                         float* __restrict__ weights, uint32_t T, uint32_t n_exp,
                                                         uint32_t k, int norm_topk) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t t = blockIdx.x * 4 + threadIdx.x / 64;
  if (t >= T) return;
  int32_t id;
  float w;
  route_one_wave(logits + static_cast<uint64_t>(t) * n_exp, n_exp, k, norm_topk, lane, &id, &w);
  if (lane < k) {
    ids[static_cast<uint64_t>(t) * k + lane] = id;
    weights[static_cast<uint64_t>(t) * k + lane] = w;
  }
}

}  // namespace

namespace obs {

int check_router_shape(obs_ctx* ctx, const char* who, uint32_t in, uint32_t n_exp, uint32_t group) {
  if (n_exp == 0 || n_exp > 256)
    return set_error(ctx, OBS_E_SHAPE, "%s: n_exp must be in [1, 256] (got %u)", who, n_exp);
  if (group == 0 || group % 4 != 0 || in % group != 0)
    return set_error(ctx, OBS_E_SHAPE, "%s: in (%u) must be a multiple of group (%u), group a multiple of 4", who, in, group);
  if (in != 512 && in != 1024 && in != 2048 && in != 4096)
    return set_error(ctx, OBS_E_SHAPE, "%s: in must be 512, 1024, 2048 or 4096 (got %u)", who, in);
  // a lane's contiguous span must not straddle groups in a way the per-word
  // scale lookup cannot express: 4 | group makes every word single-group.
  return OBS_OK;
}

int launch_gate_logits(obs_ctx* ctx, const uint32_t* w8, const uint16_t* s, const uint16_t* b,
                       const uint16_t* x, float* logits, uint32_t T, uint32_t in, uint32_t n_exp,
                       uint32_t group) {
  dim3 grid((n_exp + 3) / 4, (T + ROUTER_TOKENS_PER_WAVE - 1) / ROUTER_TOKENS_PER_WAVE);
  switch (in) {
    case 512: OBS_LAUNCH(ctx, "q8_gate_logits", q8_gate_logits_kernel<2><<<grid, 256, 0, ctx->stream>>>(w8, s, b, x, logits, T, in, n_exp, group)); break;
    case 1024: OBS_LAUNCH(ctx, "q8_gate_logits", q8_gate_logits_kernel<4><<<grid, 256, 0, ctx->stream>>>(w8, s, b, x, logits, T, in, n_exp, group)); break;
    case 2048: OBS_LAUNCH(ctx, "q8_gate_logits", q8_gate_logits_kernel<8><<<grid, 256, 0, ctx->stream>>>(w8, s, b, x, logits, T, in, n_exp, group)); break;
    default: OBS_LAUNCH(ctx, "q8_gate_logits", q8_gate_logits_kernel<16><<<grid, 256, 0, ctx->stream>>>(w8, s, b, x, logits, T, in, n_exp, group)); break;
  }
  return OBS_OK;
}

int launch_route_topk(obs_ctx* ctx, const float* logits, int32_t* ids, float* w, uint32_t T,
                      uint32_t n_exp, uint32_t k, int norm_topk) {
  OBS_LAUNCH(ctx, "route_topk", route_topk_kernel<<<(T + 3) / 4, 256, 0, ctx->stream>>>(logits, ids, w, T, n_exp, k, norm_topk));
  return OBS_OK;
}

}  // namespace obs

extern "C" {

int obs_q8_gate_logits(obs_ctx* ctx, const uint32_t* w8, const uint16_t* scales, const uint16_t* biases,
                       const uint16_t* x, float* logits, uint32_t T, uint32_t in, uint32_t n_exp,
                       uint32_t group) {
  if (!ctx) return OBS_E_INVALID;
  if (!w8 || !scales || !biases || !x || !logits)
    return obs::set_error(ctx, OBS_E_INVALID, "obs_q8_gate_logits: null pointer");
  int rc = obs::check_router_shape(ctx, "obs_q8_gate_logits", in, n_exp, group);
  if (rc) return rc;
  if (!obs::aligned(x, 16) || !obs::aligned(w8, 16))
    return obs::set_error(ctx, OBS_E_ALIGN, "obs_q8_gate_logits: x and w8 must be 16-byte aligned");
  if (T == 0) return OBS_OK;
  return obs::launch_gate_logits(ctx, w8, scales, biases, x, logits, T, in, n_exp, group);
}

int obs_route_topk(obs_ctx* ctx, const float* logits, int32_t* ids, float* weights, uint32_t T,
                   uint32_t n_exp, uint32_t k, int norm_topk) {
  if (!ctx) return OBS_E_INVALID;
  if (!logits || !ids || !weights) return obs::set_error(ctx, OBS_E_INVALID, "obs_route_topk: null pointer");
  if (n_exp == 0 || n_exp > 256)
    return obs::set_error(ctx, OBS_E_SHAPE, "obs_route_topk: n_exp must be in [1, 256] (got %u)", n_exp);
  if (k == 0 || k > n_exp || k > 64)
    return obs::set_error(ctx, OBS_E_SHAPE, "obs_route_topk: k must be in [1, min(n_exp, 64)] (got %u)", k);
  if (T == 0) return OBS_OK;
  return obs::launch_route_topk(ctx, logits, ids, weights, T, n_exp, k, norm_topk);
}

}  // extern "C"
