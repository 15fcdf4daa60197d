// obs_decode.hip — decode MoE half of one layer for one token
// (src/forward.rs:421-441): router -> per selected expert
// h = silu(gate . x) * (up . x) -> y_r = down . h -> y = sum_r w_r * y_r.
//
// The reference pages the 8 selected experts off SSD into a pool
// (disk_io.rs:79-102, forward.rs:431-435) and issues 5 dispatches per expert;
// here the whole expert table is resident in HBM (stacked [E, ...] tensors)
// and the layer runs as 4 launches: gate logits, top-k, gate/up+SwiGLU,
// down+combine. Weights are read exactly once with 16-byte coalesced loads.
//
// Numerics: dots accumulate in fp32 using the per-group factored form
//   sum_c (q_c*s + b) * x_c = s * sum_c q_c*x_c + b * sum_c x_c
// (exact algebra; it removes one multiply-add per weight). h stays fp32,
// the combine accumulates sum_r w_r*y_r in fp32 in rank order (forward.rs:440
// order) and rounds once to bf16.
#include "obs_internal.hpp"

namespace obs {
int check_router_shape(obs_ctx* ctx, const char* who, uint32_t in, uint32_t n_exp, uint32_t group);
int launch_route(obs_ctx* ctx, const uint32_t* w8, const uint16_t* s, const uint16_t* b, const uint16_t* x,
                 float* logits, int32_t* ids, float* w, uint32_t T, uint32_t in, uint32_t n_exp, uint32_t group,
                 uint32_t k, int norm_topk, int rule);
}  // namespace obs

namespace {

using namespace obsd;

constexpr int GU_ROWS_PER_WAVE = 2;
constexpr int GU_WAVES = 4;
constexpr int DN_ROWS_PER_WAVE = 2;
constexpr int DN_WAVES = 4;

// h[r, o] = silu(gate_e[o] . x) * (up_e[o] . x) for e = ids[r].
// One wave per (r, o) row pair; lane l owns the 8*WPL contiguous columns
// [l*8*WPL, (l+1)*8*WPL), which lie inside one quantization group.
template <int WPL>
__global__ void __launch_bounds__(GU_WAVES * 64) decode_gateup_kernel(
    const uint32_t* __restrict__ gw, const uint16_t* __restrict__ gs, const uint16_t* __restrict__ gb,
    const uint32_t* __restrict__ uw, const uint16_t* __restrict__ us, const uint16_t* __restrict__ ub,
    const uint16_t* __restrict__ x, const int32_t* __restrict__ ids, float* __restrict__ h,
    uint32_t n_exp, uint32_t k, uint32_t H, uint32_t I, uint32_t group) {
  constexpr int C = 8 * WPL;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = blockIdx.x * GU_WAVES + threadIdx.x / 64;
  // x chunk and its sum, once per wave
  float xf[C];
  const uint16_t* xr = x + lane * C;
#pragma unroll
  for (int c = 0; c < C; c += 8) {
    const uint4 v = *reinterpret_cast<const uint4*>(xr + c);
    xf[c + 0] = bf16lo(v.x); xf[c + 1] = bf16hi(v.x);
    xf[c + 2] = bf16lo(v.y); xf[c + 3] = bf16hi(v.y);
    xf[c + 4] = bf16lo(v.z); xf[c + 5] = bf16hi(v.z);
    xf[c + 6] = bf16lo(v.w); xf[c + 7] = bf16hi(v.w);
  }
  float xs = 0.0f;
#pragma unroll
  for (int c = 0; c < C; ++c) xs = xs + xf[c];
  const uint32_t words = H / 8, groups = H / group;
  const uint32_t g = (lane * C) / group;
#pragma unroll
  for (int rr = 0; rr < GU_ROWS_PER_WAVE; ++rr) {
    const uint32_t row = wave * GU_ROWS_PER_WAVE + rr;  // r * I + o
    if (row >= k * I) break;
    const uint32_t r = row / I, o = row % I;
    const int32_t e = ids[r];
    float hv = 0.0f;
    if (e >= 0 && static_cast<uint32_t>(e) < n_exp) {
      const uint64_t wrow = (static_cast<uint64_t>(e) * I + o);
      const uint32_t* gp = gw + wrow * words + lane * WPL;
      const uint32_t* up = uw + wrow * words + lane * WPL;
      uint32_t gq[WPL], uq[WPL];
      if constexpr (WPL % 4 == 0) {
#pragma unroll
        for (int j = 0; j < WPL; j += 4) {
          const uint4 a = *reinterpret_cast<const uint4*>(gp + j);
          const uint4 c = *reinterpret_cast<const uint4*>(up + j);
          gq[j] = a.x; gq[j + 1] = a.y; gq[j + 2] = a.z; gq[j + 3] = a.w;
          uq[j] = c.x; uq[j + 1] = c.y; uq[j + 2] = c.z; uq[j + 3] = c.w;
        }
      } else {
#pragma unroll
        for (int j = 0; j < WPL; j += 2) {
          const uint2 a = *reinterpret_cast<const uint2*>(gp + j);
          const uint2 c = *reinterpret_cast<const uint2*>(up + j);
          gq[j] = a.x; gq[j + 1] = a.y;
          uq[j] = c.x; uq[j + 1] = c.y;
        }
      }
      const uint64_t srow = wrow * groups + g;
      const float sg = bf16_to_f32(gs[srow]), bgv = bf16_to_f32(gb[srow]);
      const float su = bf16_to_f32(us[srow]), bu = bf16_to_f32(ub[srow]);
      float ag = 0.0f, au = 0.0f;
#pragma unroll
      for (int j = 0; j < WPL; ++j) {
        ag = dot8_q4(gq[j], xf + 8 * j, ag);
        au = dot8_q4(uq[j], xf + 8 * j, au);
      }
      float pg = __builtin_fmaf(sg, ag, bgv * xs);
      float pu = __builtin_fmaf(su, au, bu * xs);
      pg = wave_sum_asc(pg);
      pu = wave_sum_asc(pu);
      hv = silu_mul(pg, pu);
    }
    if (lane == 0) h[row] = hv;
  }
}

// y[o] = (residual[o]) + sum_r w_r * (down_{e_r}[o] . h_r), one wave per output
// row; lane l -> rank r = l/8 and column slice m = l%8 of CPL = I/8 columns.
template <int CPL>
__global__ void __launch_bounds__(DN_WAVES * 64) decode_down_kernel(
    const uint32_t* __restrict__ dw, const uint16_t* __restrict__ ds, const uint16_t* __restrict__ db,
    const float* __restrict__ h, const int32_t* __restrict__ ids, const float* __restrict__ wts,
    const uint16_t* __restrict__ residual, uint16_t* __restrict__ y, uint32_t n_exp, uint32_t k,
    uint32_t H, uint32_t I, uint32_t group) {
  constexpr int BLK = CPL / 32;  // 32-column blocks per lane (each inside one group)
  extern __shared__ float sh_h[];  // [k][I]
  {
    // stage h in batches of 8 independent 16-byte loads per thread (k*I % 4 == 0)
    const uint32_t n4 = (k * I) / 4;
    const float4* h4 = reinterpret_cast<const float4*>(h);
    float4* s4 = reinterpret_cast<float4*>(sh_h);
    for (uint32_t base = threadIdx.x; base < n4; base += 8 * blockDim.x) {
      float4 v[8];
#pragma unroll
      for (uint32_t u = 0; u < 8; ++u) {
        const uint32_t i = base + u * blockDim.x;
        if (i < n4) v[u] = h4[i];
      }
#pragma unroll
      for (uint32_t u = 0; u < 8; ++u) {
        const uint32_t i = base + u * blockDim.x;
        if (i < n4) s4[i] = v[u];
      }
    }
  }
  __syncthreads();
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t r = lane >> 3, m = lane & 7;
  const bool active_rank = r < k;
  int32_t e = active_rank ? ids[r] : -1;
  if (e >= static_cast<int32_t>(n_exp)) e = -1;
  const float wr = (active_rank && e >= 0) ? wts[r] : 0.0f;
  // this lane's h slice and per-block sums
  float hf[CPL];
  float hsum[BLK];
#pragma unroll
  for (int c = 0; c < CPL; ++c) hf[c] = (active_rank && e >= 0) ? sh_h[r * I + m * CPL + c] : 0.0f;
#pragma unroll
  for (int bl = 0; bl < BLK; ++bl) {
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < 32; ++c) s = s + hf[bl * 32 + c];
    hsum[bl] = s;
  }
  const uint32_t words = I / 8, groups = I / group;
  const uint32_t wave = blockIdx.x * DN_WAVES + threadIdx.x / 64;
#pragma unroll
  for (int rr = 0; rr < DN_ROWS_PER_WAVE; ++rr) {
    const uint32_t o = wave * DN_ROWS_PER_WAVE + rr;
    if (o >= H) break;
    float part = 0.0f;
    if (e >= 0) {
      const uint64_t wrow = static_cast<uint64_t>(e) * H + o;
      const uint32_t* wp = dw + wrow * words + m * (CPL / 8);
      const uint16_t* sp = ds + wrow * groups;
      const uint16_t* bp = db + wrow * groups;
#pragma unroll
      for (int bl = 0; bl < BLK; ++bl) {
        const uint4 q = *reinterpret_cast<const uint4*>(wp + 4 * bl);
        const uint32_t gi = (m * CPL + 32 * bl) / group;
        float a = 0.0f;
        a = dot8_q4(q.x, hf + 32 * bl + 0, a);
        a = dot8_q4(q.y, hf + 32 * bl + 8, a);
        a = dot8_q4(q.z, hf + 32 * bl + 16, a);
        a = dot8_q4(q.w, hf + 32 * bl + 24, a);
        part = part + __builtin_fmaf(bf16_to_f32(sp[gi]), a, bf16_to_f32(bp[gi]) * hsum[bl]);
      }
    }
    // reduce the 8 lanes of each rank
    part = part + __shfl_xor(part, 4, 64);
    part = part + __shfl_xor(part, 2, 64);
    part = part + __shfl_xor(part, 1, 64);
    // combine in rank order
    float acc = residual ? bf16_to_f32(residual[o]) : 0.0f;
    for (uint32_t rk = 0; rk < k; ++rk) {
      const float yr = __shfl(part, static_cast<int>(rk * 8), 64);
      const float wk = __shfl(wr, static_cast<int>(rk * 8), 64);
      acc = __builtin_fmaf(wk, yr, acc);
    }
    if (lane == 0) y[o] = f32_to_bf16(acc);
  }
}

constexpr size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

}  // namespace

namespace obs {

int check_moe_config(obs_ctx* ctx, const char* who, const obs_moe_config* cfg) {
  if (!cfg) return set_error(ctx, OBS_E_INVALID, "%s: null config", who);
  if (cfg->group != 64) return set_error(ctx, OBS_E_SHAPE, "%s: group must be 64 (got %u)", who, cfg->group);
  if (cfg->hidden != 1024 && cfg->hidden != 2048 && cfg->hidden != 4096)
    return set_error(ctx, OBS_E_SHAPE, "%s: hidden must be 1024, 2048 or 4096 (got %u)", who, cfg->hidden);
  if (cfg->inter == 0 || cfg->inter % 256 != 0 || cfg->inter > 2048)
    return set_error(ctx, OBS_E_SHAPE, "%s: inter must be a multiple of 256 in [256, 2048] (got %u)", who, cfg->inter);
  if (cfg->n_exp == 0 || cfg->n_exp > 256)
    return set_error(ctx, OBS_E_SHAPE, "%s: n_exp must be in [1, 256] (got %u)", who, cfg->n_exp);
  if (cfg->top_k == 0 || cfg->top_k > cfg->n_exp || cfg->top_k > 8)
    return set_error(ctx, OBS_E_SHAPE, "%s: top_k must be in [1, min(n_exp, 8)] (got %u)", who, cfg->top_k);
  if (cfg->route_rule != OBS_ROUTE_REF && cfg->route_rule != OBS_ROUTE_F32)
    return set_error(ctx, OBS_E_INVALID, "%s: unknown route_rule %d", who, cfg->route_rule);
  return OBS_OK;
}

int check_moe_layer(obs_ctx* ctx, const char* who, const obs_moe_layer* L) {
  if (!L) return set_error(ctx, OBS_E_INVALID, "%s: null layer", who);
  if (!L->gate_w || !L->gate_s || !L->gate_b || !L->up_w || !L->up_s || !L->up_b || !L->down_w ||
      !L->down_s || !L->down_b || !L->router_w || !L->router_s || !L->router_b)
    return set_error(ctx, OBS_E_INVALID, "%s: null weight pointer in layer", who);
  if (!aligned(L->gate_w, 16) || !aligned(L->up_w, 16) || !aligned(L->down_w, 16) || !aligned(L->router_w, 16))
    return set_error(ctx, OBS_E_ALIGN, "%s: packed weights must be 16-byte aligned", who);
  if (L->norm_w && !aligned(L->norm_w, 16))
    return set_error(ctx, OBS_E_ALIGN, "%s: norm_w must be 16-byte aligned", who);
  return OBS_OK;
}

int launch_decode_experts(obs_ctx* ctx, const obs_moe_config* cfg, const obs_moe_layer* L, const uint16_t* x,
                          const uint16_t* residual, uint16_t* y, const int32_t* ids, const float* w, float* h) {
  const uint32_t H = cfg->hidden, I = cfg->inter, k = cfg->top_k, E = cfg->n_exp, G = cfg->group;
  const uint32_t rows = k * I;
  const uint32_t gu_blocks = (rows + GU_WAVES * GU_ROWS_PER_WAVE - 1) / (GU_WAVES * GU_ROWS_PER_WAVE);
  switch (H) {
    case 1024:
      OBS_LAUNCH(ctx, "decode_gateup", decode_gateup_kernel<2><<<gu_blocks, GU_WAVES * 64, 0, ctx->stream>>>(L->gate_w, L->gate_s, L->gate_b, L->up_w, L->up_s, L->up_b, x, ids, h, E, k, H, I, G));
      break;
    case 2048:
      OBS_LAUNCH(ctx, "decode_gateup", decode_gateup_kernel<4><<<gu_blocks, GU_WAVES * 64, 0, ctx->stream>>>(L->gate_w, L->gate_s, L->gate_b, L->up_w, L->up_s, L->up_b, x, ids, h, E, k, H, I, G));
      break;
    default:
      OBS_LAUNCH(ctx, "decode_gateup", decode_gateup_kernel<8><<<gu_blocks, GU_WAVES * 64, 0, ctx->stream>>>(L->gate_w, L->gate_s, L->gate_b, L->up_w, L->up_s, L->up_b, x, ids, h, E, k, H, I, G));
      break;
  }
  const uint32_t dn_blocks = (H + DN_WAVES * DN_ROWS_PER_WAVE - 1) / (DN_WAVES * DN_ROWS_PER_WAVE);
  const size_t lds = sizeof(float) * k * I;
#define OBS_DOWN(CPL)                                                                                       \
  OBS_LAUNCH(ctx, "decode_down",                                                                            \
             decode_down_kernel<CPL><<<dn_blocks, DN_WAVES * 64, lds, ctx->stream>>>(L->down_w, L->down_s,  \
                                                                                     L->down_b, h, ids, w,  \
                                                                                     residual, y, E, k, H, I, G))
  switch (I / 8) {
    case 32: OBS_DOWN(32); break;
    case 64: OBS_DOWN(64); break;
    case 96: OBS_DOWN(96); break;
    case 128: OBS_DOWN(128); break;
    case 160: OBS_DOWN(160); break;
    case 192: OBS_DOWN(192); break;
    case 224: OBS_DOWN(224); break;
    default: OBS_DOWN(256); break;
  }
#undef OBS_DOWN
  return OBS_OK;
}

// Validates a decode call and picks its path (the one-launch fused kernel, or
// the 4 launches).
int decode_plan(obs_ctx* ctx, const char* who, const obs_moe_config* cfg, const obs_moe_layer* layer,
                const uint16_t* x, const uint16_t* y, bool* fused) {
  int rc = check_moe_config(ctx, who, cfg);
  if (rc) return rc;
  rc = check_moe_layer(ctx, who, layer);
  if (rc) return rc;
  if (!x || !y) return set_error(ctx, OBS_E_INVALID, "%s: null x or y", who);
  if (!aligned(x, 16)) return set_error(ctx, OBS_E_ALIGN, "%s: x must be 16-byte aligned", who);
  const bool shape_ok = fused_decode_supported(cfg);
  // the one-launch path spins on values other workgroups publish: all of its
  // workgroups must be resident at once, one per CU, and each group of 32 must
  // share an XCD (its L2) as the probe at obs_create found
  const bool cus_ok = (dispatch_gate(ctx->num_cus, ctx->xcd_map_ok, ctx->inorder_ok) & OBS_PATH_FUSED_DECODE) != 0u;
  if (ctx->decode_path == OBS_DECODE_FUSED && !shape_ok)
    return set_error(ctx, OBS_E_SHAPE, "%s: the fused path needs hidden 2048, inter 768, top_k 8, group 64, n_exp <= 256",
                     who);
  if (ctx->decode_path == OBS_DECODE_FUSED && !cus_ok)
    return set_error(ctx, OBS_E_UNSUPPORTED,
                     "%s: the fused path needs %u CUs with each group b %% 8 on one XCD (the device has %d CUs; XCD map %s)",
                     who, fused_decode_workgroups(), ctx->num_cus, ctx->xcd_map_ok ? "as expected" : "not as expected");
  *fused = shape_ok && cus_ok && ctx->decode_path != OBS_DECODE_MULTI;
  return OBS_OK;
}

// Workspace of the 4-launch path: logits [E] | ids [k] | w [k] | h [k, I] | normed x [H].
size_t multi_ws_bytes(const obs_moe_config* cfg) {
  return align256(sizeof(float) * cfg->n_exp) + align256(sizeof(int32_t) * cfg->top_k) +
         align256(sizeof(float) * cfg->top_k) + align256(sizeof(float) * cfg->top_k * cfg->inter) +
         align256(sizeof(uint16_t) * cfg->hidden);
}

// The 4-launch path over a workspace of multi_ws_bytes(cfg) at `base`.
int decode_multi(obs_ctx* ctx, const obs_moe_config* cfg, const obs_moe_layer* layer, const uint16_t* x,
                 const uint16_t* residual, uint16_t* y, int32_t* ids_out, float* w_out, char* base) {
  const uint32_t E = cfg->n_exp, k = cfg->top_k, H = cfg->hidden, I = cfg->inter;
  const size_t off_ids = align256(sizeof(float) * E);
  const size_t off_w = off_ids + align256(sizeof(int32_t) * k);
  const size_t off_h = off_w + align256(sizeof(float) * k);
  const size_t off_xn = off_h + align256(sizeof(float) * k * I);
  float* logits = reinterpret_cast<float*>(base);
  int32_t* ids = ids_out ? ids_out : reinterpret_cast<int32_t*>(base + off_ids);
  float* w = w_out ? w_out : reinterpret_cast<float*>(base + off_w);
  float* h = reinterpret_cast<float*>(base + off_h);
  int rc;
  if (layer->norm_w) {  // the router and experts see rmsnorm(x) (forward.rs:419-421)
    uint16_t* xn = reinterpret_cast<uint16_t*>(base + off_xn);
    rc = launch_rmsnorm(ctx, x, layer->norm_w, xn, 1, H, cfg->rms_eps);
    if (rc) return rc;
    x = xn;
  }
  rc = launch_route(ctx, layer->router_w, layer->router_s, layer->router_b, x, logits, ids, w, 1, H, E, cfg->group, k,
                    cfg->norm_topk, cfg->route_rule);
  if (rc) return rc;
  return launch_decode_experts(ctx, cfg, layer, x, residual, y, ids, w, h);
}

}  // namespace obs

extern "C" {

int obs_moe_decode(obs_ctx* ctx, const obs_moe_config* cfg, const obs_moe_layer* layer, const uint16_t* x,
                   const uint16_t* residual, uint16_t* y, int32_t* ids_out, float* w_out) {
  if (!ctx) return OBS_E_INVALID;
  bool fused = false;
  int rc = obs::decode_plan(ctx, "obs_moe_decode", cfg, layer, x, y, &fused);
  if (rc) return rc;
  if (fused) return obs::launch_fused_decode(ctx, cfg, layer, x, residual, y, ids_out, w_out);
  void* ws = nullptr;
  rc = obs::ensure_decode_ws(ctx, obs::multi_ws_bytes(cfg), &ws);
  if (rc) return rc;
  return obs::decode_multi(ctx, cfg, layer, x, residual, y, ids_out, w_out, static_cast<char*>(ws));
}

int obs_moe_decode_static(obs_ctx* ctx, const obs_moe_config* cfg, const obs_moe_layer* layer, const uint16_t* x,
                          const uint16_t* residual, uint16_t* y, int32_t* ids_out, float* w_out) {
  if (!ctx) return OBS_E_INVALID;
  bool fused = false;
  int rc = obs::decode_plan(ctx, "obs_moe_decode_static", cfg, layer, x, y, &fused);
  if (rc) return rc;
  if (!ctx->scratch)
    return obs::set_error(ctx, OBS_E_UNSUPPORTED, "obs_moe_decode_static: no static scratch on device %d",
                          ctx->device);
  const size_t need = obs::multi_ws_bytes(cfg);
  if (need > obs::STATIC_MULTI_BYTES)
    return obs::set_error(ctx, OBS_E_NOMEM,
                          "obs_moe_decode_static: the shape needs %zu bytes of scratch, the static array holds %zu",
                          need, obs::STATIC_MULTI_BYTES);
  ctx->scratch_used = true;
  char* base = static_cast<char*>(ctx->scratch);
  if (fused) return obs::launch_fused_decode_ws(ctx, cfg, layer, x, residual, y, ids_out, w_out, base);
  return obs::decode_multi(ctx, cfg, layer, x, residual, y, ids_out, w_out, base + obs::STATIC_FUSED_BYTES);
}

int obs_set_decode_path(obs_ctx* ctx, int path) {
  if (!ctx) return OBS_E_INVALID;
  if (path != OBS_DECODE_AUTO && path != OBS_DECODE_MULTI && path != OBS_DECODE_FUSED)
    return obs::set_error(ctx, OBS_E_INVALID, "obs_set_decode_path: unknown path %d", path);
  ctx->decode_path = path;
  return OBS_OK;
}

int obs_device_status(obs_ctx* ctx) {
  if (!ctx) return OBS_E_INVALID;
  const int a = obs::fused_decode_status(ctx);
  const int b = obs::attn_fused_status(ctx);
  const int c = ctx->scratch_used ? obs::fused_decode_status_ws(ctx, ctx->scratch) : OBS_OK;
  const int f = obs::ffn_status(ctx);
  const int l = obs::layer_fused_status(ctx);
  return a != OBS_OK ? a : b != OBS_OK ? b : c != OBS_OK ? c : f != OBS_OK ? f : l;
}

}  // extern "C"
