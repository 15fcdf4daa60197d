// obs_router.hip — MoE router: 8-bit gate logits and softmax/top-k.
//
// Replaces Model::gate_gpu (src/forward.rs:386-397) + dequant_matvec_8bit.metal
// and MoeRouter::route/route_dispatch (src/router.rs:25-83) + moe_routing_topk.metal.
//
// Logit reduction order (documented, reproduced by the CPU oracle): for each
// (token, expert row) one wave of 64 lanes; lane l owns the in/64 contiguous
// columns [l*in/64, (l+1)*in/64) and accumulates acc = fma(w_c, x_c, acc) in
// column order from 0; the lanes are combined by an xor butterfly with
// offsets 1, 2, 4, ..., 32 (wave_sum_asc in the decode kernels;
// q8_gate_logits_kernel below adds the same pairs in LDS).
//
// Selection (moe_routing_topk.metal:24-56): under the reference rule each
// logit is first rounded to f16 (dequant_matvec_8bit.metal:30 stores halves);
// m = max logit; e_i = exp(l_i - m)
// with the deterministic exp; S = sum e_i where lane l adds e_l, e_{l+64},
// e_{l+128}, e_{l+192} in that order and the lanes are combined by the xor
// butterfly; p_i = e_i / S; k rounds of argmax over p (lower id wins ties);
// wsum = serial sum of the selected p; if norm_topk and wsum > 0 the weights
// are p / wsum (under the reference rule f16(p) and f16(f16(p) / wsum)). All
// steps are correctly rounded operations, so the ids and weights are
// bit-identical to the oracle given the same logits.
#include "obs_internal.hpp"

#include <algorithm>

namespace {

using namespace obsd;

constexpr int ROUTER_TOKENS_PER_WAVE = 8;

// grid: x = ceil(n_exp / (4 EPW)) (4 waves per block, EPW expert rows each),
//       y = ceil(T / (ROUTER_TOKENS_PER_WAVE * nch)): a workgroup keeps its rows
//       dequantized in registers and runs nch chunks of 8 tokens in turn
// WPL = packed words per lane (in = 64 lanes * 4 cols * WPL). A wave keeps its
// EPW rows dequantized in registers; the workgroup stages each chunk's 8
// activation rows in LDS once for its 4 waves. Several chunks per workgroup
// (when T leaves more than 64 chunks) dequantize the rows once for all of
// them: 40 -> 33 us per layer at T = 2,048. With one row per wave and no
// staging every activation row was read from L2 once per expert (1 GB at
// T = 2048), which bounded the launch. Each lane's partial sum of every
// (token, row) pair goes to LDS, and one thread per pair adds the 64 partials
// in the butterfly's order: a wave reduction per pair (DPP steps and lane
// reads, ~20 dependent instructions) had cost as much as the pair's fmas.
// The routing step of the one-launch router (obs_route): where the range's
// ids and weights go, and the per-range counters that elect the workgroup
// that routes (context memory, zero between launches).
struct RouteTail {
  uint32_t* cnt;
  int32_t* ids;
  float* weights;
  uint32_t k;
  int norm_topk, rule;
};

// FUSED: the one-launch router for one token range (T <= 8). The grid is 8
// times the workgroups the logits need, and only those with blockIdx.x % 8 == 0
// work: the dispatcher deals workgroups round-robin over the 8 XCDs, so they
// all run on one XCD and the logits pass through its L2 (plain stores, polled
// past the CU's vector cache), as the fused decode's exchanges do. Each working
// workgroup counts itself in cnt[0] once its logits are stored, and the last
// to do so resets the counter and routes the range's tokens (route_topk_
// kernel's per-token wave). NQ: logit slots per lane when routing.
template <int WPL, int EPW, bool FUSED, int NQ>
__global__ void __launch_bounds__(256) q8_gate_logits_kernel(const uint32_t* __restrict__ w8,
                                                             const uint16_t* __restrict__ s,
                                                             const uint16_t* __restrict__ b,
                                                             const uint16_t* __restrict__ x,
                                                             float* __restrict__ logits, uint32_t T,
                                                             uint32_t in, uint32_t n_exp,
                                                             uint32_t group, uint32_t nch, RouteTail rt) {
  constexpr int C = 4 * WPL;  // columns per lane
  // lane partials, 68 floats per pair: a thread's 16-byte reads of its pair hit
  // distinct banks across 16 consecutive threads
  constexpr uint32_t PART_STRIDE = 68;
  __shared__ __attribute__((aligned(16))) float s_part[ROUTER_TOKENS_PER_WAVE * 4 * EPW * PART_STRIDE];
  extern __shared__ __attribute__((aligned(16))) uint16_t s_x[];  // [ROUTER_TOKENS_PER_WAVE][in]
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = threadIdx.x / 64u;
  if (FUSED && blockIdx.x % 8u != 0u) return;  // uniform: the working workgroups are on XCD 0
  const uint32_t bx = FUSED ? blockIdx.x / 8u : blockIdx.x;
  const uint32_t e0 = (bx * 4 + wave) * EPW;
  const uint32_t words = in / 4, groups = in / group;
  // dequantize this lane's C weights of each row once (exact: byte*scale has <= 16 bits)
  float wv[EPW][C];
#pragma unroll
  for (int r = 0; r < EPW; ++r) {
    const uint32_t e = min(e0 + r, n_exp - 1u);  // rows past the last expert: computed, not stored
    const uint32_t* wr = w8 + static_cast<uint64_t>(e) * words + lane * WPL;
    const uint16_t* sr = s + static_cast<uint64_t>(e) * groups;
    const uint16_t* br = b + static_cast<uint64_t>(e) * groups;
#pragma unroll
    for (int j = 0; j < WPL; ++j) {
      const uint32_t word = wr[j];
      const uint32_t g = (lane * C + 4 * j) / group;
      const float sc = bf16_to_f32(sr[g]), bi = bf16_to_f32(br[g]);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        wv[r][4 * j + q] = __builtin_fmaf(static_cast<float>((word >> (8 * q)) & 0xffu), sc, bi);
    }
  }
  for (uint32_t ci = 0; ci < nch; ++ci) {
    const uint32_t t0 = (blockIdx.y * nch + ci) * ROUTER_TOKENS_PER_WAVE;
    if (t0 >= T) break;  // uniform per workgroup
    const uint32_t nt = min(static_cast<uint32_t>(ROUTER_TOKENS_PER_WAVE), T - t0);
    if (ci > 0) __syncthreads();  // the previous chunk's activations and partials are read
    {
      // (the next chunk's rows loaded into registers during this chunk measured
      // slower: 41 against 33 us per layer at 2,048 tokens)
      const uint32_t row_chunks = in / 8u;  // 16-byte chunks per activation row
      for (uint32_t c = threadIdx.x; c < nt * row_chunks; c += 256u)
        *reinterpret_cast<uint4*>(s_x + 8u * c) =
            *reinterpret_cast<const uint4*>(x + static_cast<uint64_t>(t0 + c / row_chunks) * in + 8u * (c % row_chunks));
    }
    __syncthreads();
    // the lane partials (serial fma over the lane's columns) of every (token, row)
    // pair go to LDS, pair-major
    if (e0 < n_exp) {  // wave-uniform
      for (uint32_t t = 0; t < nt; ++t) {
        const uint16_t* xr = s_x + t * in + lane * C;
        float xf[C];
#pragma unroll
        for (int c = 0; c < C; c += 8) {
          const uint4 xv = *reinterpret_cast<const uint4*>(xr + c);
          xf[c + 0] = bf16lo(xv.x); xf[c + 1] = bf16hi(xv.x); xf[c + 2] = bf16lo(xv.y); xf[c + 3] = bf16hi(xv.y);
          xf[c + 4] = bf16lo(xv.z); xf[c + 5] = bf16hi(xv.z); xf[c + 6] = bf16lo(xv.w); xf[c + 7] = bf16hi(xv.w);
        }
#pragma unroll
        for (int r = 0; r < EPW; ++r) {
          float acc = 0.0f;
#pragma unroll
          for (int c = 0; c < C; ++c) acc = __builtin_fmaf(wv[r][c], xf[c], acc);
          s_part[((t * 4u + wave) * EPW + r) * PART_STRIDE + lane] = acc;
        }
      }
    }
    __syncthreads();
    // one thread per pair: its 64 lane partials summed in the xor-butterfly order
    // (at step off, lane l adds lane l ^ off; lane 0's value is the sum over
    // aligned blocks, pairwise in index order), as wave_sum_asc does in registers
    const uint32_t pairs = nt * 4u * EPW;
    for (uint32_t pr = threadIdx.x; pr < pairs; pr += 256u) {
      const uint32_t r = pr % EPW, w = (pr / EPW) % 4u, t = pr / (4u * EPW);
      const uint32_t e = (bx * 4 + w) * EPW + r;
      float v[64];
      const float4* src = reinterpret_cast<const float4*>(s_part + pr * PART_STRIDE);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float4 q = src[i];
        v[4 * i] = q.x; v[4 * i + 1] = q.y; v[4 * i + 2] = q.z; v[4 * i + 3] = q.w;
      }
#pragma unroll
      for (int off = 1; off < 64; off *= 2)
#pragma unroll
        for (int l = 0; l < 64; l += 2 * off) v[l] = v[l] + v[l + off];
      float* dst = logits + static_cast<uint64_t>(t0 + t) * n_exp + e;
      if (e < n_exp) {
        if (FUSED)  // to the XCD's L2, where the routing workgroup reads it
          __hip_atomic_store(reinterpret_cast<uint32_t*>(dst), __float_as_uint(v[0]), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_WAVEFRONT);
        else
          *dst = v[0];
      }
    }
  }
  if constexpr (FUSED) {
    // A thread's logit stores have reached the L2 once its memory counter is 0,
    // before the workgroup counts itself; the routing workgroup's loads
    // follow the count it read and skip its CU's vector cache.
    __shared__ uint32_t s_last;
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t before = __hip_atomic_fetch_add(rt.cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = before + 1u == gridDim.x / 8u ? 1u : 0u;
      if (s_last) __hip_atomic_store(rt.cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (s_last == 0u) return;  // uniform per workgroup
    const uint32_t ta = 0u, tb = T;  // one range: T <= 8
    for (uint32_t t = ta + wave; t < tb; t += 4u) {  // uniform per wave
      const uint32_t* lg = reinterpret_cast<const uint32_t*>(logits + static_cast<uint64_t>(t) * n_exp);
      float l[NQ];
#pragma unroll
      for (int j = 0; j < NQ; ++j)
        l[j] = __uint_as_float(__hip_atomic_load(lg + min(lane + 64u * j, n_exp - 1u), __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT));
      int32_t id;
      float w;
      if (rt.k == 8)
        route_wave_top8<NQ>(l, n_exp, rt.norm_topk, rt.rule, lane, &id, &w);
      else
        route_wave<NQ>(l, n_exp, rt.k, rt.norm_topk, rt.rule, lane, &id, &w);
      if (lane < rt.k) {
        rt.ids[static_cast<uint64_t>(t) * rt.k + lane] = id;
        rt.weights[static_cast<uint64_t>(t) * rt.k + lane] = w;
      }
    }
  }
}

// One wave per token (route_wave); n_exp <= 64 * NQ, k <= 64.
template <int NQ>
__global__ void __launch_bounds__(256) route_topk_kernel(const float* __restrict__ logits, int32_t* __restrict__ ids,
                                                         float* __restrict__ weights, uint32_t T, uint32_t n_exp,
                                                         uint32_t k, int norm_topk, int rule) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t t = blockIdx.x * 4 + threadIdx.x / 64;
  if (t >= T) return;  // wave-uniform: every lane of a wave shares t
  const float* lg = logits + static_cast<uint64_t>(t) * n_exp;
  float l[NQ];
#pragma unroll
  for (int j = 0; j < NQ; ++j) l[j] = lg[min(lane + 64u * j, n_exp - 1u)];
  int32_t id;
  float w;
  if (k == 8)
    route_wave_top8<NQ>(l, n_exp, norm_topk, rule, lane, &id, &w);
  else
    route_wave<NQ>(l, n_exp, k, norm_topk, rule, lane, &id, &w);
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

// A launch of q8_gate_logits_kernel: 4 rows per wave (2 at in = 4096, whose
// rows hold 64 columns per lane; 1 when T is at most 64 tokens, so that the
// rows are spread over more CUs). A workgroup runs nch chunks of 8 tokens with
// its rows dequantized once, nch chosen to keep about 64 token ranges (512
// workgroups at 128 experts).
int launch_gate_logits(obs_ctx* ctx, const uint32_t* w8, const uint16_t* s, const uint16_t* b,
                       const uint16_t* x, float* logits, uint32_t T, uint32_t in, uint32_t n_exp,
                       uint32_t group) {
  const uint32_t chunks = (T + ROUTER_TOKENS_PER_WAVE - 1) / ROUTER_TOKENS_PER_WAVE;
  const uint32_t nch = std::min(8u, std::max(1u, chunks / 64u));
  const uint32_t ty = (chunks + nch - 1) / nch;
  const bool few = chunks <= 8u;
  const dim3 grid1((n_exp + 3) / 4, ty), grid4((n_exp + 15) / 16, ty), grid2((n_exp + 7) / 8, ty);
  const size_t lds = sizeof(uint16_t) * ROUTER_TOKENS_PER_WAVE * in;  // 64 KB at in = 4096
  const RouteTail none{};
#define OBS_LOGITS(WPL, EPW, GRID)                                                                    \
  OBS_LAUNCH(ctx, "q8_gate_logits", (q8_gate_logits_kernel<WPL, EPW, false, 1><<<GRID, 256, lds, ctx->stream>>>( \
                                        w8, s, b, x, logits, T, in, n_exp, group, nch, none)))
  switch (in) {
    case 512: if (few) OBS_LOGITS(2, 1, grid1); else OBS_LOGITS(2, 4, grid4); break;
    case 1024: if (few) OBS_LOGITS(4, 1, grid1); else OBS_LOGITS(4, 4, grid4); break;
    case 2048: if (few) OBS_LOGITS(8, 1, grid1); else OBS_LOGITS(8, 4, grid4); break;
    default: if (few) OBS_LOGITS(16, 1, grid1); else OBS_LOGITS(16, 2, grid2); break;
  }
#undef OBS_LOGITS
  return OBS_OK;
}

int launch_route_topk(obs_ctx* ctx, const float* logits, int32_t* ids, float* w, uint32_t T,
                      uint32_t n_exp, uint32_t k, int norm_topk, int rule) {
  if (n_exp <= 64)
    OBS_LAUNCH(ctx, "route_topk", route_topk_kernel<1><<<(T + 3) / 4, 256, 0, ctx->stream>>>(logits, ids, w, T, n_exp, k, norm_topk, rule));
  else if (n_exp <= 128)
    OBS_LAUNCH(ctx, "route_topk", route_topk_kernel<2><<<(T + 3) / 4, 256, 0, ctx->stream>>>(logits, ids, w, T, n_exp, k, norm_topk, rule));
  else
    OBS_LAUNCH(ctx, "route_topk", route_topk_kernel<4><<<(T + 3) / 4, 256, 0, ctx->stream>>>(logits, ids, w, T, n_exp, k, norm_topk, rule));
  return OBS_OK;
}

// The router step (logits, then routing). One launch for up to 8 tokens on a
// device whose workgroups b share an XCD by b % 8 (the exchange stays in one
// L2); otherwise the two launches.
template <int NQ>
int launch_route_fused(obs_ctx* ctx, const uint32_t* w8, const uint16_t* s, const uint16_t* b, const uint16_t* x,
                       float* logits, uint32_t T, uint32_t in, uint32_t n_exp, uint32_t group, const RouteTail& rt) {
  const dim3 grid(8u * ((n_exp + 3) / 4), 1);
  const size_t lds = sizeof(uint16_t) * ROUTER_TOKENS_PER_WAVE * in;
#define OBS_ROUTE1(WPL)                                                                                 \
  OBS_LAUNCH(ctx, "route_fused", (q8_gate_logits_kernel<WPL, 1, true, NQ><<<grid, 256, lds, ctx->stream>>>( \
                                     w8, s, b, x, logits, T, in, n_exp, group, 1u, rt)))
  switch (in) {
    case 512: OBS_ROUTE1(2); break;
    case 1024: OBS_ROUTE1(4); break;
    case 2048: OBS_ROUTE1(8); break;
    default: OBS_ROUTE1(16); break;
  }
#undef OBS_ROUTE1
  return OBS_OK;
}

int launch_route(obs_ctx* ctx, const uint32_t* w8, const uint16_t* s, const uint16_t* b, const uint16_t* x,
                 float* logits, int32_t* ids, float* w, uint32_t T, uint32_t in, uint32_t n_exp, uint32_t group,
                 uint32_t k, int norm_topk, int rule) {
  if (T <= static_cast<uint32_t>(ROUTER_TOKENS_PER_WAVE) && ctx->xcd_map_ok) {
    const RouteTail rt{ctx->route_cnt, ids, w, k, norm_topk, rule};
    if (n_exp <= 64) return launch_route_fused<1>(ctx, w8, s, b, x, logits, T, in, n_exp, group, rt);
    if (n_exp <= 128) return launch_route_fused<2>(ctx, w8, s, b, x, logits, T, in, n_exp, group, rt);
    return launch_route_fused<4>(ctx, w8, s, b, x, logits, T, in, n_exp, group, rt);
  }
  const int rc = launch_gate_logits(ctx, w8, s, b, x, logits, T, in, n_exp, group);
  if (rc) return rc;
  return launch_route_topk(ctx, logits, ids, w, T, n_exp, k, norm_topk, rule);
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

int obs_route(obs_ctx* ctx, const uint32_t* w8, const uint16_t* scales, const uint16_t* biases, const uint16_t* x,
              float* logits, int32_t* ids, float* weights, uint32_t T, uint32_t in, uint32_t n_exp, uint32_t group,
              uint32_t k, int norm_topk, int rule) {
  if (!ctx) return OBS_E_INVALID;
  if (!w8 || !scales || !biases || !x || !logits || !ids || !weights)
    return obs::set_error(ctx, OBS_E_INVALID, "obs_route: null pointer");
  int rc = obs::check_router_shape(ctx, "obs_route", in, n_exp, group);
  if (rc) return rc;
  if (k == 0 || k > n_exp || k > 64)
    return obs::set_error(ctx, OBS_E_SHAPE, "obs_route: k must be in [1, min(n_exp, 64)] (got %u)", k);
  if (rule != OBS_ROUTE_REF && rule != OBS_ROUTE_F32)
    return obs::set_error(ctx, OBS_E_INVALID, "obs_route: unknown rule %d", rule);
  if (!obs::aligned(x, 16) || !obs::aligned(w8, 16))
    return obs::set_error(ctx, OBS_E_ALIGN, "obs_route: x and w8 must be 16-byte aligned");
  if (T == 0) return OBS_OK;
  return obs::launch_route(ctx, w8, scales, biases, x, logits, ids, weights, T, in, n_exp, group, k, norm_topk, rule);
}

int obs_route_topk(obs_ctx* ctx, const float* logits, int32_t* ids, float* weights, uint32_t T,
                   uint32_t n_exp, uint32_t k, int norm_topk, int rule) {
  if (!ctx) return OBS_E_INVALID;
  if (!logits || !ids || !weights) return obs::set_error(ctx, OBS_E_INVALID, "obs_route_topk: null pointer");
  if (n_exp == 0 || n_exp > 256)
    return obs::set_error(ctx, OBS_E_SHAPE, "obs_route_topk: n_exp must be in [1, 256] (got %u)", n_exp);
  if (k == 0 || k > n_exp || k > 64)
    return obs::set_error(ctx, OBS_E_SHAPE, "obs_route_topk: k must be in [1, min(n_exp, 64)] (got %u)", k);
  if (rule != OBS_ROUTE_REF && rule != OBS_ROUTE_F32)
    return obs::set_error(ctx, OBS_E_INVALID, "obs_route_topk: unknown rule %d", rule);
  if (T == 0) return OBS_OK;
  return obs::launch_route_topk(ctx, logits, ids, weights, T, n_exp, k, norm_topk, rule);
}

}  // extern "C"
