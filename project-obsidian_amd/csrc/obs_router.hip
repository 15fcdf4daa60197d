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
template <int WPL, int EPW>
__global__ void __launch_bounds__(256) q8_gate_logits_kernel(const uint32_t* __restrict__ w8,
                                                             const uint16_t* __restrict__ s,
                                                             const uint16_t* __restrict__ b,
                                                             const uint16_t* __restrict__ x,
                                                             float* __restrict__ logits, uint32_t T,
                                                             uint32_t in, uint32_t n_exp,
                                                             uint32_t group, uint32_t nch) {
  constexpr int C = 4 * WPL;  // columns per lane
  // lane partials, 68 floats per pair: a thread's 16-byte reads of its pair hit
  // distinct banks across 16 consecutive threads
  constexpr uint32_t PART_STRIDE = 68;
  __shared__ __attribute__((aligned(16))) float s_part[ROUTER_TOKENS_PER_WAVE * 4 * EPW * PART_STRIDE];
  extern __shared__ __attribute__((aligned(16))) uint16_t s_x[];  // [ROUTER_TOKENS_PER_WAVE][in]
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = threadIdx.x / 64u;
  const uint32_t e0 = (blockIdx.x * 4 + wave) * EPW;
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
      const uint32_t e = (blockIdx.x * 4 + w) * EPW + r;
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
      if (e < n_exp) logits[static_cast<uint64_t>(t0 + t) * n_exp + e] = v[0];
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

int launch_gate_logits(obs_ctx* ctx, const uint32_t* w8, const uint16_t* s, const uint16_t* b,
                       const uint16_t* x, float* logits, uint32_t T, uint32_t in, uint32_t n_exp,
                       uint32_t group) {
  // 4 rows per wave (2 at in = 4096, whose rows hold 64 columns per lane). A
  // workgroup runs nch chunks of 8 tokens with its rows dequantized once, nch
  // chosen to keep about 64 token ranges (512 workgroups at 128 experts).
  const uint32_t chunks = (T + ROUTER_TOKENS_PER_WAVE - 1) / ROUTER_TOKENS_PER_WAVE;
  const uint32_t nch = std::min(8u, std::max(1u, chunks / 64u));
  const uint32_t ty = (chunks + nch - 1) / nch;
  const dim3 grid4((n_exp + 15) / 16, ty), grid2((n_exp + 7) / 8, ty);
  const size_t lds = sizeof(uint16_t) * ROUTER_TOKENS_PER_WAVE * in;  // 64 KB at in = 4096
  switch (in) {
    case 512: OBS_LAUNCH(ctx, "q8_gate_logits", q8_gate_logits_kernel<2, 4><<<grid4, 256, lds, ctx->stream>>>(w8, s, b, x, logits, T, in, n_exp, group, nch)); break;
    case 1024: OBS_LAUNCH(ctx, "q8_gate_logits", q8_gate_logits_kernel<4, 4><<<grid4, 256, lds, ctx->stream>>>(w8, s, b, x, logits, T, in, n_exp, group, nch)); break;
    case 2048: OBS_LAUNCH(ctx, "q8_gate_logits", q8_gate_logits_kernel<8, 4><<<grid4, 256, lds, ctx->stream>>>(w8, s, b, x, logits, T, in, n_exp, group, nch)); break;
    default: OBS_LAUNCH(ctx, "q8_gate_logits", q8_gate_logits_kernel<16, 2><<<grid2, 256, lds, ctx->stream>>>(w8, s, b, x, logits, T, in, n_exp, group, nch)); break;
  }
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
