// obs_layer_fused.hip — a whole decode layer at the Qwen3-30B-A3B shape
// (forward_layer, src/forward.rs:398-443) in ONE launch: the attention half
// (obs_attn_half.hpp) and then, in the same 256 workgroups, the MoE half with
// its post-attention RMSNorm (obs_moe_half.hpp).
//
// Why: between the two halves as separate launches sit a kernel boundary and
// the MoE launch's start (its arguments, then x1 from memory): about 1.3 us
// before the MoE half's first router product. Here each workgroup publishes
// its 8 rows of x1 as epoch-tagged slots written through to memory, and every
// workgroup's MoE half polls the 2,048 values (wave w the 512 columns
// 512 w .. + 512, shared through LDS) the moment the last row lands. Each half
// keeps its own exchange slots; both are tagged with one epoch, the count of
// earlier launches of this kernel on this workspace, which workgroup 0 adds
// to as it exits (after its combine, which follows every workgroup's x1
// publish, each of which came after that workgroup read the count).
//
// The arithmetic is the two launches' instruction for instruction, so x1, y,
// the expert ids and the routing weights are bit-identical to obs_attn_decode
// followed by obs_moe_decode (the residual of the combine is the x1 row the
// workgroup itself produced, kept in a register).
#include "obs_internal.hpp"
#include "obs_attn_half.hpp"
#include "obs_moe_half.hpp"

namespace {

// Workspace: the attention half's area | the MoE half's area | x1 slots.
constexpr size_t al256(size_t v) { return (v + 255) & ~size_t(255); }
constexpr size_t LW_MOE = al256(AW_BYTES);
constexpr size_t LW_X1 = LW_MOE + al256(WS_BYTES);
constexpr size_t LW_BYTES = LW_X1 + size_t(AH / 2) * 8;
static_assert(AH == FH && ANWG == NWG && ANGRP == NGROUP, "the halves share the layer's shape and launch");

template <int NQ>
__global__ void __launch_bounds__(256, 1) __attribute__((amdgpu_waves_per_eu(1, 1)))
layer_fused_kernel(AttnArgs a, FusedArgs m) {
  uint64_t* x1_slots = reinterpret_cast<uint64_t*>(a.ws + LW_X1);
  uint32_t x1_row = 0, epoch = 0;
  if (!attn_half<true>(a, x1_slots, reinterpret_cast<const uint32_t*>(m.ws + WS_ERR), &x1_row, &epoch)) return;
  moe_half<NQ, true, MOE_X_SLOTS>(m, m.ws, epoch, x1_slots, x1_row);
  if (threadIdx.x == 0 && blockIdx.x == 0)
    __hip_atomic_fetch_add(reinterpret_cast<uint64_t*>(a.ws + AW_COUNT), uint64_t{1}, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

namespace obs {

int layer_fused_status(obs_ctx* ctx) {
  if (!ctx->layer_ws) return OBS_OK;
  OBS_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  uint32_t err[2] = {0, 0};
  unsigned char* ws = static_cast<unsigned char*>(ctx->layer_ws);
  OBS_HIP_TRY(ctx, hipMemcpy(&err[0], ws + AW_ERR, 4, hipMemcpyDeviceToHost));
  OBS_HIP_TRY(ctx, hipMemcpy(&err[1], ws + LW_MOE + WS_ERR, 4, hipMemcpyDeviceToHost));
  if (err[0] || err[1]) {
    OBS_HIP_TRY(ctx, hipMemset(ctx->layer_ws, 0, LW_BYTES));
    OBS_HIP_TRY(ctx, hipDeviceSynchronize());
    return set_error(ctx, OBS_E_HIP,
                     "one-launch decode layer: a cross-workgroup wait timed out in the %s half (were all CUs "
                     "available?); outputs since then are invalid; workspace reset",
                     err[0] ? "attention" : "MoE");
  }
  return OBS_OK;
}

}  // namespace obs

extern "C" {

int obs_layer_decode(obs_ctx* ctx, const obs_attn_layer* attn, const obs_moe_config* cfg, const obs_moe_layer* moe,
                     const uint16_t* x, uint16_t* k_cache, uint16_t* v_cache_t, uint32_t max_len, float eps,
                     float theta, const int32_t* state, uint16_t* x1, uint16_t* y, int32_t* ids_out, float* w_out) {
  if (!ctx) return OBS_E_INVALID;
  const char* who = "obs_layer_decode";
  int rc = obs::check_attn_decode(ctx, who, attn, x, k_cache, v_cache_t, state, x1, max_len);
  if (rc != OBS_OK) return rc;
  rc = obs::check_moe_config(ctx, who, cfg);
  if (rc != OBS_OK) return rc;
  rc = obs::check_moe_layer(ctx, who, moe);
  if (rc != OBS_OK) return rc;
  if (!y) return obs::set_error(ctx, OBS_E_INVALID, "%s: null y", who);
  if (!obs::fused_decode_supported(cfg) || !moe->norm_w || cfg->hidden != AH)
    return obs::set_error(ctx, OBS_E_SHAPE,
                          "%s: needs hidden 2048, inter 768, top_k 8, group 64, n_exp <= 256 and a post-attention "
                          "norm weight", who);
  if (ctx->decode_path == OBS_DECODE_MULTI)
    return obs::set_error(ctx, OBS_E_UNSUPPORTED, "%s: the context is set to the 4-launch decode path", who);
  if (!(obs::dispatch_gate(ctx->num_cus, ctx->xcd_map_ok, ctx->inorder_ok) & OBS_PATH_FUSED_DECODE))
    return obs::set_error(ctx, OBS_E_UNSUPPORTED, "%s: the device's dispatch does not allow the one-launch MoE half",
                          who);
  if (!ctx->layer_ws) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    OBS_HIP_TRY(ctx, hipStreamIsCapturing(ctx->stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
      return obs::set_error(ctx, OBS_E_INVALID, "%s: run once before capturing (workspace allocation)", who);
    OBS_HIP_TRY(ctx, hipMalloc(&ctx->layer_ws, LW_BYTES));
    OBS_HIP_TRY(ctx, hipMemset(ctx->layer_ws, 0, LW_BYTES));
    OBS_HIP_TRY(ctx, hipDeviceSynchronize());
  }
  const float* rope = nullptr;
  rc = obs::ensure_rope_table(ctx, theta, max_len, &rope);
  if (rc != OBS_OK) return rc;
  unsigned char* ws = static_cast<unsigned char*>(ctx->layer_ws);
  const obs_attn_layer* L = attn;
  AttnArgs a{L->q_w, L->q_s, L->q_b, L->k_w, L->k_s, L->k_b, L->v_w, L->v_s, L->v_b, L->o_w, L->o_s, L->o_b,
             L->in_norm, L->q_norm, L->k_norm, x, x1, k_cache, v_cache_t, state, rope, ws, max_len, eps,
             1.4426950408889634f / __builtin_sqrtf(static_cast<float>(AHD))};
  FusedArgs f{moe->gate_w, moe->gate_s, moe->gate_b, moe->up_w, moe->up_s, moe->up_b, moe->down_w, moe->down_s,
              moe->down_b, moe->router_w, moe->router_s, moe->router_b, x1, x1, y, moe->norm_w, cfg->rms_eps,
              ids_out, w_out, ws + LW_MOE, cfg->n_exp, cfg->norm_topk, cfg->route_rule};
  if (cfg->n_exp <= 128)
    OBS_LAUNCH(ctx, "layer_fused", layer_fused_kernel<2><<<ANWG, 256, 0, ctx->stream>>>(a, f));
  else
    OBS_LAUNCH(ctx, "layer_fused", layer_fused_kernel<4><<<ANWG, 256, 0, ctx->stream>>>(a, f));
  return OBS_OK;
}

}  // extern "C"
