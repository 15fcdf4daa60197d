// obs_decode_fused.hip — the decode MoE half of one layer (src/forward.rs:421-441)
// in ONE launch, for the Qwen3-30B-A3B expert shape (hidden 2048, moe_inter 768,
// top-8, group 64, up to 256 experts).
//
// Why one launch: at T=1 the layer moves ~21.5 MB, 2.7 us at the 8 TB/s HBM
// peak, while every kernel boundary costs ~1.6 us even inside a HIP graph and
// an agent-scope release or acquire fence costs 2-5 us. The layer therefore
// runs as 256 workgroups (one per CU) that exchange the few values that cross
// workgroups — router logits, the SwiGLU activations h, the per-expert down
// outputs — through epoch-tagged 64-bit slots written and polled with relaxed
// device-coherent atomics. A reader spins until every slot it needs carries the
// current launch's epoch, so the value arrives with the flag: no counters, no
// fences, no second round trip.
//
// Work split. Workgroup b belongs to group g = b % 8 (the hardware dispatches
// consecutive workgroups round-robin over the 8 XCDs, so a group shares one L2)
// and has index j = b / 8 within it.
//   1. Router: each group computes all E logits (one 2 KB row per wave) in the
//      router's documented reduction order, so every group sees bit-identical
//      logits; wave 0 of every workgroup runs softmax + top-8 on them and
//      shares the result through LDS.
//   2. Group g serves routing rank g: expert e_g = ids[g]. Its 128 waves stream
//      the 768 gate and up rows (6 each) and the scales of the down rows the
//      workgroup will need (64 rows x 384 B per workgroup); the down rows
//      themselves are issued once most of the gate/up rows are in (below), so
//      they do not compete with them.
//   3. h = silu(gate.x) * (up.x) goes to the group's h slots; each workgroup
//      polls them into LDS in three blocks, adding each block's terms to its 64
//      down rows as the block arrives (the down weights are in registers).
//   4. Every workgroup combines 8 rows: it polls the 8 ranks' outputs for them
//      and accumulates residual + sum_r w_r * y_r in rank order (forward.rs:440).
//      (Group 0 alone, 64 rows per workgroup, measured 0.2 us slower per layer
//      once the launch count took one atomic instead of 256; with 256 exit
//      atomics at once the spread combine had been 1 us slower.)
// The logit and h slots are written and polled within one XCD and live in its
// L2; the y slots cross XCDs and are written through to memory.
// The epoch is derived from a device-side count of exited workgroups (see the
// kernel's first lines), so graph replays need no host involvement.
//
// Every wait is bounded (100 ms on the GPU's constant clock); a timeout sets a
// device error flag, later launches then exit at once, and obs_device_status()
// reports it and resets the workspace.
#include "obs_internal.hpp"
#include "obs_moe_half.hpp"

namespace {

// One workgroup per CU, so one wave per SIMD: the compiler is told so and need
// not trade waits for registers.
template <int NQ, bool NORM>
__global__ void __launch_bounds__(256, 1) __attribute__((amdgpu_waves_per_eu(1, 1))) decode_fused_kernel(FusedArgs a) {
  moe_half<NQ, NORM, MOE_X_MEM>(a, a.ws, 0u, nullptr, 0u);
}

}  // namespace

namespace obs {

bool fused_decode_supported(const obs_moe_config* cfg) {
  return cfg->hidden == FH && cfg->inter == FI && cfg->top_k == FK && cfg->group == FG && cfg->n_exp <= MAX_E;
}

uint32_t fused_decode_workgroups() { return NWG; }

size_t fused_decode_ws_bytes() { return WS_BYTES; }

static_assert(WS_BYTES == STATIC_FUSED_BYTES, "the static scratch holds one exchange area");

int launch_fused_decode(obs_ctx* ctx, const obs_moe_config* cfg, const obs_moe_layer* L, const uint16_t* x,
                        const uint16_t* residual, uint16_t* y, int32_t* ids_out, float* w_out) {
  if (!ctx->fused_ws) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    OBS_HIP_TRY(ctx, hipStreamIsCapturing(ctx->stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
      return set_error(ctx, OBS_E_INVALID, "obs_moe_decode: run once before capturing (workspace allocation)");
    OBS_HIP_TRY(ctx, hipMalloc(&ctx->fused_ws, WS_BYTES));
    OBS_HIP_TRY(ctx, hipMemset(ctx->fused_ws, 0, WS_BYTES));
    OBS_HIP_TRY(ctx, hipDeviceSynchronize());
  }
  return launch_fused_decode_ws(ctx, cfg, L, x, residual, y, ids_out, w_out, ctx->fused_ws);
}

int launch_fused_decode_ws(obs_ctx* ctx, const obs_moe_config* cfg, const obs_moe_layer* L, const uint16_t* x,
                           const uint16_t* residual, uint16_t* y, int32_t* ids_out, float* w_out, void* ws) {
  FusedArgs a{L->gate_w, L->gate_s, L->gate_b, L->up_w, L->up_s, L->up_b, L->down_w, L->down_s, L->down_b,
              L->router_w, L->router_s, L->router_b, x, residual, y, L->norm_w, cfg->rms_eps, ids_out, w_out,
              static_cast<unsigned char*>(ws), cfg->n_exp, cfg->norm_topk, cfg->route_rule};
  // the layer with a post-attention norm (the decoder's) and without (the
  // bare MoE block) are two instantiations, so each is timed under its own name
  const bool norm = L->norm_w != nullptr;
  if (cfg->n_exp <= 128) {
    if (norm)
      OBS_LAUNCH(ctx, "decode_fused_norm", decode_fused_kernel<2, true><<<NWG, 256, 0, ctx->stream>>>(a));
    else
      OBS_LAUNCH(ctx, "decode_fused", decode_fused_kernel<2, false><<<NWG, 256, 0, ctx->stream>>>(a));
  } else {
    if (norm)
      OBS_LAUNCH(ctx, "decode_fused_norm", decode_fused_kernel<4, true><<<NWG, 256, 0, ctx->stream>>>(a));
    else
      OBS_LAUNCH(ctx, "decode_fused", decode_fused_kernel<4, false><<<NWG, 256, 0, ctx->stream>>>(a));
  }
  return OBS_OK;
}

int fused_decode_status(obs_ctx* ctx) { return ctx->fused_ws ? fused_decode_status_ws(ctx, ctx->fused_ws) : OBS_OK; }

int fused_decode_status_ws(obs_ctx* ctx, void* ws) {
  OBS_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  uint32_t err = 0;
  OBS_HIP_TRY(ctx, hipMemcpy(&err, static_cast<unsigned char*>(ws) + WS_ERR, 4, hipMemcpyDeviceToHost));
  if (err) {
    OBS_HIP_TRY(ctx, hipMemset(ws, 0, WS_BYTES));
    OBS_HIP_TRY(ctx, hipDeviceSynchronize());
    return set_error(ctx, OBS_E_HIP,
                     "fused decode: a cross-workgroup wait timed out (were all CUs available?); "
                     "outputs since then are invalid; workspace reset");
  }
  return OBS_OK;
}

}  // namespace obs
