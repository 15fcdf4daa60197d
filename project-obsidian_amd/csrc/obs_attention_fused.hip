// obs_attention_fused.hip — the attention half of a decode layer in ONE launch
// for the Qwen3-30B-A3B shape (hidden 2048, 32 query heads, 4 kv heads, head
// dim 128): x1 = x + o_proj(attention(rope(norm(q)), rope(norm(k)), v)) with
// q, k, v = projections of rmsnorm(x) (src/forward.rs:403-418).
//
// Why one launch: the separate launches (q/k/v mat-vec, norm + RoPE + cache
// append, split attention, split combine, o mat-vec) each move a few MB or
// less, and a launch boundary with its fences and first memory round trip
// cost about as much as their work. Here 256 workgroups (one per CU) pass the
// few values that cross workgroups through epoch-tagged slots (see
// slot_store), as decode_fused_kernel does for the MoE half.
//
// Work split. Workgroup b belongs to group g = b % 8, which the dispatcher
// places on one XCD (consecutive workgroups go round-robin over the 8 XCDs),
// and has index j = b / 8 in it. Group g serves kv head g / 2 and its query
// heads 8 (g / 2) + 4 (g % 2) .. + 3, over the whole sequence, so every
// exchange but the last stays inside the group and its L2:
//   1. each of the group's 128 waves computes 6 of its 768 q/k/v rows (4 query
//      heads, the key and the value head; RMSNorm of x fused) and publishes
//      them to the group's slots (both groups of a kv head compute its key and
//      value rows, bit-identically);
//   2. workgroup j takes split j of 32 of the sequence: it polls the group's
//      rows, applies the per-head RMSNorm and NeoX RoPE, appends the key and
//      value at pos to the caches (the even group's split holding pos) and runs
//      the split's attention with the decode kernel's MFMA block math (its own
//      key/value at pos spliced in from registers); the 4 waves' partials are
//      merged in LDS and published;
//   3. workgroup j combines query head j / 8 of the group, 16 dims, over the
//      32 splits and publishes them as bf16 pairs;
//   4. every workgroup polls the group's 512 attention outputs into LDS and
//      computes, for its 64 rows of W_o, the partial product over the group's
//      512 columns, published across XCDs;
//   5. every workgroup sums the 8 groups' partials of 8 rows with the residual:
//      x1 = x + sum_g partial_g, in group order, rounded once to bf16.
// (The earlier split of the same work over the whole grid exchanged q/k/v,
// the split partials and the attention outputs across XCDs, three round trips
// through memory that cost 1.5-3.3 us each.)
// Load order. A wave's loads complete in issue order, and a CU accepts them
// only as fast as memory drains them, so each batch sits where it delays
// nothing more urgent: the q/k/v rows at the start (they have the bandwidth
// to themselves), the first block's keys right behind them (they arrive while
// the rows are computed and exchanged, before the data of the poll that waits
// behind them; issued ahead of the rows, they shared the rows' bandwidth), its
// values right after the poll (issued before it, the poll waited for them),
// and the o rows after the attention blocks, where their latency overlaps the
// two exchanges that precede their use.
// Every wait is bounded (100 ms of the constant clock); a time-out sets the
// workspace's error flag, reported and cleared by obs_device_status.
#include "obs_internal.hpp"
#include "obs_attn_half.hpp"

namespace {

__global__ void __launch_bounds__(256, 1) __attribute__((amdgpu_waves_per_eu(1, 1)))
attn_fused_kernel(AttnArgs a) {
  attn_half<false>(a, nullptr, nullptr, nullptr, nullptr);
}

}  // namespace

namespace obs {

int attn_fused_status(obs_ctx* ctx) {
  if (!ctx->attn_ws) return OBS_OK;
  OBS_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  uint32_t err = 0;
  OBS_HIP_TRY(ctx, hipMemcpy(&err, static_cast<unsigned char*>(ctx->attn_ws) + AW_ERR, 4, hipMemcpyDeviceToHost));
  if (err) {
    OBS_HIP_TRY(ctx, hipMemset(ctx->attn_ws, 0, AW_BYTES));
    OBS_HIP_TRY(ctx, hipDeviceSynchronize());
    return set_error(ctx, OBS_E_HIP,
                     "fused attention: a cross-workgroup wait timed out (were all CUs available?); "
                     "outputs since then are invalid; workspace reset");
  }
  return OBS_OK;
}

}  // namespace obs

namespace obs {
uint32_t fused_attn_workgroups() { return ANWG; }
}  // namespace obs

namespace obs {

// Arguments of the one-launch attention half (obs_attn_decode and
// obs_layer_decode): pointers, shapes, alignment, and a device whose
// dispatch the fused kernels rely on.
int check_attn_decode(obs_ctx* ctx, const char* who, const obs_attn_layer* L, const uint16_t* x,
                      const uint16_t* k_cache, const uint16_t* v_cache_t, const int32_t* state, const uint16_t* x1,
                      uint32_t max_len) {
  if (!L || !x || !k_cache || !v_cache_t || !state || !x1) return set_error(ctx, OBS_E_INVALID, "%s: null pointer", who);
  const void* ptrs[] = {L->q_w, L->q_s, L->q_b, L->k_w, L->k_s, L->k_b, L->v_w, L->v_s, L->v_b,
                        L->o_w, L->o_s, L->o_b, L->in_norm, L->q_norm, L->k_norm};
  for (const void* p : ptrs)
    if (!p) return set_error(ctx, OBS_E_INVALID, "%s: a layer tensor is null", who);
  if (max_len == 0 || max_len % 32u != 0)
    return set_error(ctx, OBS_E_SHAPE, "%s: max_len must be a positive multiple of 32 (got %u)", who, max_len);
  if (!aligned(x, 16) || !aligned(L->in_norm, 16) || !aligned(L->q_w, 16) || !aligned(L->k_w, 16) ||
      !aligned(L->v_w, 16) || !aligned(L->o_w, 16) || !aligned(L->q_norm, 4) || !aligned(L->k_norm, 4) ||
      !aligned(k_cache, 16) || !aligned(v_cache_t, 16))
    return set_error(ctx, OBS_E_ALIGN, "%s: weights, x and the caches must be 16-byte aligned", who);
  if (!(dispatch_gate(ctx->num_cus, ctx->xcd_map_ok, ctx->inorder_ok) & OBS_PATH_FUSED_ATTN))
    return set_error(ctx, OBS_E_UNSUPPORTED,
                     "%s: needs %u CUs, one workgroup per CU, each group b %% 8 on one XCD "
                     "(the device has %d CUs; XCD map %s)",
                     who, ANWG, ctx->num_cus, ctx->xcd_map_ok ? "as expected" : "not as expected");
  return OBS_OK;
}

}  // namespace obs

extern "C" {

int obs_attn_decode(obs_ctx* ctx, const obs_attn_layer* L, const uint16_t* x, uint16_t* k_cache,
                    uint16_t* v_cache_t, uint32_t max_len, float eps, float theta, const int32_t* state,
                    uint16_t* x1) {
  if (!ctx) return OBS_E_INVALID;
  int rc = obs::check_attn_decode(ctx, "obs_attn_decode", L, x, k_cache, v_cache_t, state, x1, max_len);
  if (rc != OBS_OK) return rc;
  if (!ctx->attn_ws) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    OBS_HIP_TRY(ctx, hipStreamIsCapturing(ctx->stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
      return obs::set_error(ctx, OBS_E_INVALID, "obs_attn_decode: run once before capturing (workspace allocation)");
    OBS_HIP_TRY(ctx, hipMalloc(&ctx->attn_ws, AW_BYTES));
    OBS_HIP_TRY(ctx, hipMemset(ctx->attn_ws, 0, AW_BYTES));
    OBS_HIP_TRY(ctx, hipDeviceSynchronize());
  }
  const float* rope = nullptr;
  rc = obs::ensure_rope_table(ctx, theta, max_len, &rope);
  if (rc != OBS_OK) return rc;
  AttnArgs a{L->q_w, L->q_s, L->q_b, L->k_w, L->k_s, L->k_b, L->v_w, L->v_s, L->v_b, L->o_w, L->o_s, L->o_b,
             L->in_norm, L->q_norm, L->k_norm, x, x1, k_cache, v_cache_t, state, rope,
             static_cast<unsigned char*>(ctx->attn_ws), max_len, eps,
             1.4426950408889634f / __builtin_sqrtf(static_cast<float>(AHD))};
  OBS_LAUNCH(ctx, "attn_fused", attn_fused_kernel<<<ANWG, 256, 0, ctx->stream>>>(a));
  return OBS_OK;
}

}  // extern "C"
