// obs_prefill.hip — grouped prefill MoE (placeholder until the grouped GEMM lands).
#include "obs_internal.hpp"

extern "C" {

size_t obs_moe_prefill_workspace(const obs_moe_config* cfg, uint32_t T) { (void)cfg; (void)T; return 0; }

int obs_moe_prefill(obs_ctx* ctx, const obs_moe_config*, const obs_moe_layer*, const uint16_t*, const uint16_t*,
                    uint16_t*, uint32_t, const int32_t*, const float*, void*, size_t) {
  if (!ctx) return OBS_E_INVALID;
  return obs::set_error(ctx, OBS_E_UNSUPPORTED, "obs_moe_prefill: not built yet");
}

int obs_q4_matmul(obs_ctx* ctx, const uint32_t*, const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*,
                  uint32_t, uint32_t, uint32_t, uint32_t) {
  if (!ctx) return OBS_E_INVALID;
  return obs::set_error(ctx, OBS_E_UNSUPPORTED, "obs_q4_matmul: not built yet");
}

}  // extern "C"
