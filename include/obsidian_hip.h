/*
 * obsidian_hip.h — C ABI of the MI355X (gfx950) MoE expert hot path.
 *
 * This is the kernel-dispatch boundary of the obsidian engine re-expressed as
 * plain C: the Rust host (src/executor.rs, src/router.rs, src/forward.rs in the
 * reference) binds these functions with `extern "C"` instead of building Metal
 * pipelines. Every entry point names the reference interface it replaces.
 *
 * Conventions
 *   - All tensor arguments are DEVICE pointers (HBM), caller-owned, unless a
 *     comment says "host". Nothing here allocates on the hot path.
 *   - bf16 values travel as uint16_t bit patterns, fp32 as float.
 *   - Quantized tensors use the MLX affine layout (tools/split_experts.py:9-19):
 *       weight uint32 [rows, cols*bits/32]: element c is bits-wide field c%(32/bits)
 *         of word c/(32/bits), low bits first;
 *       scales, biases bf16 [rows, cols/group];  w = q*scale + bias.
 *     Expert tensors are stacked on a leading expert axis, as in the checkpoint's
 *     model.layers.{l}.mlp.switch_mlp.{gate,up,down}_proj.{weight,scales,biases}.
 *   - Calls are asynchronous and ordered on the context's stream (the Metal
 *     same-queue FIFO order, forward.rs:2-3). obs_sync() is the drain.
 *   - Return value: OBS_OK (0) or a negative OBS_E_* code; obs_last_error()
 *     holds the message (the reference's Result<_, String>). Arguments are
 *     validated before any launch; on error nothing is launched.
 *   - One context per host thread; a context is not internally locked.
 */
#ifndef OBSIDIAN_HIP_H
#define OBSIDIAN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct obs_ctx obs_ctx;

enum {
  OBS_OK = 0,
  OBS_E_INVALID = -1,     /* null pointer / bad enum / bad count */
  OBS_E_SHAPE = -2,       /* shape not supported (e.g. cols % group != 0) */
  OBS_E_ALIGN = -3,       /* pointer alignment requirement not met */
  OBS_E_HIP = -4,         /* HIP runtime error */
  OBS_E_NOMEM = -5,       /* allocation failed / workspace too small */
  OBS_E_UNSUPPORTED = -6, /* no HIP device of the supported architecture */
};

/* ------------------------------------------------------------------ */
/* Context / executor — replaces ObsidianExecutor (src/executor.rs:39-70) */
/* ------------------------------------------------------------------ */

/* Bind device `device`, check it is gfx950, create the context's stream.
 * Replaces ObsidianExecutor::new (executor.rs:39-58): kernels are compiled
 * offline into this library, so there is no runtime shader compilation. */
int obs_create(int device, obs_ctx** out);
void obs_destroy(obs_ctx* ctx);
/* Last error message of this context (never NULL). Result<_, String>. */
const char* obs_last_error(const obs_ctx* ctx);
/* Message of the last failed obs_create on this thread. */
const char* obs_create_error(void);
/* Use a caller-owned hipStream_t (e.g. a graph-capturing stream) instead of
 * the context's own; NULL restores the own stream. executor.rs:60-66 queue(). */
int obs_set_stream(obs_ctx* ctx, void* hip_stream);
void* obs_get_stream(const obs_ctx* ctx);

/* ------------------------------------------------------------------ */
/* Buffers — replace device().new_buffer / contents() / drain          */
/* (forward.rs:264-286). HBM is not host-visible, so copies are explicit. */
/* ------------------------------------------------------------------ */
int obs_alloc(obs_ctx* ctx, size_t bytes, void** dptr);
int obs_free(obs_ctx* ctx, void* dptr);
/* host -> device, stream-ordered; returns when the host buffer may be reused */
int obs_upload(obs_ctx* ctx, void* dst_dev, const void* src_host, size_t bytes);
/* device -> host; waits for prior work on the stream (Buffer::contents after drain) */
int obs_download(obs_ctx* ctx, void* dst_host, const void* src_dev, size_t bytes);
int obs_memset(obs_ctx* ctx, void* dst_dev, int value, size_t bytes);
/* Model::drain (forward.rs:282-286): wait for all work queued on the stream. */
int obs_sync(obs_ctx* ctx);

/* Stream-ordered timing with HIP events on the context's stream (no
 * reference counterpart; the reference times with std::time::Instant,
 * main.rs:102-115). obs_timer_stop waits and returns elapsed milliseconds. */
int obs_timer_start(obs_ctx* ctx);
int obs_timer_stop(obs_ctx* ctx, float* ms);

/* ------------------------------------------------------------------ */
/* Graph capture (no reference counterpart: the Metal engine commits one  */
/* command buffer per dispatch, forward.rs:289-301). Calls issued between */
/* begin and end are recorded, not run, and replay as one HIP graph.      */
/* Nothing that allocates may be captured: run each entry point once      */
/* before capturing it so its workspace exists.                           */
/* ------------------------------------------------------------------ */
typedef struct obs_graph obs_graph;
int obs_capture_begin(obs_ctx* ctx);
int obs_capture_end(obs_ctx* ctx, obs_graph** out);
int obs_graph_launch(obs_ctx* ctx, obs_graph* graph);
void obs_graph_destroy(obs_graph* graph);

/* ------------------------------------------------------------------ */
/* In-stream kernel timing (no reference counterpart). While enabled,     */
/* every kernel the library launches on the context's stream is bracketed */
/* by a pair of HIP events (also inside a capture). obs_profile_accumulate */
/* waits for the stream and adds each pair's elapsed time to a per-kernel */
/* total; a captured graph can be replayed and accumulated repeatedly.    */
/* ------------------------------------------------------------------ */
/* Enqueue a kernel that keeps the stream busy for `us` microseconds (capped
 * at 1 s, measured on the GPU's constant-rate clock) so the host can queue
 * the launches to be timed ahead of their execution. */
int obs_stream_hold(obs_ctx* ctx, uint32_t us);
int obs_profile_enable(obs_ctx* ctx, int on);
int obs_profile_accumulate(obs_ctx* ctx);
int obs_profile_count(const obs_ctx* ctx);
int obs_profile_stat(const obs_ctx* ctx, int i, const char** name, double* total_ms, int64_t* launches);
int obs_profile_clear(obs_ctx* ctx);

/* Achievable peaks (no reference counterpart; the reference's harness is a
 * wall-clock token timer, main.rs:99-116): the ceilings the roofline
 * fractions are read against, measured on the device itself. Both launch on
 * the context's stream and are timed by the caller (obs_timer_*).
 * obs_measure_read: every 16-byte chunk of [src, src + bytes) read once with
 * the fused decode's non-temporal 16-byte loads (8 workgroups per CU); sink is
 * a 4-byte device word the kernel never writes in practice. obs_measure_mfma:
 * v_mfma_f32_32x32x16_bf16 only, 4 independent chains per wave, 8 waves per
 * CU, `iters` steps (1 to 2^24); *flops (host) receives the flop count of the launch and
 * clocks[0..1] (device) the core clock cycles and 100 MHz constant-clock
 * ticks of one wave's loop, whose ratio is the clock the MFMAs ran at. */
int obs_measure_read(obs_ctx* ctx, const void* src, size_t bytes, uint32_t* sink);
int obs_measure_mfma(obs_ctx* ctx, uint32_t iters, float* sink, uint64_t* clocks, double* flops);

/* ------------------------------------------------------------------ */
/* Quantized tensor kernels                                            */
/* ------------------------------------------------------------------ */

/* Dequantize an MLX affine tensor (mx.dequantize, validate_dequant.py:21;
 * the unpack of fused_dequant_matvec_4bit.metal:39-42 and forward.rs:451-457).
 * bits 4 or 8; out_f32 [rows, cols] gets fl32(q*scale+bias) exactly;
 * out_bf16 (optional, may be NULL) gets its round-to-nearest-even bf16.
 * Either output may be NULL, not both. */
int obs_dequant(obs_ctx* ctx, int bits, const uint32_t* w, const uint16_t* scales,
                const uint16_t* biases, float* out_f32, uint16_t* out_bf16,
                uint32_t rows, uint32_t cols, uint32_t group);

/* y = dequant(W) . x for one token — Model::dequant (forward.rs:303-310) /
 * fused_dequant_matvec_4bit.metal. W 4-bit [out, in]; x bf16 [in];
 * y_f32 [out] (fp32 result, may be NULL) and/or y_bf16 [out] (may be NULL).
 * fp32 accumulation; requires in % group == 0, in % 64 == 0. */
int obs_q4_matvec(obs_ctx* ctx, const uint32_t* w, const uint16_t* scales,
                  const uint16_t* biases, const uint16_t* x, float* y_f32,
                  uint16_t* y_bf16, uint32_t in, uint32_t out, uint32_t group);

/* Y[T, out] = X[T, in] . dequant(W)^T, bf16 in/out, fp32 accumulate — Model::matmul_raw
 * (forward.rs:313-321) / matmul_dequant_4bit.metal. Runs the grouped
 * dequant-to-register bf16 MFMA GEMM with a single expert. Requires group == 64,
 * in % 256 == 0 and out % 128 == 0 (OBS_E_SHAPE otherwise). */
int obs_q4_matmul(obs_ctx* ctx, const uint32_t* w, const uint16_t* scales,
                  const uint16_t* biases, const uint16_t* X, uint16_t* Y,
                  uint32_t T, uint32_t in, uint32_t out, uint32_t group);

/* ------------------------------------------------------------------ */
/* Router — Model::gate_gpu (forward.rs:386-397) + MoeRouter (router.rs) */
/* ------------------------------------------------------------------ */

/* logits[T, n_exp] (fp32) = dequant8(Wg) . x[t] for T tokens — dequant_matvec_8bit.metal.
 * Fixed reduction order: 64 lanes each own in/64 contiguous columns
 * (serial fma), combined by an xor butterfly; bit-reproducible. */
int obs_q8_gate_logits(obs_ctx* ctx, const uint32_t* w8, const uint16_t* scales,
                       const uint16_t* biases, const uint16_t* x, float* logits,
                       uint32_t T, uint32_t in, uint32_t n_exp, uint32_t group);

/* Routing rules.
 * OBS_ROUTE_REF (0, the default of a zeroed obs_moe_config): the reference's
 *   rule. Each logit is rounded to f16 (round to nearest even), the type
 *   dequant_matvec_8bit.metal:30 stores it in, before the softmax; the weights
 *   are f16 values, f16(p) and, renormalised, f16(f16(p) / wsum)
 *   (moe_routing_topk.metal:47, :55; router.rs:50-54 reads them as f32).
 * OBS_ROUTE_F32 (1): the same softmax and selection on the fp32 logits, fp32
 *   weights (no reference counterpart). */
enum { OBS_ROUTE_REF = 0, OBS_ROUTE_F32 = 1 };

/* Softmax over n_exp logits, top-k by repeated argmax over the probabilities
 * (ties -> lower expert id), optional renormalisation — moe_routing_topk.metal:24-56
 * and MoeRouter::route_dispatch (router.rs:62-83). logits fp32 [T, n_exp] (rounded
 * to f16 inside under OBS_ROUTE_REF), ids int32 [T, k], weights fp32 [T, k].
 * n_exp <= 256 (the reference kernel's limit), 1 <= k <= min(n_exp, 64);
 * rule OBS_ROUTE_REF or OBS_ROUTE_F32.
 * A slot with no selectable expert (NaN logits) gets id -1 and weight 0.
 * The synchronous MoeRouter::route (router.rs:25-56) is this call followed by
 * obs_sync + obs_download. */
int obs_route_topk(obs_ctx* ctx, const float* logits, int32_t* ids, float* weights,
                   uint32_t T, uint32_t n_exp, uint32_t k, int norm_topk, int rule);

/* obs_q8_gate_logits followed by obs_route_topk: the router step of
 * MoeRouter::route_dispatch as forward.rs:386-397 and router.rs:62-83 run it
 * (gate_gpu, then the routing kernel). logits, ids and weights are written as
 * by the two calls, bit for bit. Up to 8 tokens it is one launch whose
 * workgroups share one XCD (on a device where obs_create's dispatch probe
 * found workgroup b on XCD b % 8), using a context counter that each launch
 * leaves at zero, so such calls on one context must not overlap (issue them
 * on one stream); otherwise the two launches. */
int obs_route(obs_ctx* ctx, const uint32_t* w8, const uint16_t* scales, const uint16_t* biases,
              const uint16_t* x, float* logits, int32_t* ids, float* weights, uint32_t T,
              uint32_t in, uint32_t n_exp, uint32_t group, uint32_t k, int norm_topk, int rule);

/* ------------------------------------------------------------------ */
/* Elementwise — ops.metal ew_swiglu / ew_scaled_add (forward.rs:370-380) */
/* ------------------------------------------------------------------ */
/* h = silu(g) * u, bf16 in/out, fp32 math */
int obs_swiglu(obs_ctx* ctx, const uint16_t* g, const uint16_t* u, uint16_t* h, uint32_t n);
/* acc = acc + scale * y in place, bf16, fp32 math */
int obs_scaled_add(obs_ctx* ctx, uint16_t* acc, const uint16_t* y, float scale, uint32_t n);

/* RMSNorm of `rows` rows of `dim` bf16 values — shaders/rmsnorm.metal (the
 * rmsnorm pipeline) / Model::rmsnorm (forward.rs:345-357):
 * inv = 1 / sqrt(sum(x^2) / dim + eps) once per row, out = (x * inv) * weight,
 * fp32 math, rounded once to bf16. sum(x^2) has a fixed order (64 lanes each own dim/64
 * contiguous columns, serial fma, then an xor butterfly), so the result is
 * reproducible bit for bit. dim % 64 == 0, dim <= 8192; x and out may alias. */
int obs_rmsnorm(obs_ctx* ctx, const uint16_t* x, const uint16_t* weight, uint16_t* out,
                uint32_t rows, uint32_t dim, float eps);

/* ------------------------------------------------------------------ */
/* HBM-resident expert table + fused MoE layer                         */
/* (replaces ExpertIndex / read_experts_parallel / expert_pool,        */
/*  disk_io.rs:36-102, forward.rs:79-104)                              */
/* ------------------------------------------------------------------ */

typedef struct obs_moe_config {
  uint32_t n_exp;    /* num_experts (model.rs:15), <= 256 */
  uint32_t top_k;    /* num_experts_per_tok (model.rs:16) */
  uint32_t hidden;   /* hidden_size */
  uint32_t inter;    /* moe_intermediate_size (model.rs:17) */
  uint32_t group;    /* quantization group size (64) */
  int32_t norm_topk; /* norm_topk_prob (model.rs:22) */
  float rms_eps;     /* rms_norm_eps (model.rs:18); used when layer->norm_w is set */
  int32_t route_rule; /* OBS_ROUTE_REF (0: the reference's f16 logits and weights) or OBS_ROUTE_F32 */
} obs_moe_config;

/* One layer's MoE weights, all device pointers, stacked on the expert axis. */
typedef struct obs_moe_layer {
  const uint32_t* gate_w; const uint16_t* gate_s; const uint16_t* gate_b; /* [E, I, H/8], [E, I, H/G] */
  const uint32_t* up_w;   const uint16_t* up_s;   const uint16_t* up_b;   /* [E, I, H/8], [E, I, H/G] */
  const uint32_t* down_w; const uint16_t* down_s; const uint16_t* down_b; /* [E, H, I/8], [E, H, I/G] */
  const uint32_t* router_w; const uint16_t* router_s; const uint16_t* router_b; /* 8-bit [E, H/4], [E, H/G] */
  /* post_attention_layernorm.weight, bf16 [H], 16-byte aligned (forward.rs:419);
   * NULL: the MoE input is used as given (already normalised). */
  const uint16_t* norm_w;
} obs_moe_layer;

/* Decode MoE half of one layer for one token (forward.rs:421-441):
 * logits -> top-k -> per selected expert silu(gate x) * (up x) -> down ->
 * weighted sum in rank order. x, y bf16 [hidden]. If residual is non-NULL,
 * y = residual + sum (forward.rs:440 accumulates into the residual stream x1).
 * If layer->norm_w is set, the router and the experts see rmsnorm(x) with that
 * weight and cfg->rms_eps (forward.rs:419-421, as obs_rmsnorm computes it, in
 * the same launch); pass x1 as both x and residual for x1 + MoE(rmsnorm(x1)).
 * ids_out [top_k] / w_out [top_k] (may be NULL) receive the routing.
 * Workspace comes from the context (allocated once, on first use: make the
 * first call outside a graph capture).
 * For hidden 2048 / inter 768 / top_k 8 / group 64 (Qwen3-30B-A3B) on a
 * device with at least 256 CUs the layer runs as ONE launch of 256 workgroups
 * that exchange data through bounded device-side waits; it needs the GPU's CUs
 * free for that launch (no other kernel holding them). A wait that times out
 * is reported by obs_device_status(): call it after a sequence of calls (or a
 * graph replay) before using their outputs. Other shapes, and devices with
 * fewer CUs, run as 4 launches. */
int obs_moe_decode(obs_ctx* ctx, const obs_moe_config* cfg, const obs_moe_layer* layer,
                   const uint16_t* x, const uint16_t* residual, uint16_t* y,
                   int32_t* ids_out, float* w_out);

/* obs_moe_decode without any allocation: the same kernels, results and path
 * choice, with every intermediate (the fused path's exchange area, the
 * 4-launch path's logits, routing, h and normalised x) in a file-scope device
 * array of 272,896 bytes that each GPU holds for the life of the process
 * (looked up per device by obs_create). It calls no hipMalloc, hipFree or
 * allocating routine, so it may run under HIP graph capture without a warm-up
 * call. Every shape obs_moe_decode accepts fits; a larger need would be
 * rejected with OBS_E_NOMEM. All calls on one GPU share that array: calls that
 * overlap in time on one GPU (two streams, two contexts, two threads) race and
 * give wrong results; serialise them. A timed-out wait is reported by
 * obs_device_status() of the calling context.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under graph capture, tight serving loops, harnesses that forbid it). */
int obs_moe_decode_static(obs_ctx* ctx, const obs_moe_config* cfg, const obs_moe_layer* layer,
                          const uint16_t* x, const uint16_t* residual, uint16_t* y,
                          int32_t* ids_out, float* w_out);

/* Decode path selection (no reference counterpart; like the reference's
 * OBSIDIAN_NO_GEMM switch, forward.rs:125-126, it exists to compare paths). */
enum { OBS_DECODE_AUTO = 0, OBS_DECODE_MULTI = 1, OBS_DECODE_FUSED = 2 };
int obs_set_decode_path(obs_ctx* ctx, int path);

/* Waits for the stream, then reports (OBS_E_HIP + message) and clears a
 * device-side failure: a bounded wait that timed out in the fused decode
 * path, the fused attention half or the grouped prefill's one-launch expert
 * FFN; OBS_OK otherwise. The reference never checks GPU status. */
int obs_device_status(obs_ctx* ctx);

/* Dispatch facts and the one-launch paths they allow (no reference
 * counterpart: the reference's executor setup, executor.rs:39-58, probes
 * nothing). obs_create runs two small probe kernels: one records the XCD each
 * workgroup of a 256-workgroup grid runs on (the fused kernels keep each
 * group of 32 workgroups, those with one b % 8, inside one XCD's L2, and the
 * 8 groups on 8 XCDs), one checks that each XCD starts its workgroups in index order (the
 * one-launch prefill FFN's down items wait for lower-index gate/up items).
 * obs_dispatch_gate is the pure rule (no device needed): the OBS_PATH_* bits
 * a device with num_cus CUs and those facts may take; the other paths run as
 * separate launches. obs_set_dispatch_facts overrides the probed facts
 * (tests; a caller that knows better). */
enum { OBS_PATH_FUSED_DECODE = 1, OBS_PATH_FUSED_ATTN = 2, OBS_PATH_FFN_ONE_LAUNCH = 4 };
uint32_t obs_dispatch_gate(int num_cus, int xcd_map_ok, int inorder_ok);
int obs_dispatch_info(const obs_ctx* ctx, int* num_cus, int* xcd_map_ok, int* inorder_ok);
int obs_set_dispatch_facts(obs_ctx* ctx, int xcd_map_ok, int inorder_ok);

/* Testing hook (no reference counterpart): makes the one-launch prefill FFN's
 * down items of this context wait for extra_count more counts than their
 * tile's gate/up items give, with a wait limit of wait_us (1..100,000 us), so
 * the bounded wait's time-out report can be exercised from the host: every
 * kernel still exits normally, obs_device_status then reports OBS_E_HIP once
 * and clears the flag. extra_count 0 and wait_us 100000 restore the defaults. */
int obs_debug_ffn_wait(obs_ctx* ctx, uint32_t extra_count, uint32_t wait_us);

/* Workspace bytes obs_moe_prefill needs for T tokens. */
size_t obs_moe_prefill_workspace(const obs_moe_config* cfg, uint32_t T);

/* Grouped prefill MoE for T tokens (forward.rs:164-247): routing either
 * computed from X (ids == NULL: router as obs_q8_gate_logits + obs_route_topk
 * with cfg->route_rule; the routing is left in the workspace, ids int32
 * [T, top_k] at byte 0 and weights fp32 [T, top_k] at byte
 * (4 * T * top_k + 255) / 256 * 256, where read_route reads it, forward.rs:175-182)
 * or injected (ids, weights [T, top_k] device arrays; ids must be in range and
 * distinct per token). Tokens are permuted into per-expert groups on the GPU,
 * gate/up/down run as grouped bf16 MFMA GEMMs (the gathered activation rows
 * staged in LDS; the 4-bit weights dequantized in registers, bf16 =
 * RNE(fp32(q*s + b))) with a SwiGLU epilogue (up to 2,048 row tiles both
 * GEMMs share one launch whose down items wait, bounded, for their tile's
 * gate/up items: obs_device_status of the calling context reports a
 * time-out), and outputs are combined per token in rank order in fp32.
 * X, Y bf16 [T, hidden]; residual (nullable) and layer->norm_w as in
 * obs_moe_decode (the norm runs as one more launch into the workspace).
 * ws: caller-owned device workspace of obs_moe_prefill_workspace() bytes. */
int obs_moe_prefill(obs_ctx* ctx, const obs_moe_config* cfg, const obs_moe_layer* layer,
                    const uint16_t* X, const uint16_t* residual, uint16_t* Y, uint32_t T,
                    const int32_t* ids, const float* weights, void* ws, size_t ws_bytes);

/* ------------------------------------------------------------------ */
/* The rest of a decode step around the MoE block                      */
/* (the attention half of Model::forward_layer, forward.rs:398-419;    */
/*  Model::embed :445-462; run_one_token :552-567)                     */
/* ------------------------------------------------------------------ */
/* Decode steps read their position and token from a device array
 * state = {pos, tok} (int32); obs_argmax writes the next token and advances
 * pos, so one captured graph of a whole step replays for every token.
 * Caches are bf16: keys [n_kv, max_len, head_dim] (kv_cache.rs:3), values
 * transposed [n_kv, head_dim, max_len]. */

/* One 4-bit MLX-affine matrix of a fused mat-vec: rows x in, y = W x in fp32,
 * written as fp32 (y_f32) and/or bf16 (y_bf16 = RNE(residual + W x) when
 * residual is set). Replaces Model::dequant_named (forward.rs:339-343). */
typedef struct obs_gemv_part {
  const uint32_t* w; const uint16_t* scales; const uint16_t* biases; /* [rows, in/8], [rows, in/64] */
  float* y_f32; uint16_t* y_bf16; const uint16_t* residual;
  uint32_t rows;
} obs_gemv_part;
/* y_i = W_i x for 1-3 matrices sharing x (bf16 [in]) in one launch (q, k, v
 * projections; lm_head; o_proj with the residual add of forward.rs:418).
 * With norm_w (bf16 [in], 16-byte aligned) x is first replaced by
 * bf16(rmsnorm(x) * norm_w) with eps, as obs_rmsnorm computes it (the input
 * and final norms of forward.rs:403, :560, fused). in 2048 or 4096, group 64. */
int obs_q4_gemv(obs_ctx* ctx, const uint16_t* x, uint32_t in, uint32_t group, const obs_gemv_part* parts,
                uint32_t n_parts, const uint16_t* norm_w, float eps);

/* Per-head q/k RMSNorm (q_norm/k_norm weights [head_dim], eps), NeoX RoPE at
 * state[0] with rope_theta, q rotated in place, k and v appended to the caches
 * at state[0] (forward.rs:407-416, rope.metal, ops.metal:31-36). q bf16
 * [n_heads, head_dim], k, v bf16 [n_kv, head_dim]. head_dim 128, n_heads a
 * multiple of n_kv (at most 16 per kv head), max_len a multiple of 32; a
 * position outside [0, max_len) appends nothing. */
int obs_attn_prep(obs_ctx* ctx, uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* q_norm,
                  const uint16_t* k_norm, uint16_t* k_cache, uint16_t* v_cache_t, uint32_t n_heads, uint32_t n_kv,
                  uint32_t head_dim, uint32_t max_len, float eps, float theta, const int32_t* state);

/* Workspace bytes of obs_sdpa_decode (0 for an unsupported shape). */
size_t obs_sdpa_workspace(uint32_t n_heads, uint32_t n_kv, uint32_t head_dim, uint32_t max_len);
/* Single-query GQA attention over positions [0, state[0]] (Attention::sdpa,
 * attention.rs:23-41; sdpa_decode.metal): scale 1/sqrt(head_dim), query head h
 * reads kv head h / (n_heads / n_kv). out bf16 [n_heads, head_dim]. */
int obs_sdpa_decode(obs_ctx* ctx, const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache_t, uint16_t* out,
                    uint32_t n_heads, uint32_t n_kv, uint32_t head_dim, uint32_t max_len, const int32_t* state,
                    void* ws, size_t ws_bytes);

/* out = bf16 row state[1] of a 4-bit embedding table [vocab, hidden] (Model::embed,
 * forward.rs:445-462; the token is clamped into [0, vocab)). */
int obs_embed_q4(obs_ctx* ctx, const uint32_t* w, const uint16_t* scales, const uint16_t* biases, uint32_t hidden,
                 uint32_t group, uint32_t vocab, const int32_t* state, uint16_t* out);

/* Greedy token of fp32 logits [n] (forward.rs:563-566: first index of the
 * maximum, NaN never wins, 0 when nothing exceeds -inf) into state[1], then
 * state[0] += 1. ws: obs_argmax_workspace() bytes, 8-byte aligned. */
size_t obs_argmax_workspace(void);
int obs_argmax(obs_ctx* ctx, const float* x, uint32_t n, int32_t* state, void* ws, size_t ws_bytes);

/* The attention half of a decode layer in ONE launch, for the
 * Qwen3-30B-A3B shape (hidden 2048, 32 query heads, 4 kv heads, head_dim 128):
 * x1 = x + o_proj(attention) with q, k, v = projections of rmsnorm(x, in_norm),
 * per-head q/k RMSNorm, NeoX RoPE at state[0], the key and value appended to
 * the caches at state[0] (forward.rs:403-418) — what obs_q4_gemv (q/k/v,
 * fused norm) + obs_attn_prep + obs_sdpa_decode + obs_q4_gemv (o, residual)
 * compute, in one launch of 256 workgroups that exchange values through a
 * context-owned area (allocated on the first call: run one before a graph
 * capture). Needs all 256 CUs; other shapes use the separate calls. x, the
 * weight rows and both caches must be 16-byte aligned (OBS_E_ALIGN). */
typedef struct obs_attn_layer {
  const uint32_t* q_w; const uint16_t* q_s; const uint16_t* q_b;  /* [4096, 2048/8], [4096, 32] */
  const uint32_t* k_w; const uint16_t* k_s; const uint16_t* k_b;  /* [512, ...] */
  const uint32_t* v_w; const uint16_t* v_s; const uint16_t* v_b;  /* [512, ...] */
  const uint32_t* o_w; const uint16_t* o_s; const uint16_t* o_b;  /* [2048, 4096/8], [2048, 64] */
  const uint16_t* in_norm; const uint16_t* q_norm; const uint16_t* k_norm;
} obs_attn_layer;
int obs_attn_decode(obs_ctx* ctx, const obs_attn_layer* layer, const uint16_t* x, uint16_t* k_cache,
                    uint16_t* v_cache_t, uint32_t max_len, float eps, float theta, const int32_t* state,
                    uint16_t* x1);

/* A whole decode layer, Model::forward_layer (forward.rs:398-443), in one
 * launch at the Qwen3-30B-A3B shape: obs_attn_decode (x -> x1, the caches
 * appended at state[0]) and then obs_moe_decode with the layer's
 * post-attention norm (moe->norm_w, required) and x1 as its input and
 * residual (x1 -> y, ids_out / w_out as obs_moe_decode writes them), with the
 * same results bit for bit, without the kernel boundary between the halves.
 * Needs what both calls need (256 CUs, the dispatch obs_create probed, the
 * MoE shape of the fused decode); a context-owned exchange area is allocated
 * on the first call (run one before a graph capture); obs_device_status
 * reports its bounded waits' time-outs. */
int obs_layer_decode(obs_ctx* ctx, const obs_attn_layer* attn, const obs_moe_config* cfg,
                     const obs_moe_layer* moe, const uint16_t* x, uint16_t* k_cache, uint16_t* v_cache_t,
                     uint32_t max_len, float eps, float theta, const int32_t* state, uint16_t* x1,
                     uint16_t* y, int32_t* ids_out, float* w_out);

/* ------------------------------------------------------------------ */
/* Prefill of the layers around the MoE block for a batch of tokens     */
/* (Model::prefill_batched, forward.rs:114-160, :240-261)               */
/* ------------------------------------------------------------------ */
/* out[t] = bf16 row tokens[t] of a 4-bit embedding table (Model::embed per
 * prompt token, forward.rs:136); tokens: device int32 [n_tokens], clamped into
 * [0, vocab); out bf16 [n_tokens, hidden], rows 16-byte aligned. */
int obs_embed_q4_rows(obs_ctx* ctx, const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                      uint32_t hidden, uint32_t group, uint32_t vocab, const int32_t* tokens, uint32_t n_tokens,
                      uint16_t* out);

/* obs_attn_prep for tokens [0, n_tokens) at positions pos0 + t (the per-token
 * q/k norm, RoPE and KV appends of forward.rs:147-153): q bf16 rows of q_ld
 * elements holding [n_heads, head_dim], rotated in place; k, v bf16 rows of
 * kv_ld holding [n_kv, head_dim], appended (q_ld, kv_ld even; 0 = dense rows,
 * so q, k and v may be column ranges of one fused projection's output);
 * pos0 + n_tokens <= max_len. */
int obs_attn_prep_rows(obs_ctx* ctx, uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* q_norm,
                       const uint16_t* k_norm, uint16_t* k_cache, uint16_t* v_cache_t, uint32_t n_heads,
                       uint32_t n_kv, uint32_t head_dim, uint32_t max_len, float eps, float theta, uint32_t pos0,
                       uint32_t n_tokens, uint32_t q_ld, uint32_t kv_ld);

/* Causal GQA attention of a prefill batch (the per-token Attention::sdpa of
 * forward.rs:155 for tokens at positions pos0 + t): token t attends to cache
 * positions [0, pos0 + t]; the batch's keys and values must be in the caches
 * (obs_attn_prep_rows first). q bf16 rows of q_ld elements (a multiple of 8;
 * 0 = dense) holding [n_heads, head_dim]; out bf16 [n_tokens, n_heads,
 * head_dim]; head_dim 128, query heads per kv head a divisor of 16; q, out
 * and both caches 16-byte aligned (OBS_E_ALIGN). */
int obs_sdpa_prefill(obs_ctx* ctx, const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache_t,
                     uint16_t* out, uint32_t n_heads, uint32_t n_kv, uint32_t head_dim, uint32_t max_len,
                     uint32_t pos0, uint32_t n_tokens, uint32_t q_ld);

/* ------------------------------------------------------------------ */
/* Checkpoint loading: safetensors -> HBM-resident expert table        */
/* (replaces Qwen3MoeConfig::from_file model.rs:26-30,                 */
/*  Weights::load_non_expert weight_loader.rs:19-71, ExpertIndex::open */
/*  disk_io.rs:36-63 and read_experts_parallel disk_io.rs:79-102)      */
/* ------------------------------------------------------------------ */

/* safetensors dtypes (the crate's Dtype names, safetensors 0.4.5). */
enum {
  OBS_DT_BOOL = 0, OBS_DT_U8 = 1, OBS_DT_I8 = 2, OBS_DT_F8_E5M2 = 3, OBS_DT_F8_E4M3 = 4,
  OBS_DT_I16 = 5, OBS_DT_U16 = 6, OBS_DT_F16 = 7, OBS_DT_BF16 = 8, OBS_DT_I32 = 9,
  OBS_DT_U32 = 10, OBS_DT_F32 = 11, OBS_DT_F64 = 12, OBS_DT_I64 = 13, OBS_DT_U64 = 14,
};

typedef struct obs_tensor_info {
  int32_t dtype;      /* OBS_DT_* of the bytes on disk */
  uint32_t ndim;
  uint64_t shape[8];
  uint64_t nbytes;    /* bytes on disk (prod(shape) * dtype size) */
  uint32_t n_pieces;  /* 1 for a stored tensor; num_experts when gathered from split files */
} obs_tensor_info;

typedef struct obs_ckpt obs_ckpt;

/* Opens a model directory (host only, no device work): config.json
 * (model.rs:26-30), model.safetensors.index.json's weight_map
 * (weight_loader.rs:20-30) or a single model.safetensors, and the split
 * expert files <expert_dir>/layer_{l}_experts.safetensors
 * (tools/split_experts.py:9-19); expert_dir NULL probes
 * <model_dir>/splitted_moe (main.rs:70-73). Files are opened and their
 * headers validated on first use. On failure *out is NULL and
 * obs_ckpt_error(NULL) holds the message (per thread). */
int obs_ckpt_open(const char* model_dir, const char* expert_dir, obs_ckpt** out);
void obs_ckpt_close(obs_ckpt* ck);
/* Message of the last failed call on ck; ck NULL: of this thread's last failed open. */
const char* obs_ckpt_error(const obs_ckpt* ck);

/* MoE shape from config.json (Qwen3MoeConfig, model.rs:7-23): the reference's
 * required fields must be present; group from quantization.group_size
 * (default 64, as forward.rs:306 fixes it); n_layers may be NULL. */
int obs_ckpt_config(obs_ckpt* ck, obs_moe_config* cfg, uint32_t* n_layers);

/* Describes a tensor. Stacked names model.layers.{l}.mlp.switch_mlp.{proj}.{kind}
 * resolve to the stored stacked tensor, else to the split files' e{N}.{proj}.{kind}
 * gathered in expert order (disk_io.rs:47-55 parses the same names). */
int obs_ckpt_tensor_info(obs_ckpt* ck, const char* name, obs_tensor_info* info);
/* Reads a tensor's on-disk bytes into host memory (bytes >= info.nbytes). */
int obs_ckpt_read(obs_ckpt* ck, const char* name, void* dst_host, size_t bytes);

/* Device bytes of one layer's table as obs_ckpt_load_moe_layer lays it out
 * (13 tensors, each 256-byte aligned); 0 for an unsupported config. */
size_t obs_moe_layer_bytes(const obs_moe_config* cfg);

/* Loads layer `layer`'s expert table into dst_dev (device, 256-byte aligned,
 * >= obs_moe_layer_bytes) and fills *out with pointers into it: the 4-bit
 * switch_mlp tensors [E, ...], the 8-bit router gate mlp.gate [E, H/4] and
 * post_attention_layernorm.weight (out->norm_w NULL if the checkpoint has
 * none). Shapes and dtypes are checked against cfg (U32 weights; BF16 or F16
 * scales, biases and norm; F16 is converted to bf16 on the device, round to
 * nearest even). Reads run on host threads into a pinned ring and are copied
 * to HBM on their own streams; the call returns when the table is resident.
 * Replaces the per-token SSD paging of disk_io.rs:79-102 with a one-time load. */
int obs_ckpt_load_moe_layer(obs_ctx* ctx, obs_ckpt* ck, uint32_t layer, const obs_moe_config* cfg,
                            void* dst_dev, size_t bytes, obs_moe_layer* out);
/* Loads one tensor's on-disk bytes (no conversion) to device memory
 * (weight_loader.rs:61-66 copies each tensor into its own buffer). */
int obs_ckpt_load_tensor(obs_ctx* ctx, obs_ckpt* ck, const char* name, void* dst_dev, size_t bytes);

#ifdef __cplusplus
}
#endif
#endif /* OBSIDIAN_HIP_H */
