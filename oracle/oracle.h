/*
 * oracle.h — CPU restatement of the obsidian MoE expert hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library links, loads or
 * calls this code; only tests/, the smoke check and the CPU-baseline leg of
 * bench.py use it, and only as the checker / the timed CPU path.
 *
 * Reference semantics restated here (paths relative to the reference repo):
 *   - MLX affine q4 format + dequant ........ validate_dequant.py:26-30,
 *                                             shaders/fused_dequant_matvec_4bit.metal:32-51
 *   - 8-bit router gate mat-vec ............. shaders/dequant_matvec_8bit.metal:17-30
 *   - softmax + top-k + renormalise ......... shaders/moe_routing_topk.metal:24-56
 *   - SwiGLU / scaled add ................... shaders/ops.metal:18-29
 *   - RMSNorm (post-attention, router input) . shaders/rmsnorm.metal:17-35, src/forward.rs:419
 *   - decode MoE composition ................ src/forward.rs:421-441
 *   - prefill grouping + rank-order combine . src/forward.rs:200-232
 *   - NeoX RoPE, GQA decode SDPA, argmax .... shaders/rope.metal:12-26,
 *                                             shaders/sdpa_decode.metal:22-47,
 *                                             src/forward.rs:563-566
 *
 * Every function is pinned by a check in tests/ (known-answer vectors,
 * closed forms, brute force on small inputs or invariants); the header of
 * oracle.c lists which.
 *
 * Parity unpinned (relative to the reference itself, not to this file):
 *   - the bf16 rounding of MLX mx.dequantize's output (validate_dequant.py:21):
 *     MLX is absent, so the bf16 value is defined here as one RNE of the exact
 *     fp32 q*s+b;
 *   - Metal fast-math exp and contraction inside the reference shaders: the
 *     routing softmax is restated with an IEEE-style exp (gradual underflow)
 *     and IEEE division on the f16 logits (orc_route_topk's ORC_ROUTE_REF),
 *     not with Metal's own exp.
 */
#ifndef OBSIDIAN_ORACLE_H
#define OBSIDIAN_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- 16-bit float conversions (IEEE round-to-nearest-even) ---- */
float    orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
float    orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
void     orc_bf16_to_f32_n(const uint16_t* in, float* out, int64_t n);
void     orc_f32_to_bf16_n(const float* in, uint16_t* out, int64_t n);

/* scale/bias storage type of a quantized tensor */
enum { ORC_SB_BF16 = 0, ORC_SB_F16 = 1 };

/* ---- dequant (MLX affine): w[r,c] = q[r,c]*scale[r,c/group] + bias[r,c/group] ----
 * bits = 4: element c is nibble c%8 of uint32 word c/8, low bits first.
 * bits = 8: element c is byte   c%4 of uint32 word c/4, low byte first.
 * Output fp32. */
int orc_dequant(int bits, const uint32_t* w, const uint16_t* s, const uint16_t* b, int sb_type,
                float* out, int64_t rows, int64_t cols, int group);

/* ---- mat-vec y = dequant(W) . x ----
 * _shader: one serial fp32 accumulator per output row, column order, the product
 *          rounded before the add (fused_dequant_matvec_4bit.metal:45-48,
 *          dequant_matvec_8bit.metal:27). OpenMP across rows (the CPU baseline).
 * _lanes : the documented fixed order of the HIP router kernel: `lanes` lanes
 *          each own in/lanes contiguous columns, accumulate serially with a
 *          fused multiply-add, then combine by an xor butterfly
 *          (offsets 1, 2, 4, ..., lanes/2, ascending).
 * _f64   : fp64 accumulation of the same fp32 weights (truth), plus
 *          absbound[o] = sum |w*x| for error bounds (may be NULL). */
int orc_qmatvec_shader(int bits, const uint32_t* w, const uint16_t* s, const uint16_t* b, int sb_type,
                       const float* x, float* y, int64_t in, int64_t out, int group);
int orc_qmatvec_lanes(int bits, const uint32_t* w, const uint16_t* s, const uint16_t* b, int sb_type,
                      const float* x, float* y, int64_t in, int64_t out, int group, int lanes);
int orc_qmatvec_f64(int bits, const uint32_t* w, const uint16_t* s, const uint16_t* b, int sb_type,
                    const float* x, double* y, double* absbound, int64_t in, int64_t out, int group);

/* ---- router ---- */
/* deterministic single-precision exp used by the routing softmax
 * (Cody-Waite reduction by ln2, degree-7 Taylor polynomial, explicit fma) */
float orc_exp(float x);

enum { ORC_SUM_SERIAL = 0, ORC_SUM_WAVE = 1 };
/* ORC_ROUTE_REF: the reference's rule — every logit rounded to f16 first (the
 * half output of dequant_matvec_8bit.metal:30, read back as float by
 * moe_routing_topk.metal:24), weights stored as f16: f16(p), renormalised
 * f16(f16(p) / wsum) (moe_routing_topk.metal:47, :55). ORC_ROUTE_F32: no
 * rounding of logits or weights. */
enum { ORC_ROUTE_REF = 0, ORC_ROUTE_F32 = 1 };
/* logits [T, n_exp] fp32 -> ids [T, k] int32, weights [T, k] fp32.
 * Softmax p = e/S with e = orc_exp(l - max); top-k by repeated argmax over p
 * (strict '>', lowest id wins ties); if norm_topk and wsum > 0, w = p / wsum
 * with wsum the serial fp32 sum of the selected (unrounded) p in selection order.
 * sum_order picks the order of S: serial (the reference kernel) or the wave
 * order of the HIP kernel (lane l sums experts l, l+64, l+128, l+192 in that
 * order, then an xor butterfly over 64 lanes with offsets 1, 2, ..., 32).
 * rule: ORC_ROUTE_REF or ORC_ROUTE_F32 (above).
 * A slot with no selectable expert (NaN probabilities) gets id -1, weight 0. */
int orc_route_topk(const float* logits, int64_t T, int n_exp, int k, int norm_topk,
                   int sum_order, int rule, int32_t* ids, float* w);

/* ---- RMSNorm (shaders/rmsnorm.metal:17-35, Model::rmsnorm forward.rs:345-357) ----
 * rows x dim, bf16 in and out. ss = sum of x^2 in the documented lane order
 * (64 lanes each own dim/64 contiguous columns and accumulate x*x serially with
 * fmaf from 0; lanes combined by the xor butterfly with offsets 1, 2, ..., 32);
 * inv = 1 / sqrtf(ss / dim + eps) (IEEE sqrt and division, once per row);
 * out = RNE_bf16((x * inv) * w). (rmsnorm.metal divides each x by rms under
 * Metal fast math; one reciprocal per row is the restated form.)
 * dim % 64 == 0. Returns 0, or -1 on a bad shape. */
int orc_rmsnorm(const uint16_t* x, const uint16_t* w, float eps, int64_t rows, int64_t dim, uint16_t* out);

/* ---- elementwise (ops.metal:18-29) ---- */
float orc_silu_mul(float g, float u);           /* g/(1+exp(-g))*u in fp32 */
void  orc_swiglu(const float* g, const float* u, float* h, int64_t n);
void  orc_scaled_add(float* acc, const float* y, float scale, int64_t n);

/* ---- expert table: stacked [E, ...] tensors of one layer (switch_mlp layout) ---- */
typedef struct {
  int32_t n_exp, hidden, inter, group;
  const uint32_t* gate_w; const uint16_t* gate_s; const uint16_t* gate_b;   /* [E, I, H/8], [E, I, H/G] */
  const uint32_t* up_w;   const uint16_t* up_s;   const uint16_t* up_b;
  const uint32_t* down_w; const uint16_t* down_s; const uint16_t* down_b;   /* [E, H, I/8], [E, H, I/G] */
  const uint32_t* router_w; const uint16_t* router_s; const uint16_t* router_b; /* [E, H/4], [E, H/G] (8-bit) */
} orc_layer;

enum { ORC_MODE_F64 = 0, ORC_MODE_SHADER_F16 = 1, ORC_MODE_MFMA_BF16 = 2 };

/* Router for T tokens: logits in the lanes order (64 lanes) then orc_route_topk
 * with the wave sum order and `rule`. logits_out (fp32, before any f16
 * rounding) may be NULL. */
int orc_router(const orc_layer* L, const uint16_t* x_bf16, int64_t T, int k, int norm_topk, int rule,
               float* logits_out, int32_t* ids, float* w);

/* Decode MoE half for T tokens (forward.rs:421-441 per token): y[t] = sum_rank w*expert(x[t]).
 * ids/w: if ids_in is NULL the router above computes them (written to ids_out/w_out).
 * mode ORC_MODE_F64: fp64 expert math on the exact fp32 weights (truth).
 * mode ORC_MODE_SHADER_F16: the reference engine's rounding sequence (f16 g,u,h,y and
 *   an f16 accumulate per rank, serial fp32 dots).
 * y_out [T, H] fp64 (no residual). */
int orc_moe_decode(const orc_layer* L, const uint16_t* x_bf16, int64_t T, int k, int norm_topk, int rule,
                   const int32_t* ids_in, const float* w_in, int32_t* ids_out, float* w_out,
                   int mode, double* y_out);

/* Prefill grouping (forward.rs:203-204): rows of expert e are the tokens routed to e,
 * in ascending token order. counts [E], offsets [E+1], row_token [T*k],
 * slot_row [T*k] (row index of (token t, rank r) at t*k + r). Returns 0, or -1 on a bad id. */
int orc_group_rows(const int32_t* ids, int64_t T, int k, int n_exp,
                   int32_t* counts, int32_t* offsets, int32_t* row_token, int32_t* slot_row);

/* Grouped prefill MoE (forward.rs:200-232) for X [T, H] with given ids/w [T, k].
 * mode ORC_MODE_F64: fp64 truth. mode ORC_MODE_MFMA_BF16: weights rounded to bf16,
 * fp64 dot accumulation, h and expert outputs rounded to bf16, combine in fp32 in
 * rank order (the operand roundings of the HIP grouped GEMM). y_out [T, H] fp64. */
int orc_moe_prefill(const orc_layer* L, const uint16_t* x_bf16, int64_t T, int k,
                    const int32_t* ids, const float* w, int mode, double* y_out);

/* ---- attention half of a decoder layer (forward.rs:403-419) ---- */

/* NeoX (half-split) rotary embedding at one position, in place on bf16
 * [n_heads, head_dim] (rope.metal:12-26): for i < head_dim/2 the pair
 * (x[i], x[i + head_dim/2]) rotates by angle = fl32(pos * f_i) with
 * f_i = fl32(theta^(-2i/head_dim)) (pow in double, rounded once), c and s =
 * cos and sin of that fp32 angle evaluated in double and rounded once;
 * r0 = x0*c - x1*s, r1 = x1*c + x0*s with each product rounded (no fma), then
 * RNE to bf16. head_dim even. Returns 0, or -1 on a bad shape. */
int orc_rope_neox(uint16_t* x, int64_t n_heads, int64_t head_dim, int64_t pos, float theta);

/* Single-query GQA attention over a cache (sdpa_decode.metal:22-47), fp64
 * truth: query head h reads kv head h / (n_heads / n_kv); scores
 * s_t = scale * q.k_t for t < seq_len, softmax over t, out = sum_t p_t v_t.
 * q bf16 [n_heads, head_dim]; k, v bf16 [n_kv, max_len, head_dim];
 * out fp64 [n_heads, head_dim]. Returns 0, or -1 on a bad shape. */
int orc_sdpa_decode(const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t n_heads, int64_t n_kv,
                    int64_t head_dim, int64_t max_len, int64_t seq_len, double scale, double* out);

/* Greedy token (forward.rs:563-566): the first index whose value is strictly
 * greater than every earlier one, starting from -inf at index 0; NaN never
 * wins. n == 0 or no value above -inf: 0. */
int64_t orc_argmax(const float* x, int64_t n);

/* CPU baseline: the decode MoE half of one token in the reference's shader
 * semantics, OpenMP over output rows (nthreads <= 0: all). Returns 0. */
int orc_moe_decode_baseline(const orc_layer* L, const uint16_t* x_bf16, int k, int norm_topk,
                            int nthreads, int32_t* ids, float* w, float* y);

/* CPU baseline: the router of T tokens in the reference's shader semantics
 * (serial fp32 dot per logit, f16 logits, serial softmax/top-k), OpenMP over
 * tokens (nthreads <= 0: all). Returns 0. */
int orc_router_baseline(const orc_layer* L, const uint16_t* x_bf16, int64_t T, int k, int norm_topk,
                        int nthreads, int32_t* ids, float* w);

/* CPU baseline: the grouped prefill MoE of T tokens with given routing in the
 * shader semantics of matmul_dequant_4bit.metal (serial fp32 dot per (row,
 * output)), rank-order combine into y [T, H] fp32; OpenMP over (token, rank)
 * rows. Returns 0. */
int orc_moe_prefill_baseline(const orc_layer* L, const uint16_t* x_bf16, int64_t T, int k, const int32_t* ids,
                             const float* w, int nthreads, float* y);

int orc_omp_max_threads(void);
/* Threads of the OpenMP loops above (n <= 0: unchanged). */
void orc_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
