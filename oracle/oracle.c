/*
 * oracle.c — CPU restatement of the obsidian MoE expert hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h). Built with -ffp-contract=off so the
 * rounding sequence is exactly the one written here; fused multiply-adds are
 * spelled out with fmaf()/fma() where a documented order uses them.
 *
 * How each function is pinned (tests/test_oracle.py, tests/test_golden.py):
 *   orc_bf16/f16 conversions .... exhaustive round trips over all 65536 patterns,
 *                                 numpy float16 (RNE) on random floats, ties.
 *   orc_dequant ................. known-answer words (0x76543210 -> q 0..7, all-0,
 *                                 all-0xF), group boundaries 63/64, a numpy restatement
 *                                 of validate_dequant.py:26-30 (independent code),
 *                                 committed golden fixtures.
 *   orc_qmatvec_* ............... one-hot x picks a column; fp64 brute force with
 *                                 the bound |y - y64| <= gamma_K * sum|w x|;
 *                                 _lanes with lanes=1 equals the serial fma loop.
 *   orc_exp ..................... against libm expf/exp (<= 2 ulp on a dense grid),
 *                                 exp(0) = 1 exactly, monotone on the grid.
 *   orc_route_topk .............. brute force on tiny cases (sort by (-p, id)),
 *                                 forced ties -> lowest id, permutation of logits
 *                                 permutes ids, renormalised weights sum to 1,
 *                                 closed form w_i = e_i / sum_sel e_j.
 *   orc_rmsnorm ................. closed form for a constant row (x = c, w = 1:
 *                                 ss = dim c^2 exactly, out = bf16(c * (1 / sqrtf(c^2 + eps)))),
 *                                 exact invariance under x -> 2x when eps = 0, an fp64
 *                                 numpy restatement within one bf16 step, and the
 *                                 butterfly order equal to a serial sum where exact.
 *   orc_moe_decode / _prefill ... one-hot routing weight reproduces one expert;
 *                                 prefill with T=1 equals decode; linearity in the
 *                                 routing weights; grouping invariants.
 *   orc_rope_neox ............... pos 0 is the identity bit for bit; the complex
 *                                 rotation (x0 + i x1) e^{i pos f_i} in numpy fp64
 *                                 within one bf16 step; pair norms preserved; pair
 *                                 i = 0 turns by exactly pos radians.
 *   orc_sdpa_decode ............. one position returns v; equal keys return the
 *                                 mean of v; a dominant score returns its v; the
 *                                 GQA head map (kv head h / (n_heads / n_kv)) seen
 *                                 through distinct kv heads; a numpy restatement.
 *   orc_argmax .................. ties -> first index, NaN skipped, all -inf -> 0,
 *                                 numpy argmax where no NaN.
 *   attention_half (oracle.py) .. against an fp64 restatement of forward.rs:403-418
 *                                 written from the reference (own dequant, norms,
 *                                 RoPE, attention); the restatement with the RoPE
 *                                 before the q/k norms or with the append after the
 *                                 attention lands far outside the tolerance.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------- */
/* 16-bit floats                                                              */
/* ------------------------------------------------------------------------- */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t orc_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u); /* quiet NaN */
  u += 0x7fffu + ((u >> 16) & 1u);                                                 /* RNE */
  return (uint16_t)(u >> 16);
}

float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
  if (exp == 0x1f) return u2f(sign | 0x7f800000u | (man << 13));
  if (exp == 0) {
    if (man == 0) return u2f(sign);
    /* subnormal: value = man * 2^-24 (exact in fp32) */
    float v = (float)man * 5.9604644775390625e-08f;
    return (sign ? -v : v);
  }
  return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t orc_f32_to_f16(float f) {
  uint32_t u = f2u(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t au = u & 0x7fffffffu;
  if (au > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((au >> 13) & 0x3ffu));
  if (au >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
  if (au < 0x38800000u) {
    /* result is f16-subnormal or zero: round |f| / 2^-24 to an integer, RNE */
    float a = u2f(au) * 16777216.0f; /* exact scaling by 2^24 */
    float r = rintf(a);              /* default rounding mode: nearest-even */
    return (uint16_t)(sign | (uint16_t)r);
  }
  /* normal: drop 13 mantissa bits with RNE (carry may bump the exponent) */
  uint32_t v = au - (112u << 23);
  v += 0xfffu + ((v >> 13) & 1u);
  return (uint16_t)(sign | (uint16_t)(v >> 13));
}

void orc_bf16_to_f32_n(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16_to_f32(in[i]);
}
void orc_f32_to_bf16_n(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16(in[i]);
}

static inline float sb_to_f32(uint16_t v, int sb_type) {
  return sb_type == ORC_SB_F16 ? orc_f16_to_f32(v) : orc_bf16_to_f32(v);
}

/* ------------------------------------------------------------------------- */
/* dequant                                                                    */
/* ------------------------------------------------------------------------- */

/* Element c of a row: nibble c%8 of word c/8 (4-bit) or byte c%4 of word c/4
 * (8-bit), low bits first — validate_dequant.py:26-29 and
 * fused_dequant_matvec_4bit.metal:39-42 (byte view, little-endian). */
static inline uint32_t q_at(int bits, const uint32_t* row, int64_t c) {
  if (bits == 4) return (row[c >> 3] >> (4u * (uint32_t)(c & 7))) & 0xfu;
  return (row[c >> 2] >> (8u * (uint32_t)(c & 3))) & 0xffu;
}

/* w = q*scale + bias in fp32. q*scale is exact (<= 8 bits x 11 bits), so this
 * equals the fma form used by the shaders: one rounding, at the add. */
static inline float dq(uint32_t q, float sc, float bi) { return (float)q * sc + bi; }

static int check_shape(int bits, int64_t in, int group) {
  if (bits != 4 && bits != 8) return -1;
  if (group <= 0 || in <= 0 || in % group != 0) return -2;
  if (in % (32 / bits) != 0) return -3;
  return 0;
}

int orc_dequant(int bits, const uint32_t* w, const uint16_t* s, const uint16_t* b, int sb_type,
                float* out, int64_t rows, int64_t cols, int group) {
  int rc = check_shape(bits, cols, group);
  if (rc) return rc;
  const int64_t words = cols * bits / 32, groups = cols / group;
  for (int64_t r = 0; r < rows; ++r) {
    const uint32_t* wr = w + r * words;
    for (int64_t c = 0; c < cols; ++c) {
      const int64_t g = r * groups + c / group;
      out[r * cols + c] = dq(q_at(bits, wr, c), sb_to_f32(s[g], sb_type), sb_to_f32(b[g], sb_type));
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------- */
/* mat-vec                                                                    */
/* ------------------------------------------------------------------------- */

/* Reference shader order: acc += fl(w*x), columns 0..in-1
 * (fused_dequant_matvec_4bit.metal:29-52: `acc += fma(w, x, 0.0f)`). */
static float row_dot_shader(int bits, const uint32_t* wr, const uint16_t* sr, const uint16_t* br,
                            int sb_type, const float* x, int64_t in, int group) {
  float acc = 0.0f;
  for (int64_t g = 0; g < in / group; ++g) {
    const float sc = sb_to_f32(sr[g], sb_type), bi = sb_to_f32(br[g], sb_type);
    for (int64_t j = 0; j < group; ++j) {
      const int64_t c = g * group + j;
      const float prod = dq(q_at(bits, wr, c), sc, bi) * x[c];
      acc = acc + prod;
    }
  }
  return acc;
}

int orc_qmatvec_shader(int bits, const uint32_t* w, const uint16_t* s, const uint16_t* b, int sb_type,
                       const float* x, float* y, int64_t in, int64_t out, int group) {
  int rc = check_shape(bits, in, group);
  if (rc) return rc;
  const int64_t words = in * bits / 32, groups = in / group;
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < out; ++o)
    y[o] = row_dot_shader(bits, w + o * words, s + o * groups, b + o * groups, sb_type, x, in, group);
  return 0;
}

/* The documented lane order: lane l owns columns [l*in/L, (l+1)*in/L), serial
 * fmaf accumulation; lanes combined by an xor butterfly with offsets 1, 2, ..., L/2
 * (every lane ends with the same value; lane 0's is returned). */
static float row_dot_lanes(int bits, const uint32_t* wr, const uint16_t* sr, const uint16_t* br,
                           int sb_type, const float* x, int64_t in, int group, int lanes) {
  float part[256];
  const int64_t chunk = in / lanes;
  for (int l = 0; l < lanes; ++l) {
    float acc = 0.0f;
    for (int64_t c = l * chunk; c < (l + 1) * chunk; ++c) {
      const int64_t g = c / group;
      const float wv = dq(q_at(bits, wr, c), sb_to_f32(sr[g], sb_type), sb_to_f32(br[g], sb_type));
      acc = fmaf(wv, x[c], acc);
    }
    part[l] = acc;
  }
  for (int off = 1; off < lanes; off <<= 1) {
    float nxt[256];
    for (int l = 0; l < lanes; ++l) nxt[l] = part[l] + part[l ^ off];
    memcpy(part, nxt, sizeof(float) * (size_t)lanes);
  }
  return part[0];
}

int orc_qmatvec_lanes(int bits, const uint32_t* w, const uint16_t* s, const uint16_t* b, int sb_type,
                      const float* x, float* y, int64_t in, int64_t out, int group, int lanes) {
  int rc = check_shape(bits, in, group);
  if (rc) return rc;
  if (lanes < 1 || lanes > 256 || (lanes & (lanes - 1)) || in % lanes) return -4;
  const int64_t words = in * bits / 32, groups = in / group;
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < out; ++o)
    y[o] = row_dot_lanes(bits, w + o * words, s + o * groups, b + o * groups, sb_type, x, in, group, lanes);
  return 0;
}

int orc_qmatvec_f64(int bits, const uint32_t* w, const uint16_t* s, const uint16_t* b, int sb_type,
                    const float* x, double* y, double* absbound, int64_t in, int64_t out, int group) {
  int rc = check_shape(bits, in, group);
  if (rc) return rc;
  const int64_t words = in * bits / 32, groups = in / group;
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < out; ++o) {
    const uint32_t* wr = w + o * words;
    double acc = 0.0, ab = 0.0;
    for (int64_t c = 0; c < in; ++c) {
      const int64_t g = o * groups + c / group;
      const double t = (double)dq(q_at(bits, wr, c), sb_to_f32(s[g], sb_type), sb_to_f32(b[g], sb_type)) * (double)x[c];
      acc += t;
      ab += fabs(t);
    }
    y[o] = acc;
    if (absbound) absbound[o] = ab;
  }
  return 0;
}

/* ------------------------------------------------------------------------- */
/* router                                                                     */
/* ------------------------------------------------------------------------- */

/* exp(x) for the routing softmax and SwiGLU, written from the textbook method:
 *   n = rint(x * log2(e)),  r = x - n*ln2 (Cody-Waite: ln2 = hi + lo, each
 *   step one fma), exp(r) by the degree-7 Taylor polynomial in Horner form
 *   (|r| <= ln2/2, truncation < 6e-9 relative), result = p * 2^n.
 * Below the normal range the result underflows gradually, as IEEE exp does:
 * p * 2^n is formed as (p * 2^(n+64)) * 2^-64 (the first product exact, the
 * second one rounding into the subnormals).
 * Domain conventions: x < -104 -> +0 (exp(-104) is below half the smallest
 * subnormal), x > 88.5 -> +inf, NaN -> NaN. Both the HIP kernels and this
 * oracle evaluate exactly these operations, so their results are bit-identical. */
float orc_exp(float x) {
  if (x != x) return x;
  if (x < -104.0f) return 0.0f;
  if (x > 88.5f) return INFINITY;
  const float LOG2E = 1.44269502162933349609375f;   /* fl32(1/ln 2) */
  const float LN2_HI = 0.693145751953125f;           /* ln2 rounded to 16 significant bits */
  const float LN2_LO = 1.428606765330187045e-06f;    /* fl32(ln2 - LN2_HI) */
  const float n = rintf(x * LOG2E);
  float r = fmaf(-n, LN2_HI, x);
  r = fmaf(-n, LN2_LO, r);
  float p = 1.98412698e-04f;                 /* 1/7! */
  p = fmaf(p, r, 1.38888889e-03f);           /* 1/6! */
  p = fmaf(p, r, 8.33333333e-03f);           /* 1/5! */
  p = fmaf(p, r, 4.16666667e-02f);           /* 1/4! */
  p = fmaf(p, r, 1.66666667e-01f);           /* 1/3! */
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int ni = (int)n;
  if (ni > 127) { p = p * 2.0f; ni -= 1; }
  if (ni < -126) return (p * u2f((uint32_t)(ni + 64 + 127) << 23)) * 0x1p-64f;
  return p * u2f((uint32_t)(ni + 127) << 23);
}

static inline float round_f16(float v) { return orc_f16_to_f32(orc_f32_to_f16(v)); }

/* moe_routing_topk.metal:24-56 for one token. Under ORC_ROUTE_REF the logits
 * are the f16 values dequant_matvec_8bit.metal:30 stores (each rounded RNE),
 * and the weights are stored as f16 (:47, :55). */
static void route_one(const float* l_in, int n, int k, int norm_topk, int sum_order, int rule,
                      int32_t* ids, float* w) {
  float p[1024], l[1024];
  const int f16 = (rule == ORC_ROUTE_REF);
  for (int i = 0; i < n; ++i) l[i] = f16 ? round_f16(l_in[i]) : l_in[i];
  float mx = -INFINITY;
  for (int i = 0; i < n; ++i) mx = fmaxf(mx, l[i]);
  for (int i = 0; i < n; ++i) p[i] = orc_exp(l[i] - mx);
  float sum = 0.0f;
  if (sum_order == ORC_SUM_SERIAL) {
    for (int i = 0; i < n; ++i) sum = sum + p[i];
  } else {
    float part[64];
    for (int ln = 0; ln < 64; ++ln) {
      float a = 0.0f;
      for (int j = ln; j < n; j += 64) a = a + p[j];
      part[ln] = a;
    }
    for (int off = 1; off < 64; off <<= 1) {
      float nxt[64];
      for (int ln = 0; ln < 64; ++ln) nxt[ln] = part[ln] + part[ln ^ off];
      memcpy(part, nxt, sizeof part);
    }
    sum = part[0];
  }
  for (int i = 0; i < n; ++i) p[i] = p[i] / sum;
  float wsum = 0.0f;
  for (int kk = 0; kk < k; ++kk) {
    float best = -INFINITY;
    int bi = -1;
    for (int i = 0; i < n; ++i)
      if (p[i] > best) { best = p[i]; bi = i; }
    if (bi < 0) { ids[kk] = -1; w[kk] = 0.0f; continue; }
    ids[kk] = bi;
    w[kk] = f16 ? round_f16(best) : best;
    wsum = wsum + best;
    p[bi] = -INFINITY;
  }
  if (norm_topk && wsum > 0.0f) {
    for (int kk = 0; kk < k; ++kk) {
      if (ids[kk] < 0) continue;
      const float q = w[kk] / wsum;
      w[kk] = f16 ? round_f16(q) : q;
    }
  }
}

int orc_route_topk(const float* logits, int64_t T, int n_exp, int k, int norm_topk,
                   int sum_order, int rule, int32_t* ids, float* w) {
  if (n_exp < 1 || n_exp > 256 || k < 1 || k > n_exp) return -1;
  if (sum_order != ORC_SUM_SERIAL && sum_order != ORC_SUM_WAVE) return -2;
  if (rule != ORC_ROUTE_REF && rule != ORC_ROUTE_F32) return -3;
  for (int64_t t = 0; t < T; ++t)
    route_one(logits + t * n_exp, n_exp, k, norm_topk, sum_order, rule, ids + t * k, w + t * k);
  return 0;
}

/* ------------------------------------------------------------------------- */
/* elementwise                                                                */
/* ------------------------------------------------------------------------- */

/* ops.metal:21: silu(g)*u = (g / (1 + exp(-g))) * u */
int orc_rmsnorm(const uint16_t* x, const uint16_t* w, float eps, int64_t rows, int64_t dim, uint16_t* out) {
  if (dim <= 0 || dim % 64 != 0 || rows < 0) return -1;
  const int64_t chunk = dim / 64;
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* xr = x + r * dim;
    float part[64];
    for (int l = 0; l < 64; ++l) {
      float acc = 0.0f;
      for (int64_t c = l * chunk; c < (l + 1) * chunk; ++c) {
        const float v = orc_bf16_to_f32(xr[c]);
        acc = fmaf(v, v, acc);
      }
      part[l] = acc;
    }
    for (int off = 1; off < 64; off <<= 1) {
      float nxt[64];
      for (int l = 0; l < 64; ++l) nxt[l] = part[l] + part[l ^ off];
      memcpy(part, nxt, sizeof(nxt));
    }
    const float inv = 1.0f / sqrtf(part[0] / (float)dim + eps);
    for (int64_t c = 0; c < dim; ++c)
      out[r * dim + c] = orc_f32_to_bf16((orc_bf16_to_f32(xr[c]) * inv) * orc_bf16_to_f32(w[c]));
  }
  return 0;
}

float orc_silu_mul(float g, float u) { return (g / (1.0f + orc_exp(-g))) * u; }

void orc_swiglu(const float* g, const float* u, float* h, int64_t n) {
  for (int64_t i = 0; i < n; ++i) h[i] = orc_silu_mul(g[i], u[i]);
}

/* ops.metal:28: acc = acc + scale*y */
void orc_scaled_add(float* acc, const float* y, float scale, int64_t n) {
  for (int64_t i = 0; i < n; ++i) acc[i] = acc[i] + scale * y[i];
}

/* ------------------------------------------------------------------------- */
/* layer compositions                                                         */
/* ------------------------------------------------------------------------- */

static inline double silu_mul_d(double g, double u) { return g / (1.0 + exp(-g)) * u; }

int orc_router(const orc_layer* L, const uint16_t* x_bf16, int64_t T, int k, int norm_topk, int rule,
               float* logits_out, int32_t* ids, float* w) {
  const int E = L->n_exp, H = L->hidden;
  float* x = (float*)malloc(sizeof(float) * (size_t)H);
  float* lg = (float*)malloc(sizeof(float) * (size_t)E * (size_t)T);
  int rc = 0;
  for (int64_t t = 0; t < T && !rc; ++t) {
    orc_bf16_to_f32_n(x_bf16 + t * H, x, H);
    rc = orc_qmatvec_lanes(8, L->router_w, L->router_s, L->router_b, ORC_SB_BF16, x, lg + t * E, H, E, L->group, 64);
  }
  if (!rc) rc = orc_route_topk(lg, T, E, k, norm_topk, ORC_SUM_WAVE, rule, ids, w);
  if (!rc && logits_out) memcpy(logits_out, lg, sizeof(float) * (size_t)E * (size_t)T);
  free(x);
  free(lg);
  return rc;
}

/* One expert's FFN in fp64 on the exact fp32 weights: y = Wd (silu(Wg x) * (Wu x)). */
static void expert_f64(const orc_layer* L, int e, const float* x, double* y) {
  const int H = L->hidden, I = L->inter, G = L->group;
  const size_t gw = (size_t)I * H / 8, gs = (size_t)I * H / G, dw = (size_t)H * I / 8, ds = (size_t)H * I / G;
  double* g = (double*)malloc(sizeof(double) * I);
  double* u = (double*)malloc(sizeof(double) * I);
  float* h = (float*)malloc(sizeof(float) * I);
  double* hd = (double*)malloc(sizeof(double) * I);
  orc_qmatvec_f64(4, L->gate_w + e * gw, L->gate_s + e * gs, L->gate_b + e * gs, ORC_SB_BF16, x, g, NULL, H, I, G);
  orc_qmatvec_f64(4, L->up_w + e * gw, L->up_s + e * gs, L->up_b + e * gs, ORC_SB_BF16, x, u, NULL, H, I, G);
  for (int i = 0; i < I; ++i) hd[i] = silu_mul_d(g[i], u[i]);
  /* down projection on the fp64 h: accumulate exactly in fp64 */
  const uint32_t* W = L->down_w + e * dw;
  const uint16_t* S = L->down_s + e * ds;
  const uint16_t* B = L->down_b + e * ds;
  for (int o = 0; o < H; ++o) {
    double acc = 0.0;
    for (int c = 0; c < I; ++c) {
      const int64_t gi = (int64_t)o * (I / G) + c / G;
      const float wv = dq(q_at(4, W + (size_t)o * (I / 8), c), orc_bf16_to_f32(S[gi]), orc_bf16_to_f32(B[gi]));
      acc += (double)wv * hd[c];
    }
    y[o] = acc;
  }
  (void)h;
  free(g); free(u); free(h); free(hd);
}

/* One expert in the reference engine's rounding sequence (forward.rs:436-440):
 * g,u = f16(serial fp32 dot); h = f16(silu(g)*u); y = f16(serial fp32 dot). */
static void expert_shader_f16(const orc_layer* L, int e, const float* x, float* y) {
  const int H = L->hidden, I = L->inter, G = L->group;
  const size_t gw = (size_t)I * H / 8, gs = (size_t)I * H / G, dw = (size_t)H * I / 8, ds = (size_t)H * I / G;
  float* g = (float*)malloc(sizeof(float) * I);
  float* u = (float*)malloc(sizeof(float) * I);
  float* h = (float*)malloc(sizeof(float) * I);
  orc_qmatvec_shader(4, L->gate_w + e * gw, L->gate_s + e * gs, L->gate_b + e * gs, ORC_SB_BF16, x, g, H, I, G);
  orc_qmatvec_shader(4, L->up_w + e * gw, L->up_s + e * gs, L->up_b + e * gs, ORC_SB_BF16, x, u, H, I, G);
  for (int i = 0; i < I; ++i) {
    const float gf = orc_f16_to_f32(orc_f32_to_f16(g[i])), uf = orc_f16_to_f32(orc_f32_to_f16(u[i]));
    h[i] = orc_f16_to_f32(orc_f32_to_f16(orc_silu_mul(gf, uf)));
  }
  orc_qmatvec_shader(4, L->down_w + e * dw, L->down_s + e * ds, L->down_b + e * ds, ORC_SB_BF16, h, y, I, H, G);
  for (int o = 0; o < H; ++o) y[o] = orc_f16_to_f32(orc_f32_to_f16(y[o]));
  free(g); free(u); free(h);
}

int orc_moe_decode(const orc_layer* L, const uint16_t* x_bf16, int64_t T, int k, int norm_topk, int rule,
                   const int32_t* ids_in, const float* w_in, int32_t* ids_out, float* w_out,
                   int mode, double* y_out) {
  const int H = L->hidden, E = L->n_exp;
  if (mode != ORC_MODE_F64 && mode != ORC_MODE_SHADER_F16) return -1;
  const int32_t* ids = ids_in;
  const float* w = w_in;
  if (!ids_in) {
    int rc = orc_router(L, x_bf16, T, k, norm_topk, rule, NULL, ids_out, w_out);
    if (rc) return rc;
    ids = ids_out;
    w = w_out;
  }
  float* x = (float*)malloc(sizeof(float) * H);
  double* yd = (double*)malloc(sizeof(double) * H);
  float* yf = (float*)malloc(sizeof(float) * H);
  float* acc = (float*)malloc(sizeof(float) * H);
  for (int64_t t = 0; t < T; ++t) {
    orc_bf16_to_f32_n(x_bf16 + t * H, x, H);
    double* out = y_out + t * H;
    for (int o = 0; o < H; ++o) { out[o] = 0.0; acc[o] = 0.0f; }
    for (int r = 0; r < k; ++r) {
      const int e = ids[t * k + r];
      if (e < 0 || e >= E) continue;
      const float wr = w[t * k + r];
      if (mode == ORC_MODE_F64) {
        expert_f64(L, e, x, yd);
        for (int o = 0; o < H; ++o) out[o] += (double)wr * yd[o];
      } else {
        expert_shader_f16(L, e, x, yf);
        /* ew_scaled_add into an f16 accumulator, ranks in order (forward.rs:440) */
        for (int o = 0; o < H; ++o) acc[o] = orc_f16_to_f32(orc_f32_to_f16(acc[o] + wr * yf[o]));
      }
    }
    if (mode == ORC_MODE_SHADER_F16)
      for (int o = 0; o < H; ++o) out[o] = acc[o];
  }
  free(x); free(yd); free(yf); free(acc);
  return 0;
}

int orc_group_rows(const int32_t* ids, int64_t T, int k, int n_exp,
                   int32_t* counts, int32_t* offsets, int32_t* row_token, int32_t* slot_row) {
  for (int e = 0; e < n_exp; ++e) counts[e] = 0;
  for (int64_t i = 0; i < T * k; ++i) {
    if (ids[i] < 0 || ids[i] >= n_exp) return -1;
    counts[ids[i]]++;
  }
  offsets[0] = 0;
  for (int e = 0; e < n_exp; ++e) offsets[e + 1] = offsets[e] + counts[e];
  int32_t* fill = (int32_t*)calloc((size_t)n_exp, sizeof(int32_t));
  /* tokens in ascending order within each expert (forward.rs:203-204) */
  for (int64_t t = 0; t < T; ++t)
    for (int r = 0; r < k; ++r) {
      const int e = ids[t * k + r];
      const int row = offsets[e] + fill[e]++;
      row_token[row] = (int32_t)t;
      slot_row[t * k + r] = row;
    }
  free(fill);
  return 0;
}

int orc_moe_prefill(const orc_layer* L, const uint16_t* x_bf16, int64_t T, int k,
                    const int32_t* ids, const float* w, int mode, double* y_out) {
  const int H = L->hidden, I = L->inter, E = L->n_exp, G = L->group;
  if (mode != ORC_MODE_F64 && mode != ORC_MODE_MFMA_BF16) return -1;
  const size_t gw = (size_t)I * H / 8, gs = (size_t)I * H / G, dw = (size_t)H * I / 8, ds = (size_t)H * I / G;
  int32_t* counts = (int32_t*)malloc(sizeof(int32_t) * E);
  int32_t* offsets = (int32_t*)malloc(sizeof(int32_t) * (E + 1));
  int32_t* row_token = (int32_t*)malloc(sizeof(int32_t) * (size_t)(T * k));
  int32_t* slot_row = (int32_t*)malloc(sizeof(int32_t) * (size_t)(T * k));
  if (orc_group_rows(ids, T, k, E, counts, offsets, row_token, slot_row)) {
    free(counts); free(offsets); free(row_token); free(slot_row);
    return -2;
  }
  const int64_t R = T * k;
  /* per-row expert outputs [R, H] */
  double* Y = (double*)malloc(sizeof(double) * (size_t)R * H);
  const int bf = (mode == ORC_MODE_MFMA_BF16);
  /* one expert at a time per thread: dequantize its three matrices once
   * (bf16-rounded in MFMA mode), then run all of its rows */
#pragma omp parallel
  {
    float* Wg = (float*)malloc(sizeof(float) * (size_t)I * H);
    float* Wu = (float*)malloc(sizeof(float) * (size_t)I * H);
    float* Wd = (float*)malloc(sizeof(float) * (size_t)H * I);
    float* x = (float*)malloc(sizeof(float) * H);
    double* h = (double*)malloc(sizeof(double) * I);
#pragma omp for schedule(dynamic, 1)
    for (int e = 0; e < E; ++e) {
      if (counts[e] == 0) continue;
      orc_dequant(4, L->gate_w + e * gw, L->gate_s + e * gs, L->gate_b + e * gs, ORC_SB_BF16, Wg, I, H, G);
      orc_dequant(4, L->up_w + e * gw, L->up_s + e * gs, L->up_b + e * gs, ORC_SB_BF16, Wu, I, H, G);
      orc_dequant(4, L->down_w + e * dw, L->down_s + e * ds, L->down_b + e * ds, ORC_SB_BF16, Wd, H, I, G);
      if (bf) {
        for (size_t i = 0; i < (size_t)I * H; ++i) {
          Wg[i] = orc_bf16_to_f32(orc_f32_to_bf16(Wg[i]));
          Wu[i] = orc_bf16_to_f32(orc_f32_to_bf16(Wu[i]));
          Wd[i] = orc_bf16_to_f32(orc_f32_to_bf16(Wd[i]));
        }
      }
      for (int64_t row = offsets[e]; row < offsets[e + 1]; ++row) {
        const int64_t t = row_token[row];
        orc_bf16_to_f32_n(x_bf16 + t * H, x, H);
        for (int i = 0; i < I; ++i) {
          double g = 0.0, u = 0.0;
          const float* wg = Wg + (size_t)i * H;
          const float* wu = Wu + (size_t)i * H;
          for (int c = 0; c < H; ++c) {
            g += (double)wg[c] * (double)x[c];
            u += (double)wu[c] * (double)x[c];
          }
          if (bf)
            h[i] = (double)orc_bf16_to_f32(orc_f32_to_bf16(orc_silu_mul((float)g, (float)u)));
          else
            h[i] = silu_mul_d(g, u);
        }
        for (int o = 0; o < H; ++o) {
          const float* wd = Wd + (size_t)o * I;
          double acc = 0.0;
          for (int c = 0; c < I; ++c) acc += (double)wd[c] * h[c];
          Y[row * H + o] = bf ? (double)orc_bf16_to_f32(orc_f32_to_bf16((float)acc)) : acc;
        }
      }
    }
    free(Wg); free(Wu); free(Wd); free(x); free(h);
  }
  /* un-permute and combine in rank order (forward.rs:225-232) */
  for (int64_t t = 0; t < T; ++t) {
    for (int o = 0; o < H; ++o) {
      if (bf) {
        float acc = 0.0f;
        for (int r = 0; r < k; ++r) acc = fmaf(w[t * k + r], (float)Y[(int64_t)slot_row[t * k + r] * H + o], acc);
        y_out[t * H + o] = acc;
      } else {
        double acc = 0.0;
        for (int r = 0; r < k; ++r) acc += (double)w[t * k + r] * Y[(int64_t)slot_row[t * k + r] * H + o];
        y_out[t * H + o] = acc;
      }
    }
  }
  free(Y); free(counts); free(offsets); free(row_token); free(slot_row);
  return 0;
}

/* ------------------------------------------------------------------------- */
/* CPU baseline: decode MoE half of one token, reference shader semantics    */
/* ------------------------------------------------------------------------- */

int orc_moe_decode_baseline(const orc_layer* L, const uint16_t* x_bf16, int k, int norm_topk,
                            int nthreads, int32_t* ids, float* w, float* y) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
  const int H = L->hidden, I = L->inter, E = L->n_exp, G = L->group;
  const size_t gw = (size_t)I * H / 8, gs = (size_t)I * H / G, dw = (size_t)H * I / 8, ds = (size_t)H * I / G;
  float x[8192], lg[256], g[4096], u[4096], h[4096], ye[8192];
  if (H > 8192 || I > 4096 || E > 256) return -1;
  orc_bf16_to_f32_n(x_bf16, x, H);
  /* dequant_matvec_8bit (serial per row, f16 logits) then moe_routing_topk */
  orc_qmatvec_shader(8, L->router_w, L->router_s, L->router_b, ORC_SB_BF16, x, lg, H, E, G);
  orc_route_topk(lg, 1, E, k, norm_topk, ORC_SUM_SERIAL, ORC_ROUTE_REF, ids, w);
  for (int o = 0; o < H; ++o) y[o] = 0.0f;
  for (int r = 0; r < k; ++r) {
    const int e = ids[r];
    if (e < 0) continue;
    orc_qmatvec_shader(4, L->gate_w + e * gw, L->gate_s + e * gs, L->gate_b + e * gs, ORC_SB_BF16, x, g, H, I, G);
    orc_qmatvec_shader(4, L->up_w + e * gw, L->up_s + e * gs, L->up_b + e * gs, ORC_SB_BF16, x, u, H, I, G);
    orc_swiglu(g, u, h, I);
    orc_qmatvec_shader(4, L->down_w + e * dw, L->down_s + e * ds, L->down_b + e * ds, ORC_SB_BF16, h, ye, I, H, G);
    orc_scaled_add(y, ye, w[r], H);
  }
  return 0;
}

/* CPU baseline, router of T tokens (dequant_matvec_8bit.metal: one serial
 * fp32 dot per logit, rounded to f16; moe_routing_topk.metal on those halves),
 * OpenMP over tokens. */
int orc_router_baseline(const orc_layer* L, const uint16_t* x_bf16, int64_t T, int k, int norm_topk,
                        int nthreads, int32_t* ids, float* w) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
  const int H = L->hidden, E = L->n_exp, G = L->group;
  if (H > 8192 || E > 256) return -1;
  const int64_t words = H / 4, groups = H / G;
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < T; ++t) {
    float x[8192], lg[256];
    orc_bf16_to_f32_n(x_bf16 + t * H, x, H);
    for (int e = 0; e < E; ++e)
      lg[e] = row_dot_shader(8, L->router_w + e * words, L->router_s + e * groups, L->router_b + e * groups,
                             ORC_SB_BF16, x, H, G);
    route_one(lg, E, k, norm_topk, ORC_SUM_SERIAL, ORC_ROUTE_REF, ids + t * k, w + t * k);
  }
  return 0;
}

/* CPU baseline, grouped prefill MoE (forward.rs:200-232 with
 * matmul_dequant_4bit.metal: one serial fp32 dot per (row, output), the same
 * order as the mat-vec), for T tokens with given routing: gate and up, SwiGLU,
 * down, then the rank-order combine into y [T, H] (fp32). OpenMP over the
 * (token, rank) rows. */
int orc_moe_prefill_baseline(const orc_layer* L, const uint16_t* x_bf16, int64_t T, int k, const int32_t* ids,
                             const float* w, int nthreads, float* y) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
  const int H = L->hidden, I = L->inter, E = L->n_exp, G = L->group;
  if (H > 8192 || I > 4096) return -1;
  const size_t gw = (size_t)I * H / 8, gs = (size_t)I * H / G, dw = (size_t)H * I / 8, ds = (size_t)H * I / G;
  float* ye = (float*)malloc(sizeof(float) * (size_t)T * k * H);
  if (!ye) return -2;
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t row = 0; row < T * k; ++row) {
    float x[8192], g[4096], u[4096], h[4096];
    const int e = ids[row];
    float* out = ye + row * H;
    if (e < 0 || e >= E) {
      for (int o = 0; o < H; ++o) out[o] = 0.0f;
      continue;
    }
    orc_bf16_to_f32_n(x_bf16 + (row / k) * H, x, H);
    for (int i = 0; i < I; ++i) {
      g[i] = row_dot_shader(4, L->gate_w + e * gw + (size_t)i * (H / 8), L->gate_s + e * gs + (size_t)i * (H / G),
                            L->gate_b + e * gs + (size_t)i * (H / G), ORC_SB_BF16, x, H, G);
      u[i] = row_dot_shader(4, L->up_w + e * gw + (size_t)i * (H / 8), L->up_s + e * gs + (size_t)i * (H / G),
                            L->up_b + e * gs + (size_t)i * (H / G), ORC_SB_BF16, x, H, G);
    }
    orc_swiglu(g, u, h, I);
    for (int o = 0; o < H; ++o)
      out[o] = row_dot_shader(4, L->down_w + e * dw + (size_t)o * (I / 8), L->down_s + e * ds + (size_t)o * (I / G),
                              L->down_b + e * ds + (size_t)o * (I / G), ORC_SB_BF16, h, I, G);
  }
  for (int64_t t = 0; t < T; ++t) {
    float* yt = y + t * H;
    for (int o = 0; o < H; ++o) yt[o] = 0.0f;
    for (int r = 0; r < k; ++r) orc_scaled_add(yt, ye + (t * k + r) * H, w[t * k + r], H);
  }
  free(ye);
  return 0;
}

void orc_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

int orc_omp_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------------------- */
/* Attention half of a decoder layer                                          */
/* ------------------------------------------------------------------------- */

int orc_rope_neox(uint16_t* x, int64_t n_heads, int64_t head_dim, int64_t pos, float theta) {
  if (n_heads < 0 || head_dim <= 0 || head_dim % 2 != 0 || pos < 0) return -1;
  const int64_t half = head_dim / 2;
  for (int64_t i = 0; i < half; ++i) {
    const float f = (float)pow((double)theta, -2.0 * (double)i / (double)head_dim);
    const float angle = (float)pos * f;
    const float c = (float)cos((double)angle), sn = (float)sin((double)angle);
    for (int64_t h = 0; h < n_heads; ++h) {
      uint16_t* r = x + h * head_dim;
      const float x0 = orc_bf16_to_f32(r[i]), x1 = orc_bf16_to_f32(r[i + half]);
      const float a = x0 * c, b = x1 * sn, cc = x1 * c, d = x0 * sn;
      r[i] = orc_f32_to_bf16(a - b);
      r[i + half] = orc_f32_to_bf16(cc + d);
    }
  }
  return 0;
}

int orc_sdpa_decode(const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t n_heads, int64_t n_kv,
                    int64_t head_dim, int64_t max_len, int64_t seq_len, double scale, double* out) {
  if (n_heads <= 0 || n_kv <= 0 || n_heads % n_kv != 0 || head_dim <= 0 || seq_len <= 0 || seq_len > max_len)
    return -1;
  const int64_t grp = n_heads / n_kv;
  double* p = (double*)malloc(sizeof(double) * (size_t)seq_len);
  if (!p) return -1;
  for (int64_t h = 0; h < n_heads; ++h) {
    const int64_t kv = h / grp;
    const uint16_t* qh = q + h * head_dim;
    double mx = -INFINITY;
    for (int64_t t = 0; t < seq_len; ++t) {
      const uint16_t* kt = k + (kv * max_len + t) * head_dim;
      double dot = 0.0;
      for (int64_t d = 0; d < head_dim; ++d) dot += (double)orc_bf16_to_f32(qh[d]) * (double)orc_bf16_to_f32(kt[d]);
      p[t] = dot * scale;
      if (p[t] > mx) mx = p[t];
    }
    double sum = 0.0;
    for (int64_t t = 0; t < seq_len; ++t) {
      p[t] = exp(p[t] - mx);
      sum += p[t];
    }
    for (int64_t d = 0; d < head_dim; ++d) {
      double acc = 0.0;
      for (int64_t t = 0; t < seq_len; ++t) acc += p[t] * (double)orc_bf16_to_f32(v[(kv * max_len + t) * head_dim + d]);
      out[h * head_dim + d] = acc / sum;
    }
  }
  free(p);
  return 0;
}

int64_t orc_argmax(const float* x, int64_t n) {
  int64_t best = 0;
  float bv = -INFINITY;
  for (int64_t i = 0; i < n; ++i)
    if (x[i] > bv) {
      bv = x[i];
      best = i;
    }
  return best;
}
