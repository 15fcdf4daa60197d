// obs_attention.hip — the rest of a decode step around the MoE block: the
// attention half of a decoder layer and the token step's ends
// (src/forward.rs:398-419, :445-462, :552-567; shaders/rope.metal,
// shaders/sdpa_decode.metal, shaders/ops.metal:31-36, src/attention.rs,
// src/kv_cache.rs).
//
// Device state. A decode step reads its position and token from a device
// array state = {pos, tok} and the argmax at its end writes the next token and
// advances pos, so one captured graph of a whole step replays for every
// token with no host work in between.
//
// Caches (bf16): keys [n_kv, max_len, head_dim] as the reference lays them
// out (kv_cache.rs:3), values transposed [n_kv, head_dim, max_len] so that the
// attention's value operand reads consecutive positions of one dimension.
#include "obs_internal.hpp"

namespace {

using namespace obsd;

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr uint32_t HD = 128;  // head_dim the attention kernels are written for

// ---------------------------------------------------------------------------
// 4-bit mat-vec for the decoder's projections and lm_head
// ---------------------------------------------------------------------------
// One wave per output row group of RPW rows, one pass: every load of the
// wave (its activations, the norm weights, the RPW rows with their scales and
// biases) is issued first, pinned there by a scheduling barrier, then the
// activation work runs while the rows arrive. Lane l covers columns
// [2048 s + 32 l, +32) of every 2048-column segment s: one coalesced 16-byte
// load per row and segment (a 1 KB row segment per wave load). The 32
// nibbles are dotted with the lane's activations as f16 pairs through the
// magic-offset unpack (dot8_q4_off, 9 instructions per 8 nibbles), then
// y_lane = s (sum q x) + b (sum x) with the lane's group scale and bias, and
// the wave sums in the butterfly order (wave_sum_asc). The hardware refills
// the CUs with new workgroups as waves finish, so a large matrix (lm_head)
// needs no loop, whose register copies and stores forced waits for the
// prefetched rows.
struct GemvPart {
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  float* y_f32;
  uint16_t* y_bf16;
  const uint16_t* residual;  // y = residual + W x (bf16 output only)
  uint32_t rows;
};
struct GemvArgs {
  GemvPart p[3];
  uint32_t n_parts, total_rows, in;
  const uint16_t* norm_w;  // x <- bf16(rmsnorm(x) * norm_w) first (nullptr: x as given)
  float eps;
};

template <uint32_t SEG, uint32_t RPW>
__global__ void __launch_bounds__(256) q4_gemv_kernel(const uint16_t* __restrict__ x, GemvArgs a) {
  const uint32_t lane = threadIdx.x & 63u;
  // the wave index in a scalar register, so that every row index and part
  // choice below is wave-uniform: part fields are picked by scalar selects
  // (a divergent index made the compiler fetch the argument struct with
  // vector loads and wait for them before every row)
  const uint32_t wave_g = __builtin_amdgcn_readfirstlane(blockIdx.x * 4u + (threadIdx.x >> 6));
  constexpr uint32_t IN = 2048u * SEG, GROUPS = IN / 64u;
  const uint32_t r0 = RPW * wave_g;
  if (r0 >= a.total_rows) return;  // wave-uniform
  // rows [0, end0) are part 0, [end0, end1) part 1, the rest part 2 (unused parts have 0 rows)
  const uint32_t end0 = a.p[0].rows, end1 = a.p[0].rows + a.p[1].rows;
  auto pick = [](uint32_t pi, auto v0, auto v1, auto v2) __attribute__((always_inline)) {
    return pi == 0u ? v0 : (pi == 1u ? v1 : v2);
  };
  // the lane's activations and norm weights (unconditional loads)
  const uint16_t* const nsrc = a.norm_w ? a.norm_w : x;
  uint4 xv[SEG][4], nv[SEG][4];
#pragma unroll
  for (uint32_t sg = 0; sg < SEG; ++sg)
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
      xv[sg][i] = reinterpret_cast<const uint4*>(x + 2048u * sg + 32u * lane)[i];
      nv[sg][i] = reinterpret_cast<const uint4*>(nsrc + 2048u * sg + 32u * lane)[i];
    }
  // the rows (past the end: the last row again, results unused)
  uint4 q[RPW][SEG];
  uint16_t sc[RPW][SEG], bi[RPW][SEG], res[RPW];
#pragma unroll
  for (uint32_t k = 0; k < RPW; ++k) {
    const uint32_t r = min(r0 + k, a.total_rows - 1u);
    const uint32_t pi = (r >= end0 ? 1u : 0u) + (r >= end1 ? 1u : 0u);
    const uint32_t rr = r - (pi == 0u ? 0u : (pi == 1u ? end0 : end1));
    const uint32_t* w = pick(pi, a.p[0].w, a.p[1].w, a.p[2].w);
    const uint16_t* sp = pick(pi, a.p[0].s, a.p[1].s, a.p[2].s);
    const uint16_t* bp = pick(pi, a.p[0].b, a.p[1].b, a.p[2].b);
    const uint16_t* rp = pick(pi, a.p[0].residual, a.p[1].residual, a.p[2].residual);
#pragma unroll
    for (uint32_t sg = 0; sg < SEG; ++sg) {
      q[k][sg] = load_stream(reinterpret_cast<const uint4*>(w + static_cast<size_t>(rr) * (IN / 8u) + 256u * sg) + lane);
      const size_t gi = static_cast<size_t>(rr) * GROUPS + 32u * sg + lane / 2u;
      sc[k][sg] = sp[gi];
      bi[k][sg] = bp[gi];
    }
    res[k] = *(rp ? rp + rr : sp);  // the row's residual (the scales when the part has none; unused then)
  }
  __builtin_amdgcn_sched_barrier(0);
  float xf[SEG][32];
#pragma unroll
  for (uint32_t sg = 0; sg < SEG; ++sg)
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
      const uint32_t wd[4] = {xv[sg][i].x, xv[sg][i].y, xv[sg][i].z, xv[sg][i].w};
#pragma unroll
      for (uint32_t j = 0; j < 4; ++j) {
        xf[sg][8 * i + 2 * j] = bf16lo(wd[j]);
        xf[sg][8 * i + 2 * j + 1] = bf16hi(wd[j]);
      }
    }
  {  // RMSNorm of x (obs_rmsnorm's sequence; its lane order when in == 2048),
     // computed every time and selected (no branch around the loads' use)
    const bool use_norm = a.norm_w != nullptr;
    float ss = 0.0f;
#pragma unroll
    for (uint32_t sg = 0; sg < SEG; ++sg)
#pragma unroll
      for (uint32_t c = 0; c < 32; ++c) ss = __builtin_fmaf(xf[sg][c], xf[sg][c], ss);
    const float inv = 1.0f / __builtin_sqrtf(wave_sum_asc(ss) / static_cast<float>(IN) + a.eps);
#pragma unroll
    for (uint32_t sg = 0; sg < SEG; ++sg)
#pragma unroll
      for (uint32_t i = 0; i < 4; ++i) {
        const uint32_t wd[4] = {nv[sg][i].x, nv[sg][i].y, nv[sg][i].z, nv[sg][i].w};
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
          float& e0 = xf[sg][8 * i + 2 * j];
          float& e1 = xf[sg][8 * i + 2 * j + 1];
          const uint32_t npr = pack_bf16_pair_rne((e0 * inv) * bf16lo(wd[j]), (e1 * inv) * bf16hi(wd[j]));
          e0 = use_norm ? bf16lo(npr) : e0;
          e1 = use_norm ? bf16hi(npr) : e1;
        }
      }
  }
  // f16 pairs, their sum and the offset part, per segment; the f16 range per
  // segment (the lane's 32 columns scaled by 2^-k at 2^15 and beyond, the
  // segment's dot products by 2^k; k = 0 below)
  f16x2_t xh[SEG][16];
  float xs[SEG], xoff[SEG], xup[SEG];
#pragma unroll
  for (uint32_t sg = 0; sg < SEG; ++sg) {
    float sum = 0.0f;
#pragma unroll
    for (uint32_t c = 0; c < 32; ++c) sum = sum + xf[sg][c];
    xs[sg] = sum;
    const F16Range xr = f16_range(lane_absmax<32>(xf[sg]));
    xup[sg] = xr.up;
#pragma unroll
    for (uint32_t c = 0; c < 32; ++c) xf[sg][c] = xf[sg][c] * xr.down;
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) f16_pairs8(xf[sg] + 8 * i, xh[sg] + 4 * i);
    float off = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) off = dot8_off_only(xh[sg] + 4 * i, off);
    xoff[sg] = off;
  }
  // the rows' sums; lane k keeps row k's result, so one store serves the wave
  float mine = 0.0f;
#pragma unroll
  for (uint32_t k = 0; k < RPW; ++k) {
    float part = 0.0f;
#pragma unroll
    for (uint32_t sg = 0; sg < SEG; ++sg) {
      float acc = 0.0f;
      acc = dot8_q4_off(q[k][sg].x, xh[sg] + 0, acc);
      acc = dot8_q4_off(q[k][sg].y, xh[sg] + 4, acc);
      acc = dot8_q4_off(q[k][sg].z, xh[sg] + 8, acc);
      acc = dot8_q4_off(q[k][sg].w, xh[sg] + 12, acc);
      part = part + __builtin_fmaf(bf16_to_f32(sc[k][sg]), (acc - xoff[sg]) * xup[sg], bf16_to_f32(bi[k][sg]) * xs[sg]);
    }
    part = wave_sum_asc(part);
    const float y = bf16_to_f32(res[k]) + part;  // used only where the part has a residual
    const uint32_t r = min(r0 + k, a.total_rows - 1u);
    const uint32_t pi = (r >= end0 ? 1u : 0u) + (r >= end1 ? 1u : 0u);
    const bool has_res = pick(pi, a.p[0].residual, a.p[1].residual, a.p[2].residual) != nullptr;
    mine = lane == k ? (has_res ? y : part) : mine;
  }
  const uint32_t r = r0 + lane;
  if (lane < RPW && r < a.total_rows) {
    const uint32_t pi = (r >= end0 ? 1u : 0u) + (r >= end1 ? 1u : 0u);
    const uint32_t rr = r - (pi == 0u ? 0u : (pi == 1u ? end0 : end1));
    float* yf = pick(pi, a.p[0].y_f32, a.p[1].y_f32, a.p[2].y_f32);
    uint16_t* yb = pick(pi, a.p[0].y_bf16, a.p[1].y_bf16, a.p[2].y_bf16);
    if (yf) yf[rr] = mine;
    if (yb) yb[rr] = f32_to_bf16(mine);
  }
}

// ---------------------------------------------------------------------------
// q/k RMSNorm + NeoX RoPE + cache append, one launch
// ---------------------------------------------------------------------------
// Lane l owns columns 2l, 2l+1 of a head (the RMSNorm lane order of
// obs_rmsnorm at dim 128). Heads [0, nh): query heads, normed and rotated in
// place; [nh, nh+nkv): key heads, normed, rotated, written to the key cache at
// pos; [nh+nkv, nh+2nkv): value heads, written to the transposed value cache.
// RoPE pairs column i with i + 64, held by lane l ^ 32. Frequencies, cosines
// and sines follow the oracle's restatement: f = fl32(theta^(-2i/128)) and
// cos, sin of the fp32 angle fl32(pos * f), each evaluated in double and
// rounded once; r0 = x0 c - x1 s, r1 = x1 c + x0 s with rounded products. The
// cosines and sines depend on the position and the lane only, so a wave
// evaluates them once and applies them to every head it owns.
// ROWS = false (decode): one token at pos = state[0], one wave per head; the
// position is read with a vector load issued after the head's loads (a scalar
// load would be waited for together with the kernel arguments, before any
// other load). ROWS = true (prefill; cosines and sines from the context's
// RoPE table, the same values): one workgroup per token of q (rows of
// q_ld elements holding nh x 128), k, v (rows of kv_ld holding nkv x 128) at
// position pos0 + token; wave w owns heads w, w + 4, ... of the query and key
// heads. The value heads go through LDS instead: workgroups n_tok.. each take
// (kv head, 64 consecutive tokens), read the 64 value rows and write each of
// the 128 transposed cache rows as one 128-byte run (a 2-byte store per
// token and dim, from the token's workgroup, cost as much as the rest).
constexpr uint32_t PREP_VTOK = 64;  // tokens per value-transposing workgroup
template <bool ROWS>
__global__ void __launch_bounds__(256) attn_prep_kernel(uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                        const uint16_t* __restrict__ v,
                                                        const uint16_t* __restrict__ q_norm,
                                                        const uint16_t* __restrict__ k_norm,
                                                        uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache_t,
                                                        uint32_t nh, uint32_t nkv, uint32_t max_len, float eps,
                                                        float theta, const int32_t* __restrict__ state, uint32_t pos0,
                                                        uint32_t n_tok, uint32_t q_ld, uint32_t kv_ld,
                                                        const float* __restrict__ rope) {
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  if (ROWS && blockIdx.x >= n_tok) {  // uniform: a value-transposing workgroup
    __shared__ uint32_t s_v[PREP_VTOK][HD / 2 + 1];  // token rows of dim pairs (+1 word: bank spread)
    const uint32_t vi = blockIdx.x - n_tok, kvh = vi % nkv, t0 = (vi / nkv) * PREP_VTOK;
    const uint32_t nt = min(PREP_VTOK, n_tok - t0);
#pragma unroll
    for (uint32_t i = 0; i < PREP_VTOK * HD / 2u / 256u; ++i) {
      const uint32_t idx = threadIdx.x + 256u * i, tt = idx / (HD / 2u), dp = idx % (HD / 2u);
      if (tt < nt)
        s_v[tt][dp] = *reinterpret_cast<const uint32_t*>(v + static_cast<size_t>(t0 + tt) * kv_ld + kvh * HD + 2u * dp);
    }
    __syncthreads();
    const uint32_t tt = threadIdx.x % PREP_VTOK;  // lanes: consecutive positions of one dim
    if (tt < nt) {
      uint16_t* dst = v_cache_t + static_cast<size_t>(kvh) * HD * max_len + pos0 + t0 + tt;
      for (uint32_t d = threadIdx.x / PREP_VTOK; d < HD; d += 256u / PREP_VTOK) {
        const uint32_t wd = s_v[tt][d / 2u];
        dst[static_cast<size_t>(d) * max_len] = static_cast<uint16_t>((d & 1u) ? wd >> 16 : wd & 0xffffu);
      }
    }
    return;
  }
  const uint32_t heads = ROWS ? nh + nkv : nh + 2u * nkv;  // with ROWS the value heads are transposed above
  const uint32_t tok = ROWS ? blockIdx.x : 0u;
  const uint32_t h_first = ROWS ? wave : blockIdx.x * 4u + wave, h_step = ROWS ? 4u : heads;
  if (tok >= n_tok || h_first >= heads) return;  // wave-uniform
  q += static_cast<size_t>(tok) * q_ld;
  k += static_cast<size_t>(tok) * kv_ld;
  v += static_cast<size_t>(tok) * kv_ld;
  const uint32_t c0 = 2u * lane;
  auto head_src = [&](uint32_t head) __attribute__((always_inline)) {
    const bool is_v = head >= nh + nkv, is_q = head < nh;
    const uint32_t hk = is_q ? head : (is_v ? head - nh - nkv : head - nh);
    return is_q ? q + hk * HD : (is_v ? v + hk * HD : k + hk * HD);
  };
  // the first head's values and both norm weights, before the position
  const uint32_t xv0 = *reinterpret_cast<const uint32_t*>(head_src(h_first) + c0);
  const uint32_t wq = *reinterpret_cast<const uint32_t*>(q_norm + c0);
  const uint32_t wk = *reinterpret_cast<const uint32_t*>(k_norm + c0);
  int32_t pos_i;
  if (ROWS) {
    pos_i = static_cast<int32_t>(pos0 + tok);
  } else {
    uint32_t zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero));  // a per-lane index: a vector load
    pos_i = state[zero];
  }
  const uint32_t pos = static_cast<uint32_t>(pos_i);
  const bool pos_ok = pos_i >= 0 && pos < max_len;
  float cs[2], sn[2];
  if (ROWS) {  // the context's table holds exactly these values (rope_table_kernel)
    const float4 t = *reinterpret_cast<const float4*>(rope + static_cast<size_t>(min(pos, max_len - 1u)) * 128u +
                                                      4u * (lane & 31u));
    cs[0] = t.x; sn[0] = t.y; cs[1] = t.z; sn[1] = t.w;
  } else {
#pragma unroll
    for (uint32_t j = 0; j < 2; ++j) {
      const uint32_t i = (c0 + j) & 63u;  // pair index
      const float f = static_cast<float>(pow(static_cast<double>(theta), -2.0 * static_cast<double>(i) / 128.0));
      const float angle = static_cast<float>(pos) * f;
      cs[j] = static_cast<float>(cos(static_cast<double>(angle)));
      sn[j] = static_cast<float>(sin(static_cast<double>(angle)));
    }
  }
  const bool first = lane < 32u;
  // heads in groups of 4: the group's loads first (clamped to a valid head;
  // unused past the last), so a wave waits once per group, not once per head
  for (uint32_t hb = h_first; hb < heads; hb += 4u * h_step) {
  uint32_t xvs[4];
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j)
    xvs[j] = j == 0 && hb == h_first ? xv0
                                     : *reinterpret_cast<const uint32_t*>(head_src(min(hb + j * h_step, heads - 1u)) + c0);
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j) {
    const uint32_t head = hb + j * h_step;
    if (head >= heads) break;  // wave-uniform
    const uint32_t xv = xvs[j];
    const bool is_v = head >= nh + nkv, is_q = head < nh;
    const uint32_t hk = is_q ? head : (is_v ? head - nh - nkv : head - nh);
    if (is_v) {  // value head: transposed cache column pos
      if (pos_ok) {
        uint16_t* dst = v_cache_t + (static_cast<size_t>(hk) * HD + c0) * max_len + pos;
        dst[0] = static_cast<uint16_t>(xv & 0xffffu);
        dst[max_len] = static_cast<uint16_t>(xv >> 16);
      }
      continue;
    }
    const uint32_t wv = is_q ? wq : wk;
    const float x0 = bf16lo(xv), x1 = bf16hi(xv);
    float ss = __builtin_fmaf(x0, x0, 0.0f);
    ss = __builtin_fmaf(x1, x1, ss);
    const float inv = 1.0f / __builtin_sqrtf(wave_sum_asc(ss) / static_cast<float>(HD) + eps);
    // the normed values, rounded to bf16 as the stored q/k would be
    const float n0 = bf16_to_f32(f32_to_bf16((x0 * inv) * bf16lo(wv)));
    const float n1 = bf16_to_f32(f32_to_bf16((x1 * inv) * bf16hi(wv)));
    const float p0 = __shfl_xor(n0, 32, 64), p1 = __shfl_xor(n1, 32, 64);  // columns c0 +- 64
    float r[2];
#pragma unroll
    for (uint32_t j = 0; j < 2; ++j) {
      const float own = j ? n1 : n0, other = j ? p1 : p0;
      const float a = own * cs[j], b = other * sn[j];
      r[j] = first ? a - b : a + b;  // first: own = x0 (column i), other = x1 (column i + 64)
    }
    const uint32_t out = pack_bf16x2(r[0], r[1]);
    if (is_q) {
      *reinterpret_cast<uint32_t*>(q + hk * HD + c0) = out;
    } else if (pos_ok) {
      *reinterpret_cast<uint32_t*>(k_cache + (static_cast<size_t>(hk) * max_len + pos) * HD + c0) = out;
    }
  }
  }
}

// ---------------------------------------------------------------------------
// GQA decode attention: split over positions, MFMA for both products
// ---------------------------------------------------------------------------
// Workgroup (one wave) = (kv head, split). The G <= 16 query heads of the kv
// head are the N columns of v_mfma_f32_16x16x32_bf16 (padding heads are zero).
// Per 32-position block:
//   S^T [16 positions x 16 heads] = K_block . Q^T, twice (two 16-position
//   tiles, 4 MFMAs each over 128 dims): A = key rows (one 16-byte load per
//   lane and step), B = the query slices held in registers. The 16x16 output
//   layout puts S[h][t] for h = l % 16, t = 4 (l / 16) + i in lane l.
//   Online softmax per head in base 2: running max m, running sum l, P = 2^(s - m).
//   O [16 heads x 128] += P . V_block: lane l's eight P values (positions
//   4 g + i of tile 0 and 16 + 4 g + i of tile 1, g = l / 16) are already the
//   A operand of one K = 32 MFMA; the B operand pairs them with the same
//   positions of the transposed value cache (two 8-byte loads per dim tile).
// The split's (m, l, O) go to the workspace; sdpa_combine_kernel merges them.
__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, 64); }

// Masks of a lane's four value words (positions ta, ta + 1 | ta + 2, ta + 3 |
// ta + 16, ta + 17 | ta + 18, ta + 19; low half = the first): positions at or
// past seq become zero.
__device__ __forceinline__ u32x4_t value_masks(uint32_t ta, uint32_t seq) {
  auto m = [&](uint32_t t) { return t >= seq ? 0u : (t + 1u >= seq ? 0xffffu : 0xffffffffu); };
  return u32x4_t{m(ta), m(ta + 2u), m(ta + 16u), m(ta + 18u)};
}

__global__ void __launch_bounds__(64) sdpa_split_kernel(const uint16_t* __restrict__ q,
                                                        const uint16_t* __restrict__ k_cache,
                                                        const uint16_t* __restrict__ v_cache_t,
                                                        float* __restrict__ ws, uint32_t nh, uint32_t nkv,
                                                        uint32_t max_len, uint32_t splits, float scale_log2,
                                                        const int32_t* __restrict__ state) {
  const uint32_t lane = threadIdx.x, kv = blockIdx.x / splits, sp = blockIdx.x % splits;
  const uint32_t G = nh / nkv, col = lane & 15u, g = lane >> 4;
  const int32_t pos = state[0];
  const uint32_t seq = static_cast<uint32_t>(min(max(pos + 1, 1), static_cast<int32_t>(max_len)));
  // positions of this split, in 32-position blocks
  const uint32_t nblk = (seq + 31u) / 32u, per = (nblk + splits - 1u) / splits;
  const uint32_t b0 = sp * per, b1 = min(nblk, b0 + per);
  // query slices: B operand of the score MFMA, head col, dims 32 ks + 8 g + j
  bf16x8_t qb[4];
  {
    const uint32_t h = kv * G + col;
#pragma unroll
    for (uint32_t ks = 0; ks < 4; ++ks) {
      u32x4_t v = *reinterpret_cast<const u32x4_t*>(q + static_cast<size_t>(min(h, nh - 1u)) * HD + 32u * ks + 8u * g);
      if (col >= G) v = u32x4_t{0u, 0u, 0u, 0u};
      qb[ks] = __builtin_bit_cast(bf16x8_t, v);
    }
  }
  float m_run = -__builtin_huge_valf(), l_run = 0.0f;  // per head col (replicated over g)
  f32x4_t o[8];
#pragma unroll
  for (uint32_t nt = 0; nt < 8; ++nt) o[nt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const uint16_t* kb = k_cache + static_cast<size_t>(kv) * max_len * HD;
  const uint16_t* vb = v_cache_t + static_cast<size_t>(kv) * HD * max_len;
  for (uint32_t blk = b0; blk < b1; ++blk) {
    const uint32_t t0 = 32u * blk;
    // every load of the block first: the key rows of both tiles and the value
    // columns (they do not depend on the scores)
    u32x4_t ka[2][4];
#pragma unroll
    for (uint32_t tt = 0; tt < 2; ++tt) {
      const uint16_t* kr = kb + static_cast<size_t>(t0 + 16u * tt + col) * HD + 8u * g;
#pragma unroll
      for (uint32_t ks = 0; ks < 4; ++ks) ka[tt][ks] = *reinterpret_cast<const u32x4_t*>(kr + 32u * ks);
    }
    u32x2_t va[8][2];
#pragma unroll
    for (uint32_t nt = 0; nt < 8; ++nt) {
      const uint16_t* vr = vb + static_cast<size_t>(16u * nt + col) * max_len + t0 + 4u * g;
      va[nt][0] = *reinterpret_cast<const u32x2_t*>(vr);
      va[nt][1] = *reinterpret_cast<const u32x2_t*>(vr + 16);
    }
    // all 24 loads issued before the first wait (left alone, the scheduler
    // interleaved waits between them and the kernel ran at half speed)
    __builtin_amdgcn_sched_barrier(0);
    // scores of the two 16-position tiles
    f32x4_t s[2];
#pragma unroll
    for (uint32_t tt = 0; tt < 2; ++tt) {
      f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (uint32_t ks = 0; ks < 4; ++ks)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ka[tt][ks]), qb[ks], acc, 0, 0, 0);
      s[tt] = acc;
    }
    // lane holds S[h = col][t0 + 16 tt + 4 g + i]; mask positions >= seq
    float sv[8];
#pragma unroll
    for (uint32_t tt = 0; tt < 2; ++tt)
#pragma unroll
      for (uint32_t i = 0; i < 4; ++i) {
        const uint32_t t = t0 + 16u * tt + 4u * g + i;
        sv[4 * tt + i] = t < seq ? s[tt][i] * scale_log2 : -__builtin_huge_valf();
      }
    float bm = sv[0];
#pragma unroll
    for (uint32_t i = 1; i < 8; ++i) bm = fmaxf(bm, sv[i]);
    bm = fmaxf(bm, shfl_xor_f(bm, 16));
    bm = fmaxf(bm, shfl_xor_f(bm, 32));
    const float m_new = fmaxf(m_run, bm);  // finite: every block holds a position < seq
    const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
    float p[8], psum = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
      // P is rounded to bf16 for the MFMA; the running sum adds the rounded values
      p[i] = bf16_to_f32(f32_to_bf16(__builtin_amdgcn_exp2f(sv[i] - m_new)));
      psum += p[i];
    }
    l_run = l_run * corr + psum;  // per lane; the four g lanes of a head are summed at the end
    m_run = m_new;
    // O rows are heads 4 g + i: their corrections live in lanes with col == 4 g + i
    float oc[4];
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) oc[i] = __shfl(corr, static_cast<int>(4u * g + i), 64);
    const bf16x8_t pa = __builtin_bit_cast(
        bf16x8_t, u32x4_t{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                          pack_bf16x2(p[6], p[7])});
    // values of the same positions: dim 16 nt + col, positions t0 + 4 g + i and t0 + 16 + 4 g + i
    // masked positions read zero values; only the last block needs the masks,
    // so they are applied under a (uniform) branch: here every load of the
    // block has been waited for already, and the branch-free form measured
    // slower
    const bool tail = t0 + 32u > seq;
#pragma unroll
    for (uint32_t nt = 0; nt < 8; ++nt) {
      u32x2_t v0 = va[nt][0], v1 = va[nt][1];
      if (tail) {
        const u32x4_t vm = value_masks(t0 + 4u * g, seq);
        v0 = u32x2_t{v0.x & vm.x, v0.y & vm.y};
        v1 = u32x2_t{v1.x & vm.z, v1.y & vm.w};
      }
      const bf16x8_t vbf = __builtin_bit_cast(bf16x8_t, u32x4_t{v0.x, v0.y, v1.x, v1.y});
#pragma unroll
      for (uint32_t i = 0; i < 4; ++i) o[nt][i] *= oc[i];
      o[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, vbf, o[nt], 0, 0, 0);
    }
  }
  // head col's total: the four g lanes
  l_run += shfl_xor_f(l_run, 16);
  l_run += shfl_xor_f(l_run, 32);
  // workspace [kv][split][head in group][HD + 2]: O (unnormalised), m, l
  float* base = ws + (static_cast<size_t>(kv) * splits + sp) * 16u * (HD + 2u);
  if (lane < 16u && col < G) {
    base[col * (HD + 2u) + HD] = m_run;
    base[col * (HD + 2u) + HD + 1u] = l_run;
  }
#pragma unroll
  for (uint32_t nt = 0; nt < 8; ++nt)
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
      const uint32_t h = 4u * g + i;
      if (h < G) base[h * (HD + 2u) + 16u * nt + col] = o[nt][i];
    }
}

// out[h] = sum_s O_s 2^(m_s - M) / sum_s l_s 2^(m_s - M), M = max_s m_s; bf16.
// Wave 0 reads every split's (m, l) at once and forms the weights; then each
// thread sums one dimension over a quarter of the splits with its loads all in
// flight, and the quarters meet in LDS.
__global__ void __launch_bounds__(512) sdpa_combine_kernel(const float* __restrict__ ws, uint16_t* __restrict__ out,
                                                           uint32_t nh, uint32_t nkv, uint32_t splits) {
  __shared__ float s_f[64];
  __shared__ float s_part[4][HD];
  __shared__ float s_den;
  const uint32_t h = blockIdx.x, tid = threadIdx.x, G = nh / nkv, kv = h / G, hh = h % G;
  constexpr uint32_t STRIDE = 16u * (HD + 2u);  // floats between splits
  const float* base = ws + static_cast<size_t>(kv) * splits * STRIDE + hh * (HD + 2u);
  if (tid < 64u) {  // splits <= 64
    const bool have = tid < splits;
    const float m = have ? base[tid * STRIDE + HD] : -__builtin_huge_valf();
    const float l = have ? base[tid * STRIDE + HD + 1u] : 0.0f;
    float M = m;
#pragma unroll
    for (int k = 1; k < 64; k <<= 1) M = fmaxf(M, __shfl_xor(M, k, 64));
    const float f = m == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f(m - M);  // empty split: no weight
    float den = l * f;
#pragma unroll
    for (int k = 1; k < 64; k <<= 1) den += __shfl_xor(den, k, 64);
    s_f[tid] = f;
    if (tid == 0) s_den = den;
  }
  __syncthreads();
  const uint32_t d = tid & (HD - 1u), q4 = tid >> 7;  // 4 quarters of the splits
  float num = 0.0f;
#pragma unroll 4
  for (uint32_t sp = q4; sp < splits; sp += 4u) num = __builtin_fmaf(base[sp * STRIDE + d], s_f[sp], num);
  s_part[q4][d] = num;
  __syncthreads();
  if (tid < HD)
    out[static_cast<size_t>(h) * HD + tid] =
        f32_to_bf16(((s_part[0][tid] + s_part[1][tid]) + (s_part[2][tid] + s_part[3][tid])) / s_den);
}

// ---------------------------------------------------------------------------
// Causal GQA attention for a prefill batch
// ---------------------------------------------------------------------------
// Tokens [0, n_tok) of q (rows of q_ld elements holding nh x 128) sit at
// positions pos0 + token and attend to cache positions [0, pos0 + token]; the
// batch's own keys and values are in the caches already (attn_prep over the
// rows runs first). A workgroup serves one kv head and 8 column groups of 16
// MFMA columns, a column being (token, query head) = TPG = 16 / G tokens x
// the G query heads of the kv head. It has two sets of 4 waves that split the
// 32-position blocks: set s runs blocks s, s + 2, s + 4, ..., and wave w of
// each set owns column groups 2w and 2w + 1, so a tile's chain of dependent
// blocks is half as long (the longest tiles of a prompt set the launch's
// length). Per block a set stages the keys [32][128] and the transposed
// values [128][32] in LDS once (rows padded against bank conflicts), and each
// of its waves runs sdpa_split_kernel's block math on both of its groups from
// there, so each key/value byte leaves L2 once per 8 TPG tokens instead of
// once per TPG. The next block's loads are in flight while a block is
// computed (registers, then the other LDS buffer). At the end the second set
// hands its (m, l, O) to the first through LDS, which merges them. A column's
// scores past its token's position are masked; values at or past the
// workgroup's longest sequence read as zero. Tiles are launched longest first.
constexpr uint32_t PF_KROW = HD + 8u;  // padded key row (bf16): 272 bytes
constexpr uint32_t PF_VROW = 32u + 4u; // padded transposed value row (bf16): 72 bytes
constexpr uint32_t PF_BUF = 32u * PF_KROW + HD * PF_VROW;  // bf16 elements per staged block

constexpr uint32_t PF_THREADS = 512;  // two sets of 4 waves

__global__ void __launch_bounds__(PF_THREADS, 1) sdpa_prefill_kernel(const uint16_t* __restrict__ q,
                                                                    const uint16_t* __restrict__ k_cache,
                                                                    const uint16_t* __restrict__ v_cache_t,
                                                                    uint16_t* __restrict__ out, uint32_t nh,
                                                                    uint32_t nkv, uint32_t max_len, uint32_t pos0,
                                                                    uint32_t n_tok, uint32_t q_ld, float scale_log2) {
  // per set, two staging buffers; after the block loop the second set's
  // (m, l, O) pass through them to the first
  __shared__ __attribute__((aligned(16))) uint16_t s_blk[2][2][PF_BUF];
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t set = tid >> 8, stid = tid & 255u, wave = stid >> 6;  // wave within its set
  const uint32_t G = nh / nkv, TPG = 16u / G, TPWG = 8u * TPG;
  const uint32_t n_wg_tok = (n_tok + TPWG - 1u) / TPWG;
  // tiles in launch order from the longest (last tokens) down: one workgroup
  // fills a CU, so the dispatcher hands the shorter tiles to the CUs that free
  // up first
  const uint32_t kv = blockIdx.x % nkv, r = blockIdx.x / nkv;
  const uint32_t tb = (n_wg_tok - 1u - r) * TPWG;  // first token
  const uint32_t col = lane & 15u, g = lane >> 4;
  const uint32_t cj = col / G, ci = col % G;
  const uint32_t seq = pos0 + min(tb + TPWG, n_tok);  // the workgroup's longest sequence
  const uint32_t nblk = (seq + 31u) / 32u;
  // the wave's two column groups: query slices (B operand), limits, state
  bf16x8_t qb[2][4];
  uint32_t lim[2];
#pragma unroll
  for (uint32_t cg = 0; cg < 2; ++cg) {
    const uint32_t t = tb + (2u * wave + cg) * TPG + cj;
    lim[cg] = pos0 + t + 1u;
    const uint16_t* qr = q + static_cast<size_t>(min(t, n_tok - 1u)) * q_ld + (kv * G + ci) * HD + 8u * g;
#pragma unroll
    for (uint32_t ks = 0; ks < 4; ++ks) {
      u32x4_t v = *reinterpret_cast<const u32x4_t*>(qr + 32u * ks);
      if (t >= n_tok) v = u32x4_t{0u, 0u, 0u, 0u};
      qb[cg][ks] = __builtin_bit_cast(bf16x8_t, v);
    }
  }
  float m_run[2] = {-__builtin_huge_valf(), -__builtin_huge_valf()}, l_run[2] = {0.0f, 0.0f};
  f32x4_t o[2][8];
#pragma unroll
  for (uint32_t cg = 0; cg < 2; ++cg)
#pragma unroll
    for (uint32_t nt = 0; nt < 8; ++nt) o[cg][nt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const uint16_t* kb = k_cache + static_cast<size_t>(kv) * max_len * HD;
  const uint16_t* vb = v_cache_t + static_cast<size_t>(kv) * HD * max_len;
  // staging: thread t of a set moves 16-byte chunks t and t + 256 of the key
  // block (row c / 16, column 8 (c % 16)) and of the transposed value block
  // (row c / 4, column 8 (c % 4))
  auto load_blk = [&](uint32_t blk, u32x4_t* r) __attribute__((always_inline)) {
    const uint32_t t0 = 32u * blk;
#pragma unroll
    for (uint32_t h = 0; h < 2; ++h) {
      const uint32_t c = stid + 256u * h;
      r[h] = *reinterpret_cast<const u32x4_t*>(kb + static_cast<size_t>(t0 + c / 16u) * HD + 8u * (c % 16u));
      r[2 + h] = *reinterpret_cast<const u32x4_t*>(vb + static_cast<size_t>(c / 4u) * max_len + t0 + 8u * (c % 4u));
    }
  };
  // Values at or past seq (the block past the workgroup's longest sequence) are
  // stored as zero: their scores are masked, and the cache may hold anything there.
  auto store_blk = [&](uint32_t buf, const u32x4_t* r, uint32_t blk) __attribute__((always_inline)) {
    const bool tail = 32u * blk + 32u > seq;  // uniform
#pragma unroll
    for (uint32_t h = 0; h < 2; ++h) {
      const uint32_t c = stid + 256u * h;
      *reinterpret_cast<u32x4_t*>(&s_blk[set][buf][(c / 16u) * PF_KROW + 8u * (c % 16u)]) = r[h];
      u32x4_t v = r[2 + h];
      if (tail) {
        const uint32_t ta = 32u * blk + 8u * (c % 4u);  // positions ta .. ta + 7, two per word
        auto m = [&](uint32_t w, uint32_t t) { return t >= seq ? 0u : (t + 1u >= seq ? (w & 0xffffu) : w); };
        v = u32x4_t{m(v.x, ta), m(v.y, ta + 2u), m(v.z, ta + 4u), m(v.w, ta + 6u)};
      }
      // a transposed value row of 32 positions is 4 chunks; rows are 72 bytes, so
      // each chunk is stored as two 8-byte halves (8-byte alignment)
      uint16_t* vr = &s_blk[set][buf][32u * PF_KROW + (c / 4u) * PF_VROW + 8u * (c % 4u)];
      *reinterpret_cast<u32x2_t*>(vr) = u32x2_t{v.x, v.y};
      *reinterpret_cast<u32x2_t*>(vr + 4) = u32x2_t{v.z, v.w};
    }
  };
  // A column's rescale by its correction factor is skipped while no column's
  // maximum moved (the factor is then exactly 1).
  auto run_blk = [&](uint32_t buf, uint32_t blk) __attribute__((always_inline)) {
    const uint32_t t0 = 32u * blk;
    const uint16_t* sk = s_blk[set][buf];
    const uint16_t* sv = s_blk[set][buf] + 32u * PF_KROW;
    // the scores of both column groups: each key fragment is read from LDS
    // once and feeds both groups' MFMAs (the LDS reads, not the MFMAs, set the
    // block's time)
    bf16x8_t kf[2][4];  // all 8 key fragments in flight at once
#pragma unroll
    for (uint32_t tt = 0; tt < 2; ++tt)
#pragma unroll
      for (uint32_t ks = 0; ks < 4; ++ks)
        kf[tt][ks] = __builtin_bit_cast(
            bf16x8_t, *reinterpret_cast<const u32x4_t*>(sk + (16u * tt + col) * PF_KROW + 8u * g + 32u * ks));
    __builtin_amdgcn_sched_barrier(0);
    f32x4_t sc[2][2];
#pragma unroll
    for (uint32_t tt = 0; tt < 2; ++tt) {
      f32x4_t acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
      for (uint32_t ks = 0; ks < 4; ++ks)
#pragma unroll
        for (uint32_t cg = 0; cg < 2; ++cg) acc[cg] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[tt][ks], qb[cg][ks], acc[cg], 0, 0, 0);
      sc[0][tt] = acc[0];
      sc[1][tt] = acc[1];
    }
    // the value slices (dim 16 nt + col, the lane's 8 positions), read now so
    // that their LDS latency passes during the softmax (pinned here: left
    // alone, each read sank to its MFMAs and waited there)
    bf16x8_t vf[8];
#pragma unroll
    for (uint32_t nt = 0; nt < 8; ++nt) {
      const uint16_t* vr = sv + (16u * nt + col) * PF_VROW + 4u * g;
      const u32x2_t v0 = *reinterpret_cast<const u32x2_t*>(vr);
      const u32x2_t v1 = *reinterpret_cast<const u32x2_t*>(vr + 16);
      vf[nt] = __builtin_bit_cast(bf16x8_t, u32x4_t{v0.x, v0.y, v1.x, v1.y});
    }
    __builtin_amdgcn_sched_barrier(0);
    // the scores as the softmax sees them: a block wholly below every column's
    // position (all but the last few of a long tile) needs no mask
    float svl[2][8];
    if (t0 + 32u <= pos0 + tb + 1u) {  // uniform
#pragma unroll
      for (uint32_t cg = 0; cg < 2; ++cg)
#pragma unroll
        for (uint32_t tt = 0; tt < 2; ++tt)
#pragma unroll
          for (uint32_t i = 0; i < 4; ++i) svl[cg][4 * tt + i] = sc[cg][tt][i];
    } else {
#pragma unroll
      for (uint32_t cg = 0; cg < 2; ++cg)
#pragma unroll
        for (uint32_t tt = 0; tt < 2; ++tt)
#pragma unroll
          for (uint32_t i = 0; i < 4; ++i) {
            const uint32_t t = t0 + 16u * tt + 4u * g + i;
            svl[cg][4 * tt + i] = t < lim[cg] ? sc[cg][tt][i] : -__builtin_huge_valf();
          }
    }
    // both groups' steps side by side (independent chains), one rescale for both
    bf16x8_t pa[2];
    float corr[2];
#pragma unroll
    for (uint32_t cg = 0; cg < 2; ++cg) {
      float bm = svl[cg][0];
#pragma unroll
      for (uint32_t i = 1; i < 8; ++i) bm = fmaxf(bm, svl[cg][i]);
      bm = fmaxf(bm, lane_xor16_f32(bm, lane));
      bm = fmaxf(bm, lane_xor32_f32(bm, lane));
      // -inf while none of the set's blocks so far held a position of the
      // column (the second set starts at block 1): its p and corr are then
      // taken against 0, so they are 0 and l and O stay 0 (not NaN)
      const float m_new = fmaxf(m_run[cg], bm * scale_log2);
      const float m_use = m_new == -__builtin_huge_valf() ? 0.0f : m_new;
      corr[cg] = __builtin_amdgcn_exp2f(m_run[cg] - m_use);
      // p = 2^(s * scale - m), the scale folded into one fma (the maximum is taken
      // over the unscaled scores: scaling by a positive factor keeps their
      // order), rounded to bf16 (v_cvt_pk_bf16_f32, round to nearest even); the
      // row sum adds the rounded pairs with v_dot2c_f32_bf16 against (1, 1)
      typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
      const bf16x2_v ones2 = __builtin_bit_cast(bf16x2_v, 0x3f803f80u);
      uint32_t pk[4];
      float psum = 0.0f;
#pragma unroll
      for (uint32_t i = 0; i < 4; ++i) {
        pk[i] = pack_bf16_pair_rne(__builtin_amdgcn_exp2f(__builtin_fmaf(svl[cg][2 * i], scale_log2, -m_use)),
                                   __builtin_amdgcn_exp2f(__builtin_fmaf(svl[cg][2 * i + 1], scale_log2, -m_use)));
        psum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, pk[i]), ones2, psum, false);
      }
      l_run[cg] = l_run[cg] * corr[cg] + psum;
      m_run[cg] = m_new;
      pa[cg] = __builtin_bit_cast(bf16x8_t, u32x4_t{pk[0], pk[1], pk[2], pk[3]});
    }
    if (__any(corr[0] != 1.0f || corr[1] != 1.0f)) {  // wave-uniform; a lane's O entries are all of its own column
#pragma unroll
      for (uint32_t cg = 0; cg < 2; ++cg)
#pragma unroll
        for (uint32_t nt = 0; nt < 8; ++nt)
#pragma unroll
          for (uint32_t i = 0; i < 4; ++i) o[cg][nt][i] *= corr[cg];
    }
    // O^T += V^T P of both groups: the value slice is the A operand and the
    // lane's own probabilities the B operand, so the lane ends with
    // O[column col][dims 16 nt + 4 g .. + 3] and every factor it applies
    // (correction, merge, 1 / l) is its own column's: no lane exchanges
#pragma unroll
    for (uint32_t nt = 0; nt < 8; ++nt)
#pragma unroll
      for (uint32_t cg = 0; cg < 2; ++cg) o[cg][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[nt], pa[cg], o[cg][nt], 0, 0, 0);
  };
  // Iteration i computes block 2 i + set (none past the end: the second set's
  // last iteration when nblk is odd), with two register stages in turn (no
  // copies between them): the set's block two iterations ahead is loaded while
  // the current one is computed from LDS and the next one, loaded an iteration
  // earlier, goes from registers to the other LDS buffer. Past the end the
  // last block is loaded again (unused). Both sets run the same iterations, so
  // all 8 waves meet every barrier.
  const uint32_t nit = (nblk + 1u) / 2u;
  auto blk_of = [&](uint32_t i) __attribute__((always_inline)) { return min(2u * i + set, nblk - 1u); };
  u32x4_t sa[4], sb[4];
  load_blk(blk_of(0u), sa);
  load_blk(blk_of(1u), sb);
  store_blk(0u, sa, blk_of(0u));
  __syncthreads();
  for (uint32_t i = 0;;) {
    load_blk(blk_of(i + 2u), sa);
    if (2u * i + set < nblk) run_blk(0u, 2u * i + set);  // uniform per set
    store_blk(1u, sb, blk_of(i + 1u));
    __syncthreads();
    if (++i >= nit) break;
    load_blk(blk_of(i + 2u), sb);
    if (2u * i + set < nblk) run_blk(1u, 2u * i + set);
    store_blk(0u, sa, blk_of(i + 1u));
    __syncthreads();
    if (++i >= nit) break;
  }
  // The second set's (m, l, O) go to the first through the staging buffers,
  // free after the last barrier: value k of thread stid at s_mo[k][stid]
  // (m and l of both groups, then the 64 O values).
  float* const s_mo = reinterpret_cast<float*>(&s_blk[0][0][0]);
  static_assert((4u + 64u) * 256u * sizeof(float) <= sizeof(s_blk), "the merge fits the staging buffers");
  if (set == 1u) {
#pragma unroll
    for (uint32_t cg = 0; cg < 2; ++cg) {
      s_mo[cg * 256u + stid] = m_run[cg];
      s_mo[(2u + cg) * 256u + stid] = l_run[cg];
#pragma unroll
      for (uint32_t nt = 0; nt < 8; ++nt)
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) s_mo[(4u + 32u * cg + 4u * nt + i) * 256u + stid] = o[cg][nt][i];
    }
  }
  __syncthreads();
  if (set == 1u) return;
  // merge: m = max of the two; each side's l and O scaled by 2^(its m - m)
  // (the second set's factor is 0 where it saw no position of the column)
#pragma unroll
  for (uint32_t cg = 0; cg < 2; ++cg) {
    const float m1 = s_mo[cg * 256u + stid], l1 = s_mo[(2u + cg) * 256u + stid];
    const float m = fmaxf(m_run[cg], m1);  // finite: block 0 holds position 0 of every column
    const float f0 = __builtin_amdgcn_exp2f(m_run[cg] - m), f1 = __builtin_amdgcn_exp2f(m1 - m);
    l_run[cg] = __builtin_fmaf(l1, f1, l_run[cg] * f0);
#pragma unroll
    for (uint32_t nt = 0; nt < 8; ++nt)
#pragma unroll
      for (uint32_t i = 0; i < 4; ++i)
        o[cg][nt][i] = __builtin_fmaf(s_mo[(4u + 32u * cg + 4u * nt + i) * 256u + stid], f1, o[cg][nt][i] * f0);
  }
  // normalise: lane holds O[column col][dims 16 nt + 4 g .. + 3] of each
  // group; l summed over the column's four lanes
#pragma unroll
  for (uint32_t cg = 0; cg < 2; ++cg) {
    float l = l_run[cg];
    l += lane_xor16_f32(l, lane);
    l += lane_xor32_f32(l, lane);
    const float inv = 1.0f / l;
    const uint32_t t = tb + (2u * wave + cg) * TPG + cj;
    if (t < n_tok) {
      uint16_t* orow = out + (static_cast<size_t>(t) * nh + kv * G + ci) * HD + 4u * g;
#pragma unroll
      for (uint32_t nt = 0; nt < 8; ++nt) {
        *reinterpret_cast<u32x2_t*>(orow + 16u * nt) =
            u32x2_t{pack_bf16x2(o[cg][nt][0] * inv, o[cg][nt][1] * inv), pack_bf16x2(o[cg][nt][2] * inv, o[cg][nt][3] * inv)};
      }
    }
  }
}

// ---------------------------------------------------------------------------
// token step ends: embedding row of the state's token, greedy argmax
// ---------------------------------------------------------------------------
// out = bf16(q * s + b) of row state[1] (forward.rs:445-462), one word per
// thread; with ROWS, row tokens[blockIdx.y] into out row blockIdx.y.
template <bool ROWS>
__global__ void __launch_bounds__(256) embed_q4_kernel(const uint32_t* __restrict__ w, const uint16_t* __restrict__ s,
                                                       const uint16_t* __restrict__ b, uint32_t hidden, uint32_t group,
                                                       uint32_t vocab, const int32_t* __restrict__ state,
                                                       uint16_t* __restrict__ out) {
  const uint32_t wi = blockIdx.x * 256u + threadIdx.x;
  if (wi >= hidden / 8u) return;
  const int32_t tk = ROWS ? state[blockIdx.y] : state[1];
  const uint32_t tok = min(static_cast<uint32_t>(max(tk, 0)), vocab - 1u);
  out += ROWS ? static_cast<size_t>(blockIdx.y) * hidden : 0u;
  const uint32_t word = w[static_cast<size_t>(tok) * (hidden / 8u) + wi];
  const size_t gi = static_cast<size_t>(tok) * (hidden / group) + (8u * wi) / group;
  const float sc = bf16_to_f32(s[gi]), bi = bf16_to_f32(b[gi]);
  uint32_t o[4];
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j)
    o[j] = pack_bf16x2(__builtin_fmaf(static_cast<float>((word >> (8 * j)) & 0xfu), sc, bi),
                       __builtin_fmaf(static_cast<float>((word >> (8 * j + 4)) & 0xfu), sc, bi));
  *reinterpret_cast<uint4*>(out + 8u * wi) = make_uint4(o[0], o[1], o[2], o[3]);
}

// Greedy argmax (forward.rs:563-566): the first index of the maximum, NaN never
// wins, 0 when nothing exceeds -inf. Keys order (value, -index): a 64-bit key
// (orderable value bits << 32 | ~index) whose maximum is the answer.
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t i) {
  const uint32_t u = __float_as_uint(v);
  const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);  // monotone in v
  const bool valid = !(v != v) && v > -__builtin_huge_valf();
  return valid ? (static_cast<unsigned long long>(ord) << 32) | static_cast<uint32_t>(~i) : 0ull;
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long k) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const unsigned long long o = __shfl_xor(k, m, 64);
    k = o > k ? o : k;
  }
  return k;
}
__global__ void __launch_bounds__(256) argmax_partial_kernel(const float* __restrict__ x, uint32_t n,
                                                             unsigned long long* __restrict__ part) {
  __shared__ unsigned long long s_w[4];
  const uint32_t per = (n + gridDim.x - 1u) / gridDim.x, a0 = blockIdx.x * per, a1 = min(n, a0 + per);
  unsigned long long best = 0ull;
  for (uint32_t i = a0 + threadIdx.x; i < a1; i += 256u) {
    const unsigned long long k = argmax_key(x[i], i);
    best = k > best ? k : best;
  }
  best = wave_max_u64(best);
  if ((threadIdx.x & 63u) == 0) s_w[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long r = s_w[0];
    for (int w = 1; w < 4; ++w) r = s_w[w] > r ? s_w[w] : r;
    part[blockIdx.x] = r;
  }
}
__global__ void __launch_bounds__(256) argmax_final_kernel(const unsigned long long* __restrict__ part, uint32_t nparts,
                                                           int32_t* __restrict__ state) {
  __shared__ unsigned long long s_w[4];
  unsigned long long best = 0ull;
  for (uint32_t i = threadIdx.x; i < nparts; i += 256u) best = part[i] > best ? part[i] : best;
  best = wave_max_u64(best);
  if ((threadIdx.x & 63u) == 0) s_w[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long r = s_w[0];
    for (int w = 1; w < 4; ++w) r = s_w[w] > r ? s_w[w] : r;
    state[1] = r ? static_cast<int32_t>(~static_cast<uint32_t>(r & 0xffffffffu)) : 0;
    state[0] = state[0] + 1;
  }
}

constexpr uint32_t ARGMAX_PARTS = 256;

// RoPE table entry (p, i) = (cos, sin) of fl32(p * fl32(theta^(-2i/128))), each
// in double and rounded once: the values attn_prep_kernel computes.
__global__ void __launch_bounds__(256) rope_table_kernel(float* __restrict__ table, uint32_t max_len, float theta) {
  const uint32_t e = blockIdx.x * 256u + threadIdx.x;
  if (e >= max_len * 64u) return;
  const uint32_t p = e / 64u, i = e % 64u;
  const float f = static_cast<float>(pow(static_cast<double>(theta), -2.0 * static_cast<double>(i) / 128.0));
  const float angle = static_cast<float>(p) * f;
  table[2u * e] = static_cast<float>(cos(static_cast<double>(angle)));
  table[2u * e + 1u] = static_cast<float>(sin(static_cast<double>(angle)));
}

uint32_t sdpa_splits(uint32_t max_len) {
  const uint32_t blocks = max_len / 32u;
  return blocks < 64u ? blocks : 64u;
}

}  // namespace

namespace obs {

int ensure_rope_table(obs_ctx* ctx, float theta, uint32_t max_len, const float** out) {
  for (const auto& r : ctx->rope_tables)
    if (r.theta == theta && r.len >= max_len) {
      *out = r.table;
      return OBS_OK;
    }
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  OBS_HIP_TRY(ctx, hipStreamIsCapturing(ctx->stream, &cs));
  if (cs != hipStreamCaptureStatusNone)
    return set_error(ctx, OBS_E_INVALID, "RoPE table: run once before capturing (table for theta %g, %u positions)",
                     static_cast<double>(theta), max_len);
  float* t = nullptr;
  OBS_HIP_TRY(ctx, hipMalloc(&t, sizeof(float) * 128u * max_len));
  rope_table_kernel<<<(max_len * 64u + 255u) / 256u, 256, 0, ctx->stream>>>(t, max_len, theta);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    (void)hipFree(t);
    return set_error(ctx, OBS_E_HIP, "RoPE table: %s", hipGetErrorString(e));
  }
  ctx->rope_tables.push_back({t, max_len, theta});
  *out = t;
  return OBS_OK;
}

}  // namespace obs

extern "C" {

int obs_q4_gemv(obs_ctx* ctx, const uint16_t* x, uint32_t in, uint32_t group, const obs_gemv_part* parts,
                uint32_t n_parts, const uint16_t* norm_w, float eps) {
  if (!ctx) return OBS_E_INVALID;
  if (!x || !parts || n_parts == 0 || n_parts > 3) return obs::set_error(ctx, OBS_E_INVALID, "obs_q4_gemv: null x/parts or n_parts not in 1..3");
  if (group != 64 || (in != 2048 && in != 4096))
    return obs::set_error(ctx, OBS_E_SHAPE, "obs_q4_gemv: in must be 2048 or 4096 and group 64 (got %u, %u)", in, group);
  if (!obs::aligned(x, 16)) return obs::set_error(ctx, OBS_E_ALIGN, "obs_q4_gemv: x must be 16-byte aligned");
  if (norm_w && !obs::aligned(norm_w, 16)) return obs::set_error(ctx, OBS_E_ALIGN, "obs_q4_gemv: norm_w must be 16-byte aligned");
  GemvArgs a{};
  a.n_parts = n_parts;
  a.in = in;
  a.norm_w = norm_w;
  a.eps = eps;
  uint64_t total = 0;
  for (uint32_t i = 0; i < n_parts; ++i) {
    const obs_gemv_part& p = parts[i];
    if (!p.w || !p.scales || !p.biases || (!p.y_f32 && !p.y_bf16))
      return obs::set_error(ctx, OBS_E_INVALID, "obs_q4_gemv: part %u has a null pointer", i);
    if (p.residual && !p.y_bf16)
      return obs::set_error(ctx, OBS_E_INVALID, "obs_q4_gemv: part %u: a residual needs the bf16 output", i);
    if (!obs::aligned(p.w, 16)) return obs::set_error(ctx, OBS_E_ALIGN, "obs_q4_gemv: part %u weights must be 16-byte aligned", i);
    a.p[i] = GemvPart{p.w, p.scales, p.biases, p.y_f32, p.y_bf16, p.residual, p.rows};
    total += p.rows;
  }
  if (total == 0) return OBS_OK;
  if (total > 0x7fffffffull) return obs::set_error(ctx, OBS_E_SHAPE, "obs_q4_gemv: too many rows");
  a.total_rows = static_cast<uint32_t>(total);
  // one pass: 4 rows per wave for the projections (more waves in flight),
  // 16 for large matrices (the activation work amortised over more rows)
  const bool big = a.total_rows > 16384u;
  const uint32_t rpw = big ? 16u : 4u;
  const uint32_t grid = (a.total_rows + 4u * rpw - 1u) / (4u * rpw);
  if (in == 2048) {
    if (big)
      OBS_LAUNCH(ctx, "q4_gemv", q4_gemv_kernel<1, 16><<<grid, 256, 0, ctx->stream>>>(x, a));
    else
      OBS_LAUNCH(ctx, "q4_gemv", q4_gemv_kernel<1, 4><<<grid, 256, 0, ctx->stream>>>(x, a));
  } else {
    if (big)  // 8 rows per wave at this width (16 would need more than 256 registers)
      OBS_LAUNCH(ctx, "q4_gemv", q4_gemv_kernel<2, 8><<<(a.total_rows + 31u) / 32u, 256, 0, ctx->stream>>>(x, a));
    else
      OBS_LAUNCH(ctx, "q4_gemv", q4_gemv_kernel<2, 4><<<grid, 256, 0, ctx->stream>>>(x, a));
  }
  return OBS_OK;
}

int obs_attn_prep(obs_ctx* ctx, uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* q_norm,
                  const uint16_t* k_norm, uint16_t* k_cache, uint16_t* v_cache_t, uint32_t n_heads, uint32_t n_kv,
                  uint32_t head_dim, uint32_t max_len, float eps, float theta, const int32_t* state) {
  if (!ctx) return OBS_E_INVALID;
  if (!q || !k || !v || !q_norm || !k_norm || !k_cache || !v_cache_t || !state)
    return obs::set_error(ctx, OBS_E_INVALID, "obs_attn_prep: null pointer");
  if (head_dim != HD || n_heads == 0 || n_kv == 0 || n_heads % n_kv != 0 || n_heads / n_kv > 16 || max_len == 0 ||
      max_len % 32u != 0)
    return obs::set_error(ctx, OBS_E_SHAPE,
                          "obs_attn_prep: head_dim must be 128, n_heads a multiple of n_kv with at most 16 per kv "
                          "head, max_len a multiple of 32 (got %u, %u, %u, %u)", head_dim, n_heads, n_kv, max_len);
  if (!obs::aligned(q, 4) || !obs::aligned(k, 4) || !obs::aligned(v, 4) || !obs::aligned(k_cache, 4))
    return obs::set_error(ctx, OBS_E_ALIGN, "obs_attn_prep: q, k, v and the key cache must be 4-byte aligned");
  const uint32_t heads = n_heads + 2u * n_kv;
  OBS_LAUNCH(ctx, "attn_prep", attn_prep_kernel<false><<<(heads + 3u) / 4u, 256, 0, ctx->stream>>>(
                                   q, k, v, q_norm, k_norm, k_cache, v_cache_t, n_heads, n_kv, max_len, eps, theta, state,
                                   0u, 1u, 0u, 0u, nullptr));
  return OBS_OK;
}

size_t obs_sdpa_workspace(uint32_t n_heads, uint32_t n_kv, uint32_t head_dim, uint32_t max_len) {
  if (head_dim != HD || n_kv == 0 || n_heads % n_kv != 0 || max_len < 32u) return 0;
  return sizeof(float) * static_cast<size_t>(n_kv) * sdpa_splits(max_len) * 16u * (HD + 2u);
}

int obs_sdpa_decode(obs_ctx* ctx, const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache_t, uint16_t* out,
                    uint32_t n_heads, uint32_t n_kv, uint32_t head_dim, uint32_t max_len, const int32_t* state,
                    void* ws, size_t ws_bytes) {
  if (!ctx) return OBS_E_INVALID;
  if (!q || !k_cache || !v_cache_t || !out || !state || !ws)
    return obs::set_error(ctx, OBS_E_INVALID, "obs_sdpa_decode: null pointer");
  if (head_dim != HD || n_heads == 0 || n_kv == 0 || n_heads % n_kv != 0 || n_heads / n_kv > 16 || max_len == 0 ||
      max_len % 32u != 0)
    return obs::set_error(ctx, OBS_E_SHAPE,
                          "obs_sdpa_decode: head_dim must be 128, n_heads a multiple of n_kv with at most 16 per kv "
                          "head, max_len a multiple of 32 (got %u, %u, %u, %u)", head_dim, n_heads, n_kv, max_len);
  const size_t need = obs_sdpa_workspace(n_heads, n_kv, head_dim, max_len);
  if (ws_bytes < need)
    return obs::set_error(ctx, OBS_E_NOMEM, "obs_sdpa_decode: workspace %zu bytes < %zu needed", ws_bytes, need);
  if (!obs::aligned(q, 16) || !obs::aligned(k_cache, 16) || !obs::aligned(v_cache_t, 16) || !obs::aligned(ws, 16))
    return obs::set_error(ctx, OBS_E_ALIGN, "obs_sdpa_decode: q, caches and workspace must be 16-byte aligned");
  const uint32_t splits = sdpa_splits(max_len);
  const float scale_log2 = 1.4426950408889634f / __builtin_sqrtf(static_cast<float>(HD));
  float* w = static_cast<float*>(ws);
  OBS_LAUNCH(ctx, "sdpa_split", sdpa_split_kernel<<<n_kv * splits, 64, 0, ctx->stream>>>(
                                    q, k_cache, v_cache_t, w, n_heads, n_kv, max_len, splits, scale_log2, state));
  OBS_LAUNCH(ctx, "sdpa_combine", sdpa_combine_kernel<<<n_heads, 512, 0, ctx->stream>>>(w, out, n_heads, n_kv, splits));
  return OBS_OK;
}

int obs_embed_q4(obs_ctx* ctx, const uint32_t* w, const uint16_t* scales, const uint16_t* biases, uint32_t hidden,
                 uint32_t group, uint32_t vocab, const int32_t* state, uint16_t* out) {
  if (!ctx) return OBS_E_INVALID;
  if (!w || !scales || !biases || !state || !out) return obs::set_error(ctx, OBS_E_INVALID, "obs_embed_q4: null pointer");
  if (hidden == 0 || vocab == 0 || group == 0 || group % 8u != 0 || hidden % group != 0)
    return obs::set_error(ctx, OBS_E_SHAPE, "obs_embed_q4: hidden must be a multiple of group, group of 8");
  if (!obs::aligned(out, 16)) return obs::set_error(ctx, OBS_E_ALIGN, "obs_embed_q4: out must be 16-byte aligned");
  OBS_LAUNCH(ctx, "embed_q4", embed_q4_kernel<false><<<(hidden / 8u + 255u) / 256u, 256, 0, ctx->stream>>>(
                                  w, scales, biases, hidden, group, vocab, state, out));
  return OBS_OK;
}

int obs_embed_q4_rows(obs_ctx* ctx, const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                      uint32_t hidden, uint32_t group, uint32_t vocab, const int32_t* tokens, uint32_t n_tokens,
                      uint16_t* out) {
  if (!ctx) return OBS_E_INVALID;
  if (!w || !scales || !biases || !tokens || !out)
    return obs::set_error(ctx, OBS_E_INVALID, "obs_embed_q4_rows: null pointer");
  if (hidden == 0 || vocab == 0 || group == 0 || group % 8u != 0 || hidden % group != 0 || n_tokens > 65535u)
    return obs::set_error(ctx, OBS_E_SHAPE,
                          "obs_embed_q4_rows: hidden must be a multiple of group, group of 8, at most 65535 tokens");
  if (!obs::aligned(out, 16) || hidden % 8u != 0)
    return obs::set_error(ctx, OBS_E_ALIGN, "obs_embed_q4_rows: out rows must be 16-byte aligned");
  if (n_tokens == 0) return OBS_OK;
  OBS_LAUNCH(ctx, "embed_q4_rows", embed_q4_kernel<true><<<dim3((hidden / 8u + 255u) / 256u, n_tokens), 256, 0,
                                                         ctx->stream>>>(w, scales, biases, hidden, group, vocab, tokens,
                                                                        out));
  return OBS_OK;
}

int obs_attn_prep_rows(obs_ctx* ctx, uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* q_norm,
                       const uint16_t* k_norm, uint16_t* k_cache, uint16_t* v_cache_t, uint32_t n_heads,
                       uint32_t n_kv, uint32_t head_dim, uint32_t max_len, float eps, float theta, uint32_t pos0,
                       uint32_t n_tokens, uint32_t q_ld, uint32_t kv_ld) {
  if (!ctx) return OBS_E_INVALID;
  q_ld = q_ld ? q_ld : n_heads * head_dim;
  kv_ld = kv_ld ? kv_ld : n_kv * head_dim;
  if (!q || !k || !v || !q_norm || !k_norm || !k_cache || !v_cache_t)
    return obs::set_error(ctx, OBS_E_INVALID, "obs_attn_prep_rows: null pointer");
  if (head_dim != HD || n_heads == 0 || n_kv == 0 || n_heads % n_kv != 0 || n_heads / n_kv > 16 || max_len == 0 ||
      max_len % 32u != 0)
    return obs::set_error(ctx, OBS_E_SHAPE,
                          "obs_attn_prep_rows: head_dim must be 128, n_heads a multiple of n_kv with at most 16 per "
                          "kv head, max_len a multiple of 32 (got %u, %u, %u, %u)", head_dim, n_heads, n_kv, max_len);
  if (static_cast<uint64_t>(pos0) + n_tokens > max_len)
    return obs::set_error(ctx, OBS_E_SHAPE, "obs_attn_prep_rows: positions %u..%u run past the cache (max_len %u)",
                          pos0, pos0 + n_tokens, max_len);
  if (q_ld < n_heads * head_dim || kv_ld < n_kv * head_dim || q_ld % 2u != 0 || kv_ld % 2u != 0)
    return obs::set_error(ctx, OBS_E_SHAPE, "obs_attn_prep_rows: row strides %u, %u must be even and hold a row",
                          q_ld, kv_ld);
  if (!obs::aligned(q, 4) || !obs::aligned(k, 4) || !obs::aligned(v, 4) || !obs::aligned(k_cache, 4))
    return obs::set_error(ctx, OBS_E_ALIGN, "obs_attn_prep_rows: q, k, v and the key cache must be 4-byte aligned");
  if (n_tokens == 0) return OBS_OK;
  if (n_tokens > 0x7fffffffu) return obs::set_error(ctx, OBS_E_SHAPE, "obs_attn_prep_rows: too many tokens");
  const float* rope = nullptr;
  const int rc = obs::ensure_rope_table(ctx, theta, max_len, &rope);
  if (rc != OBS_OK) return rc;
  const uint64_t grid = static_cast<uint64_t>(n_tokens) + static_cast<uint64_t>(n_kv) * ((n_tokens + PREP_VTOK - 1u) / PREP_VTOK);
  if (grid > 0x7fffffffull) return obs::set_error(ctx, OBS_E_SHAPE, "obs_attn_prep_rows: too many tokens");
  OBS_LAUNCH(ctx, "attn_prep_rows", attn_prep_kernel<true><<<static_cast<uint32_t>(grid), 256, 0,
                                                              ctx->stream>>>(q, k, v, q_norm, k_norm, k_cache, v_cache_t,
                                                                             n_heads, n_kv, max_len, eps, theta, nullptr,
                                                                             pos0, n_tokens, q_ld, kv_ld, rope));
  return OBS_OK;
}

int obs_sdpa_prefill(obs_ctx* ctx, const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache_t,
                     uint16_t* out, uint32_t n_heads, uint32_t n_kv, uint32_t head_dim, uint32_t max_len,
                     uint32_t pos0, uint32_t n_tokens, uint32_t q_ld) {
  if (!ctx) return OBS_E_INVALID;
  q_ld = q_ld ? q_ld : n_heads * head_dim;
  if (!q || !k_cache || !v_cache_t || !out) return obs::set_error(ctx, OBS_E_INVALID, "obs_sdpa_prefill: null pointer");
  if (head_dim != HD || n_kv == 0 || n_heads % n_kv != 0 || max_len == 0 || max_len % 32u != 0 ||
      16u % (n_heads / n_kv) != 0)
    return obs::set_error(ctx, OBS_E_SHAPE,
                          "obs_sdpa_prefill: head_dim must be 128, query heads per kv head a divisor of 16, "
                          "max_len a multiple of 32 (got %u, %u, %u, %u)", head_dim, n_heads, n_kv, max_len);
  if (static_cast<uint64_t>(pos0) + n_tokens > max_len)
    return obs::set_error(ctx, OBS_E_SHAPE, "obs_sdpa_prefill: positions %u..%u run past the cache (max_len %u)",
                          pos0, pos0 + n_tokens, max_len);
  if (q_ld < n_heads * head_dim || q_ld % 8u != 0)
    return obs::set_error(ctx, OBS_E_SHAPE, "obs_sdpa_prefill: q row stride %u must be a multiple of 8 holding a row",
                          q_ld);
  if (!obs::aligned(q, 16) || !obs::aligned(k_cache, 16) || !obs::aligned(v_cache_t, 16) || !obs::aligned(out, 16))
    return obs::set_error(ctx, OBS_E_ALIGN, "obs_sdpa_prefill: q, the caches and out must be 16-byte aligned");
  if (n_tokens == 0) return OBS_OK;
  const uint32_t tpwg = 8u * (16u / (n_heads / n_kv));  // tokens per workgroup
  const uint64_t wgs = static_cast<uint64_t>(n_kv) * ((n_tokens + tpwg - 1u) / tpwg);
  if (wgs > 0x7fffffffull) return obs::set_error(ctx, OBS_E_SHAPE, "obs_sdpa_prefill: too many tokens");
  const float scale_log2 = 1.4426950408889634f / __builtin_sqrtf(static_cast<float>(HD));
  OBS_LAUNCH(ctx, "sdpa_prefill", sdpa_prefill_kernel<<<static_cast<uint32_t>(wgs), PF_THREADS, 0, ctx->stream>>>(
                                      q, k_cache, v_cache_t, out, n_heads, n_kv, max_len, pos0, n_tokens, q_ld,
                                      scale_log2));
  return OBS_OK;
}

size_t obs_argmax_workspace(void) { return sizeof(unsigned long long) * ARGMAX_PARTS; }

int obs_argmax(obs_ctx* ctx, const float* x, uint32_t n, int32_t* state, void* ws, size_t ws_bytes) {
  if (!ctx) return OBS_E_INVALID;
  if (!x || !state || !ws) return obs::set_error(ctx, OBS_E_INVALID, "obs_argmax: null pointer");
  if (ws_bytes < obs_argmax_workspace())
    return obs::set_error(ctx, OBS_E_NOMEM, "obs_argmax: workspace %zu bytes < %zu needed", ws_bytes, obs_argmax_workspace());
  if (!obs::aligned(ws, 8)) return obs::set_error(ctx, OBS_E_ALIGN, "obs_argmax: workspace must be 8-byte aligned");
  auto* part = static_cast<unsigned long long*>(ws);
  OBS_LAUNCH(ctx, "argmax_partial", argmax_partial_kernel<<<ARGMAX_PARTS, 256, 0, ctx->stream>>>(x, n, part));
  OBS_LAUNCH(ctx, "argmax_final", argmax_final_kernel<<<1, 256, 0, ctx->stream>>>(part, ARGMAX_PARTS, state));
  return OBS_OK;
}

}  // extern "C"
