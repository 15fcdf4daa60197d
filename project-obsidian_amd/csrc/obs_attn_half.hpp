// obs_attn_half.hpp — the attention half of a decode layer at the
// Qwen3-30B-A3B shape (src/forward.rs:403-418) as one workgroup's part of a
// 256-workgroup launch: attn_fused_kernel (obs_attention_fused.hip) runs it
// alone, layer_fused_kernel (obs_layer_fused.hip) before the MoE half of the
// same layer. The work split, load order and exchanges are described at the
// top of obs_attention_fused.hip.
#pragma once
#include "obs_internal.hpp"

// Phase markers for timing harnesses; no code is generated unless one defines it.
#ifndef OBS_ATTN_MARK
#define OBS_ATTN_MARK(phase)
#endif

namespace {

using namespace obsd;

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr uint32_t AH = 2048, ANH = 32, ANKV = 4, AHD = 128, AG = ANH / ANKV;  // G = 8
constexpr uint32_t AQD = ANH * AHD;                                              // 4096
constexpr uint32_t ANGRP = 8, AWPG = 32, ANWG = ANGRP * AWPG;                   // groups, WGs per group
constexpr uint32_t AQPG = ANH / ANGRP;           // query heads per group: 4
constexpr uint32_t AGQD = AQPG * AHD;            // the group's attention outputs: 512
constexpr uint32_t AGR = AGQD + 2 * AHD;         // q/k/v rows per group: 768
constexpr uint32_t A_RPW = AGR / (AWPG * 4);     // q/k/v rows per wave: 6
constexpr uint32_t A_NSPLIT = AWPG;              // splits of the sequence per group: 32
constexpr uint32_t A_CDIM = AGQD / AWPG;         // combined outputs per workgroup: 16
constexpr uint32_t A_PART = AQPG * (AHD + 2);    // a split's partial: 4 heads x (O[128], m, l)
constexpr uint32_t A_ORWG = AH / AWPG;           // W_o rows per workgroup: 64
constexpr uint32_t A_ORW = A_ORWG / 4;           // per wave: 16, in two passes of 8 (8 lanes per row)
static_assert(A_RPW * AWPG * 4 == AGR && A_CDIM * AWPG == AGQD && AQPG * ANGRP == ANH, "shape");
static_assert(A_RPW == 6, "the q/k/v rows of a wave are reduced six at a time");

constexpr size_t AW_COUNT = 0, AW_ERR = 256;
constexpr size_t AW_QKV = 1024;                                              // [8][768] slots
constexpr size_t AW_PART = AW_QKV + size_t(ANGRP) * AGR * 8;                 // [8][32][520] slots
constexpr size_t AW_ATTN = AW_PART + size_t(ANGRP) * A_NSPLIT * A_PART * 8;  // [8][256] slots: bf16 pairs
constexpr size_t AW_Y = AW_ATTN + size_t(ANGRP) * (AGQD / 2) * 8;            // [8][2048] slots
constexpr size_t AW_BYTES = AW_Y + size_t(ANGRP) * AH * 8;
constexpr uint64_t A_WAIT_TICKS = 10000000ull;  // 100 ms at 100 MHz

struct AttnArgs {
  const uint32_t* q_w; const uint16_t* q_s; const uint16_t* q_b;
  const uint32_t* k_w; const uint16_t* k_s; const uint16_t* k_b;
  const uint32_t* v_w; const uint16_t* v_s; const uint16_t* v_b;
  const uint32_t* o_w; const uint16_t* o_s; const uint16_t* o_b;
  const uint16_t* in_norm; const uint16_t* q_norm; const uint16_t* k_norm;
  const uint16_t* x; uint16_t* x1;
  uint16_t* k_cache; uint16_t* v_cache_t;
  const int32_t* state;
  const float* rope;  // [max_len][64] (cos, sin) pairs, rope_table_kernel
  unsigned char* ws;
  uint32_t max_len;
  float eps, scale_log2;
};

__device__ __forceinline__ float shfl_f(float v, int src) { return __shfl(v, src, 64); }

// Poll n_u slots per thread (slot tid + 256 u of src) until all carry the
// epoch or the wait times out; values in vals. Returns false on a time-out.
template <int NU>
__device__ __forceinline__ bool poll_slots(const uint64_t* src, uint32_t epoch, float (&vals)[NU]) {
  const uint64_t t0 = wall_clock64();
  while (true) {
    bool ready = true;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const uint64_t v = slot_load(src + threadIdx.x + 256u * u);
      vals[u] = slot_val(v);
      ready = ready && slot_ready(v, epoch);
    }
    if (__all(ready)) return true;
    if (wall_clock64() - t0 > A_WAIT_TICKS) return false;
  }
}

// The attention half of a decode layer as one workgroup's part of a
// 256-workgroup launch. MERGED = false: attn_fused_kernel, which counts its
// launches and ends with the layer's x1 in memory. MERGED = true:
// layer_fused_kernel, whose MoE half follows in the same launch. Then the
// workgroup also publishes its 8 rows of x1 as epoch-tagged slots (slot i:
// rows 2i and 2i + 1 as bf16, system scope: read across the XCDs), moe_err
// (the MoE half's error word) stops the launch like the half's own, the
// launch count is left to the caller, *epoch_out is the launch's epoch and
// *x1_row the bf16 of row 256 g + 8 j + lane in lanes 0-7 of wave 0. Returns
// false when an earlier launch's error stopped this one.
template <bool MERGED>
__device__ __forceinline__ bool attn_half(const AttnArgs& a, uint64_t* x1_slots, const uint32_t* moe_err,
                                          uint32_t* x1_row, uint32_t* epoch_out) {
  __shared__ uint32_t s_epoch;
  __shared__ int s_abort, s_fail;
  __shared__ float s_qkv[AGR];                                          // the group's q (4 heads), k, v
  __shared__ __attribute__((aligned(16))) uint16_t s_rot[AQPG + 2][AHD];  // rotated q heads, k, then v (bf16)
  __shared__ float s_pm[4][16], s_pl[4][16];
  __shared__ float s_po[4][AQPG][AHD];
  __shared__ float s_cm[A_NSPLIT], s_cl[A_NSPLIT], s_co[A_NSPLIT][A_CDIM];
  __shared__ float s_rl[16][A_CDIM], s_ra[16][A_CDIM];
  __shared__ __attribute__((aligned(16))) f16x2_t s_ap[AGQD / 2];   // the group's attention output, f16 pairs
  __shared__ float s_asum[AGQD / 32], s_aoff[AGQD / 32];
  __shared__ float s_aup[AGQD / 64];  // the f16 range factor 2^k of each 64 output columns
  __shared__ float s_y[ANGRP][A_ORWG];

  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t g = blockIdx.x % ANGRP, j = blockIdx.x / ANGRP;
  const uint32_t kv = g / 2u, hq0 = AG * kv + AQPG * (g % 2u);  // kv head, first query head
  const uint32_t wl = __builtin_amdgcn_readfirstlane(4u * j + wave);  // wave within the group
  uint64_t* ctl_count = reinterpret_cast<uint64_t*>(a.ws + AW_COUNT);
  uint32_t* ctl_err = reinterpret_cast<uint32_t*>(a.ws + AW_ERR);
  uint64_t* qkv_slots = reinterpret_cast<uint64_t*>(a.ws + AW_QKV) + size_t(g) * AGR;
  uint64_t* part_slots = reinterpret_cast<uint64_t*>(a.ws + AW_PART) + size_t(g) * A_NSPLIT * A_PART;
  uint64_t* attn_slots = reinterpret_cast<uint64_t*>(a.ws + AW_ATTN) + size_t(g) * (AGQD / 2);
  uint64_t* y_slots = reinterpret_cast<uint64_t*>(a.ws + AW_Y);

  OBS_ATTN_MARK(0);
  // ---- 0. loads that the q/k/v rows and the RoPE need, in the order they are
  // used: the position, the activations, the q/k/v rows, the launch count,
  // then the RoPE cosines and sines at the position (the key/value blocks and
  // the o rows come later; see the load order above).
  // the position, as the first vector load (a per-lane index keeps it off the
  // scalar cache, whose load the compiler issued late and which returned only
  // after the flood of row loads): the RoPE load that needs it waits for it
  // alone, the memory counter being in order
  int32_t pos_i;
  {
    uint32_t zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
    pos_i = a.state[zero];
  }
  __builtin_amdgcn_sched_barrier(0);
  uint4 xq[4], nq[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    xq[i] = reinterpret_cast<const uint4*>(a.x + 32u * lane)[i];
    nq[i] = reinterpret_cast<const uint4*>(a.in_norm + 32u * lane)[i];
  }
  // the wave's rows r = 6 wl + k of the group's [q heads | key head | value head]
  uint4 rq[A_RPW];
  uint16_t rsc[A_RPW], rbi[A_RPW];
#pragma unroll
  for (uint32_t k = 0; k < A_RPW; ++k) {
    const uint32_t r = A_RPW * wl + k;  // wave-uniform
    const bool is_q = r < AGQD, is_k = !is_q && r < AGQD + AHD;
    const uint32_t rr = is_q ? AHD * hq0 + r : AHD * kv + (is_k ? r - AGQD : r - AGQD - AHD);
    const uint32_t* w = is_q ? a.q_w : (is_k ? a.k_w : a.v_w);
    const uint16_t* sp = is_q ? a.q_s : (is_k ? a.k_s : a.v_s);
    const uint16_t* bp = is_q ? a.q_b : (is_k ? a.k_b : a.v_b);
    rq[k] = load_stream(reinterpret_cast<const uint4*>(w + static_cast<size_t>(rr) * (AH / 8u)) + lane);
    rsc[k] = sp[static_cast<size_t>(rr) * (AH / 64u) + lane / 2u];
    rbi[k] = bp[static_cast<size_t>(rr) * (AH / 64u) + lane / 2u];
  }
  const uint32_t wq = *reinterpret_cast<const uint32_t*>(a.q_norm + 2u * lane);
  const uint32_t wk = *reinterpret_cast<const uint32_t*>(a.k_norm + 2u * lane);
  // this workgroup's split of the sequence, and the position's loads
  const uint32_t max_len = a.max_len;
  const uint32_t pos = static_cast<uint32_t>(pos_i);
  const bool pos_ok = pos_i >= 0 && pos < max_len;
  const uint32_t seq = static_cast<uint32_t>(min(max(pos_i + 1, 1), static_cast<int32_t>(max_len)));
  const uint32_t nblk = (seq + 31u) / 32u, per = (nblk + A_NSPLIT - 1u) / A_NSPLIT;
  const uint32_t b0 = j * per, b1 = min(nblk, b0 + per);
  const uint32_t col = lane & 15u, gq = lane >> 4;
  const uint16_t* kb = a.k_cache + static_cast<size_t>(kv) * max_len * AHD;
  const uint16_t* vb = a.v_cache_t + static_cast<size_t>(kv) * AHD * max_len;
  // wave w runs blocks b0 + w, b0 + w + 4, ...; its first block's keys go out
  // behind the q/k/v rows, its values after the poll. Row r of score tile tt (the MFMA's A rows) is
  // position t0 + 8 (r / 4) + 4 tt + r % 4 of the 32-position block, so lane
  // (col, gq) ends with the scores of positions t0 + 8 gq .. + 7 and reads
  // their values as one 16-byte run of the transposed value cache.
  u32x4_t ka[2][4];
  u32x4_t va[8];
  auto kpos = [&](uint32_t t0, uint32_t tt) __attribute__((always_inline)) {
    return t0 + 8u * (col >> 2) + 4u * tt + (col & 3u);
  };
  // (keys and values are loaded non-temporally, like the weight rows: a step
  // reads each once, and cached they pushed out what the MoE half reads again)
  auto load_keys = [&](uint32_t blk) __attribute__((always_inline)) {
    const uint32_t t0 = 32u * blk;
#pragma unroll
    for (uint32_t tt = 0; tt < 2; ++tt) {
      const uint16_t* kr = kb + static_cast<size_t>(kpos(t0, tt)) * AHD + 8u * gq;
#pragma unroll
      for (uint32_t ks = 0; ks < 4; ++ks) ka[tt][ks] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(kr + 32u * ks));
    }
  };
  auto load_values = [&](uint32_t blk) __attribute__((always_inline)) {
    const uint32_t t0 = 32u * blk;
#pragma unroll
    for (uint32_t nt = 0; nt < 8; ++nt)
      va[nt] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(vb + static_cast<size_t>(16u * nt + col) * max_len + t0 + 8u * gq));
  };
  auto load_block = [&](uint32_t blk) __attribute__((always_inline)) {
    load_keys(blk);
    load_values(blk);
  };
  // every row load above is issued before anything waits for the position
  // (left alone, the scheduler put that wait ahead of the last row's load)
  __builtin_amdgcn_sched_barrier(0);
  // workgroup 0 adds 1 to the count as it exits, after every workgroup of its
  // launch has read it: it exits after the residual add, which waits for the
  // output partials of workgroup 0 of every group, each of which waited for
  // the attention outputs of every workgroup of its group, each of which read
  // the count before its first publish. So the count is the number of earlier
  // launches (as in decode_fused_kernel). One thread per workgroup
  // loads it, after the rows and before anything that needs the position:
  // these coherent loads go to memory, and from every thread they made a hot
  // spot of two addresses; under a branch they are waited for at its join,
  // which here follows the row loads, needed first anyway.
  uint64_t counted = 0;
  uint32_t err = 0;
  if (tid == 0) {
    counted = __hip_atomic_load(ctl_count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    err = __hip_atomic_load(ctl_err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if constexpr (MERGED) err |= __hip_atomic_load(moe_err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_sched_barrier(0);
  // the lane's RoPE cosines and sines at the position, pairs (2 lane,
  // 2 lane + 1) mod 64: (cos, sin, cos, sin); needed after the first exchange
  const f32x4_t csn = *reinterpret_cast<const f32x4_t*>(a.rope + static_cast<size_t>(min(pos, max_len - 1u)) * 128u +
                                                        4u * (lane & 31u));
  // the keys of the wave's first block (clamped into the sequence when it has
  // none; unused then), behind the rows: they arrive while the q/k/v rows are
  // computed and exchanged, before the poll that waits behind them returns
  load_keys(min(b0 + wave, nblk - 1u));
  __builtin_amdgcn_sched_barrier(0);
  OBS_ATTN_MARK(1);
  // ---- 1. q/k/v rows of rmsnorm(x) (obs_rmsnorm's sequence), rounded to bf16
  {
    float xf[32];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t wd[4] = {xq[i].x, xq[i].y, xq[i].z, xq[i].w};
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        xf[8 * i + 2 * jj] = bf16lo(wd[jj]);
        xf[8 * i + 2 * jj + 1] = bf16hi(wd[jj]);
      }
    }
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < 32; ++c) ss = __builtin_fmaf(xf[c], xf[c], ss);
    const float inv = 1.0f / __builtin_sqrtf(wave_sum_asc(ss) / static_cast<float>(AH) + a.eps);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t wd[4] = {nq[i].x, nq[i].y, nq[i].z, nq[i].w};
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        // rounded to bf16 in pairs (v_cvt_pk_bf16_f32: f32_to_bf16 but for NaN payloads)
        const uint32_t pr = pack_bf16_pair_rne((xf[8 * i + 2 * jj] * inv) * bf16lo(wd[jj]),
                                               (xf[8 * i + 2 * jj + 1] * inv) * bf16hi(wd[jj]));
        xf[8 * i + 2 * jj] = bf16lo(pr);
        xf[8 * i + 2 * jj + 1] = bf16hi(pr);
      }
    }
    float xs = 0.0f;
#pragma unroll
    for (int c = 0; c < 32; ++c) xs = xs + xf[c];
    // the f16 range: the lane's 32 columns scaled by 2^-k at 2^15 and beyond,
    // the rows' dot products by 2^k (k = 0 below)
    const F16Range xr = f16_range(lane_absmax<32>(xf));
#pragma unroll
    for (int c = 0; c < 32; ++c) xf[c] = xf[c] * xr.down;
    f16x2_t xh[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) f16_pairs8(xf + 8 * i, xh + 4 * i);
    float xoff = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) xoff = dot8_off_only(xh + 4 * i, xoff);
    float part[A_RPW];
#pragma unroll
    for (uint32_t k = 0; k < A_RPW; ++k) {
      float acc = 0.0f;
      acc = dot8_q4_off(rq[k].x, xh + 0, acc);
      acc = dot8_q4_off(rq[k].y, xh + 4, acc);
      acc = dot8_q4_off(rq[k].z, xh + 8, acc);
      acc = dot8_q4_off(rq[k].w, xh + 12, acc);
      part[k] = __builtin_fmaf(bf16_to_f32(rsc[k]), (acc - xoff) * xr.up, bf16_to_f32(rbi[k]) * xs);
    }
    // the six 64-lane sums in wave_sum_asc's order (bit-identical to the
    // per-head launches), row my_row in lane l < 8
    const float mine = bf16_to_f32(f32_to_bf16(wave_sum6_scatter(part, lane)));
    const int my_row = lane < 8u ? row6_of_lane(lane) : -1;
    // the epoch is needed from the first publish on: the barrier sits here,
    // after the rows' wait, not before the compute
    if (tid == 0) {
      s_epoch = static_cast<uint32_t>(counted) + 1u;
      s_abort = err != 0u;
      s_fail = 0;
    }
    __syncthreads();
    if (s_abort) {  // a previous launch failed: the host must reset first
      if (tid == 0 && blockIdx.x == 0)
        __hip_atomic_fetch_add(ctl_count, uint64_t{1}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    if (my_row >= 0) slot_store_xcd(qkv_slots + A_RPW * wl + my_row, s_epoch, mine);  // polled by this XCD only
  }
  // the o rows of this wave: rows 64 j + 16 wave + 8 p + lane / 8, the lane's
  // 64 of the group's 512 columns (the quantization group 2 hq0 + lane % 8);
  // loaded after the attention blocks
  const uint32_t orow0 = A_ORWG * j + A_ORW * wave + lane / 8u, oc = lane & 7u;
  uint4 oq[2][2];
  uint16_t osc[2], obi[2];
  const uint32_t epoch = s_epoch;
  OBS_ATTN_MARK(2);

  // ---- 2. this workgroup's split: poll the group's q heads, key and value
  {
    float vals[3];
    if (!poll_slots<3>(qkv_slots, epoch, vals) && lane == 0) s_fail = 1;
#pragma unroll
    for (uint32_t u = 0; u < 3; ++u) s_qkv[tid + 256u * u] = vals[u];
  }
  __syncthreads();
  // the first block's values, now that no poll waits behind them
  load_values(min(b0 + wave, nblk - 1u));
  OBS_ATTN_MARK(3);
  // per-head RMSNorm + NeoX RoPE (attn_prep_kernel's sequence): wave w owns
  // query head w, and wave 0 the key head (head 4) too. Every wave computes the
  // key head beside its own, the two chains interleaved (one after the other,
  // wave 0's dependent reductions and exchanges set this phase's length), and
  // only wave 0 stores it.
  {
    const float cs[2] = {csn[0], csn[2]}, sn[2] = {csn[1], csn[3]};
    const bool first = lane < 32u;
    float xv[2][2], ss[2];
#pragma unroll
    for (uint32_t u = 0; u < 2; ++u) {
      const uint32_t h = u ? AQPG : wave;
      xv[u][0] = s_qkv[h * AHD + 2u * lane];
      xv[u][1] = s_qkv[h * AHD + 2u * lane + 1u];
      ss[u] = __builtin_fmaf(xv[u][1], xv[u][1], __builtin_fmaf(xv[u][0], xv[u][0], 0.0f));
    }
    const float tot[2] = {wave_sum_asc(ss[0]), wave_sum_asc(ss[1])};
#pragma unroll
    for (uint32_t u = 0; u < 2; ++u) {
      const uint32_t h = u ? AQPG : wave, wv = u ? wk : wq;
      const float inv = 1.0f / __builtin_sqrtf(tot[u] / static_cast<float>(AHD) + a.eps);
      const uint32_t npr = pack_bf16_pair_rne((xv[u][0] * inv) * bf16lo(wv), (xv[u][1] * inv) * bf16hi(wv));
      const float n0 = bf16lo(npr), n1 = bf16hi(npr);
      const float p0 = lane_xor32_f32(n0, lane), p1 = lane_xor32_f32(n1, lane);
      float r[2];
#pragma unroll
      for (uint32_t jj = 0; jj < 2; ++jj) {
        const float own = jj ? n1 : n0, other = jj ? p1 : p0;
        const float aa = own * cs[jj], bb = other * sn[jj];
        r[jj] = first ? aa - bb : aa + bb;
      }
      if (u == 0 || wave == 0) *reinterpret_cast<uint32_t*>(&s_rot[h][2u * lane]) = pack_bf16_pair_rne(r[0], r[1]);
    }
    if (wave == 1) {  // the value head, as bf16
      *reinterpret_cast<uint32_t*>(&s_rot[AQPG + 1][2u * lane]) =
          pack_bf16_pair_rne(s_qkv[(AQPG + 1) * AHD + 2u * lane], s_qkv[(AQPG + 1) * AHD + 2u * lane + 1u]);
    }
  }
  __syncthreads();
  OBS_ATTN_MARK(4);
  const uint32_t pblk = pos / 32u;
  // the even group of the kv head appends it (the odd one computes the same
  // key and value and splices them in from registers, like every split does)
  const bool own_pos = pos_ok && pblk >= b0 && pblk < b1 && (g % 2u) == 0u;
  if (own_pos && wave == 0) {
    *reinterpret_cast<uint32_t*>(a.k_cache + (static_cast<size_t>(kv) * max_len + pos) * AHD + 2u * lane) =
        *reinterpret_cast<const uint32_t*>(&s_rot[AQPG][2u * lane]);
  } else if (own_pos && wave == 1) {
    uint16_t* dst = a.v_cache_t + (static_cast<size_t>(kv) * AHD + 2u * lane) * max_len + pos;
    dst[0] = s_rot[AQPG + 1][2u * lane];
    dst[max_len] = s_rot[AQPG + 1][2u * lane + 1u];
  }
  // query slices: B operand, head col (zero for the padding columns 4..15)
  bf16x8_t qb[4];
#pragma unroll
  for (uint32_t ks = 0; ks < 4; ++ks) {
    u32x4_t v = *reinterpret_cast<const u32x4_t*>(&s_rot[min(col, AQPG - 1u)][32u * ks + 8u * gq]);
    if (col >= AQPG) v = u32x4_t{0u, 0u, 0u, 0u};
    qb[ks] = __builtin_bit_cast(bf16x8_t, v);
  }
  float m_run = -__builtin_huge_valf(), l_run = 0.0f;
  f32x4_t o[8];
#pragma unroll
  for (uint32_t nt = 0; nt < 8; ++nt) o[nt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  for (uint32_t blk = b0 + wave; blk < b1; blk += 4u) {
    if (blk != b0 + wave) load_block(blk);
    const uint32_t t0 = 32u * blk;
    if (pblk == blk) {  // uniform: splice this token's key and value (the cache held the old ones)
#pragma unroll
      for (uint32_t tt = 0; tt < 2; ++tt)
        if (kpos(t0, tt) == pos)
#pragma unroll
          for (uint32_t ks = 0; ks < 4; ++ks)
            ka[tt][ks] = *reinterpret_cast<const u32x4_t*>(&s_rot[AQPG][32u * ks + 8u * gq]);
      const uint32_t ta = t0 + 8u * gq;  // this lane's positions ta .. ta + 7, two per word
      if (pos >= ta && pos < ta + 8u) {
        const uint32_t e = pos - ta, wi = e >> 1, sh = 16u * (e & 1u);
#pragma unroll
        for (uint32_t nt = 0; nt < 8; ++nt) {
          const uint32_t vv = s_rot[AQPG + 1][16u * nt + col];
          uint32_t wd = wi == 0u ? va[nt].x : (wi == 1u ? va[nt].y : (wi == 2u ? va[nt].z : va[nt].w));
          wd = (wd & ~(0xffffu << sh)) | (vv << sh);
          va[nt].x = wi == 0u ? wd : va[nt].x;
          va[nt].y = wi == 1u ? wd : va[nt].y;
          va[nt].z = wi == 2u ? wd : va[nt].z;
          va[nt].w = wi == 3u ? wd : va[nt].w;
        }
      }
    }
    f32x4_t s[2];
#pragma unroll
    for (uint32_t tt = 0; tt < 2; ++tt) {
      f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (uint32_t ks = 0; ks < 4; ++ks)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ka[tt][ks]), qb[ks], acc, 0, 0, 0);
      s[tt] = acc;
    }
    float sv[8];
#pragma unroll
    for (uint32_t tt = 0; tt < 2; ++tt)
#pragma unroll
      for (uint32_t i = 0; i < 4; ++i) {
        const uint32_t t = t0 + 8u * gq + 4u * tt + i;
        sv[4 * tt + i] = t < seq ? s[tt][i] * a.scale_log2 : -__builtin_huge_valf();
      }
    float bm = sv[0];
#pragma unroll
    for (uint32_t i = 1; i < 8; ++i) bm = fmaxf(bm, sv[i]);
    bm = fmaxf(bm, lane_xor16_f32(bm, lane));
    bm = fmaxf(bm, lane_xor32_f32(bm, lane));
    const float m_new = fmaxf(m_run, bm);  // finite: every block holds a position < seq
    const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
    uint32_t pw[4];  // p rounded to bf16, in pairs: the A operand of P V as it stands
    float psum = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
      pw[i] = pack_bf16_pair_rne(__builtin_amdgcn_exp2f(sv[2 * i] - m_new), __builtin_amdgcn_exp2f(sv[2 * i + 1] - m_new));
      psum += bf16lo(pw[i]);
      psum += bf16hi(pw[i]);
    }
    l_run = l_run * corr + psum;
    m_run = m_new;
    // the rescale of O; on the wave's first block O is still zero (and corr = 0)
    const bool rescale = blk != b0 + wave;  // uniform
    float ocr[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    if (rescale) {
#pragma unroll
      for (uint32_t i = 0; i < 4; ++i) ocr[i] = shfl_f(corr, static_cast<int>(4u * gq + i));
    }
    const bf16x8_t pa = __builtin_bit_cast(bf16x8_t, u32x4_t{pw[0], pw[1], pw[2], pw[3]});
    const bool tail = t0 + 32u > seq;  // positions past seq read zero values
#pragma unroll
    for (uint32_t nt = 0; nt < 8; ++nt) {
      u32x4_t v = va[nt];
      if (tail) {
        auto keep = [&](uint32_t w, uint32_t t) { return t >= seq ? 0u : (t + 1u >= seq ? (w & 0xffffu) : w); };
        const uint32_t ta = t0 + 8u * gq;
        v.x = keep(v.x, ta);
        v.y = keep(v.y, ta + 2u);
        v.z = keep(v.z, ta + 4u);
        v.w = keep(v.w, ta + 6u);
      }
      const bf16x8_t vbf = __builtin_bit_cast(bf16x8_t, v);
      if (rescale) {
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) o[nt][i] *= ocr[i];
      }
      o[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, vbf, o[nt], 0, 0, 0);
    }
  }
  // the o rows (used after two more exchanges) and the residual of the 8 rows
  // it finishes
#pragma unroll
  for (uint32_t p = 0; p < 2; ++p) {
    const size_t r = orow0 + 8u * p;
    const uint4* op = reinterpret_cast<const uint4*>(a.o_w + r * (AQD / 8u) + (AHD * hq0 + 64u * oc) / 8u);
    oq[p][0] = load_stream(op);
    oq[p][1] = load_stream(op + 1);
    const size_t gi = r * (AQD / 64u) + 2u * hq0 + oc;
    osc[p] = a.o_s[gi];
    obi[p] = a.o_b[gi];
  }
  const uint16_t ores = a.x[256u * g + 8u * j + (lane & 7u)];  // wave 0, lanes 0-7: row 256 g + 8 j + lane
  OBS_ATTN_MARK(5);
  // the wave's partial: m, l per head column (l summed over the four gq lanes), O rows 4 gq + i
  l_run += lane_xor16_f32(l_run, lane);
  l_run += lane_xor32_f32(l_run, lane);
  if (lane < 16u) {
    s_pm[wave][lane] = m_run;
    s_pl[wave][lane] = l_run;
  }
  if (gq == 0u) {
#pragma unroll
    for (uint32_t nt = 0; nt < 8; ++nt)
#pragma unroll
      for (uint32_t i = 0; i < 4; ++i) s_po[wave][i][16u * nt + col] = o[nt][i];
  }
  __syncthreads();
  // merge the four waves (a wave without blocks has m = -inf, l = 0, O = 0) and
  // publish: thread (head h, dims d0 .. d0 + 1)
  {
    uint64_t* dst = part_slots + static_cast<size_t>(j) * A_PART;
    const uint32_t h = tid / 64u, d0 = 2u * (tid % 64u);
    float M = s_pm[0][h];
#pragma unroll
    for (uint32_t w = 1; w < 4; ++w) M = fmaxf(M, s_pm[w][h]);
    float wt[4], L = 0.0f;
#pragma unroll
    for (uint32_t w = 0; w < 4; ++w) {
      wt[w] = s_pm[w][h] == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f(s_pm[w][h] - M);
      L = __builtin_fmaf(s_pl[w][h], wt[w], L);
    }
#pragma unroll
    for (uint32_t d = 0; d < 2; ++d) {
      float acc = 0.0f;
#pragma unroll
      for (uint32_t w = 0; w < 4; ++w) acc = __builtin_fmaf(s_po[w][h][d0 + d], wt[w], acc);
      slot_store_xcd(dst + h * (AHD + 2u) + d0 + d, epoch, acc);
    }
    if (tid % 64u == 0u) {
      slot_store_xcd(dst + h * (AHD + 2u) + AHD, epoch, M);
      slot_store_xcd(dst + h * (AHD + 2u) + AHD + 1u, epoch, L);
    }
  }
  OBS_ATTN_MARK(6);
  // ---- 3. combine query head j / 8 of the group, dims 16 (j % 8) .. + 16, over the 32 splits
  {
    const uint32_t hh = j / 8u, d0 = A_CDIM * (j % 8u);
    const uint32_t s = tid / 8u, q8 = tid % 8u;  // split s, dims d0 + 2 q8, + 1
    const uint64_t* src = part_slots + static_cast<size_t>(s) * A_PART + hh * (AHD + 2u);
    float v[4];
    const uint64_t t0 = wall_clock64();
    bool ok = s_fail == 0;
    while (ok) {
      const uint64_t x0 = slot_load(src + d0 + 2u * q8), x1 = slot_load(src + d0 + 2u * q8 + 1u);
      const uint64_t xm = slot_load(src + AHD), xl = slot_load(src + AHD + 1u);
      v[0] = slot_val(x0);
      v[1] = slot_val(x1);
      v[2] = slot_val(xm);
      v[3] = slot_val(xl);
      const bool ready = slot_ready(x0, epoch) && slot_ready(x1, epoch) && slot_ready(xm, epoch) &&
                         slot_ready(xl, epoch);
      if (__all(ready)) break;
      if (wall_clock64() - t0 > A_WAIT_TICKS) {
        ok = false;
        if (lane == 0) s_fail = 1;
      }
    }
    s_co[s][2u * q8] = v[0];
    s_co[s][2u * q8 + 1u] = v[1];
    if (q8 == 0u) {
      s_cm[s] = v[2];
      s_cl[s] = v[3];
    }
    __syncthreads();
    OBS_ATTN_MARK(7);
    {  // thread (group q, dim d): splits 2 q, 2 q + 1; then the 16 groups in order
      const uint32_t d = tid % A_CDIM, q = tid / A_CDIM;
      float M = -__builtin_huge_valf();
      for (uint32_t k = 0; k < A_NSPLIT; ++k) M = fmaxf(M, s_cm[k]);
      float L = 0.0f, acc = 0.0f;
#pragma unroll
      for (uint32_t k = 2u * q; k < 2u * q + 2u; ++k) {
        const float wt = s_cm[k] == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f(s_cm[k] - M);
        L = __builtin_fmaf(s_cl[k], wt, L);
        acc = __builtin_fmaf(s_co[k][d], wt, acc);
      }
      s_rl[q][d] = L;
      s_ra[q][d] = acc;
    }
    __syncthreads();
    if (wave == 0) {  // lanes 0..15: one dim each; even lanes publish (dim, dim + 1) as a bf16 pair
      float L = 0.0f, acc = 0.0f;
#pragma unroll
      for (uint32_t q = 0; q < 16; ++q) {
        L += s_rl[q][lane & 15u];
        acc += s_ra[q][lane & 15u];
      }
      const uint32_t mine = f32_to_bf16(acc / L);
      const uint32_t next = static_cast<uint32_t>(dpp_i32<DPP_XOR1>(static_cast<int>(mine)));  // lane ^ 1
      if (lane < A_CDIM && (lane & 1u) == 0u)
        slot_store_xcd(attn_slots + (hh * AHD + d0 + lane) / 2u, epoch, __uint_as_float(mine | (next << 16)));
    }
  }
  OBS_ATTN_MARK(8);

  // ---- 4. the group's 512 attention outputs into LDS as f16 pairs in
  // dot8_q4_off order, with the sum and the offset sum of every 32 columns
  {
    float pvf[1];
    const bool ok = s_fail == 0 && poll_slots<1>(attn_slots, epoch, pvf);
    if (!ok && lane == 0) s_fail = 1;
    const uint32_t pv = __float_as_uint(pvf[0]);
    _Float16* ap16 = reinterpret_cast<_Float16*>(s_ap);
    const uint32_t i0 = 2u * tid;  // columns i0 (low half), i0 + 1
    // the f16 range per 64 columns (one quantization group of W_o, 32 lanes):
    // the outputs scaled by 2^-k at 2^15 and beyond, the group's terms by 2^k
    const F16Range asc = f16_range(half_wave_absmax(__builtin_fmaxf(__builtin_fabsf(bf16lo(pv)),
                                                                     __builtin_fabsf(bf16hi(pv)))));
    const _Float16 h0 = static_cast<_Float16>(bf16lo(pv) * asc.down), h1 = static_cast<_Float16>(bf16hi(pv) * asc.down);
    if ((tid & 31u) == 0u) s_aup[tid >> 5] = asc.up;
    const uint32_t j0 = i0 & 7u, j1 = j0 + 1u;
    ap16[(i0 & ~7u) + 2u * (j0 & 3u) + (j0 >> 2)] = h0;
    ap16[(i0 & ~7u) + 2u * (j1 & 3u) + (j1 >> 2)] = h1;
    // per 32 columns = 16 consecutive lanes: the sum and the offset sum of
    // dot8_q4_off (1024 at even positions, 64 at odd ones) over the f16 values
    float sum = static_cast<float>(h0) + static_cast<float>(h1);
    float off = static_cast<float>(h0) * 1024.0f + static_cast<float>(h1) * 64.0f;
    sum = sum + dpp_f32<DPP_XOR1>(sum);
    sum = sum + dpp_f32<DPP_XOR2>(sum);
    sum = sum + dpp_f32<DPP_HALF_MIRROR>(sum);
    sum = sum + dpp_f32<DPP_MIRROR>(sum);
    off = off + dpp_f32<DPP_XOR1>(off);
    off = off + dpp_f32<DPP_XOR2>(off);
    off = off + dpp_f32<DPP_HALF_MIRROR>(off);
    off = off + dpp_f32<DPP_MIRROR>(off);
    if ((tid & 15u) == 0u) {
      s_asum[tid >> 4] = sum;
      s_aoff[tid >> 4] = off;
    }
  }
  __syncthreads();
  OBS_ATTN_MARK(9);
  // partial W_o rows over the group's columns: lane (row 8 p + lane / 8, 64
  // columns 64 (lane % 8) .. of the group's 512 = one quantization group), then
  // the 8 lanes of a row summed
  {
    f16x2_t ah[2][16];
#pragma unroll
    for (uint32_t sg = 0; sg < 2; ++sg) {
      const uint32_t c0 = 64u * oc + 32u * sg;
#pragma unroll
      for (uint32_t i = 0; i < 4; ++i) {
        const uint4 w4 = *reinterpret_cast<const uint4*>(&s_ap[c0 / 2u + 4u * i]);
        ah[sg][4 * i] = as_f16x2(w4.x); ah[sg][4 * i + 1] = as_f16x2(w4.y);
        ah[sg][4 * i + 2] = as_f16x2(w4.z); ah[sg][4 * i + 3] = as_f16x2(w4.w);
      }
    }
    const float asum = s_asum[2u * oc] + s_asum[2u * oc + 1u], aoff = s_aoff[2u * oc] + s_aoff[2u * oc + 1u];
#pragma unroll
    for (uint32_t p = 0; p < 2; ++p) {
      float acc = 0.0f;
#pragma unroll
      for (uint32_t sg = 0; sg < 2; ++sg) {
        acc = dot8_q4_off(oq[p][sg].x, ah[sg] + 0, acc);
        acc = dot8_q4_off(oq[p][sg].y, ah[sg] + 4, acc);
        acc = dot8_q4_off(oq[p][sg].z, ah[sg] + 8, acc);
        acc = dot8_q4_off(oq[p][sg].w, ah[sg] + 12, acc);
      }
      // asum and aoff are sums of the scaled values: the 2^k factor takes the whole term
      const float part =
          group8_sum(s_aup[oc] * __builtin_fmaf(bf16_to_f32(osc[p]), acc - aoff, bf16_to_f32(obi[p]) * asum));
      if (oc == 0u) slot_store(y_slots + size_t(g) * AH + orow0 + 8u * p, epoch, part);  // polled across XCDs
    }
  }
  OBS_ATTN_MARK(10);
  // ---- 5. x1 = x + sum of the 8 groups' partials, rows 256 g + 8 j .. + 8, in
  // every workgroup (wave 0: lane 8 q + i polls group q's row i). Group 0
  // alone, 64 rows per workgroup: decoder 810-811 against 816 tokens/s.
  static_assert(AH == ANGRP * AWPG * 8u, "8 residual rows per workgroup");
  if (wave == 0) {
    const uint32_t row0c = 256u * g + 8u * j;
    bool ok = s_fail == 0;
    const uint64_t t0 = wall_clock64();
    float yv = 0.0f;
    while (ok) {
      const uint64_t v = slot_load(y_slots + size_t(lane >> 3) * AH + row0c + (lane & 7u));  // group lane/8, row lane%8
      yv = slot_val(v);
      if (__all(slot_ready(v, epoch))) break;
      if (wall_clock64() - t0 > A_WAIT_TICKS) {
        ok = false;
        if (lane == 0) s_fail = 1;
      }
    }
    s_y[lane >> 3][lane & 7u] = yv;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    float acc = bf16_to_f32(ores);
#pragma unroll
    for (uint32_t q = 0; q < ANGRP; ++q) acc += s_y[q][lane & 7u];
    const uint32_t xb = f32_to_bf16(acc);
    if (lane < 8u) a.x1[row0c + lane] = static_cast<uint16_t>(xb);
    if constexpr (MERGED) {
      *x1_row = xb;
      const uint32_t next = static_cast<uint32_t>(dpp_i32<DPP_XOR1>(static_cast<int>(xb)));  // lane ^ 1
      if (lane < 8u && (lane & 1u) == 0u)
        slot_store(x1_slots + (row0c + lane) / 2u, s_epoch, __uint_as_float(xb | (next << 16)));
    }
  }
  __syncthreads();
  OBS_ATTN_MARK(11);
  if (tid == 0) {
    if (s_fail) __hip_atomic_store(ctl_err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    // one add per launch (256 adds on one address at the end of a launch
    // delay the next launch by over a microsecond)
    if (!MERGED && blockIdx.x == 0)
      __hip_atomic_fetch_add(ctl_count, uint64_t{1}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if constexpr (MERGED) *epoch_out = s_epoch;
  return true;
}

}  // namespace
