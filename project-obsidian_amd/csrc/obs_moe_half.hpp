// obs_moe_half.hpp — the MoE half of a decode layer (src/forward.rs:421-441)
// as one workgroup's part of a 256-workgroup launch: decode_fused_kernel
// (obs_decode_fused.hip) runs it alone, layer_fused_kernel
// (obs_layer_fused.hip) right after the attention half of the same layer.
// The work split, the exchanges and their measurements are described at the
// top of obs_decode_fused.hip.
#pragma once
#include "obs_internal.hpp"

// Phase markers for timing harnesses; no code is generated unless one defines it.
#ifndef OBS_FUSED_MARK
#define OBS_FUSED_MARK(phase)
#endif

namespace {

using namespace obsd;

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr uint32_t FH = 2048, FI = 768, FK = 8, FG = 64;
constexpr uint32_t NGROUP = 8, WG_PER_GROUP = 32, NWG = NGROUP * WG_PER_GROUP;
constexpr uint32_t MAX_E = 256;
constexpr uint32_t GU_ROWS = FI / (WG_PER_GROUP * 4);  // gate/up rows per wave: 6
constexpr uint32_t DN_ROWS_WG = FH / WG_PER_GROUP;     // down rows per workgroup: 64

constexpr size_t WS_COUNT = 0, WS_ERR = 256;  // WS_COUNT: 64-bit workgroup count
constexpr size_t WS_LOGITS = 1024;                              // [8][MAX_E] slots
constexpr size_t WS_H = WS_LOGITS + size_t(NGROUP) * MAX_E * 8;  // [8][FI] slots
constexpr size_t WS_Y = WS_H + size_t(NGROUP) * FI * 8;          // [8][FH] slots
constexpr size_t WS_BYTES = WS_Y + size_t(NGROUP) * FH * 8;
constexpr uint64_t WAIT_TICKS = 10000000ull;  // 100 ms at 100 MHz

struct FusedArgs {
  const uint32_t* gate_w; const uint16_t* gate_s; const uint16_t* gate_b;
  const uint32_t* up_w; const uint16_t* up_s; const uint16_t* up_b;
  const uint32_t* down_w; const uint16_t* down_s; const uint16_t* down_b;
  const uint32_t* router_w; const uint16_t* router_s; const uint16_t* router_b;
  const uint16_t* x; const uint16_t* residual; uint16_t* y;
  const uint16_t* norm_w;  // nullable: rmsnorm the input first (forward.rs:419-421)
  float rms_eps;
  int32_t* ids_out; float* w_out;
  unsigned char* ws;
  uint32_t n_exp;
  int norm_topk;
  int route_rule;
};

__device__ __forceinline__ void raise_error(unsigned char* ws) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(ws + WS_ERR), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Gate/up rows whose lane partials are reduced together (a batch of 6 made h
// visible all at once and measured slower: blocks of h then arrive together).
constexpr uint32_t GU_BATCH = 2;

// The 64-lane sums of a wave's lane partials of 2 gate rows (pg) and 2 up rows
// (pu), reduced together, and silu(gate) * up of each row. Instead of a full
// butterfly per value (4 of them cost ~60 instructions plus their DPP hazards
// and readlanes, and each row's silu), the values are reduce-scattered over
// the lanes of a 16-lane row: at each step two lanes that hold the same set
// of values split it, each keeping half and adding its partner's copy of that
// half, until every lane of the row holds the row's sum of one value. The
// pairings are the row mirror (lane bit 3 splits gate from up) and the
// half-row mirror (bit 2 splits the two rows); lanes paired at one step agree
// in every bit split before. Two quad xors, an xor by 16 and a swap of the
// wave's halves then add the rest. Gate row r ends up in the lanes with bit 3
// clear and bit 2 = r, its up row 8 lanes higher, so one row rotation brings
// them together; `row` is the batch row lanes 0 and 4 hold (-1 elsewhere).
__device__ __forceinline__ float gateup_reduce(const float (&pg)[GU_BATCH], const float (&pu)[GU_BATCH], uint32_t lane,
                                               int& row) {
  const bool s1 = (lane & 8u) != 0u, s2 = (lane & 4u) != 0u;
  float a[GU_BATCH];
#pragma unroll
  for (uint32_t i = 0; i < GU_BATCH; ++i) a[i] = (s1 ? pu[i] : pg[i]) + dpp_f32<DPP_MIRROR>(s1 ? pg[i] : pu[i]);
  float d = (s2 ? a[1] : a[0]) + dpp_f32<DPP_HALF_MIRROR>(s2 ? a[0] : a[1]);
  d = d + dpp_f32<DPP_XOR2>(d);
  d = d + dpp_f32<DPP_XOR1>(d);
  row = lane < 8u && (lane & 3u) == 0u ? (s2 ? 1 : 0) : -1;
  d = d + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(d), 0x401F));  // lanes i, i ^ 16
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(d), __float_as_uint(d), false, false);
    d = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);  // lanes i, i ^ 32
  }
  return silu_mul_fast(d, dpp_f32<DPP_ROW_ROR8>(d));  // h is rounded to f16 for the down rows
}

__device__ __forceinline__ void unpack_bf16x8(const uint4& v, float* f) {
  f[0] = bf16lo(v.x); f[1] = bf16hi(v.x); f[2] = bf16lo(v.y); f[3] = bf16hi(v.y);
  f[4] = bf16lo(v.z); f[5] = bf16hi(v.z); f[6] = bf16lo(v.w); f[7] = bf16hi(v.w);
}

// Where the MoE half's input x comes from: memory (decode_fused_kernel, which
// also counts its launches for the epoch), or the epoch-tagged slots that the
// attention half of the same launch publishes (layer_fused_kernel: the caller
// passes the launch's epoch, has checked the error flag, hands over the
// residual row in a register and counts the launch itself).
enum MoeXSource : int { MOE_X_MEM = 0, MOE_X_SLOTS = 1 };

// x slots: slot i holds bf16 columns 2i (low half) and 2i + 1 (high half) of x
// tagged with the launch's epoch; wave w polls slots 256 w .. + 256 into LDS,
// and then lane l of every wave reads its columns 32 l .. + 32 there.
// res_bits: with MOE_X_SLOTS, the bf16 residual of row 256 g + 8 j + lane in
// lanes 0-7 of wave 0 (the rows this workgroup combines).
// NQ = router logit slots per lane: 2 for up to 128 experts, 4 for up to 256.
// NORM: the layer has a post-attention norm weight (rmsnorm of the input
// first). Run by 256 workgroups of 256 threads, one per CU.
template <int NQ, bool NORM, int XSRC>
__device__ __forceinline__ void moe_half(const FusedArgs& a, unsigned char* ws, uint32_t epoch_in,
                                         const uint64_t* x_slots, uint32_t res_bits) {
  constexpr int RT = NQ / 2;  // router rows per wave
  __shared__ uint32_t s_epoch;
  __shared__ int s_abort;
  __shared__ float s_y[FK][64];
  __shared__ __attribute__((aligned(16))) double s_ck[4][MAX_E / 4];  // routing: each wave's share of the keys
  __shared__ uint32_t s_cnt[4][MAX_E];                                // routing: each wave's partial counts
  __shared__ int32_t s_sel_id[FK];                                    // routing: expert of each rank (-1: none)
  __shared__ float s_sel_p[FK];                                       // routing: its p
  __shared__ __attribute__((aligned(16))) f16x2_t s_hp[FI / 2];  // h as f16 pairs, dot8_q4_off order
  __shared__ float s_hsum[FI / 32], s_hoff[FI / 32];              // per 32 columns: sum h, sum off*h
  __shared__ __attribute__((aligned(16))) uint16_t s_sc[4][1536];  // per wave: staged scales (see phase 3)

  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t g = blockIdx.x % NGROUP, j = blockIdx.x / NGROUP;
  uint64_t* ctl_count = reinterpret_cast<uint64_t*>(ws + WS_COUNT);
  const uint32_t* ctl_err = reinterpret_cast<const uint32_t*>(ws + WS_ERR);
  uint64_t* logit_slots = reinterpret_cast<uint64_t*>(ws + WS_LOGITS) + size_t(g) * MAX_E;
  uint64_t* h_slots = reinterpret_cast<uint64_t*>(ws + WS_H) + size_t(g) * FI;
  uint64_t* y_slots = reinterpret_cast<uint64_t*>(ws + WS_Y);
  const uint32_t n_exp = a.n_exp;

  OBS_FUSED_MARK(0);
  // this lane's 32 input columns [32*lane, 32*lane + 32)
  uint4 xq[4], nq[4];
  {
    if constexpr (XSRC == MOE_X_MEM) {
      const uint4* xp = reinterpret_cast<const uint4*>(a.x + 32u * lane);
#pragma unroll
      for (int i = 0; i < 4; ++i) xq[i] = xp[i];
    }
    if constexpr (NORM) {
      const uint4* np = reinterpret_cast<const uint4*>(a.norm_w + 32u * lane);
#pragma unroll
      for (int i = 0; i < 4; ++i) nq[i] = np[i];
    }
  }
  // router rows of this wave: e = 4j + wave (+128)
  const uint32_t e0 = 4u * j + wave;
  uint4 rq[RT][2];
  uint16_t rs[RT], rb[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) {  // unconditional (a clamped row when e >= n_exp, unused then)
    const uint32_t e = min(e0 + 128u * t, n_exp - 1u);
    const uint4* rp = reinterpret_cast<const uint4*>(a.router_w + size_t(e) * (FH / 4) + 8u * lane);
    rq[t][0] = rp[0];
    rq[t][1] = rp[1];
    rs[t] = a.router_s[size_t(e) * (FH / FG) + lane / 2u];
    rb[t] = a.router_b[size_t(e) * (FH / FG) + lane / 2u];
  }
  if (tid < FK) s_sel_id[tid] = -1;
  uint32_t epoch = epoch_in;
  if constexpr (XSRC == MOE_X_MEM) {
  // after the activation and router loads, so its two reads overlap them
  if (tid == 0) {
    // Workgroup 0 adds 1 to the count as it exits, and only after every
    // workgroup of its launch has read it: it exits after the combine, which
    // waits for the outputs of workgroup 0 of every group, each of which waited
    // for h from every workgroup of its group, each of which read the count
    // before writing h. Every earlier launch has added its 1 (the kernel
    // boundary completes it), so the count is the number of earlier launches.
    const uint64_t counted = __hip_atomic_load(ctl_count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t err = __hip_atomic_load(ctl_err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // both in flight
    s_epoch = static_cast<uint32_t>(counted) + 1u;
    s_abort = err != 0u;
  }
  __syncthreads();
  epoch = s_epoch;
  if (s_abort) {  // a previous launch failed: the host must reset first
    if (tid == 0 && blockIdx.x == 0)
      __hip_atomic_fetch_add(ctl_count, uint64_t{1}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  } else {
    // x from the slots the attention half published across the XCDs: wave w
    // polls slots 256 w .. + 256 (4 a lane, coalesced) into LDS, then every
    // lane reads its 32 columns.
    __shared__ __attribute__((aligned(16))) uint32_t s_x[FH / 2];
    const uint64_t t0 = wall_clock64();
    uint64_t v[4];
    while (true) {
      bool ready = true;
#pragma unroll
      for (uint32_t k = 0; k < 4; ++k) {
        v[k] = slot_load(x_slots + 256u * wave + lane + 64u * k);
        ready = ready && slot_ready(v[k], epoch);
      }
      if (__all(ready)) break;
      if (wall_clock64() - t0 > WAIT_TICKS) {
        if (lane == 0) raise_error(ws);
        break;
      }
    }
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) s_x[256u * wave + lane + 64u * k] = static_cast<uint32_t>(v[k]);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) xq[i] = reinterpret_cast<const uint4*>(s_x + 16u * lane)[i];
  }
  OBS_FUSED_MARK(1);

  float xf[32];
#pragma unroll
  for (int i = 0; i < 4; ++i) unpack_bf16x8(xq[i], xf + 8 * i);
  if constexpr (NORM) {
    // RMSNorm in obs_rmsnorm's sequence (the lane owns 2048/64 contiguous
    // columns): serial fma of x^2, wave butterfly, 1/sqrt(ss/2048 + eps), then
    // x*inv*w rounded to bf16 — bit-identical to the standalone kernel.
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < 32; ++c) ss = __builtin_fmaf(xf[c], xf[c], ss);
    const float inv = 1.0f / __builtin_sqrtf(wave_sum_asc(ss) / static_cast<float>(FH) + a.rms_eps);
    float wf[32];
#pragma unroll
    for (int i = 0; i < 4; ++i) unpack_bf16x8(nq[i], wf + 8 * i);
#pragma unroll
    for (int c = 0; c < 32; c += 2) {  // rounded to bf16 in pairs (v_cvt_pk_bf16_f32: f32_to_bf16 but for NaN payloads)
      const uint32_t pr = pack_bf16_pair_rne((xf[c] * inv) * wf[c], (xf[c + 1] * inv) * wf[c + 1]);
      xf[c] = bf16lo(pr);
      xf[c + 1] = bf16hi(pr);
    }
  }
  // ---- 1. router logits (order of obs_q8_gate_logits: serial fma, then wave_sum_asc)
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const uint32_t e = e0 + 128u * t;
    if (e < n_exp) {  // wave-uniform
      const float sc = bf16_to_f32(rs[t]), bi = bf16_to_f32(rb[t]);
      const uint32_t wd[8] = {rq[t][0].x, rq[t][0].y, rq[t][0].z, rq[t][0].w,
                              rq[t][1].x, rq[t][1].y, rq[t][1].z, rq[t][1].w};
      float acc = 0.0f;
#pragma unroll
      for (int c = 0; c < 32; ++c) {
        const float wv = __builtin_fmaf(static_cast<float>((wd[c >> 2] >> (8 * (c & 3))) & 0xffu), sc, bi);
        acc = __builtin_fmaf(wv, xf[c], acc);
      }
      acc = wave_sum_asc(acc);
      if (lane == 0) slot_store_xcd(logit_slots + e, epoch, acc);  // polled by this XCD only
    }
  }
  // While the logits travel: the lane's 32 activations as f16 pairs for the
  // expert rows, their sum and the offset part of dot8_q4_off over them
  // (shared by every row).
  // (The f16 range: the lane's 32 columns are scaled by 2^-k when their
  // largest magnitude reaches 2^15, and the rows' dot products by 2^k.)
  float xs = 0.0f;
#pragma unroll
  for (int c = 0; c < 32; ++c) xs = xs + xf[c];
  const F16Range xr = f16_range(lane_absmax<32>(xf));
  f16x2_t xh[16];
  if (__any(xr.down != 1.0f)) {
#pragma unroll
    for (int c = 0; c < 32; ++c) xf[c] = xf[c] * xr.down;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) f16_pairs8(xf + 8 * i, xh + 4 * i);
  float xoff = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) xoff = dot8_off_only(xh + 4 * i, xoff);

  OBS_FUSED_MARK(2);
  // ---- 2. routing (moe_routing_topk.metal:24-56). Every wave polls its
  // group's logits and turns them into selection keys itself (route_keys: the
  // softmax p of each expert, from the f16-rounded logits under the reference
  // rule), so all four waves hold the same keys without an exchange. The k
  // argmax rounds of the reference (largest p, lowest id on ties) select
  // exactly the experts that fewer than k others precede in that order, in
  // that order; composite keys (p << 9) | (511 - id) make the order strict.
  // Each wave counts, for all experts (NQ per lane), the composites that
  // exceed theirs among its quarter of the experts (read back from its own LDS
  // area as broadcasts), and one barrier adds the four partial counts. The
  // composites are integers below 2^40 held as doubles, so v - ck is exact and
  // at least 1 when v > ck: the subtraction with the output clamp to [0, 1] is
  // the compare's 0 or 1, and a second fp64 add counts it. No compare writes a
  // lane mask that the next instruction must wait for (64-bit integer compares
  // into a mask and a carry-add: 0.65 us for the count; the sign bit of the
  // subtraction, shifted and added: 2.5 instructions a compare, 0.08 us per
  // layer slower than these 2).
  bool ok = true;
  float lg[NQ];
  {
    const uint64_t t0 = wall_clock64();
    while (true) {
      // all slot loads in flight together (clamped index, no per-load branch)
      uint64_t v[NQ];
#pragma unroll
      for (int q = 0; q < NQ; ++q) v[q] = slot_load(logit_slots + min(lane + 64u * q, n_exp - 1u));
      bool ready = true;
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        lg[q] = slot_val(v[q]);
        ready = ready && slot_ready(v[q], epoch);
      }
      if (__all(ready)) break;
      if (wall_clock64() - t0 > WAIT_TICKS) { ok = false; break; }
    }
  }
  OBS_FUSED_MARK(9);
  if (!ok && lane == 0) raise_error(ws);
  int key[NQ];
  route_keys<NQ>(lg, n_exp, lane, a.route_rule, key);
  constexpr uint32_t QW = 16u * NQ;  // experts per wave's share: [QW * wave, QW * (wave + 1))
  double ck[NQ];  // (p << 9) | (511 - id), or 0 for an absent expert and a NaN p
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const uint32_t id = lane + 64u * q;
    ck[q] = key[q] >= 0 ? __builtin_fma(static_cast<double>(key[q]), 512.0, static_cast<double>(511u - id)) : 0.0;
    if (id / QW == wave) s_ck[wave][id % QW] = ck[q];
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // the wave's own LDS stores before its reads
  __builtin_amdgcn_wave_barrier();
  {
    double c[NQ][2];  // two sums per expert, so each add chain is half as long
#pragma unroll
    for (int q = 0; q < NQ; ++q) c[q][0] = c[q][1] = -0.0;  // -0.0 + x is x: the first add folds away
    const double2* cw = reinterpret_cast<const double2*>(s_ck[wave]);
#pragma unroll
    for (uint32_t i = 0; i < QW / 2; ++i) {
      const double2 v = cw[i];
#pragma unroll
      for (int q = 0; q < NQ; ++q) {  // min/max with 0 and 1 fold into v_add_f64's clamp
        c[q][0] += __builtin_fmin(__builtin_fmax(v.x - ck[q], 0.0), 1.0);
        c[q][1] += __builtin_fmin(__builtin_fmax(v.y - ck[q], 0.0), 1.0);
      }
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) s_cnt[wave][lane + 64u * q] = static_cast<uint32_t>(c[q][0] + c[q][1]);
  }
  __syncthreads();
  // rank of each of the lane's experts; the group's expert has rank g
  uint32_t rank[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const uint32_t id = lane + 64u * q;
    rank[q] = (s_cnt[0][id] + s_cnt[1][id]) + (s_cnt[2][id] + s_cnt[3][id]);
  }
  int32_t eg = -1;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const unsigned long long m = __ballot(ck[q] != 0.0 && rank[q] == g);
    eg = m ? static_cast<int32_t>(64u * q + static_cast<uint32_t>(__builtin_ctzll(m))) : eg;
  }
  const bool have = ok && eg >= 0 && static_cast<uint32_t>(eg) < n_exp;
  OBS_FUSED_MARK(3);

  // ---- 3. issue the weight loads: 6 gate + 6 up rows and the down scales (the
  // down rows follow in phase 4).
  // Wide loads only: each gate/up row is one coalesced 1 KB load; the down rows
  // are read a 128-byte line per 8 lanes (lane (r8, m) takes bytes
  // [128L + 16m, +16) of row r8, L = 0..2: columns [256L + 32m, +32)); the
  // scales and biases the wave needs (24 gate/up segments of 64 bytes, 2 x 384
  // contiguous down bytes) come in 3 16-byte loads per lane and are spread
  // through the wave's own LDS area, not one 2-byte load per value.
  uint4 gq[GU_ROWS], uq[GU_ROWS];
  uint4 dq[2][3];
  const uint4* dpp[2];
  const uint32_t m = lane & 7u;   // down: 16-byte chunk within each 128-byte line
  const uint32_t r8 = lane >> 3;  // down: row within an 8-row pass
  const uint32_t dn_row0 = DN_ROWS_WG * j + 16u * wave;  // the wave's 16 down rows
  u32x4_t scq0, scq1, scq2;  // native vectors (a uint4 array stored through a pointer went to scratch)
  {
    // Unconditional (a valid expert when this group has none, results unused):
    // loads under a branch make the compiler wait for all of them at the join.
    const uint32_t el = have ? static_cast<uint32_t>(eg) : 0u;
    const size_t eoff_gu = size_t(el) * FI;
    // Loads in the order they are consumed (the memory counter is in order): the
    // gate/up scales and rows, then the down scales (the down rows' addresses
    // are set here, their loads issued in phase 4). Lanes past the last chunk
    // reload a valid one, so no load is predicated.
#pragma unroll
    for (uint32_t i = 0; i < 2; ++i) {  // chunk c = 16 bytes of segment c/4 = (row t, array)
      const uint32_t c = min(lane + 64u * i, GU_ROWS * 16u - 1u), sg = c / 4u, t = sg / 4u, arr = sg % 4u;
      const uint16_t* base = arr == 0u ? a.gate_s : arr == 1u ? a.gate_b : arr == 2u ? a.up_s : a.up_b;
      const uint4 v = load_stream(base + (eoff_gu + e0 + 128u * t) * (FH / FG) + 8u * (c % 4u));
      if (i == 0) scq0 = u32x4_t{v.x, v.y, v.z, v.w}; else scq1 = u32x4_t{v.x, v.y, v.z, v.w};
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the issue order (see above)
#pragma unroll
    for (uint32_t t = 0; t < GU_ROWS; ++t) {
      const size_t row = eoff_gu + e0 + 128u * t;
      gq[t] = load_stream(reinterpret_cast<const uint4*>(a.gate_w + row * (FH / 8)) + lane);
      uq[t] = load_stream(reinterpret_cast<const uint4*>(a.up_w + row * (FH / 8)) + lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    {  // down scales (chunks 0..23) and biases (24..47) of the wave's 16 rows
      const uint32_t c = min(lane, 47u);
      const uint4 v = load_stream((c < 24u ? a.down_s : a.down_b) + (size_t(el) * FH + dn_row0) * (FI / FG) +
                                  8u * (c % 24u));
      scq2 = u32x4_t{v.x, v.y, v.z, v.w};
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (uint32_t p = 0; p < 2; ++p) {
      const size_t row = size_t(el) * FH + dn_row0 + 8u * p + r8;
      dpp[p] = reinterpret_cast<const uint4*>(a.down_w + row * (FI / 8)) + m;
    }
  }
  // the wave's staged scales: gate/up segment sg = 4t + {gate_s, gate_b, up_s,
  // up_b} at [32 sg], down scales at [1024 + 12 r], down biases at [1216 + 12 r]
  const uint16_t* sc16 = s_sc[wave];

  // The selected experts and their p, by rank, for the combine's weights: the
  // lane of wave 0 holding a selected expert writes it (read after the h
  // exchange's barriers; the ranks no expert takes keep the -1 set at the start).
  if (wave == 0) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      if (ck[q] != 0.0 && rank[q] < FK) {
        s_sel_id[rank[q]] = static_cast<int32_t>(lane + 64u * q);
        s_sel_p[rank[q]] = __int_as_float(key[q]);
      }
    }
  }

  OBS_FUSED_MARK(4);
  // ---- 4. gate/up rows -> h slots (factored per group: s*sum(q x) + b*sum(x))
  {  // the wave's own LDS area: no barrier (its LDS accesses run in order)
    u32x4_t* sc = reinterpret_cast<u32x4_t*>(s_sc[wave]);
    sc[lane] = scq0;
    sc[64u + lane] = scq1;  // chunks 96..127: padding
  }
  // this lane's group's scale and bias of every row, read at once (one LDS wait)
  uint16_t rsb[GU_ROWS][4];
#pragma unroll
  for (uint32_t t = 0; t < GU_ROWS; ++t) {
    const uint16_t* sg = sc16 + 128u * t + lane / 2u;
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) rsb[t][q] = sg[32u * q];  // gate s, gate b, up s, up b
  }
#pragma unroll
  for (uint32_t t0 = 0; t0 < GU_ROWS; t0 += GU_BATCH) {
    float pg[GU_BATCH], pu[GU_BATCH];
#pragma unroll
    for (uint32_t i = 0; i < GU_BATCH; ++i) {
      const uint32_t t = t0 + i;
      float ag = 0.0f, au = 0.0f;
      ag = dot8_q4_off(gq[t].x, xh + 0, ag);
      ag = dot8_q4_off(gq[t].y, xh + 4, ag);
      ag = dot8_q4_off(gq[t].z, xh + 8, ag);
      ag = dot8_q4_off(gq[t].w, xh + 12, ag);
      au = dot8_q4_off(uq[t].x, xh + 0, au);
      au = dot8_q4_off(uq[t].y, xh + 4, au);
      au = dot8_q4_off(uq[t].z, xh + 8, au);
      au = dot8_q4_off(uq[t].w, xh + 12, au);
      pg[i] = __builtin_fmaf(bf16_to_f32(rsb[t][0]), (ag - xoff) * xr.up, bf16_to_f32(rsb[t][1]) * xs);
      pu[i] = __builtin_fmaf(bf16_to_f32(rsb[t][2]), (au - xoff) * xr.up, bf16_to_f32(rsb[t][3]) * xs);
    }
    int row;
    float hv = gateup_reduce(pg, pu, lane, row);
    hv = have ? hv : 0.0f;  // without an expert the rows are expert 0's, loaded but not used
    if (row >= 0) slot_store_xcd(h_slots + e0 + 128u * (t0 + row), epoch, hv);  // polled by this XCD only
    if (t0 == 2u) {
      // The down rows, between the second and the last gate/up batch: issued
      // with the gate/up rows they competed with them for bandwidth, and the h
      // polls below wait for them (a wave's loads complete in issue order), so
      // issued here they are in flight during the last batch and the exchange.
      // Per layer (48-layer sweep, timing build, graph replay): blocks 1 and 2
      // after the first h poll and block 0 with the gate/up rows 13.40 us;
      // blocks 1 and 2 here 13.17; all three here 12.93 (after the first batch
      // 13.12; the down scales here too 13.02).
#pragma unroll
      for (uint32_t p = 0; p < 2; ++p) {
        dq[p][0] = load_stream(dpp[p]);
        dq[p][1] = load_stream(dpp[p] + 8);
        dq[p][2] = load_stream(dpp[p] + 16);
      }
    }
  }

  OBS_FUSED_MARK(5);
  // ---- 5/6. h arrives in three 256-column blocks. Block L = h[256L, 256L + 256)
  // holds every workgroup's rows t = 2L and 2L + 1, which it finishes before
  // its later rows, so the blocks become visible in order. The first poll of
  // all three blocks is issued at once (one slot per thread and block), so a
  // workgroup whose blocks are all complete by then, the last one of its group
  // among them, spends one round trip on them instead of three; a block not yet
  // complete is polled again on its own. Each block goes to LDS as f16 in the
  // pair order of dot8_q4_off with the sum and the offset sum of every 32
  // columns (32 consecutive columns sit in one half-wave), and its terms are
  // added to the workgroup's 64 down rows (of expert e_g, unscaled by w_g) while the later
  // blocks are still being computed. The terms are added in block order, as a
  // single pass over the row would add them.
  reinterpret_cast<u32x4_t*>(s_sc[wave])[128u + lane] = scq2;  // down scales; chunks 176..191: padding
  float part[2] = {0.0f, 0.0f};
  {
    _Float16* hp16 = reinterpret_cast<_Float16*>(s_hp);
    const uint64_t t0 = wall_clock64();
    uint64_t hq[3];
#pragma unroll
    for (uint32_t L = 0; L < 3; ++L) hq[L] = slot_load(h_slots + tid + 256u * L);
#pragma unroll
    for (uint32_t L = 0; L < 3; ++L) {
      uint64_t v = hq[L];
      bool wave_ok = ok;
      while (wave_ok && !__all(slot_ready(v, epoch))) {
        if (wall_clock64() - t0 > WAIT_TICKS) {
          wave_ok = false;
          if (lane == 0) raise_error(ws);
        }
        v = slot_load(h_slots + tid + 256u * L);
      }
      const float hv = slot_val(v);
      ok = ok && wave_ok;
      {
        const uint32_t idx = tid + 256u * L, jn = idx & 7u;  // column idx = 8 * word + jn
        const _Float16 h16 = static_cast<_Float16>(hv);
        hp16[(idx & ~7u) + 2u * (jn & 3u) + (jn >> 2)] = h16;
        // offsets of dot8_q4_off: 1024 at even nibble positions, 64 at odd ones;
        // the sums use the f16-rounded values the dot products see
        const float hr = static_cast<float>(h16);
        const float sum = half_wave_sum(hr);
        const float off = half_wave_sum(hr * ((jn & 1u) ? 64.0f : 1024.0f));
        if ((idx & 31u) == 0u) {
          s_hsum[idx >> 5] = sum;
          s_hoff[idx >> 5] = off;
        }
      }
      __syncthreads();
      if (L == 0) OBS_FUSED_MARK(6);
      // the lane's columns of block L: [256L + 32m, +32)
      f16x2_t hp[16];
#pragma unroll
      for (uint32_t c = 0; c < 16; c += 4) {
        const uint4 v = *reinterpret_cast<const uint4*>(s_hp + 128u * L + 16u * m + c);
        hp[c] = as_f16x2(v.x); hp[c + 1] = as_f16x2(v.y);
        hp[c + 2] = as_f16x2(v.z); hp[c + 3] = as_f16x2(v.w);
      }
      const float hsum = s_hsum[8u * L + m], hoff = s_hoff[8u * L + m];
      if (have) {
#pragma unroll
        for (uint32_t p = 0; p < 2; ++p) {
          const uint16_t* dsb = sc16 + 1024u + 12u * (8u * p + r8);
          float acc = 0.0f;
          acc = dot8_q4_off(dq[p][L].x, hp + 0, acc);
          acc = dot8_q4_off(dq[p][L].y, hp + 4, acc);
          acc = dot8_q4_off(dq[p][L].z, hp + 8, acc);
          acc = dot8_q4_off(dq[p][L].w, hp + 12, acc);
          const uint32_t gi = 4u * L + m / 2u;  // quantization group of block L
          part[p] = part[p] + __builtin_fmaf(bf16_to_f32(dsb[gi]), acc - hoff, bf16_to_f32(dsb[192u + gi]) * hsum);
        }
      }
    }
  }
  // The f16 range of h. An h of 2^15 or more may round to an infinite f16,
  // which makes its rows' sums NaN (inf - inf). A wave holding such a sum
  // recomputes its two rows without the LDS copy: each lane reads its 32
  // columns of every block from the h slots (this launch's values, already
  // seen complete), scales them by 2^-k below 2^15 (f16_range), and adds the
  // block's terms times 2^k. Checking the sums once here keeps the blocks'
  // exchange path as it is (a check per block measured 0.07 us per layer).
  if (__any(!__builtin_isfinite(part[0]) || !__builtin_isfinite(part[1]))) {
    part[0] = part[1] = 0.0f;
#pragma unroll
    for (uint32_t L = 0; L < 3; ++L) {
      float hc[32];
#pragma unroll
      for (uint32_t c = 0; c < 32; ++c) hc[c] = slot_val(slot_load(h_slots + 256u * L + 32u * m + c));
      const F16Range r = f16_range(lane_absmax<32>(hc));
      float hsum = 0.0f;
#pragma unroll
      for (uint32_t c = 0; c < 32; ++c) {
        hc[c] = static_cast<float>(static_cast<_Float16>(hc[c] * r.down));  // the f16 values the dot products see
        hsum = hsum + hc[c];
      }
      f16x2_t hp[16];
#pragma unroll
      for (uint32_t i = 0; i < 4; ++i) f16_pairs8(hc + 8 * i, hp + 4 * i);
      float hoff = 0.0f;
#pragma unroll
      for (uint32_t i = 0; i < 4; ++i) hoff = dot8_off_only(hp + 4 * i, hoff);
      if (have) {
#pragma unroll
        for (uint32_t p = 0; p < 2; ++p) {
          const uint16_t* dsb = sc16 + 1024u + 12u * (8u * p + r8);
          float acc = 0.0f;
          acc = dot8_q4_off(dq[p][L].x, hp + 0, acc);
          acc = dot8_q4_off(dq[p][L].y, hp + 4, acc);
          acc = dot8_q4_off(dq[p][L].z, hp + 8, acc);
          acc = dot8_q4_off(dq[p][L].w, hp + 12, acc);
          const uint32_t gi = 4u * L + m / 2u;
          part[p] = part[p] + r.up * __builtin_fmaf(bf16_to_f32(dsb[gi]), acc - hoff, bf16_to_f32(dsb[192u + gi]) * hsum);
        }
      }
    }
  }
#pragma unroll
  for (uint32_t p = 0; p < 2; ++p) {
    const float v = group8_sum(part[p]);
    const uint32_t row = dn_row0 + 8u * p + r8;
    if (m == 0) slot_store(y_slots + size_t(g) * FH + row, epoch, v);
  }

  OBS_FUSED_MARK(7);
  // ---- 7. every workgroup combines the 8 ranks for its 8 rows 256 g + 8 j ..
  // in rank order (wave 0: lane 8 r + i polls rank r's row i). Group 0 alone,
  // 64 rows per workgroup: 10.87 against 10.66 us per layer.
  if (wave == 0) {
    // the routing weights (moe_routing_topk.metal:47-55): lane r < 8 holds rank
    // r's; wsum is the serial sum of the selected p in rank order
    const int32_t sel_id = lane < FK ? s_sel_id[lane] : -1;
    float wsum = 0.0f;
#pragma unroll
    for (uint32_t r = 0; r < FK; ++r) wsum = s_sel_id[r] >= 0 ? wsum + s_sel_p[r] : wsum;
    const float sel_w =
        sel_id >= 0 ? route_weight(s_sel_p[lane & (FK - 1u)], wsum, a.norm_topk, a.route_rule) : 0.0f;
    if (blockIdx.x == 0 && lane < FK) {
      if (a.ids_out) a.ids_out[lane] = sel_id;
      if (a.w_out) a.w_out[lane] = sel_w;
    }
    const uint32_t row0c = 256u * g + 8u * j;
    bool wave_ok = ok;
    const uint64_t t0 = wall_clock64();
    float yv = 0.0f;
    while (wave_ok) {
      const uint64_t v = slot_load(y_slots + size_t(lane >> 3) * FH + row0c + (lane & 7u));  // rank lane/8, row lane%8
      yv = slot_val(v);
      if (__all(slot_ready(v, epoch))) break;
      if (wall_clock64() - t0 > WAIT_TICKS) {
        wave_ok = false;
        if (lane == 0) raise_error(ws);
      }
    }
    s_y[lane >> 3][lane & 7u] = yv;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    if (lane < 8u) {
      const uint32_t o = row0c + lane;
      float acc;
      if constexpr (XSRC == MOE_X_SLOTS)
        acc = bf16_to_f32(static_cast<uint16_t>(res_bits));
      else
        acc = a.residual ? bf16_to_f32(a.residual[o]) : 0.0f;
#pragma unroll
      for (uint32_t r = 0; r < FK; ++r) acc = __builtin_fmaf(readlane_f32(sel_w, static_cast<int>(r)), s_y[r][lane], acc);
      a.y[o] = f32_to_bf16(acc);
    }
  }

  OBS_FUSED_MARK(8);
  // ---- 8. exit: workgroup 0 counts the launch (a no-return add). One add per
  // workgroup, 256 on one address at the end of the launch, delayed the next
  // launch by ~1.3 us (12.04 against 10.75 us per layer on the 48-layer sweep).
  if constexpr (XSRC == MOE_X_MEM) {
    if (tid == 0 && blockIdx.x == 0)
      __hip_atomic_fetch_add(ctl_count, uint64_t{1}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace
