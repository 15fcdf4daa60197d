// obs_internal.hpp — shared internals of libobsidian_hip (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>
#include <type_traits>
#include <vector>

#include "../../include/obsidian_hip.h"

// ---------------------------------------------------------------------------
// Context
// ---------------------------------------------------------------------------
struct obs_prof_pair {
  const char* name;
  hipEvent_t e0, e1;
};
struct obs_prof_stat {
  const char* name;
  double total_ms;
  int64_t launches;
};

struct obs_ctx {
  int device = 0;
  int num_cus = 0;
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;  // own_stream or a caller stream
  hipEvent_t ev_start = nullptr, ev_stop = nullptr;
  std::string err;
  // decode workspace (logits, ids, weights, h), grown on demand
  void* decode_ws = nullptr;
  size_t decode_ws_bytes = 0;
  // fused decode workspace (epoch-tagged exchange slots + counters), zeroed once
  void* fused_ws = nullptr;
  // fused attention-half workspace (exchange slots + counters), zeroed once
  void* attn_ws = nullptr;
  // one-launch decode layer workspace (both halves' slots, the x1 slots and
  // one launch counter), zeroed once
  void* layer_ws = nullptr;
  // this device's file-scope scratch array (obs_moe_decode_static), looked up
  // once per device by obs_create; null if the lookup was not possible
  void* scratch = nullptr;
  bool scratch_used = false;  // obs_device_status then checks its error flag too
  // RoPE (cos, sin) tables [len][64][2] fp32, one per (theta, length) built;
  // a graph captured with one keeps reading it, so none is freed before
  // obs_destroy (a call uses the first table of its theta that is long enough)
  struct rope_entry {
    float* table;
    uint32_t len;
    float theta;
  };
  std::vector<rope_entry> rope_tables;
  // decode workspaces replaced by larger ones, kept for the same reason
  std::vector<void*> retired;
  int decode_path = 0;  // OBS_DECODE_AUTO / _MULTI / _FUSED
  // Context-owned device status words (obs::CTX_ST_*), zeroed by obs_create,
  // read and cleared by obs_device_status: the one-launch prefill FFN's flags.
  uint32_t* status_dev = nullptr;
  // The one-launch router's counter (obs_route), zeroed by obs_create; the
  // workgroup that routes sets it back to 0.
  uint32_t* route_cnt = nullptr;
  // Dispatch facts the one-launch kernels build on, probed by obs_create
  // (obs::probe_dispatch): the workgroups b of one b % 8 share an XCD (8
  // groups, 8 XCDs), and an XCD starts its workgroups in index order.
  bool xcd_map_ok = false;
  bool inorder_ok = false;
  // Test hook (obs_debug_ffn_wait): counts the one-launch FFN's down items
  // wait for beyond their tile's gate/up items, and their wait limit (ticks of
  // the 100 MHz constant clock).
  uint32_t ffn_extra_count = 0;
  uint64_t ffn_wait_ticks = 10000000ull;
  // in-stream kernel timing
  bool prof_on = false;
  std::vector<obs_prof_pair> prof_pairs;
  std::vector<obs_prof_stat> prof_stats;
};

struct obs_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

namespace obs {

// The scratch of obs_moe_decode_static: one file-scope device array per GPU
// (obs_context.hip), the fused decode's exchange area followed by the
// 4-launch path's logits / ids / weights / h / normalised x at the largest
// shape obs_moe_decode accepts (E 256, top_k 8, inter 2048, hidden 4096).
constexpr size_t STATIC_FUSED_BYTES = 197632;
constexpr size_t STATIC_MULTI_BYTES = 1024 + 256 + 256 + 8 * 2048 * 4 + 4096 * 2;
constexpr size_t STATIC_SCRATCH_BYTES = STATIC_FUSED_BYTES + STATIC_MULTI_BYTES;

int set_error(obs_ctx* ctx, int code, const char* fmt, ...);

// Words of obs_ctx::status_dev.
enum : uint32_t {
  CTX_ST_FFN_WAIT = 0,   // a one-launch FFN down item's wait for its tile timed out
  CTX_ST_FFN_SCHED = 1,  // a one-launch FFN work table did not fit its launch
  CTX_ST_WORDS = 64
};
// Words of the one-launch router's counter block in the context (word 0 is
// the count of its working workgroups).
constexpr uint32_t ROUTE_CNT_WORDS = 64;

// Which one-launch paths a device may take (OBS_PATH_* bits of
// obs_dispatch_gate): the fused decode and fused attention need all 256 of
// their workgroups resident, one per CU, and each group b % 8 on one XCD; the
// one-launch prefill FFN needs the XCD map and in-order dispatch per XCD.
uint32_t dispatch_gate(int num_cus, bool xcd_map_ok, bool inorder_ok);
// Runs the dispatch probe kernels on the context's device and records the facts.
int probe_dispatch(obs_ctx* ctx);
// Per-context setup of the grouped GEMM kernels (LDS limits raised once).
int prefill_init(obs_ctx* ctx);

// Kernel bracketing for obs_profile_*: call prof_begin before a launch and
// prof_end after it; both are no-ops unless profiling is enabled.
int prof_begin(obs_ctx* ctx, const char* name);
int prof_end(obs_ctx* ctx);

#define OBS_HIP_TRY(ctx, call)                                                   \
  do {                                                                           \
    hipError_t e_ = (call);                                                      \
    if (e_ != hipSuccess)                                                        \
      return ::obs::set_error((ctx), OBS_E_HIP, "%s failed: %s", #call,          \
                              hipGetErrorString(e_));                            \
  } while (0)

// Checks the launch just issued (invalid configuration and the like).
#define OBS_LAUNCH_CHECK(ctx) OBS_HIP_TRY(ctx, hipGetLastError())

// Launch statement bracketed for in-stream timing, then checked.
#define OBS_LAUNCH(ctx, name, ...)                         \
  do {                                                     \
    int rc_ = ::obs::prof_begin((ctx), (name));            \
    if (rc_) return rc_;                                   \
    __VA_ARGS__;                                           \
    OBS_LAUNCH_CHECK(ctx);                                 \
    rc_ = ::obs::prof_end(ctx);                            \
    if (rc_) return rc_;                                   \
  } while (0)

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Workspace for decode: returns device pointer of at least `bytes`.
int ensure_decode_ws(obs_ctx* ctx, size_t bytes, void** out);

// RMSNorm of rows x dim bf16 (obs_elementwise.hip); dim % 64 == 0, <= 8192.
int launch_rmsnorm(obs_ctx* ctx, const uint16_t* x, const uint16_t* w, uint16_t* out, uint32_t rows, uint32_t dim,
                   float eps);

// Fused single-launch decode (obs_decode_fused.hip).
bool fused_decode_supported(const obs_moe_config* cfg);
uint32_t fused_decode_workgroups();  // workgroups of one launch (each needs a CU of its own)
uint32_t fused_attn_workgroups();    // the same for the fused attention half (obs_attention_fused.hip)
size_t fused_decode_ws_bytes();
int launch_fused_decode(obs_ctx* ctx, const obs_moe_config* cfg, const obs_moe_layer* L, const uint16_t* x,
                        const uint16_t* residual, uint16_t* y, int32_t* ids_out, float* w_out);
// The same launch on a caller-provided exchange area of fused_decode_ws_bytes()
// (zeroed before its first use; never cleared between launches).
int launch_fused_decode_ws(obs_ctx* ctx, const obs_moe_config* cfg, const obs_moe_layer* L, const uint16_t* x,
                           const uint16_t* residual, uint16_t* y, int32_t* ids_out, float* w_out, void* ws);
// Reads and clears the fused path's device error flag (synchronizes).
int fused_decode_status(obs_ctx* ctx);
// The same for an exchange area `ws` (resets it when the flag is set).
int fused_decode_status_ws(obs_ctx* ctx, void* ws);

// Fused attention half of a decode layer (obs_attention_fused.hip): its
// device error flag, read and cleared (synchronizes).
int attn_fused_status(obs_ctx* ctx);
int ffn_status(obs_ctx* ctx);  // the one-launch prefill FFN's wait flag
// The one-launch attention half's arguments (obs_attn_decode, obs_layer_decode).
int check_attn_decode(obs_ctx* ctx, const char* who, const obs_attn_layer* L, const uint16_t* x,
                      const uint16_t* k_cache, const uint16_t* v_cache_t, const int32_t* state, const uint16_t* x1,
                      uint32_t max_len);
// The MoE half's configuration and layer tensors (obs_decode.hip).
int check_moe_config(obs_ctx* ctx, const char* who, const obs_moe_config* cfg);
int check_moe_layer(obs_ctx* ctx, const char* who, const obs_moe_layer* L);
// One-launch decode layer (obs_layer_fused.hip): its device error flags, read
// and cleared (synchronizes).
int layer_fused_status(obs_ctx* ctx);

// The context's RoPE table for (theta, max_len) (obs_attention.hip): entry
// [p][i] = (cos, sin) of fl32(p * fl32(theta^(-2i/128))), each evaluated in
// double and rounded once (attn_prep_kernel's values). Built on first use
// (not under graph capture).
int ensure_rope_table(obs_ctx* ctx, float theta, uint32_t max_len, const float** out);

}  // namespace obs

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
namespace obsd {

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
// low / high bf16 of a packed pair
__device__ __forceinline__ float bf16lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

// fp32 -> bf16, round to nearest even, NaN kept quiet. Written as a select:
// an early return for NaN compiled to a divergent branch per value.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t nan = (u >> 16) | 0x40u;
  return static_cast<uint16_t>((u & 0x7fffffffu) > 0x7f800000u ? nan : rne);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}
// The same pair with one v_cvt_pk_bf16_f32 (round to nearest even, as
// f32_to_bf16 for every value that is not a NaN).
__device__ __forceinline__ uint32_t pack_bf16_pair_rne(float lo, float hi) {
  typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
  typedef float f32x2_v __attribute__((ext_vector_type(2)));
  const f32x2_v f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_v));
}

// exp(x) by Cody-Waite reduction with ln2 = HI + LO and a degree-7 Taylor
// polynomial (|r| <= ln2/2, truncation error < 6e-9 relative); every step is a
// correctly rounded fp32 operation, so the result is reproducible bit for bit
// on any IEEE fp32 machine that evaluates the same sequence. Results below the
// normal range underflow gradually, as IEEE exp does: p * 2^n is formed as
// (p * 2^(n+64)) * 2^-64, one rounding into the subnormals. x < -104 -> +0
// (exp(-104) is below half the smallest subnormal), x > 88.5 -> +inf, NaN -> NaN.
// Branch-free: the polynomial runs on x clamped into [-104, 88.5] and the
// special cases are selected at the end (a branch per case made the routing
// wave diverge and reconverge around every call).
__device__ __forceinline__ float exp_det(float x) {
  const float xc = __builtin_fminf(__builtin_fmaxf(x, -104.0f), 88.5f);
  const float LOG2E = 1.44269502162933349609375f;
  const float LN2_HI = 0.693145751953125f;
  const float LN2_LO = 1.428606765330187045e-06f;
  const float n = __builtin_rintf(xc * LOG2E);
  float r = __builtin_fmaf(-n, LN2_HI, xc);
  r = __builtin_fmaf(-n, LN2_LO, r);
  float p = 1.98412698e-04f;
  p = __builtin_fmaf(p, r, 1.38888889e-03f);
  p = __builtin_fmaf(p, r, 8.33333333e-03f);
  p = __builtin_fmaf(p, r, 4.16666667e-02f);
  p = __builtin_fmaf(p, r, 1.66666667e-01f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int ni = static_cast<int>(n);
  const bool big = ni > 127;
  p = big ? p * 2.0f : p;
  ni = big ? ni - 1 : ni;
  const bool tiny = ni < -126;  // the result is subnormal: scale by 2^(n+64), then by 2^-64
  float res = p * __uint_as_float(static_cast<uint32_t>(ni + (tiny ? 64 : 0) + 127) << 23);
  res = tiny ? res * 0x1p-64f : res;
  res = x < -104.0f ? 0.0f : res;
  res = x > 88.5f ? __builtin_huge_valf() : res;
  return x != x ? x : res;
}

// fp32 -> f16 (round to nearest even) -> fp32: the value a half holds
__device__ __forceinline__ float round_f16(float v) { return static_cast<float>(static_cast<_Float16>(v)); }

// silu(g) * u with the deterministic exp (ops.metal:21 form).
__device__ __forceinline__ float silu_mul(float g, float u) { return (g / (1.0f + exp_det(-g))) * u; }

// silu(g) * u with the hardware exp2 and reciprocal (about 2 ulp in fp32), for
// results rounded to bf16 or f16 right after: the grouped GEMM's epilogue and
// the fused decode's h.
__device__ __forceinline__ float silu_mul_fast(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(-g * 1.44269504088896341f);
  return (g * __builtin_amdgcn_rcpf(1.0f + e)) * u;
}

// Sum over the 8 nibbles of `w` of q_j * x[j] (nibble j = (w >> 4j) & 15),
// fp32 fma chain in nibble order. The nibbles are split into the bytes of two
// words so each converts with one byte-to-float instruction.
__device__ __forceinline__ float dot8_q4(uint32_t w, const float* x, float acc) {
  const uint32_t lo = w & 0x0f0f0f0fu;         // nibbles 0,2,4,6 in bytes 0..3
  const uint32_t hi = (w >> 4) & 0x0f0f0f0fu;  // nibbles 1,3,5,7
  acc = __builtin_fmaf(static_cast<float>(lo & 0xffu), x[0], acc);
  acc = __builtin_fmaf(static_cast<float>(hi & 0xffu), x[1], acc);
  acc = __builtin_fmaf(static_cast<float>((lo >> 8) & 0xffu), x[2], acc);
  acc = __builtin_fmaf(static_cast<float>((hi >> 8) & 0xffu), x[3], acc);
  acc = __builtin_fmaf(static_cast<float>((lo >> 16) & 0xffu), x[4], acc);
  acc = __builtin_fmaf(static_cast<float>((hi >> 16) & 0xffu), x[5], acc);
  acc = __builtin_fmaf(static_cast<float>(lo >> 24), x[6], acc);
  acc = __builtin_fmaf(static_cast<float>(hi >> 24), x[7], acc);
  return acc;
}

// ---- DPP cross-lane primitives (gfx9 DPP controls) -------------------------
constexpr int DPP_XOR1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141; // lane i <- lane 7-i within each 8-lane half row
constexpr int DPP_MIRROR = 0x140;      // lane i <- lane 15-i within each 16-lane row

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
__device__ __forceinline__ float readlane_f32(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Xor-butterfly sum over 64 lanes with ascending offsets 1, 2, 4, 8, 16, 32;
// the result is returned on every lane. Offsets 1 and 2 are quad
// permutations; on quad-uniform (then half-row-uniform) data the half-row and
// row mirrors pair exactly the lanes an xor by 4 (then 8) would; the last two
// steps combine the four row sums as (r0 + r1) + (r2 + r3). fp32 addition is
// commutative, so this is value-for-value the textbook butterfly.
__device__ __forceinline__ float wave_sum_asc(float v) {
  v = v + dpp_f32<DPP_XOR1>(v);
  v = v + dpp_f32<DPP_XOR2>(v);
  v = v + dpp_f32<DPP_HALF_MIRROR>(v);
  v = v + dpp_f32<DPP_MIRROR>(v);
  const float r0 = readlane_f32(v, 0), r1 = readlane_f32(v, 16);
  const float r2 = readlane_f32(v, 32), r3 = readlane_f32(v, 48);
  return (r0 + r1) + (r2 + r3);
}

constexpr int DPP_ROW_SHL4 = 0x104;  // lane i <- lane i + 4 within the row
constexpr int DPP_ROW_SHR4 = 0x114;  // lane i <- lane i - 4 within the row
constexpr int DPP_ROW_ROR8 = 0x128;  // lane i <- lane (i + 8) mod 16 within the row: an xor by 8

// Lane i ^ 4's value on any data (the half-row mirror pairs the same lanes
// only on quad-uniform data): banks 0 and 2 of each row (lanes 0-3, 8-11)
// read 4 lanes up, banks 1 and 3 read 4 lanes down.
__device__ __forceinline__ float dpp_xor4_f32(float v) {
  int r = __builtin_amdgcn_update_dpp(0, __float_as_int(v), DPP_ROW_SHL4, 0xF, 0x5, false);
  r = __builtin_amdgcn_update_dpp(r, __float_as_int(v), DPP_ROW_SHR4, 0xF, 0xA, false);
  return __int_as_float(r);
}

// A 16-byte load of data read once per use, such as expert weight rows and
// their scales (global_load_dwordx4 ... nt). Marking the weight stream
// non-temporal keeps the small data that is read again (router rows,
// activations, exchange slots) cached: measured on the 48-layer decode sweep,
// the router rows arrive 0.3 us sooner and a layer takes 12.48 us instead of
// 13.00.
typedef uint32_t u32x4_nt_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream(const void* p) {
  const u32x4_nt_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt_t*>(p));
  return uint4{v.x, v.y, v.z, v.w};
}

// Lane i ^ 32's and lane i ^ 16's values through the VALU's half and row swaps
// (v_permlane32_swap, v_permlane16_swap) instead of a ds_bpermute round trip
// through the LDS crossbar. With both operands v, the swap returns v with its
// upper half (odd rows) replaced by the lower half (even rows), and v with its
// lower half (even rows) replaced by the upper half (odd rows).
__device__ __forceinline__ float lane_xor32_f32(float v, uint32_t lane) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(lane < 32u ? r[1] : r[0]);
}
__device__ __forceinline__ float lane_xor16_f32(float v, uint32_t lane) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((lane & 16u) ? r[0] : r[1]);
}

// The wave_sum_asc of six values at once, bit for bit: the same pairs are
// added in the same order (xor 1, 2, 4, 8 within a row, then the four row sums
// as (r0 + r1) + (r2 + r3)), but at the first three steps the two lanes of a
// pair split the values they hold (each keeps half and adds its partner's
// copy of that half) instead of both adding all of them: 3 + 2 + 1 + 1 + 1 + 1
// additions per lane instead of 6 x 6, and no scalar reads. Lane l < 8 returns
// the sum of value row6_of_lane(l) (lanes 6 and 7 hold padding).
__device__ __forceinline__ int row6_of_lane(uint32_t lane) {
  const uint32_t b0 = lane & 1u, b1 = (lane >> 1) & 1u, b2 = (lane >> 2) & 1u;
  const int i = b1 ? (b2 ? -1 : 1) : (b2 ? 2 : 0);
  return i < 0 ? -1 : static_cast<int>(3u * b0) + i;
}
__device__ __forceinline__ float wave_sum6_scatter(const float (&v)[6], uint32_t lane) {
  const bool b0 = (lane & 1u) != 0u, b1 = (lane & 2u) != 0u, b2 = (lane & 4u) != 0u;
  float a[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) a[i] = (b0 ? v[3 + i] : v[i]) + dpp_f32<DPP_XOR1>(b0 ? v[i] : v[3 + i]);
  const float c0 = (b1 ? a[1] : a[0]) + dpp_f32<DPP_XOR2>(b1 ? a[0] : a[1]);
  const float c1 = (b1 ? 0.0f : a[2]) + dpp_f32<DPP_XOR2>(b1 ? a[2] : 0.0f);
  float d = (b2 ? c1 : c0) + dpp_xor4_f32(b2 ? c0 : c1);
  d = d + dpp_f32<DPP_ROW_ROR8>(d);
  d = d + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(d), 0x401F));  // lanes i, i ^ 16
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(d), __float_as_uint(d), false, false);
  return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);  // lanes i, i ^ 32
}

// Sum over each aligned group of 8 lanes (xor offsets 1, 2, 4); uniform in the group.
__device__ __forceinline__ float group8_sum(float v) {
  v = v + dpp_f32<DPP_XOR1>(v);
  v = v + dpp_f32<DPP_XOR2>(v);
  v = v + dpp_f32<DPP_HALF_MIRROR>(v);
  return v;
}

// Sum over each 32-lane half of the wave (every lane of the half gets it).
// Epoch-tagged exchange slots between the workgroups of one launch:
// (epoch << 32) | fp32 bits, so a reader knows a value is this launch's from
// the value itself (no flag, no fence, no clearing between launches). Stores
// are system-scope (written through to memory): measured on MI355X, an
// agent-scope store polled by an agent-scope load from a CU of the same XCD
// takes ~2.7 us to become visible, a write-through store ~0.55 us.
__device__ __forceinline__ void slot_store(uint64_t* p, uint32_t epoch, float v) {
  __hip_atomic_store(p, (static_cast<uint64_t>(epoch) << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_SYSTEM);
}
// Exchange between workgroups of one XCD: a plain store (no write-through)
// stays in the XCD's L2, where the agent-scope poll of slot_load reads it.
// Measured on MI355X with two workgroups of one XCD: 0.27 us one way, against
// 0.40 us for the write-through store; the line never queues behind HBM
// traffic. Across XCDs such a store is not seen (each XCD has its own L2), so
// only slots that one XCD both writes and polls use it.
__device__ __forceinline__ void slot_store_xcd(uint64_t* p, uint32_t epoch, float v) {
  __hip_atomic_store(p, (static_cast<uint64_t>(epoch) << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_WAVEFRONT);
}
__device__ __forceinline__ uint64_t slot_load(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool slot_ready(uint64_t v, uint32_t epoch) {
  return static_cast<uint32_t>(v >> 32) == epoch;
}
__device__ __forceinline__ float slot_val(uint64_t v) { return __uint_as_float(static_cast<uint32_t>(v)); }

__device__ __forceinline__ float half_wave_sum(float v) {
  v = v + dpp_f32<DPP_XOR1>(v);
  v = v + dpp_f32<DPP_XOR2>(v);
  v = v + dpp_f32<DPP_HALF_MIRROR>(v);
  v = v + dpp_f32<DPP_MIRROR>(v);
  // lanes i and i^16 within each 32-lane group: ds_swizzle bit mode, xor mask 16
  return v + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
}

// ---- 4-bit dot products through f16 pairs (v_dot2_f32_f16) -------------------
// A nibble q becomes an exact f16 by OR-ing it into the mantissa of a constant:
// at bits 3:0 of 0x6400 (1024.0) it reads 1024 + q, at bits 7:4 of 0x5400 (64.0)
// it reads 64 + q (one mantissa unit there is 1/16 of 16 = 1). So for a word w
// holding nibbles q0..q7 of columns c..c+7,
//   (w & 0x000F000F) | 0x64006400        = (1024 + q0, 1024 + q4)
//   (w & 0x00F000F0) | 0x54005400        = (  64 + q1,   64 + q5)
//   ((w>>8) & 0x000F000F) | 0x64006400   = (1024 + q2, 1024 + q6)
//   ((w>>8) & 0x00F000F0) | 0x54005400   = (  64 + q3,   64 + q7)
// and four dot2 against the f16 activation pairs (x0,x4), (x1,x5), (x2,x6),
// (x3,x7) accumulate sum_j (off_j + q_j) x_j in fp32 (each product is exact).
// The offset part sum_j off_j x_j depends on x only, so it is computed once
// (dot8_q4_off with w = 0) and subtracted per row: 9 instructions per 8
// nibbles instead of a convert and an fma per nibble.
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f16x2_t as_f16x2(uint32_t v) { return __builtin_bit_cast(f16x2_t, v); }

__device__ __forceinline__ f16x2_t f16x2_of(float a, float b) {  // round to nearest even
  f16x2_t r;
  r.x = static_cast<_Float16>(a);
  r.y = static_cast<_Float16>(b);
  return r;
}

// A constant the compiler must keep in a VGPR (an empty asm it cannot see
// through; identical ones are merged, so each constant is materialized once).
__device__ __forceinline__ uint32_t vgpr_const(uint32_t c) {
  asm("" : "+v"(c));
  return c;
}

// (w & mask) | magic in one v_and_or_b32. VOP3 here takes no literal, so with
// both constants as literals the compiler splits it into an AND and an OR; with
// the mask in a VGPR and the magic in an SGPR (one constant-bus read) it emits
// the single instruction. (An inline-asm v_and_or_b32 did too, but the
// compiler then assumes the worst of it: a wait state before every dot product
// that reads its result, and no reordering around it.)
__device__ __forceinline__ uint32_t and_or(uint32_t w, uint32_t mask, uint32_t magic) {
  return (w & vgpr_const(mask)) | magic;
}

// xp[0..3] = (x0,x4), (x1,x5), (x2,x6), (x3,x7) of the word's eight columns
__device__ __forceinline__ float dot8_q4_off(uint32_t w, const f16x2_t* xp, float acc) {
  const uint32_t w8 = w >> 8;
  acc = __builtin_amdgcn_fdot2(as_f16x2(and_or(w, 0x000F000Fu, 0x64006400u)), xp[0], acc, false);
  acc = __builtin_amdgcn_fdot2(as_f16x2(and_or(w, 0x00F000F0u, 0x54005400u)), xp[1], acc, false);
  acc = __builtin_amdgcn_fdot2(as_f16x2(and_or(w8, 0x000F000Fu, 0x64006400u)), xp[2], acc, false);
  acc = __builtin_amdgcn_fdot2(as_f16x2(and_or(w8, 0x00F000F0u, 0x54005400u)), xp[3], acc, false);
  return acc;
}

// The offset part sum_j off_j x_j of dot8_q4_off (its value for w = 0).
__device__ __forceinline__ float dot8_off_only(const f16x2_t* xp, float acc) {
  acc = __builtin_amdgcn_fdot2(as_f16x2(0x64006400u), xp[0], acc, false);
  acc = __builtin_amdgcn_fdot2(as_f16x2(0x54005400u), xp[1], acc, false);
  acc = __builtin_amdgcn_fdot2(as_f16x2(0x64006400u), xp[2], acc, false);
  acc = __builtin_amdgcn_fdot2(as_f16x2(0x54005400u), xp[3], acc, false);
  return acc;
}

// ---- The range of the f16 operands ----------------------------------------
// dot8_q4_off takes its activations as f16, which holds magnitudes up to
// 65504. A block of values whose largest magnitude amax is 2^15 or more is
// scaled by 2^-k before the conversion, exactly (a power of two; values
// 2^25 below amax may lose bits as f16 subnormals), with k the smallest that
// brings amax below 2^15; the block's fp32 dot products are multiplied by 2^k
// afterwards, also exactly. For amax below 2^15 (and for a non-finite amax,
// whose inf or NaN propagates anyway) k = 0 and both factors are 1.0, so the
// results there are the unscaled ones bit for bit.
struct F16Range {
  float up;    // 2^k: multiplies the block's dot products
  float down;  // 2^-k: multiplies the block's values before the f16 conversion
};
__device__ __forceinline__ F16Range f16_range(float amax) {
  const uint32_t e = (__float_as_uint(amax) >> 23) & 0xffu;   // biased exponent: amax < 2^(e - 126)
  const uint32_t k = (e >= 142u && e < 255u) ? e - 141u : 0u;  // amax * 2^-k < 2^15
  return F16Range{__uint_as_float((127u + k) << 23), __uint_as_float((127u - k) << 23)};
}
// Largest magnitude over each aligned group of 32 lanes (every lane gets it).
__device__ __forceinline__ float half_wave_absmax(float v) {
  v = __builtin_fabsf(v);
  v = __builtin_fmaxf(v, dpp_f32<DPP_XOR1>(v));
  v = __builtin_fmaxf(v, dpp_f32<DPP_XOR2>(v));
  v = __builtin_fmaxf(v, dpp_f32<DPP_HALF_MIRROR>(v));  // quad-uniform data: pairs quads 0-1, 2-3
  v = __builtin_fmaxf(v, dpp_f32<DPP_MIRROR>(v));       // 8-uniform data: pairs the half-rows
  return __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F)));  // lanes i, i ^ 16
}
// Largest magnitude of n values held by one lane.
template <int N>
__device__ __forceinline__ float lane_absmax(const float* v) {
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < N; ++i) m = __builtin_fmaxf(m, __builtin_fabsf(v[i]));
  return m;
}

// f16 pairs of eight consecutive fp32 values in the order dot8_q4_off expects
__device__ __forceinline__ void f16_pairs8(const float* x, f16x2_t* xp) {
  xp[0] = f16x2_of(x[0], x[4]);
  xp[1] = f16x2_of(x[1], x[5]);
  xp[2] = f16x2_of(x[2], x[6]);
  xp[3] = f16x2_of(x[3], x[7]);
}

// Maximum over the 64 lanes, returned uniform: the row maxima meet in lane 63
// through the row broadcasts (one lane read instead of four).
constexpr int DPP_ROW_BCAST15 = 0x142;  // lane 15 of each row -> the next row (rows 1 and 3 enabled)
constexpr int DPP_ROW_BCAST31 = 0x143;  // lane 31 -> rows 2 and 3
__device__ __forceinline__ int wave_max_i32(int v) {
  v = max(v, dpp_i32<DPP_XOR1>(v));
  v = max(v, dpp_i32<DPP_XOR2>(v));
  v = max(v, dpp_i32<DPP_HALF_MIRROR>(v));
  v = max(v, dpp_i32<DPP_MIRROR>(v));
  v = max(v, __builtin_amdgcn_update_dpp(v, v, DPP_ROW_BCAST15, 0xA, 0xF, false));
  v = max(v, __builtin_amdgcn_update_dpp(v, v, DPP_ROW_BCAST31, 0xC, 0xF, false));
  return __builtin_amdgcn_readlane(v, 63);
}

// Order-preserving int image of a float (larger float <-> larger int; NaN
// maps above +inf).
__device__ __forceinline__ int f32_order(float f) {
  const int b = __float_as_int(f);
  return b >= 0 ? b : b ^ 0x7fffffff;
}
__device__ __forceinline__ float f32_unorder(int k) { return __int_as_float(k >= 0 ? k : k ^ 0x7fffffff); }


// Softmax + top-k of one token on one wave (moe_routing_topk.metal:24-56).
// lane l holds the logits of experts l, l+64, l+128, l+192 (absent ones are
// ignored). Under the reference rule (rule == OBS_ROUTE_REF) each logit is
// first rounded to f16, the type dequant_matvec_8bit.metal:30 stores it in.
// m = max logit; e = exp_det(l - m); S = sum of e in the wave order
// (lane-serial over its experts from 0, then wave_sum_asc); p = e / S; k rounds
// select the largest p (lowest expert id on ties); wsum is the serial sum of
// the selected p; weights are p / wsum when norm_topk and wsum > 0. Under the
// reference rule the weights are stored as f16 values: f16(p), renormalised as
// f16(f16(p) / wsum) (moe_routing_topk.metal:47, :55).
// Lane kk < k receives slot kk (id -1, weight 0 if nothing is selectable).
// Must be called with all 64 lanes active. NQ = logit slots per lane
// (ceil(n_exp / 64), at most 4); selection is branch-free per round.
// Softmax of one token's logits (expert 64j + lane in lg[j]) as selection keys:
// key = bit pattern of p = e / S (non-negative, so integer order = p order),
// -1 for an absent expert, -2 for NaN.
template <int NQ>
__device__ __forceinline__ void route_keys(const float (&lg_in)[NQ], uint32_t n_exp, uint32_t lane, int rule,
                                           int (&key)[NQ]) {
  bool present[NQ];
  float lg[NQ];
  int mk = f32_order(-__builtin_huge_valf());
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    present[j] = lane + 64u * j < n_exp;
    lg[j] = rule == OBS_ROUTE_REF ? round_f16(lg_in[j]) : lg_in[j];
    mk = present[j] ? max(mk, f32_order(lg[j])) : mk;
  }
  // The maximum through the order-preserving int image. A NaN logit becomes
  // the maximum here where fmaxf would skip it; either way every l - m, e and
  // S then holds a NaN (a NaN logit's own e is NaN), so no expert is selectable.
  const float m = f32_unorder(wave_max_i32(mk));
  float e[NQ];
  float a = 0.0f;
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    e[j] = exp_det(present[j] ? lg[j] - m : -1000.0f);  // absent -> 0, not added below
    a = present[j] ? a + e[j] : a;
  }
  const float S = wave_sum_asc(a);
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    const float p = e[j] / S;
    key[j] = present[j] ? ((p != p) ? -2 : __float_as_int(p)) : -1;
  }
}

// Weight of a selected expert from its p and the sum of the selected p.
__device__ __forceinline__ float route_weight(float p, float wsum, int norm_topk, int rule) {
  if (rule == OBS_ROUTE_REF) {
    const float w = round_f16(p);
    return (norm_topk && wsum > 0.0f) ? round_f16(w / wsum) : w;
  }
  return (norm_topk && wsum > 0.0f) ? p / wsum : p;
}

template <int NQ>
__device__ __forceinline__ void route_wave(const float (&lg)[NQ], uint32_t n_exp, uint32_t k, int norm_topk,
                                           int rule, uint32_t lane, int32_t* my_id, float* my_w) {
  int key[NQ];
  route_keys<NQ>(lg, n_exp, lane, rule, key);
  float wsum = 0.0f;
  int32_t sel_id = -1;
  float sel_p = 0.0f;
  for (uint32_t kk = 0; kk < k; ++kk) {
    int lm = key[0];
#pragma unroll
    for (int j = 1; j < NQ; ++j) lm = max(lm, key[j]);
    const int bk = wave_max_i32(lm);
    // Branch-free: once nothing is selectable (bk < 0; keys only decrease) no
    // key equals bk, so no id is taken and the later slots keep id -1.
    // lowest expert id holding bk: slot-major (ids 64j + lane), lowest lane first
    uint32_t bidx = 0xffffffffu;
#pragma unroll
    for (int j = NQ - 1; j >= 0; --j) {
      const unsigned long long mj = __ballot(key[j] == bk && bk >= 0);
      bidx = mj ? 64u * j + static_cast<uint32_t>(__builtin_ctzll(mj)) : bidx;
    }
    const float p = __int_as_float(bk);
    const bool take = bk >= 0;
    sel_id = (lane == kk && take) ? static_cast<int32_t>(bidx) : sel_id;
    sel_p = (lane == kk && take) ? p : sel_p;
    wsum = take ? wsum + p : wsum;
#pragma unroll
    for (int j = 0; j < NQ; ++j) key[j] = (64u * j + lane == bidx) ? -1 : key[j];
  }
  *my_id = sel_id;
  *my_w = sel_id >= 0 ? route_weight(sel_p, wsum, norm_topk, rule) : 0.0f;
}

// Same contract and bit-identical result as route_wave for k = 8, without
// eight dependent argmax rounds: (1) a binary search over the 31-bit keys
// (ballot population counts) finds T, the 8th largest key; (2) the selected set
// is every key > T plus the lowest-id keys == T up to 8; (3) the (key, id)
// pairs are gathered into scalar registers in id order and sorted by
// (key desc, id asc) with a 19-comparator network; lane s takes slot s.
// Because (key desc, id asc) is a strict total order, this equals k rounds of
// "largest p, lowest id on ties".
template <int NQ>
__device__ __forceinline__ void route_wave_top8(const float (&lg)[NQ], uint32_t n_exp, int norm_topk, int rule,
                                                uint32_t lane, int32_t* my_id, float* my_w) {
  constexpr int K = 8;
  int key[NQ];
  route_keys<NQ>(lg, n_exp, lane, rule, key);
  // (1) T = largest value with count(key >= T) >= K (0 if fewer than K selectable)
  int T = 0;
#pragma unroll
  for (int bit = 30; bit >= 0; --bit) {
    const int cand = T | (1 << bit);
    uint32_t c = 0;
#pragma unroll
    for (int j = 0; j < NQ; ++j) c += static_cast<uint32_t>(__popcll(__ballot(key[j] >= cand)));
    T = (c >= static_cast<uint32_t>(K)) ? cand : T;
  }
  // (2) membership
  uint32_t n_gt = 0;
#pragma unroll
  for (int j = 0; j < NQ; ++j) n_gt += static_cast<uint32_t>(__popcll(__ballot(key[j] > T)));
  const unsigned long long lt_mask = (1ull << lane) - 1ull;
  uint32_t eq_before = 0;
  unsigned long long msel[NQ];
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    const unsigned long long meq = __ballot(key[j] == T);
    const uint32_t r = eq_before + static_cast<uint32_t>(__popcll(meq & lt_mask));
    msel[j] = __ballot(key[j] > T || (key[j] == T && n_gt + r < static_cast<uint32_t>(K)));
    eq_before += static_cast<uint32_t>(__popcll(meq));
  }
  // (3) gather in ascending id order (uniform values)
  int sk[K], si[K];
#pragma unroll
  for (int s = 0; s < K; ++s) {
    sk[s] = -1;
    si[s] = -1;
    bool found = false;
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      if (!found && msel[j] != 0ull) {
        const int l = __builtin_ctzll(msel[j]);
        msel[j] &= msel[j] - 1ull;
        sk[s] = __builtin_amdgcn_readlane(key[j], l);
        si[s] = 64 * j + l;
        found = true;
      }
    }
  }
  // (4) sort: element a precedes b iff key_a > key_b or (key_a == key_b and id_a < id_b);
  // empty entries (key -1) sort last
#define OBS_CSWAP(A, B)                                                                  \
  do {                                                                                   \
    const bool sw = (sk[B] > sk[A]) || (sk[B] == sk[A] && si[B] < si[A]);                \
    const int tk = sw ? sk[B] : sk[A], ti = sw ? si[B] : si[A];                          \
    sk[B] = sw ? sk[A] : sk[B];                                                          \
    si[B] = sw ? si[A] : si[B];                                                          \
    sk[A] = tk;                                                                          \
    si[A] = ti;                                                                          \
  } while (0)
  OBS_CSWAP(0, 2); OBS_CSWAP(1, 3); OBS_CSWAP(4, 6); OBS_CSWAP(5, 7);
  OBS_CSWAP(0, 4); OBS_CSWAP(1, 5); OBS_CSWAP(2, 6); OBS_CSWAP(3, 7);
  OBS_CSWAP(0, 1); OBS_CSWAP(2, 3); OBS_CSWAP(4, 5); OBS_CSWAP(6, 7);
  OBS_CSWAP(2, 4); OBS_CSWAP(3, 5);
  OBS_CSWAP(1, 4); OBS_CSWAP(3, 6);
  OBS_CSWAP(1, 2); OBS_CSWAP(3, 4); OBS_CSWAP(5, 6);
#undef OBS_CSWAP
  // (5) weights: wsum is the serial sum of the selected p in rank order
  float wsum = 0.0f;
  int32_t sel_id = -1;
  float sel_p = 0.0f;
#pragma unroll
  for (int s = 0; s < K; ++s) {
    const float ps = __int_as_float(sk[s]);
    wsum = si[s] >= 0 ? wsum + ps : wsum;
    sel_id = (lane == static_cast<uint32_t>(s)) ? si[s] : sel_id;
    sel_p = (lane == static_cast<uint32_t>(s)) ? ps : sel_p;
  }
  *my_id = sel_id;
  *my_w = sel_id >= 0 ? route_weight(sel_p, wsum, norm_topk, rule) : 0.0f;
}

}  // namespace obsd
