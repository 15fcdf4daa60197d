// obs_prefill.hip — grouped prefill MoE (src/forward.rs:164-247) and the
// per-expert batched dequant matmul (Model::matmul_raw, forward.rs:313-321).
//
// Pipeline for T tokens (all on the GPU, no host round trip):
//   1. routing: computed (gate logits + top-k kernels) or injected;
//   2. grouping: rows of expert e are the tokens routed to e in ascending
//      token order (forward.rs:203-204); one wave per 64-token chunk counts,
//      one workgroup scans the counts into row bases and emits the tile list
//      (expert, first row, rows <= 128), then one wave per chunk ranks its
//      tokens with LDS lane bitmasks and scatters the row maps;
//   3. gate/up grouped GEMM with a SwiGLU epilogue -> H [T*k, I] bf16;
//   4. down grouped GEMM -> Yp, written at the token-major slot t*k + r;
//   5. combine: y[t] = residual[t] + sum_r w[t,r] * Yp[t*k+r], fp32, rank order
//      (forward.rs:225-232), rounded once to bf16.
//
// The GEMM. A workgroup (4 waves) owns a tile of up to 128 permuted rows x 128
// output columns; wave w owns columns [32w, 32w+32) (and the same columns of
// the up matrix for gate/up). Per 64-column quantization group:
//   - A (activations, gathered by row through a_rows) is staged in LDS,
//     double-buffered, row stride padded to 72 bf16;
//   - B is read straight from HBM into registers: lane l takes 16 bytes
//     (32 nibbles) of weight row n = n0 + 32w + l%32, columns
//     [k0 + 32(l/32), +32), and dequantizes them to bf16 = RNE(q*s + b) with
//     the tile's scales and biases, staged once per tile in LDS;
//   - v_mfma_f32_32x32x16_bf16 accumulates in fp32. The MFMA's 16 k-slots of
//     K-step s map to columns k0 + 32h + 8s + j (h = lane half, j = 0..7), for
//     A and B alike, so each lane's 16-byte load feeds all four K-steps.
#include "obs_internal.hpp"

namespace obs {
int check_moe_config(obs_ctx* ctx, const char* who, const obs_moe_config* cfg);
int check_moe_layer(obs_ctx* ctx, const char* who, const obs_moe_layer* L);
int launch_gate_logits(obs_ctx* ctx, const uint32_t* w8, const uint16_t* s, const uint16_t* b,
                       const uint16_t* x, float* logits, uint32_t T, uint32_t in, uint32_t n_exp, uint32_t group);
int launch_route_topk(obs_ctx* ctx, const float* logits, int32_t* ids, float* w, uint32_t T,
                      uint32_t n_exp, uint32_t k, int norm_topk);
}  // namespace obs

namespace {

using namespace obsd;

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));  // register-friendly 16-byte word

constexpr uint32_t TM = 128;          // tile rows
constexpr uint32_t TN = 128;          // tile output columns (4 waves x 32)
constexpr uint32_t GK = 64;           // quantization group = K step of the main loop
constexpr uint32_t LDS_STRIDE = 72;   // bf16 per staged A row (64 + 8 padding)
constexpr uint32_t GROUP_TOKENS = 64; // tokens per grouping chunk (one wave)
constexpr uint32_t SB_STRIDE = TN + 1;  // words per (matrix, group) row of staged scale|bias
constexpr uint32_t SB_LDS_MAX = 96u * 1024u;  // bytes of staged scale|bias per workgroup

struct GemmArgs {
  const uint16_t* A;        // bf16 [a_rows_total, K]
  const int32_t* a_rows;    // permuted row -> A row (nullptr: identity)
  uint32_t a_rows_total;    // bound for a_rows values
  const uint32_t* w0; const uint16_t* s0; const uint16_t* b0;  // [E, N, K/8], [E, N, K/64]
  const uint32_t* w1; const uint16_t* s1; const uint16_t* b1;  // up matrix (SwiGLU only)
  uint16_t* out;            // bf16 rows of N
  const int32_t* out_rows;  // permuted row -> output row (nullptr: identity)
  const int4* tiles;        // {expert, row0, rows, 0}; nullptr: dense rows of expert 0
  const int32_t* n_tiles;   // device tile count (grouped mode)
  uint32_t dense_rows;      // row count in dense mode
  uint32_t K, N;
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two fp32 values -> one packed bf16 pair (RNE, v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16_rne(float lo, float hi) {
  const f32x2_t f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}

// fp32 fma(h, s, b) where h is the low (HI = 0) or high (HI = 1) f16 half of v
// (v_fma_mix_f32: the f16 operand converts exactly to fp32 inside the fma).
template <int HI>
__device__ __forceinline__ float fma_mix_f16(uint32_t v, float s, float b) {
  float r;
  if (HI)
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(v), "v"(s), "v"(b));
  else
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(v), "v"(s), "v"(b));
  return r;
}

// Scale operands of dequant_word_mix for one (row, group): s * 2^24, s * 2^20.
struct MixScale {
  float s24, s20, b;
};
__device__ __forceinline__ MixScale mix_scale(uint32_t packed_sb) {
  const float s = bf16lo(packed_sb);
  return MixScale{s * 0x1p24f, s * 0x1p20f, bf16hi(packed_sb)};
}

// One 32-bit word = 8 nibbles of a weight row -> one bf16x8 MFMA fragment,
// bf16 = RNE(fp32(q*s + b)), with 17 VALU instructions. A nibble masked in
// place at bits 3:0 (or 7:4) of a 16-bit half is the f16 subnormal q * 2^-24
// (or q * 2^-20), exactly; fma_mix multiplies it by s * 2^24 (or s * 2^20),
// which is exact (a power-of-two scaling of the bf16 s, then a 4 x 8-bit
// significand product), and adds b with the single fp32 rounding of
// fmaf(q, s, b). Valid for |s| <= 2^100 (so s * 2^24 cannot overflow); tiles
// holding larger scales use dequant_word. Checked bit for bit against
// fmaf(q, s, b) for every finite bf16 s in that range, on the target GPU.
__device__ __forceinline__ bf16x8_t dequant_word_mix(uint32_t w, const MixScale& m) {
  const uint32_t w8 = w >> 8;
  const uint32_t p04 = w & 0x000F000Fu;   // (q0, q4) * 2^-24
  const uint32_t p15 = w & 0x00F000F0u;   // (q1, q5) * 2^-20
  const uint32_t p26 = w8 & 0x000F000Fu;  // (q2, q6) * 2^-24
  const uint32_t p37 = w8 & 0x00F000F0u;  // (q3, q7) * 2^-20
  u32x4_t r;
  r.x = pack_bf16_rne(fma_mix_f16<0>(p04, m.s24, m.b), fma_mix_f16<0>(p15, m.s20, m.b));
  r.y = pack_bf16_rne(fma_mix_f16<0>(p26, m.s24, m.b), fma_mix_f16<0>(p37, m.s20, m.b));
  r.z = pack_bf16_rne(fma_mix_f16<1>(p04, m.s24, m.b), fma_mix_f16<1>(p15, m.s20, m.b));
  r.w = pack_bf16_rne(fma_mix_f16<1>(p26, m.s24, m.b), fma_mix_f16<1>(p37, m.s20, m.b));
  return __builtin_bit_cast(bf16x8_t, r);
}

// silu(g) * u for the GEMM epilogue with the hardware exp2 and reciprocal
// (about 2 ulp in fp32; the result is rounded to bf16 right after).
__device__ __forceinline__ float silu_mul_fast(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(-g * 1.44269504088896341f);
  return (g * __builtin_amdgcn_rcpf(1.0f + e)) * u;
}

// A staged scale|bias word whose scale is beyond dequant_word_mix's range
// (|s| > 2^100, inf, NaN): bf16 exponent field above 127 + 100.
__device__ __forceinline__ bool scale_out_of_mix_range(uint32_t packed_sb) {
  return (packed_sb & 0x7f80u) > (227u << 7);
}

// Reference-form dequant of one word (convert, fma, round), for any scale.
__device__ __forceinline__ bf16x8_t dequant_word(uint32_t w, float s, float b) {
  uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
  // opaque to the optimizer, so each byte converts with one v_cvt_f32_ubyteN
  // instead of being re-derived from w with a shift and a mask
  asm("" : "+v"(lo), "+v"(hi));
  float v[8];
  v[0] = __builtin_fmaf(static_cast<float>(lo & 0xffu), s, b);
  v[1] = __builtin_fmaf(static_cast<float>(hi & 0xffu), s, b);
  v[2] = __builtin_fmaf(static_cast<float>((lo >> 8) & 0xffu), s, b);
  v[3] = __builtin_fmaf(static_cast<float>((hi >> 8) & 0xffu), s, b);
  v[4] = __builtin_fmaf(static_cast<float>((lo >> 16) & 0xffu), s, b);
  v[5] = __builtin_fmaf(static_cast<float>((hi >> 16) & 0xffu), s, b);
  v[6] = __builtin_fmaf(static_cast<float>(lo >> 24), s, b);
  v[7] = __builtin_fmaf(static_cast<float>(hi >> 24), s, b);
  u32x4_t r;
  r.x = pack_bf16_rne(v[0], v[1]);
  r.y = pack_bf16_rne(v[2], v[3]);
  r.z = pack_bf16_rne(v[4], v[5]);
  r.w = pack_bf16_rne(v[6], v[7]);
  return __builtin_bit_cast(bf16x8_t, r);
}

// One tile's main loop and epilogue, NB = active 32-row blocks (1..4), so the
// MFMA sequence is straight-line code. MIX: every staged scale is within
// dequant_word_mix's range (decided per tile).
template <bool SWIGLU, uint32_t NB, bool MIX>
__device__ __forceinline__ void gemm_tile(const GemmArgs& a, uint16_t (&sA)[2][TM * LDS_STRIDE],
                                          const int32_t* s_arow, const int32_t* s_orow, const uint32_t* s_sb,
                                          uint32_t e, uint32_t row0,
                                          uint32_t nrows, uint32_t n0) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t nl = 32u * wave + (lane & 31u);                   // this lane's column in the tile
  const uint32_t n = n0 + nl;                                      // this lane's weight row
  const uint32_t h = lane >> 5;                                    // k half within a group
  const uint32_t K = a.K, groups = K / GK;

  // A staging: thread t -> 16 bytes (8 bf16, chunk t % 8 of the group) of tile
  // rows t/8 + 32i, i = 0..3, so each wave instruction reads 8 whole 128-byte
  // row segments. Rows of blocks >= NB are never read by the MFMAs and are not
  // staged (i is unrolled, so this costs no branch).
  const uint32_t ac = 8u * (tid & 7u);
  const uint16_t* aptr[4];
#pragma unroll
  for (uint32_t i = 0; i < 4; ++i) {
    const int32_t arow = s_arow[tid / 8u + 32u * i];
    // Padding rows (no A row) stage row 0: row i of an MFMA product depends on
    // row i of A only, and the epilogue discards padding rows.
    aptr[i] = a.A + static_cast<size_t>(arow >= 0 ? arow : 0) * K + ac;
  }
  auto load_a = [&](uint32_t g, u32x4_t (&r)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (uint32_t i = 0; i < NB; ++i) r[i] = *reinterpret_cast<const u32x4_t*>(aptr[i] + g * GK);
  };
  auto store_a = [&](uint32_t buf, const u32x4_t (&r)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (uint32_t i = 0; i < NB; ++i)
      *reinterpret_cast<u32x4_t*>(&sA[buf][(tid / 8u + 32u * i) * LDS_STRIDE + ac]) = r[i];
  };

  // B pointers of this lane's weight row(s)
  const size_t wrow = static_cast<size_t>(e) * a.N + n;
  const u32x4_t* w0p = reinterpret_cast<const u32x4_t*>(a.w0 + wrow * (K / 8)) + h;  // + 2*g per group
  const u32x4_t* w1p = SWIGLU ? reinterpret_cast<const u32x4_t*>(a.w1 + wrow * (K / 8)) + h : nullptr;
  // staged scale|bias of this lane's column: [matrix][group] at stride SB_STRIDE words
  const uint32_t* sb0 = s_sb + nl;
  const uint32_t* sb1 = s_sb + static_cast<size_t>(groups) * SB_STRIDE + nl;

  struct BRaw {
    u32x4_t q0, q1;
  };
  auto load_b = [&](uint32_t g) __attribute__((always_inline)) {
    BRaw r;
    const uint32_t gg = g < groups ? g : groups - 1u;  // clamped: the tail loads are never used
    r.q0 = w0p[2u * gg];
    if (SWIGLU) r.q1 = w1p[2u * gg];
    return r;
  };

  f32x16_t acc0[NB], acc1[NB];
#pragma unroll
  for (int mb = 0; mb < NB; ++mb) {
#pragma unroll
    for (int v = 0; v < 16; ++v) { acc0[mb][v] = 0.0f; acc1[mb][v] = 0.0f; }
  }

  // Pipeline, sized for two resident waves per SIMD: B two groups ahead (two
  // register slots), A one group ahead (registers, then the other LDS buffer).
  // Per K-step the A fragments are read and the B fragment dequantized just
  // before its MFMAs, so few values are live; the co-resident workgroup hides
  // the LDS and memory latencies. Unrolled by two so each slot is a fixed set
  // of registers.
  BRaw bs0 = load_b(0), bs1 = load_b(1);
  u32x4_t ras[4];
  load_a(0, ras);
  store_a(0, ras);

  auto step = [&](uint32_t g, BRaw& bcur) __attribute__((always_inline)) {
    const uint32_t buf = g & 1u;
    __syncthreads();  // A of group g visible in sA[buf]; sA[buf^1] no longer read
    load_a(g + 1 < groups ? g + 1 : g, ras);  // the tail reload is stored but never read
    // keep the A loads here, a whole group ahead of their LDS store: left to
    // itself the scheduler sinks them next to the store and exposes their latency
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t sv0 = sb0[g * SB_STRIDE];
    const uint32_t sv1 = SWIGLU ? sb1[g * SB_STRIDE] : 0u;
    const uint32_t q0w[4] = {bcur.q0.x, bcur.q0.y, bcur.q0.z, bcur.q0.w};
    const uint32_t q1w[4] = {bcur.q1.x, bcur.q1.y, bcur.q1.z, bcur.q1.w};
    const MixScale m0 = mix_scale(sv0), m1 = mix_scale(sv1);
#pragma unroll
    for (uint32_t st = 0; st < 4; ++st) {
      bf16x8_t af[NB];
#pragma unroll
      for (uint32_t mb = 0; mb < NB; ++mb)
        af[mb] = *reinterpret_cast<const bf16x8_t*>(
            &sA[buf][(32u * mb + (lane & 31u)) * LDS_STRIDE + 32u * h + 8u * st]);
      const bf16x8_t f0 = MIX ? dequant_word_mix(q0w[st], m0) : dequant_word(q0w[st], bf16lo(sv0), bf16hi(sv0));
      bf16x8_t f1;
      if (SWIGLU) f1 = MIX ? dequant_word_mix(q1w[st], m1) : dequant_word(q1w[st], bf16lo(sv1), bf16hi(sv1));
#pragma unroll
      for (uint32_t mb = 0; mb < NB; ++mb) {
        acc0[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mb], f0, acc0[mb], 0, 0, 0);
        if (SWIGLU) acc1[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mb], f1, acc1[mb], 0, 0, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // the A store waits for its loads: keep it last
    bcur = load_b(g + 2);    // clamped past the end; never used there
    store_a(buf ^ 1u, ras);  // read after the next barrier
  };
  for (uint32_t g = 0; g < groups; g += 2) {  // groups % 4 == 0 (K % 256 == 0, checked by the host)
    step(g, bs0);
    step(g + 1, bs1);
  }

  // Epilogue: lane holds C[i][nl] for i = 32mb + 8(v/4) + 4h + v%4. The tile
  // goes through LDS (the A buffers are free now) so each output row leaves as
  // sixteen coalesced 16-byte stores instead of 128 scattered 2-byte ones.
  // Lanes nl and nl^1 (columns c, c+1) swap halves of their packed row pairs,
  // so each LDS write is a 4-byte (row, c..c+1) pair: the even lane writes rows
  // i0 and i0+2, the odd lane rows i0+1 and i0+3.
  constexpr uint32_t C_STRIDE = TN + 8;  // bf16 per staged row (bank spread)
  static_assert(TM * C_STRIDE <= 2 * TM * LDS_STRIDE, "C tile must fit the A buffers");
  uint16_t* sC = reinterpret_cast<uint16_t*>(sA);
  const uint32_t odd = nl & 1u, c_even = nl & ~1u;
  const uint32_t sel = odd ? 0x03020706u : 0x05040100u;  // v_perm: (partner.hi, own.hi) : (own.lo, partner.lo)
  __syncthreads();  // every wave is done reading sA
#pragma unroll
  for (uint32_t mb = 0; mb < NB; ++mb) {
#pragma unroll
    for (uint32_t qd = 0; qd < 4; ++qd) {
      float v[4];
#pragma unroll
      for (uint32_t j = 0; j < 4; ++j)
        v[j] = SWIGLU ? silu_mul_fast(acc0[mb][4 * qd + j], acc1[mb][4 * qd + j]) : acc0[mb][4 * qd + j];
      const uint32_t p01 = pack_bf16_rne(v[0], v[1]), p23 = pack_bf16_rne(v[2], v[3]);
      const uint32_t s01 = static_cast<uint32_t>(dpp_i32<DPP_XOR1>(static_cast<int>(p01)));
      const uint32_t s23 = static_cast<uint32_t>(dpp_i32<DPP_XOR1>(static_cast<int>(p23)));
      const uint32_t i0 = 32u * mb + 8u * qd + 4u * h + odd;
      *reinterpret_cast<uint32_t*>(&sC[i0 * C_STRIDE + c_even]) = __builtin_amdgcn_perm(s01, p01, sel);
      *reinterpret_cast<uint32_t*>(&sC[(i0 + 2u) * C_STRIDE + c_even]) = __builtin_amdgcn_perm(s23, p23, sel);
    }
  }
  __syncthreads();
#pragma unroll
  for (uint32_t q = 0; q < TM * TN / 8u / 256u; ++q) {
    const uint32_t chunk = tid + 256u * q, i = chunk / (TN / 8u), c8 = 8u * (chunk % (TN / 8u));
    if (i < nrows) {
      const uint4 v = *reinterpret_cast<const uint4*>(&sC[i * C_STRIDE + c8]);
      *reinterpret_cast<uint4*>(a.out + static_cast<size_t>(s_orow[i]) * a.N + n0 + c8) = v;
    }
  }
}

// Work items are (tile, 128-column block) pairs in tile order, and tiles are in
// expert order. The dispatcher deals consecutive workgroups round-robin over
// the 8 XCDs, so workgroup l takes item (l % 8) * chunk + l / 8: each XCD runs
// a contiguous run of items, and the tiles of one expert share its weights (and
// the column blocks of one tile share its activation rows) in that XCD's L2.
// Two workgroups per CU (at most 256 registers per lane): the co-resident
// workgroup hides each one's load, LDS and barrier latency.
template <bool SWIGLU>
__global__ void __launch_bounds__(256, 2) grouped_gemm_kernel(GemmArgs a) {
  __shared__ uint16_t sA[2][TM * LDS_STRIDE];
  __shared__ int32_t s_arow[TM], s_orow[TM];
  extern __shared__ uint32_t s_sb[];  // [matrix][group][SB_STRIDE]: scale | bias << 16
  const uint32_t ncb = a.N / TN;
  const uint32_t n_tiles = a.tiles ? static_cast<uint32_t>(*a.n_tiles) : (a.dense_rows + TM - 1) / TM;
  const uint32_t n_items = n_tiles * ncb, chunk = (n_items + 7u) / 8u;
  const uint32_t item = (blockIdx.x % 8u) * chunk + blockIdx.x / 8u;
  if (blockIdx.x / 8u >= chunk || item >= n_items) return;  // uniform per workgroup
  const uint32_t t_idx = item / ncb, n0 = (item % ncb) * TN;
  int4 tile;
  if (a.tiles) {
    tile = a.tiles[t_idx];
  } else {
    const uint32_t r0 = t_idx * TM;
    tile = make_int4(0, static_cast<int32_t>(r0), static_cast<int32_t>(min(TM, a.dense_rows - r0)), 0);
  }
  const uint32_t e = static_cast<uint32_t>(tile.x), row0 = static_cast<uint32_t>(tile.y);
  const uint32_t nrows = static_cast<uint32_t>(tile.z);
  const uint32_t tid = threadIdx.x;
  if (tid < TM) {
    int32_t r = -1;
    if (tid < nrows) {
      const uint32_t p = row0 + tid;
      r = a.a_rows ? a.a_rows[p] : static_cast<int32_t>(p);
      if (r < 0 || static_cast<uint32_t>(r) >= a.a_rows_total) r = -1;
    }
    s_arow[tid] = r;
    if (tid < nrows) {
      const uint32_t p = row0 + tid;
      s_orow[tid] = a.out_rows ? a.out_rows[p] : static_cast<int32_t>(p);
    }
  }
  // Stage the scales and biases of the tile's 128 weight rows. Rows n0.. of
  // expert e are contiguous ([E, N, groups] bf16), so 8-byte chunks (4 groups
  // of one row; groups % 4 == 0) load coalesced; each becomes 4 packed words.
  // All of a batch's loads (up to 4 chunks per thread and matrix) are issued
  // before any is stored, so the staging pays one memory latency per batch
  // (one batch for K <= 2048) instead of one per chunk.
  bool wide_scale = false;  // some staged |s| is beyond dequant_word_mix's range
  {
    constexpr uint32_t NMAT = SWIGLU ? 2u : 1u, PER = 4u;
    const uint32_t groups = a.K / GK, cpr = groups / 4u, nchunk = TN * cpr;  // chunks per row, per matrix
    const size_t base = (static_cast<size_t>(e) * a.N + n0) * groups;
    for (uint32_t c0 = 0; c0 < nchunk; c0 += PER * 256u) {
      uint2 sv[NMAT][PER], bv[NMAT][PER];
#pragma unroll
      for (uint32_t mat = 0; mat < NMAT; ++mat) {
        const uint2* sp = reinterpret_cast<const uint2*>((mat ? a.s1 : a.s0) + base);
        const uint2* bp = reinterpret_cast<const uint2*>((mat ? a.b1 : a.b0) + base);
#pragma unroll
        for (uint32_t j = 0; j < PER; ++j) {
          const uint32_t c = c0 + tid + 256u * j;
          if (c < nchunk) {
            sv[mat][j] = sp[c];
            bv[mat][j] = bp[c];
          }
        }
      }
#pragma unroll
      for (uint32_t mat = 0; mat < NMAT; ++mat) {
#pragma unroll
        for (uint32_t j = 0; j < PER; ++j) {
          const uint32_t c = c0 + tid + 256u * j;
          if (c < nchunk) {
            const uint2 s2 = sv[mat][j], b2 = bv[mat][j];
            const uint32_t row = c / cpr, g0 = 4u * (c % cpr);
            uint32_t* d = s_sb + (static_cast<size_t>(mat) * groups + g0) * SB_STRIDE + row;
            d[0] = (s2.x & 0xffffu) | (b2.x << 16);
            d[SB_STRIDE] = (s2.x >> 16) | (b2.x & 0xffff0000u);
            d[2u * SB_STRIDE] = (s2.y & 0xffffu) | (b2.y << 16);
            d[3u * SB_STRIDE] = (s2.y >> 16) | (b2.y & 0xffff0000u);
            wide_scale = wide_scale || scale_out_of_mix_range(s2.x) || scale_out_of_mix_range(s2.x >> 16) ||
                         scale_out_of_mix_range(s2.y) || scale_out_of_mix_range(s2.y >> 16);
          }
        }
      }
    }
  }
  const bool mix = !__syncthreads_or(wide_scale);  // uniform per workgroup
  const uint32_t nb = (nrows + 31u) / 32u;
  if (mix) {
    switch (nb) {
      case 1: gemm_tile<SWIGLU, 1, true>(a, sA, s_arow, s_orow, s_sb, e, row0, nrows, n0); break;
      case 2: gemm_tile<SWIGLU, 2, true>(a, sA, s_arow, s_orow, s_sb, e, row0, nrows, n0); break;
      case 3: gemm_tile<SWIGLU, 3, true>(a, sA, s_arow, s_orow, s_sb, e, row0, nrows, n0); break;
      default: gemm_tile<SWIGLU, 4, true>(a, sA, s_arow, s_orow, s_sb, e, row0, nrows, n0); break;
    }
  } else {  // scales beyond 2^100 (never in real checkpoints): reference-form dequant
    gemm_tile<SWIGLU, 4, false>(a, sA, s_arow, s_orow, s_sb, e, row0, nrows, n0);
  }
}

// ---- grouping: rows of expert e are its routed (token, rank) pairs in
// ascending token order (forward.rs:203-204). Three launches: per 64-token
// chunk counts, one scan, per chunk ranks + scatter.

// A token's k (<= 8) ids in registers, -1 where invalid: out of range or a
// repeat of an earlier rank of the same token.
__device__ __forceinline__ void load_token_ids(const int32_t* __restrict__ ids, uint32_t t, uint32_t T, uint32_t k,
                                               uint32_t E, int32_t (&ev)[8]) {
#pragma unroll
  for (uint32_t r = 0; r < 8; ++r) ev[r] = (t < T && r < k) ? ids[static_cast<size_t>(t) * k + r] : -1;
#pragma unroll
  for (uint32_t r = 0; r < 8; ++r) {
    bool ok = ev[r] >= 0 && static_cast<uint32_t>(ev[r]) < E;
#pragma unroll
    for (uint32_t q = 0; q < r; ++q) ok = ok && ev[q] != ev[r];
    ev[r] = ok ? ev[r] : -1;
  }
}

// 1. one wave per chunk: chunk_cnt[c][e] = rows of expert e among the chunk's tokens
__global__ void __launch_bounds__(64) group_count_kernel(const int32_t* __restrict__ ids, uint32_t T, uint32_t k,
                                                         uint32_t E, int32_t* __restrict__ chunk_cnt) {
  __shared__ int32_t hist[256];
  const uint32_t lane = threadIdx.x, c = blockIdx.x;
  for (uint32_t e = lane; e < E; e += 64u) hist[e] = 0;
  __syncthreads();
  int32_t ev[8];
  load_token_ids(ids, c * GROUP_TOKENS + lane, T, k, E, ev);
#pragma unroll
  for (uint32_t r = 0; r < 8; ++r)
    if (ev[r] >= 0) atomicAdd(&hist[ev[r]], 1);
  __syncthreads();
  for (uint32_t e = lane; e < E; e += 64u) chunk_cnt[static_cast<size_t>(c) * E + e] = hist[e];
}

// Exclusive prefix sum over one workgroup of 256 threads (v per thread).
__device__ __forceinline__ int32_t block_exclusive_scan256(int32_t v, int32_t* s_wave, int32_t* total) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  int32_t x = v;
#pragma unroll
  for (uint32_t d = 1; d < 64; d <<= 1) {
    const int32_t y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63u) s_wave[wave] = x;
  __syncthreads();
  int32_t before = 0;
  for (uint32_t w = 0; w < wave; ++w) before += s_wave[w];
  *total = s_wave[0] + s_wave[1] + s_wave[2] + s_wave[3];
  __syncthreads();
  return before + x - v;
}

// 2. one workgroup (thread e = expert e, E <= 256): chunk counts -> absolute row
// bases per (chunk, expert), expert offsets and counts, the tile list.
__global__ void __launch_bounds__(256) group_scan_kernel(uint32_t nchunks, uint32_t E, int32_t* __restrict__ chunk_cnt,
                                                         int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                                                         int4* __restrict__ tiles, int32_t* __restrict__ n_tiles) {
  __shared__ int32_t s_wave[4];
  const uint32_t e = threadIdx.x;
  const bool have = e < E;
  int32_t tot = 0;
  if (have) {  // chunk-exclusive prefix per expert, in place
    for (uint32_t c0 = 0; c0 < nchunks; c0 += 16u) {
      int32_t v[16];
#pragma unroll
      for (uint32_t i = 0; i < 16; ++i) v[i] = c0 + i < nchunks ? chunk_cnt[static_cast<size_t>(c0 + i) * E + e] : 0;
#pragma unroll
      for (uint32_t i = 0; i < 16; ++i) {
        if (c0 + i < nchunks) chunk_cnt[static_cast<size_t>(c0 + i) * E + e] = tot;
        tot += v[i];
      }
    }
  }
  int32_t all_rows, all_tiles;
  const int32_t nt = (tot + static_cast<int32_t>(TM) - 1) / static_cast<int32_t>(TM);
  const int32_t off = block_exclusive_scan256(tot, s_wave, &all_rows);
  const int32_t toff = block_exclusive_scan256(nt, s_wave, &all_tiles);
  if (have) {
    counts[e] = tot;
    offsets[e] = off;
    for (int32_t q = 0; q < nt; ++q) {
      const int32_t r0 = q * static_cast<int32_t>(TM);
      tiles[toff + q] = make_int4(static_cast<int32_t>(e), off + r0, min(static_cast<int32_t>(TM), tot - r0), 0);
    }
    for (uint32_t c0 = 0; c0 < nchunks; c0 += 16u) {  // batched: all loads in flight together
      int32_t v[16];
#pragma unroll
      for (uint32_t i = 0; i < 16; ++i) v[i] = c0 + i < nchunks ? chunk_cnt[static_cast<size_t>(c0 + i) * E + e] : 0;
#pragma unroll
      for (uint32_t i = 0; i < 16; ++i)
        if (c0 + i < nchunks) chunk_cnt[static_cast<size_t>(c0 + i) * E + e] = v[i] + off;
    }
  }
  if (e == 0) {
    offsets[E] = all_rows;
    *n_tiles = all_tiles;
  }
}

// 3. one wave per chunk: a token's row in expert e = chunk base + the number of
// lower lanes (earlier tokens) of the chunk routed to e (LDS lane bitmasks).
__global__ void __launch_bounds__(64) group_rank_kernel(const int32_t* __restrict__ ids, uint32_t T, uint32_t k,
                                                        uint32_t E, const int32_t* __restrict__ chunk_base,
                                                        int32_t* __restrict__ row_token, int32_t* __restrict__ row_slot) {
  __shared__ unsigned long long wb[256];
  const uint32_t lane = threadIdx.x, c = blockIdx.x, t = c * GROUP_TOKENS + lane;
  for (uint32_t e = lane; e < E; e += 64u) wb[e] = 0ull;
  __syncthreads();
  int32_t ev[8];
  load_token_ids(ids, t, T, k, E, ev);
#pragma unroll
  for (uint32_t r = 0; r < 8; ++r)
    if (ev[r] >= 0) atomicOr(&wb[ev[r]], 1ull << lane);
  __syncthreads();
  const unsigned long long lt = (1ull << lane) - 1ull;
  const int32_t* base = chunk_base + static_cast<size_t>(c) * E;
#pragma unroll
  for (uint32_t r = 0; r < 8; ++r) {
    if (ev[r] < 0) continue;
    const uint32_t e = static_cast<uint32_t>(ev[r]);
    const int32_t row = base[e] + __popcll(wb[e] & lt);
    row_token[row] = static_cast<int32_t>(t);
    row_slot[row] = static_cast<int32_t>(t * k + r);
  }
}

// y[t, :] = residual + sum_r w[t, r] * Yp[t*k + r, :] (fp32, rank order). One
// workgroup per token (H / 8 threads, 8 columns each): the token's ids and
// weights are uniform, so they load once into scalar registers.
__global__ void __launch_bounds__(512) combine_kernel(const uint16_t* __restrict__ Yp, const int32_t* __restrict__ ids,
                                                      const float* __restrict__ w, const uint16_t* __restrict__ residual,
                                                      uint16_t* __restrict__ y, uint32_t k, uint32_t H, uint32_t E) {
  const uint32_t t = blockIdx.x, c = 8u * threadIdx.x;
  float acc[8];
  if (residual) {
    const uint4 rv = *reinterpret_cast<const uint4*>(residual + static_cast<size_t>(t) * H + c);
    acc[0] = bf16lo(rv.x); acc[1] = bf16hi(rv.x); acc[2] = bf16lo(rv.y); acc[3] = bf16hi(rv.y);
    acc[4] = bf16lo(rv.z); acc[5] = bf16hi(rv.z); acc[6] = bf16lo(rv.w); acc[7] = bf16hi(rv.w);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
  }
  const int32_t* tid_ids = ids + static_cast<size_t>(t) * k;
  for (uint32_t r = 0; r < k; ++r) {
    const int32_t e = tid_ids[r];
    bool skip = e < 0 || static_cast<uint32_t>(e) >= E;  // rows the grouping skipped
    for (uint32_t q = 0; q < r; ++q) skip = skip || tid_ids[q] == e;
    if (skip) continue;
    const float wr = w[static_cast<size_t>(t) * k + r];
    const uint4 v = *reinterpret_cast<const uint4*>(Yp + (static_cast<size_t>(t) * k + r) * H + c);
    acc[0] = __builtin_fmaf(wr, bf16lo(v.x), acc[0]); acc[1] = __builtin_fmaf(wr, bf16hi(v.x), acc[1]);
    acc[2] = __builtin_fmaf(wr, bf16lo(v.y), acc[2]); acc[3] = __builtin_fmaf(wr, bf16hi(v.y), acc[3]);
    acc[4] = __builtin_fmaf(wr, bf16lo(v.z), acc[4]); acc[5] = __builtin_fmaf(wr, bf16hi(v.z), acc[5]);
    acc[6] = __builtin_fmaf(wr, bf16lo(v.w), acc[6]); acc[7] = __builtin_fmaf(wr, bf16hi(v.w), acc[7]);
  }
  *reinterpret_cast<uint4*>(y + static_cast<size_t>(t) * H + c) =
      make_uint4(pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]), pack_bf16x2(acc[4], acc[5]),
                 pack_bf16x2(acc[6], acc[7]));
}

constexpr size_t al256(size_t v) { return (v + 255) & ~size_t(255); }

struct PrefillWs {
  size_t logits, ids, w, counts, offsets, ntiles, chunk_cnt, row_token, row_slot, tiles, H, Yp, Xn, total;
  uint32_t max_tiles, nchunks;
};

PrefillWs prefill_layout(const obs_moe_config* cfg, uint32_t T) {
  PrefillWs L{};
  const size_t R = static_cast<size_t>(T) * cfg->top_k;
  L.max_tiles = static_cast<uint32_t>((R + TM - 1) / TM + cfg->n_exp);
  size_t o = 0;
  L.logits = o; o += al256(sizeof(float) * T * cfg->n_exp);
  L.ids = o; o += al256(sizeof(int32_t) * R);
  L.w = o; o += al256(sizeof(float) * R);
  L.counts = o; o += al256(sizeof(int32_t) * cfg->n_exp);
  L.offsets = o; o += al256(sizeof(int32_t) * (cfg->n_exp + 1));
  L.ntiles = o; o += 256;
  L.nchunks = (T + GROUP_TOKENS - 1) / GROUP_TOKENS;
  L.chunk_cnt = o; o += al256(sizeof(int32_t) * L.nchunks * cfg->n_exp);
  L.row_token = o; o += al256(sizeof(int32_t) * R);
  L.row_slot = o; o += al256(sizeof(int32_t) * R);
  L.tiles = o; o += al256(sizeof(int4) * L.max_tiles);
  L.H = o; o += al256(sizeof(uint16_t) * R * cfg->inter);
  L.Yp = o; o += al256(sizeof(uint16_t) * R * cfg->hidden);
  L.Xn = o; o += al256(sizeof(uint16_t) * static_cast<size_t>(T) * cfg->hidden);  // rmsnorm(X) when layer->norm_w
  L.total = o;
  return L;
}

// Staged scale|bias bytes per workgroup.
size_t gemm_sb_bytes(bool swiglu, uint32_t K) {
  return sizeof(uint32_t) * (swiglu ? 2u : 1u) * (K / GK) * SB_STRIDE;
}

// grid_tiles: an upper bound of the tile count (the device holds the exact one)
int launch_gemm(obs_ctx* ctx, bool swiglu, const GemmArgs& a, uint32_t grid_tiles) {
  const uint32_t items = grid_tiles * (a.N / TN);
  const uint32_t grid = (items + 7u) / 8u * 8u;  // every XCD gets the same number of slots
  const size_t lds = gemm_sb_bytes(swiglu, a.K);
  // the staged scales can take the block past 64 KB of LDS (gfx950 has 160 KB)
  static bool lds_raised = false;
  if (!lds_raised) {
    OBS_HIP_TRY(ctx, hipFuncSetAttribute(reinterpret_cast<const void*>(&grouped_gemm_kernel<true>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, SB_LDS_MAX));
    OBS_HIP_TRY(ctx, hipFuncSetAttribute(reinterpret_cast<const void*>(&grouped_gemm_kernel<false>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, SB_LDS_MAX));
    lds_raised = true;
  }
  if (swiglu)
    OBS_LAUNCH(ctx, "grouped_gemm_gateup", grouped_gemm_kernel<true><<<grid, 256, lds, ctx->stream>>>(a));
  else
    OBS_LAUNCH(ctx, "grouped_gemm_down", grouped_gemm_kernel<false><<<grid, 256, lds, ctx->stream>>>(a));
  return OBS_OK;
}

}  // namespace

extern "C" {

size_t obs_moe_prefill_workspace(const obs_moe_config* cfg, uint32_t T) {
  if (!cfg || T == 0) return 0;
  return prefill_layout(cfg, T).total;
}

int obs_moe_prefill(obs_ctx* ctx, const obs_moe_config* cfg, const obs_moe_layer* layer, const uint16_t* X,
                    const uint16_t* residual, uint16_t* Y, uint32_t T, const int32_t* ids, const float* weights,
                    void* ws, size_t ws_bytes) {
  if (!ctx) return OBS_E_INVALID;
  int rc = obs::check_moe_config(ctx, "obs_moe_prefill", cfg);
  if (rc) return rc;
  rc = obs::check_moe_layer(ctx, "obs_moe_prefill", layer);
  if (rc) return rc;
  if (!X || !Y || !ws) return obs::set_error(ctx, OBS_E_INVALID, "obs_moe_prefill: null X, Y or workspace");
  if ((ids == nullptr) != (weights == nullptr))
    return obs::set_error(ctx, OBS_E_INVALID, "obs_moe_prefill: pass both ids and weights, or neither");
  if (T == 0) return OBS_OK;
  const uint32_t E = cfg->n_exp, k = cfg->top_k, H = cfg->hidden, I = cfg->inter;
  if (H % TN != 0 || I % TN != 0)
    return obs::set_error(ctx, OBS_E_SHAPE, "obs_moe_prefill: hidden and inter must be multiples of %u", TN);
  const PrefillWs L = prefill_layout(cfg, T);
  if (ws_bytes < L.total)
    return obs::set_error(ctx, OBS_E_NOMEM, "obs_moe_prefill: workspace %zu bytes < %zu needed", ws_bytes, L.total);
  if (!obs::aligned(X, 16) || !obs::aligned(Y, 16) || (residual && !obs::aligned(residual, 16)) || !obs::aligned(ws, 256))
    return obs::set_error(ctx, OBS_E_ALIGN, "obs_moe_prefill: X/Y/residual need 16-byte, ws 256-byte alignment");
  char* base = static_cast<char*>(ws);
  const uint16_t* Xin = X;  // the MoE input: X, or rmsnorm(X) (forward.rs:419-421); X stays the caller's
  if (layer->norm_w) {
    uint16_t* Xn = reinterpret_cast<uint16_t*>(base + L.Xn);
    rc = obs::launch_rmsnorm(ctx, X, layer->norm_w, Xn, T, H, cfg->rms_eps);
    if (rc) return rc;
    Xin = Xn;
  }
  int32_t* d_ids = reinterpret_cast<int32_t*>(base + L.ids);
  float* d_w = reinterpret_cast<float*>(base + L.w);
  if (!ids) {
    rc = obs::launch_gate_logits(ctx, layer->router_w, layer->router_s, layer->router_b, Xin,
                                 reinterpret_cast<float*>(base + L.logits), T, H, E, cfg->group);
    if (rc) return rc;
    rc = obs::launch_route_topk(ctx, reinterpret_cast<float*>(base + L.logits), d_ids, d_w, T, E, k, cfg->norm_topk);
    if (rc) return rc;
    ids = d_ids;
    weights = d_w;
  }
  int32_t* counts = reinterpret_cast<int32_t*>(base + L.counts);
  int32_t* offsets = reinterpret_cast<int32_t*>(base + L.offsets);
  int32_t* ntiles = reinterpret_cast<int32_t*>(base + L.ntiles);
  int32_t* row_token = reinterpret_cast<int32_t*>(base + L.row_token);
  int32_t* row_slot = reinterpret_cast<int32_t*>(base + L.row_slot);
  int4* tiles = reinterpret_cast<int4*>(base + L.tiles);
  uint16_t* Hbuf = reinterpret_cast<uint16_t*>(base + L.H);
  uint16_t* Yp = reinterpret_cast<uint16_t*>(base + L.Yp);
  int32_t* chunk_cnt = reinterpret_cast<int32_t*>(base + L.chunk_cnt);
  OBS_LAUNCH(ctx, "moe_group_count", group_count_kernel<<<L.nchunks, 64, 0, ctx->stream>>>(ids, T, k, E, chunk_cnt));
  OBS_LAUNCH(ctx, "moe_group_scan", group_scan_kernel<<<1, 256, 0, ctx->stream>>>(L.nchunks, E, chunk_cnt, counts,
                                                                                   offsets, tiles, ntiles));
  OBS_LAUNCH(ctx, "moe_group_rank", group_rank_kernel<<<L.nchunks, 64, 0, ctx->stream>>>(ids, T, k, E, chunk_cnt,
                                                                                          row_token, row_slot));
  GemmArgs g{};
  g.A = Xin; g.a_rows = row_token; g.a_rows_total = T;
  g.w0 = layer->gate_w; g.s0 = layer->gate_s; g.b0 = layer->gate_b;
  g.w1 = layer->up_w; g.s1 = layer->up_s; g.b1 = layer->up_b;
  g.out = Hbuf; g.out_rows = nullptr;
  g.tiles = tiles; g.n_tiles = ntiles;
  g.K = H; g.N = I;
  rc = launch_gemm(ctx, true, g, L.max_tiles);
  if (rc) return rc;
  GemmArgs d{};
  d.A = Hbuf; d.a_rows = nullptr; d.a_rows_total = T * k;
  d.w0 = layer->down_w; d.s0 = layer->down_s; d.b0 = layer->down_b;
  d.out = Yp; d.out_rows = row_slot;
  d.tiles = tiles; d.n_tiles = ntiles;
  d.K = I; d.N = H;
  rc = launch_gemm(ctx, false, d, L.max_tiles);
  if (rc) return rc;
  OBS_LAUNCH(ctx, "moe_combine", combine_kernel<<<T, H / 8u, 0, ctx->stream>>>(Yp, ids, weights, residual, Y, k, H, E));
  return OBS_OK;
}

int obs_q4_matmul(obs_ctx* ctx, const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                  const uint16_t* X, uint16_t* Y, uint32_t T, uint32_t in, uint32_t out, uint32_t group) {
  if (!ctx) return OBS_E_INVALID;
  if (!w || !scales || !biases || !X || !Y) return obs::set_error(ctx, OBS_E_INVALID, "obs_q4_matmul: null pointer");
  if (group != GK) return obs::set_error(ctx, OBS_E_SHAPE, "obs_q4_matmul: group must be %u (got %u)", GK, group);
  if (in == 0 || in % (4u * GK) != 0 || out == 0 || out % TN != 0)
    return obs::set_error(ctx, OBS_E_SHAPE, "obs_q4_matmul: in must be a multiple of %u and out of %u (got %u, %u)",
                          4u * GK, TN, in, out);
  if (gemm_sb_bytes(false, in) > SB_LDS_MAX)
    return obs::set_error(ctx, OBS_E_SHAPE, "obs_q4_matmul: in must be at most %u (got %u)",
                          static_cast<uint32_t>(SB_LDS_MAX / (sizeof(uint32_t) * SB_STRIDE)) * GK, in);
  if (!obs::aligned(X, 16) || !obs::aligned(w, 16) || !obs::aligned(Y, 16))
    return obs::set_error(ctx, OBS_E_ALIGN, "obs_q4_matmul: X, w and Y must be 16-byte aligned");
  if (T == 0) return OBS_OK;
  const uint32_t tiles = (T + TM - 1) / TM;
  GemmArgs g{};
  g.A = X; g.a_rows = nullptr; g.a_rows_total = T;
  g.w0 = w; g.s0 = scales; g.b0 = biases;
  g.out = Y; g.out_rows = nullptr;
  g.tiles = nullptr; g.n_tiles = nullptr; g.dense_rows = T;
  g.K = in; g.N = out;
  return launch_gemm(ctx, false, g, tiles);
}

}  // extern "C"
