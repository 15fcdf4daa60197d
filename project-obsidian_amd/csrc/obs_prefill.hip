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
// output columns; wave w owns columns [32w, 32w+32) and, in two of the three
// modes, a second set of 32 B columns: the same columns of the up matrix
// (gate/up, SwiGLU epilogue) or columns [128 + 32w, +32) of the same matrix
// (wide mode, a 256-column tile: down). Per 64-column quantization group:
//   - A (activations, gathered by row through a_rows) is staged in LDS,
//     double-buffered, row stride padded to 72 bf16;
//   - B is read straight from HBM into registers: lane l takes 16 bytes
//     (32 nibbles) of weight row n = n0 + 32w + l%32, columns
//     [k0 + 32(l/32), +32), and dequantizes them to bf16 = RNE(q*s + b) with
//     the tile's scales and biases, staged once per tile in LDS;
//   - v_mfma_f32_32x32x16_bf16 accumulates in fp32. The MFMA's 16 k-slots of
//     K-step s map to columns k0 + 32h + 8s + j (h = lane half, j = 0..7), for
//     A and B alike, so each lane's 16-byte load feeds all four K-steps.
#include <algorithm>

#include "obs_internal.hpp"

namespace obs {
int check_moe_config(obs_ctx* ctx, const char* who, const obs_moe_config* cfg);
int check_moe_layer(obs_ctx* ctx, const char* who, const obs_moe_layer* L);
int launch_route(obs_ctx* ctx, const uint32_t* w8, const uint16_t* s, const uint16_t* b, const uint16_t* x,
                 float* logits, int32_t* ids, float* w, uint32_t T, uint32_t in, uint32_t n_exp, uint32_t group,
                 uint32_t k, int norm_topk, int rule);
}  // namespace obs

namespace {

using namespace obsd;

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));  // register-friendly 16-byte word

constexpr uint32_t TM = 128;          // tile rows
constexpr uint32_t TN = 128;          // tile output columns per B column set (4 waves x 32)
constexpr uint32_t GK = 64;           // quantization group = K step of the main loop
constexpr uint32_t LDS_STRIDE = 72;   // bf16 per staged A row (64 + 8 padding)
constexpr uint32_t GROUP_TOKENS = 64; // tokens per grouping chunk (one wave)
constexpr uint32_t SB_STRIDE = TN + 1;  // words per (matrix, group) row of staged scale|bias
constexpr uint32_t SB_LDS_MAX = 96u * 1024u;  // bytes of staged scale|bias per workgroup

// Kernel modes: one B matrix, 128 columns; gate and up with a SwiGLU epilogue;
// one B matrix, 256 columns (the second column set is the first one + 128 rows).
enum GemmMode : uint32_t { MODE_NARROW = 0, MODE_SWIGLU = 1, MODE_WIDE = 2 };
// Which row maps and work source a launch has (template flags, so that no load
// sits under a branch: a load on one side of a branch makes the compiler wait
// for every load at the join).
enum GemmFlags : uint32_t { F_WORK = 1, F_AROWS = 2, F_OROWS = 4 };
__host__ __device__ constexpr uint32_t mode_cols(uint32_t mode) { return mode == MODE_WIDE ? 2u * TN : TN; }

struct GemmArgs {
  const uint16_t* A;        // bf16 [a_rows_total, K]
  const int32_t* a_rows;    // permuted row -> A row (with F_AROWS; else identity)
  uint32_t a_rows_total;    // bound for a_rows values
  const uint32_t* w0; const uint16_t* s0; const uint16_t* b0;  // [E, N, K/8], [E, N, K/64]
  const uint32_t* w1; const uint16_t* s1; const uint16_t* b1;  // second B column set: up (SwiGLU), +128 rows (wide)
  uint16_t* out;            // bf16 rows of N
  const int32_t* out_rows;  // permuted row -> output row (with F_OROWS; else identity)
  const int4* work;         // per workgroup {expert, row0, rows, n0} with F_WORK; else dense rows of expert 0
  const int32_t* work_count;  // items per XCD: workgroup l has one iff l / 8 < work_count[l % 8]
  uint32_t dense_rows;      // row count in dense mode
  uint32_t K, N;
};

// Two fp32 values -> one packed bf16 pair (RNE, v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16_rne(float lo, float hi) { return pack_bf16_pair_rne(lo, hi); }

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

// B operand of one 64-column group for one lane: 16 bytes (32 nibbles) of its
// weight row in each B column set.
struct BRaw {
  u32x4_t q0, q1;
};

// Per-thread operand pointers of a tile, set up by the kernel's prologue.
struct TileIn {
  const uint16_t* aptr[4];  // A row of staging row t/8 + 32i, at this thread's 16-byte chunk
  const u32x4_t* w0p;       // this lane's weight row (k half h), first column set; + 2g per group
  const u32x4_t* w1p;       // second column set (up matrix, or 128 rows further)
};

template <bool TWO>
__device__ __forceinline__ BRaw load_b(const TileIn& in, uint32_t g, uint32_t groups) {
  BRaw r;
  const uint32_t gg = g < groups ? g : groups - 1u;  // clamped: the tail loads are never used
  r.q0 = in.w0p[2u * gg];
  if (TWO) r.q1 = in.w1p[2u * gg];
  return r;
}

// One tile's main loop and epilogue, NB = active 32-row blocks (1..4), so the
// MFMA sequence is straight-line code. MIX: every staged scale is within
// dequant_word_mix's range (decided per tile). The prologue has loaded B
// groups 0 and 1 (bs0, bs1) and A group 0 (ras).
template <uint32_t MODE, uint32_t NB, bool MIX>
__device__ __forceinline__ void gemm_tile(const GemmArgs& a, uint16_t (&sA)[2][TM * LDS_STRIDE],
                                          const int32_t* s_orow, const uint32_t* s_sb, const TileIn& in,
                                          uint32_t nrows, uint32_t n0, BRaw bs0, BRaw bs1, u32x4_t (&ras)[4]) {
  constexpr bool SWIGLU = MODE == MODE_SWIGLU, TWO = MODE != MODE_NARROW;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t nl = 32u * wave + (lane & 31u);                   // this lane's column in the tile
  const uint32_t h = lane >> 5;                                    // k half within a group
  const uint32_t K = a.K, groups = K / GK;

  // A staging: thread t -> 16 bytes (8 bf16, chunk t % 8 of the group) of tile
  // rows t/8 + 32i, i = 0..3, so each wave instruction reads 8 whole 128-byte
  // row segments. Rows of blocks >= NB are never read by the MFMAs and are not
  // staged (i is unrolled, so this costs no branch).
  const uint32_t ac = 8u * (tid & 7u);
  auto load_a = [&](uint32_t g, u32x4_t (&r)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (uint32_t i = 0; i < NB; ++i) r[i] = *reinterpret_cast<const u32x4_t*>(in.aptr[i] + g * GK);
  };
  auto store_a = [&](uint32_t buf, const u32x4_t (&r)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (uint32_t i = 0; i < NB; ++i)
      *reinterpret_cast<u32x4_t*>(&sA[buf][(tid / 8u + 32u * i) * LDS_STRIDE + ac]) = r[i];
  };
  // staged scale|bias of this lane's column: [matrix][group] at stride SB_STRIDE words
  const uint32_t* sb0 = s_sb + nl;
  const uint32_t* sb1 = s_sb + static_cast<size_t>(groups) * SB_STRIDE + nl;

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
  store_a(0, ras);

  auto step = [&](uint32_t g, BRaw& bcur) __attribute__((always_inline)) {
    const uint32_t buf = g & 1u;
    __syncthreads();  // A of group g visible in sA[buf]; sA[buf^1] no longer read
    load_a(g + 1 < groups ? g + 1 : g, ras);  // the tail reload is stored but never read
    // B two groups ahead, issued right after A: loads complete in issue order,
    // so the A store at the end of this group waits only for loads issued a
    // group or more earlier, and B has two groups to arrive
    const BRaw bnext = load_b<TWO>(in, g + 2, groups);  // clamped past the end; never used there
    // keep the loads here, a whole group ahead of their use: left to itself the
    // scheduler sinks them next to the store and exposes their latency
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t sv0 = sb0[g * SB_STRIDE];
    const uint32_t sv1 = TWO ? sb1[g * SB_STRIDE] : 0u;
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
      if (TWO) f1 = MIX ? dequant_word_mix(q1w[st], m1) : dequant_word(q1w[st], bf16lo(sv1), bf16hi(sv1));
#pragma unroll
      for (uint32_t mb = 0; mb < NB; ++mb) {
        acc0[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mb], f0, acc0[mb], 0, 0, 0);
        if (TWO) acc1[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mb], f1, acc1[mb], 0, 0, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // the A store waits for its loads: keep it last
    bcur = bnext;
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
  // i0 and i0+2, the odd lane rows i0+1 and i0+3. The wide mode writes its two
  // 128-column halves one after the other through the same buffer.
  constexpr uint32_t C_STRIDE = TN + 8;  // bf16 per staged row (bank spread)
  static_assert(TM * C_STRIDE <= 2 * TM * LDS_STRIDE, "C tile must fit the A buffers");
  uint16_t* sC = reinterpret_cast<uint16_t*>(sA);
  const uint32_t odd = nl & 1u, c_even = nl & ~1u;
  const uint32_t sel = odd ? 0x03020706u : 0x05040100u;  // v_perm: (partner.hi, own.hi) : (own.lo, partner.lo)
  auto emit = [&](uint32_t half) __attribute__((always_inline)) {
    __syncthreads();  // every wave is done reading sA (or the previous half)
#pragma unroll
    for (uint32_t mb = 0; mb < NB; ++mb) {
#pragma unroll
      for (uint32_t qd = 0; qd < 4; ++qd) {
        float v[4];
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
          const float c0 = acc0[mb][4 * qd + j], c1 = acc1[mb][4 * qd + j];
          v[j] = SWIGLU ? silu_mul_fast(c0, c1) : (half ? c1 : c0);
        }
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
        *reinterpret_cast<uint4*>(a.out + static_cast<size_t>(s_orow[i]) * a.N + n0 + TN * half + c8) = v;
      }
    }
  };
  emit(0);
  if (MODE == MODE_WIDE) emit(1);
}

// Work items are (tile, column block) pairs in tile order, and tiles are in
// expert order. The dispatcher deals consecutive workgroups round-robin over
// the 8 XCDs, so workgroup l takes item (l % 8) * chunk + l / 8 (the grouping
// writes that table, work_table_fill): each XCD runs a contiguous run of
// items, and the tiles of one expert share its weights (and the column blocks
// of one tile share its activation rows) in that XCD's L2.
// Two workgroups per CU (at most 256 registers per lane): the co-resident
// workgroup hides each one's load, LDS and barrier latency.
template <uint32_t MODE, uint32_t FLAGS>
__device__ __forceinline__ void gemm_item(const GemmArgs& a, uint32_t e, uint32_t row0, uint32_t nrows, uint32_t n0,
                                          uint16_t (&sA)[2][TM * LDS_STRIDE], int32_t* s_orow, uint32_t* s_sb);

template <uint32_t MODE, uint32_t FLAGS>
__global__ void __launch_bounds__(256, 2) grouped_gemm_kernel(GemmArgs a) {
  __shared__ uint16_t sA[2][TM * LDS_STRIDE];
  __shared__ int32_t s_orow[TM];
  extern __shared__ uint32_t s_sb[];  // [matrix][group][SB_STRIDE]: scale | bias << 16
  // The work item: one load from the grouping's per-workgroup table, or, for
  // dense rows, arithmetic on the launch index.
  uint32_t e, row0, nrows, n0;
  if (FLAGS & F_WORK) {
    // both loads at once: the entry is inside the table even where it is unused
    const int32_t count = a.work_count[blockIdx.x % 8u];
    const int4 w = a.work[blockIdx.x];
    if (static_cast<int32_t>(blockIdx.x / 8u) >= count) return;  // uniform per workgroup
    e = static_cast<uint32_t>(w.x);
    row0 = static_cast<uint32_t>(w.y);
    nrows = static_cast<uint32_t>(w.z);
    n0 = static_cast<uint32_t>(w.w);
  } else {
    const uint32_t ncb = a.N / mode_cols(MODE);
    const uint32_t n_items = (a.dense_rows + TM - 1u) / TM * ncb, chunk = (n_items + 7u) / 8u;
    const uint32_t item = (blockIdx.x % 8u) * chunk + blockIdx.x / 8u;
    if (blockIdx.x / 8u >= chunk || item >= n_items) return;
    e = 0;
    row0 = item / ncb * TM;
    nrows = min(TM, a.dense_rows - row0);
    n0 = item % ncb * mode_cols(MODE);
  }
  gemm_item<MODE, FLAGS>(a, e, row0, nrows, n0, sA, s_orow, s_sb);
}

// One work item: rows [row0, row0 + nrows) of expert e's group (at most TM),
// output columns from n0 (mode_cols(MODE) of them).
template <uint32_t MODE, uint32_t FLAGS>
__device__ __forceinline__ void gemm_item(const GemmArgs& a, uint32_t e, uint32_t row0, uint32_t nrows, uint32_t n0,
                                          uint16_t (&sA)[2][TM * LDS_STRIDE], int32_t* s_orow, uint32_t* s_sb) {
  constexpr bool TWO = MODE != MODE_NARROW;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t K = a.K, groups = K / GK;

  // Every load that depends on the work item alone is issued before any is
  // waited for: this thread's A row ids, the output row map, the tile's scales
  // and biases, B groups 0 and 1. A group 0 follows as soon as its row ids are
  // in. All of them are unconditional (indices clamped into the tile, results
  // selected afterwards), so the waits count exactly the loads they need.
  // Padding rows (r >= nrows) repeat the tile's last row: row i of an MFMA
  // product depends on row i of A only, and the epilogue discards them. They
  // never name a row outside the tile: in the one-launch FFN the A of a down
  // item is H, and only its own tile's rows are complete once its wait passes.
  int32_t arow[4];
#pragma unroll
  for (uint32_t i = 0; i < 4; ++i) {
    const uint32_t r = min(tid / 8u + 32u * i, nrows - 1u);
    arow[i] = (FLAGS & F_AROWS) ? a.a_rows[row0 + r] : static_cast<int32_t>(row0 + r);
  }
  // threads t and t + 128 load and store the same entry (an unconditional store
  // keeps the load from sinking under a branch)
  const uint32_t orow_i = min(tid & (TM - 1u), nrows - 1u);
  const int32_t orow = (FLAGS & F_OROWS) ? a.out_rows[row0 + orow_i] : static_cast<int32_t>(row0 + orow_i);

  // Scales and biases of the tile's weight rows: rows n0.. of expert e are
  // contiguous ([E, N, groups] bf16), so 8-byte chunks (4 groups of one row;
  // groups % 4 == 0) load coalesced; each becomes 4 packed words in LDS. A
  // batch (4 chunks per thread and matrix; past the end they reload the last
  // chunk) covers K <= 2048; all its loads are issued before any is stored.
  constexpr uint32_t NMAT = TWO ? 2u : 1u, PER = 4u;
  const uint32_t cpr = groups / 4u, nchunk = TN * cpr;  // chunks per row, per matrix
  const size_t sbase = (static_cast<size_t>(e) * a.N + n0) * groups;
  bool wide_scale = false;  // some staged |s| is beyond dequant_word_mix's range
  uint2 sv[NMAT][PER], bv[NMAT][PER];
  auto issue_scales = [&](uint32_t c0) __attribute__((always_inline)) {
#pragma unroll
    for (uint32_t mat = 0; mat < NMAT; ++mat) {
      const uint2* sp = reinterpret_cast<const uint2*>((mat ? a.s1 : a.s0) + sbase);
      const uint2* bp = reinterpret_cast<const uint2*>((mat ? a.b1 : a.b0) + sbase);
#pragma unroll
      for (uint32_t j = 0; j < PER; ++j) {
        const uint32_t c = min(c0 + tid + 256u * j, nchunk - 1u);
        sv[mat][j] = sp[c];
        bv[mat][j] = bp[c];
      }
    }
  };
  auto store_scales = [&](uint32_t c0) __attribute__((always_inline)) {
#pragma unroll
    for (uint32_t mat = 0; mat < NMAT; ++mat) {
#pragma unroll
      for (uint32_t j = 0; j < PER; ++j) {
        // clamped like the load: past the end, the last chunk is written again with
        // the same values (no branch, so the loads cannot sink next to the stores)
        const uint32_t c = min(c0 + tid + 256u * j, nchunk - 1u);
        uint2 s2 = sv[mat][j], b2 = bv[mat][j];
        // an opaque use here, after the issue phase: without it the range checks
        // below are hoisted above the scheduling barrier, and their wait with them
        asm volatile("" : "+v"(s2.x), "+v"(s2.y), "+v"(b2.x), "+v"(b2.y));
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
  };
  issue_scales(0);

  TileIn in;
  {
    const uint32_t n = n0 + 32u * wave + (lane & 31u), h = lane >> 5;  // this lane's weight row, k half
    const size_t wrow = static_cast<size_t>(e) * a.N + n;
    in.w0p = reinterpret_cast<const u32x4_t*>(a.w0 + wrow * (K / 8)) + h;
    in.w1p = TWO ? reinterpret_cast<const u32x4_t*>(a.w1 + wrow * (K / 8)) + h : nullptr;
  }
  const BRaw bs0 = load_b<TWO>(in, 0, groups), bs1 = load_b<TWO>(in, 1, groups);

  const uint32_t nb = (nrows + 31u) / 32u, ac = 8u * (tid & 7u);
  u32x4_t ras[4];
#pragma unroll
  for (uint32_t i = 0; i < 4; ++i) {
    // clamped into A: a corrupt row map (the grouping never writes one) reads
    // a wrong row instead of faulting
    const int32_t r = min(max(arow[i], 0), static_cast<int32_t>(a.a_rows_total) - 1);
    in.aptr[i] = a.A + static_cast<size_t>(r) * K + ac;
    ras[i] = *reinterpret_cast<const u32x4_t*>(in.aptr[i]);  // A group 0 (rows of unused blocks too)
  }
  // every load above is issued before the first wait below: left alone, the
  // scheduler moves the scale stores (and their waits) ahead of the B and A loads
  __builtin_amdgcn_sched_barrier(0);

  s_orow[tid & (TM - 1u)] = orow;
  store_scales(0);
  for (uint32_t c0 = PER * 256u; c0 < nchunk; c0 += PER * 256u) {  // K > 2048 only
    issue_scales(c0);
    store_scales(c0);
  }
  const bool mix = !__syncthreads_or(wide_scale);  // uniform per workgroup
  if (mix) {
    switch (nb) {
      case 1: gemm_tile<MODE, 1, true>(a, sA, s_orow, s_sb, in, nrows, n0, bs0, bs1, ras); break;
      case 2: gemm_tile<MODE, 2, true>(a, sA, s_orow, s_sb, in, nrows, n0, bs0, bs1, ras); break;
      case 3: gemm_tile<MODE, 3, true>(a, sA, s_orow, s_sb, in, nrows, n0, bs0, bs1, ras); break;
      default: gemm_tile<MODE, 4, true>(a, sA, s_orow, s_sb, in, nrows, n0, bs0, bs1, ras); break;
    }
  } else {  // scales beyond 2^100 (never in real checkpoints): reference-form dequant
    gemm_tile<MODE, 4, false>(a, sA, s_orow, s_sb, in, nrows, n0, bs0, bs1, ras);
  }
}

// ---- the expert FFN of a prefill in one launch: the gate/up items, then the
// down items, of each XCD. Workgroup l = 8p + x runs XCD x's p-th item: its
// gate/up items first (p < g.work_count[x]), then its down items. Both
// lists cover the same tiles per XCD (the tables split the tiles by their
// combined cost), so a tile's H rows are written and read through one L2: a
// gate/up item counts itself in tile_done[row0] once its H stores are
// complete, and a down item starts when all ncb_gu of its tile's items have
// counted. The dispatcher hands out workgroups in index order, so a waiting
// down item waits only for gate/up items already running; the down items of
// the first tiles fill the slots the last gate/up items leave idle. The wait
// is bounded: a time-out sets the calling context's status word (read and
// cleared by obs_device_status of that context) and the item runs anyway, so
// the grid always drains.
struct FfnSync {
  int32_t* tile_done;  // per tile, at its first grouped row: gate/up items done
  int32_t need;        // counts a down item waits for: the tile's gate/up items (more only under a test hook)
  uint64_t ticks;      // wait limit in ticks of wall_clock64 (100 MHz); 100 ms unless a test shortens it
  uint32_t* err;       // the context's status words (obs::CTX_ST_FFN_WAIT)
};

template <uint32_t MODE_DN>
__global__ void __launch_bounds__(256, 2) moe_ffn_kernel(GemmArgs g, GemmArgs d, FfnSync sy) {
  __shared__ uint16_t sA[2][TM * LDS_STRIDE];
  __shared__ int32_t s_orow[TM];
  extern __shared__ uint32_t s_sb[];
  const uint32_t x = blockIdx.x % 8u, p = blockIdx.x / 8u, tid = threadIdx.x;
  const uint32_t ngu = static_cast<uint32_t>(g.work_count[x]), ndn = static_cast<uint32_t>(d.work_count[x]);
  if (p < ngu) {
    const int4 w = g.work[blockIdx.x];
    gemm_item<MODE_SWIGLU, F_WORK | F_AROWS>(g, static_cast<uint32_t>(w.x), static_cast<uint32_t>(w.y),
                                             static_cast<uint32_t>(w.z), static_cast<uint32_t>(w.w), sA, s_orow, s_sb);
    // this thread's H stores are complete (on gfx9 the vector memory counter
    // counts stores too); then one add for the workgroup, in this XCD's L2
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (tid == 0) __hip_atomic_fetch_add(sy.tile_done + w.y, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else if (p - ngu < ndn) {
    const int4 w = d.work[8u * (p - ngu) + x];
    if (tid == 0) {
      const uint64_t t0 = wall_clock64();
      while (__hip_atomic_load(sy.tile_done + w.y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < sy.need) {
        if (wall_clock64() - t0 > sy.ticks) {
          __hip_atomic_store(sy.err + obs::CTX_ST_FFN_WAIT, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
          break;
        }
      }
    }
    __syncthreads();
    gemm_item<MODE_DN, F_WORK | F_OROWS>(d, static_cast<uint32_t>(w.x), static_cast<uint32_t>(w.y),
                                         static_cast<uint32_t>(w.z), static_cast<uint32_t>(w.w), sA, s_orow, s_sb);
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

// Measured cost of one (tile, column block) item by its active 32-row blocks
// (1..4), in thousands of core cycles (per-wave timestamps at T = 2048 on
// MI355X, two workgroups per CU, items in this schedule's order; 2 and 3
// interpolated): gate/up 66, 82, 98, 114; down (256 columns) 35, 41, 48, 54.
// Only their ratios matter: they balance the XCDs.
// Four 16-bit costs in one word: the device extracts one with a shift (a
// four-entry array, or a select chain the compiler turns into one, would be
// read from scratch memory).
struct ItemCost {
  unsigned long long packed;
  __host__ __device__ constexpr uint32_t of(uint32_t nb) const {
    return static_cast<uint32_t>((packed >> (16u * (nb - 1u))) & 0xffffu);
  }
};
constexpr ItemCost item_cost(uint32_t c1, uint32_t c2, uint32_t c3, uint32_t c4) {
  return ItemCost{c1 | (static_cast<unsigned long long>(c2) << 16) | (static_cast<unsigned long long>(c3) << 32) |
                  (static_cast<unsigned long long>(c4) << 48)};
}
constexpr ItemCost COST_GATEUP = item_cost(66, 82, 98, 114);
constexpr ItemCost COST_DOWN = item_cost(35, 41, 48, 54);
// Per-tile cost of a tile's items in one GEMM (ncb of them), or in both GEMMs.
constexpr ItemCost tile_cost(const ItemCost& c, uint32_t ncb) {
  return item_cost(c.of(1) * ncb, c.of(2) * ncb, c.of(3) * ncb, c.of(4) * ncb);
}
constexpr ItemCost tile_cost2(const ItemCost& a, uint32_t na, const ItemCost& b, uint32_t nb) {
  return item_cost(a.of(1) * na + b.of(1) * nb, a.of(2) * na + b.of(2) * nb, a.of(3) * na + b.of(3) * nb,
                   a.of(4) * na + b.of(4) * nb);
}
constexpr uint32_t SCHED_MAX_TILES = 2048;  // tiles the cost-balanced schedule handles (else even split)

// Workgroups a grouped GEMM launch needs for at most max_tiles tiles: an XCD's
// cost share (total / 8) holds at most max_tiles * cmax / (8 * cmin) + 1 tiles
// (cost: the per-tile cost the tiles are split by).
uint32_t sched_grid(uint32_t max_tiles, uint32_t ncb, const ItemCost& cost) {
  const uint64_t cmin = cost.of(1), cmax = cost.of(4);
  const uint64_t per_xcd = (static_cast<uint64_t>(max_tiles) * cmax + 8u * cmin - 1u) / (8u * cmin) + 1u;
  const uint64_t even = (static_cast<uint64_t>(max_tiles) + 7u) / 8u;
  return static_cast<uint32_t>(8u * (per_xcd > even ? per_xcd : even) * ncb);
}

// One GEMM's work table: where it goes and what its items cost. count[x] is the
// number of items XCD x runs; entries at or beyond it are not written.
struct WorkTable {
  int4* work;
  int32_t* count;
  uint32_t grid, ncb, cols;
  ItemCost split;       // per-tile cost the tiles are split over the XCDs by
  int32_t* tile_done;   // when set: zeroed at each tile's first row (the one-launch FFN's counters)
  uint32_t* err;        // with tile_done: the context's status words (obs::CTX_ST_FFN_SCHED)
};

// Exclusive prefix sum over the wave (64 lanes) and the wave total.
template <typename T>
__device__ __forceinline__ T wave_exclusive_scan(T v, T* total) {
  const uint32_t lane = threadIdx.x & 63u;
  T x = v;
#pragma unroll
  for (uint32_t d = 1; d < 64; d <<= 1) {
    const T y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  *total = __shfl(x, 63, 64);
  return x - v;
}

struct SchedLds {
  uint8_t te[SCHED_MAX_TILES];   // tile -> expert (E <= 256)
  uint8_t tnb[SCHED_MAX_TILES];  // tile -> active 32-row blocks (1..4)
  int32_t toff[257], roff[256], cnt[256];  // expert's first tile (toff[E] = all tiles), first row, rows
  uint32_t first[9];             // XCD x's tiles are [first[x], first[x + 1])
  unsigned long long pfirst[9];  // tiles with 1..4 blocks before first[x], 16-bit fields
  uint32_t over;                 // some XCD's share exceeds the launch's workgroups
};

// One GEMM's per-workgroup work table (read by grouped_gemm_kernel), built by
// one wave. The dispatcher deals consecutive workgroups round-robin over the
// 8 XCDs and, within an XCD, to the first free slot, so workgroup l = 8p + x is
// the p-th item XCD x runs. Tiles (expert order) are split into 8 contiguous
// ranges of equal measured cost, one per XCD, so an expert's tiles share its
// weights in one L2; within an XCD the items run in decreasing cost (longest
// first). W.count[x] = the number of items XCD x runs. When the schedule does
// not fit (more than SCHED_MAX_TILES tiles, or an XCD share beyond the
// launch), the items are split evenly by count instead, in item order.
__device__ void work_table_fill(const WorkTable W, uint32_t E, SchedLds& L) {  // by value: no scratch copy
  const uint32_t lane = threadIdx.x & 63u, T_all = static_cast<uint32_t>(L.toff[E]), slots = W.grid / 8u;
  const uint32_t ncb = W.ncb;
  auto cost = [&](uint32_t nb) __attribute__((always_inline)) { return W.split.of(nb); };
  auto item_of = [&](uint32_t e, uint32_t q, uint32_t cb) __attribute__((always_inline)) {
    const int32_t r0 = static_cast<int32_t>(q * TM);
    return make_int4(static_cast<int32_t>(e), L.roff[e] + r0, min(static_cast<int32_t>(TM), L.cnt[e] - r0),
                     static_cast<int32_t>(cb * W.cols));
  };
  if (T_all <= SCHED_MAX_TILES) {
    // Tallies of tiles by block count are packed 16 bits per count (T_all <=
    // 2048 fits), so they add and scan as one integer: an array indexed by the
    // block count would live in scratch memory.
    auto unit = [](uint32_t nb) { return 1ull << (16u * (nb - 1u)); };
    auto field = [](unsigned long long p, uint32_t nb) { return static_cast<uint32_t>((p >> (16u * (nb - 1u))) & 0xffffu); };
    // this lane's contiguous block of tiles: cost and tallies
    const uint32_t P = (T_all + 63u) / 64u, ta = min(lane * P, T_all), tb = min(ta + P, T_all);
    uint32_t csum = 0;
    unsigned long long vsum = 0;
    for (uint32_t t = ta; t < tb; ++t) {
      csum += cost(L.tnb[t]);
      vsum += unit(L.tnb[t]);
    }
    uint32_t total;
    unsigned long long vtot;
    const uint32_t cpre = wave_exclusive_scan(csum, &total);
    const unsigned long long vpre = wave_exclusive_scan(vsum, &vtot);
    if (lane < 9) {
      L.first[lane] = T_all;
      L.pfirst[lane] = vtot;
    }
    if (lane == 0) L.over = 0;
    __syncthreads();
    // XCD of a tile: where its cost starts (32-bit: total <= 2048 tiles x 1,116)
    auto xcd_at = [&](uint32_t c) __attribute__((always_inline)) {
      return total ? min(7u, c * 8u / total) : 0u;
    };
    {
      uint32_t c = cpre;
      unsigned long long v = vpre;
      int32_t xprev = ta == 0 ? -1 : static_cast<int32_t>(xcd_at(cpre - cost(L.tnb[ta - 1u])));
      for (uint32_t t = ta; t < tb; ++t) {
        const int32_t x = static_cast<int32_t>(xcd_at(c));
        for (int32_t y = xprev + 1; y <= x; ++y) {
          L.first[y] = t;
          L.pfirst[y] = v;
        }
        xprev = x;
        c += cost(L.tnb[t]);
        v += unit(L.tnb[t]);
      }
    }
    __syncthreads();
    if (lane < 8 && (L.first[lane + 1] - L.first[lane]) * ncb > slots) L.over = 1;
    __syncthreads();
    if (L.over == 0) {
      uint32_t c = cpre;
      unsigned long long v = vpre;
      for (uint32_t t = ta; t < tb; ++t) {
        const uint32_t x = xcd_at(c), nb = L.tnb[t], e = L.te[t], q = t - static_cast<uint32_t>(L.toff[e]);
        const unsigned long long lo = L.pfirst[x], hi = L.pfirst[x + 1];
        uint32_t pos = field(v, nb) - field(lo, nb);  // same block count, earlier in this XCD
        for (uint32_t w = nb + 1u; w <= 4u; ++w) pos += field(hi, w) - field(lo, w);
        for (uint32_t cb = 0; cb < ncb; ++cb) W.work[8u * (pos * ncb + cb) + x] = item_of(e, q, cb);
        if (W.tile_done) W.tile_done[L.roff[e] + static_cast<int32_t>(q * TM)] = 0;
        c += cost(nb);
        v += unit(nb);
      }
      if (lane < 8) W.count[lane] = static_cast<int32_t>((L.first[lane + 1] - L.first[lane]) * ncb);
      return;
    }
  }
  // The one-launch FFN needs the cost-balanced split (a tile's items on one
  // XCD, its counters zeroed); its launch is sized so that split always fits
  // (sched_grid), so this is never reached with tile_done set. Should it be,
  // the context's status word says the launch's outputs are invalid.
  if (W.tile_done && lane == 0)
    __hip_atomic_store(W.err + obs::CTX_ST_FFN_SCHED, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  // even split by count: XCD x runs items [x * chunk, (x + 1) * chunk) in item order
  const uint32_t n_items = T_all * ncb, chunk = (n_items + 7u) / 8u;
  for (uint32_t i = lane; i < n_items; i += 64u) {
    const int32_t t = static_cast<int32_t>(i / ncb);
    uint32_t lo = 0, hi = E;  // the last expert whose first tile is <= t: toff[lo] <= t < toff[hi]
    while (hi - lo > 1u) {
      const uint32_t mid = (lo + hi) / 2u;
      if (L.toff[mid] <= t) lo = mid; else hi = mid;
    }
    W.work[8u * (i % chunk) + i / chunk] = item_of(lo, static_cast<uint32_t>(t - L.toff[lo]), i % ncb);
  }
  if (lane < 8) W.count[lane] = static_cast<int32_t>(min(chunk, n_items - min(n_items, lane * chunk)));
}

// A scheduling wave: per-expert tiles from the row counts, then one GEMM's
// work table. The rank launch runs one per GEMM beside the ranking waves
// (nothing they write is read before the GEMMs).
__device__ void build_work_table(const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets, uint32_t E,
                                 const WorkTable W) {
  __shared__ SchedLds L;
  const uint32_t lane = threadIdx.x & 63u;
  // lane owns experts 4 * lane + j (E <= 256), kept in registers (static indices)
  uint32_t rows[4], nts = 0;
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j) {
    const uint32_t e = 4u * lane + j, ec = min(e, E - 1u);  // clamped loads: no branch to wait at
    const int32_t c = counts[ec], o = offsets[ec];
    rows[j] = e < E ? static_cast<uint32_t>(c) : 0u;
    if (e < E) {
      L.cnt[e] = c;
      L.roff[e] = o;
    }
    nts += (rows[j] + TM - 1u) / TM;
  }
  uint32_t T_all;
  uint32_t t = wave_exclusive_scan(nts, &T_all);
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j) {
    const uint32_t e = 4u * lane + j, nt = (rows[j] + TM - 1u) / TM;
    if (e < E) L.toff[e] = static_cast<int32_t>(t);
    if (T_all <= SCHED_MAX_TILES) {
      for (uint32_t q = 0; q < nt; ++q) {
        L.te[t + q] = static_cast<uint8_t>(e);
        L.tnb[t + q] = static_cast<uint8_t>((min(TM, rows[j] - q * TM) + 31u) / 32u);
      }
    }
    t += nt;
  }
  if (lane == 0) L.toff[E] = static_cast<int32_t>(T_all);
  __syncthreads();
  work_table_fill(W, E, L);
}

// 2. one workgroup (thread e = expert e, E <= 256): chunk counts -> absolute row
// bases per (chunk, expert), expert offsets and counts.
__global__ void __launch_bounds__(256) group_scan_kernel(uint32_t nchunks, uint32_t E, int32_t* __restrict__ chunk_cnt,
                                                         int32_t* __restrict__ counts, int32_t* __restrict__ offsets) {
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
  int32_t all_rows;
  const int32_t off = block_exclusive_scan256(tot, s_wave, &all_rows);
  if (have) {
    counts[e] = tot;
    offsets[e] = off;
    for (uint32_t c0 = 0; c0 < nchunks; c0 += 16u) {  // batched: all loads in flight together
      int32_t v[16];
#pragma unroll
      for (uint32_t i = 0; i < 16; ++i) v[i] = c0 + i < nchunks ? chunk_cnt[static_cast<size_t>(c0 + i) * E + e] : 0;
#pragma unroll
      for (uint32_t i = 0; i < 16; ++i)
        if (c0 + i < nchunks) chunk_cnt[static_cast<size_t>(c0 + i) * E + e] = v[i] + off;
    }
  }
  if (e == 0) offsets[E] = all_rows;
}

// 3. one wave per chunk: a token's row in expert e = chunk base + the number of
// lower lanes (earlier tokens) of the chunk routed to e (LDS lane bitmasks).
// Two more waves (the last two workgroups) build the GEMMs' work tables meanwhile.
__global__ void __launch_bounds__(64) group_rank_kernel(const int32_t* __restrict__ ids, uint32_t T, uint32_t k,
                                                        uint32_t E, const int32_t* __restrict__ chunk_base,
                                                        int32_t* __restrict__ row_token, int32_t* __restrict__ row_slot,
                                                        const int32_t* __restrict__ counts,
                                                        const int32_t* __restrict__ offsets, WorkTable gu,
                                                        WorkTable dn) {
  if (blockIdx.x + 2u >= gridDim.x) {  // uniform per workgroup
    build_work_table(counts, offsets, E, blockIdx.x + 2u == gridDim.x ? gu : dn);
    return;
  }
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

// The kernel mode of a GEMM: one-matrix GEMMs run wide when N allows it.
uint32_t gemm_mode(bool swiglu, uint32_t N) {
  return swiglu ? MODE_SWIGLU : (N % (2u * TN) == 0 ? MODE_WIDE : MODE_NARROW);
}
// Workgroups of a GEMM launch over at most `tiles` tiles: every XCD gets the same number.
uint32_t gemm_grid(uint32_t tiles, uint32_t N, uint32_t mode) {
  const uint32_t items = tiles * (N / mode_cols(mode));
  return (items + 7u) / 8u * 8u;
}

struct PrefillWs {
  size_t logits, ids, w, counts, offsets, chunk_cnt, row_token, row_slot, work_gu, work_dn, work_cnt, tile_done, H,
      Yp, Xn, total;
  uint32_t max_tiles, nchunks, grid_gu, grid_dn;
  bool ffn_one_launch;  // both GEMMs in moe_ffn_kernel (the tables then split tiles by their combined cost)
  ItemCost split_gu, split_dn;
};

// one_launch_ok: the device's dispatch allows the one-launch FFN (the workspace
// size does not depend on it).
PrefillWs prefill_layout(const obs_moe_config* cfg, uint32_t T, bool one_launch_ok) {
  PrefillWs L{};
  const size_t R = static_cast<size_t>(T) * cfg->top_k;
  L.max_tiles = static_cast<uint32_t>((R + TM - 1) / TM + cfg->n_exp);
  size_t o = 0;
  // the routing first, at the offsets the C ABI documents (read after a computed routing)
  L.ids = o; o += al256(sizeof(int32_t) * R);
  L.w = o; o += al256(sizeof(float) * R);
  L.logits = o; o += al256(sizeof(float) * T * cfg->n_exp);
  L.counts = o; o += al256(sizeof(int32_t) * cfg->n_exp);
  L.offsets = o; o += al256(sizeof(int32_t) * (cfg->n_exp + 1));
  L.nchunks = (T + GROUP_TOKENS - 1) / GROUP_TOKENS;
  L.chunk_cnt = o; o += al256(sizeof(int32_t) * L.nchunks * cfg->n_exp);
  L.row_token = o; o += al256(sizeof(int32_t) * R);
  L.row_slot = o; o += al256(sizeof(int32_t) * R);
  const uint32_t ncb_gu = cfg->inter / mode_cols(gemm_mode(true, cfg->inter));
  const uint32_t ncb_dn = cfg->hidden / mode_cols(gemm_mode(false, cfg->hidden));
  // One launch for both GEMMs needs the cost-balanced schedule for both tables
  // (the even split would put a tile's down items on other XCDs than its
  // gate/up items) and per-tile costs within 16 bits.
  L.ffn_one_launch = one_launch_ok && L.max_tiles <= SCHED_MAX_TILES &&
                     COST_GATEUP.of(4) * ncb_gu + COST_DOWN.of(4) * ncb_dn < 65536u;
  L.split_gu = L.ffn_one_launch ? tile_cost2(COST_GATEUP, ncb_gu, COST_DOWN, ncb_dn) : tile_cost(COST_GATEUP, ncb_gu);
  L.split_dn = L.ffn_one_launch ? L.split_gu : tile_cost(COST_DOWN, ncb_dn);
  L.grid_gu = sched_grid(L.max_tiles, ncb_gu, L.split_gu);
  L.grid_dn = sched_grid(L.max_tiles, ncb_dn, L.split_dn);
  L.work_gu = o; o += al256(sizeof(int4) * L.grid_gu);
  L.work_dn = o; o += al256(sizeof(int4) * L.grid_dn);
  L.work_cnt = o; o += 256;  // items per XCD, gate/up then down
  L.tile_done = o; o += al256(sizeof(int32_t) * R);  // by a tile's first row
  L.H = o; o += al256(sizeof(uint16_t) * R * cfg->inter);
  L.Yp = o; o += al256(sizeof(uint16_t) * R * cfg->hidden);
  L.Xn = o; o += al256(sizeof(uint16_t) * static_cast<size_t>(T) * cfg->hidden);  // rmsnorm(X) when layer->norm_w
  L.total = o;
  return L;
}

// Staged scale|bias bytes per workgroup.
size_t gemm_sb_bytes(uint32_t mode, uint32_t K) {
  return sizeof(uint32_t) * (mode == MODE_NARROW ? 1u : 2u) * (K / GK) * SB_STRIDE;
}

// grid: gemm_grid() of the launch; a.work (when set) has that many entries.
// A one-matrix GEMM whose N is a multiple of 256 runs in the wide mode: its
// second B column set is the first one 128 rows further on.
int launch_gemm(obs_ctx* ctx, GemmArgs a, uint32_t grid, uint32_t mode) {
  if (mode == MODE_WIDE) {
    a.w1 = a.w0 + static_cast<size_t>(TN) * (a.K / 8u);
    a.s1 = a.s0 + static_cast<size_t>(TN) * (a.K / GK);
    a.b1 = a.b0 + static_cast<size_t>(TN) * (a.K / GK);
  }
  const size_t lds = gemm_sb_bytes(mode, a.K);
  const uint32_t flags = (a.work ? F_WORK : 0u) | (a.a_rows ? F_AROWS : 0u) | (a.out_rows ? F_OROWS : 0u);
  // The launches this library makes: gate/up (work, A row map), down (work,
  // output row map) and dense matmuls (neither).
  struct Variant {
    uint32_t mode, flags;
    const void* fn;
    const char* name;
  };
  static const Variant variants[] = {
      {MODE_SWIGLU, F_WORK | F_AROWS, reinterpret_cast<const void*>(&grouped_gemm_kernel<MODE_SWIGLU, F_WORK | F_AROWS>),
       "grouped_gemm_gateup"},
      {MODE_WIDE, F_WORK | F_OROWS, reinterpret_cast<const void*>(&grouped_gemm_kernel<MODE_WIDE, F_WORK | F_OROWS>),
       "grouped_gemm_down"},
      {MODE_NARROW, F_WORK | F_OROWS,
       reinterpret_cast<const void*>(&grouped_gemm_kernel<MODE_NARROW, F_WORK | F_OROWS>), "grouped_gemm_down"},
      {MODE_WIDE, 0, reinterpret_cast<const void*>(&grouped_gemm_kernel<MODE_WIDE, 0>), "q4_matmul"},
      {MODE_NARROW, 0, reinterpret_cast<const void*>(&grouped_gemm_kernel<MODE_NARROW, 0>), "q4_matmul"},
  };
  int v = -1;
  for (int i = 0; i < static_cast<int>(sizeof(variants) / sizeof(variants[0])); ++i)
    if (variants[i].mode == mode && variants[i].flags == flags) v = i;
  if (v < 0) return obs::set_error(ctx, OBS_E_INVALID, "grouped GEMM: unsupported launch (mode %u, flags %u)", mode, flags);
  const void* fn = variants[v].fn;
  const char* name = variants[v].name;
  void* args[] = {&a};
  OBS_LAUNCH(ctx, name, OBS_HIP_TRY(ctx, hipLaunchKernel(fn, dim3(grid), dim3(256), args, lds, ctx->stream)));
  return OBS_OK;
}

// The expert FFN of a grouped prefill in one launch (moe_ffn_kernel): the
// gate/up items of g.work, then the down items of d.work, per XCD.
int launch_ffn(obs_ctx* ctx, GemmArgs g, GemmArgs d, int32_t* tile_done, uint32_t ncb_gu, uint32_t grid,
               uint32_t mode_dn) {
  if (mode_dn == MODE_WIDE) {
    d.w1 = d.w0 + static_cast<size_t>(TN) * (d.K / 8u);
    d.s1 = d.s0 + static_cast<size_t>(TN) * (d.K / GK);
    d.b1 = d.b0 + static_cast<size_t>(TN) * (d.K / GK);
  }
  const size_t lds = std::max(gemm_sb_bytes(MODE_SWIGLU, g.K), gemm_sb_bytes(mode_dn, d.K));
  const void* fn = mode_dn == MODE_WIDE ? reinterpret_cast<const void*>(&moe_ffn_kernel<MODE_WIDE>)
                                        : reinterpret_cast<const void*>(&moe_ffn_kernel<MODE_NARROW>);
  FfnSync sy{tile_done, static_cast<int32_t>(ncb_gu + ctx->ffn_extra_count), ctx->ffn_wait_ticks, ctx->status_dev};
  void* args[] = {&g, &d, &sy};
  OBS_LAUNCH(ctx, "moe_ffn", OBS_HIP_TRY(ctx, hipLaunchKernel(fn, dim3(grid), dim3(256), args, lds, ctx->stream)));
  return OBS_OK;
}

}  // namespace

namespace obs {

// The one-launch FFN's flags in the context's status words: reported (and
// cleared) like the fused decode's time-outs.
int ffn_status(obs_ctx* ctx) {
  uint32_t st[2] = {0, 0};
  OBS_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  OBS_HIP_TRY(ctx, hipMemcpy(st, ctx->status_dev, sizeof(st), hipMemcpyDeviceToHost));
  if (st[CTX_ST_FFN_WAIT] || st[CTX_ST_FFN_SCHED]) {
    OBS_HIP_TRY(ctx, hipMemset(ctx->status_dev, 0, sizeof(st)));
    OBS_HIP_TRY(ctx, hipDeviceSynchronize());
    if (st[CTX_ST_FFN_SCHED])
      return set_error(ctx, OBS_E_HIP, "grouped prefill: a one-launch work table did not fit its launch; outputs invalid");
    return set_error(ctx, OBS_E_HIP, "grouped prefill: a down item's wait for its tile timed out; its output is invalid");
  }
  return OBS_OK;
}

// The staged scales can take a grouped GEMM workgroup past 64 KB of LDS
// (gfx950 has 160 KB per CU): every variant's limit is raised once per
// context, at creation, so no launch sets a kernel attribute.
int prefill_init(obs_ctx* ctx) {
  const void* fns[] = {
      reinterpret_cast<const void*>(&grouped_gemm_kernel<MODE_SWIGLU, F_WORK | F_AROWS>),
      reinterpret_cast<const void*>(&grouped_gemm_kernel<MODE_WIDE, F_WORK | F_OROWS>),
      reinterpret_cast<const void*>(&grouped_gemm_kernel<MODE_NARROW, F_WORK | F_OROWS>),
      reinterpret_cast<const void*>(&grouped_gemm_kernel<MODE_WIDE, 0>),
      reinterpret_cast<const void*>(&grouped_gemm_kernel<MODE_NARROW, 0>),
      reinterpret_cast<const void*>(&moe_ffn_kernel<MODE_WIDE>),
      reinterpret_cast<const void*>(&moe_ffn_kernel<MODE_NARROW>)};
  for (const void* fn : fns)
    OBS_HIP_TRY(ctx, hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, SB_LDS_MAX));
  return OBS_OK;
}

}  // namespace obs

extern "C" {

size_t obs_moe_prefill_workspace(const obs_moe_config* cfg, uint32_t T) {
  if (!cfg || T == 0) return 0;
  // the larger of the two layouts (the work tables are sized by the schedule the device allows)
  return std::max(prefill_layout(cfg, T, false).total, prefill_layout(cfg, T, true).total);
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
  const PrefillWs L = prefill_layout(cfg, T, (obs::dispatch_gate(ctx->num_cus, ctx->xcd_map_ok, ctx->inorder_ok) &
                                               OBS_PATH_FFN_ONE_LAUNCH) != 0u);
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
    rc = obs::launch_route(ctx, layer->router_w, layer->router_s, layer->router_b, Xin,
                           reinterpret_cast<float*>(base + L.logits), d_ids, d_w, T, H, E, cfg->group, k,
                           cfg->norm_topk, cfg->route_rule);
    if (rc) return rc;
    ids = d_ids;
    weights = d_w;
  }
  int32_t* counts = reinterpret_cast<int32_t*>(base + L.counts);
  int32_t* offsets = reinterpret_cast<int32_t*>(base + L.offsets);
  int32_t* row_token = reinterpret_cast<int32_t*>(base + L.row_token);
  int32_t* row_slot = reinterpret_cast<int32_t*>(base + L.row_slot);
  int4* work_gu = reinterpret_cast<int4*>(base + L.work_gu);
  int4* work_dn = reinterpret_cast<int4*>(base + L.work_dn);
  uint16_t* Hbuf = reinterpret_cast<uint16_t*>(base + L.H);
  uint16_t* Yp = reinterpret_cast<uint16_t*>(base + L.Yp);
  int32_t* chunk_cnt = reinterpret_cast<int32_t*>(base + L.chunk_cnt);
  OBS_LAUNCH(ctx, "moe_group_count", group_count_kernel<<<L.nchunks, 64, 0, ctx->stream>>>(ids, T, k, E, chunk_cnt));
  OBS_LAUNCH(ctx, "moe_group_scan",
             group_scan_kernel<<<1, 256, 0, ctx->stream>>>(L.nchunks, E, chunk_cnt, counts, offsets));
  const uint32_t cols_dn = mode_cols(gemm_mode(false, H));
  int32_t* work_cnt = reinterpret_cast<int32_t*>(base + L.work_cnt);
  int32_t* tile_done = reinterpret_cast<int32_t*>(base + L.tile_done);
  const WorkTable wt_gu{work_gu, work_cnt, L.grid_gu, I / TN, TN, L.split_gu, nullptr, nullptr};
  const WorkTable wt_dn{work_dn, work_cnt + 8, L.grid_dn, H / cols_dn, cols_dn, L.split_dn,
                        L.ffn_one_launch ? tile_done : nullptr, ctx->status_dev};
  OBS_LAUNCH(ctx, "moe_group_rank",
             group_rank_kernel<<<L.nchunks + 2u, 64, 0, ctx->stream>>>(ids, T, k, E, chunk_cnt, row_token, row_slot,
                                                                       counts, offsets, wt_gu, wt_dn));
  GemmArgs g{};
  g.A = Xin; g.a_rows = row_token; g.a_rows_total = T;
  g.w0 = layer->gate_w; g.s0 = layer->gate_s; g.b0 = layer->gate_b;
  g.w1 = layer->up_w; g.s1 = layer->up_s; g.b1 = layer->up_b;
  g.out = Hbuf; g.out_rows = nullptr;
  g.work = work_gu; g.work_count = work_cnt;
  g.K = H; g.N = I;
  GemmArgs d{};
  d.A = Hbuf; d.a_rows = nullptr; d.a_rows_total = T * k;
  d.w0 = layer->down_w; d.s0 = layer->down_s; d.b0 = layer->down_b;
  d.out = Yp; d.out_rows = row_slot;
  d.work = work_dn; d.work_count = work_cnt + 8;
  d.K = I; d.N = H;
  if (L.ffn_one_launch) {
    rc = launch_ffn(ctx, g, d, tile_done, I / TN, L.grid_gu + L.grid_dn, gemm_mode(false, H));
    if (rc) return rc;
  } else {
    rc = launch_gemm(ctx, g, L.grid_gu, MODE_SWIGLU);
    if (rc) return rc;
    rc = launch_gemm(ctx, d, L.grid_dn, gemm_mode(false, H));
    if (rc) return rc;
  }
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
  // the wide mode (256 columns per item) unless that leaves CUs idle and the
  // 128-column mode would not
  const uint32_t tiles = T == 0 ? 1u : (T + TM - 1) / TM;
  uint32_t mode = gemm_mode(false, out);
  if (mode == MODE_WIDE && (tiles * (out / (2u * TN)) < static_cast<uint32_t>(ctx->num_cus) ||
                            gemm_sb_bytes(mode, in) > SB_LDS_MAX))
    mode = MODE_NARROW;
  if (gemm_sb_bytes(mode, in) > SB_LDS_MAX)
    return obs::set_error(ctx, OBS_E_SHAPE, "obs_q4_matmul: in must be at most %u (got %u)",
                          static_cast<uint32_t>(SB_LDS_MAX / (sizeof(uint32_t) * SB_STRIDE)) * GK, in);
  if (!obs::aligned(X, 16) || !obs::aligned(w, 16) || !obs::aligned(Y, 16))
    return obs::set_error(ctx, OBS_E_ALIGN, "obs_q4_matmul: X, w and Y must be 16-byte aligned");
  if (T == 0) return OBS_OK;
  const uint32_t grid = gemm_grid(tiles, out, mode);
  GemmArgs g{};
  g.A = X; g.a_rows = nullptr; g.a_rows_total = T;
  g.w0 = w; g.s0 = scales; g.b0 = biases;
  g.out = Y; g.out_rows = nullptr;
  g.work = nullptr; g.work_count = nullptr; g.dense_rows = T;
  g.K = in; g.N = out;
  return launch_gemm(ctx, g, grid, mode);
}

}  // extern "C"
