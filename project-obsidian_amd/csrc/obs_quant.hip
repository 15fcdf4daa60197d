// obs_quant.hip — MLX affine dequant and the standalone 4-bit mat-vec.
//
// Format (tools/split_experts.py:9-19, validate_dequant.py:26-29): element c of
// a row is the bits-wide field c % (32/bits) of uint32 word c / (32/bits), low
// bits first; w = q*scale + bias with bf16 scale/bias per `group` columns.
// q*scale is exact in fp32 (4/8-bit integer times an 8-bit-significand bf16),
// so fl32(q*scale + bias) has a single rounding and equals the fma form of
// fused_dequant_matvec_4bit.metal:45.
#include "obs_internal.hpp"

namespace {

using namespace obsd;

// One thread per packed word: dequantizes 32/bits elements.
template <int BITS>
__global__ void __launch_bounds__(256) dequant_kernel(const uint32_t* __restrict__ w,
                                                      const uint16_t* __restrict__ s,
                                                      const uint16_t* __restrict__ b,
                                                      float* __restrict__ out_f32,
                                                      uint16_t* __restrict__ out_bf16,
                                                      uint32_t rows, uint32_t cols, uint32_t group) {
  constexpr uint32_t PER = 32 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  const uint32_t words = cols / PER;
  const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<uint64_t>(rows) * words) return;
  const uint32_t r = static_cast<uint32_t>(idx / words), wi = static_cast<uint32_t>(idx % words);
  const uint32_t word = w[idx];
  const uint32_t c0 = wi * PER;
  const uint64_t gidx = static_cast<uint64_t>(r) * (cols / group) + c0 / group;  // PER | group
  const float sc = bf16_to_f32(s[gidx]), bi = bf16_to_f32(b[gidx]);
  float v[PER];
#pragma unroll
  for (uint32_t j = 0; j < PER; ++j) v[j] = __builtin_fmaf(static_cast<float>((word >> (BITS * j)) & MASK), sc, bi);
  const uint64_t o = static_cast<uint64_t>(r) * cols + c0;
  if (out_f32) {
#pragma unroll
    for (uint32_t j = 0; j < PER; j += 4)
      *reinterpret_cast<float4*>(out_f32 + o + j) = make_float4(v[j], v[j + 1], v[j + 2], v[j + 3]);
  }
  if (out_bf16) {
    if constexpr (PER == 8) {
      *reinterpret_cast<uint4*>(out_bf16 + o) =
          make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
    } else {
      *reinterpret_cast<uint2*>(out_bf16 + o) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    }
  }
}

// One wave per output row; lane l walks words l, l+64, ... (coalesced 4-byte
// loads); fp32 fma accumulation, xor-butterfly combine.
__global__ void __launch_bounds__(256) q4_matvec_kernel(const uint32_t* __restrict__ w,
                                                        const uint16_t* __restrict__ s,
                                                        const uint16_t* __restrict__ b,
                                                        const uint16_t* __restrict__ x,
                                                        float* __restrict__ y_f32,
                                                        uint16_t* __restrict__ y_bf16,
                                                        uint32_t in, uint32_t out, uint32_t group) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t row = blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
  if (row >= out) return;
  const uint32_t words = in / 8, groups = in / group;
  const uint32_t* wr = w + static_cast<uint64_t>(row) * words;
  const uint16_t* sr = s + static_cast<uint64_t>(row) * groups;
  const uint16_t* br = b + static_cast<uint64_t>(row) * groups;
  float acc = 0.0f;
  for (uint32_t wi = lane; wi < words; wi += 64) {
    const uint32_t word = wr[wi];
    const uint4 xv = *reinterpret_cast<const uint4*>(x + wi * 8);
    const uint32_t g = (wi * 8) / group;
    const float sc = bf16_to_f32(sr[g]), bi = bf16_to_f32(br[g]);
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float q = static_cast<float>((word >> (4 * j)) & 0xfu);
      const float xf = (j & 1) ? bf16hi(xw[j >> 1]) : bf16lo(xw[j >> 1]);
      acc = __builtin_fmaf(__builtin_fmaf(q, sc, bi), xf, acc);
    }
  }
  acc = wave_sum_asc(acc);
  if (lane == 0) {
    if (y_f32) y_f32[row] = acc;
    if (y_bf16) y_bf16[row] = f32_to_bf16(acc);
  }
}

}  // namespace

extern "C" {

int obs_dequant(obs_ctx* ctx, int bits, const uint32_t* w, const uint16_t* scales,
                const uint16_t* biases, float* out_f32, uint16_t* out_bf16,
                uint32_t rows, uint32_t cols, uint32_t group) {
  if (!ctx) return OBS_E_INVALID;
  if (bits != 4 && bits != 8) return obs::set_error(ctx, OBS_E_INVALID, "obs_dequant: bits must be 4 or 8 (got %d)", bits);
  if (!w || !scales || !biases || (!out_f32 && !out_bf16))
    return obs::set_error(ctx, OBS_E_INVALID, "obs_dequant: null pointer");
  const uint32_t per = 32u / static_cast<uint32_t>(bits);
  if (rows == 0 || cols == 0) return OBS_OK;
  if (group == 0 || cols % group != 0 || group % per != 0)
    return obs::set_error(ctx, OBS_E_SHAPE, "obs_dequant: cols (%u) must be a multiple of group (%u), group a multiple of %u", cols, group, per);
  if ((out_f32 && !obs::aligned(out_f32, 16)) || (out_bf16 && !obs::aligned(out_bf16, 16)) || !obs::aligned(w, 4))
    return obs::set_error(ctx, OBS_E_ALIGN, "obs_dequant: outputs must be 16-byte aligned");
  const uint64_t n = static_cast<uint64_t>(rows) * (cols / per);
  const uint32_t blocks = static_cast<uint32_t>((n + 255) / 256);
  if (bits == 4)
    OBS_LAUNCH(ctx, "dequant4", dequant_kernel<4><<<blocks, 256, 0, ctx->stream>>>(w, scales, biases, out_f32, out_bf16, rows, cols, group));
  else
    OBS_LAUNCH(ctx, "dequant8", dequant_kernel<8><<<blocks, 256, 0, ctx->stream>>>(w, scales, biases, out_f32, out_bf16, rows, cols, group));
  return OBS_OK;
}

int obs_q4_matvec(obs_ctx* ctx, const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                  const uint16_t* x, float* y_f32, uint16_t* y_bf16, uint32_t in, uint32_t out,
                  uint32_t group) {
  if (!ctx) return OBS_E_INVALID;
  if (!w || !scales || !biases || !x || (!y_f32 && !y_bf16))
    return obs::set_error(ctx, OBS_E_INVALID, "obs_q4_matvec: null pointer");
  if (out == 0) return OBS_OK;
  // the reference kernel silently drops tail columns when in % group != 0
  // (fused_dequant_matvec_4bit.metal:27,32); here it is an error.
  if (in == 0 || group == 0 || in % group != 0 || group % 8 != 0)
    return obs::set_error(ctx, OBS_E_SHAPE, "obs_q4_matvec: in (%u) must be a non-zero multiple of group (%u), group a multiple of 8", in, group);
  if (!obs::aligned(x, 16)) return obs::set_error(ctx, OBS_E_ALIGN, "obs_q4_matvec: x must be 16-byte aligned");
  const uint32_t blocks = (out + 3) / 4;
  OBS_LAUNCH(ctx, "q4_matvec", q4_matvec_kernel<<<blocks, 256, 0, ctx->stream>>>(w, scales, biases, x, y_f32, y_bf16, in, out, group));
  return OBS_OK;
}

}  // extern "C"
