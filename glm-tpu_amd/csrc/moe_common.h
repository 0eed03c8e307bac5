// Shared device helpers of the routed-expert MoE library (gfx950 / CDNA4).
//
// Numerics follow glm-tpu's FP8 block decode: an e4m3fn byte is decoded
// exactly to FP32, multiplied by its FP32 128x128 block scale in FP32 and
// rounded once (RNE) to bf16 (reference glm_tpu/layers/fp8.py:113-126).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace glm_moe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kScaleBlock = 128;  // checkpoint scale block along N and K
constexpr int kWave = 64;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// RNE float -> bf16 bits (v_cvt_pk_bf16_f32 on gfx950; NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  __bf16 h = (__bf16)f;
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float round_to_bf16(float f) {
  return bf16_bits_to_f32(f32_to_bf16_bits(f));
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
}

// Eight e4m3fn bytes (two little-endian dwords, byte 0 = lowest K) decoded to
// eight bf16 MFMA operand values: bf16(f32(e4m3(b)) * scale).
__device__ __forceinline__ bf16x8 decode_fp8x8(uint32_t lo, uint32_t hi, float scale) {
  const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);
  const f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
  const f32x2 c = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
  const f32x2 d = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
  bf16x8 r;
  r[0] = (__bf16)(a[0] * scale);
  r[1] = (__bf16)(a[1] * scale);
  r[2] = (__bf16)(b[0] * scale);
  r[3] = (__bf16)(b[1] * scale);
  r[4] = (__bf16)(c[0] * scale);
  r[5] = (__bf16)(c[1] * scale);
  r[6] = (__bf16)(d[0] * scale);
  r[7] = (__bf16)(d[1] * scale);
  return r;
}

// Eight bf16 values held as four dwords reinterpreted as an MFMA operand.
__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) {
  return __builtin_bit_cast(bf16x8, v);
}

// FP32 logistic 1 / (1 + exp(-x)).
__device__ __forceinline__ float sigmoid_f32(float x) {
  return 1.0f / (1.0f + expf(-x));
}

// bf16(bf16(g * bf16(sigmoid(g))) * u) with g, u already bf16 values: the
// SwiGLU of the reference with one bf16 rounding per elementwise op
// (glm_tpu/layers/moe/routed_experts.py:102,280).  The sigmoid is
// 1 / (1 + 2^(-g log2 e)) from the hardware exp2, its quotient a reciprocal
// refined by one Newton step, except where 1 + exp(-g) >= 2^126, whose
// quotient is an FP32 subnormal that the reciprocal would flush: there
// 1 / (1 + expf(-g)) with the IEEE division.  bf16(sigmoid(g)) so computed
// equals sigmoid_f32's for every bf16 g (all 65,536 checked on the GPU), and
// bf16(g * s) is all of the sigmoid that the later rounding sees.
__device__ __forceinline__ float swiglu_bf16(float g, float u) {
  const float y = 1.0f + __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
  float q;
  if (__builtin_expect(y < 0x1p126f, 1)) {
    const float r = __builtin_amdgcn_rcpf(y);
    q = __builtin_fmaf(__builtin_fmaf(-y, r, 1.0f), r, r);
  } else {
    q = sigmoid_f32(g);
  }
  const float s = round_to_bf16(q);
  return round_to_bf16(round_to_bf16(g * s) * u);
}

// max(v, v of the lane that DPP control CTRL names).  fmaxf ignores a NaN
// operand, so a maximum built from these does not depend on the pairing order.
template <int CTRL>
__device__ __forceinline__ float max_dpp(float v) {
  return fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF,
                                                                        0xF, false)));
}

// Maximum over each 16-lane row of the wave (every lane of the row gets it):
// quad lanes xor 1 and xor 2, then the half-row and row mirrors.
__device__ __forceinline__ float row16_max_f32(float v) {
  v = max_dpp<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v = max_dpp<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v = max_dpp<0x141>(v);  // row_half_mirror
  return max_dpp<0x140>(v);  // row_mirror
}

// Activation quantisation of the native FP8 mode for one 128-value block held
// by the 16 lanes of a 16-lane row, 8 values a lane: scale = amax / 448 (1 for
// an all-zero block), q = e4m3fn(clamp(v / scale, +-448)) rounded to nearest
// even (v_cvt_pk_fp8_f32), NaN stays NaN.  Returns the block's scale; the
// lane's codes of values 0..3 in lo and 4..7 in hi (byte j = value j).
__device__ __forceinline__ float quantize_block16_fp8(const float (&f)[8], uint32_t& lo, uint32_t& hi) {
  float a = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) a = fmaxf(a, fabsf(f[j]));
  const float m = row16_max_f32(a);
  const float scale = m > 0.0f ? m / 448.0f : 1.0f;
  auto clamp448 = [](float t) { return t != t ? t : fminf(fmaxf(t, -448.0f), 448.0f); };
  uint32_t w0 = 0, w1 = 0;
  w0 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(clamp448(f[0] / scale), clamp448(f[1] / scale), (int)w0, false);
  w0 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(clamp448(f[2] / scale), clamp448(f[3] / scale), (int)w0, true);
  w1 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(clamp448(f[4] / scale), clamp448(f[5] / scale), (int)w1, false);
  w1 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(clamp448(f[6] / scale), clamp448(f[7] / scale), (int)w1, true);
  lo = w0;
  hi = w1;
  return scale;
}

}  // namespace glm_moe
