// The integer softmax contract of rejection-sampling acceptance, shared by the acceptance
// kernels and the LM-head GEMM epilogue that produces the target rows' chunk statistics.
//
//   s_v = t_v * inv_temp (fp32); the vocabulary is cut into chunks of kContractChunk = 64
//   entries and blocks of kContractBlock = 8192; m_c = max of chunk c's non-NaN s_v;
//   E_v = floor(2^31 * exp_c(s_v - m_c)); S_c = sum of the chunk's E_v (< 2^37); chunk and
//   block factors F_c = floor(2^31 * exp_c(m_c - M_b)) and G_b = floor(2^31 * exp_c(M_b - M))
//   refer chunks to their block's maximum and blocks to the row's. exp_c is a Cody-Waite
//   reduction + degree-7 Taylor polynomial written as explicit fp32 fused multiply-adds;
//   every other operation here is a single IEEE-754 operation, never contracted into a fused
//   multiply-add, so this code and its CPU restatement round identically. Each function below disables contraction for its
//   own body, and every multiply whose result feeds an add or subtract of the contract
//   happens inside one of them.
#pragma once

#include "npn_common.h"

namespace npn {

constexpr int kContractChunk = 64;     // vocabulary entries per chunk of the contract
constexpr int kContractBlock = 8192;   // vocabulary entries per block (128 chunks)

constexpr float kL2E = 0x1.715476p+0f;        // log2(e) in fp32
constexpr float kLn2Hi = 0x1.62ep-1f;         // ln2, low 12 mantissa bits cleared
constexpr float kLn2Lo = 0x1.0bfbe8p-15f;     // ln2 - kLn2Hi in fp32
constexpr float kMagic = 0x1.8p+23f;          // 1.5 * 2^23: fma(x, kL2E, kMagic) rounds to an integer
// Taylor coefficients 1/k! in fp32, scaled by 2^31 (exact), k = 7..0
constexpr float kP7 = 0x1.a01a02p+18f;
constexpr float kP6 = 0x1.6c16c2p+21f;
constexpr float kP5 = 0x1.111112p+24f;
constexpr float kP4 = 0x1.555556p+26f;
constexpr float kP3 = 0x1.555556p+28f;
constexpr float kP2 = 0x1p+30f;
constexpr float kP1 = 0x1p+31f;               // 2^31 / 1! and 2^31 / 0!
constexpr float kXMin = -32.0f;               // at and below: 2^31 exp(x) < 1

// E = floor(2^31 * exp_c(x)) for x <= 0 (NaN and x <= -32 give 0; E(0) = 2^31).
// kf = t - kMagic is round(x * log2 e) as an exact fp32 integer, and t's bit pattern holds
// kf in its low bits, so adding (bits(t) << 23) to p's pattern multiplies p by 2^kf exactly
// (the exponent stays in the normal range: p >= 2^30 and kf >= -47). The conversion to
// uint32 truncates, which is the floor of a value in [0, 2^31].
__device__ __forceinline__ uint32_t expfix(float x) {
#pragma clang fp contract(off)
  x = fmaxf(x, kXMin);
  const float t = __builtin_fmaf(x, kL2E, kMagic);
  const float kf = t - kMagic;
  float r = __builtin_fmaf(-kf, kLn2Hi, x);
  r = __builtin_fmaf(-kf, kLn2Lo, r);
  float p = __builtin_fmaf(kP7, r, kP6);
  p = __builtin_fmaf(p, r, kP5);
  p = __builtin_fmaf(p, r, kP4);
  p = __builtin_fmaf(p, r, kP3);
  p = __builtin_fmaf(p, r, kP2);
  p = __builtin_fmaf(p, r, kP1);
  p = __builtin_fmaf(p, r, kP1);
  return (uint32_t)__uint_as_float(__float_as_uint(p) + (__float_as_uint(t) << 23));
}

// E of a scaled logit s relative to a maximum m: expfix(s - m), the subtraction unfused.
__device__ __forceinline__ uint32_t expfix_rel(float s, float m) {
#pragma clang fp contract(off)
  return expfix(s - m);
}

// s = t * inv_temp, one fp32 multiply (t itself when inv_temp is 1: x * 1 == x, NaN stays NaN).
__device__ __forceinline__ float scaled(float v, float inv_temp) {
#pragma clang fp contract(off)
  return v * inv_temp;
}

// U = floor(u * 2^24) for a uniform u in [0, 1).
__device__ __forceinline__ uint32_t uniform_fix(float u) {
#pragma clang fp contract(off)
  return (uint32_t)(u * 16777216.0f);
}

}  // namespace npn
