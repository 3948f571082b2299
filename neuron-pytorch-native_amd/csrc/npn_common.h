// Shared device helpers and host-side argument checks for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "npn_spec_verify.h"

namespace npn {

constexpr int kWave = 64;  // CDNA wavefront width

// ---- bf16 bit conversions (storage is raw uint16 bits) -----------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// float -> bf16 bits, round to nearest even (NaN kept quiet). Both results are formed and one
// is selected (v_cndmask): an early return for NaN compiled to an exec-mask branch around
// every conversion of the GEMM epilogues.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rounded = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  const uint32_t quiet = (u >> 16) | 0x40u;
  return static_cast<uint16_t>(f != f ? quiet : rounded);
}

// Two bf16 packed in a uint32 (low half = first element).
__device__ __forceinline__ float bf16lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf16hi(uint32_t p) { return __uint_as_float(p & 0xFFFF0000u); }

__device__ __forceinline__ float silu(float x) { return x / (1.0f + __expf(-x)); }
// The same with the fast division (reciprocal and multiply, denominators past 2^96 scaled
// first; about 2 ulp in fp32 instead of a correctly rounded quotient), for the SwiGLU, whose
// callers round the result to bf16 at once. Every SwiGLU path (the GEMM epilogues, the split-K
// SwiGLU and glue::silu_mul) uses this one, so fused and unfused outputs stay bit-identical.
__device__ __forceinline__ float silu_bf16(float x) { return __fdividef(x, 1.0f + __expf(-x)); }
__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + __expf(-x)); }
__device__ __forceinline__ float softplus(float x) {
  // torch.nn.functional.softplus (beta=1, threshold=20)
  return x > 20.0f ? x : log1pf(__expf(x));
}

// ---- wave reductions (64 lanes) -----------------------------------------------------

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// ---- reductions inside 16-lane rows by DPP (VALU lane permutes, no LDS traffic) -----------
// quad_perm [1,0,3,2] and [2,3,0,1] combine lanes within each quad; row_half_mirror (lane i with
// 7 - i of its half-row) then row_mirror (i with 15 - i of its row) combine the quads and the
// halves. After n steps every lane holds the reduction over its aligned group of 2^n lanes
// (n = 2: quads, 3: eight lanes, 4: the 16-lane row). Every source lane of these patterns is
// inside the row, so the move needs no old value (bound_ctrl), which lets the compiler fold it
// into the operation that uses it.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}

constexpr int kDppStep[4] = {0xB1, 0x4E, 0x141, 0x140};

// Maximum of a non-NaN float over the aligned group of 2^STEPS lanes. The reduction runs on an
// order-preserving integer key (bits, with the magnitude bits flipped for negatives; -0 sorts
// below +0), as v_max_i32 with the DPP move folded in.
template <int STEPS>
__device__ __forceinline__ float row_max_dpp(float v) {
  const uint32_t u = __float_as_uint(v);
  int k = (int)(u ^ ((uint32_t)((int)u >> 31) & 0x7FFFFFFFu));
  if constexpr (STEPS >= 1) k = max(k, (int)dpp32<kDppStep[0]>((uint32_t)k));
  if constexpr (STEPS >= 2) k = max(k, (int)dpp32<kDppStep[1]>((uint32_t)k));
  if constexpr (STEPS >= 3) k = max(k, (int)dpp32<kDppStep[2]>((uint32_t)k));
  if constexpr (STEPS >= 4) k = max(k, (int)dpp32<kDppStep[3]>((uint32_t)k));
  return __uint_as_float((uint32_t)k ^ ((uint32_t)(k >> 31) & 0x7FFFFFFFu));
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp64(uint64_t v) {
  return ((uint64_t)dpp32<CTRL>((uint32_t)(v >> 32)) << 32) | dpp32<CTRL>((uint32_t)v);
}

template <int STEPS>
__device__ __forceinline__ uint64_t row_sum_dpp(uint64_t v) {
  if constexpr (STEPS >= 1) v += dpp64<kDppStep[0]>(v);
  if constexpr (STEPS >= 2) v += dpp64<kDppStep[1]>(v);
  if constexpr (STEPS >= 3) v += dpp64<kDppStep[2]>(v);
  if constexpr (STEPS >= 4) v += dpp64<kDppStep[3]>(v);
  return v;
}

// ---- LDS DMA -----------------------------------------------------------------------------
// 16 bytes per lane from global address g into LDS at lds_base + 16 * lane
// (global_load_lds_dwordx4; lds_base must be the same for the whole wave). Issued through
// inline asm so the compiler does not add a conservative vmcnt(0) wait before later LDS
// reads of other buffers: callers track completion themselves with s_waitcnt vmcnt(n)
// and make it visible to the other waves with s_barrier.
// The DMA takes its LDS base from m0, a register the compiler reserves (it does not honour
// m0 in a clobber list). The statement therefore leaves m0 as it found it: it copies m0 to a
// scratch SGPR, sets the base, and restores m0 after the issue (the instruction reads m0
// when it issues). GFX9 needs one wait state between an SALU write of m0 and an LDS DMA
// that reads it, hence the s_nop.
__device__ __forceinline__ void lds_dma16(const void* g, const void* lds_base) {
  const unsigned base = __builtin_amdgcn_readfirstlane(
      (unsigned)(uintptr_t)(__attribute__((address_space(3))) const void*)lds_base);
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(base)
      : "memory");
}

// Same DMA with a wave-uniform global base (SGPR pair), a 32-bit per-lane byte offset (one
// VGPR per lane live instead of a 64-bit address) and the LDS base as a wave-uniform LDS
// address (no generic-to-LDS pointer conversion, whose null check costs four scalar
// instructions per DMA).
__device__ __forceinline__ void lds_dma16_soff(const void* sbase, unsigned voff,
                                               unsigned lds_addr) {
  const unsigned base = __builtin_amdgcn_readfirstlane(lds_addr);
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(sbase), "s"(base)
      : "memory");
}

// LDS address of a pointer into __shared__ memory.
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return (unsigned)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

__device__ __forceinline__ void lds_dma16_soff(const void* sbase, unsigned voff,
                                               const void* lds_base) {
  const unsigned base = __builtin_amdgcn_readfirstlane(lds_addr(lds_base));
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(sbase), "s"(base)
      : "memory");
}

}  // namespace npn

// ---- host-side checks ------------------------------------------------------------------

#define NPN_REQUIRE(cond, code) \
  do {                          \
    if (!(cond)) return (code); \
  } while (0)

#define NPN_ALIGNED16(p) ((reinterpret_cast<uintptr_t>(p) & 15u) == 0)

static inline int npn_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? NPN_OK : NPN_ERR_LAUNCH;
}
