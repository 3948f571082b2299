// Speculative-decode acceptance on gfx950: greedy and rejection sampling.
//
// Greedy (the reference's on-device argmax, contrib/qwen3.6-27b/static_decode.py:1313, with
// the exact sharded top-1 order of contrib/qwen3.6-35b-a3b/static_decode_35b.py:1532-1570):
//   tid[b,t] = argmax_v target[b,t,v], first index on ties, NaN counts as the maximum;
//   accepted a_b = number of leading drafts equal to tid[b, position before them].
//
// Rejection sampling (Leviathan et al. 2023, Alg. 1) under an integer softmax contract
// that this file and its CPU restatement evaluate with identical IEEE-754 operations:
//   s_v = t_v * inv_temp (fp32); m = max_v s_v; E_v = floor(2^31 * exp_c(s_v - m)) where
//   exp_c is a Cody-Waite reduction + degree-7 Taylor polynomial evaluated with explicit
//   fp32 fused multiply-adds (this file is compiled with -ffp-contract=off, so no other
//   multiply and add is fused);
//   Z = sum_v E_v in 64-bit integers (exact, so the reduction order does not matter).
//   Accept draft x at position i iff U * Eq_x * Zp <= 2^24 * Ep_x * Zq (128-bit integers,
//   U = floor(u * 2^24)). At the first rejection sample from R_v = max(0, Ep_v Zq - Eq_v Zp),
//   after K acceptances from R_v = Ep_v of the bonus row: the token is the smallest v with
//   2^24 * sum_{w<=v} R_w > U_s * sum_w R_w.
//
// Kernels (each over B sequences, T = K+1 positions, vocabulary split into 8192-wide chunks):
//   greedy:    argmax partials per (row, chunk) -> per-sequence merge + accept
//   rejection: one pass per (row, chunk): the chunk maximum, the sum of E and E at the draft
//              token -> per-sequence row totals and decision -> residual/bonus mass per
//              (sequence, chunk) -> per-sequence inverse-CDF pick
#include "npn_common.h"

#include <mutex>

namespace {

constexpr int CHK = 8192;      // vocabulary entries per chunk (logit passes)
constexpr int THREADS = 256;   // CHK / THREADS = 32 entries per thread
constexpr int PER_T = CHK / THREADS;
constexpr int MCHK = 2048;     // entries per chunk of the residual mass / inverse-CDF pass
constexpr int PER_M = MCHK / THREADS;  // 8 consecutive entries per thread
constexpr int kRejMaxV = 1 << 20;  // largest vocabulary of the rejection path

typedef unsigned __int128 u128;

// ---- exp contract (must match oracle.accept.expfix bit for bit) -------------------------
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

__device__ __forceinline__ float scaled(float v, float inv_temp) {
#pragma clang fp contract(off)
  return v * inv_temp;
}

__device__ __forceinline__ uint32_t uniform_fix(float u) {
#pragma clang fp contract(off)
  return (uint32_t)(u * 16777216.0f);
}

// ---- block reductions ----------------------------------------------------------------------
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor((uint32_t)v, m, 64);
  const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), m, 64);
  return ((uint64_t)hi << 32) | lo;
}

__device__ uint64_t block_sum_u64(uint64_t v, uint64_t* sh) {
  for (int off = 32; off > 0; off >>= 1) v += shfl_xor_u64(v, off);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) sh[w] = v;
  __syncthreads();
  uint64_t s = 0;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) s += sh[i];
  __syncthreads();
  return s;
}

__device__ u128 block_sum_u128(u128 v, u128* sh) {
  for (int off = 32; off > 0; off >>= 1) {
    const uint64_t lo = shfl_xor_u64((uint64_t)v, off);
    const uint64_t hi = shfl_xor_u64((uint64_t)(v >> 64), off);
    v += ((u128)hi << 64) | lo;
  }
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) sh[w] = v;
  __syncthreads();
  u128 s = 0;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) s += sh[i];
  __syncthreads();
  return s;
}

__device__ float block_max(float v, float* sh) {
  v = npn::wave_max(v);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) sh[w] = v;
  __syncthreads();
  float m = sh[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i) m = fmaxf(m, sh[i]);
  __syncthreads();
  return m;
}

// ---- chunk visitor -----------------------------------------------------------------------
// Calls f(v, x) for this thread's share of entries [v0, v0 + CHK) of a row (x = src[v]).
// With vec4 (row 16-byte aligned, V % 4 == 0) the thread reads PER_T/4 float4s at
// v0 + 4 * (j * THREADS + tid), else PER_T floats at v0 + j * THREADS + tid. Every caller
// combines the visited values with an order-independent operation (max, exact integer
// sums, or the total order of the argmax), so the assignment does not affect results.
template <typename F>
__device__ __forceinline__ void visit_chunk(const float* src, int v0, int V, bool vec4, F f) {
  if (vec4 && v0 + CHK <= V) {  // whole chunk in the row: all loads first, no guards
    float4 x[PER_T / 4];
#pragma unroll
    for (int j = 0; j < PER_T / 4; ++j)
      x[j] = *reinterpret_cast<const float4*>(src + v0 + 4 * (j * THREADS + (int)threadIdx.x));
#pragma unroll
    for (int j = 0; j < PER_T / 4; ++j) {
      const int v = v0 + 4 * (j * THREADS + (int)threadIdx.x);
      f(v, x[j].x);
      f(v + 1, x[j].y);
      f(v + 2, x[j].z);
      f(v + 3, x[j].w);
    }
  } else if (vec4) {
#pragma unroll
    for (int j = 0; j < PER_T / 4; ++j) {
      const int v = v0 + 4 * (j * THREADS + (int)threadIdx.x);
      if (v < V) {
        const float4 x = *reinterpret_cast<const float4*>(src + v);
        f(v, x.x);
        f(v + 1, x.y);
        f(v + 2, x.z);
        f(v + 3, x.w);
      }
    }
  } else {
    for (int j = 0; j < PER_T; ++j) {
      const int v = v0 + j * THREADS + (int)threadIdx.x;
      if (v < V) f(v, src[v]);
    }
  }
}

// The same over a bf16 row (the LM head's logits): with vec (row 16-byte aligned, V % 8 == 0)
// the thread reads PER_T/8 16-byte pieces of 8 entries at v0 + 8 * (j * THREADS + tid).
template <typename F>
__device__ __forceinline__ void visit_chunk(const uint16_t* src, int v0, int V, bool vec, F f) {
  auto unpack = [&](int v, uint4 x) {
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      f(v + 2 * k, npn::bf16_to_f32(w[k] & 0xFFFFu));
      f(v + 2 * k + 1, npn::bf16_to_f32(w[k] >> 16));
    }
  };
  if (vec && v0 + CHK <= V) {
    uint4 x[PER_T / 8];
#pragma unroll
    for (int j = 0; j < PER_T / 8; ++j)
      x[j] = *reinterpret_cast<const uint4*>(src + v0 + 8 * (j * THREADS + (int)threadIdx.x));
#pragma unroll
    for (int j = 0; j < PER_T / 8; ++j) unpack(v0 + 8 * (j * THREADS + (int)threadIdx.x), x[j]);
  } else if (vec) {
#pragma unroll
    for (int j = 0; j < PER_T / 8; ++j) {
      const int v = v0 + 8 * (j * THREADS + (int)threadIdx.x);
      if (v < V) unpack(v, *reinterpret_cast<const uint4*>(src + v));
    }
  } else {
    for (int j = 0; j < PER_T; ++j) {
      const int v = v0 + j * THREADS + (int)threadIdx.x;
      if (v < V) f(v, npn::bf16_to_f32(src[v]));
    }
  }
}

__device__ __forceinline__ float elem(const float* p, int v) { return p[v]; }
__device__ __forceinline__ float elem(const uint16_t* p, int v) { return npn::bf16_to_f32(p[v]); }

// ---- greedy ------------------------------------------------------------------------------
// (val, idx) order: NaN above every number (first NaN wins), then larger value, then
// smaller index. A total order, so any merge order gives the same winner.
__device__ __forceinline__ bool beats(float bv, int bi, float av, int ai) {
  const bool an = isnan(av), bn = isnan(bv);
  if (an || bn) return bn && (!an || bi < ai);
  return bv > av || (bv == av && bi < ai);
}

struct ArgPart {
  float v;
  int i;
};

__global__ __launch_bounds__(THREADS) void argmax_chunk_kernel(const float* __restrict__ logits,
                                                                ArgPart* __restrict__ part,
                                                                int V, int nch, bool vec4) {
  const int row = blockIdx.y, c = blockIdx.x;
  const float* src = logits + (size_t)row * V;
  const int v0 = c * CHK;
  float bv = -INFINITY;
  int bi = 0x7FFFFFFF;
  visit_chunk(src, v0, V, vec4, [&](int v, float x) {
    if (beats(x, v, bv, bi)) { bv = x; bi = v; }
  });
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (beats(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  __shared__ ArgPart sh[THREADS / 64];
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) sh[w] = ArgPart{bv, bi};
  __syncthreads();
  if (threadIdx.x == 0) {
    ArgPart best = sh[0];
    for (int k = 1; k < THREADS / 64; ++k)
      if (beats(sh[k].v, sh[k].i, best.v, best.i)) best = sh[k];
    part[(size_t)row * nch + c] = best;
  }
}

__global__ void greedy_accept_kernel(const ArgPart* __restrict__ part,
                                     const int64_t* __restrict__ draft_ids,
                                     int32_t* __restrict__ accepted, int64_t* __restrict__ out_ids,
                                     int B, int K, int nch) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const int T = K + 1;
  int a = K;
  bool stopped = false;
  for (int t = 0; t < T; ++t) {
    ArgPart best = part[((size_t)b * T + t) * nch];
    for (int c = 1; c < nch; ++c) {
      const ArgPart p = part[((size_t)b * T + t) * nch + c];
      if (beats(p.v, p.i, best.v, best.i)) best = p;
    }
    if (!stopped) out_ids[(size_t)b * T + t] = best.i;
    else out_ids[(size_t)b * T + t] = -1;
    if (!stopped && t < K && draft_ids[(size_t)b * K + t] != (int64_t)best.i) {
      a = t;
      stopped = true;
    }
  }
  accepted[b] = a;
}

// Best of one row's nparts partials, in every lane of the calling wave: lanes take the
// partials lane, lane + 64, ... (each lane keeps its first best), then a shuffle tree. The
// rule (NaN max, lower index on ties) is order-independent, so this equals a serial scan.
__device__ __forceinline__ ArgPart wave_best(const ArgPart* __restrict__ row, int nparts) {
  const int lane = threadIdx.x & 63;
  float bv = -INFINITY;
  int bi = 0x7FFFFFFF;
  for (int c = lane; c < nparts; c += 64) {
    const ArgPart p = row[c];
    if (beats(p.v, p.i, bv, bi)) { bv = p.v; bi = p.i; }
  }
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (beats(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  return ArgPart{bv, bi};
}

// Row argmax from per-row partials [M][nparts]: one wave per row.
__global__ __launch_bounds__(256) void argmax_parts_kernel(const ArgPart* __restrict__ part,
                                                           int nparts, int64_t* __restrict__ ids,
                                                           float* __restrict__ values, int M) {
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= M) return;
  const ArgPart best = wave_best(part + (size_t)m * nparts, nparts);
  if ((threadIdx.x & 63) == 0) {
    ids[m] = best.i;
    if (values != nullptr) values[m] = best.v;
  }
}

// Greedy acceptance from per-row partials: one workgroup per sequence, wave t reduces row
// (b, t); then one lane applies the acceptance rule of greedy_accept_kernel.
__global__ __launch_bounds__(1024) void greedy_accept_parts_kernel(
    const ArgPart* __restrict__ part, int nparts, const int64_t* __restrict__ draft_ids,
    int32_t* __restrict__ accepted, int64_t* __restrict__ out_ids, int K) {
  const int b = blockIdx.x, T = K + 1;
  const int w = threadIdx.x >> 6;
  __shared__ int best_id[16];
  const ArgPart best = wave_best(part + ((size_t)b * T + w) * nparts, nparts);
  if ((threadIdx.x & 63) == 0) best_id[w] = best.i;
  __syncthreads();
  if (threadIdx.x != 0) return;
  int a = K;
  bool stopped = false;
  for (int t = 0; t < T; ++t) {
    out_ids[(size_t)b * T + t] = stopped ? -1 : best_id[t];
    if (!stopped && t < K && draft_ids[(size_t)b * K + t] != (int64_t)best_id[t]) {
      a = t;
      stopped = true;
    }
  }
  accepted[b] = a;
}

// ---- rejection sampling ------------------------------------------------------------------
// 192-bit unsigned integers (three 64-bit limbs, little end first) for the exact products of
// the contract: W (< 2^63) times Z (< 2^80), times a 24-bit uniform or shift.
struct u192 {
  uint64_t w0, w1, w2;
};

__device__ __forceinline__ u192 u192_from(u128 x) { return u192{(uint64_t)x, (uint64_t)(x >> 64), 0}; }

__device__ __forceinline__ u192 add192(u192 a, u192 b) {
  const u128 s0 = (u128)a.w0 + b.w0;
  const u128 s1 = (u128)a.w1 + b.w1 + (uint64_t)(s0 >> 64);
  return u192{(uint64_t)s0, (uint64_t)s1, a.w2 + b.w2 + (uint64_t)(s1 >> 64)};
}

__device__ __forceinline__ u192 sub192(u192 a, u192 b) {  // a >= b
  const uint64_t b0 = a.w0 < b.w0;
  const u128 d1 = (u128)a.w1 - b.w1 - b0;
  const uint64_t b1 = (uint64_t)(d1 >> 64) != 0;  // borrow out of limb 1
  return u192{a.w0 - b.w0, (uint64_t)d1, a.w2 - b.w2 - b1};
}

__device__ __forceinline__ bool gt192(u192 a, u192 b) {
  if (a.w2 != b.w2) return a.w2 > b.w2;
  if (a.w1 != b.w1) return a.w1 > b.w1;
  return a.w0 > b.w0;
}

__device__ __forceinline__ bool is_zero192(u192 a) { return (a.w0 | a.w1 | a.w2) == 0; }

// x * y for x < 2^64 and y < 2^128, exact (< 2^192).
__device__ __forceinline__ u192 mul64x128(uint64_t x, u128 y) {
  const u128 lo = (u128)x * (uint64_t)y;
  const u128 hi = (u128)x * (uint64_t)(y >> 64);
  const u128 mid = (lo >> 64) + (uint64_t)hi;
  return u192{(uint64_t)lo, (uint64_t)mid, (uint64_t)(hi >> 64) + (uint64_t)(mid >> 64)};
}

// x * m for x < 2^128 and m < 2^32, exact (< 2^160).
__device__ __forceinline__ u192 mul128x32(u128 x, uint32_t m) {
  const u128 p0 = (u128)(uint64_t)x * m;
  const u128 p1 = (u128)(uint64_t)(x >> 64) * m + (uint64_t)(p0 >> 64);
  return u192{(uint64_t)p0, (uint64_t)p1, (uint64_t)(p1 >> 64)};
}

// a * m for m < 2^32 (exact while the product stays below 2^192).
__device__ __forceinline__ u192 mul192x32(u192 a, uint32_t m) {
  const u128 p0 = (u128)a.w0 * m;
  const u128 p1 = (u128)a.w1 * m + (uint64_t)(p0 >> 64);
  return u192{(uint64_t)p0, (uint64_t)p1, a.w2 * m + (uint64_t)(p1 >> 64)};
}

__device__ __forceinline__ u192 shl24_192(u192 a) {
  return u192{a.w0 << 24, (a.w1 << 24) | (a.w0 >> 40), (a.w2 << 24) | (a.w1 >> 40)};
}

struct RejArgs {
  const void* target;    // [B][K+1][V] fp32, or bf16 (the LM head's logits)
  const float* draft;    // [B][K][V]
  const int64_t* draft_ids;
  const float* u_accept;
  const float* u_sample;
  float inv_temp;
  int32_t* accepted;
  int64_t* out_ids;
  int B, K, V, nch, nchm;  // chunks of CHK (logit pass) and of MCHK (mass / pick)
  bool vec4;          // logit rows 16-byte aligned and V % 4 == 0 (V % 8 for bf16 rows)
  // workspace (rows = B*(K+1) target rows, then B*K draft rows)
  u128* zrow;         // [rows]        Z of each row
  float* mrow;        // [rows]        row maximum M (scaled logits)
  uint32_t* ex;       // [rows]        E at the row's draft token (target/draft rows i < K)
  float* rmax;        // [rows][nch]   chunk maxima m_c
  uint64_t* rsum;     // [rows][nch]   chunk sums S_c
  int32_t* dec_row;   // [B]           sampling position (target row; draft row or none)
  u128* dec_z;        // [B][2]        Zp, Zq of the sampling rows
  float* dec_m;       // [B][2]        row maxima of the sampling rows
  u192* cmass;        // [B][nchm]
};

template <typename TT>
__device__ __forceinline__ const TT* target_row(const RejArgs& a, int row) {
  return static_cast<const TT*>(a.target) + (size_t)row * a.V;
}

// Whether a draft id names a vocabulary entry. Ids outside [0, V) are never accepted: the
// position is a rejection whatever the uniform (greedy rejects them too, an argmax being in
// range), so no emitted id lies outside the vocabulary.
__device__ __forceinline__ bool draft_id_ok(int64_t x, int V) { return x >= 0 && x < V; }

// Draft token whose E this row reports, or -1 (bonus rows, and out-of-range draft ids).
__device__ __forceinline__ int row_token(const RejArgs& a, int row) {
  const int nt = a.B * (a.K + 1);
  int b, i;
  if (row < nt) {
    b = row / (a.K + 1);
    i = row - b * (a.K + 1);
    if (i == a.K) return -1;
  } else {
    b = (row - nt) / a.K;
    i = (row - nt) - b * a.K;
  }
  const int64_t x = a.draft_ids[(size_t)b * a.K + i];
  return draft_id_ok(x, a.V) ? (int)x : -1;
}

// This thread's entries of chunk [v0, v0 + CHK) of a row, in registers, scaled (NaN for
// entries past V: the maximum ignores them and they get E = 0). Same entry assignment as
// visit_chunk; the sums are exact, so the assignment does not affect results.
template <bool kUnitTemp>
__device__ __forceinline__ void load_chunk(const float* src, int v0, int V, bool vec4,
                                           float inv_temp, float (&x)[PER_T]) {
  if (vec4 && v0 + CHK <= V) {
#pragma unroll
    for (int j = 0; j < PER_T / 4; ++j) {
      const float4 f =
          *reinterpret_cast<const float4*>(src + v0 + 4 * (j * THREADS + (int)threadIdx.x));
      x[4 * j] = f.x; x[4 * j + 1] = f.y; x[4 * j + 2] = f.z; x[4 * j + 3] = f.w;
    }
  } else if (vec4) {
#pragma unroll
    for (int j = 0; j < PER_T / 4; ++j) {
      const int v = v0 + 4 * (j * THREADS + (int)threadIdx.x);
      float4 f = make_float4(NAN, NAN, NAN, NAN);
      if (v < V) f = *reinterpret_cast<const float4*>(src + v);
      x[4 * j] = f.x; x[4 * j + 1] = f.y; x[4 * j + 2] = f.z; x[4 * j + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < PER_T; ++j) {
      const int v = v0 + j * THREADS + (int)threadIdx.x;
      x[j] = v < V ? src[v] : NAN;
    }
  }
  if (!kUnitTemp) {
#pragma unroll
    for (int j = 0; j < PER_T; ++j) x[j] = scaled(x[j], inv_temp);
  }
}

template <bool kUnitTemp>
__device__ __forceinline__ void load_chunk(const uint16_t* src, int v0, int V, bool vec,
                                           float inv_temp, float (&x)[PER_T]) {
  if (vec) {
#pragma unroll
    for (int j = 0; j < PER_T / 8; ++j) {
      const int v = v0 + 8 * (j * THREADS + (int)threadIdx.x);
      uint4 q = make_uint4(0x7FC07FC0u, 0x7FC07FC0u, 0x7FC07FC0u, 0x7FC07FC0u);  // bf16 NaNs
      if (v < V) q = *reinterpret_cast<const uint4*>(src + v);
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        x[8 * j + 2 * k] = npn::bf16_to_f32(w[k] & 0xFFFFu);
        x[8 * j + 2 * k + 1] = npn::bf16_to_f32(w[k] >> 16);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < PER_T; ++j) {
      const int v = v0 + j * THREADS + (int)threadIdx.x;
      x[j] = v < V ? npn::bf16_to_f32(src[v]) : NAN;
    }
  }
  if (!kUnitTemp) {
#pragma unroll
    for (int j = 0; j < PER_T; ++j) x[j] = scaled(x[j], inv_temp);
  }
}

// The one logit pass: chunk c of a row, read once into registers; its maximum m_c, then
// S_c = sum of E_v = expfix(s_v - m_c), and E at the row's draft token if it lies here.
// kUnitTemp skips the multiply by inv_temp == 1 (x * 1 == x, NaN stays NaN).
template <bool kUnitTemp, typename TT>
__global__ __launch_bounds__(THREADS) void rej_scan_kernel(RejArgs a) {
  __shared__ float shm[THREADS / 64];
  __shared__ uint64_t shs[THREADS / 64];
  const int row = (int)blockIdx.y, c = (int)blockIdx.x;
  const int nt = a.B * (a.K + 1);
  const int v0 = c * CHK;
  float x[PER_T];
  if (row >= nt)
    load_chunk<kUnitTemp>(a.draft + (size_t)(row - nt) * a.V, v0, a.V, a.vec4, a.inv_temp, x);
  else
    load_chunk<kUnitTemp>(target_row<TT>(a, row), v0, a.V, a.vec4, a.inv_temp, x);
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < PER_T; ++j) m = fmaxf(m, x[j]);
  m = block_max(m, shm);
  uint64_t z = 0;
#pragma unroll
  for (int j = 0; j < PER_T; ++j) z += expfix(x[j] - m);
  z = block_sum_u64(z, shs);
  if (threadIdx.x == 0) {
    a.rmax[(size_t)row * a.nch + c] = m;
    a.rsum[(size_t)row * a.nch + c] = z;
    const int tok = row_token(a, row);
    if (tok >= v0 && tok < v0 + CHK) {
      const float xt = row >= nt ? a.draft[(size_t)(row - nt) * a.V + tok]
                                 : elem(target_row<TT>(a, row), tok);
      a.ex[row] = expfix(scaled(xt, a.inv_temp) - m);
    }
  }
}

// Sampling weight of vocabulary entry v for sequence b (residual or bonus), in one MCHK chunk
// (inside one CHK chunk c, whose m_c and F_c are fixed per call). After a rejection the
// residual W^p Zq - W^q Zp = E^p (F^p Zq) - E^q (F^q Zp): the two bracketed products
// (< 2^111) are formed once per call, so each entry costs two 32 x 128-bit products.
template <typename TT>
struct SampleRow {
  const TT* p;
  const float* q;  // nullptr for the bonus row
  float mp, mq;    // chunk maxima of the chunk being weighed
  uint64_t fp;     // F^p_c (the bonus weight is E^p F^p_c)
  u128 gp, gq;     // F^p_c Zq and F^q_c Zp
  double gpd, gqd; // the same, rounded to fp64 (relative error below 2^-51)
};

__device__ __forceinline__ double u128_to_f64(u128 x) {
  return (double)(uint64_t)(x >> 64) * 0x1p64 + (double)(uint64_t)x;
}

// The sampling rows of sequence b at position acc (the first rejection, or K: bonus), with
// row maxima Mp, Mq and totals Zp, Zq, positioned at the CHK chunk c.
template <typename TT>
__device__ __forceinline__ SampleRow<TT> sample_row(const RejArgs& a, int b, int acc, float Mp,
                                                    float Mq, u128 zp, u128 zq, int c) {
  const int K = a.K, T = K + 1;
  const int nt = a.B * T;
  SampleRow<TT> s;
  const int rp = b * T + acc;
  s.p = target_row<TT>(a, rp);
  s.mp = a.rmax[(size_t)rp * a.nch + c];
  s.fp = expfix(s.mp - Mp);
  s.gp = (u128)s.fp * zq;
  if (acc < K) {
    const int rq = nt + b * K + acc;
    s.q = a.draft + (size_t)(b * K + acc) * a.V;
    s.mq = a.rmax[(size_t)rq * a.nch + c];
    s.gq = (u128)expfix(s.mq - Mq) * zp;
  } else {
    s.q = nullptr;
    s.mq = 0.f;
    s.gq = 0;
  }
  s.gpd = u128_to_f64(s.gp);
  s.gqd = u128_to_f64(s.gq);
  return s;
}

template <typename TT>
__device__ __forceinline__ u192 weight_of(const SampleRow<TT>& s, float pv, float qv,
                                          float inv_temp) {
  const uint32_t ep = expfix(scaled(pv, inv_temp) - s.mp);
  if (s.q == nullptr) return u192{(uint64_t)ep * s.fp, 0, 0};
  const uint32_t eq = expfix(scaled(qv, inv_temp) - s.mq);
  const u192 x = mul128x32(s.gp, ep), y = mul128x32(s.gq, eq);
  return gt192(x, y) ? sub192(x, y) : u192{0, 0, 0};
}

// Whether an entry after a rejection has residual weight, gp E^p > gq E^q, decided exactly.
// Each fp64 product is within a relative 2^-50 of the exact one, so a margin of 2^-40 settles
// every pair that is not nearly tied; the rest compare the exact 160-bit products.
template <typename TT>
__device__ __forceinline__ bool residual_positive(const SampleRow<TT>& s, uint32_t ep,
                                                  uint32_t eq) {
  const double x = s.gpd * (double)ep, y = s.gqd * (double)eq;
  if (x > y * (1.0 + 0x1p-40)) return true;
  if (y > x * (1.0 + 0x1p-40)) return false;
  return gt192(mul128x32(s.gp, ep), mul128x32(s.gq, eq));
}

// This thread's PER_M consecutive sampling-row entries starting at v0 (p, and q after a
// rejection), loaded once; entries at or past V read as p = q = -inf (weight 0 is not
// used for them: callers stop at V).
struct RunVals {
  float p[PER_M], q[PER_M];
};

__device__ __forceinline__ void load_p(const float* p, int v0, float (&dst)[PER_M]) {
#pragma unroll
  for (int j = 0; j < PER_M; j += 4) {
    const float4 pv = *reinterpret_cast<const float4*>(p + v0 + j);
    dst[j] = pv.x; dst[j + 1] = pv.y; dst[j + 2] = pv.z; dst[j + 3] = pv.w;
  }
}

__device__ __forceinline__ void load_p(const uint16_t* p, int v0, float (&dst)[PER_M]) {
  static_assert(PER_M == 8, "one 16-byte piece of bf16 per run");
  const uint4 x = *reinterpret_cast<const uint4*>(p + v0);
  const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    dst[2 * k] = npn::bf16_to_f32(w[k] & 0xFFFFu);
    dst[2 * k + 1] = npn::bf16_to_f32(w[k] >> 16);
  }
}

template <typename TT>
__device__ __forceinline__ RunVals load_run(const RejArgs& a, const SampleRow<TT>& s, int v0) {
  RunVals r;
  if (a.vec4 && v0 + PER_M <= a.V) {
    load_p(s.p, v0, r.p);
#pragma unroll
    for (int j = 0; j < PER_M; j += 4) {
      if (s.q != nullptr) {
        const float4 qv = *reinterpret_cast<const float4*>(s.q + v0 + j);
        r.q[j] = qv.x; r.q[j + 1] = qv.y; r.q[j + 2] = qv.z; r.q[j + 3] = qv.w;
      } else {
        r.q[j] = r.q[j + 1] = r.q[j + 2] = r.q[j + 3] = 0.f;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < PER_M; ++j) {
      const int v = v0 + j;
      r.p[j] = v < a.V ? elem(s.p, v) : -INFINITY;
      r.q[j] = (v < a.V && s.q != nullptr) ? s.q[v] : 0.f;
    }
  }
  return r;
}

// Sampling weight of the run's entries below V, exactly: after a rejection the sum of
// gp E^p - gq E^q over the entries with positive residual equals gp (sum of their E^p) -
// gq (sum of their E^q), so each entry costs its two exponentials, an fp64 membership test
// and two 64-bit adds, and the 192-bit products are formed once per run. The bonus row's
// weights E^p F^p sum to F^p (sum of E^p).
template <typename TT>
__device__ __forceinline__ u192 run_mass(const SampleRow<TT>& s, const RunVals& r, int v0, int V,
                                         float inv_temp) {
  uint64_t sp = 0, sq = 0;
  if (s.q == nullptr) {
#pragma unroll
    for (int j = 0; j < PER_M; ++j)
      if (v0 + j < V) sp += expfix(scaled(r.p[j], inv_temp) - s.mp);
    return mul64x128(sp, (u128)s.fp);
  }
#pragma unroll
  for (int j = 0; j < PER_M; ++j) {
    if (v0 + j < V) {
      const uint32_t ep = expfix(scaled(r.p[j], inv_temp) - s.mp);
      const uint32_t eq = expfix(scaled(r.q[j], inv_temp) - s.mq);
      if (residual_positive(s, ep, eq)) {
        sp += ep;
        sq += eq;
      }
    }
  }
  return sub192(mul64x128(sp, s.gp), mul64x128(sq, s.gq));
}

// ---- 192-bit wave and block sums and scans -----------------------------------------------
__device__ __forceinline__ u192 shfl_u192(u192 v, int src_lane) {
  uint32_t w[6] = {(uint32_t)v.w0, (uint32_t)(v.w0 >> 32), (uint32_t)v.w1,
                   (uint32_t)(v.w1 >> 32), (uint32_t)v.w2, (uint32_t)(v.w2 >> 32)};
#pragma unroll
  for (int k = 0; k < 6; ++k) w[k] = __shfl(w[k], src_lane, 64);
  return u192{((uint64_t)w[1] << 32) | w[0], ((uint64_t)w[3] << 32) | w[2],
              ((uint64_t)w[5] << 32) | w[4]};
}

__device__ __forceinline__ u192 shfl_up_u192(u192 v, int d) {
  uint32_t w[6] = {(uint32_t)v.w0, (uint32_t)(v.w0 >> 32), (uint32_t)v.w1,
                   (uint32_t)(v.w1 >> 32), (uint32_t)v.w2, (uint32_t)(v.w2 >> 32)};
#pragma unroll
  for (int k = 0; k < 6; ++k) w[k] = __shfl_up(w[k], d, 64);
  return u192{((uint64_t)w[1] << 32) | w[0], ((uint64_t)w[3] << 32) | w[2],
              ((uint64_t)w[5] << 32) | w[4]};
}

__device__ __forceinline__ u192 shfl_xor_u192(u192 v, int m) {
  uint32_t w[6] = {(uint32_t)v.w0, (uint32_t)(v.w0 >> 32), (uint32_t)v.w1,
                   (uint32_t)(v.w1 >> 32), (uint32_t)v.w2, (uint32_t)(v.w2 >> 32)};
#pragma unroll
  for (int k = 0; k < 6; ++k) w[k] = __shfl_xor(w[k], m, 64);
  return u192{((uint64_t)w[1] << 32) | w[0], ((uint64_t)w[3] << 32) | w[2],
              ((uint64_t)w[5] << 32) | w[4]};
}

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ u192 wave_incl_scan_u192(u192 v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const u192 o = shfl_up_u192(v, d);
    if (lane >= d) v = add192(v, o);
  }
  return v;
}

__device__ u192 block_sum_u192(u192 v, u192* sh) {
  for (int off = 32; off > 0; off >>= 1) v = add192(v, shfl_xor_u192(v, off));
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) sh[w] = v;
  __syncthreads();
  u192 s{0, 0, 0};
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) s = add192(s, sh[i]);
  __syncthreads();
  return s;
}

// ---- decision + residual mass -------------------------------------------------------------
constexpr int kMaxRowsPerSeq = 2 * 64 + 1;  // 2K+1 rows of a sequence (K <= 64)

__device__ __forceinline__ u128 wave_sum_u128(u128 v) {
  for (int off = 32; off > 0; off >>= 1) {
    const uint64_t lo = shfl_xor_u64((uint64_t)v, off);
    const uint64_t hi = shfl_xor_u64((uint64_t)(v >> 64), off);
    v += ((u128)hi << 64) | lo;
  }
  return v;
}

// One workgroup per sequence. Its waves take the sequence's 2K+1 rows (target rows j <= K,
// then draft rows), each row's chunks spread over the lanes: M = max_c m_c,
// Z = sum_c F_c * S_c with F_c = expfix(m_c - M), and the weight W = E * F_c of the row's
// draft token; Z and M go to the workspace. Then lane i < K of wave 0 runs the accept test
// of draft position i (all tests at once; the first failing lane is the rejection), and the
// decision, the emitted draft ids and the sampling rows' Z and M are recorded.
__global__ __launch_bounds__(1024) void rej_decide_kernel(RejArgs a) {
  const int b = blockIdx.x;
  const int K = a.K, T = K + 1;
  const int nt = a.B * T;
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  __shared__ u128 s_z[kMaxRowsPerSeq];
  __shared__ float s_m[kMaxRowsPerSeq];
  __shared__ uint64_t s_w[kMaxRowsPerSeq];
  for (int j = wv; j < T + K; j += nw) {
    const int row = j < T ? b * T + j : nt + b * K + (j - T);
    const float* rm = a.rmax + (size_t)row * a.nch;
    const uint64_t* rs = a.rsum + (size_t)row * a.nch;
    float M = -INFINITY;
    for (int c = lane; c < a.nch; c += 64) M = fmaxf(M, rm[c]);
    M = npn::wave_max(M);
    u128 z = 0;
    for (int c = lane; c < a.nch; c += 64) z += (u128)rs[c] * expfix(rm[c] - M);
    z = wave_sum_u128(z);
    if (lane == 0) {
      const int tok = row_token(a, row);
      s_z[j] = z;
      s_m[j] = M;
      s_w[j] = tok < 0 ? 0 : (uint64_t)a.ex[row] * expfix(rm[tok / CHK] - M);
      a.zrow[row] = z;
      a.mrow[row] = M;
    }
  }
  __syncthreads();
  if (wv != 0) return;
  bool reject = false;
  if (lane < K) {
    const uint32_t U = uniform_fix(a.u_accept[(size_t)b * K + lane]);
    const u192 lhs = mul192x32(mul64x128(s_w[T + lane], s_z[lane]), U);
    const u192 rhs = shl24_192(mul64x128(s_w[lane], s_z[T + lane]));
    reject = !draft_id_ok(a.draft_ids[(size_t)b * K + lane], a.V) || gt192(lhs, rhs);
  }
  const uint64_t rej = __builtin_amdgcn_ballot_w64(reject);
  const int acc = rej ? __builtin_ctzll(rej) : K;
  if (lane == 0) {
    a.accepted[b] = acc;
    a.dec_row[b] = acc;
    a.dec_z[2 * b] = s_z[acc];
    a.dec_z[2 * b + 1] = acc < K ? s_z[T + acc] : 0;
    a.dec_m[2 * b] = s_m[acc];  // maxima of the sampling rows
    a.dec_m[2 * b + 1] = acc < K ? s_m[T + acc] : 0.f;
  }
  for (int t = lane; t < T; t += 64) {
    if (t < acc) a.out_ids[(size_t)b * T + t] = a.draft_ids[(size_t)b * K + t];
    else if (t > acc) a.out_ids[(size_t)b * T + t] = -1;
  }
}

// Residual (or bonus) mass of sequence b's MCHK chunk c.
template <typename TT>
__global__ __launch_bounds__(THREADS) void rej_mass_kernel(RejArgs a) {
  const int b = blockIdx.y, c = blockIdx.x;
  const int acc = a.dec_row[b];
  const SampleRow<TT> s = sample_row<TT>(a, b, acc, a.dec_m[2 * b], a.dec_m[2 * b + 1],
                                         a.dec_z[2 * b], a.dec_z[2 * b + 1], (c * MCHK) / CHK);
  const int v0 = c * MCHK + (int)threadIdx.x * PER_M;
  u192 m{0, 0, 0};
  if (v0 < a.V) m = run_mass(s, load_run(a, s, v0), v0, a.V, a.inv_temp);
  __shared__ u192 sh[THREADS / 64];
  m = block_sum_u192(m, sh);
  if (threadIdx.x == 0) a.cmass[(size_t)b * a.nchm + c] = m;
}

// Inverse CDF: the smallest v with 2^24 * C_v > U_s * S (C_v the inclusive prefix of the
// sampling weights, S their total). Wave 0 finds the MCHK chunk whose inclusive mass
// crosses the target (64 chunks per scan window, carry between windows); then each thread
// sums its run of PER_M consecutive entries of that chunk (values held in registers), a
// block-wide exclusive scan of the runs gives every thread its starting prefix, and the
// thread whose run crosses reports the first crossing entry (atomicMin over the block).
template <typename TT>
__global__ __launch_bounds__(THREADS) void rej_pick_kernel(RejArgs a) {
  const int b = blockIdx.x;
  const int K = a.K, T = K + 1;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __shared__ int s_chunk;
  __shared__ u192 s_before;
  __shared__ u192 s_target;
  __shared__ u192 s_wtot[THREADS / 64];
  __shared__ int s_tok;
  __shared__ int s_empty;
  __shared__ ArgPart s_best[THREADS / 64];
  const u192* cm = a.cmass + (size_t)b * a.nchm;
  // The sampling row's decision values do not depend on the chunk: their loads are issued
  // before the chunk search, so they are in registers when it ends.
  const int acc = a.dec_row[b];
  const float dmp = a.dec_m[2 * b], dmq = a.dec_m[2 * b + 1];
  const u128 dzp = a.dec_z[2 * b], dzq = a.dec_z[2 * b + 1];
  if (w == 0) {
    u192 tot{0, 0, 0};
    for (int c = lane; c < a.nchm; c += 64) tot = add192(tot, cm[c]);
    tot = wave_incl_scan_u192(tot);
    tot = shfl_u192(tot, 63);
    if (lane == 0) s_empty = is_zero192(tot);
    const u192 target = mul192x32(tot, uniform_fix(a.u_sample[b]));  // need 2^24 C > target
    u192 carry{0, 0, 0};
    int chunk = a.nchm - 1;
    u192 before{0, 0, 0};
    bool found = false;
    for (int c0 = 0; c0 < a.nchm && !found; c0 += 64) {
      const int c = c0 + lane;
      const u192 m = c < a.nchm ? cm[c] : u192{0, 0, 0};
      const u192 incl = add192(wave_incl_scan_u192(m), carry);
      const uint64_t hit =
          __builtin_amdgcn_ballot_w64(c < a.nchm && gt192(shl24_192(incl), target));
      if (hit != 0) {
        const int l = __builtin_ctzll(hit);
        chunk = c0 + l;
        before = shfl_u192(sub192(incl, m), l);
        found = true;
      }
      carry = shfl_u192(incl, 63);
    }
    // (selected limb by limb: a select of whole structs went through private memory)
    const u192 bsel{found ? before.w0 : carry.w0, found ? before.w1 : carry.w1,
                    found ? before.w2 : carry.w2};
    if (lane == 0) {
      s_chunk = chunk;
      s_before = bsel;
      s_target = target;
      s_tok = 0x7FFFFFFF;
    }
  }
  __syncthreads();
  if (s_empty) {
    // No sampling mass: every weight of the sampling row is 0, which happens only for a
    // bonus row whose logits are all NaN or -inf or include +inf (a residual after a
    // rejection always has mass). The token is then the row's greedy choice: its argmax,
    // NaN counting as the maximum and ties going to the lowest index (the order of
    // argmax_chunk_kernel).
    const TT* p = target_row<TT>(a, b * T + acc);
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int v = (int)threadIdx.x; v < a.V; v += THREADS) {
      const float pv = elem(p, v);
      if (beats(pv, v, bv, bi)) { bv = pv; bi = v; }
    }
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const int oi = __shfl_xor(bi, off, 64);
      if (beats(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) s_best[w] = ArgPart{bv, bi};
    __syncthreads();
    if (threadIdx.x == 0) {
      ArgPart best = s_best[0];
      for (int k = 1; k < THREADS / 64; ++k)
        if (beats(s_best[k].v, s_best[k].i, best.v, best.i)) best = s_best[k];
      a.out_ids[(size_t)b * T + acc] = best.i;
    }
    return;
  }
  const int chunk = s_chunk;
  const SampleRow<TT> s = sample_row<TT>(a, b, acc, dmp, dmq, dzp, dzq, (chunk * MCHK) / CHK);
  const int v0 = chunk * MCHK + (int)threadIdx.x * PER_M;
  RunVals rv;
  u192 run{0, 0, 0};
  if (v0 < a.V) {
    rv = load_run(a, s, v0);
    run = run_mass(s, rv, v0, a.V, a.inv_temp);
  }
  const u192 incl = wave_incl_scan_u192(run);
  if (lane == 63) s_wtot[w] = incl;
  __syncthreads();
  u192 c = add192(s_before, sub192(incl, run));
  for (int k = 0; k < w; ++k) c = add192(c, s_wtot[k]);
  const u192 target = s_target;
  if (v0 < a.V && gt192(shl24_192(add192(c, run)), target)) {  // the crossing is in this run
#pragma unroll
    for (int j = 0; j < PER_M; ++j) {
      const int v = v0 + j;
      if (v >= a.V) break;
      const u192 wv = weight_of(s, rv.p[j], rv.q[j], a.inv_temp);
      c = add192(c, wv);
      if (!is_zero192(wv) && gt192(shl24_192(c), target)) {
        atomicMin(&s_tok, v);
        break;
      }
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) a.out_ids[(size_t)b * T + acc] = s_tok;
}

// The per-row Z sums come first and the row maxima second: the header documents both as
// results that the rejection call leaves in the workspace.
struct WsLayout {
  size_t zrow, mrow, ex, rmax, rsum, dec_row, dec_z, dec_m, cmass, total;
};

WsLayout layout(int B, int K, int V) {
  const int nch = (V + CHK - 1) / CHK;
  const size_t rows = (size_t)B * (2 * K + 1);
  auto up = [](size_t x) { return (x + 255) & ~size_t(255); };
  WsLayout l{};
  size_t o = 0;
  l.zrow = o; o += up(rows * sizeof(u128));
  l.mrow = o; o += up(rows * sizeof(float));
  l.ex = o; o += up(rows * sizeof(uint32_t));
  // chunk maxima; the greedy path's argmax partials share the region
  l.rmax = o; o += up(rows * nch * sizeof(float) > (size_t)B * (K + 1) * nch * sizeof(ArgPart)
                          ? rows * nch * sizeof(float)
                          : (size_t)B * (K + 1) * nch * sizeof(ArgPart));
  l.rsum = o; o += up(rows * nch * sizeof(uint64_t));
  l.dec_row = o; o += up((size_t)B * sizeof(int32_t));
  l.dec_z = o; o += up((size_t)B * 2 * sizeof(u128));
  l.dec_m = o; o += up((size_t)B * 2 * sizeof(float));
  l.cmass = o; o += up((size_t)B * ((V + MCHK - 1) / MCHK) * sizeof(u192));
  l.total = o;
  return l;
}

bool shape_ok(int B, int K, int V) {
  return B >= 1 && B <= 65536 && K >= 1 && K <= 64 && V >= 1 && V <= (1 << 26);
}

}  // namespace

extern "C" size_t npn_accept_workspace_size(int B, int K, int V) {
  if (!shape_ok(B, K, V)) return 0;
  return layout(B, K, V).total;
}

extern "C" int npn_accept_greedy(const float* target_logits, const int64_t* draft_ids,
                                 int32_t* accepted, int64_t* out_ids, int B, int K, int V,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  NPN_REQUIRE(target_logits && draft_ids && accepted && out_ids, NPN_ERR_NULL);
  NPN_REQUIRE(shape_ok(B, K, V), NPN_ERR_SHAPE);
  const WsLayout l = layout(B, K, V);
  NPN_REQUIRE(workspace != nullptr && workspace_bytes >= l.total, NPN_ERR_WORKSPACE);
  NPN_REQUIRE(NPN_ALIGNED16(workspace), NPN_ERR_ALIGN);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nch = (V + CHK - 1) / CHK;
  ArgPart* part = reinterpret_cast<ArgPart*>(static_cast<uint8_t*>(workspace) + l.rmax);
  const bool vec4 = V % 4 == 0 && NPN_ALIGNED16(target_logits);
  hipLaunchKernelGGL(argmax_chunk_kernel, dim3(nch, B * (K + 1)), dim3(THREADS), 0, s,
                     target_logits, part, V, nch, vec4);
  hipLaunchKernelGGL(greedy_accept_kernel, dim3((B + 63) / 64), dim3(64), 0, s, part, draft_ids,
                     accepted, out_ids, B, K, nch);
  return npn_launch_status();
}

namespace {

// Argument checks shared by the rejection entry points (everything but the workspace).
int rejection_args_ok(const float* target_logits, const float* draft_logits,
                      const int64_t* draft_ids, const float* u_accept, const float* u_sample,
                      float inv_temperature, const int32_t* accepted, const int64_t* out_ids,
                      int B, int K, int V) {
  NPN_REQUIRE(target_logits && draft_logits && draft_ids && u_accept && u_sample && accepted &&
                  out_ids,
              NPN_ERR_NULL);
  NPN_REQUIRE(shape_ok(B, K, V), NPN_ERR_SHAPE);
  // Z < 2^80 and every residual sum below 2^162 for V <= 2^20, so the contract's products
  // stay below 2^192
  NPN_REQUIRE(V <= kRejMaxV, NPN_ERR_SHAPE);
  NPN_REQUIRE(inv_temperature > 0.0f && inv_temperature < 1e30f, NPN_ERR_VALUE);
  return NPN_OK;
}

// The four rejection kernels on `stream` (one logit pass, row totals + decision, residual
// mass, pick),
// with the workspace at `ws` (layout(B, K, V).total bytes, 16-byte aligned, checked by the
// caller). TT is the target rows' element type: float, or bf16 bits (uint16_t) for the
// LM-head form.
template <typename TT>
int rejection_launch(const TT* target_logits, const float* draft_logits,
                     const int64_t* draft_ids, const float* u_accept, const float* u_sample,
                     float inv_temperature, int32_t* accepted, int64_t* out_ids, int B, int K,
                     int V, uint8_t* ws, hipStream_t s) {
  const WsLayout l = layout(B, K, V);
  const int nch = (V + CHK - 1) / CHK;
  // 16-byte pieces of whole rows: V % 8 for bf16 target rows (and V % 4 for the fp32 ones)
  const bool vec4 = V % (sizeof(TT) == 2 ? 8 : 4) == 0 && NPN_ALIGNED16(target_logits) &&
                    NPN_ALIGNED16(draft_logits);
  RejArgs a{target_logits, draft_logits, draft_ids, u_accept, u_sample, inv_temperature,
            accepted, out_ids, B, K, V, nch, (V + MCHK - 1) / MCHK, vec4,
            reinterpret_cast<u128*>(ws + l.zrow), reinterpret_cast<float*>(ws + l.mrow),
            reinterpret_cast<uint32_t*>(ws + l.ex), reinterpret_cast<float*>(ws + l.rmax),
            reinterpret_cast<uint64_t*>(ws + l.rsum), reinterpret_cast<int32_t*>(ws + l.dec_row),
            reinterpret_cast<u128*>(ws + l.dec_z), reinterpret_cast<float*>(ws + l.dec_m),
            reinterpret_cast<u192*>(ws + l.cmass)};
  const int rows = B * (2 * K + 1);
  if (inv_temperature == 1.0f)
    hipLaunchKernelGGL((rej_scan_kernel<true, TT>), dim3(nch, rows), dim3(THREADS), 0, s, a);
  else
    hipLaunchKernelGGL((rej_scan_kernel<false, TT>), dim3(nch, rows), dim3(THREADS), 0, s, a);
  const int dthreads = 64 * (2 * K + 1 < 16 ? 2 * K + 1 : 16);
  hipLaunchKernelGGL(rej_decide_kernel, dim3(B), dim3(dthreads), 0, s, a);
  hipLaunchKernelGGL(rej_mass_kernel<TT>, dim3(a.nchm, B), dim3(THREADS), 0, s, a);
  hipLaunchKernelGGL(rej_pick_kernel<TT>, dim3(B), dim3(THREADS), 0, s, a);
  return npn_launch_status();
}

// ---- no-allocation variant -------------------------------------------------------------------
// The workspace of npn_accept_rejection_noalloc: a fixed device array. Each GPU holds its own
// copy, at its own address, for the life of the process. In host code `scratch` names a host
// stand-in, not device memory: kernels get the address hipGetSymbolAddress returns for the
// device they run on (scratch_on_device), never the array's name.
constexpr size_t kScratchBytes = (size_t)NPN_ACCEPT_SCRATCH_BYTES;
__device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the device `stream` belongs to (the current device for the
// null stream), looked up once per device with that device current.
int scratch_on_device(hipStream_t stream, uint8_t** out) {
  int cur = 0;
  if (hipGetDevice(&cur) != hipSuccess) return NPN_ERR_LAUNCH;
  int dev = cur;
  if (stream != nullptr) {
    hipDevice_t sd;
    if (hipStreamGetDevice(stream, &sd) != hipSuccess) return NPN_ERR_LAUNCH;
    dev = (int)sd;
  }
  NPN_REQUIRE(dev >= 0 && dev < kMaxDevices, NPN_ERR_VALUE);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    if (dev != cur && hipSetDevice(dev) != hipSuccess) return NPN_ERR_LAUNCH;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) (void)hipSetDevice(cur);
    if (e != hipSuccess || p == nullptr) return NPN_ERR_LAUNCH;
    g_scratch_ptr[dev] = p;
  }
  *out = static_cast<uint8_t*>(g_scratch_ptr[dev]);
  return NPN_OK;
}

}  // namespace

extern "C" int npn_accept_rejection(const float* target_logits, const float* draft_logits,
                                    const int64_t* draft_ids, const float* u_accept,
                                    const float* u_sample, float inv_temperature,
                                    int32_t* accepted, int64_t* out_ids, int B, int K, int V,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  const int st = rejection_args_ok(target_logits, draft_logits, draft_ids, u_accept, u_sample,
                                   inv_temperature, accepted, out_ids, B, K, V);
  if (st != NPN_OK) return st;
  NPN_REQUIRE(workspace != nullptr && workspace_bytes >= layout(B, K, V).total,
              NPN_ERR_WORKSPACE);
  NPN_REQUIRE(NPN_ALIGNED16(workspace), NPN_ERR_ALIGN);
  return rejection_launch(target_logits, draft_logits, draft_ids, u_accept, u_sample,
                          inv_temperature, accepted, out_ids, B, K, V,
                          static_cast<uint8_t*>(workspace), static_cast<hipStream_t>(stream));
}

extern "C" int npn_accept_rejection_noalloc(const float* target_logits,
                                            const float* draft_logits,
                                            const int64_t* draft_ids, const float* u_accept,
                                            const float* u_sample, float inv_temperature,
                                            int32_t* accepted, int64_t* out_ids, int B, int K,
                                            int V, void* stream) {
  const int st = rejection_args_ok(target_logits, draft_logits, draft_ids, u_accept, u_sample,
                                   inv_temperature, accepted, out_ids, B, K, V);
  if (st != NPN_OK) return st;
  NPN_REQUIRE(layout(B, K, V).total <= kScratchBytes, NPN_ERR_SCRATCH);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t* ws = nullptr;
  const int sst = scratch_on_device(s, &ws);
  if (sst != NPN_OK) return sst;
  return rejection_launch(target_logits, draft_logits, draft_ids, u_accept, u_sample,
                          inv_temperature, accepted, out_ids, B, K, V, ws, s);
}

extern "C" int npn_accept_greedy_parts(const void* parts, int nparts, const int64_t* draft_ids,
                                       int32_t* accepted, int64_t* out_ids, int B, int K,
                                       void* stream) {
  NPN_REQUIRE(parts && draft_ids && accepted && out_ids, NPN_ERR_NULL);
  NPN_REQUIRE(B >= 1 && K >= 0 && K + 1 <= 16 && nparts >= 1, NPN_ERR_SHAPE);
  hipLaunchKernelGGL(greedy_accept_parts_kernel, dim3(B), dim3(64 * (K + 1)), 0,
                     static_cast<hipStream_t>(stream), static_cast<const ArgPart*>(parts), nparts,
                     draft_ids, accepted, out_ids, K);
  return npn_launch_status();
}

extern "C" int npn_argmax_parts(const void* parts, int nparts, int64_t* ids, float* values,
                                int M, void* stream) {
  NPN_REQUIRE(parts && ids, NPN_ERR_NULL);
  NPN_REQUIRE(M >= 1 && nparts >= 1, NPN_ERR_SHAPE);
  hipLaunchKernelGGL(argmax_parts_kernel, dim3((M + 3) / 4), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const ArgPart*>(parts), nparts,
                     ids, values, M);
  return npn_launch_status();
}

// ---- rejection sampling straight from the LM head --------------------------------------------
// The LM head's GEMM writes the target logits in bf16; the rejection pass then reads the
// target rows in bf16 (half the bytes). The decisions equal npn_accept_rejection's on the
// same logits cast to fp32 (every step of the contract sees the same values).
namespace {

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

extern "C" size_t npn_accept_rejection_lm_head_workspace_size(int B, int K, int H, int V) {
  if (!shape_ok(B, K, V) || V > kRejMaxV) return 0;
  if (npn_fp8_matmul_argmax_groups(B * (K + 1), H, V) <= 0) return 0;  // GEMM shape rules
  return align256(layout(B, K, V).total) + npn_fp8_matmul_workspace_size(B * (K + 1), H, V);
}

extern "C" int npn_accept_rejection_lm_head(const uint16_t* hidden, const int8_t* lm_head_w,
                                            const float* lm_head_scale,
                                            const float* draft_logits, const int64_t* draft_ids,
                                            const float* u_accept, const float* u_sample,
                                            float inv_temperature, uint16_t* target_logits,
                                            int32_t* accepted, int64_t* out_ids, int B, int K,
                                            int H, int V, void* workspace,
                                            size_t workspace_bytes, void* stream) {
  NPN_REQUIRE(hidden && lm_head_w && lm_head_scale, NPN_ERR_NULL);
  const int st = rejection_args_ok(reinterpret_cast<const float*>(target_logits), draft_logits,
                                   draft_ids, u_accept, u_sample, inv_temperature, accepted,
                                   out_ids, B, K, V);
  if (st != NPN_OK) return st;
  const int M = B * (K + 1);
  const size_t need = npn_accept_rejection_lm_head_workspace_size(B, K, H, V);
  NPN_REQUIRE(need > 0, NPN_ERR_SHAPE);
  NPN_REQUIRE(workspace != nullptr && workspace_bytes >= need, NPN_ERR_WORKSPACE);
  NPN_REQUIRE(NPN_ALIGNED16(workspace), NPN_ERR_ALIGN);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const size_t gemm_off = align256(layout(B, K, V).total);
  const int gst = npn_fp8_matmul(hidden, lm_head_w, lm_head_scale, target_logits, M, H, V,
                                 ws + gemm_off, need - gemm_off, stream);
  if (gst != NPN_OK) return gst;
  return rejection_launch(static_cast<const uint16_t*>(target_logits), draft_logits, draft_ids,
                          u_accept, u_sample, inv_temperature, accepted, out_ids, B, K, V, ws,
                          static_cast<hipStream_t>(stream));
}
