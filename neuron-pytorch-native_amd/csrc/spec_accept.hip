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
//   rejection: row max partials -> E sums per (row, chunk) added into each row's Z, and
//              E at the draft token -> residual/bonus mass per (sequence, chunk), each block
//              making its sequence's decision first -> per-sequence inverse-CDF pick
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
struct RejArgs {
  const void* target;    // [B][K+1][V] fp32, or bf16 (the LM head's logits)
  const float* draft;    // [B][K][V]
  const int64_t* draft_ids;
  const float* u_accept;
  const float* u_sample;
  float inv_temp;
  int32_t* accepted;
  int64_t* out_ids;
  int B, K, V, nch, nchm;  // chunks of CHK (logit passes) and of MCHK (mass / pick)
  bool vec4;          // logit rows 16-byte aligned and V % 4 == 0
  // workspace (rows = B*(K+1) target rows, then B*K draft rows)
  uint64_t* zrow;     // [rows]        Z of each row (chunk sums added atomically)
  float* mrow;        // [rows]        max scaled logit of each row
  uint32_t* ex;       // [rows]        E at the row's draft token (target/draft rows i < K)
  float* rmax;        // [rows][nch]   chunk maxima
  int32_t* dec_row;   // [B]           sampling row index (target row; draft row or -1)
  uint64_t* dec_z;    // [B][2]        Zp, Zq of the sampling rows
  float* dec_m;       // [B][2]        row maxima of the sampling rows (scaled logits)
  u128* cmass;        // [B][nchm]
  const float* tgmax; // or null: [B*(K+1)][ngmax] group maxima of the target rows (NaN ignored)
  int ngmax;
};

template <typename TT>
__device__ __forceinline__ const TT* target_row(const RejArgs& a, int row) {
  return static_cast<const TT*>(a.target) + (size_t)row * a.V;
}

// Draft token whose E this row reports, or -1 (bonus rows).
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
  long x = a.draft_ids[(size_t)b * a.K + i];
  x = x < 0 ? 0 : (x >= a.V ? a.V - 1 : x);
  return (int)x;
}

// Chunk c of a row: its max scaled logit into the row's chunk maxima (and, from chunk 0,
// a zero into the row's Z, which the sum pass adds into in a later launch).
template <typename E>
__device__ __forceinline__ void max_chunk(const RejArgs& a, const E* src, int row, int c,
                                          float* sh) {
  const int v0 = c * CHK;
  float m = -INFINITY;
  visit_chunk(src, v0, a.V, a.vec4, [&](int, float x) { m = fmaxf(m, scaled(x, a.inv_temp)); });
  m = block_max(m, sh);
  if (threadIdx.x == 0) {
    a.rmax[(size_t)row * a.nch + c] = m;
    if (c == 0) a.zrow[row] = 0;
  }
}

__device__ __forceinline__ float row_max(const RejArgs& a, int row) {
  float m = a.rmax[(size_t)row * a.nch];
  for (int c = 1; c < a.nch; ++c) m = fmaxf(m, a.rmax[(size_t)row * a.nch + c]);
  return m;
}

// Chunk c of a row: its E sum added into the row's Z (exact 64-bit atomics, so the order of
// the chunks does not matter), the row max from chunk 0 and E at the draft token from the
// chunk that holds it. kUnitTemp skips the multiply by inv_temp == 1 (x * 1 == x, NaN
// stays NaN).
template <bool kUnitTemp, typename E>
__device__ __forceinline__ void sum_chunk(const RejArgs& a, const E* src, int row, int c,
                                          uint64_t* sh) {
  const float m = row_max(a, row);
  const float it = a.inv_temp;
  const int v0 = c * CHK;
  uint64_t z = 0;
  visit_chunk(src, v0, a.V, a.vec4,
              [&](int, float x) { z += expfix((kUnitTemp ? x : scaled(x, it)) - m); });
  z = block_sum_u64(z, sh);
  if (threadIdx.x == 0) {
    atomicAdd(reinterpret_cast<unsigned long long*>(a.zrow + row), (unsigned long long)z);
    if (c == 0) a.mrow[row] = m;
    const int x = row_token(a, row);
    if (x >= v0 && x < v0 + CHK) a.ex[row] = expfix(scaled(elem(src, x), it) - m);
  }
}

// The logit passes: chunk maxima of every row, then E sums. The sum pass runs its rows and
// chunks last-first, the reverse of the max pass's dispatch order, so the first chunks it
// re-reads are the ones read last.
// With group maxima of the target rows (the LM head's epilogue), a target row's max is the
// max of its groups, scaled: for inv_temp > 0, scaled(max t) == max scaled(t) (rounding is
// monotone), so the value is the one the max pass would find, without reading the row.
__device__ __forceinline__ void max_from_groups(const RejArgs& a, int row, int c, float* sh) {
  if (c != 0) {
    if (threadIdx.x == 0) a.rmax[(size_t)row * a.nch + c] = -INFINITY;
    return;
  }
  float m = -INFINITY;
  for (int g = (int)threadIdx.x; g < a.ngmax; g += THREADS)
    m = fmaxf(m, a.tgmax[(size_t)row * a.ngmax + g]);
  m = block_max(m, sh);
  if (threadIdx.x == 0) {
    a.rmax[(size_t)row * a.nch] = scaled(m, a.inv_temp);
    a.zrow[row] = 0;
  }
}

template <typename TT>
__global__ __launch_bounds__(THREADS) void rej_max_kernel(RejArgs a) {
  __shared__ float sh[THREADS / 64];
  const int row = (int)blockIdx.y, c = (int)blockIdx.x;
  const int nt = a.B * (a.K + 1);
  if (row >= nt)
    max_chunk(a, a.draft + (size_t)(row - nt) * a.V, row, c, sh);
  else if (a.tgmax != nullptr)
    max_from_groups(a, row, c, sh);
  else
    max_chunk(a, target_row<TT>(a, row), row, c, sh);
}

template <bool kUnitTemp, typename TT>
__global__ __launch_bounds__(THREADS) void rej_sum_kernel(RejArgs a) {
  __shared__ uint64_t sh[THREADS / 64];
  const int row = (int)(gridDim.y - 1 - blockIdx.y), c = (int)(gridDim.x - 1 - blockIdx.x);
  const int nt = a.B * (a.K + 1);
  if (row >= nt)
    sum_chunk<kUnitTemp>(a, a.draft + (size_t)(row - nt) * a.V, row, c, sh);
  else
    sum_chunk<kUnitTemp>(a, target_row<TT>(a, row), row, c, sh);
}

// The decision for sequence b, by one wave: lane i < K runs the accept test of draft position
// i (all tests at once; the first failing lane is the rejection). Returns the accepted count
// in every lane; with `record`, also writes accepted, the emitted draft ids (-1 past the
// sampled position) and which rows to sample from, with their Z sums and maxima, for the pick
// kernel.
__device__ __forceinline__ int decide_wave(const RejArgs& a, int b, int i, bool record) {
  const int K = a.K, T = K + 1;
  const int nt = a.B * T;
  bool reject = false;
  if (i < K) {
    const int rt = b * T + i, rd = nt + b * K + i;
    const uint64_t ueq = (uint64_t)uniform_fix(a.u_accept[(size_t)b * K + i]) * a.ex[rd];
    const u128 lhs = (u128)ueq * a.zrow[rt];                   // < 2^24 * 2^31 * 2^51
    const u128 rhs = ((u128)a.ex[rt] * a.zrow[rd]) << 24;
    reject = lhs > rhs;
  }
  const uint64_t rej = __builtin_amdgcn_ballot_w64(reject);
  const int acc = rej ? __builtin_ctzll(rej) : K;
  if (record) {
    if (i == 0) {
      a.accepted[b] = acc;
      a.dec_row[b] = acc;
      a.dec_z[2 * b] = a.zrow[b * T + acc];
      a.dec_z[2 * b + 1] = acc < K ? a.zrow[nt + b * K + acc] : 0;
      a.dec_m[2 * b] = a.mrow[b * T + acc];  // maxima of the sampling rows
      a.dec_m[2 * b + 1] = acc < K ? a.mrow[nt + b * K + acc] : 0.f;
    }
    for (int t = i; t < T; t += 64) {
      if (t < acc) a.out_ids[(size_t)b * T + t] = a.draft_ids[(size_t)b * K + t];
      else if (t > acc) a.out_ids[(size_t)b * T + t] = -1;
    }
  }
  return acc;
}

// Sampling weight of vocabulary entry v for sequence b (residual or bonus).
template <typename TT>
struct SampleRow {
  const TT* p;
  const float* q;  // nullptr for the bonus row
  float mp, mq;
  uint64_t zp, zq;
};

template <typename TT>
__device__ __forceinline__ SampleRow<TT> sample_row(const RejArgs& a, int b) {
  const int K = a.K, T = K + 1;
  const int acc = a.dec_row[b];
  SampleRow<TT> s;
  const int rt = b * T + acc;
  s.p = target_row<TT>(a, rt);
  s.mp = a.dec_m[2 * b];
  s.zp = a.dec_z[2 * b];
  s.zq = a.dec_z[2 * b + 1];
  if (acc < K) {
    s.q = a.draft + (size_t)(b * K + acc) * a.V;
    s.mq = a.dec_m[2 * b + 1];
  } else {
    s.q = nullptr;
    s.mq = 0.f;
  }
  return s;
}

// The same rows from the row statistics, for a block that has just made the decision.
template <typename TT>
__device__ __forceinline__ SampleRow<TT> sample_row_at(const RejArgs& a, int b, int acc) {
  const int K = a.K, T = K + 1;
  const int nt = a.B * T;
  SampleRow<TT> s;
  s.p = target_row<TT>(a, b * T + acc);
  s.mp = a.mrow[b * T + acc];
  s.zp = a.zrow[b * T + acc];
  if (acc < K) {
    s.q = a.draft + (size_t)(b * K + acc) * a.V;
    s.mq = a.mrow[nt + b * K + acc];
    s.zq = a.zrow[nt + b * K + acc];
  } else {
    s.q = nullptr;
    s.mq = 0.f;
    s.zq = 0;
  }
  return s;
}

template <typename TT>
__device__ __forceinline__ u128 weight_of(const SampleRow<TT>& s, float pv, float qv,
                                          float inv_temp) {
  const uint32_t ep = expfix(scaled(pv, inv_temp) - s.mp);
  if (s.q == nullptr) return ep;
  const uint32_t eq = expfix(scaled(qv, inv_temp) - s.mq);
  const u128 x = (u128)ep * s.zq, y = (u128)eq * s.zp;
  return x > y ? x - y : 0;
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

// Residual (or bonus) mass of sequence b's chunk c. Wave 0 of every block makes the
// sequence's decision (a few integer products), and chunk 0's block records it for the pick
// kernel, so the decision takes no launch of its own.
template <typename TT>
__global__ __launch_bounds__(THREADS) void rej_mass_kernel(RejArgs a) {
  const int b = blockIdx.y, c = blockIdx.x;
  __shared__ int s_acc;
  if (threadIdx.x < 64) {
    const int acc = decide_wave(a, b, (int)threadIdx.x, c == 0);
    if (threadIdx.x == 0) s_acc = acc;
  }
  __syncthreads();
  const SampleRow<TT> s = sample_row_at<TT>(a, b, s_acc);
  const int v0 = c * MCHK + (int)threadIdx.x * PER_M;
  u128 m = 0;
  if (v0 < a.V) {
    const RunVals r = load_run(a, s, v0);
#pragma unroll
    for (int j = 0; j < PER_M; ++j)
      if (v0 + j < a.V) m += weight_of(s, r.p[j], r.q[j], a.inv_temp);
  }
  __shared__ u128 sh[THREADS / 64];
  m = block_sum_u128(m, sh);
  if (threadIdx.x == 0) a.cmass[(size_t)b * a.nchm + c] = m;
}

// ---- 128-bit wave scans (exact integers) ---------------------------------------------------
__device__ __forceinline__ u128 shfl_u128(u128 v, int src_lane) {
  uint32_t w[4] = {(uint32_t)v, (uint32_t)(v >> 32), (uint32_t)(v >> 64), (uint32_t)(v >> 96)};
#pragma unroll
  for (int k = 0; k < 4; ++k) w[k] = __shfl(w[k], src_lane, 64);
  return ((u128)w[3] << 96) | ((u128)w[2] << 64) | ((u128)w[1] << 32) | w[0];
}

__device__ __forceinline__ u128 shfl_up_u128(u128 v, int d) {
  uint32_t w[4] = {(uint32_t)v, (uint32_t)(v >> 32), (uint32_t)(v >> 64), (uint32_t)(v >> 96)};
#pragma unroll
  for (int k = 0; k < 4; ++k) w[k] = __shfl_up(w[k], d, 64);
  return ((u128)w[3] << 96) | ((u128)w[2] << 64) | ((u128)w[1] << 32) | w[0];
}

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ u128 wave_incl_scan_u128(u128 v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const u128 o = shfl_up_u128(v, d);
    if (lane >= d) v += o;
  }
  return v;
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
  const SampleRow<TT> s = sample_row<TT>(a, b);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __shared__ int s_chunk;
  __shared__ u128 s_before;
  __shared__ u128 s_target;
  __shared__ u128 s_wtot[THREADS / 64];
  __shared__ int s_tok;
  __shared__ int s_empty;
  __shared__ ArgPart s_best[THREADS / 64];
  const u128* cm = a.cmass + (size_t)b * a.nchm;
  if (w == 0) {
    u128 tot = 0;
    for (int c = lane; c < a.nchm; c += 64) tot += cm[c];
    tot = wave_incl_scan_u128(tot);
    tot = shfl_u128(tot, 63);
    if (lane == 0) s_empty = tot == 0;
    const u128 target = (u128)uniform_fix(a.u_sample[b]) * tot;  // need 2^24 * C > target
    u128 carry = 0;
    int chunk = a.nchm - 1;
    u128 before = 0;
    bool found = false;
    for (int c0 = 0; c0 < a.nchm && !found; c0 += 64) {
      const int c = c0 + lane;
      const u128 m = c < a.nchm ? cm[c] : 0;
      const u128 incl = wave_incl_scan_u128(m) + carry;
      const uint64_t hit = __builtin_amdgcn_ballot_w64(c < a.nchm && (incl << 24) > target);
      if (hit != 0) {
        const int l = __builtin_ctzll(hit);
        chunk = c0 + l;
        before = shfl_u128(incl - m, l);
        found = true;
      }
      carry = shfl_u128(incl, 63);
    }
    if (lane == 0) {
      s_chunk = chunk;
      s_before = found ? before : carry;
      s_target = target;
      s_tok = 0x7FFFFFFF;
    }
  }
  __syncthreads();
  if (s_empty) {
    // No sampling mass: every E of the sampling row is 0, which happens only for a bonus row
    // whose logits are all NaN or -inf or include +inf (a residual after a rejection always
    // has mass). The token is then the row's greedy choice: its argmax, NaN counting as the
    // maximum and ties going to the lowest index (the order of argmax_chunk_kernel).
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int v = (int)threadIdx.x; v < a.V; v += THREADS) {
      const float pv = elem(s.p, v);
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
      a.out_ids[(size_t)b * (a.K + 1) + a.dec_row[b]] = best.i;
    }
    return;
  }
  const int v0 = s_chunk * MCHK + (int)threadIdx.x * PER_M;
  RunVals rv;
  u128 run = 0;
  if (v0 < a.V) {
    rv = load_run(a, s, v0);
#pragma unroll
    for (int j = 0; j < PER_M; ++j)
      if (v0 + j < a.V) run += weight_of(s, rv.p[j], rv.q[j], a.inv_temp);
  }
  const u128 incl = wave_incl_scan_u128(run);
  if (lane == 63) s_wtot[w] = incl;
  __syncthreads();
  u128 c = s_before + incl - run;
  for (int k = 0; k < w; ++k) c += s_wtot[k];
  const u128 target = s_target;
  if (v0 < a.V && ((c + run) << 24) > target) {  // the crossing lies in this run or before
#pragma unroll
    for (int j = 0; j < PER_M; ++j) {
      const int v = v0 + j;
      if (v >= a.V) break;
      const u128 wv = weight_of(s, rv.p[j], rv.q[j], a.inv_temp);
      c += wv;
      if (wv != 0 && (c << 24) > target) {
        atomicMin(&s_tok, v);
        break;
      }
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const int T = a.K + 1;
    a.out_ids[(size_t)b * T + a.dec_row[b]] = s_tok;
  }
}

// The per-row Z sums come first and the row maxima second: the header documents both as
// results that the rejection call leaves in the workspace.
struct WsLayout {
  size_t zrow, mrow, ex, rmax, dec_row, dec_z, dec_m, cmass, total;
};

WsLayout layout(int B, int K, int V) {
  const int nch = (V + CHK - 1) / CHK;
  const size_t rows = (size_t)B * (2 * K + 1);
  auto up = [](size_t x) { return (x + 255) & ~size_t(255); };
  WsLayout l{};
  size_t o = 0;
  l.zrow = o; o += up(rows * sizeof(uint64_t));
  l.mrow = o; o += up(rows * sizeof(float));
  l.ex = o; o += up(rows * sizeof(uint32_t));
  l.rmax = o; o += up(rows * nch * sizeof(float) > (size_t)B * (K + 1) * nch * sizeof(ArgPart)
                          ? rows * nch * sizeof(float)
                          : (size_t)B * (K + 1) * nch * sizeof(ArgPart));
  l.dec_row = o; o += up((size_t)B * sizeof(int32_t));
  l.dec_z = o; o += up((size_t)B * 2 * sizeof(uint64_t));
  l.dec_m = o; o += up((size_t)B * 2 * sizeof(float));
  l.cmass = o; o += up((size_t)B * ((V + MCHK - 1) / MCHK) * sizeof(u128));
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
  // Z <= V * 2^31, so 2^24 * sum R <= 2^24 * Zp * Zq stays below 2^128 for V <= 2^20
  NPN_REQUIRE(V <= kRejMaxV, NPN_ERR_SHAPE);
  NPN_REQUIRE(inv_temperature > 0.0f && inv_temperature < 1e30f, NPN_ERR_VALUE);
  return NPN_OK;
}

// The five rejection kernels on `stream`, with the workspace at `ws` (layout(B, K, V).total
// bytes, 16-byte aligned, checked by the caller).
// TT is the target rows' element type: float, or bf16 bits (uint16_t) for the LM-head form,
// which passes the target rows' group maxima (tgmax, ngmax per row) so the max pass skips them.
template <typename TT>
int rejection_launch(const TT* target_logits, const float* draft_logits,
                     const int64_t* draft_ids, const float* u_accept, const float* u_sample,
                     float inv_temperature, int32_t* accepted, int64_t* out_ids, int B, int K,
                     int V, uint8_t* ws, hipStream_t s, const float* tgmax = nullptr,
                     int ngmax = 0) {
  const WsLayout l = layout(B, K, V);
  const int nch = (V + CHK - 1) / CHK;
  // 16-byte pieces of whole rows: V % 8 for bf16 target rows (and V % 4 for the fp32 ones)
  const bool vec4 = V % (sizeof(TT) == 2 ? 8 : 4) == 0 && NPN_ALIGNED16(target_logits) &&
                    NPN_ALIGNED16(draft_logits);
  RejArgs a{target_logits, draft_logits, draft_ids, u_accept, u_sample, inv_temperature,
            accepted, out_ids, B, K, V, nch, (V + MCHK - 1) / MCHK, vec4,
            reinterpret_cast<uint64_t*>(ws + l.zrow), reinterpret_cast<float*>(ws + l.mrow),
            reinterpret_cast<uint32_t*>(ws + l.ex), reinterpret_cast<float*>(ws + l.rmax),
            reinterpret_cast<int32_t*>(ws + l.dec_row), reinterpret_cast<uint64_t*>(ws + l.dec_z),
            reinterpret_cast<float*>(ws + l.dec_m), reinterpret_cast<u128*>(ws + l.cmass),
            tgmax, ngmax};
  const int rows = B * (2 * K + 1);
  hipLaunchKernelGGL(rej_max_kernel<TT>, dim3(nch, rows), dim3(THREADS), 0, s, a);
  if (inv_temperature == 1.0f)
    hipLaunchKernelGGL((rej_sum_kernel<true, TT>), dim3(nch, rows), dim3(THREADS), 0, s, a);
  else
    hipLaunchKernelGGL((rej_sum_kernel<false, TT>), dim3(nch, rows), dim3(THREADS), 0, s, a);
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
// The LM head's GEMM writes the target logits in bf16 and, in its epilogue, each row's maxima
// per column group; the rejection passes then read the target rows in bf16 (half the bytes)
// and skip them in the max pass. The decisions equal npn_accept_rejection's on the same
// logits cast to fp32 (every step of the contract sees the same values).
namespace {

size_t lm_head_gmax_bytes(int M, int G) { return ((size_t)M * G * sizeof(float) + 255) & ~(size_t)255; }

}  // namespace

extern "C" size_t npn_accept_rejection_lm_head_workspace_size(int B, int K, int H, int V) {
  if (!shape_ok(B, K, V) || V > kRejMaxV) return 0;
  const int G = npn_fp8_matmul_argmax_groups(B * (K + 1), H, V);
  if (G <= 0) return 0;
  return layout(B, K, V).total + lm_head_gmax_bytes(B * (K + 1), G);
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
  const int G = npn_fp8_matmul_argmax_groups(M, H, V);
  NPN_REQUIRE(G > 0, NPN_ERR_SHAPE);
  const size_t need = npn_accept_rejection_lm_head_workspace_size(B, K, H, V);
  NPN_REQUIRE(workspace != nullptr && workspace_bytes >= need, NPN_ERR_WORKSPACE);
  NPN_REQUIRE(NPN_ALIGNED16(workspace), NPN_ERR_ALIGN);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  float* gmax = reinterpret_cast<float*>(ws + layout(B, K, V).total);
  const int gst = npn_fp8_matmul_rowmax(hidden, lm_head_w, lm_head_scale, target_logits, gmax, M,
                                        H, V, stream);
  if (gst != NPN_OK) return gst;
  return rejection_launch(static_cast<const uint16_t*>(target_logits), draft_logits, draft_ids,
                          u_accept, u_sample, inv_temperature, accepted, out_ids, B, K, V, ws,
                          static_cast<hipStream_t>(stream), gmax, G);
}
