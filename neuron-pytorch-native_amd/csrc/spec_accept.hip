// Speculative-decode acceptance on gfx950: greedy and rejection sampling.
//
// Greedy (the reference's on-device argmax, contrib/qwen3.6-27b/static_decode.py:1313, with
// the exact sharded top-1 order of contrib/qwen3.6-35b-a3b/static_decode_35b.py:1532-1570):
//   tid[b,t] = argmax_v target[b,t,v], first index on ties, NaN counts as the maximum;
//   accepted a_b = number of leading drafts equal to tid[b, position before them].
//
// Rejection sampling (Leviathan et al. 2023, Alg. 1) under an integer softmax contract
// (accept_contract.h) that this file and its CPU restatement evaluate with identical
// IEEE-754 operations:
//   s_v = t_v * inv_temp (fp32); 64-entry chunks c with maxima m_c inside 8192-entry blocks b
//   with maxima M_b; E_v = floor(2^31 exp_c(s_v - m_c)), F_c = floor(2^31 exp_c(m_c - M_b)),
//   G_b = floor(2^31 exp_c(M_b - M)); the weight of v is W_v = E_v F_c G_b and
//   Z = sum_b G_b S_b with S_b = sum_c F_c S_c, S_c = sum of the chunk's E (exact integers).
//   Accept draft x at position i iff U * Wq_x * Zp <= 2^24 * Wp_x * Zq (U = floor(u * 2^24));
//   a draft id outside [0, V) is a rejection. At the first rejection sample from
//   R_v = max(0, Wp_v Zq - Wq_v Zp), after K acceptances from R_v = Wp_v of the bonus row: the
//   token is the smallest v with 2^24 * sum_{w<=v} R_w > U_s * sum_w R_w.
//
// Kernels (each over B sequences, T = K+1 positions):
//   greedy:    argmax partials per (row, 8192-entry chunk) -> per-sequence merge + accept
//   rejection: block statistics (M_b, S_b) of every row, and each row's draft-token weight
//              E F, in one pass over the logits, the 64-entry chunk statistics kept on chip
//              (for the LM head the target rows' chunk statistics come from the GEMM epilogue
//              and a small kernel folds them into blocks) -> row totals and decision (every
//              workgroup of the next kernel works it out from the block statistics) with the
//              residual (or bonus) mass per 64-entry chunk and per 2048 entries, the chunk
//              maxima recomputed from the logits read anyway -> per-sequence inverse CDF
//              walking sub-chunk, chunk and entry
#include "accept_contract.h"
#include "npn_internal.h"

#include <mutex>

namespace {

constexpr int CHK = 8192;      // vocabulary entries per greedy argmax partial
constexpr int THREADS = 256;   // CHK / THREADS = 32 entries per thread
constexpr int PER_T = CHK / THREADS;
constexpr int CC = npn::kContractChunk;  // 64 entries per chunk of the rejection contract
constexpr int MCHK = 2048;     // entries per sub-chunk of the sampling masses
constexpr int kRejMaxV = 1 << 20;  // largest vocabulary of the rejection path
static_assert(npn::kContractBlock / THREADS == 32, "entry layout of the statistics pass");

typedef unsigned __int128 u128;

using npn::expfix;
using npn::expfix_rel;
using npn::scaled;
using npn::uniform_fix;

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
// partials lane, lane + 64, ..., eight loads in flight per lane at a time, then a shuffle
// tree. The rule (NaN max, lower index on ties) is a total order, so any grouping equals a
// serial scan.
__device__ __forceinline__ ArgPart wave_best(const ArgPart* __restrict__ row, int nparts) {
  constexpr int kBatch = 8;
  const int lane = threadIdx.x & 63;
  float bv = -INFINITY;
  int bi = 0x7FFFFFFF;
  for (int c0 = lane; c0 < nparts; c0 += 64 * kBatch) {
    ArgPart p[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int c = c0 + 64 * k;
      p[k] = c < nparts ? row[c] : ArgPart{-INFINITY, 0x7FFFFFFF};
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k)
      if (beats(p[k].v, p[k].i, bv, bi)) { bv = p[k].v; bi = p[k].i; }
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
// Exact unsigned integers of 192 and 256 bits (64-bit limbs, little end first) for the
// contract's products: W (<= 2^93) times Z (<= 2^113), times a 24-bit uniform or shift.
struct u192 {
  uint64_t w0, w1, w2;
};

struct u256 {
  uint64_t w0, w1, w2, w3;
};

constexpr u256 kZero256 = {0, 0, 0, 0};

__device__ __forceinline__ u256 add256(u256 a, u256 b) {
  const u128 s0 = (u128)a.w0 + b.w0;
  const u128 s1 = (u128)a.w1 + b.w1 + (uint64_t)(s0 >> 64);
  const u128 s2 = (u128)a.w2 + b.w2 + (uint64_t)(s1 >> 64);
  return u256{(uint64_t)s0, (uint64_t)s1, (uint64_t)s2, a.w3 + b.w3 + (uint64_t)(s2 >> 64)};
}

__device__ __forceinline__ u256 sub256(u256 a, u256 b) {  // a >= b
  const u128 d0 = (u128)a.w0 - b.w0;
  const uint64_t c0 = (uint64_t)(d0 >> 64) != 0;
  const u128 d1 = (u128)a.w1 - b.w1 - c0;
  const uint64_t c1 = (uint64_t)(d1 >> 64) != 0;
  const u128 d2 = (u128)a.w2 - b.w2 - c1;
  const uint64_t c2 = (uint64_t)(d2 >> 64) != 0;
  return u256{(uint64_t)d0, (uint64_t)d1, (uint64_t)d2, a.w3 - b.w3 - c2};
}

__device__ __forceinline__ bool gt256(u256 a, u256 b) {
  if (a.w3 != b.w3) return a.w3 > b.w3;
  if (a.w2 != b.w2) return a.w2 > b.w2;
  if (a.w1 != b.w1) return a.w1 > b.w1;
  return a.w0 > b.w0;
}

__device__ __forceinline__ bool is_zero256(u256 a) { return (a.w0 | a.w1 | a.w2 | a.w3) == 0; }

__device__ __forceinline__ u256 shl24_256(u256 a) {
  return u256{a.w0 << 24, (a.w1 << 24) | (a.w0 >> 40), (a.w2 << 24) | (a.w1 >> 40),
              (a.w3 << 24) | (a.w2 >> 40)};
}

// a * b for a, b < 2^128, exact.
__device__ __forceinline__ u256 mul128x128(u128 a, u128 b) {
  const uint64_t a0 = (uint64_t)a, a1 = (uint64_t)(a >> 64);
  const uint64_t b0 = (uint64_t)b, b1 = (uint64_t)(b >> 64);
  const u128 p00 = (u128)a0 * b0, p01 = (u128)a0 * b1, p10 = (u128)a1 * b0, p11 = (u128)a1 * b1;
  const u128 mid = (p00 >> 64) + (uint64_t)p01 + (uint64_t)p10;
  const u128 hi = (mid >> 64) + (p01 >> 64) + (p10 >> 64) + (uint64_t)p11;
  return u256{(uint64_t)p00, (uint64_t)mid, (uint64_t)hi,
              (uint64_t)(hi >> 64) + (uint64_t)(p11 >> 64)};
}

// a * m for m < 2^64, exact while the product stays below 2^256.
__device__ __forceinline__ u256 mul192x64(u192 a, uint64_t m) {
  const u128 p0 = (u128)a.w0 * m;
  const u128 p1 = (u128)a.w1 * m + (uint64_t)(p0 >> 64);
  const u128 p2 = (u128)a.w2 * m + (uint64_t)(p1 >> 64);
  return u256{(uint64_t)p0, (uint64_t)p1, (uint64_t)p2, (uint64_t)(p2 >> 64)};
}

// a * m for m < 2^32, exact while the product stays below 2^256.
__device__ __forceinline__ u256 mul256x32(u256 a, uint32_t m) {
  const u128 p0 = (u128)a.w0 * m;
  const u128 p1 = (u128)a.w1 * m + (uint64_t)(p0 >> 64);
  const u128 p2 = (u128)a.w2 * m + (uint64_t)(p1 >> 64);
  return u256{(uint64_t)p0, (uint64_t)p1, (uint64_t)p2, a.w3 * m + (uint64_t)(p2 >> 64)};
}

// x * y for x < 2^64 and y < 2^128 (< 2^192).
__device__ __forceinline__ u192 mul64x128(uint64_t x, u128 y) {
  const u128 lo = (u128)x * (uint64_t)y;
  const u128 hi = (u128)x * (uint64_t)(y >> 64);
  const u128 mid = (lo >> 64) + (uint64_t)hi;
  return u192{(uint64_t)lo, (uint64_t)mid, (uint64_t)(hi >> 64) + (uint64_t)(mid >> 64)};
}

__device__ __forceinline__ double u192_to_f64(u192 x) {
  return (double)x.w2 * 0x1p128 + (double)x.w1 * 0x1p64 + (double)x.w0;
}

// 64-bit, 128-bit and 256-bit values through lane shuffles (32-bit words).
__device__ __forceinline__ u128 shfl_u128(u128 v, int src_lane) {
  uint32_t w[4] = {(uint32_t)v, (uint32_t)(v >> 32), (uint32_t)(v >> 64), (uint32_t)(v >> 96)};
#pragma unroll
  for (int k = 0; k < 4; ++k) w[k] = __shfl(w[k], src_lane, 64);
  return ((u128)w[3] << 96) | ((u128)w[2] << 64) | ((u128)w[1] << 32) | w[0];
}

template <typename F>
__device__ __forceinline__ u256 map256(u256 v, F f) {
  uint32_t w[8] = {(uint32_t)v.w0, (uint32_t)(v.w0 >> 32), (uint32_t)v.w1, (uint32_t)(v.w1 >> 32),
                   (uint32_t)v.w2, (uint32_t)(v.w2 >> 32), (uint32_t)v.w3, (uint32_t)(v.w3 >> 32)};
#pragma unroll
  for (int k = 0; k < 8; ++k) w[k] = f(w[k]);
  return u256{((uint64_t)w[1] << 32) | w[0], ((uint64_t)w[3] << 32) | w[2],
              ((uint64_t)w[5] << 32) | w[4], ((uint64_t)w[7] << 32) | w[6]};
}

__device__ __forceinline__ u256 shfl_u256(u256 v, int src) {
  return map256(v, [&](uint32_t x) { return (uint32_t)__shfl(x, src, 64); });
}
__device__ __forceinline__ u256 shfl_up_u256(u256 v, int d) {
  return map256(v, [&](uint32_t x) { return (uint32_t)__shfl_up(x, d, 64); });
}
__device__ __forceinline__ u256 shfl_xor_u256(u256 v, int m) {
  return map256(v, [&](uint32_t x) { return (uint32_t)__shfl_xor(x, m, 64); });
}
template <int CTRL>
__device__ __forceinline__ u256 dpp_u256(u256 v) {
  return map256(v, [](uint32_t x) { return npn::dpp32<CTRL>(x); });
}

// Sum over the 64 lanes of a wave, in every lane: DPP inside each 16-lane row, then rows.
__device__ __forceinline__ u256 wave_sum_u256(u256 v) {
  v = add256(v, dpp_u256<npn::kDppStep[0]>(v));
  v = add256(v, dpp_u256<npn::kDppStep[1]>(v));
  v = add256(v, dpp_u256<npn::kDppStep[2]>(v));
  v = add256(v, dpp_u256<npn::kDppStep[3]>(v));
  v = add256(v, shfl_xor_u256(v, 16));
  return add256(v, shfl_xor_u256(v, 32));
}

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ u256 wave_incl_scan_u256(u256 v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const u256 o = shfl_up_u256(v, d);
    if (lane >= d) v = add256(v, o);
  }
  return v;
}

__device__ __forceinline__ u128 wave_sum_u128(u128 v) {
  for (int off = 32; off > 0; off >>= 1) {
    const uint64_t lo = shfl_xor_u64((uint64_t)v, off);
    const uint64_t hi = shfl_xor_u64((uint64_t)(v >> 64), off);
    v += ((u128)hi << 64) | lo;
  }
  return v;
}

constexpr int CPB = npn::kContractBlock / CC;  // contract chunks per block (128)
constexpr int kMaxRowsPerSeq = 2 * 64 + 1;      // 2K+1 rows of a sequence (K <= 64)

// The accept decision of one sequence and its sampling rows (target row acc, and draft row
// acc after a rejection): their maxima and totals.
struct Decision {
  u128 zp, zq;
  float mp, mq;
  int acc;
  int pad;
};

struct RejArgs {
  const void* target;    // [B][K+1][V] fp32, or bf16 (the LM head's logits)
  const float* draft;    // [B][K][V]
  const int64_t* draft_ids;
  const float* u_accept;
  const float* u_sample;
  float inv_temp;
  int32_t* accepted;
  int64_t* out_ids;
  int B, K, V, nb, nchm, nc;  // contract blocks, 2048-entry sub-chunks, contract chunks per row
  bool vec4;              // fp32 logit rows 16-byte aligned and V % 4 == 0 (bf16: V % 8)
  // workspace (rows: the B*(K+1) target rows, then the B*K draft rows)
  u128* zrow;             // [rows]      Z of each row
  float* mrow;            // [rows]      row maximum M (scaled logits)
  float* bmax;            // [rows][nb]  block maxima M_b
  u128* bsum;             // [rows][nb]  block sums S_b
  uint64_t* tw;           // [rows]      E F of the row's draft token (rows that have one)
  Decision* dec;          // [B]
  u256* cmass;            // [B][nchm]   sampling mass of each 2048-entry sub-chunk
  u256* cm64;             // [B][nc]     sampling mass of each contract chunk
};

template <typename TT>
__device__ __forceinline__ const TT* target_row(const RejArgs& a, int row) {
  return static_cast<const TT*>(a.target) + (size_t)row * a.V;
}

// Whether a draft id names a vocabulary entry. Ids outside [0, V) are never accepted: the
// position is a rejection whatever the uniform (greedy rejects them too, an argmax being in
// range), so no emitted id lies outside the vocabulary.
__device__ __forceinline__ bool draft_id_ok(int64_t x, int V) { return x >= 0 && x < V; }

// *p through a per-lane (vector) load, even when p is uniform: the compiler cannot see that
// the lane offset is 0, so the load is waited for with the other vector loads, in issue order.
__device__ __forceinline__ int64_t load_opaque(const int64_t* p) {
  int z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return p[z];
}

// The draft id a row's token weight refers to, or nullptr for bonus rows.
__device__ __forceinline__ const int64_t* row_draft_id(const RejArgs& a, int row) {
  const int nt = a.B * (a.K + 1);
  int b, i;
  if (row < nt) {
    b = row / (a.K + 1);
    i = row - b * (a.K + 1);
    if (i == a.K) return nullptr;
  } else {
    b = (row - nt) / a.K;
    i = (row - nt) - b * a.K;
  }
  return a.draft_ids + (size_t)b * a.K + i;
}

// Draft token whose weight this row reports, or -1 (bonus rows, and out-of-range draft ids).
__device__ __forceinline__ int row_token(const RejArgs& a, int row) {
  const int64_t* id = row_draft_id(a, row);
  return id != nullptr && draft_id_ok(*id, a.V) ? (int)*id : -1;
}

__device__ __forceinline__ float elem_at(const RejArgs& a, int row, int v, const float*) {
  const int nt = a.B * (a.K + 1);
  return row < nt ? static_cast<const float*>(a.target)[(size_t)row * a.V + v]
                  : a.draft[(size_t)(row - nt) * a.V + v];
}

__device__ __forceinline__ float elem_at(const RejArgs& a, int row, int v, const uint16_t*) {
  const int nt = a.B * (a.K + 1);
  return row < nt ? npn::bf16_to_f32(static_cast<const uint16_t*>(a.target)[(size_t)row * a.V + v])
                  : a.draft[(size_t)(row - nt) * a.V + v];
}

// Block statistics of one 8192-entry block from its 128 chunk statistics, one chunk per
// thread (every thread of the workgroup calls this; threads past the chunks pass m = -inf,
// s = 0): M_b = max m_c, S_b = sum F_c S_c with F_c = expfix(m_c - M_b), in every thread.
__device__ __forceinline__ void block_from_chunks(float m, uint64_t s, float* sh_m, u128* sh_s,
                                                  float& Mb, u128& Sb) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  const float mx = npn::wave_max(m);
  if (lane == 0) sh_m[w] = mx;
  __syncthreads();
  Mb = sh_m[0];
  for (int i = 1; i < nw; ++i) Mb = fmaxf(Mb, sh_m[i]);
  const u128 t = wave_sum_u128((u128)s * expfix_rel(m, Mb));
  if (lane == 0) sh_s[w] = t;
  __syncthreads();
  Sb = 0;
  for (int i = 0; i < nw; ++i) Sb += sh_s[i];
}

// Entries [v0, v0 + 8192) of one logit row into registers: thread t holds entries
// v0 + 4 (256 j + t) + k, j < 8, k < 4 (16-byte float4 loads for fp32 rows, 8-byte loads of
// four bf16 for bf16 rows) when the whole block lies inside the row and rows are aligned
// (`full`), else element by element with entries past V read as NaN.
template <typename T>
__device__ __forceinline__ void load_block(const T* src, int v0, int V, bool full,
                                           float (&x)[32]) {
  const int t = threadIdx.x;
  if (full) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int v = v0 + 4 * (j * THREADS + t);
      if constexpr (sizeof(T) == 4) {
        const float4 f = *reinterpret_cast<const float4*>(src + v);
        x[4 * j] = f.x; x[4 * j + 1] = f.y; x[4 * j + 2] = f.z; x[4 * j + 3] = f.w;
      } else {
        const uint2 h = *reinterpret_cast<const uint2*>(src + v);
        x[4 * j] = npn::bf16lo(h.x); x[4 * j + 1] = npn::bf16hi(h.x);
        x[4 * j + 2] = npn::bf16lo(h.y); x[4 * j + 3] = npn::bf16hi(h.y);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int v = v0 + 4 * (j * THREADS + t) + k;
        x[4 * j + k] = v < V ? elem(src, v) : NAN;
      }
  }
}

// Block statistics of logit rows (target rows of element type TT: fp32, or bf16 from the LM
// head; draft rows fp32): block (x, y) reads entries [8192 x, 8192 x + 8192) of row row0 + y
// once, into registers (for each j the 16 lanes of a DPP row hold one 64-entry chunk); each
// chunk's maximum m_c of the scaled logits (NaN ignored; entries past V read as NaN) and
// S_c = sum of expfix(s_v - m_c) stay on chip, and only M_b and S_b = sum F_c S_c are written.
// The thread that holds the row's draft token also writes its E F = expfix(s - m_c)
// expfix(m_c - M_b), so the decision reads no logits.
template <bool kUnitTemp, typename TT>
__global__ __launch_bounds__(THREADS) void rej_stats_kernel(RejArgs a, int row0) {
  __shared__ float sh_cm[CPB];
  __shared__ uint64_t sh_cs[CPB];
  __shared__ float sh_m[THREADS / 64];
  __shared__ u128 sh_s[THREADS / 64];
  const int row = row0 + (int)blockIdx.y;
  const int nt = a.B * (a.K + 1);
  const int v0 = (int)blockIdx.x * npn::kContractBlock;
  const int t = threadIdx.x;
  const int64_t* idp = row_draft_id(a, row);
  float x[32];
  const bool full = a.vec4 && v0 + npn::kContractBlock <= a.V;
  if (row < nt)
    load_block(target_row<TT>(a, row), v0, a.V, full, x);
  else
    load_block(a.draft + (size_t)(row - nt) * a.V, v0, a.V, full, x);
  // the draft id through a vector load issued after the logits', so that no wait for it holds
  // them back (a scalar load of the uniform address would be waited for first)
  const int64_t id = idp != nullptr ? load_opaque(idp) : -1;
  if (!kUnitTemp) {
#pragma unroll
    for (int e = 0; e < 32; ++e) x[e] = scaled(x[e], a.inv_temp);
  }
  // the thread whose four entries (toff >> 2 = 256 j + t) include the draft token keeps its value
  const int toff = draft_id_ok(id, a.V) ? (int)id - v0 : -1;
  const bool tok_here =
      toff >= 0 && toff < npn::kContractBlock && ((toff >> 2) & (THREADS - 1)) == t;
  float tx = 0.f;
  if (tok_here) {
    const int e = ((toff >> 10) << 2) | (toff & 3);
#pragma unroll
    for (int k = 0; k < 32; ++k)
      if (k == e) tx = x[k];
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < 4; ++k) m = fmaxf(m, x[4 * j + k]);
    m = npn::row_max_dpp<4>(m);
    uint64_t sm = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) sm += expfix_rel(x[4 * j + k], m);
    sm = npn::row_sum_dpp<4>(sm);
    if ((t & 15) == 0) {
      sh_cm[(j * THREADS + t) >> 4] = m;
      sh_cs[(j * THREADS + t) >> 4] = sm;
    }
  }
  __syncthreads();
  float Mb;
  u128 Sb;
  block_from_chunks(t < CPB ? sh_cm[t] : -INFINITY, t < CPB ? sh_cs[t] : 0, sh_m, sh_s, Mb, Sb);
  if (t == 0) {
    a.bmax[(size_t)row * a.nb + blockIdx.x] = Mb;
    a.bsum[(size_t)row * a.nb + blockIdx.x] = Sb;
  }
  if (tok_here) {
    const float tm = sh_cm[toff / CC];
    a.tw[row] = (uint64_t)expfix_rel(tx, tm) * expfix_rel(tm, Mb);
  } else if (toff < 0 && blockIdx.x == 0 && t == 0) {
    a.tw[row] = 0;  // no token: every row's entry is written
  }
}

// Block statistics from chunk statistics ([rows][nc], the LM-head GEMM epilogue's) of bf16
// target rows, one 128-thread workgroup per (block, row); chunks past the row's last read as
// empty. The thread of the draft token's chunk also writes the token's E F, reading the one
// logit.
__global__ __launch_bounds__(CPB) void rej_block_from_chunks_kernel(RejArgs a, int row0,
                                                                    const float* cmax,
                                                                    const uint64_t* csum,
                                                                    int nc) {
  __shared__ float sh_m[CPB / 64];
  __shared__ u128 sh_s[CPB / 64];
  const int b = (int)blockIdx.x, r = (int)blockIdx.y, row = row0 + r;
  const int c = b * CPB + (int)threadIdx.x;
  const float m = c < nc ? cmax[(size_t)r * nc + c] : -INFINITY;
  const uint64_t s = c < nc ? csum[(size_t)r * nc + c] : 0;
  const int tok = row_token(a, row);
  const bool has_tok = tok >= 0 && tok / CC == c;
  const float tx =
      has_tok ? scaled(elem_at(a, row, tok, static_cast<const uint16_t*>(nullptr)), a.inv_temp)
              : 0.f;
  float Mb;
  u128 Sb;
  block_from_chunks(m, s, sh_m, sh_s, Mb, Sb);
  if (threadIdx.x == 0) {
    a.bmax[(size_t)row * a.nb + b] = Mb;
    a.bsum[(size_t)row * a.nb + b] = Sb;
  }
  if (has_tok)
    a.tw[row] = (uint64_t)expfix_rel(tx, m) * expfix_rel(m, Mb);
  else if (tok < 0 && c == 0)
    a.tw[row] = 0;  // no token: every row's entry is written
}

// Sum over each 16-lane row (DPP), in every lane of the row.
template <int CTRL>
__device__ __forceinline__ u128 dpp_u128(u128 v) {
  return ((u128)npn::dpp64<CTRL>((uint64_t)(v >> 64)) << 64) | npn::dpp64<CTRL>((uint64_t)v);
}

__device__ __forceinline__ u128 row_sum_u128(u128 v) {
  v += dpp_u128<npn::kDppStep[0]>(v);
  v += dpp_u128<npn::kDppStep[1]>(v);
  v += dpp_u128<npn::kDppStep[2]>(v);
  return v + dpp_u128<npn::kDppStep[3]>(v);
}

// Block statistics per lane in the decision: V <= 2^20 gives at most 128 blocks, 8 per lane.
constexpr int kDecideBlocksPerLane = (kRejMaxV / npn::kContractBlock + 15) / 16;

struct DecideSmem {
  u128 z[kMaxRowsPerSeq];
  u128 w[kMaxRowsPerSeq];
  float m[kMaxRowsPerSeq];
  Decision d;
};

// Row totals and the decision of sequence b, by a whole THREADS-wide workgroup: each 16-lane
// row of lanes takes one of the sequence's 2K+1 rows at a time, lane l its blocks l, l + 16, ...:
// M = max_b M_b, Z = sum_b G_b S_b (G_b = expfix(M_b - M)), and the weight of the row's draft
// token W = (E F) G_b from the statistics pass's E F. Then lane i < K of wave 0 runs the
// accept test of position i (all at once; the first failing lane is the rejection). With
// `write` it also stores every row's Z and M, the decision record, accepted[b] and out_ids but
// the sampled token. Ends with a barrier, after which sm.d holds the decision.
__device__ void decide_sequence(const RejArgs& a, int b, bool write, DecideSmem& sm) {
  const int K = a.K, T = K + 1, nt = a.B * T;
  const int t = threadIdx.x, lane = t & 63, gl = t & 15;
  int64_t id = 0;  // wave 0's accept-test inputs, issued first
  float u = 0.f;
  if (t < K) {
    id = a.draft_ids[(size_t)b * K + t];
    u = a.u_accept[(size_t)b * K + t];
  }
  for (int j = t >> 4; j < T + K; j += THREADS / 16) {
    const int row = j < T ? b * T + j : nt + b * K + (j - T);
    const int tok = row_token(a, row);
    const uint64_t ef = a.tw[row];  // issued with the other loads; 0 without a token
    float bm[kDecideBlocksPerLane];
    u128 bs[kDecideBlocksPerLane];
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < kDecideBlocksPerLane; ++k) {
      const int bb = gl + 16 * k;
      bm[k] = bb < a.nb ? a.bmax[(size_t)row * a.nb + bb] : -INFINITY;
      bs[k] = bb < a.nb ? a.bsum[(size_t)row * a.nb + bb] : 0;
      mx = fmaxf(mx, bm[k]);
    }
    const float M = npn::row_max_dpp<4>(mx);
    u128 z = 0;
#pragma unroll
    for (int k = 0; k < kDecideBlocksPerLane; ++k) z += bs[k] * expfix_rel(bm[k], M);
    z = row_sum_u128(z);
    // M_b of the token's block: lane tb & 15 of the row holds it in bm[tb >> 4]
    const int tb = tok >= 0 ? tok / npn::kContractBlock : 0;
    float mb = bm[0];
#pragma unroll
    for (int k = 1; k < kDecideBlocksPerLane; ++k)
      if ((tb >> 4) == k) mb = bm[k];
    mb = __shfl(mb, (lane & 48) | (tb & 15), 64);
    if (gl == 0) {
      sm.z[j] = z;
      sm.m[j] = M;
      sm.w[j] = tok >= 0 ? (u128)ef * expfix_rel(mb, M) : 0;
      if (write) {
        a.zrow[row] = z;
        a.mrow[row] = M;
      }
    }
  }
  __syncthreads();
  if (t < 64) {
    bool reject = false;
    if (lane < K) {
      const uint32_t U = uniform_fix(u);
      const u256 lhs = mul256x32(mul128x128(sm.w[T + lane], sm.z[lane]), U);
      const u256 rhs = shl24_256(mul128x128(sm.w[lane], sm.z[T + lane]));
      reject = !draft_id_ok(id, a.V) || gt256(lhs, rhs);
    }
    const uint64_t rej = __builtin_amdgcn_ballot_w64(reject);
    const int acc = rej ? __builtin_ctzll(rej) : K;
    if (lane == 0) {
      Decision d;
      d.acc = acc;
      d.pad = 0;
      d.zp = sm.z[acc];
      d.mp = sm.m[acc];
      d.zq = acc < K ? sm.z[T + acc] : 0;
      d.mq = acc < K ? sm.m[T + acc] : 0.f;
      sm.d = d;
      if (write) {
        a.dec[b] = d;
        a.accepted[b] = acc;
      }
    }
    // position tt < acc holds lane tt's draft id (tt < acc <= K <= 64 only in the first pass)
    if (write)
      for (int tt = lane; tt < T; tt += 64)
        if (tt != acc) a.out_ids[(size_t)b * T + tt] = tt < acc ? id : -1;
  }
  __syncthreads();
}

// The sampling rows of one sequence for a thread's run inside one contract chunk: after a
// rejection at position acc the residual W^p Zq - W^q Zp = E^p (F^p G^p Zq) - E^q (F^q G^q Zp),
// whose bracketed products (< 2^176) are formed once per run; the bonus row's weight is
// E^p (F^p G^p).
template <typename TT>
struct SampleRow {
  const TT* p;
  const float* q;  // nullptr for the bonus row
  float mp, mq;    // chunk maxima of the run's chunk
  uint64_t fgp;    // F^p G^p
  u192 gp, gq;     // F^p G^p Zq and F^q G^q Zp
  float r;         // gq / gp rounded to fp32 (via fp64; +inf for gp = 0, NaN for both 0)
};

// The thread's N entries [v0, v0 + N) of the sampling rows, loaded once (p, and q after a
// rejection); entries at or past V read as p = -inf, q = NaN (weight 0, and ignored by the
// chunk maxima).
template <int N>
struct RunVals {
  float p[N], q[N];
};

template <int N>
__device__ __forceinline__ void load_p(const float* p, int v0, float (&dst)[N]) {
#pragma unroll
  for (int j = 0; j < N; j += 4) {
    const float4 pv = *reinterpret_cast<const float4*>(p + v0 + j);
    dst[j] = pv.x; dst[j + 1] = pv.y; dst[j + 2] = pv.z; dst[j + 3] = pv.w;
  }
}

template <int N>
__device__ __forceinline__ void load_p(const uint16_t* p, int v0, float (&dst)[N]) {
  static_assert(N % 8 == 0, "16-byte pieces of bf16");
#pragma unroll
  for (int j = 0; j < N; j += 8) {
    const uint4 x = *reinterpret_cast<const uint4*>(p + v0 + j);
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      dst[j + 2 * k] = npn::bf16_to_f32(w[k] & 0xFFFFu);
      dst[j + 2 * k + 1] = npn::bf16_to_f32(w[k] >> 16);
    }
  }
}

template <int N, bool kUnitTemp, typename TT>
__device__ __forceinline__ RunVals<N> load_run(const RejArgs& a, const TT* p, const float* q,
                                               int v0) {
  RunVals<N> r;
  if (a.vec4 && v0 + N <= a.V) {
    load_p<N>(p, v0, r.p);
    if (q != nullptr) load_p<N>(q, v0, r.q);
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int v = v0 + j;
      r.p[j] = v < a.V ? elem(p, v) : NAN;
      r.q[j] = (v < a.V && q != nullptr) ? q[v] : NAN;
    }
  }
  if (q == nullptr) {
#pragma unroll
    for (int j = 0; j < N; ++j) r.q[j] = NAN;
  }
  if (!kUnitTemp) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      r.p[j] = scaled(r.p[j], a.inv_temp);
      r.q[j] = scaled(r.q[j], a.inv_temp);
    }
  }
  return r;
}

// The run's constants from its chunk maxima (reduced by the caller over the chunk's lanes) and
// the sampling rows' block maxima of the run's block.
template <typename TT>
__device__ __forceinline__ SampleRow<TT> sample_row(const Decision& d, const TT* p,
                                                    const float* q, float mpc, float mqc,
                                                    float Mbp, float Mbq) {
  SampleRow<TT> s;
  s.p = p;
  s.q = q;
  s.mp = mpc;
  s.fgp = (uint64_t)expfix_rel(mpc, Mbp) * expfix_rel(Mbp, d.mp);
  s.gp = mul64x128(s.fgp, d.zq);
  if (q != nullptr) {
    s.mq = mqc;
    const uint64_t fgq = (uint64_t)expfix_rel(mqc, Mbq) * expfix_rel(Mbq, d.mq);
    s.gq = mul64x128(fgq, d.zp);
  } else {
    s.mq = 0.f;
    s.gq = u192{0, 0, 0};
  }
  s.r = (float)(u192_to_f64(s.gq) / u192_to_f64(s.gp));
  return s;
}

__device__ __forceinline__ bool gt192(u192 a, u192 b) {
  if (a.w2 != b.w2) return a.w2 > b.w2;
  if (a.w1 != b.w1) return a.w1 > b.w1;
  return a.w0 > b.w0;
}

// a * m for m < 2^32 (< 2^224, exact).
__device__ __forceinline__ u256 mul192x32(u192 a, uint32_t m) { return mul192x64(a, m); }

// Whether an entry after a rejection has residual weight, gp E^p > gq E^q, decided exactly.
// In fp32, x = E^p and y = E^q r (r = gq / gp) are each within 4 roundings of 2^-24 of the
// exact ratio's sides, so a margin of 2^-20 settles every pair that is not nearly tied; the
// rest (and the NaN cases 0 * inf and 0 / 0, where both comparisons fail) compare the exact
// products. An r outside fp32's normal range only meets E values of [0, 2^31] far from a
// tie, where its lost precision cannot change the side.
template <typename TT>
__device__ __forceinline__ bool residual_positive(const SampleRow<TT>& s, uint32_t ep,
                                                  uint32_t eq) {
#pragma clang fp contract(off)
  const float x = (float)ep, y = (float)eq * s.r;
  if (x > y * (1.0f + 0x1p-20f)) return true;
  if (y > x * (1.0f + 0x1p-20f)) return false;
  return gt256(mul192x32(s.gp, ep), mul192x32(s.gq, eq));
}

// Exact sampling weight of one entry (scaled logits pv, qv).
template <typename TT>
__device__ __forceinline__ u256 weight_of(const SampleRow<TT>& s, float pv, float qv) {
  const uint32_t ep = expfix_rel(pv, s.mp);
  if (s.q == nullptr) {
    const u128 w = (u128)s.fgp * ep;
    return u256{(uint64_t)w, (uint64_t)(w >> 64), 0, 0};
  }
  const uint32_t eq = expfix_rel(qv, s.mq);
  const u256 x = mul192x32(s.gp, ep), y = mul192x32(s.gq, eq);
  return gt256(x, y) ? sub256(x, y) : kZero256;
}

// Sampling weight of the run's entries below V, exactly: after a rejection the sum of
// gp E^p - gq E^q over the entries with positive residual equals gp (sum of their E^p) -
// gq (sum of their E^q), so each entry costs its two exponentials, a membership test and two
// 64-bit adds, and the wide products are formed once per run. The bonus row's weights
// E^p F^p G^p sum to F^p G^p (sum of E^p).
template <int N, typename TT>
__device__ __forceinline__ u256 run_mass(const SampleRow<TT>& s, const RunVals<N>& r) {
  uint64_t sp = 0, sq = 0;
  if (s.q == nullptr) {
#pragma unroll
    for (int j = 0; j < N; ++j) sp += expfix_rel(r.p[j], s.mp);
    const u128 w = (u128)s.fgp * sp;
    return u256{(uint64_t)w, (uint64_t)(w >> 64), 0, 0};
  }
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const uint32_t ep = expfix_rel(r.p[j], s.mp);
    const uint32_t eq = expfix_rel(r.q[j], s.mq);
    if (residual_positive(s, ep, eq)) {
      sp += ep;
      sq += eq;
    }
  }
  return sub256(mul192x64(s.gp, sp), mul192x64(s.gq, sq));
}

// Max of a run's values and the other lanes of its chunk (LANES adjacent lanes, 2 or 8).
template <int LANES, int N>
__device__ __forceinline__ float chunk_max(const float (&v)[N]) {
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < N; ++j) m = fmaxf(m, v[j]);
  return npn::row_max_dpp<LANES == 2 ? 1 : (LANES == 4 ? 2 : 3)>(m);
}

// Residual (or bonus) mass per contract chunk and per 2048-entry sub-chunk of the sampling rows.
// Every workgroup first works out its sequence's decision (block statistics only; workgroup
// x == 0 writes it out), then block x covers the contract block x of the sampling rows, each
// wave one sub-chunk, each lane a run of 32 entries, the lanes 2c, 2c + 1 of a wave forming
// chunk c of its sub-chunk (whose maxima they reduce between them). The chunk masses go to
// cm64 and the wave's sum to cmass; no workgroup reads another's results (the pick kernel,
// launched after this one, does).
constexpr int MRUN = MCHK / 64;  // entries per lane of the mass kernel
static_assert(2 * MRUN == CC, "two lanes per contract chunk");

template <bool kUnitTemp, typename TT>
__global__ __launch_bounds__(THREADS) void rej_mass_kernel(RejArgs a) {
  __shared__ DecideSmem sm;
  const int b = (int)blockIdx.y;
  decide_sequence(a, b, blockIdx.x == 0, sm);
  const int lane = threadIdx.x & 63;
  const int sub = (int)blockIdx.x * (THREADS / 64) + (int)(threadIdx.x >> 6);
  if (sub >= a.nchm) return;  // the whole wave
  const Decision d = sm.d;
  const int K = a.K, T = K + 1, nt = a.B * T;
  const int rp = b * T + d.acc, rq = nt + b * K + d.acc;
  const TT* p = target_row<TT>(a, rp);
  const float* q = d.acc < K ? a.draft + (size_t)(b * K + d.acc) * a.V : nullptr;
  const float Mbp = a.bmax[(size_t)rp * a.nb + blockIdx.x];
  const float Mbq = q != nullptr ? a.bmax[(size_t)rq * a.nb + blockIdx.x] : 0.f;
  const int v0 = sub * MCHK + lane * MRUN;
  const RunVals<MRUN> rv = load_run<MRUN, kUnitTemp>(a, p, q, v0);
  const float mpc = chunk_max<2>(rv.p), mqc = chunk_max<2>(rv.q);
  u256 m = kZero256;
  if (v0 < a.V) m = run_mass<MRUN>(sample_row<TT>(d, p, q, mpc, mqc, Mbp, Mbq), rv);
  const u256 mc = add256(m, dpp_u256<npn::kDppStep[0]>(m));  // lanes 2c and 2c + 1
  const int c = v0 / CC;
  if ((lane & 1) == 0 && c < a.nc) a.cm64[(size_t)b * a.nc + c] = mc;
  m = wave_sum_u256(m);
  if (lane == 0) a.cmass[(size_t)b * a.nchm + sub] = m;
}

// Inverse CDF, one block per sequence, three levels walked by wave 0. (1) The sequence's
// sub-chunk masses, lane l a group of G = ceil(nchm / 64) consecutive ones: one scan of the
// group sums gives the total and the group whose inclusive mass first crosses the target, whose
// masses (broadcast from its lane) then locate the sub-chunk. (2) That sub-chunk's 32 chunk
// masses, one per lane, scanned: the crossing chunk. (3) That chunk's 64 entries, one per lane,
// weighed exactly and scanned: the first crossing lane gives the token. Chunk masses are exact
// sums of their entries' weights, so each level's crossing lies inside the previous level's.
// With no mass at all every wave helps with the argmax fallback.
constexpr int kPickMaxGroup = 8;  // sub-chunk masses per lane: V <= 64 * 8 * 2048
static_assert(MCHK / CC <= 64, "one lane per chunk of a sub-chunk");

template <bool kUnitTemp, typename TT>
__global__ __launch_bounds__(THREADS) void rej_pick_kernel(RejArgs a) {
  const int b = (int)blockIdx.x;
  const int K = a.K, T = K + 1, nt = a.B * T;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __shared__ int s_tok;  // -1: no sampling mass
  __shared__ ArgPart s_best[THREADS / 64];
  const Decision d = a.dec[b];
  const int acc = d.acc;
  const int rp = b * T + acc, rq = nt + b * K + acc;
  const TT* p = target_row<TT>(a, rp);
  const float* q = acc < K ? a.draft + (size_t)(b * K + acc) * a.V : nullptr;
  if (w == 0) {
    const u256* cm = a.cmass + (size_t)b * a.nchm;
    const int G = (a.nchm + 63) / 64;
    u256 mv[kPickMaxGroup];
#pragma unroll
    for (int k = 0; k < kPickMaxGroup; ++k) {
      const int c = lane * G + k;
      mv[k] = (k < G && c < a.nchm) ? cm[c] : kZero256;
    }
    u256 gsum = kZero256;
#pragma unroll
    for (int k = 0; k < kPickMaxGroup; ++k) gsum = add256(gsum, mv[k]);
    const u256 incl = wave_incl_scan_u256(gsum);
    const u256 tot = shfl_u256(incl, 63);
    const u256 target = mul256x32(tot, uniform_fix(a.u_sample[b]));  // need 2^24 C > target
    // a positive total always crosses (U < 2^24)
    const uint64_t hit = __builtin_amdgcn_ballot_w64(gt256(shl24_256(incl), target));
    if (hit == 0) {
      if (lane == 0) s_tok = -1;
    } else {
      const int l = __builtin_ctzll(hit);
      u256 run = shfl_u256(sub256(incl, gsum), l);  // mass before lane l's group
      int sub = a.nchm - 1;
      u256 before = kZero256;
      bool found = false;
#pragma unroll
      for (int k = 0; k < kPickMaxGroup; ++k) {
        const u256 mk = shfl_u256(mv[k], l);
        const u256 next = add256(run, mk);
        if (k < G && !found && gt256(shl24_256(next), target)) {
          sub = l * G + k;
          before = run;
          found = true;
        }
        run = next;
      }
      // (2) the sub-chunk's chunk masses
      const int c = sub * (MCHK / CC) + lane;
      const bool cin = lane < MCHK / CC && c < a.nc;
      const u256 mc = cin ? a.cm64[(size_t)b * a.nc + c] : kZero256;
      const int blk = sub / (npn::kContractBlock / MCHK);
      const float Mbp = a.bmax[(size_t)rp * a.nb + blk];
      const float Mbq = q != nullptr ? a.bmax[(size_t)rq * a.nb + blk] : 0.f;
      const u256 cincl = wave_incl_scan_u256(mc);
      const uint64_t chit =
          __builtin_amdgcn_ballot_w64(cin && gt256(shl24_256(add256(before, cincl)), target));
      const int cl = chit ? __builtin_ctzll(chit) : 0;
      const u256 cbefore = add256(before, shfl_u256(sub256(cincl, mc), cl));
      // (3) the chunk's entries
      const int v = (sub * (MCHK / CC) + cl) * CC + lane;
      float pv = NAN, qv = NAN;
      if (v < a.V) {
        pv = elem(p, v);
        if (q != nullptr) qv = q[v];
      }
      if (!kUnitTemp) {
        pv = scaled(pv, a.inv_temp);
        qv = scaled(qv, a.inv_temp);
      }
      const float mpc = npn::wave_max(fmaxf(pv, -INFINITY));
      const float mqc = npn::wave_max(fmaxf(qv, -INFINITY));
      const u256 wv = weight_of(sample_row<TT>(d, p, q, mpc, mqc, Mbp, Mbq), pv, qv);
      const u256 vincl = add256(cbefore, wave_incl_scan_u256(wv));
      const uint64_t vhit =
          __builtin_amdgcn_ballot_w64(v < a.V && gt256(shl24_256(vincl), target));
      if (lane == 0) s_tok = v + (vhit ? __builtin_ctzll(vhit) : 0);
    }
  }
  __syncthreads();
  int tok = s_tok;
  if (tok < 0) {
    // No sampling mass: every weight of the sampling row is 0, which happens only for a
    // bonus row whose logits are all NaN or -inf or include +inf, or for the residual after
    // an out-of-range draft id where Wp Zq == Wq Zp everywhere (a residual after a failed
    // test always has mass). The token is then the target row's greedy choice: its argmax,
    // NaN counting as the maximum and ties going to the lowest index (the order of
    // argmax_chunk_kernel).
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int vv = (int)threadIdx.x; vv < a.V; vv += THREADS) {
      const float pv = elem(p, vv);
      if (beats(pv, vv, bv, bi)) { bv = pv; bi = vv; }
    }
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const int oi = __shfl_xor(bi, off, 64);
      if (beats(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) s_best[w] = ArgPart{bv, bi};
    __syncthreads();
    ArgPart best = s_best[0];
    for (int k = 1; k < THREADS / 64; ++k)
      if (beats(s_best[k].v, s_best[k].i, best.v, best.i)) best = s_best[k];
    tok = best.i;
  }
  if (threadIdx.x == 0) a.out_ids[(size_t)b * T + acc] = tok;
}

// Workspace of the acceptance calls. The per-row Z sums come first and the row maxima second:
// the header documents both as results that the rejection call leaves in the workspace.
struct WsLayout {
  size_t zrow, mrow, bmax, bsum, tw, dec, cmass, cm64, total;
};

WsLayout layout(int B, int K, int V) {
  const int nb = (V + npn::kContractBlock - 1) / npn::kContractBlock;
  const int nch = (V + CHK - 1) / CHK;
  const size_t rows = (size_t)B * (2 * K + 1);
  auto up = [](size_t x) { return (x + 255) & ~size_t(255); };
  WsLayout l{};
  size_t o = 0;
  l.zrow = o; o += up(rows * sizeof(u128));
  l.mrow = o; o += up(rows * sizeof(float));
  // block maxima; the greedy path's argmax partials share the region
  const size_t bmax_bytes = rows * nb * sizeof(float);
  const size_t part_bytes = (size_t)B * (K + 1) * nch * sizeof(ArgPart);
  l.bmax = o; o += up(bmax_bytes > part_bytes ? bmax_bytes : part_bytes);
  l.bsum = o; o += up(rows * nb * sizeof(u128));
  l.tw = o; o += up(rows * sizeof(uint64_t));
  l.dec = o; o += up((size_t)B * sizeof(Decision));
  l.cmass = o; o += up((size_t)B * ((V + MCHK - 1) / MCHK) * sizeof(u256));
  l.cm64 = o; o += up((size_t)B * ((V + CC - 1) / CC) * sizeof(u256));
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
  ArgPart* part = reinterpret_cast<ArgPart*>(static_cast<uint8_t*>(workspace) + l.bmax);
  const bool vec4 = V % 4 == 0 && NPN_ALIGNED16(target_logits);
  hipLaunchKernelGGL(argmax_chunk_kernel, dim3(nch, B * (K + 1)), dim3(THREADS), 0, s,
                     target_logits, part, V, nch, vec4);
  hipLaunchKernelGGL(greedy_accept_kernel, dim3((B + 63) / 64), dim3(64), 0, s, part, draft_ids,
                     accepted, out_ids, B, K, nch);
  return npn_launch_status();
}

namespace {

// Argument checks shared by the rejection entry points (everything but the workspace).
int rejection_args_ok(const void* target_logits, const float* draft_logits,
                      const int64_t* draft_ids, const float* u_accept, const float* u_sample,
                      float inv_temperature, const int32_t* accepted, const int64_t* out_ids,
                      int B, int K, int V) {
  NPN_REQUIRE(target_logits && draft_logits && draft_ids && u_accept && u_sample && accepted &&
                  out_ids,
              NPN_ERR_NULL);
  NPN_REQUIRE(shape_ok(B, K, V), NPN_ERR_SHAPE);
  // Z <= V 2^93 <= 2^113 and every residual sum at most 2^226 for V <= 2^20, so the
  // contract's products stay below 2^256
  NPN_REQUIRE(V <= kRejMaxV, NPN_ERR_SHAPE);
  NPN_REQUIRE(inv_temperature > 0.0f && inv_temperature < 1e30f, NPN_ERR_VALUE);
  return NPN_OK;
}

RejArgs rej_args(const void* target_logits, const float* draft_logits, const int64_t* draft_ids,
                 const float* u_accept, const float* u_sample, float inv_temperature,
                 int32_t* accepted, int64_t* out_ids, int B, int K, int V, bool bf16_target,
                 uint8_t* ws) {
  const WsLayout l = layout(B, K, V);
  // 16-byte pieces of whole rows: V % 8 for bf16 target rows (and V % 4 for the fp32 ones)
  const bool vec4 = V % (bf16_target ? 8 : 4) == 0 && NPN_ALIGNED16(target_logits) &&
                    NPN_ALIGNED16(draft_logits);
  return RejArgs{target_logits, draft_logits, draft_ids, u_accept, u_sample, inv_temperature,
                 accepted, out_ids, B, K, V,
                 (V + npn::kContractBlock - 1) / npn::kContractBlock, (V + MCHK - 1) / MCHK,
                 (V + CC - 1) / CC, vec4, reinterpret_cast<u128*>(ws + l.zrow),
                 reinterpret_cast<float*>(ws + l.mrow), reinterpret_cast<float*>(ws + l.bmax),
                 reinterpret_cast<u128*>(ws + l.bsum), reinterpret_cast<uint64_t*>(ws + l.tw),
                 reinterpret_cast<Decision*>(ws + l.dec), reinterpret_cast<u256*>(ws + l.cmass),
                 reinterpret_cast<u256*>(ws + l.cm64)};
}

// Block statistics of `rows` rows starting at row0 (target rows of element type TT).
template <typename TT>
void launch_stats(const RejArgs& a, int row0, int rows, hipStream_t s) {
  const dim3 grid(a.nb, rows);
  if (a.inv_temp == 1.0f)
    hipLaunchKernelGGL((rej_stats_kernel<true, TT>), grid, dim3(THREADS), 0, s, a, row0);
  else
    hipLaunchKernelGGL((rej_stats_kernel<false, TT>), grid, dim3(THREADS), 0, s, a, row0);
}

// Decision with sampling mass, then the pick (every row's block statistics and draft-token
// weight in place). TT is the target rows' element type: float, or bf16 bits (uint16_t) for
// the LM-head form.
template <typename TT>
int launch_decide_sample(const RejArgs& a, hipStream_t s) {
  const dim3 mgrid((a.nchm + THREADS / 64 - 1) / (THREADS / 64), a.B);
  if (a.inv_temp == 1.0f) {
    hipLaunchKernelGGL((rej_mass_kernel<true, TT>), mgrid, dim3(THREADS), 0, s, a);
    hipLaunchKernelGGL((rej_pick_kernel<true, TT>), dim3(a.B), dim3(THREADS), 0, s, a);
  } else {
    hipLaunchKernelGGL((rej_mass_kernel<false, TT>), mgrid, dim3(THREADS), 0, s, a);
    hipLaunchKernelGGL((rej_pick_kernel<false, TT>), dim3(a.B), dim3(THREADS), 0, s, a);
  }
  return npn_launch_status();
}

// The three rejection kernels over fp32 logits on `stream`, with the workspace at `ws`
// (layout(B, K, V).total bytes, 16-byte aligned, checked by the caller).
int rejection_launch(const float* target_logits, const float* draft_logits,
                     const int64_t* draft_ids, const float* u_accept, const float* u_sample,
                     float inv_temperature, int32_t* accepted, int64_t* out_ids, int B, int K,
                     int V, uint8_t* ws, hipStream_t s) {
  const RejArgs a = rej_args(target_logits, draft_logits, draft_ids, u_accept, u_sample,
                             inv_temperature, accepted, out_ids, B, K, V, false, ws);
  launch_stats<float>(a, 0, B * (2 * K + 1), s);
  return launch_decide_sample<float>(a, s);
}

// ---- no-allocation variant -------------------------------------------------------------------
// The workspace of npn_accept_rejection_noalloc: a fixed device array. Each GPU holds its own
// copy, at its own address, for the life of the process. In host code `scratch` names a host
// stand-in, not device memory: kernels get the address hipGetSymbolAddress returns for the
// device they run on (scratch_on_device), never the array's name. Nothing in it needs clearing
// between calls: every word a call reads was written earlier in the same call.
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
  hipLaunchKernelGGL(argmax_parts_kernel, dim3((M + 3) / 4), dim3(256),
                     0, static_cast<hipStream_t>(stream), static_cast<const ArgPart*>(parts),
                     nparts, ids, values, M);
  return npn_launch_status();
}

// ---- rejection sampling straight from the LM head --------------------------------------------
// The LM head's GEMM writes the target logits in bf16 and, in its epilogue, the contract's
// chunk statistics of every target row, so the target rows are never read back in full: the
// statistics pass covers only the draft rows, and the sampling kernel re-reads only each
// sequence's sampling row. The decisions equal npn_accept_rejection's on the same logits cast
// to fp32 (every step of the contract sees the same values).
namespace {

// The LM-head call's workspace: the acceptance layout, then the GEMM epilogue's chunk
// statistics of the target rows ([M][V / 64] maxima and sums).
struct LmLayout {
  size_t cmax, csum, total;
};

LmLayout lm_layout(int B, int K, int V) {
  auto up = [](size_t x) { return (x + 255) & ~size_t(255); };
  const size_t rows = (size_t)B * (K + 1), nc = (size_t)V / CC;
  LmLayout l{};
  l.cmax = up(layout(B, K, V).total);
  l.csum = l.cmax + up(rows * nc * sizeof(float));
  l.total = l.csum + up(rows * nc * sizeof(uint64_t));
  return l;
}

}  // namespace

extern "C" size_t npn_accept_rejection_lm_head_workspace_size(int B, int K, int H, int V) {
  if (!shape_ok(B, K, V) || V > kRejMaxV) return 0;
  if (!npn::fp8_matmul_chunk_stats_ok(B * (K + 1), H, V)) return 0;  // GEMM shape rules
  return lm_layout(B, K, V).total;
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
  const int st = rejection_args_ok(target_logits, draft_logits, draft_ids, u_accept, u_sample,
                                   inv_temperature, accepted, out_ids, B, K, V);
  if (st != NPN_OK) return st;
  const int T = K + 1, M = B * T;
  const size_t need = npn_accept_rejection_lm_head_workspace_size(B, K, H, V);
  NPN_REQUIRE(need > 0, NPN_ERR_SHAPE);
  NPN_REQUIRE(workspace != nullptr && workspace_bytes >= need, NPN_ERR_WORKSPACE);
  NPN_REQUIRE(NPN_ALIGNED16(workspace), NPN_ERR_ALIGN);
  NPN_REQUIRE(NPN_ALIGNED16(hidden) && NPN_ALIGNED16(lm_head_w) && NPN_ALIGNED16(target_logits),
              NPN_ERR_ALIGN);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const LmLayout ll = lm_layout(B, K, V);
  float* cmax = reinterpret_cast<float*>(ws + ll.cmax);
  uint64_t* csum = reinterpret_cast<uint64_t*>(ws + ll.csum);
  const RejArgs a = rej_args(target_logits, draft_logits, draft_ids, u_accept, u_sample,
                             inv_temperature, accepted, out_ids, B, K, V, true, ws);
  if (npn::fp8_matmul_stats_pass_cheaper(M, H, V)) {
    // the plain GEMM, then one statistics pass over the bf16 target rows and the draft rows
    const int gst = npn::fp8_matmul_unsplit(hidden, lm_head_w, lm_head_scale, target_logits, M,
                                            H, V, s);
    if (gst != NPN_OK) return gst;
    launch_stats<uint16_t>(a, 0, B * (2 * K + 1), s);
    return launch_decide_sample<uint16_t>(a, s);
  }
  launch_stats<uint16_t>(a, M, B * K, s);  // draft rows
  const int gst = npn::fp8_matmul_chunk_stats(hidden, lm_head_w, lm_head_scale, target_logits,
                                              cmax, csum, inv_temperature, M, H, V, s);
  if (gst != NPN_OK) return gst;
  hipLaunchKernelGGL(rej_block_from_chunks_kernel, dim3(a.nb, M), dim3(CPB), 0, s, a, 0, cmax,
                     csum, V / CC);
  return launch_decide_sample<uint16_t>(a, s);
}
