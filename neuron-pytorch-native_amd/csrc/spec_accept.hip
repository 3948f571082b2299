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
//   s_v = t_v * inv_temp (fp32); 64-entry chunks c with maxima m_c; E_v = floor(2^31 *
//   exp_c(s_v - m_c)); S_c = sum of E over the chunk; M = max_c m_c; F_c = floor(2^31 *
//   exp_c(m_c - M)); the weight of v is W_v = E_v F_c and Z = sum_c F_c S_c (exact integers).
//   Accept draft x at position i iff U * Wq_x * Zp <= 2^24 * Wp_x * Zq (U = floor(u * 2^24));
//   a draft id outside [0, V) is a rejection. At the first rejection sample from
//   R_v = max(0, Wp_v Zq - Wq_v Zp), after K acceptances from R_v = Wp_v of the bonus row: the
//   token is the smallest v with 2^24 * sum_{w<=v} R_w > U_s * sum_w R_w.
//
// Kernels (each over B sequences, T = K+1 positions):
//   greedy:    argmax partials per (row, 8192-entry chunk) -> per-sequence merge + accept
//   rejection: chunk statistics (m_c, S_c) of every row in one pass over the logits (for the
//              LM head the target rows' come from the GEMM epilogue) -> per-row totals M, Z
//              and the draft token's weight -> one sampling kernel: every block re-derives the
//              sequence's decision, adds the residual (or bonus) mass of its 2048 entries,
//              and the last block of each sequence to finish runs the inverse CDF
#include "accept_contract.h"
#include "npn_internal.h"

#include <mutex>

namespace {

constexpr int CHK = 8192;      // vocabulary entries per greedy argmax partial
constexpr int THREADS = 256;   // CHK / THREADS = 32 entries per thread
constexpr int PER_T = CHK / THREADS;
constexpr int CC = npn::kContractChunk;  // 64 entries per chunk of the rejection contract
constexpr int SBLK = 8192;     // entries per block of the chunk-statistics pass (128 chunks)
constexpr int MCHK = 2048;     // entries per block of the sampling kernel
constexpr int PER_M = MCHK / THREADS;  // 8 consecutive entries per thread, inside one chunk
constexpr int kRejMaxV = 1 << 20;  // largest vocabulary of the rejection path
static_assert(SBLK / THREADS == 32 && CC % PER_M == 0, "entry layouts of the rejection kernels");

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
// the contract: W (<= 2^62) times Z (<= 2^82), times a 24-bit uniform or shift.
struct u192 {
  uint64_t w0, w1, w2;
};

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
  int B, K, V, nc, nchm;  // contract chunks per row; sampling-kernel blocks per row
  bool vec4;              // fp32 logit rows 16-byte aligned and V % 4 == 0 (bf16: V % 8)
  // workspace (rows: the B*(K+1) target rows, then the B*K draft rows)
  u128* zrow;             // [rows]      Z of each row
  float* mrow;            // [rows]      row maximum M (scaled logits)
  uint64_t* wtok;         // [rows]      W of the row's draft token (0: bonus row, bad id)
  float* cmax;            // [rows][nc]  chunk maxima m_c
  uint64_t* csum;         // [rows][nc]  chunk sums S_c
  u192* cmass;            // [B][nchm]   sampling mass of each sampling-kernel block
  uint32_t* cnt;          // [B]         sampling-kernel blocks finished, per sequence
};

template <typename TT>
__device__ __forceinline__ const TT* target_row(const RejArgs& a, int row) {
  return static_cast<const TT*>(a.target) + (size_t)row * a.V;
}

// Whether a draft id names a vocabulary entry. Ids outside [0, V) are never accepted: the
// position is a rejection whatever the uniform (greedy rejects them too, an argmax being in
// range), so no emitted id lies outside the vocabulary.
__device__ __forceinline__ bool draft_id_ok(int64_t x, int V) { return x >= 0 && x < V; }

// Draft token whose weight this row reports, or -1 (bonus rows, and out-of-range draft ids).
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

// The 16-lane shuffles of the statistics pass (lanes that share a chunk).
__device__ __forceinline__ float max16(float m) {
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  return m;
}

__device__ __forceinline__ uint64_t sum16(uint64_t s) {
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) s += shfl_xor_u64(s, off);
  return s;
}

// Chunk statistics of fp32 logit rows: block (x, y) reads entries [8192 x, 8192 x + 8192) of
// row row0 + y once, into registers (thread t holds the float4s at v0 + 4 (256 j + t),
// j < 8, so for each j the 16 lanes of a 16-lane group hold one 64-entry chunk), and writes
// each chunk's maximum m_c of the scaled logits (NaN ignored; entries past V read as NaN)
// and S_c = sum of expfix(s_v - m_c).
template <bool kUnitTemp>
__global__ __launch_bounds__(THREADS) void rej_stats_kernel(RejArgs a, int row0) {
  const int row = row0 + (int)blockIdx.y;
  const int nt = a.B * (a.K + 1);
  const float* src = row < nt ? static_cast<const float*>(a.target) + (size_t)row * a.V
                              : a.draft + (size_t)(row - nt) * a.V;
  const int v0 = (int)blockIdx.x * SBLK;
  const int t = threadIdx.x;
  float x[32];
  if (a.vec4 && v0 + SBLK <= a.V) {  // whole block inside the row: all loads first, no guards
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float4 f = *reinterpret_cast<const float4*>(src + v0 + 4 * (j * THREADS + t));
      x[4 * j] = f.x; x[4 * j + 1] = f.y; x[4 * j + 2] = f.z; x[4 * j + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int v = v0 + 4 * (j * THREADS + t) + k;
        x[4 * j + k] = v < a.V ? src[v] : NAN;
      }
  }
  if (!kUnitTemp) {
#pragma unroll
    for (int e = 0; e < 32; ++e) x[e] = scaled(x[e], a.inv_temp);
  }
  float* cm = a.cmax + (size_t)row * a.nc;
  uint64_t* cs = a.csum + (size_t)row * a.nc;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < 4; ++k) m = fmaxf(m, x[4 * j + k]);
    m = max16(m);
    uint64_t s = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) s += expfix_rel(x[4 * j + k], m);
    s = sum16(s);
    const int c = (v0 >> 6) + ((j * THREADS + t) >> 4);
    if ((t & 15) == 0 && c < a.nc) {
      cm[c] = m;
      cs[c] = s;
    }
  }
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

// Row totals, one block per row: M = max_c m_c, Z = sum_c F_c S_c (F_c = expfix(m_c - M)),
// and W = E F_c of the row's draft token (its logit and chunk maximum are loaded first). The
// first target row of each sequence also clears the sequence's counter of finished
// sampling-kernel blocks (the sampling kernel runs after this one, on the same stream).
template <typename TT>
__global__ __launch_bounds__(THREADS) void rej_rowtotal_kernel(RejArgs a) {
  __shared__ float shm[THREADS / 64];
  __shared__ u128 shz[THREADS / 64];
  const int row = (int)blockIdx.x;
  const int nt = a.B * (a.K + 1);
  const float* cm = a.cmax + (size_t)row * a.nc;
  const uint64_t* cs = a.csum + (size_t)row * a.nc;
  const int tok = row_token(a, row);
  float xt = 0.f, mt = 0.f;
  if (threadIdx.x == 0 && tok >= 0) {
    xt = elem_at(a, row, tok, static_cast<const TT*>(nullptr));
    mt = cm[tok / CC];
  }
  constexpr int U = 8;  // chunks per thread per batch, loads issued together
  float M = -INFINITY;
  for (int c0 = threadIdx.x; c0 < a.nc; c0 += U * THREADS) {
    float v[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int c = c0 + k * THREADS;
      v[k] = c < a.nc ? cm[c] : -INFINITY;
    }
#pragma unroll
    for (int k = 0; k < U; ++k) M = fmaxf(M, v[k]);
  }
  M = block_max(M, shm);
  u128 z = 0;
  for (int c0 = threadIdx.x; c0 < a.nc; c0 += U * THREADS) {
    float v[U];
    uint64_t s[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int c = c0 + k * THREADS;
      v[k] = c < a.nc ? cm[c] : -INFINITY;
      s[k] = c < a.nc ? cs[c] : 0;
    }
#pragma unroll
    for (int k = 0; k < U; ++k) z += (u128)s[k] * expfix_rel(v[k], M);
  }
  z = block_sum_u128(z, shz);
  if (threadIdx.x == 0) {
    a.zrow[row] = z;
    a.mrow[row] = M;
    a.wtok[row] = tok < 0 ? 0
                          : (uint64_t)expfix_rel(scaled(xt, a.inv_temp), mt) * expfix_rel(mt, M);
    if (row < nt && row % (a.K + 1) == 0) a.cnt[row / (a.K + 1)] = 0;
  }
}

// The sampling rows of one sequence, as seen by one thread at the contract chunk cc of its
// run: after a rejection at position acc the residual W^p Zq - W^q Zp = E^p (F^p Zq) -
// E^q (F^q Zp), whose bracketed products (< 2^114) are formed once per thread; for the bonus
// row the weight is E^p F^p.
template <typename TT>
struct SampleRow {
  const TT* p;
  const float* q;  // nullptr for the bonus row
  float mp, mq;    // chunk maxima of chunk cc
  uint64_t fp;     // F^p of chunk cc
  u128 gp, gq;     // F^p Zq and F^q Zp
  double gpd, gqd; // the same, rounded to fp64 (relative error below 2^-51)
};

__device__ __forceinline__ double u128_to_f64(u128 x) {
  return (double)(uint64_t)(x >> 64) * 0x1p64 + (double)(uint64_t)x;
}

// Decision of sequence b, shared by the blocks of the sampling kernel.
struct Decision {
  int acc;         // accepted drafts (the sampling position)
  float mp, mq;    // row maxima of the sampling rows (mq: draft row, after a rejection)
  u128 zp, zq;     // their totals
};

template <typename TT>
__device__ __forceinline__ SampleRow<TT> sample_row(const RejArgs& a, int b, const Decision& d,
                                                    int cc) {
  const int K = a.K, T = K + 1;
  const int nt = a.B * T;
  SampleRow<TT> s;
  const int rp = b * T + d.acc;
  s.p = target_row<TT>(a, rp);
  s.mp = a.cmax[(size_t)rp * a.nc + cc];
  s.fp = expfix_rel(s.mp, d.mp);
  s.gp = (u128)s.fp * d.zq;
  if (d.acc < K) {
    const int rq = nt + b * K + d.acc;
    s.q = a.draft + (size_t)(b * K + d.acc) * a.V;
    s.mq = a.cmax[(size_t)rq * a.nc + cc];
    s.gq = (u128)expfix_rel(s.mq, d.mq) * d.zp;
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
  const uint32_t ep = expfix_rel(scaled(pv, inv_temp), s.mp);
  if (s.q == nullptr) return u192{(uint64_t)ep * s.fp, 0, 0};
  const uint32_t eq = expfix_rel(scaled(qv, inv_temp), s.mq);
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
// rejection), loaded once; entries at or past V read as p = -inf (callers stop at V).
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
      if (v0 + j < V) sp += expfix_rel(scaled(r.p[j], inv_temp), s.mp);
    return mul64x128(sp, (u128)s.fp);
  }
#pragma unroll
  for (int j = 0; j < PER_M; ++j) {
    if (v0 + j < V) {
      const uint32_t ep = expfix_rel(scaled(r.p[j], inv_temp), s.mp);
      const uint32_t eq = expfix_rel(scaled(r.q[j], inv_temp), s.mq);
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

__device__ __forceinline__ u128 shfl_u128(u128 v, int src_lane) {
  uint32_t w[4] = {(uint32_t)v, (uint32_t)(v >> 32), (uint32_t)(v >> 64), (uint32_t)(v >> 96)};
#pragma unroll
  for (int k = 0; k < 4; ++k) w[k] = __shfl(w[k], src_lane, 64);
  return ((u128)w[3] << 96) | ((u128)w[2] << 64) | ((u128)w[1] << 32) | w[0];
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

// The accept decision of sequence b, by wave 0 (lane i < K tests draft position i, all at
// once; the first failing lane is the rejection), with the sampling rows' maxima and totals.
// Lane l <= K also loads target row l's M and Z, so the bonus row's are at hand.
__device__ Decision decide(const RejArgs& a, int b) {
  const int K = a.K, T = K + 1, nt = a.B * T;
  const int lane = threadIdx.x & 63;
  bool reject = false;
  u128 zp = 0, zq = 0;
  float mp = 0.f, mq = 0.f;
  if (lane <= K) {
    const int rp = b * T + lane;
    zp = a.zrow[rp];
    mp = a.mrow[rp];
  }
  if (lane < K) {
    const int rp = b * T + lane, rq = nt + b * K + lane;
    const int64_t id = a.draft_ids[(size_t)b * K + lane];
    zq = a.zrow[rq];
    mq = a.mrow[rq];
    const uint64_t wp = a.wtok[rp], wq = a.wtok[rq];
    const uint32_t U = uniform_fix(a.u_accept[(size_t)b * K + lane]);
    const u192 lhs = mul192x32(mul64x128(wq, zp), U);
    const u192 rhs = shl24_192(mul64x128(wp, zq));
    reject = !draft_id_ok(id, a.V) || gt192(lhs, rhs);
  }
  const uint64_t rej = __builtin_amdgcn_ballot_w64(reject);
  Decision d;
  d.acc = rej ? __builtin_ctzll(rej) : K;
  if (d.acc < 64) {
    d.zp = shfl_u128(zp, d.acc);
    d.mp = __shfl(mp, d.acc, 64);
  } else {  // the bonus row of K = 64 has no lane
    d.zp = a.zrow[b * T + K];
    d.mp = a.mrow[b * T + K];
  }
  if (d.acc < K) {
    d.zq = shfl_u128(zq, d.acc);
    d.mq = __shfl(mq, d.acc, 64);
  } else {
    d.zq = 0;
    d.mq = 0.f;
  }
  return d;
}

// Sampling: block (c, b) re-derives sequence b's decision (wave 0, then shared), adds the
// residual (or bonus) mass of entries [2048 c, 2048 c + 2048) -- each thread a run of 8 inside
// one contract chunk -- and publishes it. The last block of the sequence to finish (a counter
// cleared by the row-totals kernel, bumped after a device-scope fence) then runs the inverse
// CDF: wave 0 finds the 2048-entry block whose inclusive mass crosses the target (64 blocks per
// scan window, carry between windows); each thread sums its run of that block (values held in
// registers), a block-wide exclusive scan of the runs gives every thread its starting prefix,
// and the thread whose run crosses reports the first crossing entry (atomicMin over the block).
// The same block writes the sequence's outputs.
template <typename TT>
__global__ __launch_bounds__(THREADS) void rej_sample_kernel(RejArgs a) {
  const int b = (int)blockIdx.y, c = (int)blockIdx.x;
  const int K = a.K, T = K + 1;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __shared__ Decision s_dec;
  __shared__ u192 sh[THREADS / 64];
  __shared__ int s_last;
  __shared__ int s_chunk;
  __shared__ u192 s_before;
  __shared__ u192 s_target;
  __shared__ u192 s_wtot[THREADS / 64];
  __shared__ int s_tok;
  __shared__ int s_empty;
  __shared__ ArgPart s_best[THREADS / 64];
  if (w == 0) {
    const Decision d = decide(a, b);
    if (lane == 0) s_dec = d;
  }
  __syncthreads();
  const Decision d = s_dec;
  {
    const int v0 = c * MCHK + (int)threadIdx.x * PER_M;
    u192 m{0, 0, 0};
    if (v0 < a.V) {
      const SampleRow<TT> s = sample_row<TT>(a, b, d, v0 / CC);
      m = run_mass(s, load_run(a, s, v0), v0, a.V, a.inv_temp);
    }
    m = block_sum_u192(m, sh);
    if (threadIdx.x == 0) {
      a.cmass[(size_t)b * a.nchm + c] = m;
      __threadfence();  // the mass is visible device-wide before the count says so
      s_last = atomicAdd(&a.cnt[b], 1u) == (unsigned)(a.nchm - 1);
    }
    __syncthreads();
  }
  if (!s_last) return;
  __threadfence();  // every other block's mass, published before its count, is visible
  const u192* cm = a.cmass + (size_t)b * a.nchm;
  if (w == 0) {
    u192 tot{0, 0, 0};
    for (int k = lane; k < a.nchm; k += 64) tot = add192(tot, cm[k]);
    tot = wave_incl_scan_u192(tot);
    tot = shfl_u192(tot, 63);
    if (lane == 0) s_empty = is_zero192(tot);
    const u192 target = mul192x32(tot, uniform_fix(a.u_sample[b]));  // need 2^24 C > target
    u192 carry{0, 0, 0};
    int chunk = a.nchm - 1;
    u192 before{0, 0, 0};
    bool found = false;
    for (int c0 = 0; c0 < a.nchm && !found; c0 += 64) {
      const int k = c0 + lane;
      const u192 m = k < a.nchm ? cm[k] : u192{0, 0, 0};
      const u192 incl = add192(wave_incl_scan_u192(m), carry);
      const uint64_t hit =
          __builtin_amdgcn_ballot_w64(k < a.nchm && gt192(shl24_192(incl), target));
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
  const int acc = d.acc;
  int tok;
  if (s_empty) {
    // No sampling mass: every weight of the sampling row is 0, which happens only for a
    // bonus row whose logits are all NaN or -inf or include +inf, or for the residual after
    // an out-of-range draft id where Wp Zq == Wq Zp everywhere (a residual after a failed
    // test always has mass). The token is then the target row's greedy choice: its argmax,
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
    ArgPart best = s_best[0];
    for (int k = 1; k < THREADS / 64; ++k)
      if (beats(s_best[k].v, s_best[k].i, best.v, best.i)) best = s_best[k];
    tok = best.i;
  } else {
    const int chunk = s_chunk;
    const int v0 = chunk * MCHK + (int)threadIdx.x * PER_M;
    RunVals rv;
    u192 run{0, 0, 0};
    SampleRow<TT> s;
    if (v0 < a.V) {
      s = sample_row<TT>(a, b, d, v0 / CC);
      rv = load_run(a, s, v0);
      run = run_mass(s, rv, v0, a.V, a.inv_temp);
    }
    const u192 incl = wave_incl_scan_u192(run);
    if (lane == 63) s_wtot[w] = incl;
    __syncthreads();
    u192 cpre = add192(s_before, sub192(incl, run));
    for (int k = 0; k < w; ++k) cpre = add192(cpre, s_wtot[k]);
    const u192 target = s_target;
    if (v0 < a.V && gt192(shl24_192(add192(cpre, run)), target)) {  // crossing in this run
#pragma unroll
      for (int j = 0; j < PER_M; ++j) {
        const int v = v0 + j;
        if (v >= a.V) break;
        const u192 wv = weight_of(s, rv.p[j], rv.q[j], a.inv_temp);
        cpre = add192(cpre, wv);
        if (!is_zero192(wv) && gt192(shl24_192(cpre), target)) {
          atomicMin(&s_tok, v);
          break;
        }
      }
    }
    __syncthreads();
    tok = s_tok;
  }
  if (threadIdx.x == 0) a.accepted[b] = acc;
  for (int t = (int)threadIdx.x; t < T; t += THREADS) {
    int64_t id = -1;
    if (t < acc) id = a.draft_ids[(size_t)b * K + t];
    else if (t == acc) id = tok;
    a.out_ids[(size_t)b * T + t] = id;
  }
}

// Workspace of the acceptance calls. The per-row Z sums come first and the row maxima second:
// the header documents both as results that the rejection call leaves in the workspace.
struct WsLayout {
  size_t zrow, mrow, wtok, cmax, csum, cmass, cnt, total;
};

WsLayout layout(int B, int K, int V) {
  const int nc = (V + CC - 1) / CC;
  const int nch = (V + CHK - 1) / CHK;
  const size_t rows = (size_t)B * (2 * K + 1);
  auto up = [](size_t x) { return (x + 255) & ~size_t(255); };
  WsLayout l{};
  size_t o = 0;
  l.zrow = o; o += up(rows * sizeof(u128));
  l.mrow = o; o += up(rows * sizeof(float));
  l.wtok = o; o += up(rows * sizeof(uint64_t));
  // chunk maxima; the greedy path's argmax partials share the region
  const size_t cmax_bytes = rows * nc * sizeof(float);
  const size_t part_bytes = (size_t)B * (K + 1) * nch * sizeof(ArgPart);
  l.cmax = o; o += up(cmax_bytes > part_bytes ? cmax_bytes : part_bytes);
  l.csum = o; o += up(rows * nc * sizeof(uint64_t));
  l.cmass = o; o += up((size_t)B * ((V + MCHK - 1) / MCHK) * sizeof(u192));
  l.cnt = o; o += up((size_t)B * sizeof(uint32_t));
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
  ArgPart* part = reinterpret_cast<ArgPart*>(static_cast<uint8_t*>(workspace) + l.cmax);
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
  // Z <= V 2^62 <= 2^82 and every residual sum at most 2^164 for V <= 2^20, so the
  // contract's products stay below 2^192
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
                 accepted, out_ids, B, K, V, (V + CC - 1) / CC, (V + MCHK - 1) / MCHK, vec4,
                 reinterpret_cast<u128*>(ws + l.zrow), reinterpret_cast<float*>(ws + l.mrow),
                 reinterpret_cast<uint64_t*>(ws + l.wtok), reinterpret_cast<float*>(ws + l.cmax),
                 reinterpret_cast<uint64_t*>(ws + l.csum), reinterpret_cast<u192*>(ws + l.cmass),
                 reinterpret_cast<uint32_t*>(ws + l.cnt)};
}

// Chunk statistics of `rows` fp32 rows starting at row0.
void launch_stats(const RejArgs& a, int row0, int rows, hipStream_t s) {
  const dim3 grid((a.V + SBLK - 1) / SBLK, rows);
  if (a.inv_temp == 1.0f)
    hipLaunchKernelGGL(rej_stats_kernel<true>, grid, dim3(THREADS), 0, s, a, row0);
  else
    hipLaunchKernelGGL(rej_stats_kernel<false>, grid, dim3(THREADS), 0, s, a, row0);
}

// Row totals and sampling (every row's chunk statistics in place). TT is the target rows'
// element type: float, or bf16 bits (uint16_t) for the LM-head form.
template <typename TT>
int launch_decide_sample(const RejArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(rej_rowtotal_kernel<TT>, dim3(a.B * (2 * a.K + 1)), dim3(THREADS), 0, s, a);
  hipLaunchKernelGGL(rej_sample_kernel<TT>, dim3(a.nchm, a.B), dim3(THREADS), 0, s, a);
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
  launch_stats(a, 0, B * (2 * K + 1), s);
  return launch_decide_sample<float>(a, s);
}

// ---- no-allocation variant -------------------------------------------------------------------
// The workspace of npn_accept_rejection_noalloc: a fixed device array. Each GPU holds its own
// copy, at its own address, for the life of the process. In host code `scratch` names a host
// stand-in, not device memory: kernels get the address hipGetSymbolAddress returns for the
// device they run on (scratch_on_device), never the array's name. Nothing in it needs clearing
// between calls: every word a call reads was written earlier in the same call (the counters of
// the sampling kernel are cleared by the row-totals kernel before it).
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
extern "C" size_t npn_accept_rejection_lm_head_workspace_size(int B, int K, int H, int V) {
  if (!shape_ok(B, K, V) || V > kRejMaxV) return 0;
  if (!npn::fp8_matmul_chunk_stats_ok(B * (K + 1), H, V)) return 0;  // GEMM shape rules
  return layout(B, K, V).total;
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
  const RejArgs a = rej_args(target_logits, draft_logits, draft_ids, u_accept, u_sample,
                             inv_temperature, accepted, out_ids, B, K, V, true,
                             static_cast<uint8_t*>(workspace));
  launch_stats(a, M, B * K, s);  // draft rows
  const int gst = npn::fp8_matmul_chunk_stats(hidden, lm_head_w, lm_head_scale, target_logits,
                                              a.cmax, a.csum, inv_temperature, M, H, V, s);
  if (gst != NPN_OK) return gst;
  return launch_decide_sample<uint16_t>(a, s);
}
