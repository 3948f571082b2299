// Speculative-decode acceptance on gfx950: greedy and rejection sampling.
//
// Greedy (the reference's on-device argmax, contrib/qwen3.6-27b/static_decode.py:1313, with
// the exact sharded top-1 order of contrib/qwen3.6-35b-a3b/static_decode_35b.py:1532-1570):
//   tid[b,t] = argmax_v target[b,t,v], first index on ties, NaN counts as the maximum;
//   accepted a_b = number of leading drafts equal to tid[b, position before them].
//
// Rejection sampling (Leviathan et al. 2023, Alg. 1) under an integer softmax contract
// that this file and its CPU restatement evaluate with identical IEEE-754 operations:
//   s_v = t_v * inv_temp (fp32); m = max_v s_v; E_v = floor(2^32 * exp_c(s_v - m)) where
//   exp_c is a Cody-Waite reduction + degree-7 Taylor polynomial evaluated with separately
//   rounded fp32 multiplies and adds (this file is compiled with -ffp-contract=off);
//   Z = sum_v E_v in 64-bit integers (exact, so the reduction order does not matter).
//   Accept draft x at position i iff U * Eq_x * Zp <= 2^24 * Ep_x * Zq (128-bit integers,
//   U = floor(u * 2^24)). At the first rejection sample from R_v = max(0, Ep_v Zq - Eq_v Zp),
//   after K acceptances from R_v = Ep_v of the bonus row: the token is the smallest v with
//   2^24 * sum_{w<=v} R_w > U_s * sum_w R_w.
//
// Kernels (each over B sequences, T = K+1 positions, vocabulary split into 8192-wide chunks):
//   greedy:    argmax partials per (row, chunk) -> per-sequence merge + accept
//   rejection: row max partials -> E sums per (row, chunk) and E at the draft token ->
//              per-sequence decision -> residual/bonus mass per (sequence, chunk) ->
//              per-sequence inverse-CDF pick
#include "npn_common.h"

namespace {

constexpr int CHK = 8192;      // vocabulary entries per chunk (logit passes)
constexpr int THREADS = 256;   // CHK / THREADS = 32 entries per thread
constexpr int PER_T = CHK / THREADS;
constexpr int MCHK = 2048;     // entries per chunk of the residual mass / inverse-CDF pass
constexpr int PER_M = MCHK / THREADS;  // 8 consecutive entries per thread

typedef unsigned __int128 u128;

// ---- exp contract (must match oracle.accept.expfix bit for bit) -------------------------
constexpr float kL2E = 0x1.715476p+0f;        // log2(e) in fp32
constexpr float kLn2Hi = 0x1.62ep-1f;         // ln2, low 12 mantissa bits cleared
constexpr float kLn2Lo = 0x1.0bfbe8p-15f;     // ln2 - kLn2Hi in fp32
constexpr float kC7 = 0x1.a01a02p-13f;        // 1/7!
constexpr float kC6 = 0x1.6c16c2p-10f;        // 1/6!
constexpr float kC5 = 0x1.111112p-7f;         // 1/5!
constexpr float kC4 = 0x1.555556p-5f;         // 1/4!
constexpr float kC3 = 0x1.555556p-3f;         // 1/3!
constexpr float kXMin = -32.0f;               // below: 2^32 exp(x) < 1

__device__ __forceinline__ uint64_t expfix(float x) {
#pragma clang fp contract(off)
  if (!(x > kXMin)) return 0;
  const float kf = floorf(x * kL2E + 0.5f);
  float r = x - kf * kLn2Hi;
  r = r - kf * kLn2Lo;
  float p = kC7;
  p = p * r + kC6;
  p = p * r + kC5;
  p = p * r + kC4;
  p = p * r + kC3;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  const uint32_t bits = __float_as_uint(p);
  const int e = (int)((bits >> 23) & 0xFFu);
  const uint64_t m = (uint64_t)((bits & 0x7FFFFFu) | 0x800000u);
  const int shift = e + (int)kf - 118;
  if (shift >= 0) return m << shift;
  const int rs = -shift;
  return rs >= 64 ? 0 : (m >> rs);
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
  if (vec4) {
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
  const float* target;   // [B][K+1][V]
  const float* draft;    // [B][K][V]
  const int64_t* draft_ids;
  const float* u_accept;
  const float* u_sample;
  float inv_temp;
  int32_t* accepted;
  int64_t* out_ids;
  int B, K, V, nch, nchm;  // chunks of CHK (logit passes) and of MCHK (mass / pick)
  bool vec4;          // logit rows 16-byte aligned and V % 4 == 0
  // workspace
  float* rmax;        // [rows][nch]   rows = B*(K+1) target rows, then B*K draft rows
  uint64_t* zsum;     // [rows][nch]
  uint64_t* ex;       // [rows]        E at the row's draft token (target/draft rows i < K)
  int32_t* dec_row;   // [B]           sampling row index (target row; draft row or -1)
  uint64_t* dec_z;    // [B][2]        Zp, Zq of the sampling rows
  float* dec_m;       // [B][2]        row maxima of the sampling rows (scaled logits)
  u128* cmass;        // [B][nchm]
};

__device__ __forceinline__ const float* row_ptr(const RejArgs& a, int row) {
  const int nt = a.B * (a.K + 1);
  return row < nt ? a.target + (size_t)row * a.V : a.draft + (size_t)(row - nt) * a.V;
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

__global__ __launch_bounds__(THREADS) void rej_max_kernel(RejArgs a) {
  const int row = blockIdx.y, c = blockIdx.x;
  const float* src = row_ptr(a, row);
  const int v0 = c * CHK;
  float m = -INFINITY;
  visit_chunk(src, v0, a.V, a.vec4, [&](int, float x) { m = fmaxf(m, scaled(x, a.inv_temp)); });
  __shared__ float sh[THREADS / 64];
  m = block_max(m, sh);
  if (threadIdx.x == 0) a.rmax[(size_t)row * a.nch + c] = m;
}

__device__ __forceinline__ float row_max(const RejArgs& a, int row) {
  float m = a.rmax[(size_t)row * a.nch];
  for (int c = 1; c < a.nch; ++c) m = fmaxf(m, a.rmax[(size_t)row * a.nch + c]);
  return m;
}

__global__ __launch_bounds__(THREADS) void rej_sum_kernel(RejArgs a) {
  const int row = blockIdx.y, c = blockIdx.x;
  const float* src = row_ptr(a, row);
  const float m = row_max(a, row);
  const int v0 = c * CHK;
  uint64_t z = 0;
  visit_chunk(src, v0, a.V, a.vec4,
              [&](int, float x) { z += expfix(scaled(x, a.inv_temp) - m); });
  __shared__ uint64_t sh[THREADS / 64];
  z = block_sum_u64(z, sh);
  if (threadIdx.x == 0) {
    a.zsum[(size_t)row * a.nch + c] = z;
    const int x = row_token(a, row);
    if (x >= v0 && x < v0 + CHK) a.ex[row] = expfix(scaled(src[x], a.inv_temp) - m);
  }
}

// One workgroup per sequence: the Z sums of its 2K+1 rows (chunk partials added in LDS with
// exact 64-bit atomics, so the order does not matter), the K accept tests, then which rows
// to sample from, with their Z sums and maxima for the mass and pick kernels.
__global__ __launch_bounds__(THREADS) void rej_decide_kernel(RejArgs a) {
  const int b = blockIdx.x;
  const int K = a.K, T = K + 1;
  const int nt = a.B * T;
  const int nrows = 2 * K + 1;  // local row r: target row r (r <= K), draft row r - T
  __shared__ unsigned long long zs[2 * 64 + 1];
  __shared__ int s_acc;
  __shared__ float shm[THREADS / 64];
  for (int r = threadIdx.x; r < nrows; r += THREADS) zs[r] = 0;
  __syncthreads();
  for (int p = threadIdx.x; p < nrows * a.nch; p += THREADS) {
    const int r = p / a.nch, c = p - r * a.nch;
    const int row = r <= K ? b * T + r : nt + b * K + (r - T);
    atomicAdd(&zs[r], (unsigned long long)a.zsum[(size_t)row * a.nch + c]);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int acc = K;
    uint64_t zp_s = 0, zq_s = 0;
    for (int i = 0; i < K; ++i) {
      const int rt = b * T + i, rd = nt + b * K + i;
      const uint64_t zp = zs[i], zq = zs[T + i];
      const uint64_t ep = a.ex[rt], eq = a.ex[rd];
      const u128 lhs = (u128)uniform_fix(a.u_accept[(size_t)b * K + i]) * eq * zp;
      const u128 rhs = ((u128)ep * zq) << 24;
      if (lhs > rhs) {
        acc = i;
        zp_s = zp;
        zq_s = zq;
        break;
      }
    }
    if (acc == K) zp_s = zs[K];
    a.accepted[b] = acc;
    a.dec_row[b] = acc;
    a.dec_z[2 * b] = zp_s;
    a.dec_z[2 * b + 1] = zq_s;
    for (int t = 0; t < T; ++t) {
      if (t < acc) a.out_ids[(size_t)b * T + t] = a.draft_ids[(size_t)b * K + t];
      else if (t > acc) a.out_ids[(size_t)b * T + t] = -1;
    }
    s_acc = acc;
  }
  __syncthreads();
  const int acc = s_acc;
  // maxima of the sampling rows (the draft row only after a rejection)
  const int rows[2] = {b * T + acc, nt + b * K + acc};
  for (int k = 0; k < (acc < K ? 2 : 1); ++k) {
    float m = -INFINITY;
    for (int c = threadIdx.x; c < a.nch; c += THREADS)
      m = fmaxf(m, a.rmax[(size_t)rows[k] * a.nch + c]);
    m = block_max(m, shm);
    if (threadIdx.x == 0) a.dec_m[2 * b + k] = m;
  }
}

// Sampling weight of vocabulary entry v for sequence b (residual or bonus).
struct SampleRow {
  const float* p;
  const float* q;  // nullptr for the bonus row
  float mp, mq;
  uint64_t zp, zq;
};

__device__ __forceinline__ SampleRow sample_row(const RejArgs& a, int b) {
  const int K = a.K, T = K + 1;
  const int acc = a.dec_row[b];
  SampleRow s;
  const int rt = b * T + acc;
  s.p = a.target + (size_t)rt * a.V;
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

__device__ __forceinline__ u128 weight_of(const SampleRow& s, float pv, float qv,
                                          float inv_temp) {
  const uint64_t ep = expfix(scaled(pv, inv_temp) - s.mp);
  if (s.q == nullptr) return ep;
  const uint64_t eq = expfix(scaled(qv, inv_temp) - s.mq);
  const u128 x = (u128)ep * s.zq, y = (u128)eq * s.zp;
  return x > y ? x - y : 0;
}


// This thread's PER_M consecutive sampling-row entries starting at v0 (p, and q after a
// rejection), loaded once; entries at or past V read as p = q = -inf (weight 0 is not
// used for them: callers stop at V).
struct RunVals {
  float p[PER_M], q[PER_M];
};

__device__ __forceinline__ RunVals load_run(const RejArgs& a, const SampleRow& s, int v0) {
  RunVals r;
  if (a.vec4 && v0 + PER_M <= a.V) {
#pragma unroll
    for (int j = 0; j < PER_M; j += 4) {
      const float4 pv = *reinterpret_cast<const float4*>(s.p + v0 + j);
      r.p[j] = pv.x; r.p[j + 1] = pv.y; r.p[j + 2] = pv.z; r.p[j + 3] = pv.w;
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
      r.p[j] = v < a.V ? s.p[v] : -INFINITY;
      r.q[j] = (v < a.V && s.q != nullptr) ? s.q[v] : 0.f;
    }
  }
  return r;
}

__global__ __launch_bounds__(THREADS) void rej_mass_kernel(RejArgs a) {
  const int b = blockIdx.y, c = blockIdx.x;
  const SampleRow s = sample_row(a, b);
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
__global__ __launch_bounds__(THREADS) void rej_pick_kernel(RejArgs a) {
  const int b = blockIdx.x;
  const SampleRow s = sample_row(a, b);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __shared__ int s_chunk;
  __shared__ u128 s_before;
  __shared__ u128 s_target;
  __shared__ u128 s_wtot[THREADS / 64];
  __shared__ int s_tok;
  const u128* cm = a.cmass + (size_t)b * a.nchm;
  if (w == 0) {
    u128 tot = 0;
    for (int c = lane; c < a.nchm; c += 64) tot += cm[c];
    tot = wave_incl_scan_u128(tot);
    tot = shfl_u128(tot, 63);
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

struct WsLayout {
  size_t rmax, zsum, ex, dec_row, dec_z, dec_m, cmass, total;
};

WsLayout layout(int B, int K, int V) {
  const int nch = (V + CHK - 1) / CHK;
  const size_t rows = (size_t)B * (2 * K + 1);
  auto up = [](size_t x) { return (x + 255) & ~size_t(255); };
  WsLayout l{};
  size_t o = 0;
  l.rmax = o; o += up(rows * nch * sizeof(float) > (size_t)B * (K + 1) * nch * sizeof(ArgPart)
                          ? rows * nch * sizeof(float)
                          : (size_t)B * (K + 1) * nch * sizeof(ArgPart));
  l.zsum = o; o += up(rows * nch * sizeof(uint64_t));
  l.ex = o; o += up(rows * sizeof(uint64_t));
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

extern "C" int npn_accept_rejection(const float* target_logits, const float* draft_logits,
                                    const int64_t* draft_ids, const float* u_accept,
                                    const float* u_sample, float inv_temperature,
                                    int32_t* accepted, int64_t* out_ids, int B, int K, int V,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  NPN_REQUIRE(target_logits && draft_logits && draft_ids && u_accept && u_sample && accepted &&
                  out_ids,
              NPN_ERR_NULL);
  NPN_REQUIRE(shape_ok(B, K, V), NPN_ERR_SHAPE);
  NPN_REQUIRE(inv_temperature > 0.0f && inv_temperature < 1e30f, NPN_ERR_VALUE);
  const WsLayout l = layout(B, K, V);
  NPN_REQUIRE(workspace != nullptr && workspace_bytes >= l.total, NPN_ERR_WORKSPACE);
  NPN_REQUIRE(NPN_ALIGNED16(workspace), NPN_ERR_ALIGN);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const int nch = (V + CHK - 1) / CHK;
  const bool vec4 = V % 4 == 0 && NPN_ALIGNED16(target_logits) && NPN_ALIGNED16(draft_logits);
  RejArgs a{target_logits, draft_logits, draft_ids, u_accept, u_sample, inv_temperature,
            accepted, out_ids, B, K, V, nch, (V + MCHK - 1) / MCHK, vec4,
            reinterpret_cast<float*>(ws + l.rmax), reinterpret_cast<uint64_t*>(ws + l.zsum),
            reinterpret_cast<uint64_t*>(ws + l.ex), reinterpret_cast<int32_t*>(ws + l.dec_row),
            reinterpret_cast<uint64_t*>(ws + l.dec_z), reinterpret_cast<float*>(ws + l.dec_m),
            reinterpret_cast<u128*>(ws + l.cmass)};
  const int rows = B * (2 * K + 1);
  hipLaunchKernelGGL(rej_max_kernel, dim3(nch, rows), dim3(THREADS), 0, s, a);
  hipLaunchKernelGGL(rej_sum_kernel, dim3(nch, rows), dim3(THREADS), 0, s, a);
  hipLaunchKernelGGL(rej_decide_kernel, dim3(B), dim3(THREADS), 0, s, a);
  hipLaunchKernelGGL(rej_mass_kernel, dim3(a.nchm, B), dim3(THREADS), 0, s, a);
  hipLaunchKernelGGL(rej_pick_kernel, dim3(B), dim3(THREADS), 0, s, a);
  return npn_launch_status();
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
