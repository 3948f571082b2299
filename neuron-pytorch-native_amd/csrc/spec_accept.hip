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

constexpr int CHK = 8192;      // vocabulary entries per chunk
constexpr int THREADS = 256;   // CHK / THREADS = 32 entries per thread
constexpr int PER_T = CHK / THREADS;

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
                                                                int V, int nch) {
  const int row = blockIdx.y, c = blockIdx.x;
  const float* src = logits + (size_t)row * V;
  const int v0 = c * CHK;
  float bv = -INFINITY;
  int bi = 0x7FFFFFFF;
  for (int j = 0; j < PER_T; ++j) {
    const int v = v0 + j * THREADS + threadIdx.x;
    if (v < V) {
      const float x = src[v];
      if (beats(x, v, bv, bi)) { bv = x; bi = v; }
    }
  }
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
  int B, K, V, nch;
  // workspace
  float* rmax;        // [rows][nch]   rows = B*(K+1) target rows, then B*K draft rows
  uint64_t* zsum;     // [rows][nch]
  uint64_t* ex;       // [rows]        E at the row's draft token (target/draft rows i < K)
  int32_t* dec_row;   // [B]           sampling row index (target row; draft row or -1)
  uint64_t* dec_z;    // [B][2]        Zp, Zq of the sampling rows
  u128* cmass;        // [B][nch]
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
  for (int j = 0; j < PER_T; ++j) {
    const int v = v0 + j * THREADS + threadIdx.x;
    if (v < a.V) m = fmaxf(m, scaled(src[v], a.inv_temp));
  }
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
  for (int j = 0; j < PER_T; ++j) {
    const int v = v0 + j * THREADS + threadIdx.x;
    if (v < a.V) z += expfix(scaled(src[v], a.inv_temp) - m);
  }
  __shared__ uint64_t sh[THREADS / 64];
  z = block_sum_u64(z, sh);
  if (threadIdx.x == 0) {
    a.zsum[(size_t)row * a.nch + c] = z;
    const int x = row_token(a, row);
    if (x >= v0 && x < v0 + CHK) a.ex[row] = expfix(scaled(src[x], a.inv_temp) - m);
  }
}

__device__ __forceinline__ uint64_t row_z(const RejArgs& a, int row) {
  uint64_t z = 0;
  for (int c = 0; c < a.nch; ++c) z += a.zsum[(size_t)row * a.nch + c];
  return z;
}

// One thread per sequence: the K accept tests, then which rows to sample from.
__global__ void rej_decide_kernel(RejArgs a) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= a.B) return;
  const int K = a.K, T = K + 1;
  const int nt = a.B * T;
  int acc = K;
  uint64_t zp_s = 0, zq_s = 0;
  for (int i = 0; i < K; ++i) {
    const int rt = b * T + i, rd = nt + b * K + i;
    const uint64_t zp = row_z(a, rt), zq = row_z(a, rd);
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
  if (acc == K) zp_s = row_z(a, b * T + K);
  a.accepted[b] = acc;
  a.dec_row[b] = acc;
  a.dec_z[2 * b] = zp_s;
  a.dec_z[2 * b + 1] = zq_s;
  for (int t = 0; t < T; ++t) {
    if (t < acc) a.out_ids[(size_t)b * T + t] = a.draft_ids[(size_t)b * K + t];
    else if (t > acc) a.out_ids[(size_t)b * T + t] = -1;
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
  s.mp = row_max(a, rt);
  s.zp = a.dec_z[2 * b];
  s.zq = a.dec_z[2 * b + 1];
  if (acc < K) {
    const int rd = a.B * T + b * K + acc;
    s.q = a.draft + (size_t)(b * K + acc) * a.V;
    s.mq = row_max(a, rd);
  } else {
    s.q = nullptr;
    s.mq = 0.f;
  }
  return s;
}

__device__ __forceinline__ u128 weight(const SampleRow& s, int v, float inv_temp) {
  const uint64_t ep = expfix(scaled(s.p[v], inv_temp) - s.mp);
  if (s.q == nullptr) return ep;
  const uint64_t eq = expfix(scaled(s.q[v], inv_temp) - s.mq);
  const u128 x = (u128)ep * s.zq, y = (u128)eq * s.zp;
  return x > y ? x - y : 0;
}

__global__ __launch_bounds__(THREADS) void rej_mass_kernel(RejArgs a) {
  const int b = blockIdx.y, c = blockIdx.x;
  const SampleRow s = sample_row(a, b);
  const int v0 = c * CHK;
  u128 m = 0;
  for (int j = 0; j < PER_T; ++j) {
    const int v = v0 + j * THREADS + threadIdx.x;
    if (v < a.V) m += weight(s, v, a.inv_temp);
  }
  __shared__ u128 sh[THREADS / 64];
  m = block_sum_u128(m, sh);
  if (threadIdx.x == 0) a.cmass[(size_t)b * a.nch + c] = m;
}

// Inverse CDF: chunk by chunk on the chunk masses, then inside the chosen chunk with a
// block-wide exclusive scan over per-thread runs of PER_T consecutive entries.
__global__ __launch_bounds__(THREADS) void rej_pick_kernel(RejArgs a) {
  const int b = blockIdx.x;
  const SampleRow s = sample_row(a, b);
  __shared__ int s_chunk;
  __shared__ u128 s_before;
  __shared__ u128 s_target;
  __shared__ u128 s_run[THREADS];
  __shared__ int s_tok;
  if (threadIdx.x == 0) {
    u128 total = 0;
    for (int c = 0; c < a.nch; ++c) total += a.cmass[(size_t)b * a.nch + c];
    const u128 target = (u128)uniform_fix(a.u_sample[b]) * total;  // need 2^24 * C > target
    u128 before = 0;
    int chunk = a.nch - 1;
    for (int c = 0; c < a.nch; ++c) {
      const u128 m = a.cmass[(size_t)b * a.nch + c];
      if (((before + m) << 24) > target) { chunk = c; break; }
      before += m;
    }
    s_chunk = chunk;
    s_before = before;
    s_target = target;
    s_tok = 0x7FFFFFFF;
  }
  __syncthreads();
  const int v0 = s_chunk * CHK + threadIdx.x * PER_T;
  u128 run = 0;
  for (int j = 0; j < PER_T; ++j) {
    const int v = v0 + j;
    if (v < a.V) run += weight(s, v, a.inv_temp);
  }
  s_run[threadIdx.x] = run;
  __syncthreads();
  if (threadIdx.x == 0) {  // sequential exclusive scan of the 256 run sums (exact integers)
    u128 acc = s_before;
    for (int t = 0; t < THREADS; ++t) {
      const u128 r = s_run[t];
      s_run[t] = acc;
      acc += r;
    }
  }
  __syncthreads();
  u128 c = s_run[threadIdx.x];
  for (int j = 0; j < PER_T; ++j) {
    const int v = v0 + j;
    if (v >= a.V) break;
    const u128 wv = weight(s, v, a.inv_temp);
    c += wv;
    if (wv != 0 && (c << 24) > s_target) {
      atomicMin(&s_tok, v);  // first crossing in this run; lowest v over the block
      break;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const int T = a.K + 1;
    a.out_ids[(size_t)b * T + a.dec_row[b]] = s_tok;
  }
}

struct WsLayout {
  size_t rmax, zsum, ex, dec_row, dec_z, cmass, total;
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
  l.cmass = o; o += up((size_t)B * nch * sizeof(u128));
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
  hipLaunchKernelGGL(argmax_chunk_kernel, dim3(nch, B * (K + 1)), dim3(THREADS), 0, s,
                     target_logits, part, V, nch);
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
  RejArgs a{target_logits, draft_logits, draft_ids, u_accept, u_sample, inv_temperature,
            accepted, out_ids, B, K, V, nch,
            reinterpret_cast<float*>(ws + l.rmax), reinterpret_cast<uint64_t*>(ws + l.zsum),
            reinterpret_cast<uint64_t*>(ws + l.ex), reinterpret_cast<int32_t*>(ws + l.dec_row),
            reinterpret_cast<uint64_t*>(ws + l.dec_z), reinterpret_cast<u128*>(ws + l.cmass)};
  const int rows = B * (2 * K + 1);
  hipLaunchKernelGGL(rej_max_kernel, dim3(nch, rows), dim3(THREADS), 0, s, a);
  hipLaunchKernelGGL(rej_sum_kernel, dim3(nch, rows), dim3(THREADS), 0, s, a);
  hipLaunchKernelGGL(rej_decide_kernel, dim3((B + 63) / 64), dim3(64), 0, s, a);
  hipLaunchKernelGGL(rej_mass_kernel, dim3(nch, B), dim3(THREADS), 0, s, a);
  hipLaunchKernelGGL(rej_pick_kernel, dim3(B), dim3(THREADS), 0, s, a);
  return npn_launch_status();
}
