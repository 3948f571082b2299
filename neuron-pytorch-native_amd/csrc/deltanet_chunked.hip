// Chunked gated-DeltaNet prefill on gfx950: the op deltanet::chunked_prefill
// (contrib/qwen3.6-27b/kernels/deltanet_chunked_ops.py:26-42, kernel
// contrib/qwen3.6-27b/kernels/deltanet_chunked_v2.py:46-105).
//
// Per head h (rows h*S + t of q, k, v, g, beta), with q, k L2-normalised inside as
// x * rsqrt(sum x^2 + 1e-6) and q scaled by 1/sqrt(128), over chunks of CH = 64 tokens:
//   g_cum = cumsum(g); dm[a, b] = exp(g_cum[a] - g_cum[b]) for a >= b
//   A = -(beta k) k^T * dm (strictly lower); T = (I - A)^-1
//   v_new = T (beta * (v - (e^g_cum k) S))          [= T(beta v) - T(beta e^g k) S]
//   out = (e^g_cum q) S + ((q k^T) * dm, lower incl. diagonal) v_new
//   S <- e^g_cum[-1] S + (k * e^(g_cum[-1] - g_cum))^T v_new
// The reference takes the chunk size from its [C, C] constants and builds T with a doubling
// product; here the chunk is 64 whatever C is (the result is the same up to rounding) and T
// is formed by blocked forward substitution, which stays finite where the doubling product
// does not (contrib/qwen3.6-27b/kernels/tests/test_doubling_pad_stability.py:1-19). A last
// partial chunk is padded with beta = g = 0 tokens (no effect on the state; outputs not
// written).
//
// Two kernels:
// - dn_chunk_prep_kernel, one workgroup per (chunk, head), all chunks at once: everything that
//   does not depend on the state -- the per-token scales (row norms folded with e^g_cum), A,
//   T and the intra-chunk attention -- into a workspace record per (head, chunk).
// - dn_chunk_scan_kernel, one workgroup per (head, 32-column block of V), chunk after chunk:
//   only the products with the state. The columns of the state evolve independently, so the
//   4 blocks of a head run side by side, each holding its 128 x 32 block (transposed) in LDS.
//   The 4 workgroups of a head are placed on one XCD so that they share its L2 for the
//   head's q, k and records.
//
// All products are 16 x 16 fp32 MFMA tiles (v_mfma_f32_16x16x4f32: lane l = 16 g + c supplies
// A[c][k] and B[k][c] for the k of its group g; acc[r] is D[4 g + r][c]). In a tile over K,
// group g takes k in [g K/4, (g + 1) K/4), so each lane reads row c of A and row c of B^T four
// values at a time (float4 LDS reads). In the blocked inverse the output of one product feeds
// the next as its B operand directly, with k = 4 g + r at step r.
#include "npn_common.h"

namespace {

constexpr int CH = 64;                  // tokens per chunk
constexpr int D = 128;                  // k and v head dims
constexpr int NCB = 4;                  // 32-column blocks of V per head
constexpr int RS = D + 4;               // LDS row stride of q, k and S^T (float4 rows)
constexpr int MS = CH + 4;              // LDS row stride of A, T, intra and the [32][64] blocks
constexpr float kNormEps = 1e-6f;
constexpr float kQScale = 0.08838834764831845f;  // 1/sqrt(128)

// Workspace record per (head, chunk), in floats (a multiple of 64: 256-byte aligned records).
constexpr int REC_T = 0;                 // T [64][64] row-major, zero above the diagonal
constexpr int REC_I = CH * CH;           // intra [64][64], zero above the diagonal
constexpr int REC_SC = 2 * CH * CH;      // [64] x {sq, sk1, sk2, beta}
constexpr int REC_ET = REC_SC + 4 * CH;  // e^(sum of the chunk's g)
constexpr int REC = REC_ET + 64;
// sq_i  = rsqrt(|q_i|^2 + eps) e^g_cum_i / sqrt(128)   scales row i of (raw q) S
// sk1_i = rsqrt(|k_i|^2 + eps) e^g_cum_i               scales row i of (raw k) S
// sk2_i = rsqrt(|k_i|^2 + eps) e^(g_cum_63 - g_cum_i)  weight of raw k_i in the state update

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float4 ld4(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}
__device__ __forceinline__ void st4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }
__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// acc += A (16 x K) B (K x 16) with pa = &A[c][0] and pb = &B^T[c][0] (k contiguous in both).
template <int K>
__device__ __forceinline__ void tile16(f32x4& acc, const float* pa, const float* pb) {
  const int k0 = ((threadIdx.x >> 4) & 3) * (K / 4);
#pragma unroll
  for (int u = 0; u < K / 16; ++u) {
    const float4 a = ld4(pa + k0 + 4 * u), b = ld4(pb + k0 + 4 * u);
    acc = mfma16(a.x, b.x, acc);
    acc = mfma16(a.y, b.y, acc);
    acc = mfma16(a.z, b.z, acc);
    acc = mfma16(a.w, b.w, acc);
  }
}

// The 10 lower 16 x 16 blocks (I >= J) of a 64 x 64 matrix, t = I (I + 1) / 2 + J.
__device__ __forceinline__ void lower_block(int t, int& I, int& J) {
  I = t < 1 ? 0 : t < 3 ? 1 : t < 6 ? 2 : 3;
  J = t - I * (I + 1) / 2;
}

// ---- stage 1: per (chunk, head), independent of the state -----------------------------------

struct PrepArgs {
  const float* q;
  const float* k;
  const float* g;
  const float* beta;
  float* ws;
  int S;
  int nch;
};

struct PrepSmem {
  union {
    float q[CH * RS];                    // raw q rows, until the intra blocks are done
    struct {
      float a[CH * MS];                  // A
      float t[CH * MS];                  // T's diagonal blocks
    } at;
  } u;
  float k[CH * RS];                      // raw k rows
  float gcum[CH], bt[CH], rq[CH], rk[CH];
};

__global__ __launch_bounds__(256, 2) void dn_chunk_prep_kernel(PrepArgs a) {
  __shared__ __attribute__((aligned(16))) PrepSmem sm;
  const int ci = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, c = lane & 15;
  const int S = a.S, t0 = ci * CH;
  const size_t row0 = (size_t)h * S;
  float* rec = a.ws + ((size_t)h * a.nch + ci) * REC;

  // raw q, k rows (zero past the end of the prompt); g_cum by a wave scan
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = 8 * j + (tid >> 5), c4 = tid & 31;
    const bool ok = t0 + i < S;
    const size_t r = ok ? row0 + t0 + i : row0;
    const float4 qv = reinterpret_cast<const float4*>(a.q + r * D)[c4];
    const float4 kv = reinterpret_cast<const float4*>(a.k + r * D)[c4];
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    st4(sm.u.q + i * RS + 4 * c4, ok ? qv : z4);
    st4(sm.k + i * RS + 4 * c4, ok ? kv : z4);
  }
  if (wv == 0) {
    const bool ok = t0 + lane < S;
    const size_t r = ok ? row0 + t0 + lane : row0;
    const float gv = a.g[r], bv = a.beta[r];
    float gi = ok ? gv : 0.f;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float o = __shfl_up(gi, d, 64);
      if (lane >= d) gi += o;
    }
    sm.gcum[lane] = gi;
    sm.bt[lane] = ok ? bv : 0.f;
  }
  __syncthreads();
  {  // row norms, 4 threads per row
    const int i = tid >> 2, part = tid & 3;
    const float* qp = sm.u.q + i * RS + 32 * part;
    const float* kp = sm.k + i * RS + 32 * part;
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int j = 0; j < 32; j += 4) {
      const float4 x = ld4(qp + j), y = ld4(kp + j);
      sq += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
      sk += y.x * y.x + y.y * y.y + y.z * y.z + y.w * y.w;
    }
    sq += __shfl_xor(sq, 1, 64);
    sq += __shfl_xor(sq, 2, 64);
    sk += __shfl_xor(sk, 1, 64);
    sk += __shfl_xor(sk, 2, 64);
    if (part == 0) {
      sm.rq[i] = rsqrtf(sq + kNormEps);
      sm.rk[i] = rsqrtf(sk + kNormEps);
    }
  }
  __syncthreads();
  if (wv == 0) {
    const float gi = sm.gcum[lane], tot = sm.gcum[CH - 1], rk = sm.rk[lane];
    st4(rec + REC_SC + 4 * lane, make_float4(sm.rq[lane] * kQScale * __expf(gi), rk * __expf(gi),
                                             rk * __expf(tot - gi), sm.bt[lane]));
    if (lane == 0) rec[REC_ET] = __expf(tot);
  }
  if (wv >= 2) {  // the blocks above the diagonal of T and intra are zero
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int e = tid - 128; e < 6 * 64; e += 128) {
      const int b = e >> 6, row = (e >> 2) & 15, c4 = e & 3;
      const int I = b < 3 ? 0 : b < 5 ? 1 : 2, J = b < 3 ? b + 1 : b < 5 ? b - 1 : 3;
      const int off = (16 * I + row) * CH + 16 * J + 4 * c4;
      st4(rec + REC_T + off, z4);
      st4(rec + REC_I + off, z4);
    }
  }
  // intra[i][j] = (q_i . k_j) rq_i rk_j / sqrt(128) dm(i, j) for i >= j
  for (int t = wv; t < 10; t += 4) {
    int I, J;
    lower_block(t, I, J);
    f32x4 acc = zero4();
    tile16<D>(acc, sm.u.q + (16 * I + c) * RS, sm.k + (16 * J + c) * RS);
    const int j = 16 * J + c;
    const float rkj = sm.rk[j], gj = sm.gcum[j];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * I + 4 * g4 + r;
      rec[REC_I + i * CH + j] =
          i >= j ? sm.rq[i] * kQScale * rkj * acc[r] * __expf(sm.gcum[i] - gj) : 0.f;
    }
  }
  __syncthreads();  // the q rows are consumed: A and T take their place
  // A[i][j] = -beta_i (k_i . k_j) rk_i rk_j dm(i, j) for i > j
  for (int t = wv; t < 10; t += 4) {
    int I, J;
    lower_block(t, I, J);
    f32x4 acc = zero4();
    tile16<D>(acc, sm.k + (16 * I + c) * RS, sm.k + (16 * J + c) * RS);
    const int j = 16 * J + c;
    const float rkj = sm.rk[j], gj = sm.gcum[j];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * I + 4 * g4 + r;
      sm.u.at.a[i * MS + j] =
          i > j ? -sm.bt[i] * sm.rk[i] * rkj * acc[r] * __expf(sm.gcum[i] - gj) : 0.f;
    }
  }
  __syncthreads();
  if (wv == 0) {
    // T's diagonal blocks by forward substitution, lane 16 b + j holding column j of block b:
    // T_bb[i][j] = sum_{m < i} A_bb[i][m] T_bb[m][j] for i > j (A_bb is zero on and above
    // its diagonal, so the row reads may run past m = i - 1)
    const int b = g4, j = c;
    const float* ab = sm.u.at.a + 16 * b * MS + 16 * b;
    float col[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) col[m] = m == j ? 1.f : 0.f;
#pragma unroll
    for (int i = 1; i < 16; ++i) {
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int m4 = 0; m4 < i; m4 += 4) {
        const float4 av = ld4(ab + i * MS + m4);
        s0 += av.x * col[m4] + av.z * col[m4 + 2];
        s1 += av.y * col[m4 + 1] + av.w * col[m4 + 3];
      }
      if (i > j) col[i] = s0 + s1;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      sm.u.at.t[(16 * b + i) * MS + 16 * b + j] = col[i];
      rec[REC_T + (16 * b + i) * CH + 16 * b + j] = col[i];
    }
  }
  __syncthreads();
  if (wv < 3) {
    // block column Jb = wave: T_IJ = T_II sum_{M = J}^{I - 1} A_IM T_MJ for I > J; each T_MJ
    // stays in registers (acc layout) as the B operand of the next block row
    const int Jb = wv;
    const float* am = sm.u.at.a;
    const float* tm = sm.u.at.t;
    f32x4 tj[4];
#pragma unroll
    for (int M = 0; M < 3; ++M) {
      tj[M] = zero4();
      if (M == Jb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) tj[M][r] = tm[(16 * M + 4 * g4 + r) * MS + 16 * M + c];
      }
    }
#pragma unroll
    for (int I = 1; I < 4; ++I) {
      if (I <= Jb) continue;
      f32x4 R = zero4();
#pragma unroll
      for (int M = 0; M < 3; ++M) {
        if (M < Jb || M >= I) continue;
        const float4 av = ld4(am + (16 * I + c) * MS + 16 * M + 4 * g4);
        R = mfma16(av.x, tj[M][0], R);
        R = mfma16(av.y, tj[M][1], R);
        R = mfma16(av.z, tj[M][2], R);
        R = mfma16(av.w, tj[M][3], R);
      }
      const float4 tv = ld4(tm + (16 * I + c) * MS + 16 * I + 4 * g4);
      f32x4 X = zero4();
      X = mfma16(tv.x, R[0], X);
      X = mfma16(tv.y, R[1], X);
      X = mfma16(tv.z, R[2], X);
      X = mfma16(tv.w, R[3], X);
      tj[I] = X;
#pragma unroll
      for (int r = 0; r < 4; ++r) rec[REC_T + (16 * I + 4 * g4 + r) * CH + 16 * Jb + c] = X[r];
    }
  }
}

// ---- stage 2: per (head, column block), chunk after chunk -----------------------------------

struct ScanArgs {
  const float* state;
  const float* q;
  const float* k;
  const float* v;
  const float* ws;
  float* out;
  float* new_state;
  int S;
  int nch;
  int Hv;
};

struct ScanSmem {
  float q[CH * RS];      // raw q rows of the chunk
  float k[CH * RS];      // raw k rows
  float t[CH * MS];      // T
  float in[CH * MS];     // intra
  float sT[32 * RS];     // the state block, transposed: [column][k index]
  float zT[32 * MS];     // v^T of the chunk, then Z^T
  float vnT[32 * MS];    // v_new^T
  float vsT[32 * MS];    // (sk2 v_new)^T
  float4 sc[CH];         // sq, sk1, sk2, beta
  float etot;
};

// Wave roles: column half J = wave & 1 and the row blocks {I1, I2} = {0, 3} (waves 0, 1) or
// {1, 2} (waves 2, 3), which balances the triangular products.

// X = (raw k) S and O = (raw q) S for the wave's rows; Z = beta (v - sk1 X) into zT; O *= sq.
template <int I1, int I2>
__device__ __forceinline__ void scan_state_products(ScanSmem& sm, int J, f32x4& o1, f32x4& o2) {
  const int lane = threadIdx.x & 63, g4 = lane >> 4, c = lane & 15;
  f32x4 x1 = zero4(), x2 = zero4();
  o1 = zero4();
  o2 = zero4();
  const float* pb = sm.sT + (16 * J + c) * RS + 32 * g4;
  const float* pk1 = sm.k + (16 * I1 + c) * RS + 32 * g4;
  const float* pk2 = sm.k + (16 * I2 + c) * RS + 32 * g4;
  const float* pq1 = sm.q + (16 * I1 + c) * RS + 32 * g4;
  const float* pq2 = sm.q + (16 * I2 + c) * RS + 32 * g4;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const float4 b = ld4(pb + 4 * u), k1 = ld4(pk1 + 4 * u), k2 = ld4(pk2 + 4 * u),
                 q1 = ld4(pq1 + 4 * u), q2 = ld4(pq2 + 4 * u);
    x1 = mfma16(k1.x, b.x, x1); x2 = mfma16(k2.x, b.x, x2);
    o1 = mfma16(q1.x, b.x, o1); o2 = mfma16(q2.x, b.x, o2);
    x1 = mfma16(k1.y, b.y, x1); x2 = mfma16(k2.y, b.y, x2);
    o1 = mfma16(q1.y, b.y, o1); o2 = mfma16(q2.y, b.y, o2);
    x1 = mfma16(k1.z, b.z, x1); x2 = mfma16(k2.z, b.z, x2);
    o1 = mfma16(q1.z, b.z, o1); o2 = mfma16(q2.z, b.z, o2);
    x1 = mfma16(k1.w, b.w, x1); x2 = mfma16(k2.w, b.w, x2);
    o1 = mfma16(q1.w, b.w, o1); o2 = mfma16(q2.w, b.w, o2);
  }
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int i0 = 16 * (p == 0 ? I1 : I2) + 4 * g4;
    const f32x4& x = p == 0 ? x1 : x2;
    f32x4& o = p == 0 ? o1 : o2;
    float* zp = sm.zT + (16 * J + c) * MS + i0;
    const float4 v = ld4(zp);
    const float4 s0 = sm.sc[i0], s1 = sm.sc[i0 + 1], s2 = sm.sc[i0 + 2], s3 = sm.sc[i0 + 3];
    st4(zp, make_float4(s0.w * (v.x - s0.y * x[0]), s1.w * (v.y - s1.y * x[1]),
                        s2.w * (v.z - s2.y * x[2]), s3.w * (v.w - s3.y * x[3])));
    o[0] *= s0.x;
    o[1] *= s1.x;
    o[2] *= s2.x;
    o[3] *= s3.x;
  }
}

// v_new rows of block I = T Z (K = 16 (I + 1): T is lower triangular) into vnT and vsT.
template <int I>
__device__ __forceinline__ void scan_vnew(ScanSmem& sm, int J) {
  const int lane = threadIdx.x & 63, g4 = lane >> 4, c = lane & 15;
  f32x4 acc = zero4();
  tile16<16 * (I + 1)>(acc, sm.t + (16 * I + c) * MS, sm.zT + (16 * J + c) * MS);
  const int i0 = 16 * I + 4 * g4, o = (16 * J + c) * MS + i0;
  st4(sm.vnT + o, make_float4(acc[0], acc[1], acc[2], acc[3]));
  st4(sm.vsT + o, make_float4(acc[0] * sm.sc[i0].z, acc[1] * sm.sc[i0 + 1].z,
                              acc[2] * sm.sc[i0 + 2].z, acc[3] * sm.sc[i0 + 3].z));
}

// out rows of block I = O + intra v_new, written where the token exists.
template <int I>
__device__ __forceinline__ void scan_out(ScanSmem& sm, float* orow, int J, f32x4 o, int nvalid) {
  const int lane = threadIdx.x & 63, g4 = lane >> 4, c = lane & 15;
  tile16<16 * (I + 1)>(o, sm.in + (16 * I + c) * MS, sm.vnT + (16 * J + c) * MS);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = 16 * I + 4 * g4 + r;
    if (i < nvalid) orow[(size_t)i * D + 16 * J + c] = o[r];
  }
}

// S'^T[col][kk] = e^tot S^T[col][kk] + sum_i (sk2 v_new)^T[col][i] k[i][kk], for the wave's
// column half and the four 16-blocks of kk from P0; in place (each element is read and
// written by one lane).
__device__ __forceinline__ void scan_state_update(ScanSmem& sm, int J, int P0) {
  const int lane = threadIdx.x & 63, g4 = lane >> 4, c = lane & 15;
  const float et = sm.etot;
  f32x4 s[4];
#pragma unroll
  for (int p = 0; p < 4; ++p)
#pragma unroll
    for (int r = 0; r < 4; ++r) s[p][r] = et * sm.sT[(16 * J + 4 * g4 + r) * RS + 16 * (P0 + p) + c];
  const float* va = sm.vsT + (16 * J + c) * MS + 16 * g4;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const float4 av = ld4(va + 4 * u);
    const float* kr = sm.k + (16 * g4 + 4 * u) * RS + 16 * P0 + c;
    const float ae[4] = {av.x, av.y, av.z, av.w};
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int p = 0; p < 4; ++p) s[p] = mfma16(ae[e], kr[e * RS + 16 * p], s[p]);
  }
#pragma unroll
  for (int p = 0; p < 4; ++p)
#pragma unroll
    for (int r = 0; r < 4; ++r) sm.sT[(16 * J + 4 * g4 + r) * RS + 16 * (P0 + p) + c] = s[p][r];
}

__global__ __launch_bounds__(256, 1) void dn_chunk_scan_kernel(ScanArgs a) {
  __shared__ __attribute__((aligned(16))) ScanSmem sm;
  // workgroup L runs on XCD L % 8: the 4 column blocks of head h all get XCD h % 8
  const int L = blockIdx.x, grp = L / (8 * NCB), rem = L % (8 * NCB);
  const int cb = rem >> 3, h = 8 * grp + (rem & 7);
  if (h >= a.Hv) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int J = wv & 1;
  const int S = a.S;
  const size_t row0 = (size_t)h * S;
  const int c0 = 32 * cb;

  for (int e = tid; e < D * 32; e += 256) {
    const int kk = e >> 5, cc = e & 31;
    sm.sT[cc * RS + kk] = a.state[((size_t)h * D + kk) * D + c0 + cc];
  }
  // The next chunk's inputs, loaded into registers while the current chunk computes: q, k rows
  // (rows 8j + (tid >> 5), float4 column tid & 31), this block's v columns (row tid >> 2,
  // columns 8 (tid & 3) .. +7), the record's T and intra (float4 tid + 256 j) and scales.
  float4 pq[8], pk[8], pv[2], pt[4], pi[4];
  float4 psc = make_float4(0.f, 0.f, 0.f, 0.f);
  float pet = 0.f;
  auto fetch = [&](int ci) {
    const int t0 = ci * CH;
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = 8 * j + (tid >> 5), c4 = tid & 31;
      const bool ok = t0 + i < S;
      const size_t r = ok ? row0 + t0 + i : row0;
      const float4 qv = reinterpret_cast<const float4*>(a.q + r * D)[c4];
      const float4 kv = reinterpret_cast<const float4*>(a.k + r * D)[c4];
      pq[j] = ok ? qv : z4;
      pk[j] = ok ? kv : z4;
    }
    {
      const int i = tid >> 2;
      const bool ok = t0 + i < S;
      const size_t r = ok ? row0 + t0 + i : row0;
      const float4* src = reinterpret_cast<const float4*>(a.v + r * D + c0 + 8 * (tid & 3));
      const float4 v0 = src[0], v1 = src[1];
      pv[0] = ok ? v0 : z4;
      pv[1] = ok ? v1 : z4;
    }
    const float* rec = a.ws + ((size_t)h * a.nch + ci) * REC;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pt[j] = reinterpret_cast<const float4*>(rec + REC_T)[tid + 256 * j];
      pi[j] = reinterpret_cast<const float4*>(rec + REC_I)[tid + 256 * j];
    }
    if (wv == 0) {
      psc = reinterpret_cast<const float4*>(rec + REC_SC)[lane];
      pet = rec[REC_ET];
    }
  };
  fetch(0);
  f32x4 o1, o2;
  for (int ci = 0; ci < a.nch; ++ci) {
    const int t0 = ci * CH;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = 8 * j + (tid >> 5), c4 = tid & 31;
      st4(sm.q + i * RS + 4 * c4, pq[j]);
      st4(sm.k + i * RS + 4 * c4, pk[j]);
    }
    {
      float* zd = sm.zT + 8 * (tid & 3) * MS + (tid >> 2);
      zd[0] = pv[0].x; zd[MS] = pv[0].y; zd[2 * MS] = pv[0].z; zd[3 * MS] = pv[0].w;
      zd[4 * MS] = pv[1].x; zd[5 * MS] = pv[1].y; zd[6 * MS] = pv[1].z; zd[7 * MS] = pv[1].w;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = tid + 256 * j, r = e >> 4, c4 = e & 15;
      st4(sm.t + r * MS + 4 * c4, pt[j]);
      st4(sm.in + r * MS + 4 * c4, pi[j]);
    }
    if (wv == 0) {
      sm.sc[lane] = psc;
      if (lane == 0) sm.etot = pet;
    }
    if (ci + 1 < a.nch) fetch(ci + 1);  // in flight during this chunk's work
    __syncthreads();
    if (wv < 2) scan_state_products<0, 3>(sm, J, o1, o2);
    else scan_state_products<1, 2>(sm, J, o1, o2);
    __syncthreads();
    if (wv < 2) {
      scan_vnew<0>(sm, J);
      scan_vnew<3>(sm, J);
    } else {
      scan_vnew<1>(sm, J);
      scan_vnew<2>(sm, J);
    }
    __syncthreads();
    const int nvalid = min(CH, S - t0);
    float* orow = a.out + (row0 + t0) * D + c0;
    if (wv < 2) {
      scan_out<0>(sm, orow, J, o1, nvalid);
      scan_out<3>(sm, orow, J, o2, nvalid);
    } else {
      scan_out<1>(sm, orow, J, o1, nvalid);
      scan_out<2>(sm, orow, J, o2, nvalid);
    }
    scan_state_update(sm, J, 4 * (wv >> 1));
  }
  __syncthreads();
  for (int e = tid; e < D * 32; e += 256) {
    const int kk = e >> 5, cc = e & 31;
    a.new_state[((size_t)h * D + kk) * D + c0 + cc] = sm.sT[cc * RS + kk];
  }
}

bool shape_ok(int v_heads, int S) {
  return v_heads >= 1 && v_heads <= 65535 && S >= 1 && (long)v_heads * S <= (1L << 26);
}

}  // namespace

extern "C" size_t npn_deltanet_chunked_workspace_size(int v_heads, int S) {
  if (!shape_ok(v_heads, S)) return 0;
  return (size_t)v_heads * ((S + CH - 1) / CH) * REC * sizeof(float);
}

extern "C" int npn_deltanet_chunked_prefill(const float* state, const float* query,
                                            const float* key, const float* value, const float* g,
                                            const float* beta, float* out, float* new_state,
                                            int v_heads, int S, void* workspace,
                                            size_t workspace_bytes, void* stream) {
  NPN_REQUIRE(state && query && key && value && g && beta && out && new_state, NPN_ERR_NULL);
  NPN_REQUIRE(shape_ok(v_heads, S), NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(state) && NPN_ALIGNED16(query) && NPN_ALIGNED16(key) &&
                  NPN_ALIGNED16(value) && NPN_ALIGNED16(out) && NPN_ALIGNED16(new_state) &&
                  NPN_ALIGNED16(workspace),
              NPN_ERR_ALIGN);
  NPN_REQUIRE(workspace && workspace_bytes >= npn_deltanet_chunked_workspace_size(v_heads, S),
              NPN_ERR_WORKSPACE);
  const int nch = (S + CH - 1) / CH;
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* ws = static_cast<float*>(workspace);
  hipLaunchKernelGGL(dn_chunk_prep_kernel, dim3(nch, v_heads), dim3(256), 0, st,
                     PrepArgs{query, key, g, beta, ws, S, nch});
  const int groups = (v_heads + 7) / 8;
  hipLaunchKernelGGL(dn_chunk_scan_kernel, dim3(groups * 8 * NCB), dim3(256), 0, st,
                     ScanArgs{state, query, key, value, ws, out, new_state, S, nch, v_heads});
  return npn_launch_status();
}
