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
// - dn_chunk_prep_kernel, persistent workgroups over all (head, chunk) items at once:
//   everything that does not depend on the state -- the per-token scales (row norms folded
//   with e^g_cum), A, T and the intra-chunk attention -- into a workspace record per item.
// - dn_chunk_scan_kernel, one workgroup of 8 waves per (head, 32-column block of V), chunk
//   after chunk: only the products with the state. The columns of the state evolve
//   independently, so the 4 blocks of a head run side by side, each holding its 128 x 32
//   block in registers (and its split in LDS). The 4 workgroups of a head are placed on one
//   XCD so that they share its L2 for the head's q, k and records.
//
// Products. Matrix products over the 128 k indices or the 64 tokens of a chunk take split
// operands: x = hi + lo with hi = bf16(x), lo = bf16(x - hi), and a product of two split
// values is hi*hi + hi*lo + lo*hi in bf16 MFMAs (v_mfma_f32_16x16x32_bf16) accumulating in fp32;
// the dropped lo*lo term and lo's rounding leave about 2^-16 relative per product, and the
// results stay within 2e-5 of the float64 rule after 64 chunks. In a 16 x 16 tile lane
// l = 16 g + c supplies A[c][k] and B[k][c] for the 8 consecutive k of its group g per
// instruction, so each lane reads 16-byte rows of A and of B^T; acc[r] is D[4 g + r][c]. The
// triangular inverse stays in fp32 (v_mfma_f32_16x16x4f32 and VALU): in the blocked inverse
// the output of one product feeds the next as its B operand directly, with k = 4 g + r at
// step r.
#include "npn_common.h"

namespace {

constexpr int CH = 64;                  // tokens per chunk
constexpr int D = 128;                  // k and v head dims
constexpr int NCB = 4;                  // 32-column blocks of V per head
constexpr int MS = CH + 4;              // LDS row stride of the prep's fp32 A and T
constexpr float kNormEps = 1e-6f;
constexpr float kQScale = 0.08838834764831845f;  // 1/sqrt(128)

// Workspace record per (head, chunk), in floats (a multiple of 64: 256-byte aligned records).
constexpr int REC_T = 0;                 // T [64][64] row-major, zero above the diagonal: bf16 hi
                                         // then bf16 lo (T = hi + lo)
constexpr int REC_I = CH * CH;           // intra [64][64], zero above the diagonal, split alike
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

// Raw buffer reads: one instruction per float4 with a per-lane byte offset, and reads at or
// past `bytes` (checked on the per-lane offset) return zeros, which pads a last partial chunk.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}
__device__ __forceinline__ float4 bload4(rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// Split operands: x = hi + lo with hi = bf16(x), lo = bf16(x - hi), and a product of two
// split values as hi*hi + hi*lo + lo*hi in bf16 MFMAs accumulating in fp32 (the dropped
// lo*lo term and lo's rounding leave about 2^-16 relative per product).
typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef __bf16 bf16x4 __attribute__((__vector_size__(4 * sizeof(__bf16))));
typedef short s16x4 __attribute__((ext_vector_type(4)));

constexpr int RB = D + 8;    // LDS row stride (bf16) of the split S^T rows (scan) and q, k rows
                             // (prep): 272 bytes
constexpr int VB = CH + 8;   // ... of the split 64-wide rows (T, intra, Z^T, v_new^T): 144 bytes

__device__ __forceinline__ f32x4 mfma3(bf16x8 ah, bf16x8 al, bf16x8 bh, bf16x8 bl, f32x4 c) {
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, c, 0, 0, 0);
  return c;
}
__device__ __forceinline__ void split4(float4 x, bf16x4& h, bf16x4& l) {
  h[0] = (__bf16)x.x;
  h[1] = (__bf16)x.y;
  h[2] = (__bf16)x.z;
  h[3] = (__bf16)x.w;
  l[0] = (__bf16)(x.x - (float)h[0]);
  l[1] = (__bf16)(x.y - (float)h[1]);
  l[2] = (__bf16)(x.z - (float)h[2]);
  l[3] = (__bf16)(x.w - (float)h[3]);
}
__device__ __forceinline__ bf16x8 ld8(const __bf16* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}
// ds_read_tr16_b64: in each group of 16 lanes, lane i addresses 4 consecutive 16-bit values
// of row (i >> 2) of a 4 x 16 block (columns 4 (i & 3) .. + 3) and receives column i of the
// block's 4 rows.
__device__ __forceinline__ s16x4 lds_tr16(const __bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
}
__device__ __forceinline__ bf16x8 pack8(s16x4 a, s16x4 b) {
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  const s16x8 v = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  return __builtin_bit_cast(bf16x8, v);
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
  int items;   // Hv * nch, item = h * nch + chunk
};

struct PrepSmem {
  union {
    struct {
      __bf16 h[CH * RB], l[CH * RB];     // q rows split, until the intra blocks are done
    } q;
    struct {
      float a[CH * MS];                  // A
      float t[CH * MS];                  // T's diagonal blocks
    } at;
  } u;
  __bf16 kh[CH * RB], kl[CH * RB];       // k rows split
  float gcum[CH], bt[CH], rq[CH], rk[CH];
};

// A 16 x 16 block over the 128 k indices from split operands: ah = &A_hi[row c][8 g], al, and
// bh / bl the same for B^T (rows of both are k-contiguous); step st covers k = 32 st + 8 g ..
// + 7. Operands are read two steps at a time (32 VGPRs live).
__device__ __forceinline__ f32x4 tile_split128(const __bf16* ah, const __bf16* al,
                                               const __bf16* bh, const __bf16* bl) {
  f32x4 acc = zero4();
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    bf16x8 x[2][4];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int d = 64 * hh + 32 * u;
      x[u][0] = ld8(ah + d);
      x[u][1] = ld8(al + d);
      x[u][2] = ld8(bh + d);
      x[u][3] = ld8(bl + d);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 2; ++u) acc = mfma3(x[u][0], x[u][1], x[u][2], x[u][3], acc);
  }
  return acc;
}

// Persistent: each workgroup takes items blockIdx.x, + gridDim.x, ..., with the next item's q, k
// rows, g and beta read into registers while the current one computes.
__global__ __launch_bounds__(256, 2) void dn_chunk_prep_kernel(PrepArgs a) {
  __shared__ __attribute__((aligned(16))) PrepSmem sm;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, c = lane & 15;
  const int S = a.S;
  // raw q, k rows 8j + (tid >> 5), float4 column tid & 31; g and beta of token lane (wave 0);
  // reads past the end of the prompt return zeros
  const int qk_off = (tid >> 5) * (D * 4) + (tid & 31) * 16;
  float4 pq[8], pk[8];
  float pg = 0.f, pb = 0.f;
  // half 0: rows 0..31 of q and k; half 1: rows 32..63, g and beta
  auto fetch = [&](int item, int half) {
    const int h = item / a.nch, t0 = (item - h * a.nch) * CH;
    const size_t r0 = (size_t)h * S + t0;
    const int rest = S - t0;
    const rsrc_t rq = make_rsrc(a.q + r0 * D, rest * D * 4);
    const rsrc_t rk = make_rsrc(a.k + r0 * D, rest * D * 4);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if ((j >> 2) != half) continue;
      pq[j] = bload4(rq, qk_off + 4096 * j, 0);
      pk[j] = bload4(rk, qk_off + 4096 * j, 0);
    }
    if (half == 1 && wv == 0) {
      pg = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                         make_rsrc(a.g + r0, rest * 4), lane * 4, 0, 0));
      pb = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                         make_rsrc(a.beta + r0, rest * 4), lane * 4, 0, 0));
    }
  };
  if ((int)blockIdx.x < a.items) {
    fetch(blockIdx.x, 0);
    fetch(blockIdx.x, 1);
  }
  for (int item = blockIdx.x; item < a.items; item += gridDim.x) {
    const int h = item / a.nch, ci = item - h * a.nch;
    float* rec = a.ws + ((size_t)h * a.nch + ci) * REC;
    __bf16* rth = reinterpret_cast<__bf16*>(rec + REC_T);   // T hi [64][64], then lo
    __bf16* rih = reinterpret_cast<__bf16*>(rec + REC_I);   // intra hi, then lo
    __syncthreads();  // the previous item is done with LDS
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int o = (8 * j + (tid >> 5)) * RB + 4 * (tid & 31);
      bf16x4 hh, ll;
      split4(pq[j], hh, ll);
      *reinterpret_cast<bf16x4*>(sm.u.q.h + o) = hh;
      *reinterpret_cast<bf16x4*>(sm.u.q.l + o) = ll;
      split4(pk[j], hh, ll);
      *reinterpret_cast<bf16x4*>(sm.kh + o) = hh;
      *reinterpret_cast<bf16x4*>(sm.kl + o) = ll;
    }
    if (wv == 0) {  // g_cum by a wave scan
      float gi = pg;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const float o = __shfl_up(gi, d, 64);
        if (lane >= d) gi += o;
      }
      sm.gcum[lane] = gi;
      sm.bt[lane] = pb;
    }
    // the next item's reads, in two halves (unconditional, so that no branch forces an early
    // wait: the last item reads itself again)
    const int nx = min(item + (int)gridDim.x, a.items - 1);
    fetch(nx, 0);
    __syncthreads();
    {  // row norms from the split rows (hi + lo is x to 2^-17), 4 threads per row
      const int i = tid >> 2, part = tid & 3;
      float sq = 0.f, sk = 0.f;
#pragma unroll
      for (int j = 0; j < 32; j += 8) {
        const int o = i * RB + 32 * part + j;
        const bf16x8 qh = ld8(sm.u.q.h + o), ql = ld8(sm.u.q.l + o), kh = ld8(sm.kh + o),
                     kl = ld8(sm.kl + o);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = (float)qh[e] + (float)ql[e], y = (float)kh[e] + (float)kl[e];
          sq += x * x;
          sk += y * y;
        }
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
      st4(rec + REC_SC + 4 * lane,
          make_float4(sm.rq[lane] * kQScale * __expf(gi), rk * __expf(gi), rk * __expf(tot - gi),
                      sm.bt[lane]));
      if (lane == 0) rec[REC_ET] = __expf(tot);
    }
    if (wv >= 2) {  // the blocks above the diagonal of T and intra are zero (hi and lo)
      const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int e = tid - 128; e < 2 * 6 * 32; e += 128) {
        const int half = e / 192, f = e % 192, b = f >> 5, row = (f >> 1) & 15, c8 = f & 1;
        const int I = b < 3 ? 0 : b < 5 ? 1 : 2, J = b < 3 ? b + 1 : b < 5 ? b - 1 : 3;
        const int off = half * CH * CH + (16 * I + row) * CH + 16 * J + 8 * c8;
        *reinterpret_cast<float4*>(rth + off) = z4;
        *reinterpret_cast<float4*>(rih + off) = z4;
      }
    }
    // intra[i][j] = (q_i . k_j) rq_i rk_j / sqrt(128) dm(i, j) for i >= j, written split
    for (int t = wv; t < 10; t += 4) {
      int I, J;
      lower_block(t, I, J);
      const int ao = (16 * I + c) * RB + 8 * g4, bo = (16 * J + c) * RB + 8 * g4;
      const f32x4 acc = tile_split128(sm.u.q.h + ao, sm.u.q.l + ao, sm.kh + bo, sm.kl + bo);
      const int j = 16 * J + c;
      const float rkj = sm.rk[j], gj = sm.gcum[j];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * I + 4 * g4 + r;
        const float x =
            i >= j ? sm.rq[i] * kQScale * rkj * acc[r] * __expf(sm.gcum[i] - gj) : 0.f;
        const __bf16 hb = (__bf16)x;
        rih[i * CH + j] = hb;
        rih[CH * CH + i * CH + j] = (__bf16)(x - (float)hb);
      }
    }
    fetch(nx, 1);
    __syncthreads();  // the q rows are consumed: A and T take their place
    // A[i][j] = -beta_i (k_i . k_j) rk_i rk_j dm(i, j) for i > j
    for (int t = wv; t < 10; t += 4) {
      int I, J;
      lower_block(t, I, J);
      const int ao = (16 * I + c) * RB + 8 * g4, bo = (16 * J + c) * RB + 8 * g4;
      const f32x4 acc = tile_split128(sm.kh + ao, sm.kl + ao, sm.kh + bo, sm.kl + bo);
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
        const int o = (16 * b + i) * CH + 16 * b + j;
        const __bf16 hb = (__bf16)col[i];
        rth[o] = hb;
        rth[CH * CH + o] = (__bf16)(col[i] - (float)hb);
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
        for (int r = 0; r < 4; ++r) {
          const int o = (16 * I + 4 * g4 + r) * CH + 16 * Jb + c;
          const __bf16 hb = (__bf16)X[r];
          rth[o] = hb;
          rth[CH * CH + o] = (__bf16)(X[r] - (float)hb);
        }
      }
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

// The scan's q and k rows: 128 bf16 (256 bytes) per row, 16-byte chunk m of row r stored at
// chunk m ^ f(r), f(r) = 2 (r & 3) + ((r >> 2) & 1). Eight consecutive rows then put a chunk on
// 8 distinct LDS bank groups (the row reads of the state products), and 4 rows from a
// multiple of 4 put a pair of chunks on 8 distinct ones (the transposed column reads of the
// state update); a plain padded stride serves one pattern or the other.
__device__ __forceinline__ int qk_idx(int r, int e) {
  return r * D + (((e >> 3) ^ (2 * (r & 3) + ((r >> 2) & 1))) << 3) + (e & 7);
}

constexpr int VS = 32 + 4;   // LDS row stride (fp32) of the block's v rows: 144 bytes
constexpr int ZB = 32 + 16;  // LDS row stride (bf16) of the split Z rows: 96 bytes, so that a
                             // transposed read's 4 rows fall on distinct banks

struct ScanSmem {
  __bf16 qh[CH * D], ql[CH * D];      // q rows of the chunk, split (qk_idx layout)
  __bf16 kh[CH * D], kl[CH * D];      // k rows, split (qk_idx layout)
  __bf16 sh[32 * RB], sl[32 * RB];    // the state block transposed ([column][k index]), split
  __bf16 th[CH * VB], tl[CH * VB];    // T, split (as the record holds it)
  __bf16 ih[CH * VB], il[CH * VB];    // intra, split
  __bf16 zh[CH * ZB], zl[CH * ZB];    // Z rows ([token][column]), split
  __bf16 nh[32 * VB], nl[32 * VB];    // v_new^T, split
  __bf16 vsh[32 * VB], vsl[32 * VB];  // (sk2 v_new)^T, split
  float vr[CH * VS];                  // v rows of the chunk, the block's 32 columns (fp32)
  float4 sc[CH];                      // sq, sk1, sk2, beta
  float etot;
};

// Wave w of the 8 owns row block I of the chunk and column half J = w & 1 of the block's 32
// state columns: I = 3 - ((w >> 1) & 1) for w < 4, (w >> 1) & 1 for w >= 4. Waves w and w + 4
// share a SIMD, so each SIMD holds row blocks {3, 0} or {2, 1}: the triangular products
// (T Z, intra v_new) are balanced per SIMD, and its two waves cover each other's waits. The
// older wave, which wins the SIMD's issue arbitration, takes the longer triangular chain.
// The wave also owns the state tiles S[16 (P0 + p) .. + 15][16 J .. + 15] of the block's 32
// columns (p = 0, 1; P0 = 2 ((w >> 1) & 3)) in fp32 registers for the whole prompt.

// Pa: X = (raw k) S and O = (raw q) S for rows of block I (split products over the 128 k
// indices, step st covering 32 st + 8 g .. + 7 for lane group g), formed as transposed tiles
// (S^T as the A operand) so that x[r], o[r] hold token 16 I + c, column 16 J + 4 g + r: a
// lane's v row, scales, Z and out are then one 16-byte access each. Z = beta (v - sk1 X),
// split into zh / zl; O *= sq. pre(st) issues part of the next chunk's reads between the
// products.
template <typename Pre>
__device__ __forceinline__ void scan_state_products(ScanSmem& sm, int I, int J, f32x4& o,
                                                    Pre&& pre) {
  const int lane = threadIdx.x & 63, g4 = lane >> 4, c = lane & 15;
  f32x4 x = zero4();
  o = zero4();
  const int rr = 16 * I + c, so = (16 * J + c) * RB + 8 * g4;
  int ro = qk_idx(rr, 8 * g4);
  bf16x8 nkh = ld8(sm.kh + ro), nkl = ld8(sm.kl + ro), nqh = ld8(sm.qh + ro),
         nql = ld8(sm.ql + ro), nsh = ld8(sm.sh + so), nsl = ld8(sm.sl + so);
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    const bf16x8 kh = nkh, kl = nkl, qh = nqh, ql = nql, sh = nsh, sl = nsl;
    if (st < 3) {
      const int d = 32 * (st + 1);
      ro = qk_idx(rr, d + 8 * g4);
      nkh = ld8(sm.kh + ro);
      nkl = ld8(sm.kl + ro);
      nqh = ld8(sm.qh + ro);
      nql = ld8(sm.ql + ro);
      nsh = ld8(sm.sh + so + d);
      nsl = ld8(sm.sl + so + d);
    }
    pre(st);
    __builtin_amdgcn_sched_barrier(0);
    x = mfma3(sh, sl, kh, kl, x);
    o = mfma3(sh, sl, qh, ql, o);
  }
  const int i = 16 * I + c, zo = i * ZB + 16 * J + 4 * g4;
  const float4 v = ld4(sm.vr + i * VS + 16 * J + 4 * g4);
  const float4 sc = sm.sc[i];
  bf16x4 zh, zl;
  split4(make_float4(sc.w * (v.x - sc.y * x[0]), sc.w * (v.y - sc.y * x[1]),
                     sc.w * (v.z - sc.y * x[2]), sc.w * (v.w - sc.y * x[3])),
         zh, zl);
  *reinterpret_cast<bf16x4*>(sm.zh + zo) = zh;
  *reinterpret_cast<bf16x4*>(sm.zl + zo) = zl;
  o *= sc.x;
}

// acc += T Z for rows of block I over the tokens below 32 ceil((I + 1) / 2) (T is zero above
// its diagonal, so the rounding up adds zero products), step st covering tokens 32 st + 8 g ..
// + 7: T's rows as the A operand, Z's columns read transposed from its rows as the B operand.
template <int NST>
__device__ __forceinline__ void tile_tz(f32x4& acc, ScanSmem& sm, int I, int J) {
  const int lane = threadIdx.x & 63, g4 = lane >> 4, c = lane & 15;
  const int ao = (16 * I + c) * VB + 8 * g4;
  bf16x8 x[NST][4];
#pragma unroll
  for (int st = 0; st < NST; ++st) {
    x[st][0] = ld8(sm.th + ao + 32 * st);
    x[st][1] = ld8(sm.tl + ao + 32 * st);
    const int b0 = (32 * st + 8 * g4 + (c >> 2)) * ZB + 16 * J + 4 * (c & 3);
    x[st][2] = pack8(lds_tr16(sm.zh + b0), lds_tr16(sm.zh + b0 + 4 * ZB));
    x[st][3] = pack8(lds_tr16(sm.zl + b0), lds_tr16(sm.zl + b0 + 4 * ZB));
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int st = 0; st < NST; ++st) acc = mfma3(x[st][0], x[st][1], x[st][2], x[st][3], acc);
}

// Pb: v_new rows of block I = T Z, split into nh / nl, and sk2 v_new split into vsh / vsl.
__device__ __forceinline__ void scan_vnew(ScanSmem& sm, int I, int J) {
  const int lane = threadIdx.x & 63, g4 = lane >> 4, c = lane & 15;
  f32x4 acc = zero4();
  const int i0 = 16 * I + 4 * g4, o = (16 * J + c) * VB + i0;
  const float z0 = sm.sc[i0].z, z1 = sm.sc[i0 + 1].z, z2 = sm.sc[i0 + 2].z, z3 = sm.sc[i0 + 3].z;
  if (I < 2) tile_tz<1>(acc, sm, I, J);
  else tile_tz<2>(acc, sm, I, J);
  bf16x4 h, l;
  split4(make_float4(acc[0], acc[1], acc[2], acc[3]), h, l);
  *reinterpret_cast<bf16x4*>(sm.nh + o) = h;
  *reinterpret_cast<bf16x4*>(sm.nl + o) = l;
  split4(make_float4(acc[0] * z0, acc[1] * z1, acc[2] * z2, acc[3] * z3), h, l);
  *reinterpret_cast<bf16x4*>(sm.vsh + o) = h;
  *reinterpret_cast<bf16x4*>(sm.vsl + o) = l;
}

// Operands that Pc takes from buffers the next chunk's inputs overwrite during Pc, read into
// registers in Pb: the wave's intra rows (A of the output product, tokens 32 st + 8 g .. + 7;
// blocks above the diagonal are zero), k's token columns for state tiles P0 + p (B of the
// state update, read transposed) and e^tot.
struct PcOps {
  bf16x8 ih[2], il[2];
  bf16x8 kh[2][2], kl[2][2];
  float et;
};
__device__ __forceinline__ void scan_pc_loads(ScanSmem& sm, int I, int P0, PcOps& op) {
  const int lane = threadIdx.x & 63, g4 = lane >> 4, c = lane & 15;
  const int ao = (16 * I + c) * VB + 8 * g4;
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    op.ih[st] = ld8(sm.ih + ao + 32 * st);
    op.il[st] = ld8(sm.il + ao + 32 * st);
    const int r0 = 32 * st + 8 * g4 + (c >> 2);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int e = 16 * (P0 + p) + 4 * (c & 3);
      const int b0 = qk_idx(r0, e), b1 = qk_idx(r0 + 4, e);
      op.kh[st][p] = pack8(lds_tr16(sm.kh + b0), lds_tr16(sm.kh + b1));
      op.kl[st][p] = pack8(lds_tr16(sm.kl + b0), lds_tr16(sm.kl + b1));
    }
  }
  op.et = sm.etot;
}

// Pc: out rows of block I = O + intra v_new (over the tokens below 32 ceil((I + 1) / 2)), a
// transposed tile like O (v_new^T rows as the A operand, intra rows as the B operand), written
// where the token exists.
template <int NST>
__device__ __forceinline__ void out_tile(ScanSmem& sm, int J, const PcOps& op, f32x4& o) {
  const int lane = threadIdx.x & 63, g4 = lane >> 4, c = lane & 15;
  const int bo = (16 * J + c) * VB + 8 * g4;
  bf16x8 bh[NST], bl[NST];
#pragma unroll
  for (int st = 0; st < NST; ++st) {
    bh[st] = ld8(sm.nh + bo + 32 * st);
    bl[st] = ld8(sm.nl + bo + 32 * st);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int st = 0; st < NST; ++st) o = mfma3(bh[st], bl[st], op.ih[st], op.il[st], o);
}
__device__ __forceinline__ void scan_out(ScanSmem& sm, float* orow, int I, int J, f32x4 o,
                                         int nvalid, const PcOps& op) {
  const int lane = threadIdx.x & 63, g4 = lane >> 4, c = lane & 15;
  if (I < 2) out_tile<1>(sm, J, op, o);
  else out_tile<2>(sm, J, op, o);
  const int i = 16 * I + c;
  if (i < nvalid)
    *reinterpret_cast<float4*>(orow + (size_t)i * D + 16 * J + 4 * g4) =
        make_float4(o[0], o[1], o[2], o[3]);
}

// The wave's state tiles (P0 + p, J), held in registers as S[16 (P0 + p) + 4 g + r][16 J + c]:
// S' = e^tot S + k^T (sk2 v_new) over the 64 tokens (split products, step st covering tokens
// 32 st + 8 g .. + 7: the A operand k's token columns from op, the B operand from vsh / vsl
// rows), then the split of S' to LDS, where a lane's 4 values are consecutive k indices of one
// S^T row (one 8-byte store per half and tile).
__device__ __forceinline__ void scan_state_update(ScanSmem& sm, int J, int P0, f32x4 (&s)[2],
                                                  const PcOps& op) {
  const int lane = threadIdx.x & 63, g4 = lane >> 4, c = lane & 15;
  bf16x8 ah[2], al[2];
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    const int ao = (16 * J + c) * VB + 32 * st + 8 * g4;
    ah[st] = ld8(sm.vsh + ao);
    al[st] = ld8(sm.vsl + ao);
  }
#pragma unroll
  for (int p = 0; p < 2; ++p) s[p] *= op.et;
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int p = 0; p < 2; ++p) s[p] = mfma3(op.kh[st][p], op.kl[st][p], ah[st], al[st], s[p]);
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int o = (16 * J + c) * RB + 16 * (P0 + p) + 4 * g4;
    bf16x4 h, l;
    split4(make_float4(s[p][0], s[p][1], s[p][2], s[p][3]), h, l);
    *reinterpret_cast<bf16x4*>(sm.sh + o) = h;
    *reinterpret_cast<bf16x4*>(sm.sl + o) = l;
  }
}

constexpr int kScanThreads = 512;

__global__ __launch_bounds__(kScanThreads, 1) void dn_chunk_scan_kernel(ScanArgs a) {
  __shared__ __attribute__((aligned(16))) ScanSmem sm;
  // workgroup L runs on XCD L % 8: the 4 column blocks of head h all get XCD h % 8
  const int L = blockIdx.x, grp = L / (8 * NCB), rem = L % (8 * NCB);
  const int cb = rem >> 3, h = 8 * grp + (rem & 7);
  if (h >= a.Hv) return;
  const int tid = threadIdx.x, lane = tid & 63, g4 = lane >> 4, c = lane & 15;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int J = wv & 1;
  const int I = wv < 4 ? 3 - ((wv >> 1) & 1) : (wv >> 1) & 1;
  const int P0 = 2 * ((wv >> 1) & 3);
  const int S = a.S;
  const size_t row0 = (size_t)h * S;
  const int c0 = 32 * cb;

  // this wave's state tiles: S[16 (P0 + p) + 4 g + r][c0 + 16 J + c] in s[p][r], and their split
  f32x4 s[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const float* src = a.state + ((size_t)h * D + 16 * (P0 + p) + 4 * g4) * D + c0 + 16 * J + c;
#pragma unroll
    for (int r = 0; r < 4; ++r) s[p][r] = src[r * D];
    const int o = (16 * J + c) * RB + 16 * (P0 + p) + 4 * g4;
    bf16x4 hh, ll;
    split4(make_float4(s[p][0], s[p][1], s[p][2], s[p][3]), hh, ll);
    *reinterpret_cast<bf16x4*>(sm.sh + o) = hh;
    *reinterpret_cast<bf16x4*>(sm.sl + o) = ll;
  }
  // The next chunk's inputs are read into registers while the current chunk computes, in
  // parts issued between the products (reading a chunk's 104 KB at once stalls every wave on
  // the memory pipeline), and each goes to LDS as soon as the current chunk is done with that
  // buffer, which keeps the registers held short (issued in / stored in):
  //   part 0..3    q rows (tid >> 5) + 16 j, float4 column tid & 31    Pa / Pb (split)
  //   part 4       this block's v: row tid >> 3, columns 4 (tid & 7)    Pa / Pc
  //   part 5..6    T hi, lo (16 bytes tid of each)                      Pa / Pc
  //   part 7       scales (wave 0, lane = token) and e^tot              Pa / Pc
  //   part 8..11   k rows, as q                                         Pa / Pc (end)
  //   part 12..13  intra hi, lo, as T                                   Pb / Pc (end)
  // Reads go through buffer descriptors based at the chunk's first row, sized to the end of
  // the prompt, so rows past it read as zeros.
  float4 pq[4], pk[4], pv, pt[2], pi[2];
  float4 psc = make_float4(0.f, 0.f, 0.f, 0.f);
  float pet = 0.f;
  const int qk_off = (tid >> 5) * (D * 4) + (tid & 31) * 16;        // + 8192 j
  const int v_off = (tid >> 3) * (D * 4) + (c0 + 4 * (tid & 7)) * 4;
  auto fetch_part = [&](int ci, int part) {
    const int t0 = ci * CH;
    const int rest = (S - t0) * (D * 4);
    const float* rec = a.ws + ((size_t)h * a.nch + ci) * REC;
    if (part < 4) {
      pq[part] = bload4(make_rsrc(a.q + (row0 + t0) * D, rest), qk_off + 8192 * part, 0);
    } else if (part == 4) {
      pv = bload4(make_rsrc(a.v + (row0 + t0) * D, rest), v_off, 0);
    } else if (part < 7) {
      pt[part - 5] = bload4(make_rsrc(rec, REC * 4), tid * 16, (REC_T + 2048 * (part - 5)) * 4);
    } else if (part == 7) {
      psc = bload4(make_rsrc(rec, REC * 4), lane * 16, REC_SC * 4);
      pet = rec[REC_ET];
    } else if (part < 12) {
      pk[part - 8] =
          bload4(make_rsrc(a.k + (row0 + t0) * D, rest), qk_off + 8192 * (part - 8), 0);
    } else if (part < 14) {
      pi[part - 12] =
          bload4(make_rsrc(rec, REC * 4), tid * 16, (REC_I + 2048 * (part - 12)) * 4);
    }
  };
  // q or k rows of the registers, split, to LDS
  auto store_split = [&](const float4 (&src)[4], __bf16* hi, __bf16* lo) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int o = qk_idx((tid >> 5) + 16 * j, 4 * (tid & 31));
      bf16x4 hh, ll;
      split4(src[j], hh, ll);
      *reinterpret_cast<bf16x4*>(hi + o) = hh;
      *reinterpret_cast<bf16x4*>(lo + o) = ll;
    }
  };
  // a split 64 x 64 record matrix: 16 bytes tid of the hi half and of the lo half (row tid >> 3,
  // columns 8 (tid & 7) .. + 7)
  const int m_off = (tid >> 3) * VB + 8 * (tid & 7);
  auto store_v_t_sc = [&]() {
    *reinterpret_cast<float4*>(sm.vr + (tid >> 3) * VS + 4 * (tid & 7)) = pv;
    *reinterpret_cast<float4*>(sm.th + m_off) = pt[0];
    *reinterpret_cast<float4*>(sm.tl + m_off) = pt[1];
    if (wv == 0) sm.sc[lane] = psc;
  };
  auto store_k_intra = [&]() {
    store_split(pk, sm.kh, sm.kl);
    *reinterpret_cast<float4*>(sm.ih + m_off) = pi[0];
    *reinterpret_cast<float4*>(sm.il + m_off) = pi[1];
    if (wv == 0 && lane == 0) sm.etot = pet;
  };
#pragma unroll
  for (int part = 0; part < 14; ++part) fetch_part(0, part);
  store_split(pq, sm.qh, sm.ql);
  store_v_t_sc();
  store_k_intra();
  f32x4 o;
  PcOps op;
  for (int ci = 0; ci < a.nch; ++ci) {
    const int t0 = ci * CH;
    // the next chunk's reads (unconditional, so that no branch forces an early wait: the last
    // chunk reads itself again, and its late stores only rewrite buffers it no longer reads)
    const int nx = min(ci + 1, a.nch - 1);
    auto pre_a = [&](int st) {
#pragma unroll
      for (int d = 0; d < 3; ++d) fetch_part(nx, 3 * st + d);
    };
    __syncthreads();
    scan_state_products(sm, I, J, o, pre_a);
    __syncthreads();
    fetch_part(nx, 12);
    fetch_part(nx, 13);
    scan_vnew(sm, I, J);
    // after v_new's operand reads (a wave's LDS requests return in order): frees k, intra and
    // e^tot for the next chunk's stores in Pc
    scan_pc_loads(sm, I, P0, op);
    store_split(pq, sm.qh, sm.ql);  // q of this chunk was last read in Pa
    __syncthreads();
    scan_state_update(sm, J, P0, s, op);  // first: the next chunk waits on its split of S
    scan_out(sm, a.out + (row0 + t0) * D + c0, I, J, o, min(CH, S - t0), op);
    store_v_t_sc();  // v, T and the scales were last read in Pa / Pb
    store_k_intra();  // k, intra and e^tot of this chunk were last read in Pa / Pb
  }
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    float* dst = a.new_state + ((size_t)h * D + 16 * (P0 + p) + 4 * g4) * D + c0 + 16 * J + c;
#pragma unroll
    for (int r = 0; r < 4; ++r) dst[r * D] = s[p][r];
  }
}

constexpr int kPrepGrid = 512;  // two prep workgroups per CU (70 KB of LDS each)

// S * 512 bytes must fit the 32-bit buffer offsets
bool shape_ok(int v_heads, int S) {
  return v_heads >= 1 && v_heads <= 65535 && S >= 1 && S <= (1 << 22) &&
         (long)v_heads * S <= (1L << 26);
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
  const int items = nch * v_heads;
  hipLaunchKernelGGL(dn_chunk_prep_kernel, dim3(std::min(items, kPrepGrid)), dim3(256), 0, st,
                     PrepArgs{query, key, g, beta, ws, S, nch, items});
  const int groups = (v_heads + 7) / 8;
  hipLaunchKernelGGL(dn_chunk_scan_kernel, dim3(groups * 8 * NCB), dim3(kScanThreads), 0, st,
                     ScanArgs{state, query, key, value, ws, out, new_state, S, nch, v_heads});
  return npn_launch_status();
}
