// FP8 (OCP e4m3fn) W8A16 GEMM for gfx950: out[M,N] = bf16((x[M,K] . W[K,N]) * scale[N]).
//
// Semantics of the reference op fp8::matmul (contrib/qwen3.6-27b/kernels/fp8_matmul_ops.py:14-21,
// kernel contrib/qwen3.6-27b/kernels/fp8_matmul.py:55-184): fp8 weight bytes pre-transposed
// to [K, N] (N contiguous), bf16 activations, fp32 accumulation, per-output-channel scale
// applied to the fp32 sum, then a bf16 cast.
//
// Two kernels, both staging W tiles in LDS with direct global-to-LDS loads.
// v_mfma_f32_16x16x32_bf16's B operand wants 8 consecutive k of one column per lane, but
// [K, N] stores a column with stride N. Up to 64 rows (the narrow kernel, HBM-bound) each lane
// reads 4 to 16 adjacent columns from each of its 8 k rows out of LDS, transposes each 8x4
// byte quarter in registers with v_perm_b32 and dequantises each column's 8 bytes to bf16
// with v_cvt_scalef32_pk_bf16_fp8 (exact: every e4m3fn value is a bf16 value). Above 64 rows
// (the wide kernel, MFMA-bound) the B operands are read back transposed (ds_read_b64_tr_b8)
// and converted the same way; details with each kernel below.
#include "accept_contract.h"
#include "npn_internal.h"

namespace {

constexpr int KSTEP = 32;   // k per MFMA

typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((__vector_size__(2 * sizeof(__bf16))));

// Row argmax over the GEMM's bf16 outputs (the LM head's greedy decision without writing the
// logits): per (row, column group) the largest bf16(acc * scale) and its column, NaN counting
// as the maximum and ties going to the lower column (torch.argmax). Same 8-byte layout as the
// acceptance kernels' per-chunk partials, which reduce and consume it.
struct ArgPart {
  float v;
  int i;
};

__device__ __forceinline__ bool arg_beats(float bv, int bi, float av, int ai) {
  const bool an = isnan(av), bn = isnan(bv);
  if (an || bn) return bn && (!an || bi < ai);
  return bv > av || (bv == av && bi < ai);
}

// (v, i) of the best of the 16 lanes of this lane's 16-lane group, in every lane of it.
__device__ __forceinline__ void arg_merge16(float& v, int& i) {
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) {
    const float ov = __shfl_xor(v, off, 64);
    const int oi = __shfl_xor(i, off, 64);
    if (arg_beats(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
}

// The same merge over each aligned 16-lane row by DPP moves (quad, quad pairs, half-row
// mirror, row mirror): the rule is a total order, so the pairing does not change the result.
template <int CTRL>
__device__ __forceinline__ void arg_step_dpp(float& v, int& i) {
  const float ov = __uint_as_float(npn::dpp32<CTRL>(__float_as_uint(v)));
  const int oi = (int)npn::dpp32<CTRL>((uint32_t)i);
  if (arg_beats(ov, oi, v, i)) {
    v = ov;
    i = oi;
  }
}

__device__ __forceinline__ void arg_merge16_dpp(float& v, int& i) {
  arg_step_dpp<npn::kDppStep[0]>(v, i);
  arg_step_dpp<npn::kDppStep[1]>(v, i);
  arg_step_dpp<npn::kDppStep[2]>(v, i);
  arg_step_dpp<npn::kDppStep[3]>(v, i);
}

__device__ __forceinline__ float bf16_round(float x) {
  return npn::bf16_to_f32(npn::f32_to_bf16(x));
}

// Bytes 0-1 (HI = false) or 2-3 (HI = true) of w -> two bf16 (OCP e4m3fn decode, scale 1).
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2(uint32_t w) {
  const bf16x2 v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI);
  return __builtin_bit_cast(uint32_t, v);
}

// d[0..7]: byte b of d[j] = W[k0 + 8G + j][n0 + 4i + b]. Returns, for each column b, the
// 8 k-values as a bf16x8 MFMA B operand.
__device__ __forceinline__ void transpose_dequant(const uint32_t (&d)[8], bf16x8 (&bop)[4]) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {  // k rows 0-3, then 4-7
    const uint32_t d0 = d[4 * h], d1 = d[4 * h + 1], d2 = d[4 * h + 2], d3 = d[4 * h + 3];
    const uint32_t t0 = __builtin_amdgcn_perm(d1, d0, 0x05010400u);  // d0[0] d1[0] d0[1] d1[1]
    const uint32_t t1 = __builtin_amdgcn_perm(d1, d0, 0x07030602u);  // d0[2] d1[2] d0[3] d1[3]
    const uint32_t u0 = __builtin_amdgcn_perm(d3, d2, 0x05010400u);
    const uint32_t u1 = __builtin_amdgcn_perm(d3, d2, 0x07030602u);
    const uint32_t e[4] = {
        __builtin_amdgcn_perm(u0, t0, 0x05040100u),  // column 0: k rows 4h..4h+3
        __builtin_amdgcn_perm(u0, t0, 0x07060302u),  // column 1
        __builtin_amdgcn_perm(u1, t1, 0x05040100u),  // column 2
        __builtin_amdgcn_perm(u1, t1, 0x07060302u),  // column 3
    };
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      u32x4 cur = __builtin_bit_cast(u32x4, bop[ct]);
      cur[2 * h] = fp8x2_to_bf16x2<false>(e[ct]);
      cur[2 * h + 1] = fp8x2_to_bf16x2<true>(e[ct]);
      bop[ct] = __builtin_bit_cast(bf16x8, cur);
    }
  }
}

struct GemmArgs {
  const uint16_t* x;
  const uint8_t* w;
  const float* scale;
  uint16_t* out;     // used when split_k == 1 and !to_partial
  float* partial;    // [split_k][M][N] fp32, unscaled, when split_k > 1 or to_partial
  int M, K, N, split_k, to_partial;
  ArgPart* amax;     // row argmax partials [M][column groups] instead of out (split_k == 1)
  float* gmax;       // with out: per-(row, column group) max of the bf16 outputs, NaN ignored
  int sk_wg;         // narrow kernel, > 0: stream-K over this many workgroups (split_k slots)
  // with out (split_k == 1): the acceptance contract's statistics of each row's 64-column
  // chunks of the bf16 outputs scaled by inv_temp, [M][N / 64] (cmax == nullptr: none)
  float* cmax;
  uint64_t* csum;
  float inv_temp;
  // narrow kernel, tiles1 > 0: a second matrix in the same launch (partials only, no
  // stream-K): column tiles [0, tiles1) are w's, the rest w2's [K, N2] with partials2
  const uint8_t* w2;
  float* partial2;
  int N2, tiles1;
};

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor((uint32_t)v, m, 64);
  const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), m, 64);
  return ((uint64_t)hi << 32) | lo;
}

// ---------------------------------------------------------------------------------------
// Narrow kernel for M <= 64 rows (HBM-bound: each weight byte feeds 2*M flops).
// The weights stream once from HBM, so what matters is how the reads meet the DRAM: consecutive
// rows of W are N bytes apart, and a W row read in pieces of 64 contiguous bytes streams at
// about 2.4 TB/s on MI355X, in pieces of 128 bytes at 4.1 TB/s and of 256 bytes at 4.8 TB/s,
// whatever the bytes per lane (measured with a pure-load kernel, 178 MB of W, 544
// workgroups). So a workgroup owns a 256-column tile, and each k step's W tile (32 rows x
// 256 columns, 256-byte row runs) and x rows (16 RB rows x 32 k) move HBM -> LDS by direct
// loads (global_load_lds_dwordx4), NS stages deep: every W byte is fetched once per
// workgroup, whatever its number of row blocks, and NS - 1 tiles are in flight. The NWV waves
// split the tile by rows and columns with no k split: RB row blocks of 16 rows x CH = NWV / RB
// column slices of 256 / CH columns; lane (i, G) reads CB = 16 / CH bytes (columns) from each
// of its 8 k rows 8 G + j out of LDS, and each 4-column quarter is transposed and dequantised
// in registers into the B operands of 4 MFMAs (column ct of quarter q feeds MFMA 4 q + ct).
// Each wave issues the same DMA instructions for every tile, so a vmcnt of (tiles issued
// after tile t) x (this wave's DMAs per tile) names "tile t landed"; an s_barrier then
// publishes it. For wide N, K is also split across workgroups (split_k); partials then go
// through an fp32 workspace and a fixed-order reduction kernel.
constexpr int NT = 256;     // columns per narrow tile

// s_waitcnt vmcnt(pend * DPT) for a wave-uniform pend in [0, C] (the count is an immediate).
template <int C, int DPT>
__device__ __forceinline__ void wait_tiles(int pend) {
  if constexpr (C > 0) {
    if (pend >= C) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(C * DPT) : "memory");
      return;
    }
    wait_tiles<C - 1, DPT>(pend);
  } else {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
}

template <int RB, int NS, int NWV>
__global__ __launch_bounds__(NWV * 64, 1) void fp8_gemm_narrow_kernel(GemmArgs ka) {
  // A two-matrix launch runs the second matrix's tiles with its pointers and width.
  GemmArgs a = ka;
  int tile = blockIdx.x;
  if (ka.tiles1 > 0 && tile >= ka.tiles1) {
    a.w = ka.w2;
    a.N = ka.N2;
    a.partial = ka.partial2;
    tile -= ka.tiles1;
  }
  constexpr int NTH = NWV * 64;
  constexpr int CH = NWV / RB;               // column slices
  constexpr int CB = 16 / CH;                // columns (bytes) per lane
  static_assert(CB >= 4 && CB <= 16, "4 to 16 columns per lane");
  constexpr int WST = 32 * NT;               // W stage bytes
  constexpr int XST = 16 * RB * 64;          // x stage bytes (rows x 32 k bf16)
  constexpr int STAGE = WST + XST;
  constexpr int WQ = WST / 16 / NTH;         // W DMA instructions (16 bytes) per thread
  constexpr int XW = XST / 16 / 64;          // waves that move x, one 16-byte DMA per lane
  static_assert(WQ * 16 * NTH == WST && XW * 64 * 16 == XST && XW <= NWV,
                "whole DMA instructions per stage");
  __shared__ __attribute__((aligned(16))) uint8_t smem[NS * STAGE];

  const int m_pass = blockIdx.z * 16 * RB;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int i = lane & 15, G = lane >> 4;
  const int rb = w / CH, ch = w - rb * CH;
  const int nks = a.K / KSTEP;
  const int mrow = m_pass + 16 * rb + i;              // A operand row of this lane
  const bool row_ok = mrow < a.M;
  const int lcol = ch * 16 * CB + CB * i;             // the lane's first column in the tile

  // k steps ks_lo .. ks_lo + ntile - 1 of the tile at column n0, summed into acc.
  auto run = [&](int n0, int ks_lo, int ntile, f32x4 (&acc)[CB]) {
    // DMA of k step ks into stage st: W rows (WQ x 16 bytes per thread), then x rows.
    auto issue = [&](int ks, int st) {
      uint8_t* ws = smem + st * STAGE;
      uint8_t* xs = ws + WST;
      const int k0 = ks * KSTEP;
#pragma unroll
      for (int q = 0; q < WQ; ++q) {
        const int s = q * NTH + tid;                  // 16-byte slot of the W stage
        const int row = s >> 4;
        int col = n0 + 16 * (s & 15);
        col = col < a.N ? col : a.N - 16;             // a partial last tile re-reads valid bytes
        npn::lds_dma16(a.w + (size_t)(k0 + row) * a.N + col, ws + q * (NTH * 16) + (tid & ~63) * 16);
      }
      if (w < XW) {                                   // 16-byte slots, 4 per 64-byte row
        const int s = w * 64 + lane;
        int m = m_pass + (s >> 2);
        m = m < a.M ? m : a.M - 1;
        npn::lds_dma16(a.x + (size_t)m * a.K + k0 + 8 * (s & 3), xs + w * 1024);
      }
    };
#pragma unroll
    for (int p = 0; p < NS - 1; ++p)
      if (p < ntile) issue(ks_lo + p, p);
    for (int t = 0; t < ntile; ++t) {
      // Tiles t + 1 .. min(t + NS - 2, ntile - 1) were issued after tile t: wait until at
      // most their DMAs are outstanding (this wave's count per tile is WQ, plus one x DMA
      // for waves w < XW), then publish tile t.
      const int pend = min(ntile - 1 - t, NS - 2);
      if (w < XW) wait_tiles<NS - 2, WQ + 1>(pend);
      else wait_tiles<NS - 2, WQ>(pend);
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      const int tn = t + NS - 1;                      // into the stage tile t - 1 used
      if (tn < ntile) issue(ks_lo + tn, tn % NS);
      const uint8_t* ws = smem + (t % NS) * STAGE;
      const uint8_t* xs = ws + WST;
      const u32x4 xv = *reinterpret_cast<const u32x4*>(xs + (16 * rb + i) * 64 + 16 * G);
      const u32x4 zero = {0u, 0u, 0u, 0u};
      const bf16x8 aop = __builtin_bit_cast(bf16x8, row_ok ? xv : zero);
      uint32_t d[8][CB / 4];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint8_t* src = ws + (8 * G + j) * NT + lcol;
        if constexpr (CB == 16) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(src);
#pragma unroll
          for (int q = 0; q < 4; ++q) d[j][q] = v[q];
        } else if constexpr (CB == 8) {
          const uint2 v = *reinterpret_cast<const uint2*>(src);
          d[j][0] = v.x;
          d[j][1] = v.y;
        } else {
          d[j][0] = *reinterpret_cast<const uint32_t*>(src);
        }
      }
#pragma unroll
      for (int q = 0; q < CB / 4; ++q) {
        uint32_t dq[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) dq[j] = d[j][q];
        bf16x8 bop[4];
        transpose_dequant(dq, bop);
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
          acc[4 * q + ct] =
              __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop, bop[ct], acc[4 * q + ct], 0, 0, 0);
      }
    }
    // (every DMA has landed: the last tile waited with vmcnt(0))
  };

  // fp32 sums (unscaled) of this lane's rows and columns of the tile at n0 into partial
  // slot `slot` ([split_k][M][N]); zero sums when `zero`.
  auto store_partial = [&](int slot, int n0, const f32x4 (&acc)[CB], bool zero) {
    const int nc = n0 + lcol;
    if (nc >= a.N) return;
    float* part = a.partial + (size_t)slot * a.M * a.N;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m_pass + 16 * rb + 4 * G + r;
      if (m >= a.M) continue;
      float4* dst = reinterpret_cast<float4*>(part + (size_t)m * a.N + nc);
#pragma unroll
      for (int c = 0; c < CB / 4; ++c)
        dst[c] = zero ? make_float4(0.f, 0.f, 0.f, 0.f)
                      : make_float4(acc[4 * c][r], acc[4 * c + 1][r], acc[4 * c + 2][r],
                                    acc[4 * c + 3][r]);
    }
  };

  if (a.sk_wg > 0) {
    // Stream-K: the tiles' k steps laid end to end (U units), workgroup wg taking units
    // [wg U / W, (wg + 1) U / W). A tile's units are covered by workgroups wfirst .. wlast
    // (closed form: the workgroup that holds unit x is ((x + 1) W - 1) / U); workgroup wg
    // writes its sums of tile t to slot wg - wfirst, and wlast zeroes the slots past the
    // tile's last, so every tile's split_k slots add to its full sum in slot order.
    const long U = (long)((a.N + NT - 1) / NT) * nks;
    const long W = a.sk_wg;
    const long wg = blockIdx.x;
    const long u0 = wg * U / W, u1 = (wg + 1) * U / W;
    for (long t = u0 / nks; t * nks < u1; ++t) {
      const long tb = t * nks;
      const int lo = (int)(u0 > tb ? u0 - tb : 0);
      const int hi = (int)(u1 - tb < nks ? u1 - tb : nks);
      const int wfirst = (int)(((tb + 1) * W - 1) / U);
      const int wlast = (int)(((tb + nks) * W - 1) / U);
      f32x4 acc[CB];
#pragma unroll
      for (int c = 0; c < CB; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
      __syncthreads();  // every wave is done with the ring's previous segment
      run((int)t * NT, lo, hi - lo, acc);
      store_partial((int)wg - wfirst, (int)t * NT, acc, false);
      if (wg == wlast)
        for (int sl = wlast - wfirst + 1; sl < a.split_k; ++sl)
          store_partial(sl, (int)t * NT, acc, true);
    }
    return;
  }

  const int n0 = tile * NT;
  const int sk = blockIdx.y;
  const int ks_lo = (int)(((long)nks * sk) / a.split_k);
  const int ks_hi = (int)(((long)nks * (sk + 1)) / a.split_k);
  f32x4 acc[CB];
#pragma unroll
  for (int c = 0; c < CB; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  run(n0, ks_lo, ks_hi - ks_lo, acc);


  // Lane (i, G) holds rows m_pass + 16 rb + 4 G + r and columns nc + c in acc[c][r]; its
  // group for the row maxima is the (tile, column slice) pair.
  const int nc = n0 + lcol;
  const bool col_ok = nc < a.N;
  const int groups = gridDim.x * CH;
  const int grp = blockIdx.x * CH + ch;
  if (a.amax != nullptr) {
    float sc[CB];
#pragma unroll
    for (int c = 0; c < CB; ++c) sc[c] = col_ok ? a.scale[nc + c] : 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float bv = -__builtin_inff();
      int bi = 0x7FFFFFFF;
      if (col_ok) {
#pragma unroll
        for (int c = 0; c < CB; ++c) {
          const float v = bf16_round(acc[c][r] * sc[c]);
          if (arg_beats(v, nc + c, bv, bi)) {
            bv = v;
            bi = nc + c;
          }
        }
      }
      arg_merge16(bv, bi);
      const int m = m_pass + 16 * rb + 4 * G + r;
      if (i == 0 && m < a.M) a.amax[(size_t)m * groups + grp] = ArgPart{bv, bi};
    }
    return;
  }
  if (a.split_k == 1 && !a.to_partial) {
    float sc[CB];
#pragma unroll
    for (int c = 0; c < CB; ++c) sc[c] = col_ok ? a.scale[nc + c] : 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m_pass + 16 * rb + 4 * G + r;
      uint32_t pk[CB / 2];
      float mx = -__builtin_inff();  // max of the row's bf16 outputs (fmaxf ignores NaN)
#pragma unroll
      for (int c = 0; c < CB / 2; ++c) {
        const uint32_t lo = npn::f32_to_bf16(acc[2 * c][r] * sc[2 * c]);
        const uint32_t hi = npn::f32_to_bf16(acc[2 * c + 1][r] * sc[2 * c + 1]);
        pk[c] = lo | (hi << 16);
        mx = fmaxf(mx, fmaxf(npn::bf16_to_f32(lo), npn::bf16_to_f32(hi)));
      }
      if (col_ok && m < a.M) {
        uint16_t* dst = a.out + (size_t)m * a.N + nc;
        if constexpr (CB == 16) {
          reinterpret_cast<uint4*>(dst)[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
          reinterpret_cast<uint4*>(dst)[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
        } else if constexpr (CB == 8) {
          *reinterpret_cast<uint4*>(dst) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        } else {
          *reinterpret_cast<uint2*>(dst) = make_uint2(pk[0], pk[1]);
        }
      }
      if (a.gmax != nullptr) {  // the 16 lanes of a group share the row; lanes past N add -inf
        if (!col_ok) mx = -__builtin_inff();
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        if (i == 0 && m < a.M) a.gmax[(size_t)m * groups + grp] = mx;
      }
      if (a.cmax != nullptr) {
        // Contract chunk statistics: a 64-column chunk is held by LPC adjacent lanes of the
        // 16-lane group (N % 64 == 0, so a chunk is wholly inside or wholly past N).
        constexpr int LPC = 64 / CB;  // 16, 8 or 4: a DPP row, half-row or quad
        constexpr int STEPS = LPC == 16 ? 4 : (LPC == 8 ? 3 : 2);
        float xs[CB];
#pragma unroll
        for (int c = 0; c < CB / 2; ++c) {
          xs[2 * c] = npn::scaled(npn::bf16lo(pk[c]), a.inv_temp);
          xs[2 * c + 1] = npn::scaled(npn::bf16hi(pk[c]), a.inv_temp);
        }
        float cmx = -__builtin_inff();
#pragma unroll
        for (int c = 0; c < CB; ++c) cmx = fmaxf(cmx, xs[c]);
        cmx = npn::row_max_dpp<STEPS>(cmx);
        uint64_t csm = 0;
#pragma unroll
        for (int c = 0; c < CB; ++c) csm += npn::expfix_rel(xs[c], cmx);
        csm = npn::row_sum_dpp<STEPS>(csm);
        if (i % LPC == 0 && col_ok && m < a.M) {
          const size_t o = (size_t)m * (a.N / 64) + (nc >> 6);
          a.cmax[o] = cmx;
          a.csum[o] = csm;
        }
      }
    }
  } else {
    store_partial(sk, n0, acc, false);
  }
}

// ---------------------------------------------------------------------------------------
// Wide kernel for 64 < M <= 256 rows per pass (MFMA-bound: each weight byte feeds 2*M flops).
// The grid is one workgroup of 8 waves per CU. A single wave per SIMD issues independent
// bf16 MFMAs at about 55 % of the SIMD's peak, two waves at about 83 % (measured on MI355X),
// so each SIMD runs two waves. Columns are split into 16-wide units spread evenly over the
// workgroups (u0..u1, at most 2*NH units each), so every CU gets the same work up to one
// unit; workgroups are placed so logically adjacent column ranges share an XCD and its L2
// (a range is a 128..160-byte segment of each weight row, so neighbours share lines).
//
// Data path, all global reads by LDS DMA (npn::lds_dma16, no VGPR staging) into a
// 3-stage ring, two 64-k chunks ahead of the MFMAs:
//   x chunk  [256 rows][64 k] bf16, 16-byte chunks XOR-swizzled by (row >> 1) & 7, so the
//            16 rows of an A-operand read cover all 64 LDS banks once (row parity x chunk)
//   W chunk  [64 k][16 * nup] raw e4m3fn bytes: each k row's nu 16-byte column units (the
//            [K, N] layout, one row segment per k) padded to nup = nu | 1 units, so the 16
//            rows of a transposed B read start on 16 distinct 4-bank groups (nup odd)
// Wave w owns rows 64*(w & 3) .. +63 and column tiles NH*(w >> 2) .. +NH-1 of the
// workgroup's units, so the x tile is loaded once per CU and each B tile is read and
// converted by the four waves of its column half (one per row quarter). A operands come from
// the x tile (ds_read_b128), B operands from the W tile with the 8-bit transposed read
// ds_read_b64_tr_b8 -- in each 16-lane group, lane i gets byte (i & 7) of the 8-byte chunk
// supplied by lane 2j + (i >> 3) as its j-th byte, so lanes 2j + h supply row k0 + 8G + j,
// columns 8h..8h+7, and lane i receives column i's 8 consecutive k -- then 4
// v_cvt_scalef32_pk_bf16_fp8 make the bf16 B operand.
constexpr int KC = 64;          // k per pipeline chunk
constexpr int WIDE_WG = 256;    // workgroups per pass (one per CU)
constexpr int WIDE_THREADS = 512;
constexpr int NSTAGE = 3;

struct WideArgs {
  const uint16_t* x;
  const uint8_t* w;
  const float* scale;
  uint16_t* out;
  float* partial;  // [split_k][M][N] fp32, unscaled, when split_k > 1 or to_partial
  int M, K, N, units, groups, split_k, to_partial;
  ArgPart* amax;   // row argmax partials [M][groups] instead of out (split_k == 1)
  float* gmax;     // with out: per-(row, group) max of the bf16 outputs, NaN ignored
  // SwiGLU epilogue (split_k == 1): W = [gate | up] along N; units counts gate units, each
  // workgroup takes gate units u0..u1 (at most NH) and the up units N/2 columns to their
  // right, wave column half 0 computing gate and 1 up; out [M, N/2] = bf16(bf16(silu(g)) * u)
  int swiglu;
  int ualign;      // column groups hold whole runs of ualign units (4: 64-column chunks)
  // with out (split_k == 1): the acceptance contract's statistics of each row's 64-column
  // chunks of the bf16 outputs scaled by inv_temp, [M][N / 64] (cmax == nullptr: none;
  // then ualign == 4)
  float* cmax;
  uint64_t* csum;
  float inv_temp;
};

typedef int i32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ i32x2 lds_tr8(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) i32x2*)(p));
}

// Rows [0, 256) of a staged bf16 tile (row stride rs elements; column j of the tile is output
// column n0 + j, 16 nu columns per row) to out (row stride ld), as 16-byte pieces; rows at or
// past M are skipped.
__device__ __forceinline__ void store_staged_bf16(const uint16_t* st, int rs, uint16_t* out,
                                                  int ld, int m_base, int M, int n0, int nu) {
  const int pieces = 2 * nu;
  for (int p = threadIdx.x; p < 256 * pieces; p += WIDE_THREADS) {
    const int row = p / pieces, q = p - row * pieces;
    const int m = m_base + row;
    if (m < M)
      *reinterpret_cast<uint4*>(out + (size_t)m * ld + n0 + 8 * q) =
          *reinterpret_cast<const uint4*>(st + row * rs + 8 * q);
  }
}

// Byte offset of the SwiGLU staging tile: past the gate/up exchange slots (4 row quarters x 64
// lanes x 16 NH bf16), 16-byte aligned.
// Per-row max of a staged bf16 tile (256 rows of 16 nu values, row stride rs), NaN ignored
// (fmaxf), into gmax[m][grp] (stride ld): two threads per row, alternating 16-byte pieces.
__device__ __forceinline__ void staged_row_max(const uint16_t* st, int rs, float* gmax, int ld,
                                               int grp, int m_base, int M, int nu) {
  const int row = threadIdx.x >> 1, half = threadIdx.x & 1;
  float mx = -__builtin_inff();
  for (int q = half; q < 2 * nu; q += 2) {
    const uint4 v = *reinterpret_cast<const uint4*>(st + row * rs + 8 * q);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k)
      mx = fmaxf(mx, fmaxf(npn::bf16_to_f32(w[k] & 0xFFFFu), npn::bf16_to_f32(w[k] >> 16)));
  }
  mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
  if (half == 0 && m_base + row < M) gmax[(size_t)(m_base + row) * ld + grp] = mx;
}

// The acceptance contract's statistics of a staged bf16 tile (256 rows of 16 nu values, row
// stride rs; nu a multiple of 4 and the tile's column 0 at output column n0, a multiple of 64):
// per (row, 64-column chunk) the max of s = value * inv_temp (NaN ignored) and the sum of
// expfix(s - max), into cmax / csum [M][nc]. Two threads per row, 32 columns of each chunk.
__device__ __forceinline__ void staged_chunk_stats(const uint16_t* st, int rs, float* cmax,
                                                   uint64_t* csum, float inv_temp, int nc,
                                                   int m_base, int M, int n0, int nu) {
  const int row = threadIdx.x >> 1, half = threadIdx.x & 1;
  const int m = m_base + row;
  for (int q = 0; q < nu / 4; ++q) {
    float x[32];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint4 v = *reinterpret_cast<const uint4*>(st + row * rs + 64 * q + 32 * half + 8 * p);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        x[8 * p + 2 * k] = npn::scaled(npn::bf16lo(w[k]), inv_temp);
        x[8 * p + 2 * k + 1] = npn::scaled(npn::bf16hi(w[k]), inv_temp);
      }
    }
    float mx = -__builtin_inff();
#pragma unroll
    for (int e = 0; e < 32; ++e) mx = fmaxf(mx, x[e]);
    mx = npn::row_max_dpp<1>(mx);  // the row's two threads are lanes 2j, 2j + 1
    uint64_t sm = 0;
#pragma unroll
    for (int e = 0; e < 32; ++e) sm += npn::expfix_rel(x[e], mx);
    sm = npn::row_sum_dpp<1>(sm);
    if (half == 0 && m < M) {
      const size_t o = (size_t)m * nc + (n0 >> 6) + q;
      cmax[o] = mx;
      csum[o] = sm;
    }
  }
}

template <int NH>
constexpr int kSwigluStageOff = 4 * 64 * 16 * NH * 2;

template <int NH>  // column tiles per wave; a workgroup holds up to 2*NH units
__global__ __launch_bounds__(WIDE_THREADS, 1) void fp8_gemm_wide_kernel(WideArgs a) {
  constexpr int XBYTES = 256 * KC * 2;                          // 32 KiB x stage
  constexpr int WI = (KC * (2 * NH + 1) + WIDE_THREADS - 1) / WIDE_THREADS;  // W DMA per thread
  constexpr int WBYTES = WI * WIDE_THREADS * 16;                // W stage incl. slack
  constexpr int STAGE = XBYTES + WBYTES;
  constexpr int XI = XBYTES / (WIDE_THREADS * 16);              // x DMA per thread (4)
  __shared__ __attribute__((aligned(16))) uint8_t smem[NSTAGE * STAGE];
  static_assert(256 * (32 * NH + 8) * 2 <= NSTAGE * STAGE, "bf16 staging exceeds the LDS ring");
  static_assert(128 * (32 * NH + 4) * 4 <= NSTAGE * STAGE, "fp32 staging exceeds the LDS ring");
  static_assert(kSwigluStageOff<NH> + 256 * (16 * NH + 8) * 2 <= NSTAGE * STAGE,
                "SwiGLU staging exceeds the LDS ring");

  const int nwg = gridDim.x;
  const int per_xcd = nwg / 8;
  const int logical = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  const int sk = logical % a.split_k;
  const int grp = logical / a.split_k;
  if (grp >= a.groups) return;
  const int ua = a.ualign;  // groups of whole ua-unit runs, balanced over the workgroups
  const int u0 = ua * (int)((long)grp * (a.units / ua) / a.groups);
  const int u1 = ua * (int)((long)(grp + 1) * (a.units / ua) / a.groups);
  const int nu = u1 - u0;
  if (nu <= 0) return;
  const int n0 = 16 * u0;
  // W row stride in the stage, in 16-byte units (odd); SwiGLU: NH gate slots, NH up slots
  const int nup = a.swiglu ? 2 * NH + 1 : (nu | 1);
  const int nchunks = a.K / KC;
  const int c_lo = (int)((long)nchunks * sk / a.split_k);
  const int c_hi = (int)((long)nchunks * (sk + 1) / a.split_k);
  const int m_base = blockIdx.y * 256;
  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int wr = wv & 3, wc = wv >> 2;  // row quarter, column half
  const int i = lane & 15, G = lane >> 4;
  const int mlast = a.M - 1;

  // DMA of chunk c into stage st: x rows (XI instructions / thread), then W rows.
  auto issue = [&](int c, int st) {
    uint8_t* xs = smem + st * STAGE;
    uint8_t* ws = xs + XBYTES;
#pragma unroll
    for (int q = 0; q < XI; ++q) {
      const int f = q * WIDE_THREADS + tid;   // 16-byte slot in the x stage
      const int row = f >> 3, pos = f & 7;    // 8 slots per 128-byte row
      int m = m_base + row;
      m = m <= mlast ? m : mlast;
      const uint16_t* src = a.x + (size_t)m * a.K + c * KC + 8 * (pos ^ ((row >> 1) & 7));
      npn::lds_dma16(src, xs + q * (WIDE_THREADS * 16) + (tid & ~63) * 16);
    }
#pragma unroll
    for (int q = 0; q < WI; ++q) {
      int f = q * WIDE_THREADS + tid;         // 16-byte slot of the W stage
      if (f >= KC * nup) f = 0;               // lanes past the stage re-read slot 0 (slack)
      const int r = f / nup;
      const int cc = f - r * nup;
      int col;
      if (a.swiglu) {                         // slots [0, NH) gate, [NH, 2NH) up, 2NH pad
        const int hsel = cc >= NH && cc < 2 * NH ? 1 : 0;
        int uu = cc - NH * hsel;
        uu = uu < nu ? uu : 0;                // unused or pad slot: re-read unit u0
        col = n0 + 16 * uu + hsel * (a.N / 2);
      } else {
        col = n0 + 16 * (cc < nu ? cc : 0);   // row pad slot: re-read the row's first unit
      }
      const uint8_t* src = a.w + (size_t)(c * KC + r) * a.N + col;
      npn::lds_dma16(src, ws + q * (WIDE_THREADS * 16) + (tid & ~63) * 16);
    }
  };

  f32x4 acc[4][NH];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < NH; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // B-operand tr8 address parts: lane supplies row 8G + (i >> 1), column half (i & 1), of
  // this wave's first column tile.
  const int trow = 8 * G + (i >> 1);
  const int tcol = 8 * (i & 1) + 16 * NH * wc;

  // Ring: chunk c in stage (c - c_lo) % 3, issued two chunks ahead of its use.
  if (c_lo < c_hi) issue(c_lo, 0);
  if (c_lo + 1 < c_hi) issue(c_lo + 1, 1);
  // The scales of this lane's output columns, loaded now so that the epilogue does not wait
  // for them after the last MFMA (every epilogue but the fp32 partials scales its sums):
  // SwiGLU column tile nt of column half wc is gate (wc 0) or up (wc 1) unit u0 + nt, the
  // others tile NH wc + nt of the group.
  float scp[NH];
  {
    const bool scaled_out = a.swiglu || a.amax != nullptr || (a.split_k == 1 && !a.to_partial);
#pragma unroll
    for (int nt = 0; nt < NH; ++nt) {
      const int unit = a.swiglu ? nt : NH * wc + nt;
      const int col = a.swiglu ? wc * (a.N / 2) + n0 + 16 * nt + i : n0 + 16 * unit + i;
      scp[nt] = scaled_out && unit < nu ? a.scale[col] : 0.0f;
    }
  }

  for (int c = c_lo; c < c_hi; ++c) {
    const int st = (c - c_lo) % NSTAGE;
    // LDS here is written only by the DMA, whose completion vmcnt tracks: wait for this
    // thread's chunk-c transfers (chunk c+1 may stay in flight), then a plain s_barrier.
    // (__syncthreads() would add a workgroup fence, i.e. vmcnt(0), and drain the ring.)
    if (c + 1 < c_hi) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(XI + WI) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();  // chunk c is in LDS for every wave; stage (c+2)%3 is free
    asm volatile("" ::: "memory");
    if (c + 2 < c_hi) issue(c + 2, (c + 2 - c_lo) % NSTAGE);
    const uint8_t* xs = smem + st * STAGE;
    const uint8_t* ws = xs + XBYTES;
    // Every wave runs NH column tiles: tiles past the workgroup's nu read in-bounds LDS
    // (the next rows / stage slack) and are never stored.
    // All A and B fragments of the chunk are read first; the B tiles of k-step 0 are
    // converted, then k-step 0's MFMAs alternate with k-step 1's conversions, so the MFMA
    // stream is not stalled behind a convert-then-use chain per tile.
    bf16x8 aop[2][4];
    i32x2 raw[2][NH];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int row = 64 * wr + 16 * mt + i;
        const int pos = (4 * ks + G) ^ ((row >> 1) & 7);
        aop[ks][mt] = *reinterpret_cast<const bf16x8*>(xs + row * (KC * 2) + pos * 16);
      }
      const uint8_t* wrow = ws + (32 * ks + trow) * (16 * nup) + tcol;
#pragma unroll
      for (int nt = 0; nt < NH; ++nt) raw[ks][nt] = lds_tr8(wrow + 16 * nt);
    }
    bf16x8 bop[2][NH];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int nt = 0; nt < NH; ++nt) {
        u32x4 bw;
        bw[0] = fp8x2_to_bf16x2<false>((uint32_t)raw[ks][nt][0]);
        bw[1] = fp8x2_to_bf16x2<true>((uint32_t)raw[ks][nt][0]);
        bw[2] = fp8x2_to_bf16x2<false>((uint32_t)raw[ks][nt][1]);
        bw[3] = fp8x2_to_bf16x2<true>((uint32_t)raw[ks][nt][1]);
        bop[ks][nt] = __builtin_bit_cast(bf16x8, bw);
      }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int nt = 0; nt < NH; ++nt)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop[ks][mt], bop[ks][nt],
                                                                acc[mt][nt], 0, 0, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * (4 + NH), 0);  // LDS reads
    __builtin_amdgcn_sched_group_barrier(0x002, 4 * NH, 0);        // k-step 0 conversions
#pragma unroll
    for (int j = 0; j < 4 * NH; ++j) {                             // k-step 0 MFMAs with
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);           // k-step 1 conversions
      __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4 * NH, 0);        // k-step 1 MFMAs
  }

  // Epilogue: lane (i, G) holds rows 64wr + 16mt + 4G + r, column n0 + 16(NH wc + nt) + i.
  if (a.swiglu) {
    // Wave (wr, 1) holds up for exactly the rows and columns that wave (wr, 0) holds for gate,
    // lane for lane. The two split the SwiGLU: (wr, 0) finishes row blocks mt = 0, 1 and
    // (wr, 1) mt = 2, 3, each handing the other its bf16 values of the other's blocks through
    // LDS (the stages are free once every wave has passed the first barrier), then applying
    // the glue kernel's rounding.
    const int I = a.N / 2;
    __syncthreads();
    uint16_t* slot = reinterpret_cast<uint16_t*>(smem) + (size_t)(wr * 64 + lane) * (16 * NH);
#pragma unroll
    for (int nt = 0; nt < NH; ++nt) {
      if (nt >= nu) continue;
      const float sc = scp[nt];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        if ((mt >> 1) == wc) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) slot[16 * nt + 4 * mt + r] = npn::f32_to_bf16(acc[mt][nt][r] * sc);
      }
    }
    __syncthreads();
    // results go to a row-major staging tile past the exchange slots, then out in 16-byte
    // pieces (a row's 32 nu contiguous bytes per workgroup)
    constexpr int RSW = 16 * NH + 8;  // staged row stride in bf16 (16 bytes of padding)
    uint16_t* st = reinterpret_cast<uint16_t*>(smem + kSwigluStageOff<NH>);
#pragma unroll
    for (int nt = 0; nt < NH; ++nt) {
      if (nt >= nu) continue;
      const float sc = scp[nt];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        if ((mt >> 1) != wc) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 64 * wr + 16 * mt + 4 * G + r;
          const float own = npn::bf16_to_f32(npn::f32_to_bf16(acc[mt][nt][r] * sc));
          const float other = npn::bf16_to_f32(slot[16 * nt + 4 * mt + r]);
          const float g = wc == 0 ? own : other, u = wc == 0 ? other : own;
          const float sg = npn::bf16_to_f32(npn::f32_to_bf16(npn::silu_bf16(g)));
          st[row * RSW + 16 * nt + i] = npn::f32_to_bf16(sg * u);
        }
      }
    }
    __syncthreads();
    store_staged_bf16(st, RSW, a.out, I, m_base, a.M, n0, nu);
    return;
  }
  if (a.amax != nullptr) {
    float bv[4][4];
    int bi[4][4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        bv[mt][r] = -__builtin_inff();
        bi[mt][r] = 0x7FFFFFFF;
      }
#pragma unroll
    for (int nt = 0; nt < NH; ++nt) {
      const int unit = NH * wc + nt;
      if (unit >= nu) continue;
      const int col = n0 + 16 * unit + i;
      const float sc = scp[nt];
      // a lane meets its columns in increasing order, so after its first column a later one
      // wins only by being strictly larger, or NaN against a number (the first NaN stays):
      // arg_beats for a larger index
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v = bf16_round(acc[mt][nt][r] * sc);
          const float b = bv[mt][r];
          if (bi[mt][r] == 0x7FFFFFFF || (b == b && (v > b || v != v))) {
            bv[mt][r] = v;
            bi[mt][r] = col;
          }
        }
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) arg_merge16_dpp(bv[mt][r], bi[mt][r]);
    // The column half wc = 1 hands its per-row bests to wc = 0 through LDS (the stages are
    // free once every wave has passed this barrier).
    __syncthreads();
    ArgPart* sh = reinterpret_cast<ArgPart*>(smem);
    if (wc == 1 && i == 0) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) sh[64 * wr + 16 * mt + 4 * G + r] = ArgPart{bv[mt][r], bi[mt][r]};
    }
    __syncthreads();
    if (wc == 0 && i == 0) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 64 * wr + 16 * mt + 4 * G + r;
          ArgPart best{bv[mt][r], bi[mt][r]};
          const ArgPart o = sh[row];
          if (arg_beats(o.v, o.i, best.v, best.i)) best = o;
          const int m = m_base + row;
          if (m < a.M) a.amax[(size_t)m * a.groups + grp] = best;
        }
    }
    return;
  }
  // Outputs are staged row-major in LDS (the ring is free once every wave has passed this
  // barrier) and written in 16-byte pieces: 2-byte or 64-byte-run stores straight from the
  // MFMA layout cost several times the bytes' time.
  __syncthreads();
  if (a.split_k == 1 && !a.to_partial) {
    constexpr int RSW = 32 * NH + 8;  // staged row stride in bf16 (16 bytes of padding)
    uint16_t* st = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
    for (int nt = 0; nt < NH; ++nt) {
      const int unit = NH * wc + nt;
      if (unit >= nu) continue;
      const float sc = scp[nt];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          st[(64 * wr + 16 * mt + 4 * G + r) * RSW + 16 * unit + i] =
              npn::f32_to_bf16(acc[mt][nt][r] * sc);
    }
    __syncthreads();
    store_staged_bf16(st, RSW, a.out, a.N, m_base, a.M, n0, nu);
    if (a.gmax != nullptr) staged_row_max(st, RSW, a.gmax, a.groups, grp, m_base, a.M, nu);
    if (a.cmax != nullptr)
      staged_chunk_stats(st, RSW, a.cmax, a.csum, a.inv_temp, a.N / 64, m_base, a.M, n0, nu);
    return;
  }
  // fp32 partials (unscaled; the scale pointer may then be NULL), staged 128 rows at a time
  constexpr int RSF = 32 * NH + 4;  // staged row stride in floats (16 bytes of padding)
  float* stf = reinterpret_cast<float*>(smem);
  float* part = a.partial + (size_t)sk * a.M * a.N;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    if ((wr >> 1) == half) {
#pragma unroll
      for (int nt = 0; nt < NH; ++nt) {
        const int unit = NH * wc + nt;
        if (unit >= nu) continue;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            stf[(64 * (wr & 1) + 16 * mt + 4 * G + r) * RSF + 16 * unit + i] = acc[mt][nt][r];
      }
    }
    __syncthreads();
    const int pieces = 4 * nu;  // 16-byte pieces per staged row
    for (int p = tid; p < 128 * pieces; p += WIDE_THREADS) {
      const int row = p / pieces, q = p - row * pieces;
      const int m = m_base + 128 * half + row;
      if (m < a.M)
        *reinterpret_cast<float4*>(part + (size_t)m * a.N + n0 + 4 * q) =
            *reinterpret_cast<const float4*>(stf + row * RSF + 4 * q);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------------
// The wide kernel on 128-row tiles (64 < M), chosen by the plan where it needs less padded
// MFMA work per CU than the 256-row kernel at the same split-K factor. Row tiles of one
// column group take adjacent logical workgroup indices, so they run on one XCD at the same
// time and each W byte comes from HBM once; each CU streams half the x block of the 256-row
// kernel, and its W row pieces are about twice as long.
// Waves: row half rh = w >> 2 (64 rows) and column quarter q. The workgroup's units form two
// halves of H units, each half two quarters of NH and NH - ODD column tiles; quarters 0/1 are
// half 0 and 2/3 half 1 (SwiGLU: half 0 gate units, half 1 the up units N/2 to their right,
// so quarter q and q + 2 hold gate and up for the same rows and columns, lane for lane).
// With ODD the quarters of one SIMD's two waves are q and q ^ 1 (q = (w & 3) ^ rh, the waves
// of a workgroup going to the SIMDs in turn), one long and one short: every SIMD issues
// 2 NH - 1 tiles' MFMAs per k step, and a workgroup holds 4 NH - 2 units instead of 4 NH,
// a granularity that fits the step's shapes into 256 workgroups with less padding (gate/up:
// 121 groups of 18 units instead of 218 of 10 at 256 rows). Same x / W stage layouts, DMA,
// B-operand reads and per-output k order as the 256-row kernel (the ring four stages deep
// where it fits), so every output (and every split-K partial) is bit-identical to it.
template <int N>
struct TileCount {
  static constexpr int value = N;
};

template <int NH, bool ODD>
__global__ __launch_bounds__(WIDE_THREADS, 1) void fp8_gemm_wide128_kernel(WideArgs a) {
  constexpr int H = ODD ? 2 * NH - 1 : 2 * NH;  // units per half
  constexpr int QN0 = NH, QN1 = ODD ? NH - 1 : NH;
  constexpr int NUP = 2 * H + 1;                // W stage row stride in 16-byte units (odd)
  constexpr int XBYTES = 128 * KC * 2;          // 16 KiB x stage
  constexpr int XI = XBYTES / (WIDE_THREADS * 16);
  constexpr int WI = (KC * NUP + WIDE_THREADS - 1) / WIDE_THREADS;
  constexpr int WBYTES = WI * WIDE_THREADS * 16;
  constexpr int STAGE = XBYTES + WBYTES;
  // a 4-stage ring (three chunks in flight) wherever it fits the 160 KiB of LDS: at gate/up
  // (H = 9) 107 -> 103 us against 3 stages, same box
  constexpr int NSTG = 4 * STAGE <= 160 * 1024 ? 4 : 3;
  __shared__ __attribute__((aligned(16))) uint8_t smem[NSTG * STAGE];
  constexpr int RSW = 32 * H + 8;  // bf16 staging row stride (16 bytes of padding)
  constexpr int RSF = 32 * H + 4;  // fp32 staging row stride, 64 rows at a time
  constexpr int SWOFF = 4 * 64 * 16 * NH * 2;  // SwiGLU staging past the exchange slots
  constexpr int RS2 = 16 * H + 8;
  static_assert(128 * RSW * 2 <= NSTG * STAGE, "bf16 staging exceeds the LDS ring");
  static_assert(64 * RSF * 4 <= NSTG * STAGE, "fp32 staging exceeds the LDS ring");
  static_assert(SWOFF + 128 * RS2 * 2 <= NSTG * STAGE, "SwiGLU staging exceeds the LDS ring");

  const int nwg = gridDim.x;
  const int per_xcd = nwg / 8;
  const int logical = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  const int rtiles = (a.M + 127) >> 7;
  const int rt = logical % rtiles;
  const int gs = logical / rtiles;
  const int sk = gs % a.split_k;
  const int grp = gs / a.split_k;
  if (grp >= a.groups) return;
  const int u0 = (int)((long)grp * a.units / a.groups);
  const int u1 = (int)((long)(grp + 1) * a.units / a.groups);
  const int nu = u1 - u0;  // units (SwiGLU: gate units) of this group
  if (nu <= 0) return;
  const int n0 = 16 * u0;
  const int nch_all = a.K / KC;
  const int c_lo = (int)((long)nch_all * sk / a.split_k);
  const int nchunks = (int)((long)nch_all * (sk + 1) / a.split_k) - c_lo;
  const int m_base = rt * 128;
  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int rh = wv >> 2;
  const int q = (wv & 3) ^ (ODD ? rh : 0);
  const int qslot = (q >= 2 ? H : 0) + ((q & 1) ? QN0 : 0);  // the quarter's first unit slot
  const bool is_short = ODD && (q & 1);
  const int i = lane & 15, G = lane >> 4;
  const int mlast = a.M - 1;
  const int halfcol = a.swiglu ? a.N / 2 : 16 * H;  // column offset of half 1

  // DMA of chunk c (relative to c_lo) into stage st: x rows, then W rows.
  auto issue = [&](int c, int st) {
    uint8_t* xs = smem + st * STAGE;
    uint8_t* ws = xs + XBYTES;
    const int kc = (c_lo + c) * KC;
#pragma unroll
    for (int qq = 0; qq < XI; ++qq) {
      const int f = qq * WIDE_THREADS + tid;  // 16-byte slot in the x stage
      const int row = f >> 3, pos = f & 7;
      int m = m_base + row;
      m = m <= mlast ? m : mlast;
      const uint16_t* src = a.x + (size_t)m * a.K + kc + 8 * (pos ^ ((row >> 1) & 7));
      npn::lds_dma16(src, xs + qq * (WIDE_THREADS * 16) + (tid & ~63) * 16);
    }
#pragma unroll
    for (int qq = 0; qq < WI; ++qq) {
      int f = qq * WIDE_THREADS + tid;        // 16-byte slot of the W stage
      if (f >= KC * NUP) f = 0;               // lanes past the stage re-read slot 0 (slack)
      const int r = f / NUP;
      const int s = f - r * NUP;
      int col;
      if (a.swiglu) {                         // slots [0, H) gate, [H, 2H) up, 2H pad
        const int hs = s >= H && s < 2 * H ? 1 : 0;
        int uu = s - H * hs;
        uu = uu < nu ? uu : 0;                // unused or pad slot: re-read unit u0
        col = n0 + 16 * uu + hs * halfcol;
      } else {
        col = n0 + 16 * (s < nu ? s : 0);
      }
      const uint8_t* src = a.w + (size_t)(kc + r) * a.N + col;
      npn::lds_dma16(src, ws + qq * (WIDE_THREADS * 16) + (tid & ~63) * 16);
    }
  };

  f32x4 acc[4][NH];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < NH; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int trow = 8 * G + (i >> 1);
  const int tcol = 8 * (i & 1) + 16 * qslot;

#pragma unroll
  for (int c = 0; c < NSTG - 1; ++c)
    if (c < nchunks) issue(c, c);
  // column scales of this lane's tiles, loaded before the main loop (scaled epilogues only)
  const bool scaled_out = a.swiglu || (a.split_k == 1 && !a.to_partial);
  float scp[NH];
#pragma unroll
  for (int nt = 0; nt < NH; ++nt) {
    const int s = qslot + nt;
    const int hs = s >= H ? 1 : 0;
    const int uu = s - H * hs;
    const bool ok = a.swiglu ? uu < nu : s < nu;
    scp[nt] = scaled_out && ok ? a.scale[n0 + 16 * uu + hs * halfcol + i] : 0.0f;
  }

  // The chunk loop for a wave of NTW column tiles (both loops pass the same barriers).
  auto main_loop = [&](auto tiles) {
    constexpr int NTW = decltype(tiles)::value;
    for (int c = 0; c < nchunks; ++c) {
      const int st = c % NSTG;
      // this thread's chunk-c DMAs have landed once at most those of the chunks after it
      // (up to NSTG - 2 of them, XI + WI each) are outstanding
      if (NSTG == 4 && c + 2 < nchunks) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * (XI + WI)) : "memory");
      else if (c + 1 < nchunks) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(XI + WI) : "memory");
      else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();  // chunk c is in LDS for every wave; stage (c - 1) % NSTG is free
      asm volatile("" ::: "memory");
      if (c + NSTG - 1 < nchunks) issue(c + NSTG - 1, (c + NSTG - 1) % NSTG);
      const uint8_t* xs = smem + st * STAGE;
      const uint8_t* ws = xs + XBYTES;
      bf16x8 aop[2][4];
      i32x2 raw[2][NTW];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          const int row = 64 * rh + 16 * mt + i;
          const int pos = (4 * ks + G) ^ ((row >> 1) & 7);
          aop[ks][mt] = *reinterpret_cast<const bf16x8*>(xs + row * (KC * 2) + pos * 16);
        }
        const uint8_t* wrow = ws + (32 * ks + trow) * (16 * NUP) + tcol;
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) raw[ks][nt] = lds_tr8(wrow + 16 * nt);
      }
      bf16x8 bop[2][NTW];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) {
          u32x4 bw;
          bw[0] = fp8x2_to_bf16x2<false>((uint32_t)raw[ks][nt][0]);
          bw[1] = fp8x2_to_bf16x2<true>((uint32_t)raw[ks][nt][0]);
          bw[2] = fp8x2_to_bf16x2<false>((uint32_t)raw[ks][nt][1]);
          bw[3] = fp8x2_to_bf16x2<true>((uint32_t)raw[ks][nt][1]);
          bop[ks][nt] = __builtin_bit_cast(bf16x8, bw);
        }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
          for (int mt = 0; mt < 4; ++mt)
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop[ks][mt], bop[ks][nt],
                                                                  acc[mt][nt], 0, 0, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * (4 + NTW), 0);  // LDS reads
      __builtin_amdgcn_sched_group_barrier(0x002, 4 * NTW, 0);        // k-step 0 conversions
#pragma unroll
      for (int j = 0; j < 4 * NTW; ++j) {                             // k-step 0 MFMAs with
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);            // k-step 1 conversions
        __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4 * NTW, 0);        // k-step 1 MFMAs
    }
  };
  if (is_short) main_loop(TileCount<QN1>{});
  else main_loop(TileCount<QN0>{});
  const int ntw = is_short ? QN1 : QN0;

  // Epilogues: lane (i, G) holds rows 64 rh + 16 mt + 4 G + r, unit slot qslot + nt, column i.
  if (a.swiglu) {
    // The gate wave (quarter q < 2) finishes row blocks 0-1 and the up wave (q + 2) blocks
    // 2-3, each handing the other its bf16 values of the other's blocks through LDS.
    const int I = a.N / 2;
    __syncthreads();
    const int pair = rh * 2 + (q & 1);
    const int gw = q >> 1;  // 0 gate, 1 up
    uint16_t* slot = reinterpret_cast<uint16_t*>(smem) + (size_t)(pair * 64 + lane) * (16 * NH);
#pragma unroll
    for (int nt = 0; nt < NH; ++nt) {
      if (nt >= ntw) continue;
      const float sc = scp[nt];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        if ((mt >> 1) == gw) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) slot[16 * nt + 4 * mt + r] = npn::f32_to_bf16(acc[mt][nt][r] * sc);
      }
    }
    __syncthreads();
    uint16_t* st = reinterpret_cast<uint16_t*>(smem + SWOFF);
    const int gbase = (q & 1) ? QN0 : 0;  // gate unit of this wave's tile 0
#pragma unroll
    for (int nt = 0; nt < NH; ++nt) {
      if (nt >= ntw) continue;
      const float sc = scp[nt];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        if ((mt >> 1) != gw) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 64 * rh + 16 * mt + 4 * G + r;
          const float own = npn::bf16_to_f32(npn::f32_to_bf16(acc[mt][nt][r] * sc));
          const float other = npn::bf16_to_f32(slot[16 * nt + 4 * mt + r]);
          const float g = gw == 0 ? own : other, u = gw == 0 ? other : own;
          const float sg = npn::bf16_to_f32(npn::f32_to_bf16(npn::silu_bf16(g)));
          st[row * RS2 + 16 * (gbase + nt) + i] = npn::f32_to_bf16(sg * u);
        }
      }
    }
    __syncthreads();
    const int pieces = 2 * nu;
    for (int p = tid; p < 128 * pieces; p += WIDE_THREADS) {
      const int row = p / pieces, qq = p - row * pieces;
      const int m = m_base + row;
      if (m < a.M)
        *reinterpret_cast<uint4*>(a.out + (size_t)m * I + n0 + 8 * qq) =
            *reinterpret_cast<const uint4*>(st + row * RS2 + 8 * qq);
    }
    return;
  }
  __syncthreads();
  if (a.split_k == 1 && !a.to_partial) {
    uint16_t* st = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
    for (int nt = 0; nt < NH; ++nt) {
      const int s = qslot + nt;
      if (nt >= ntw || s >= nu) continue;
      const float sc = scp[nt];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          st[(64 * rh + 16 * mt + 4 * G + r) * RSW + 16 * s + i] =
              npn::f32_to_bf16(acc[mt][nt][r] * sc);
    }
    __syncthreads();
    const int pieces = 2 * nu;
    for (int p = tid; p < 128 * pieces; p += WIDE_THREADS) {
      const int row = p / pieces, qq = p - row * pieces;
      const int m = m_base + row;
      if (m < a.M)
        *reinterpret_cast<uint4*>(a.out + (size_t)m * a.N + n0 + 8 * qq) =
            *reinterpret_cast<const uint4*>(st + row * RSW + 8 * qq);
    }
    return;
  }
  // fp32 partials (unscaled) into slot sk, staged one row half at a time
  float* stf = reinterpret_cast<float*>(smem);
  float* part = a.partial + (size_t)sk * a.M * a.N;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    if (rh == half) {
#pragma unroll
      for (int nt = 0; nt < NH; ++nt) {
        const int s = qslot + nt;
        if (nt >= ntw || s >= nu) continue;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r) stf[(16 * mt + 4 * G + r) * RSF + 16 * s + i] = acc[mt][nt][r];
      }
    }
    __syncthreads();
    const int pieces = 4 * nu;  // 16-byte pieces per staged row
    for (int p = tid; p < 64 * pieces; p += WIDE_THREADS) {
      const int row = p / pieces, qq = p - row * pieces;
      const int m = m_base + 64 * half + row;
      if (m < a.M)
        *reinterpret_cast<float4*>(part + (size_t)m * a.N + n0 + 4 * qq) =
            *reinterpret_cast<const float4*>(stf + row * RSF + 4 * qq);
    }
    __syncthreads();
  }
}

// out = bf16(scale * sum_s partial[s]), summed in order s = 0..split_k-1.
__global__ void fp8_splitk_reduce_kernel(const float* __restrict__ partial,
                                         const float* __restrict__ scale,
                                         uint16_t* __restrict__ out, int M, int N, int split_k) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t total = (size_t)M * N;
  if (idx >= total) return;
  float s = 0.f;
  for (int k = 0; k < split_k; ++k) s += partial[(size_t)k * total + idx];
  out[idx] = npn::f32_to_bf16(s * scale[idx % N]);
}

// SwiGLU of split-K partials of W = [gate | up] (N = 2 I): out[m][j] =
// bf16(bf16(silu(g)) * u), g and u the bf16 outputs bf16(scale * sum_s partial[s]) of columns
// j and I + j (the reduction above, then the glue kernel's SwiGLU rounding).
__global__ void fp8_splitk_swiglu_kernel(const float* __restrict__ partial,
                                         const float* __restrict__ scale,
                                         uint16_t* __restrict__ out, int M, int N, int split_k) {
  const int I = N / 2;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)M * I) return;
  const size_t m = idx / I, j = idx - m * I;
  const size_t total = (size_t)M * N;
  const float* pg = partial + m * N + j;
  float g = 0.f, u = 0.f;
  for (int k = 0; k < split_k; ++k) {
    g += pg[(size_t)k * total];
    u += pg[(size_t)k * total + I];
  }
  const float gb = npn::bf16_to_f32(npn::f32_to_bf16(g * scale[j]));
  const float ub = npn::bf16_to_f32(npn::f32_to_bf16(u * scale[I + j]));
  const float sb = npn::bf16_to_f32(npn::f32_to_bf16(npn::silu_bf16(gb)));
  out[idx] = npn::f32_to_bf16(sb * ub);
}

struct GemmPlan {
  int mt, passes, split_k;
  size_t ws;
  bool wide;
  int units, groups, ntm;
  int sk_wg;   // narrow: stream-K workgroups (0: a tiles x split_k grid)
  int ualign;  // wide: column groups hold whole runs of ualign 16-column units
  // wide on 128-row tiles (fp8_gemm_wide128_kernel<ntm, odd>): groups column groups of up to
  // 2 h128 units, each run for every 128-row tile
  bool rows128, odd;
  int h128;
};

// 128-row wide kernel instantiations (NH, ODD), by units per half H = 2 NH - ODD: a
// workgroup holds up to 2 H units (SwiGLU: H gate units and their up units).
struct Wide128Cfg {
  int nh;
  bool odd;
};
constexpr Wide128Cfg kWide128[] = {{1, false}, {2, true}, {2, false}, {3, true}, {3, false},
                                   {4, true},  {4, false}, {5, true}, {5, false}, {6, true},
                                   {6, false}};

// Wide-kernel instantiations: column tiles per wave (a workgroup holds twice as many units).
// 7 is the widest whose 3-stage ring fits the 160 KiB of LDS (8 would need 168 KiB).
constexpr int kWideNH[] = {1, 2, 3, 4, 5, 6, 7};

// Wide-kernel plan: split-K factor s, column groups g (one workgroup per (group, split)),
// column tiles per wave ntm. Modelled time, additive because the three do not overlap well
// in this kernel (fitted to measurements at M = 256 on MI355X):
//   x:        every workgroup streams its 256 x (K / s) activation block from L2 into LDS,
//             at about 51 GB/s per CU when all CUs do so at once;
//   MFMA:     a workgroup computes 2 * ntm 16-column tiles whether or not all are real
//             columns, at about 2.07 PFLOP/s / 256 per CU (two waves per SIMD);
//   split-K:  partials written by the GEMM and read by the reduction, about 4.5 TB/s while
//             one split-K buffer stays under 48 MB, plus the reduction's launch.
// For each s the smallest ntm whose group count ceil(units / (2 ntm)) fits in 256 / s
// workgroups is taken: fewest padded tiles, and every workgroup's tiles nearly all real.
// Wider N (an LM head's vocabulary) runs in rounds of 256 workgroups of the widest tiles,
// without split-K. `no_split` (the argmax epilogue, which needs whole sums) keeps s = 1.
// ua > 1 makes every column group a whole number of ua-unit runs (4: the 64-column chunks of
// the acceptance statistics), so a group of up to 2 ntm units holds floor(2 ntm / ua) runs.
bool plan_wide(int M, int K, int N, GemmPlan& p, bool no_split, int ua) {
  if (M <= 64 || K % KC != 0 || N % (16 * ua) != 0) return false;
  const int units = N / 16;
  const int passes = (M + 255) / 256;
  double best = 1e30;
  for (int s = 1; s <= (no_split ? 1 : 8); s *= 2) {
    if (K / KC < 2 * s) break;
    const double part_bytes = (double)s * M * N * 4;
    if (s > 1 && part_bytes > 48e6) break;
    const int gmax = WIDE_WG / s;
    const int runs = units / ua;
    int ntm = 0, groups = 0;
    for (int v : kWideNH) {
      const int cap = 2 * v / ua;  // runs per group
      if (cap == 0) continue;
      const int g = (runs + cap - 1) / cap;
      if (g <= gmax) { ntm = v; groups = g; break; }
    }
    if (ntm == 0) {
      if (s > 1) continue;
      ntm = kWideNH[sizeof(kWideNH) / sizeof(kWideNH[0]) - 1];
      const int cap = 2 * ntm / ua;
      groups = (runs + cap - 1) / cap;
    }
    const int rounds = (groups * s + WIDE_WG - 1) / WIDE_WG;
    const double kk = (double)K / s;
    const double t_x = kk * 512.0 / 51e9;
    const double t_mfma = 2.0 * ntm * 16 * 256 * 2 * kk / (2.07e15 / WIDE_WG);
    const double t_part = s > 1 ? 2.0 * part_bytes / 4.5e12 + 3e-6 : 0.0;
    const double t = (t_x + t_mfma) * passes * rounds + t_part;
    if (t < best * 0.97) {
      best = t;
      p.wide = true;
      p.units = units;
      p.groups = groups;
      p.split_k = s;
      p.ntm = ntm;
    }
  }
  if (!p.wide) return false;
  p.passes = passes;
  p.ualign = ua;
  p.ws = p.split_k > 1 ? (size_t)p.split_k * M * N * sizeof(float) : 0;
  return true;
}

// The 128-row kernel at the 256-row plan's split-K factor s, when its whole grid fits in one
// round of 256 workgroups and it computes at most 92 % of the padded MFMA work per workgroup
// (128 rows x 2 H units against 256 rows x 2 ntm units per pass and round). Measured on
// MI355X at M = 256, weights rotated through 700 MB, against the 256-row kernel at the same
// split: gate/up 5120 x 34816 with the SwiGLU epilogue 111 -> 99 us (H = 9, 242 workgroups),
// q/k/v 5120 x 14336 split 2 45.9 -> 43.1 us, out-projection 6144 x 5120 split 4 26.5 ->
// 24.8 us, DeltaNet in-projection 5120 x 16512 split 2 51.8 -> 50.9 us; at equal padded
// work (down, 17408 x 5120 split 8: 52.1 against 54.5 us) the 256-row kernel stays.
void plan_wide128(int M, GemmPlan& p) {
  const int rtiles = (M + 127) / 128;
  const int s = p.split_k;
  for (const Wide128Cfg& c : kWide128) {
    const int h = 2 * c.nh - (c.odd ? 1 : 0);
    const int groups = (p.units + 2 * h - 1) / (2 * h);
    if ((long)groups * rtiles * s > WIDE_WG) continue;
    const int rounds = (p.groups * s + WIDE_WG - 1) / WIDE_WG;
    const long work128 = 128L * 2 * h;
    const long work256 = 256L * 2 * p.ntm * p.passes * rounds;
    if (100 * work128 <= 92 * work256) {
      p.rows128 = true;
      p.odd = c.odd;
      p.ntm = c.nh;
      p.h128 = h;
      p.groups = groups;
    }
    return;
  }
}

GemmPlan plan(int M, int K, int N, bool no_split = false, int ua = 1) {
  GemmPlan p{};
  if (plan_wide(M, K, N, p, no_split, ua)) {
    // the argmax and chunk-statistics epilogues exist only in the 256-row kernel
    if (!no_split && ua == 1) plan_wide128(M, p);
    return p;
  }
  p = GemmPlan{};
  p.ualign = 1;
  // Narrow plan: one pass of RB = 1, 2 or 4 row blocks (M <= 64), and a split-K factor: the
  // largest power of two up to 8 whose grid stays at or under 576 workgroups (up to 16 and
  // 1152 workgroups for at most 16 rows, whose partials are small) with at least 8 k steps
  // each. Measured on MI355X at
  // M = 8, 32 and 64, K = 5120, N = 5120 / 17408 / 34816 (GEMM plus reduction, weights
  // rotated through 600 MB): one workgroup per CU keeps only NS - 1 tiles in flight and
  // reaches about 21 GB/s per CU, so the split that engages every CU wins (N = 34816 split
  // 4: 0.092 -> 0.070 ms at M = 64; split 8: 0.043 -> 0.040 ms at M = 8) until the partial
  // traffic outgrows it.
  const int mtiles = (M + 15) / 16;
  p.mt = mtiles >= 3 ? 4 : mtiles;
  p.passes = (M + 16 * p.mt - 1) / (16 * p.mt);
  const int tiles = ((N + NT - 1) / NT) * p.passes;
  const int nks = K / KSTEP;
  const int max_wg = M <= 16 ? 1152 : 576;
  const int max_split = M <= 16 ? 16 : 8;
  p.split_k = 1;
  while (!no_split && p.split_k < max_split && tiles * p.split_k * 2 <= max_wg &&
         nks >= 16 * p.split_k)
    p.split_k *= 2;
  // Stream-K where the tiles x split grid cannot fill the CUs evenly (136 tiles x 4 = 544
  // workgroups leave 32 CUs with three while the rest run two): up to 512 workgroups (two per
  // CU) share the tiles' k steps equally, at least 8 each, with at most 8 partial slots per
  // tile (so at most 7 workgroups' shares per tile). Measured on MI355X, M = 64, K = 5120: a
  // 512-workgroup grid (N = 32768, split 4) streams W at 3.3 TB/s, the 544 of N = 34816 at
  // 2.9 TB/s.
  if (!no_split && p.passes == 1 && tiles < 256) {
    const long W = 7L * tiles < 512 ? 7L * tiles : 512;
    const long U = (long)tiles * nks;
    if (W > 384 && U >= 8 * W) {
      int slots = 0;
      for (long t = 0; t < tiles; ++t) {
        const long wfirst = ((t * nks + 1) * W - 1) / U, wlast = (((t + 1) * nks) * W - 1) / U;
        slots = (int)(wlast - wfirst + 1) > slots ? (int)(wlast - wfirst + 1) : slots;
      }
      if (slots >= 2 && slots <= 8) {
        p.sk_wg = (int)W;
        p.split_k = slots;
      }
    }
  }
  p.ws = p.split_k > 1 ? (size_t)p.split_k * M * N * sizeof(float) : 0;
  return p;
}

// Column slices per narrow tile (the kernel's CH = waves / row blocks): its row-maximum and
// argmax groups are (tile, slice) pairs.
int narrow_slices(int mt) { return mt == 1 ? 4 : (mt == 2 ? 4 : 2); }

bool shape_ok(int M, int K, int N) {
  return M >= 1 && M <= 4096 && K >= 64 && K % 64 == 0 && N >= 64 && N % 64 == 0 &&
         (long)K * N < (1L << 40);
}

// Launches the plan's GEMM kernel; with split-K (or to_partial) it writes fp32 partials
// [split_k][M][N] to `partial` and, when `reduce`, the fixed-order reduction into `out`.
int launch_gemm(const GemmPlan& p, const uint16_t* x, const int8_t* w, const float* scale,
                uint16_t* out, float* partial, int M, int K, int N, int to_partial, bool reduce,
                hipStream_t s, ArgPart* amax = nullptr, bool swiglu = false,
                float* gmax = nullptr, float* cmax = nullptr, uint64_t* csum = nullptr,
                float inv_temp = 1.0f) {
  if (p.wide && p.rows128) {
    // amax / gmax / cmax are never requested on these plans (the planner keeps them on the
    // 256-row kernel)
    WideArgs wa{x, reinterpret_cast<const uint8_t*>(w), scale, out, partial, M, K, N,
                swiglu ? p.units / 2 : p.units, p.groups, p.split_k, to_partial, nullptr,
                nullptr, swiglu ? 1 : 0, 1, nullptr, nullptr, 1.0f};
    const int rtiles = (M + 127) / 128;
    const dim3 grid(((p.groups * rtiles * p.split_k + 7) / 8) * 8);
    const dim3 block(WIDE_THREADS);
#define NPN_W128(NH, ODD) \
  if (p.ntm == NH && p.odd == ODD) hipLaunchKernelGGL((fp8_gemm_wide128_kernel<NH, ODD>), grid, block, 0, s, wa)
    NPN_W128(1, false);
    NPN_W128(2, true);
    NPN_W128(2, false);
    NPN_W128(3, true);
    NPN_W128(3, false);
    NPN_W128(4, true);
    NPN_W128(4, false);
    NPN_W128(5, true);
    NPN_W128(5, false);
    NPN_W128(6, true);
    NPN_W128(6, false);
#undef NPN_W128
  } else if (p.wide) {
    // SwiGLU: the same groups, each of at most ntm gate units (plus their up units)
    WideArgs wa{x, reinterpret_cast<const uint8_t*>(w), scale, out, partial, M, K, N,
                swiglu ? p.units / 2 : p.units, p.groups, p.split_k, to_partial, amax, gmax,
                swiglu ? 1 : 0, p.ualign, cmax, csum, inv_temp};
    const int nwg = ((p.groups * p.split_k + 7) / 8) * 8;  // multiple of 8 for the XCD map
    const dim3 grid(nwg, p.passes);
    const dim3 block(WIDE_THREADS);
    switch (p.ntm) {
      case 1: hipLaunchKernelGGL(fp8_gemm_wide_kernel<1>, grid, block, 0, s, wa); break;
      case 2: hipLaunchKernelGGL(fp8_gemm_wide_kernel<2>, grid, block, 0, s, wa); break;
      case 3: hipLaunchKernelGGL(fp8_gemm_wide_kernel<3>, grid, block, 0, s, wa); break;
      case 4: hipLaunchKernelGGL(fp8_gemm_wide_kernel<4>, grid, block, 0, s, wa); break;
      case 5: hipLaunchKernelGGL(fp8_gemm_wide_kernel<5>, grid, block, 0, s, wa); break;
      case 6: hipLaunchKernelGGL(fp8_gemm_wide_kernel<6>, grid, block, 0, s, wa); break;
      default: hipLaunchKernelGGL(fp8_gemm_wide_kernel<7>, grid, block, 0, s, wa); break;
    }
  } else {
    GemmArgs ga{x, reinterpret_cast<const uint8_t*>(w), scale, out, partial, M, K, N, p.split_k,
                to_partial, amax, gmax, p.sk_wg, cmax, csum, inv_temp};
    const dim3 grid = p.sk_wg > 0 ? dim3(p.sk_wg, 1, 1) : dim3((N + NT - 1) / NT, p.split_k, p.passes);
    switch (p.mt) {
      case 1: hipLaunchKernelGGL((fp8_gemm_narrow_kernel<1, 4, 4>), grid, dim3(256), 0, s, ga); break;
      case 2: hipLaunchKernelGGL((fp8_gemm_narrow_kernel<2, 4, 8>), grid, dim3(512), 0, s, ga); break;
      default: hipLaunchKernelGGL((fp8_gemm_narrow_kernel<4, 4, 8>), grid, dim3(512), 0, s, ga); break;
    }
  }
  if (reduce && p.split_k > 1) {
    const size_t total = (size_t)M * N;
    hipLaunchKernelGGL(fp8_splitk_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256),
                       0, s, partial, scale, out, M, N, p.split_k);
  }
  return npn_launch_status();
}

// The split-K partials of two GEMMs of the same x ([M, K], M <= 64) in one narrow launch,
// W1 [K, N1] into p1 [S][M][N1] and W2 [K, N2] into p2 [S][M][N2]: the same tiles, k ranges
// and sums as two launches of their plans, which must be narrow tiles x split grids with one
// pass and the same row blocks and split-K factor S. Returns false (nothing launched) when
// they are not.
bool launch_gemm_pair_partials(const uint16_t* x, const int8_t* w1, float* p1, int N1,
                               const int8_t* w2, float* p2, int N2, int M, int K,
                               hipStream_t s) {
  const GemmPlan a = plan(M, K, N1), b = plan(M, K, N2);
  if (a.wide || b.wide || a.sk_wg > 0 || b.sk_wg > 0 || a.passes != 1 || b.passes != 1 ||
      a.mt != b.mt || a.split_k != b.split_k)
    return false;
  const int t1 = (N1 + NT - 1) / NT, t2 = (N2 + NT - 1) / NT;
  GemmArgs ga{x, reinterpret_cast<const uint8_t*>(w1), nullptr, nullptr, p1, M, K, N1,
              a.split_k, 1, nullptr, nullptr, 0, nullptr, nullptr, 1.0f,
              reinterpret_cast<const uint8_t*>(w2), p2, N2, t1};
  const dim3 grid(t1 + t2, a.split_k, 1);
  switch (a.mt) {
    case 1: hipLaunchKernelGGL((fp8_gemm_narrow_kernel<1, 4, 4>), grid, dim3(256), 0, s, ga); break;
    case 2: hipLaunchKernelGGL((fp8_gemm_narrow_kernel<2, 4, 8>), grid, dim3(512), 0, s, ga); break;
    default: hipLaunchKernelGGL((fp8_gemm_narrow_kernel<4, 4, 8>), grid, dim3(512), 0, s, ga); break;
  }
  return true;
}

// The end of deltanet::full_fp8's in-projections, in one launch after the two GEMMs:
//  - blocks [0, nq): the qkv GEMM's split-K partials reduced in slot order and scaled into
//    bf16 mixed_qkv (the values npn_fp8_matmul writes; a sum of one slot is that slot), and the
//    new conv window [conv_state[:, 1:] | mixed_qkv];
//  - blocks [nq, nq + nz): the same reduction for z;
//  - the last 2 * hv blocks: the thin in_proj_a / in_proj_b projections in float32, column n
//    of matrix j per block: out_j[n] = (sum_k x[k] * W_j[k][n]) * scale_j[n], W_j [K, hv]
//    e4m3fn bytes (rows hv bytes apart: the two matrices are a few hundred KB, read once from
//    HBM and then from L2). Thread t adds k = t, t + 256, ... in order, then the wave sums
//    (fixed butterfly) and the four waves in order: the same bits every run.
struct InprojFinishArgs {
  const float* pq;          // [sq][qkv] partials of x . qkv_w
  const float* qs;
  uint16_t* mixed;
  const uint16_t* conv_in;  // [qkv][3]
  uint16_t* conv_out;
  const float* pz;          // [sz][zn] partials of x . z_w
  const float* zs;
  uint16_t* z;
  const uint16_t* x;
  const uint8_t* wa;
  const float* sa;
  float* a;
  const uint8_t* wb;
  const float* sb;
  float* b;
  int sq, qkv, sz, zn, K, hv;
};

__global__ __launch_bounds__(256) void dn_fp8_inproj_finish_kernel(InprojFinishArgs p) {
  const int nq = (p.qkv + 255) / 256, nz = (p.zn + 255) / 256;
  const int blk = blockIdx.x;
  if (blk < nq + nz) {
    const bool isq = blk < nq;
    const int n = isq ? p.qkv : p.zn;
    const int i = (isq ? blk : blk - nq) * 256 + threadIdx.x;
    if (i >= n) return;
    const float* P = isq ? p.pq : p.pz;
    const int S = isq ? p.sq : p.sz;
    float acc = P[i];
    for (int k = 1; k < S; ++k) acc += P[(size_t)k * n + i];
    const uint16_t v = npn::f32_to_bf16(acc * (isq ? p.qs : p.zs)[i]);
    if (isq) {
      p.mixed[i] = v;
      p.conv_out[3 * i] = p.conv_in[3 * i + 1];
      p.conv_out[3 * i + 1] = p.conv_in[3 * i + 2];
      p.conv_out[3 * i + 2] = v;
    } else {
      p.z[i] = v;
    }
    return;
  }
  const int j = (blk - nq - nz) / p.hv, col = (blk - nq - nz) - j * p.hv;
  const uint8_t* w = j ? p.wb : p.wa;
  // U loads per thread in flight at once (one batch for HIDDEN = 5120); indices past K are
  // clamped to K - 1 so the loads need no branch, and their products are not added
  constexpr int U = 20;
  float acc = 0.f;
  for (int k0 = threadIdx.x; k0 < p.K; k0 += 256 * U) {
    float xv[U], wv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = min(k0 + 256 * u, p.K - 1);
      xv[u] = npn::bf16_to_f32(p.x[k]);
      wv[u] = npn::bf16lo(fp8x2_to_bf16x2<false>(w[(size_t)k * p.hv + col]));
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (k0 + 256 * u < p.K) acc += xv[u] * wv[u];
  }
  acc = npn::wave_sum(acc);
  __shared__ float part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float sc = (j ? p.sb : p.sa)[col];
    (j ? p.b : p.a)[col] = (((part[0] + part[1]) + part[2]) + part[3]) * sc;
  }
}

// Workspace of npn_deltanet_full_fp8, 256-byte aligned regions: mixed_qkv [QKV] bf16, z
// [Hv * 128] bf16, a_out and b_out [Hv] f32, then the split-K partials of the qkv and z GEMMs
// ([S][N] f32 each, S from the GEMM plan for one row).
struct FullFp8Layout {
  size_t z, a, b, pq, pz, total;
  int sq, sz;
};

FullFp8Layout full_fp8_layout(int H, int qkv, int hv) {
  auto up = [](size_t n) { return (n + 255) & ~(size_t)255; };
  FullFp8Layout l;
  l.sq = plan(1, H, qkv).split_k;
  l.sz = plan(1, H, hv * 128).split_k;
  l.z = up((size_t)qkv * 2);
  l.a = l.z + up((size_t)hv * 128 * 2);
  l.b = l.a + up((size_t)hv * 4);
  l.pq = l.b + up((size_t)hv * 4);
  l.pz = l.pq + up((size_t)l.sq * qkv * 4);
  l.total = l.pz + up((size_t)l.sz * hv * 128 * 4);
  return l;
}

bool full_fp8_heads_ok(int k_heads, int v_heads) {
  return k_heads > 0 && v_heads > 0 && v_heads % k_heads == 0 && v_heads <= 4096;
}

}  // namespace

extern "C" size_t npn_fp8_matmul_workspace_size(int M, int K, int N) {
  if (!shape_ok(M, K, N)) return 0;
  return plan(M, K, N).ws;
}

extern "C" int npn_fp8_matmul(const uint16_t* x, const int8_t* w, const float* scale,
                              uint16_t* out, int M, int K, int N, void* workspace,
                              size_t workspace_bytes, void* stream) {
  NPN_REQUIRE(x && w && scale && out, NPN_ERR_NULL);
  NPN_REQUIRE(shape_ok(M, K, N), NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(x) && NPN_ALIGNED16(w) && NPN_ALIGNED16(out), NPN_ERR_ALIGN);
  const GemmPlan p = plan(M, K, N);
  if (p.split_k > 1) {
    NPN_REQUIRE(workspace != nullptr && workspace_bytes >= p.ws, NPN_ERR_WORKSPACE);
    NPN_REQUIRE(NPN_ALIGNED16(workspace), NPN_ERR_ALIGN);
  }
  return launch_gemm(p, x, w, scale, out, static_cast<float*>(workspace), M, K, N, 0, true,
                     static_cast<hipStream_t>(stream));
}

extern "C" int npn_fp8_matmul_split_k(int M, int K, int N) {
  if (!shape_ok(M, K, N)) return 0;
  return plan(M, K, N).split_k;
}

extern "C" int npn_fp8_matmul_plan(int M, int K, int N, int* info) {
  NPN_REQUIRE(info != nullptr, NPN_ERR_NULL);
  NPN_REQUIRE(shape_ok(M, K, N), NPN_ERR_SHAPE);
  const GemmPlan p = plan(M, K, N);
  if (p.wide && p.rows128) {
    info[0] = 3;
    info[1] = p.split_k;
    info[2] = 2 * p.h128;
    info[3] = ((p.groups * ((M + 127) / 128) * p.split_k + 7) / 8) * 8;
  } else if (p.wide) {
    info[0] = 2;
    info[1] = p.split_k;
    info[2] = p.ntm;
    info[3] = ((p.groups * p.split_k + 7) / 8) * 8 * p.passes;
  } else {
    info[0] = p.sk_wg > 0 ? 1 : 0;
    info[1] = p.split_k;
    info[2] = p.mt;
    info[3] = p.sk_wg > 0 ? p.sk_wg : ((N + NT - 1) / NT) * p.split_k * p.passes;
  }
  return NPN_OK;
}

extern "C" int npn_fp8_matmul_partials(const uint16_t* x, const int8_t* w, float* partial, int M,
                                       int K, int N, void* stream) {
  NPN_REQUIRE(x && w && partial, NPN_ERR_NULL);
  NPN_REQUIRE(shape_ok(M, K, N), NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(x) && NPN_ALIGNED16(w) && NPN_ALIGNED16(partial), NPN_ERR_ALIGN);
  const GemmPlan p = plan(M, K, N);
  // Neither kernel reads the scale or writes `out` when it writes partials.
  return launch_gemm(p, x, w, nullptr, nullptr, partial, M, K, N, 1, false,
                     static_cast<hipStream_t>(stream));
}

// SwiGLU of the GEMM output: out [M, N/2] = bf16(bf16(silu(g)) * u), [g | u] = bf16((x . w) *
// scale). Wide plans without split-K fuse it into the GEMM epilogue; other shapes write
// [g | u] to the workspace and run the glue kernel.
extern "C" int npn_silu_mul(const uint16_t* gate_up, uint16_t* out, int M, int I, void* stream);

// The fused form takes npn_fp8_matmul's own plan (so the sums are the same) when that plan is
// a wide one without split-K.
static bool swiglu_fused(const GemmPlan& p) { return p.wide && p.split_k == 1 && p.units % 2 == 0; }

extern "C" size_t npn_fp8_matmul_swiglu_workspace_size(int M, int K, int N) {
  if (!shape_ok(M, K, N) || N % 128 != 0) return 0;
  const GemmPlan p = plan(M, K, N);
  if (swiglu_fused(p)) return 0;
  return (((size_t)M * N * 2 + 255) & ~(size_t)255) + p.ws;
}

extern "C" int npn_fp8_matmul_swiglu(const uint16_t* x, const int8_t* w, const float* scale,
                                     uint16_t* out, int M, int K, int N, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  NPN_REQUIRE(x && w && scale && out, NPN_ERR_NULL);
  NPN_REQUIRE(shape_ok(M, K, N) && N % 128 == 0, NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(x) && NPN_ALIGNED16(w) && NPN_ALIGNED16(out), NPN_ERR_ALIGN);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const GemmPlan p = plan(M, K, N);
  if (swiglu_fused(p))
    return launch_gemm(p, x, w, scale, out, nullptr, M, K, N, 0, false, s, nullptr, true);
  const size_t need = npn_fp8_matmul_swiglu_workspace_size(M, K, N);
  NPN_REQUIRE(workspace != nullptr && workspace_bytes >= need, NPN_ERR_WORKSPACE);
  NPN_REQUIRE(NPN_ALIGNED16(workspace), NPN_ERR_ALIGN);
  uint16_t* gu = static_cast<uint16_t*>(workspace);
  const size_t gu_bytes = ((size_t)M * N * 2 + 255) & ~(size_t)255;
  float* part = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + gu_bytes);
  if (p.split_k > 1) {  // the reduction and the SwiGLU in one pass over the partials
    const int st = launch_gemm(p, x, w, scale, nullptr, part, M, K, N, 0, false, s);
    if (st != NPN_OK) return st;
    const size_t n = (size_t)M * (N / 2);
    hipLaunchKernelGGL(fp8_splitk_swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       s, part, scale, out, M, N, p.split_k);
    return npn_launch_status();
  }
  const int st = launch_gemm(p, x, w, scale, gu, part, M, K, N, 0, true, s);
  if (st != NPN_OK) return st;
  return npn_silu_mul(gu, out, M, N / 2, stream);
}

// Row argmax of out = bf16((x . w) * scale) without writing out: partials per (row, column
// group) for the acceptance kernels to reduce.
extern "C" int npn_fp8_matmul_argmax_groups(int M, int K, int N) {
  if (!shape_ok(M, K, N)) return 0;
  const GemmPlan p = plan(M, K, N, true);
  return p.wide ? p.groups : ((N + NT - 1) / NT) * narrow_slices(p.mt);
}

extern "C" int npn_fp8_matmul_argmax(const uint16_t* x, const int8_t* w, const float* scale,
                                     void* parts, int M, int K, int N, void* stream) {
  NPN_REQUIRE(x && w && scale && parts, NPN_ERR_NULL);
  NPN_REQUIRE(shape_ok(M, K, N), NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(x) && NPN_ALIGNED16(w) && NPN_ALIGNED16(parts), NPN_ERR_ALIGN);
  const GemmPlan p = plan(M, K, N, true);
  return launch_gemm(p, x, w, scale, nullptr, nullptr, M, K, N, 0, false,
                     static_cast<hipStream_t>(stream), static_cast<ArgPart*>(parts));
}

// out = bf16((x . w) * scale) and, per (row, column group) of the argmax plan
// (npn_fp8_matmul_argmax_groups groups), the max of the row's bf16 outputs in the group with
// NaN ignored (-inf if none): the row maxima the rejection-sampling passes would otherwise
// read the logits for. The plan never splits K, so out equals npn_fp8_matmul's whenever
// that plan does not split either (true for vocabulary-wide N).
extern "C" int npn_fp8_matmul_rowmax(const uint16_t* x, const int8_t* w, const float* scale,
                                     uint16_t* out, float* gmax, int M, int K, int N,
                                     void* stream) {
  NPN_REQUIRE(x && w && scale && out && gmax, NPN_ERR_NULL);
  NPN_REQUIRE(shape_ok(M, K, N), NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(x) && NPN_ALIGNED16(w) && NPN_ALIGNED16(out), NPN_ERR_ALIGN);
  const GemmPlan p = plan(M, K, N, true);
  return launch_gemm(p, x, w, scale, out, nullptr, M, K, N, 0, false,
                     static_cast<hipStream_t>(stream), nullptr, false, gmax);
}

namespace npn {

bool fp8_matmul_chunk_stats_ok(int M, int K, int N) {
  if (!shape_ok(M, K, N) || N % 64 != 0) return false;
  const GemmPlan p = plan(M, K, N, true, 4);
  return p.split_k == 1 && (!p.wide || p.ualign == 4);
}

bool fp8_matmul_stats_pass_cheaper(int M, int K, int N) {
  if (!shape_ok(M, K, N)) return false;
  const GemmPlan q = plan(M, K, N);
  if (!q.wide || q.split_k != 1) return false;
  if (!fp8_matmul_chunk_stats_ok(M, K, N)) return true;
  const GemmPlan e = plan(M, K, N, true, 4);
  if (!e.wide) return false;
  const int q_rounds = q.rows128 ? 1 : (q.groups + WIDE_WG - 1) / WIDE_WG;
  return q_rounds < (e.groups + WIDE_WG - 1) / WIDE_WG;
}

int fp8_matmul_unsplit(const uint16_t* x, const int8_t* w, const float* scale, uint16_t* out,
                       int M, int K, int N, hipStream_t stream) {
  NPN_REQUIRE(x && w && scale && out, NPN_ERR_NULL);
  NPN_REQUIRE(shape_ok(M, K, N), NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(x) && NPN_ALIGNED16(w) && NPN_ALIGNED16(out), NPN_ERR_ALIGN);
  const GemmPlan p = plan(M, K, N);
  NPN_REQUIRE(p.split_k == 1, NPN_ERR_SHAPE);
  return launch_gemm(p, x, w, scale, out, nullptr, M, K, N, 0, false, stream);
}

int fp8_matmul_chunk_stats(const uint16_t* x, const int8_t* w, const float* scale, uint16_t* out,
                           float* cmax, uint64_t* csum, float inv_temp, int M, int K, int N,
                           hipStream_t stream) {
  NPN_REQUIRE(x && w && scale && out && cmax && csum, NPN_ERR_NULL);
  NPN_REQUIRE(fp8_matmul_chunk_stats_ok(M, K, N), NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(x) && NPN_ALIGNED16(w) && NPN_ALIGNED16(out), NPN_ERR_ALIGN);
  const GemmPlan p = plan(M, K, N, true, 4);
  return launch_gemm(p, x, w, scale, out, nullptr, M, K, N, 0, false, stream, nullptr, false,
                     nullptr, cmax, csum, inv_temp);
}

}  // namespace npn

// deltanet::full_fp8: the four in-projections of one decode token, then the token step of
// deltanet::full on their outputs. Three launches: the qkv and z GEMMs writing split-K partials
// (the plans of npn_fp8_matmul for one row, both in one narrow launch where the two plans share
// their split-K factor, else one launch each), the finishing kernel above (mixed_qkv and z as
// npn_fp8_matmul's bf16 outputs, the new conv window, a_out and b_out in float32, not rounded),
// and the DeltaNet token step (npn_deltanet_verify with T = 1).
extern "C" size_t npn_deltanet_full_fp8_workspace_size(int hidden, int k_heads, int v_heads) {
  if (!full_fp8_heads_ok(k_heads, v_heads)) return 0;
  const int qkv = (2 * k_heads + v_heads) * 128;
  if (!shape_ok(1, hidden, qkv)) return 0;
  return full_fp8_layout(hidden, qkv, v_heads).total;
}

extern "C" int npn_deltanet_full_fp8(
    const uint16_t* x, const float* state, const uint16_t* conv_state, const float* conv_weight,
    const float* conv_bias, const float* A_log, const float* dt_bias, const float* norm_weight,
    const int8_t* qkv_w, const float* qkv_s, const int8_t* z_w, const float* z_s,
    const int8_t* a_w, const float* a_s, const int8_t* b_w, const float* b_s, float* new_state,
    uint16_t* new_conv_state, uint16_t* out, int hidden, int k_heads, int v_heads,
    void* workspace, size_t workspace_bytes, void* stream) {
  NPN_REQUIRE(x && state && conv_state && conv_weight && conv_bias && A_log && dt_bias &&
                  norm_weight && qkv_w && qkv_s && z_w && z_s && a_w && a_s && b_w && b_s &&
                  new_state && new_conv_state && out,
              NPN_ERR_NULL);
  NPN_REQUIRE(full_fp8_heads_ok(k_heads, v_heads), NPN_ERR_SHAPE);
  const int qkv = (2 * k_heads + v_heads) * 128, zn = v_heads * 128;
  NPN_REQUIRE(shape_ok(1, hidden, qkv), NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(x) && NPN_ALIGNED16(qkv_w) && NPN_ALIGNED16(z_w), NPN_ERR_ALIGN);
  // the new conv window is written before the token step reads the old one, so the two
  // [QKV, 3] bf16 spans must not share a byte
  {
    const uintptr_t n0 = reinterpret_cast<uintptr_t>(new_conv_state);
    const uintptr_t c0 = reinterpret_cast<uintptr_t>(conv_state);
    const uintptr_t span = (uintptr_t)qkv * 3 * sizeof(uint16_t);
    NPN_REQUIRE(n0 + span <= c0 || c0 + span <= n0, NPN_ERR_VALUE);
  }
  const FullFp8Layout l = full_fp8_layout(hidden, qkv, v_heads);
  NPN_REQUIRE(workspace != nullptr && workspace_bytes >= l.total, NPN_ERR_WORKSPACE);
  NPN_REQUIRE(NPN_ALIGNED16(workspace), NPN_ERR_ALIGN);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* pq = reinterpret_cast<float*>(ws + l.pq);
  float* pz = reinterpret_cast<float*>(ws + l.pz);
  // both GEMMs in one launch where their plans allow (the same partials as two launches)
  int st = NPN_OK;
  if (launch_gemm_pair_partials(x, qkv_w, pq, qkv, z_w, pz, zn, 1, hidden, s)) {
    st = npn_launch_status();
  } else {
    st = launch_gemm(plan(1, hidden, qkv), x, qkv_w, nullptr, nullptr, pq, 1, hidden, qkv, 1,
                     false, s);
    if (st == NPN_OK)
      st = launch_gemm(plan(1, hidden, zn), x, z_w, nullptr, nullptr, pz, 1, hidden, zn, 1,
                       false, s);
  }
  if (st != NPN_OK) return st;
  InprojFinishArgs fa{pq, qkv_s, reinterpret_cast<uint16_t*>(ws), conv_state, new_conv_state,
                      pz, z_s, reinterpret_cast<uint16_t*>(ws + l.z), x,
                      reinterpret_cast<const uint8_t*>(a_w), a_s, reinterpret_cast<float*>(ws + l.a),
                      reinterpret_cast<const uint8_t*>(b_w), b_s, reinterpret_cast<float*>(ws + l.b),
                      l.sq, qkv, l.sz, zn, hidden, v_heads};
  const int blocks = (qkv + 255) / 256 + (zn + 255) / 256 + 2 * v_heads;
  hipLaunchKernelGGL(dn_fp8_inproj_finish_kernel, dim3(blocks), dim3(256), 0, s, fa);
  st = npn_launch_status();
  if (st != NPN_OK) return st;
  return npn_deltanet_verify(state, nullptr, 0, fa.mixed, conv_state, conv_weight, conv_bias,
                             fa.a, fa.b, fa.z, A_log, dt_bias, norm_weight, new_state, out, 1, 1,
                             k_heads, v_heads, stream);
}
