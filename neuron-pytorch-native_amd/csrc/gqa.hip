// GQA attention-tail kernels for gfx950: decode tail (reference gqa::tail), T-token
// verify tail over a bf16 KV cache, and the KV append that precedes it.
//
// Math per query row, from contrib/qwen3.6-27b/kernels/gqa_tail_ref.py:31-70 (kernel
// doc contrib/qwen3.6-27b/kernels/gqa_tail.py:1-23):
//   q' = (1 + w) * q * rsqrt(mean(q^2) + 1e-6); partial RoPE on q'[:64] (rotate_half
//   inside the 64); s_j = q'.k_j / 16 (+ mask); p = softmax(s); out = (p V) * sigmoid(gate).
//
// Verify tail (T tokens x grp q-heads per kv head = R query rows per (b, kv head)):
//  1. qprep: q' per row, scaled by log2(e)/16 and split into bf16 hi + lo parts
//     (hi = bf16(q'), lo = bf16(q' - hi)), so the bf16 MFMA sees q' to ~16 mantissa bits.
//  2. attn: split-KV. One workgroup per (chunk of 512 keys, b, kv head), one wave per
//     16-row tile of the R rows; the chunk streams through LDS in 32-key K/V tiles:
//       S^T[32 keys x 16] = K Q'^T  (K rows from LDS as MFMA A operands, q' hi/lo held in
//                                   VGPRs as B operands)              v_mfma_f32_16x16x32_bf16
//       online softmax per row in fp32 (exp2), causal limit kv_len + t per row
//       O^T[256 x 16] += V^T P^T    (V tile read back transposed with ds_read_b64_tr_b16;
//                                   P hi/lo in bf16, taken directly from the S^T
//                                   accumulator registers)
//     Each wave writes its rows' (m, l, O) partial for the chunk.
//  3. merge: log-sum-exp merge of the chunk partials, * sigmoid(gate) -> bf16.
//
// HBM layout: cache [B][Hkv][s_max][256] bf16, each (b, kv head) a contiguous block of
// rows; query/gate/out [B][T][Hq][256]; query row r of (b, g) is token r / grp,
// q-head g*grp + r % grp.
#include "npn_common.h"

namespace {

constexpr int DH = 256;
constexpr int ROPE = 64;
constexpr float kEps = 1e-6f;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1.0e30f;   // finite "no key yet" running max (avoids inf - inf)

constexpr int CH = 512;               // keys per workgroup (split-KV chunk)
constexpr int KS = 32;                // keys per step

typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ bf16x8 pack8(s16x4 a, s16x4 b) {
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  s16x8 v = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ s16x4 lds_tr16(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(p));
}

// ---------------------------------------------------------------------------------------
// 1. q' = rope((1+w) * rmsnorm(q)) * log2(e)/16, split into bf16 hi/lo.
//    One wave per padded query row (b, g, r); lane l owns dims 4l..4l+3.
struct QPrepArgs {
  const uint16_t* query;
  const float* q_norm;
  const float* cos;
  const float* sin;
  uint16_t* qhi;   // [B][Hkv][R][DH]
  uint16_t* qlo;
  int B, T, Hq, Hkv, R;
};

__global__ __launch_bounds__(256) void gqa_qprep_kernel(QPrepArgs a) {
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int grp = a.Hq / a.Hkv;
  if (wave >= a.B * a.Hkv * a.R) return;
  const int r = wave % a.R;
  const int bg = wave / a.R;
  const int b = bg / a.Hkv, g = bg - b * a.Hkv;
  uint16_t* dhi = a.qhi + (size_t)wave * DH + 4 * lane;
  uint16_t* dlo = a.qlo + (size_t)wave * DH + 4 * lane;
  if (r >= a.T * grp) {  // padding rows of the MFMA tile
    for (int j = 0; j < 4; ++j) { dhi[j] = 0; dlo[j] = 0; }
    return;
  }
  const int t = r / grp, qh = g * grp + (r - (r / grp) * grp);
  const uint16_t* src = a.query + (((size_t)b * a.T + t) * a.Hq + qh) * DH + 4 * lane;
  float x[4];
  float ss = 0.f;
  for (int j = 0; j < 4; ++j) {
    x[j] = npn::bf16_to_f32(src[j]);
    ss += x[j] * x[j];
  }
  ss = npn::wave_sum(ss);
  const float rn = rsqrtf(ss * (1.0f / DH) + kEps);
  for (int j = 0; j < 4; ++j) x[j] = (1.0f + a.q_norm[4 * lane + j]) * (x[j] * rn);
  // partial RoPE: dims 0..63 live in lanes 0..15; partner of dim d is d ^ 32 (lane ^ 8)
  float y[4];
  for (int j = 0; j < 4; ++j) y[j] = __shfl_xor(x[j], 8, 64);
  if (lane < ROPE / 4) {
    const float* cs = a.cos + ((size_t)b * a.T + t) * ROPE + 4 * lane;
    const float* sn = a.sin + ((size_t)b * a.T + t) * ROPE + 4 * lane;
    const float sign = lane < ROPE / 8 ? -1.0f : 1.0f;  // rotate_half = cat(-x[32:], x[:32])
    for (int j = 0; j < 4; ++j) x[j] = x[j] * cs[j] + sign * y[j] * sn[j];
  }
  const float scale = kLog2e / 16.0f;  // softmax scale 1/sqrt(256), in base 2
  for (int j = 0; j < 4; ++j) {
    const float v = x[j] * scale;
    const uint16_t hi = npn::f32_to_bf16(v);
    dhi[j] = hi;
    dlo[j] = npn::f32_to_bf16(v - npn::bf16_to_f32(hi));
  }
}

// ---------------------------------------------------------------------------------------
// 2. split-KV attention over one 512-key chunk of one (b, kv head).
//    Workgroup = NRT waves; wave w owns query rows 16w..16w+15 (its q' hi/lo lives in
//    VGPRs as MFMA B operands) and all waves share each 32-key K/V tile, which is DMA'd
//    from HBM straight into LDS (global_load_lds_dwordx4), double-buffered.
//    Tile rows keep their 16-byte chunks XOR-swizzled (K: kswz, V: vswz) so the MFMA
//    operand reads of 16 rows at one column spread over the LDS banks.
struct AttnArgs {
  const uint16_t* qhi;
  const uint16_t* qlo;
  const uint16_t* cache_k;
  const uint16_t* cache_v;
  const int32_t* kv_len;
  float* part_o;   // [B*Hkv][nch][R][DH]
  float* part_ml;  // [B*Hkv][nch][R][2]
  int Hkv, s_max, T, grp, nch;
};

__device__ __forceinline__ int kswz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }
__device__ __forceinline__ int vswz(int r) { return (r & 7) << 1; }

template <int NRT>
__global__ __launch_bounds__(NRT * 64, 2) void gqa_attn_kernel(AttnArgs a) {
  constexpr int R = NRT * 16;
  constexpr int TILE = KS * DH * 2;  // bytes of one 32-key K or V tile
  const int c = blockIdx.x;
  const int bg = blockIdx.y;
  const int b = bg / a.Hkv;
  const int L = a.kv_len[b] > 0 ? a.kv_len[b] : 0;
  const int kend = L + a.T < a.s_max ? L + a.T : a.s_max;  // rows [0, kend) are read
  const int c0 = c * CH;
  if (c0 >= kend) return;

  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i = lane & 15, G = lane >> 4;
  const int row = w * 16 + i;  // this lane's query row (B-operand column / C column)

  __shared__ __attribute__((aligned(16))) uint8_t smem[2][2][TILE];  // [buffer][K|V]

  const uint16_t* kb = a.cache_k + (size_t)bg * a.s_max * DH;
  const uint16_t* vb = a.cache_v + (size_t)bg * a.s_max * DH;
  const int steps = min(CH / KS, (kend - c0 + KS - 1) / KS);

  // DMA of step s's K and V tiles into buffer s&1: 32 instructions of 1 KiB (2 rows each),
  // spread over the NRT waves.
  auto dma = [&](int s) {
    const int k0 = c0 + s * KS;
    for (int j = w; j < 2 * (KS / 2); j += NRT) {
      const int isv = j >= KS / 2;
      const int it = isv ? j - KS / 2 : j;
      const int r = 2 * it + (lane >> 5);
      const int q = lane & 31;
      int key = k0 + r;
      key = key < kend ? key : kend - 1;
      const int sq = q ^ (isv ? vswz(r) : kswz(r));
      const uint16_t* src = (isv ? vb : kb) + (size_t)key * DH + sq * 8;
      npn::lds_dma16(src, &smem[s & 1][isv][it * 2 * DH * 2]);
    }
  };
  dma(0);

  // q' hi/lo of this lane's row as B operands: dims 32*ks + 8*G .. +7.
  u32x4 qh[8], ql[8];
  {
    const size_t qo = ((size_t)bg * R + row) * DH + 8 * G;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      qh[ks] = *reinterpret_cast<const u32x4*>(a.qhi + qo + 32 * ks);
      ql[ks] = *reinterpret_cast<const u32x4*>(a.qlo + qo + 32 * ks);
    }
  }
  const int lim = row < a.T * a.grp ? L + row / a.grp : kend - 1;  // last key this row sees

  float m_run = kNegBig, l_run = 0.f;
  f32x4 acc[16];
#pragma unroll
  for (int dt = 0; dt < 16; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Transposed V reads: this lane supplies rows 4G + (i>>2) (+16), dims 16*dt + 4*(i&3).
  const int tr_row = 4 * G + (i >> 2);
  const int tr_half = (i & 1) * 8;
  const int tr_cq = (i & 3) >> 1;

  for (int s = 0; s < steps; ++s) {
    const int k0 = c0 + s * KS;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's DMA of step s landed
    __builtin_amdgcn_s_barrier();                     // ... and every other wave's
    asm volatile("" ::: "memory");
    if (s + 1 < steps) dma(s + 1);                    // buffer (s+1)&1 is free again
    const uint8_t* kt_lds = smem[s & 1][0];
    const uint8_t* vt_lds = smem[s & 1][1];

    // S^T[32 keys x 16 rows] = K Q'^T
    f32x4 st[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      st[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int r = 16 * kt + i;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const int pos = (4 * ks + G) ^ kswz(r);
        const bf16x8 ka = as_bf16x8(*reinterpret_cast<const u32x4*>(kt_lds + r * DH * 2 + pos * 16));
        st[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, as_bf16x8(qh[ks]), st[kt], 0, 0, 0);
        st[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, as_bf16x8(ql[ks]), st[kt], 0, 0, 0);
      }
    }

    // causal mask + online softmax (base 2); P hi/lo become the B operands of P.V.
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = k0 + 16 * kt + 4 * G + r;
        if (key > lim) st[kt][r] = -INFINITY;
        mx = fmaxf(mx, st[kt][r]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mnew = fmaxf(m_run, mx);
    const float corr = exp2f(m_run - mnew);
    m_run = mnew;
    bf16x8 ph, pl;
    float psum = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = exp2f(st[kt][r] - mnew);
        psum += p;
        const __bf16 h = (__bf16)p;
        ph[kt * 4 + r] = h;
        pl[kt * 4 + r] = (__bf16)(p - (float)h);
      }
    l_run = l_run * corr + psum;

    // O^T[256 x 16 rows] += V^T P^T
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) {
      const int q = 2 * dt + tr_cq;
      const uint8_t* p1 = vt_lds + tr_row * DH * 2 + ((q ^ vswz(tr_row)) * 16) + tr_half;
      const uint8_t* p2 = vt_lds + (tr_row + 16) * DH * 2 + ((q ^ vswz(tr_row + 16)) * 16) + tr_half;
      const bf16x8 va = pack8(lds_tr16(p1), lds_tr16(p2));
      acc[dt] *= corr;
      acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, ph, acc[dt], 0, 0, 0);
      acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pl, acc[dt], 0, 0, 0);
    }
  }

  // Row sum over the 4 lane groups, then this wave's 16 rows of the chunk partial.
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  float* po = a.part_o + (((size_t)bg * a.nch + c) * R + row) * DH;
#pragma unroll
  for (int dt = 0; dt < 16; ++dt) *reinterpret_cast<f32x4*>(po + 16 * dt + 4 * G) = acc[dt];
  if (G == 0) {
    float* pml = a.part_ml + (((size_t)bg * a.nch + c) * R + row) * 2;
    pml[0] = m_run;
    pml[1] = l_run;
  }
}

// ---------------------------------------------------------------------------------------
// 3. merge chunk partials, apply sigmoid(gate), write bf16. One 64-thread block per
//    (query row, b, kv head); lane l owns output dims 4l..4l+3 (float4 partial reads).
struct MergeArgs {
  const float* part_o;
  const float* part_ml;
  const int32_t* kv_len;
  const uint16_t* gate;
  uint16_t* out;
  int T, Hq, Hkv, R, nch, s_max;
};

__global__ __launch_bounds__(64) void gqa_merge_kernel(MergeArgs a) {
  const int r = blockIdx.x;
  const int bg = blockIdx.y;
  const int b = bg / a.Hkv, g = bg - b * a.Hkv;
  const int grp = a.Hq / a.Hkv;
  const int lane = threadIdx.x;
  const int L = a.kv_len[b] > 0 ? a.kv_len[b] : 0;
  const int kend = L + a.T < a.s_max ? L + a.T : a.s_max;
  const int nc = (kend + CH - 1) / CH;
  const float* pml = a.part_ml + ((size_t)bg * a.nch * a.R + r) * 2;
  const float* po = a.part_o + ((size_t)bg * a.nch * a.R + r) * DH + 4 * lane;
  const size_t cstride_ml = (size_t)a.R * 2, cstride_o = (size_t)a.R * DH;
  float M = kNegBig;
  for (int c = 0; c < nc; ++c) M = fmaxf(M, pml[c * cstride_ml]);
  float l = 0.f;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
  for (int c = 0; c < nc; ++c) {
    const float f = exp2f(pml[c * cstride_ml] - M);
    l += f * pml[c * cstride_ml + 1];
    o += f * *reinterpret_cast<const f32x4*>(po + c * cstride_o);
  }
  const int t = r / grp, qh = g * grp + (r - t * grp);
  const size_t oi = (((size_t)b * a.T + t) * a.Hq + qh) * DH + 4 * lane;
  const float inv = 1.0f / l;
  uint32_t w[2];
  for (int j = 0; j < 2; ++j) {
    const float g0 = npn::sigmoid(npn::bf16_to_f32(a.gate[oi + 2 * j]));
    const float g1 = npn::sigmoid(npn::bf16_to_f32(a.gate[oi + 2 * j + 1]));
    w[j] = npn::f32_to_bf16(o[2 * j] * inv * g0) |
           ((uint32_t)npn::f32_to_bf16(o[2 * j + 1] * inv * g1) << 16);
  }
  *reinterpret_cast<uint2*>(a.out + oi) = make_uint2(w[0], w[1]);
}

// ---------------------------------------------------------------------------------------
// KV append: cache row kv_len[b]+t of head g <- bf16(rope(bf16(rmsnorm_1p(key)))), value copy.
// One wave per (b, t, g); lane l owns dims 4l..4l+3.
struct AppendArgs {
  const uint16_t* key;
  const uint16_t* value;
  const float* k_norm;
  const float* cos;
  const float* sin;
  uint16_t* cache_k;
  uint16_t* cache_v;
  const int32_t* kv_len;
  int B, T, Hkv, s_max;
};

__global__ __launch_bounds__(256) void gqa_kv_append_kernel(AppendArgs a) {
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (wave >= a.B * a.T * a.Hkv) return;
  const int g = wave % a.Hkv;
  const int bt = wave / a.Hkv;
  const int b = bt / a.T, t = bt - b * a.T;
  const int pos = a.kv_len[b] + t;
  if (pos < 0 || pos >= a.s_max) return;
  const uint16_t* src = a.key + (size_t)wave * DH + 4 * lane;
  float x[4];
  float ss = 0.f;
  for (int j = 0; j < 4; ++j) {
    x[j] = npn::bf16_to_f32(src[j]);
    ss += x[j] * x[j];
  }
  ss = npn::wave_sum(ss);
  const float rn = rsqrtf(ss * (1.0f / DH) + kEps);
  for (int j = 0; j < 4; ++j)
    x[j] = npn::bf16_to_f32(npn::f32_to_bf16((1.0f + a.k_norm[4 * lane + j]) * (x[j] * rn)));
  float y[4];
  for (int j = 0; j < 4; ++j) y[j] = __shfl_xor(x[j], 8, 64);
  if (lane < ROPE / 4) {
    const float* cs = a.cos + ((size_t)b * a.T + t) * ROPE + 4 * lane;
    const float* sn = a.sin + ((size_t)b * a.T + t) * ROPE + 4 * lane;
    const float sign = lane < ROPE / 8 ? -1.0f : 1.0f;
    for (int j = 0; j < 4; ++j) x[j] = x[j] * cs[j] + sign * y[j] * sn[j];
  }
  const size_t row = (((size_t)b * a.Hkv + g) * a.s_max + pos) * DH + 4 * lane;
  for (int j = 0; j < 4; ++j) a.cache_k[row + j] = npn::f32_to_bf16(x[j]);
  const uint16_t* vs = a.value + (size_t)wave * DH + 4 * lane;
  for (int j = 0; j < 4; ++j) a.cache_v[row + j] = vs[j];
}

// ---------------------------------------------------------------------------------------
// Decode tail of the reference op (fp32 cache, one kv head, mask shared over the batch).
// One 256-thread block per sequence b handles its Hq rows; keys in blocks of 64, online
// softmax in fp32. Wave w scores keys w, w+4, ...: lane l holds dims 4l..4l+3.
constexpr int TAIL_MAXQ = 16;
constexpr int TAIL_KB = 64;

__global__ __launch_bounds__(256) void gqa_tail_kernel(const float* __restrict__ query,
                                                       const float* __restrict__ gate,
                                                       const float* __restrict__ q_norm,
                                                       const float* __restrict__ cos,
                                                       const float* __restrict__ sin,
                                                       const float* __restrict__ ck,
                                                       const float* __restrict__ cv,
                                                       const float* __restrict__ mask,
                                                       float* __restrict__ out, int Hq, int S) {
  const int b = blockIdx.x;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  __shared__ __attribute__((aligned(16))) float s_q[TAIL_MAXQ][DH];
  __shared__ float s_p[TAIL_MAXQ][TAIL_KB];
  __shared__ float s_m[TAIL_MAXQ], s_l[TAIL_MAXQ], s_corr[TAIL_MAXQ];

  // q' rows: wave w prepares rows w, w+4, ...
  for (int h = w; h < Hq; h += 4) {
    const float* src = query + ((size_t)b * Hq + h) * DH + 4 * lane;
    float x[4], ss = 0.f;
    for (int j = 0; j < 4; ++j) { x[j] = src[j]; ss += x[j] * x[j]; }
    ss = npn::wave_sum(ss);
    const float rn = rsqrtf(ss * (1.0f / DH) + kEps);
    for (int j = 0; j < 4; ++j) x[j] = (1.0f + q_norm[4 * lane + j]) * (x[j] * rn);
    float y[4];
    for (int j = 0; j < 4; ++j) y[j] = __shfl_xor(x[j], 8, 64);
    if (lane < ROPE / 4) {
      const float sign = lane < ROPE / 8 ? -1.0f : 1.0f;
      for (int j = 0; j < 4; ++j) x[j] = x[j] * cos[4 * lane + j] + sign * y[j] * sin[4 * lane + j];
    }
    for (int j = 0; j < 4; ++j) s_q[h][4 * lane + j] = x[j];
  }
  if (tid < Hq) { s_m[tid] = -INFINITY; s_l[tid] = 0.f; }
  float o[TAIL_MAXQ];
#pragma unroll
  for (int h = 0; h < TAIL_MAXQ; ++h) o[h] = 0.f;
  __syncthreads();

  const float* kb = ck + (size_t)b * S * DH;
  const float* vb = cv + (size_t)b * S * DH;
  for (int j0 = 0; j0 < S; j0 += TAIL_KB) {
    const int nk = S - j0 < TAIL_KB ? S - j0 : TAIL_KB;
    for (int jj = w; jj < nk; jj += 4) {
      const float4 kv = reinterpret_cast<const float4*>(kb + (size_t)(j0 + jj) * DH)[lane];
      const float bias = (1.0f - mask[j0 + jj]) * -1e9f;
      for (int h = 0; h < Hq; ++h) {
        const float4 q = reinterpret_cast<const float4*>(s_q[h])[lane];
        const float s = npn::wave_sum(q.x * kv.x + q.y * kv.y + q.z * kv.z + q.w * kv.w);
        if (lane == 0) s_p[h][jj] = s * (1.0f / 16.0f) + bias;
      }
    }
    __syncthreads();
    if (tid < Hq) {
      float mx = s_m[tid];
      for (int jj = 0; jj < nk; ++jj) mx = fmaxf(mx, s_p[tid][jj]);
      const float corr = __expf(s_m[tid] - mx);
      float l = s_l[tid] * (s_m[tid] == -INFINITY ? 0.f : corr);
      for (int jj = 0; jj < nk; ++jj) {
        const float p = __expf(s_p[tid][jj] - mx);
        s_p[tid][jj] = p;
        l += p;
      }
      s_corr[tid] = s_m[tid] == -INFINITY ? 0.f : corr;
      s_m[tid] = mx;
      s_l[tid] = l;
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < TAIL_MAXQ; ++h)
      if (h < Hq) o[h] *= s_corr[h];
    for (int jj = 0; jj < nk; ++jj) {
      const float v = vb[(size_t)(j0 + jj) * DH + tid];
#pragma unroll
      for (int h = 0; h < TAIL_MAXQ; ++h)
        if (h < Hq) o[h] += s_p[h][jj] * v;
    }
    __syncthreads();
  }
#pragma unroll
  for (int h = 0; h < TAIL_MAXQ; ++h) {
    if (h < Hq) {
      const size_t oi = ((size_t)b * Hq + h) * DH + tid;
      out[oi] = o[h] / s_l[h] * npn::sigmoid(gate[oi]);
    }
  }
}

struct VerifyPlan {
  int grp, R, nrt, nch;
  size_t q_bytes, po_bytes, pml_bytes, total;
};

VerifyPlan plan(int B, int T, int Hq, int Hkv, int s_max) {
  VerifyPlan p{};
  p.grp = Hq / Hkv;
  p.nrt = (T * p.grp + 15) / 16;
  p.R = p.nrt * 16;
  p.nch = (s_max + CH - 1) / CH;
  auto up = [](size_t x) { return (x + 255) & ~size_t(255); };
  p.q_bytes = up((size_t)B * Hkv * p.R * DH * 2);
  p.po_bytes = up((size_t)B * Hkv * p.nch * p.R * DH * 4);
  p.pml_bytes = up((size_t)B * Hkv * p.nch * p.R * 2 * 4);
  p.total = 2 * p.q_bytes + p.po_bytes + p.pml_bytes;
  return p;
}

bool verify_shape_ok(int B, int T, int Hq, int Hkv, int s_max) {
  return B >= 1 && B <= 65536 && T >= 1 && Hkv >= 1 && Hq >= Hkv && Hq % Hkv == 0 &&
         T * (Hq / Hkv) <= 48 && s_max >= T && s_max <= (1 << 24);
}

}  // namespace

extern "C" size_t npn_gqa_tail_verify_workspace_size(int B, int T, int q_heads, int kv_heads,
                                                     int s_max) {
  if (!verify_shape_ok(B, T, q_heads, kv_heads, s_max)) return 0;
  return plan(B, T, q_heads, kv_heads, s_max).total;
}

extern "C" int npn_gqa_tail_verify(const uint16_t* query, const uint16_t* gate,
                                   const float* q_norm, const float* cos, const float* sin,
                                   const uint16_t* cache_k, const uint16_t* cache_v,
                                   const int32_t* kv_len, uint16_t* out, int B, int T,
                                   int q_heads, int kv_heads, int s_max, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  NPN_REQUIRE(query && gate && q_norm && cos && sin && cache_k && cache_v && kv_len && out,
              NPN_ERR_NULL);
  NPN_REQUIRE(verify_shape_ok(B, T, q_heads, kv_heads, s_max), NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(cache_k) && NPN_ALIGNED16(cache_v) && NPN_ALIGNED16(workspace),
              NPN_ERR_ALIGN);
  const VerifyPlan p = plan(B, T, q_heads, kv_heads, s_max);
  NPN_REQUIRE(workspace != nullptr && workspace_bytes >= p.total, NPN_ERR_WORKSPACE);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint16_t* qhi = reinterpret_cast<uint16_t*>(ws);
  uint16_t* qlo = reinterpret_cast<uint16_t*>(ws + p.q_bytes);
  float* po = reinterpret_cast<float*>(ws + 2 * p.q_bytes);
  float* pml = reinterpret_cast<float*>(ws + 2 * p.q_bytes + p.po_bytes);

  QPrepArgs qa{query, q_norm, cos, sin, qhi, qlo, B, T, q_heads, kv_heads, p.R};
  const int rows = B * kv_heads * p.R;
  hipLaunchKernelGGL(gqa_qprep_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, qa);

  AttnArgs aa{qhi, qlo, cache_k, cache_v, kv_len, po, pml, kv_heads, s_max, T, p.grp, p.nch};
  const dim3 grid(p.nch, B * kv_heads);
  if (p.nrt == 1) hipLaunchKernelGGL(gqa_attn_kernel<1>, grid, dim3(64), 0, s, aa);
  else if (p.nrt == 2) hipLaunchKernelGGL(gqa_attn_kernel<2>, grid, dim3(128), 0, s, aa);
  else hipLaunchKernelGGL(gqa_attn_kernel<3>, grid, dim3(192), 0, s, aa);

  MergeArgs ma{po, pml, kv_len, gate, out, T, q_heads, kv_heads, p.R, p.nch, s_max};
  hipLaunchKernelGGL(gqa_merge_kernel, dim3(T * p.grp, B * kv_heads), dim3(64), 0, s, ma);
  return npn_launch_status();
}

extern "C" int npn_gqa_kv_append(const uint16_t* key, const uint16_t* value, const float* k_norm,
                                 const float* cos, const float* sin, uint16_t* cache_k,
                                 uint16_t* cache_v, const int32_t* kv_len, int B, int T,
                                 int kv_heads, int s_max, void* stream) {
  NPN_REQUIRE(key && value && k_norm && cos && sin && cache_k && cache_v && kv_len, NPN_ERR_NULL);
  NPN_REQUIRE(B >= 1 && T >= 1 && kv_heads >= 1 && s_max >= T, NPN_ERR_SHAPE);
  AppendArgs aa{key, value, k_norm, cos, sin, cache_k, cache_v, kv_len, B, T, kv_heads, s_max};
  const int waves = B * T * kv_heads;
  hipLaunchKernelGGL(gqa_kv_append_kernel, dim3((waves + 3) / 4), dim3(256), 0,
                     static_cast<hipStream_t>(stream), aa);
  return npn_launch_status();
}

extern "C" int npn_gqa_tail(const float* query, const float* gate, const float* q_norm,
                            const float* cos, const float* sin, const float* cached_k,
                            const float* cached_v, const float* mask, float* out, int B,
                            int q_heads, int S, void* stream) {
  NPN_REQUIRE(query && gate && q_norm && cos && sin && cached_k && cached_v && mask && out,
              NPN_ERR_NULL);
  NPN_REQUIRE(B >= 1 && q_heads >= 1 && q_heads <= TAIL_MAXQ && S >= 1, NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(cached_k) && NPN_ALIGNED16(cached_v), NPN_ERR_ALIGN);
  hipLaunchKernelGGL(gqa_tail_kernel, dim3(B), dim3(DH), 0, static_cast<hipStream_t>(stream),
                     query, gate, q_norm, cos, sin, cached_k, cached_v, mask, out, q_heads, S);
  return npn_launch_status();
}
