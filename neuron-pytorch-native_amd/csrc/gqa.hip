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
//     Block 0 of the same launch writes the split-KV plan; with the fused append
//     (npn_gqa_tail_verify_append) further blocks append the T new K/V rows to the cache,
//     and the RoPE rows come straight from the position table.
//  2. attn: split-KV over a balanced partition. The (b, kv head) pairs' 32-key steps
//     are laid end to end (prefix sums from a one-block plan kernel) and cut into
//     W = min(kAttnWG, S / 16) equal ranges (S steps in all), one per workgroup of the
//     kAttnWG launched (the rest exit at once), so every workgroup streams the same
//     number of K/V bytes whatever the kv_len spread; a range may cover the end of one
//     pair and the start of the next. One wave per 16-row tile of the R rows; each
//     pair segment streams through LDS in 32-key K/V tiles:
//       S^T[32 keys x 16] = K Q'^T  (K rows from LDS as MFMA A operands, q' hi/lo held in
//                                   VGPRs as B operands)              v_mfma_f32_16x16x32_bf16
//       online softmax per row in fp32 (exp2), causal limit kv_len + t per row
//       O^T[256 x 16] += V^T P^T    (V tile read back transposed with ds_read_b64_tr_b16;
//                                   P hi/lo in bf16, taken directly from the S^T
//                                   accumulator registers)
//     Each wave writes its rows' (m, l, O) partial per pair segment, into slot w + p
//     (workgroup w, pair p: unique, as a workgroup's pairs are consecutive).
//  3. merge: log-sum-exp merge of a pair's segment partials, * sigmoid(gate) -> bf16.
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

constexpr int kAttnWG = 512;          // attention workgroups (2 per CU on a 256-CU part)
constexpr float kRescaleLog2 = 8.0f;  // exponent base moves only when a row max grows > 2^8
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
// RoPE rows of verify position (b, t): the caller's [B, T, 64] rows, or with a table [P, 64]
// (the reference's _init_rope table, contrib/qwen3.6-27b/static_decode.py:489-502) its row
// kv_len[b] + t clamped to [0, P), the rows gqa::rope_rows would gather.
struct RopeSrc {
  const float* cos;   // [B, T, 64], or the table [P, 64] when P > 0
  const float* sin;
  int P;
};

__device__ __forceinline__ size_t rope_row(const RopeSrc& r, const int32_t* kv_len, int b, int t,
                                           int T) {
  if (r.P <= 0) return ((size_t)b * T + t) * ROPE;
  long pos = (long)kv_len[b] + t;
  pos = pos < 0 ? 0 : (pos >= r.P ? r.P - 1 : pos);
  return (size_t)pos * ROPE;
}

// ---------------------------------------------------------------------------------------
// KV append: cache row kv_len[b]+t of head g <- bf16(rope(bf16(rmsnorm_1p(key)))), value copy.
// One wave per (b, t, g); lane l owns dims 4l..4l+3.
struct AppendArgs {
  const uint16_t* key;
  const uint16_t* value;
  const float* k_norm;
  RopeSrc rope;
  uint16_t* cache_k;
  uint16_t* cache_v;
  const int32_t* kv_len;
  int B, T, Hkv, s_max;
};

__device__ __forceinline__ void kv_append_wave(const AppendArgs& a, int wave, int lane) {
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
    const size_t ro = rope_row(a.rope, a.kv_len, b, t, a.T) + 4 * lane;
    const float* cs = a.rope.cos + ro;
    const float* sn = a.rope.sin + ro;
    const float sign = lane < ROPE / 8 ? -1.0f : 1.0f;
    for (int j = 0; j < 4; ++j) x[j] = x[j] * cs[j] + sign * y[j] * sn[j];
  }
  const size_t row = (((size_t)b * a.Hkv + g) * a.s_max + pos) * DH + 4 * lane;
  for (int j = 0; j < 4; ++j) a.cache_k[row + j] = npn::f32_to_bf16(x[j]);
  const uint16_t* vs = a.value + (size_t)wave * DH + 4 * lane;
  for (int j = 0; j < 4; ++j) a.cache_v[row + j] = vs[j];
}

__global__ __launch_bounds__(256) void gqa_kv_append_kernel(AppendArgs a) {
  kv_append_wave(a, blockIdx.x * 4 + (threadIdx.x >> 6), threadIdx.x & 63);
}

// ---------------------------------------------------------------------------------------
// 1. q' = rope((1+w) * rmsnorm(q)) * log2(e)/16, split into bf16 hi/lo.
//    One wave per padded query row (b, g, r); lane l owns dims 4l..4l+3. Block 0 of the same
//    launch writes the split-KV plan instead (pstart, below), which the attention reads.
struct QPrepArgs {
  const uint16_t* query;
  const float* q_norm;
  RopeSrc rope;
  uint16_t* qhi;   // [B][Hkv][R][DH]
  uint16_t* qlo;
  const int32_t* kv_len;
  int32_t* pstart;  // [P + 1]
  int B, T, Hq, Hkv, R, P, s_max;
  int qblocks;      // blocks 1..qblocks prepare q'; any blocks after them append the new
  AppendArgs app;   // K/V rows to the cache (app.key != nullptr), one wave per row
};

__device__ __forceinline__ int pair_kend(const int32_t* kv_len, int b, int T, int s_max);

// The plan: pstart[p] = sum of the steps of pairs before p (exclusive scan over one block of
// 256 threads), pstart[P] = all steps.
__device__ void plan_block(const int32_t* kv_len, int32_t* pstart, int P, int Hkv, int T,
                           int s_max) {
  __shared__ int part[256];
  const int t = threadIdx.x;
  const int per = (P + 255) / 256;
  const int p0 = min(P, t * per), p1 = min(P, p0 + per);
  int sum = 0;
  for (int p = p0; p < p1; ++p) sum += (pair_kend(kv_len, p / Hkv, T, s_max) + KS - 1) / KS;
  part[t] = sum;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {  // inclusive Hillis-Steele scan
    const int v = t >= off ? part[t - off] : 0;
    __syncthreads();
    part[t] += v;
    __syncthreads();
  }
  int run = part[t] - sum;
  for (int p = p0; p < p1; ++p) {
    pstart[p] = run;
    run += (pair_kend(kv_len, p / Hkv, T, s_max) + KS - 1) / KS;
  }
  if (t == 255) pstart[P] = part[255];
}

__global__ __launch_bounds__(256) void gqa_qprep_kernel(QPrepArgs a) {
  if (blockIdx.x == 0) {
    plan_block(a.kv_len, a.pstart, a.P, a.Hkv, a.T, a.s_max);
    return;
  }
  if ((int)blockIdx.x > a.qblocks) {
    kv_append_wave(a.app, (blockIdx.x - 1 - a.qblocks) * 4 + (threadIdx.x >> 6), threadIdx.x & 63);
    return;
  }
  const int wave = (blockIdx.x - 1) * 4 + (threadIdx.x >> 6);
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
    const size_t ro = rope_row(a.rope, a.kv_len, b, t, a.T) + 4 * lane;
    const float* cs = a.rope.cos + ro;
    const float* sn = a.rope.sin + ro;
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
//    from HBM straight into LDS (global_load_lds_dwordx4) through an NST-stage ring.
//
//    LDS tile layout: one DMA instruction (64 lanes x 16 B) moves cache rows 2k and 2k+1
//    into "block" k, interleaved by 16-byte chunk: lane l carries row 2k + (l & 1), chunk
//    l >> 1, so chunk c of row r sits at block(r >> 1) + (2c + (r & 1)) * 16. Blocks are
//    1024 B plus a pad (K: 32 B, V: 64 B). With that layout
//      - every DMA source is the wave-uniform address of row 2k plus a per-lane constant
//        ((l & 1) * 512 + (l >> 1) * 16), and
//      - every MFMA operand read is one per-lane base plus an immediate offset,
//    and the reads spread over the LDS banks: 16 K rows at one column land on 16 distinct
//    16-byte bank groups (pad 32), and the transposed V reads of 4 rows x 64 B per 16-lane
//    group on 4 distinct 64-byte groups (pad 64).
struct AttnArgs {
  const uint16_t* qhi;
  const uint16_t* qlo;
  const uint16_t* cache_k;
  const uint16_t* cache_v;
  const int32_t* kv_len;
  const int32_t* pstart;  // [P + 1] first step of each pair; pstart[P] = total steps
  float* part_o;          // [kAttnWG + P][R][DH]
  float* part_ml;         // [kAttnWG + P][R][2]
  int Hkv, s_max, T, grp, npairs;
};

// Steps of pair p = (b, kv head): ceil(kend_b / KS), kend_b = min(kv_len[b] + T, s_max).
__device__ __forceinline__ int pair_kend(const int32_t* kv_len, int b, int T, int s_max) {
  const int L = kv_len[b] > 0 ? kv_len[b] : 0;
  return L + T < s_max ? L + T : s_max;
}

// Workgroups that take part for S steps in all: kAttnWG, or fewer when that would leave a
// workgroup under kMinSteps steps (small batches), so a workgroup's fixed costs (its q' rows,
// its partial rows, the ring's fill) stay small against its key stream and a pair's
// partials stay few for the merge.
constexpr int kMinSteps = 16;
__device__ __forceinline__ int attn_wgs(int S) {
  const int w = S / kMinSteps;
  return w < 1 ? 1 : (w > kAttnWG ? kAttnWG : w);
}

// Workgroup w's step range is [w * S / W, (w + 1) * S / W), W = attn_wgs(S).
__device__ __forceinline__ int wg_first_step(int w, int S) {
  return (int)((int64_t)w * S / attn_wgs(S));
}

// Largest p in [0, P) with pstart[p] <= x (pstart is strictly increasing, pstart[0] = 0):
// 64-way search, one sample per lane per round. Wave-uniform result.
__device__ __forceinline__ int find_pair(const int32_t* pstart, int P, int x, int lane) {
  int lo = 0, n = P;
  while (n > 1) {
    const int stride = (n + 63) / 64;
    const int idx = lo + lane * stride;
    const bool le = idx < lo + n && pstart[idx] <= x;
    const int t = __popcll(__builtin_amdgcn_ballot_w64(le)) - 1;  // last lane with le
    const int nlo = lo + t * stride;
    n = min(stride, lo + n - nlo);
    lo = nlo;
  }
  return __builtin_amdgcn_readfirstlane(lo);
}

constexpr int KBLK = 1024 + 32;            // bytes per 2-row block of the K tile
constexpr int VBLK = 1024 + 64;            // ... of the V tile
constexpr int KTILE = (KS / 2) * KBLK;     // 16896
constexpr int VTILE = (KS / 2) * VBLK;     // 17408
constexpr int STAGE = KTILE + VTILE + 1024;  // + one block of slack for padded DMA slots

// Reductions over the 4 lane groups (lanes i, i+16, i+32, i+48) that hold one query row,
// with gfx950's cross-row swaps instead of LDS permutes: after permlane32_swap(x, x) the
// pair holds (x[l & 31], x[(l & 31) + 32]); after permlane16_swap(y, y) it holds the two
// 16-lane rows of y's 32-lane half.
__device__ __forceinline__ float max_over_groups(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_over_groups(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

template <int NRT, int NST>  // NST: K/V ring stages
__global__ __launch_bounds__(NRT * 64, NST <= 2 ? 2 : 1) void gqa_attn_kernel(AttnArgs a) {
  constexpr int R = NRT * 16;
  constexpr int DPW = (KS + NRT - 1) / NRT;  // DMA instructions per wave per step
  const int wg = blockIdx.x;
  const int S = a.pstart[a.npairs];
  if (wg >= attn_wgs(S)) return;
  int x = wg_first_step(wg, S);
  const int x_end = wg_first_step(wg + 1, S);
  if (x >= x_end) return;

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int i = lane & 15, G = lane >> 4;
  const int row = w * 16 + i;  // this lane's query row (B-operand column / C column)

  __shared__ __attribute__((aligned(16))) uint8_t smem[NST * STAGE];
  const unsigned smem_lds = __builtin_amdgcn_readfirstlane(npn::lds_addr(smem));

  // Per-lane constants. DMA source offset within a 2-row block; LDS bases of the operand
  // reads: K row i (+16 for the second key tile), chunk 4*ks + G; V (transposed reads)
  // key rows 4G + (i>>2) (+16) of dims 16*dt + 4*(i&3) .. +3, i.e. chunk
  // 2*dt + ((i&3)>>1), half (i&1).
  const unsigned lane_src = (unsigned)((lane & 1) * DH * 2 + (lane >> 1) * 16);
  const int tr_row = 4 * G + (i >> 2);
  const int k_base0 = (i >> 1) * KBLK + (2 * G + (i & 1)) * 16;
  const int v_base0 = KTILE + (tr_row >> 1) * VBLK + (2 * ((i & 3) >> 1) + (tr_row & 1)) * 16 +
                      (i & 1) * 8;

  int p = find_pair(a.pstart, a.npairs, x, lane);
  while (x < x_end) {
    const int pbeg = a.pstart[p];
    const int s_lo = x - pbeg;
    const int steps = min(x_end, (int)a.pstart[p + 1]) - x;
    const int bg = p;
    const int b = bg / a.Hkv;
    const int L = a.kv_len[b] > 0 ? a.kv_len[b] : 0;
    const int kend = pair_kend(a.kv_len, b, a.T, a.s_max);  // rows [0, kend) are read
    const int c0 = s_lo * KS;
    const uint8_t* kb = reinterpret_cast<const uint8_t*>(a.cache_k + (size_t)bg * a.s_max * DH);
    const uint8_t* vb = reinterpret_cast<const uint8_t*>(a.cache_v + (size_t)bg * a.s_max * DH);

    // Every wave has finished reading the previous segment's stages.
    __builtin_amdgcn_s_barrier();

    // DMA of step s's tiles into stage s % NST: slot j < 16 is K block j, 16 <= j < 32 is
    // V block j - 16, DPW slots per wave; slots past 32 (NRT * DPW > 32) fill the slack.
    // A step that reaches past kend (a pair's last) clamps its rows to kend - 1, so V rows
    // the mask removes still hold finite cache data.
    // Each slot's LDS offset within a stage and its source at step 0 are fixed for the
    // segment (wave-uniform, kept in SGPRs), so a step's DMAs are one 64-bit add each; the
    // test for a step past kend is made once per step rather than once per slot.
    unsigned sdst[DPW];
    const uint8_t* ssrc[DPW];
#pragma unroll
    for (int q = 0; q < DPW; ++q) {
      const int j = w + NRT * q;  // wave-uniform slot
      const bool isv = j >= KS / 2;
      const int blk = (isv ? j - KS / 2 : j) & (KS / 2 - 1);
      sdst[q] = j < KS ? (isv ? KTILE + blk * VBLK : blk * KBLK) : KTILE + VTILE;
      ssrc[q] = (isv ? vb : kb) + (size_t)(c0 + 2 * blk) * DH * 2;
    }
    auto dma = [&](int s) {
      const int k0 = c0 + s * KS;
      uint8_t* st = smem + (s % NST) * STAGE;
      if (k0 + KS <= kend) {
        const size_t step = (size_t)s * KS * DH * 2;
        const unsigned st_lds = smem_lds + (unsigned)((s % NST) * STAGE);
#pragma unroll
        for (int q = 0; q < DPW; ++q) npn::lds_dma16_soff(ssrc[q] + step, lane_src, st_lds + sdst[q]);
      } else {
#pragma unroll
        for (int q = 0; q < DPW; ++q) {
          const int j = w + NRT * q;
          const bool isv = j >= KS / 2;
          const int blk = (isv ? j - KS / 2 : j) & (KS / 2 - 1);
          const int key = min(k0 + 2 * blk + (lane & 1), kend - 1);
          npn::lds_dma16_soff(isv ? vb : kb, (unsigned)key * DH * 2 + (unsigned)(lane >> 1) * 16,
                              st + sdst[q]);
        }
      }
    };
    // q' hi/lo of this lane's row as B operands: dims 32*ks + 8*G .. +7. Loaded by inline
    // asm ahead of the K/V DMAs, so the loop's own vmcnt wait for step 0 covers them (a
    // compiler-tracked load would make the compiler wait for every DMA issued after it).
    u32x4 qh[8], ql[8];
    {
      const size_t qo = ((size_t)bg * R + row) * DH + 8 * G;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(qh[ks]) : "v"(a.qhi + qo + 32 * ks)
                     : "memory");
        asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(ql[ks]) : "v"(a.qlo + qo + 32 * ks)
                     : "memory");
      }
    }
    for (int s = 0; s < NST - 1 && s < steps; ++s) dma(s);

    const int lim = row < a.T * a.grp ? L + row / a.grp : kend - 1;  // last key this row sees

    float m_run = kNegBig, l_run = 0.f;
    f32x4 acc[16];
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int s = 0; s < steps; ++s) {
      const int k0 = c0 + s * KS;
      // This wave's DMA of step s has landed once at most the DMAs of the steps after it
      // stay in flight: steps up to s + NST - 2 are issued here (vmcnt holds 6 bits; a
      // smaller count only waits longer).
      if (NST >= 4 && s + 2 < steps)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * DPW < 63 ? 2 * DPW : 63) : "memory");
      else if (NST >= 3 && s + 1 < steps)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DPW < 63 ? DPW : 63) : "memory");
      else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();  // ... and every other wave's; stage of step s-1 is free
      asm volatile("" ::: "memory");
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {  // q' registers are read only after that wait
        asm volatile("" : "+v"(qh[ks]));
        asm volatile("" : "+v"(ql[ks]));
      }
      if (s + NST - 1 < steps) dma(s + NST - 1);
      const uint8_t* stage = smem + (s % NST) * STAGE;
      const uint8_t* kp = stage + k_base0;
      const uint8_t* vp = stage + v_base0;

      // S^T[32 keys x 16 rows] = K Q'^T. All 16 K fragments are read first so their LDS
      // latencies overlap; the two key tiles' accumulation chains alternate.
      u32x4 kf[2][8];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
          kf[kt][ks] = *reinterpret_cast<const u32x4*>(kp + kt * (KS / 4) * KBLK + ks * 128);
      f32x4 st[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
          st[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kf[kt][ks]),
                                                           as_bf16x8(qh[ks]), st[kt], 0, 0, 0);
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
          st[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kf[kt][ks]),
                                                           as_bf16x8(ql[ks]), st[kt], 0, 0, 0);
      }
      // Keep the 16 K reads ahead of the 32 MFMAs (the scheduler would otherwise pair each
      // read with its MFMAs and expose the LDS latency 8 times); V fragments then reuse
      // the K fragments' registers.
      __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 32, 0);
      __builtin_amdgcn_sched_barrier(0);

      // V^T fragments of all 16 dim tiles, read before the softmax so their latency
      // overlaps it.
      bf16x8 vf[16];
#pragma unroll
      for (int dt = 0; dt < 16; ++dt)
        vf[dt] = pack8(lds_tr16(vp + dt * 64), lds_tr16(vp + dt * 64 + (KS / 4) * VBLK));

      // causal mask (only a step that reaches past the first query row's limit L needs
      // one) + online softmax (base 2); P hi/lo become the B operands of P.V.
      if (k0 + KS - 1 > L) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (k0 + 16 * kt + 4 * G + r > lim) st[kt][r] = -INFINITY;
      }
      float mx = fmaxf(fmaxf(fmaxf(st[0][0], st[0][1]), fmaxf(st[0][2], st[0][3])),
                       fmaxf(fmaxf(st[1][0], st[1][1]), fmaxf(st[1][2], st[1][3])));
      mx = max_over_groups(mx);
      // The exponent base m_run moves only when a row's max exceeds it by more than 2^8,
      // so p = 2^(s - m_run) <= 256 and most steps skip rescaling O; O / l does not depend
      // on the base. The branch is wave-uniform.
      const bool grow = mx > m_run + kRescaleLog2;
      if (__builtin_amdgcn_ballot_w64(grow) != 0) {
        const float mnew = grow ? mx : m_run;
        const float corr = exp2f(m_run - mnew);
        m_run = mnew;
        l_run *= corr;
#pragma unroll
        for (int dt = 0; dt < 16; ++dt) acc[dt] *= corr;
      }
      bf16x8 ph, pl;
      float psum = 0.f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pv = exp2f(st[kt][r] - m_run);
          psum += pv;
          const __bf16 h = (__bf16)pv;
          ph[kt * 4 + r] = h;
          pl[kt * 4 + r] = (__bf16)(pv - (float)h);
        }
      l_run += psum;

      // O^T[256 x 16 rows] += V^T P^T
#pragma unroll
      for (int dt = 0; dt < 16; ++dt)
        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[dt], ph, acc[dt], 0, 0, 0);
#pragma unroll
      for (int dt = 0; dt < 16; ++dt)
        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[dt], pl, acc[dt], 0, 0, 0);
    }

    // Row sum over the 4 lane groups, then this wave's 16 rows of the segment partial.
    l_run = sum_over_groups(l_run);
    const size_t slot = (size_t)wg + p;
    float* po = a.part_o + (slot * R + row) * DH;
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) *reinterpret_cast<f32x4*>(po + 16 * dt + 4 * G) = acc[dt];
    if (G == 0) {
      float* pml = a.part_ml + (slot * R + row) * 2;
      pml[0] = m_run;
      pml[1] = l_run;
    }
    x += steps;
    ++p;
  }
}

// ---------------------------------------------------------------------------------------
// 3. merge a pair's segment partials, apply sigmoid(gate), write bf16. One 256-thread block
//    per (query row, pair); lane l of every wave owns output dims 4l..4l+3 (float4 partial
//    reads). The workgroups that covered pair p are w(first step) .. w(last step), with
//    w(x) = ((x + 1) * W - 1) / S, W = attn_wgs(S). Wave q merges segments q, q + 4, ... of
//    the pair (loads issued four segments at a time), and wave 0 then merges the four
//    waves' (m, l, O) in wave order: a small batch's pairs have tens of segments each, which
//    one wave walking them in turn paid for in memory latency.
struct MergeArgs {
  const float* part_o;
  const float* part_ml;
  const int32_t* pstart;
  const uint16_t* gate;
  uint16_t* out;
  int T, Hq, Hkv, R, npairs;
};

constexpr int kMergeRowsMinPairs = 64;  // pairs from which gqa_merge_rows_kernel merges

__global__ __launch_bounds__(256) void gqa_merge_kernel(MergeArgs a) {
  const int r = blockIdx.x;
  const int pr = blockIdx.y;
  const int b = pr / a.Hkv, g = pr - b * a.Hkv;
  const int grp = a.Hq / a.Hkv;
  const int q = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int S = a.pstart[a.npairs];
  const int64_t W = attn_wgs(S);
  const int x0 = a.pstart[pr], x1 = a.pstart[pr + 1] - 1;
  const int w0 = (int)(((int64_t)(x0 + 1) * W - 1) / S);
  const int w1 = (int)(((int64_t)(x1 + 1) * W - 1) / S);
  const size_t stride_ml = (size_t)a.R * 2, stride_o = (size_t)a.R * DH;
  const float* pml = a.part_ml + ((size_t)(w0 + pr) * a.R + r) * 2;
  const float* po = a.part_o + ((size_t)(w0 + pr) * a.R + r) * DH + 4 * lane;
  auto live = [&](int w) { return w <= w1 && wg_first_step(w, S) < wg_first_step(w + 1, S); };
  const int t = r / grp, qh = g * grp + (r - t * grp);
  const size_t oi = (((size_t)b * a.T + t) * a.Hq + qh) * DH + 4 * lane;
  // The gate is needed only by wave 0's output, after the merge: its load is issued first.
  uint2 gate_bits = make_uint2(0u, 0u);
  if (q == 0) gate_bits = *reinterpret_cast<const uint2*>(a.gate + oi);
  // This wave's segments w0 + q + 4 j: their maximum, then their rescaled sums. The first
  // batch of four (all of a pair's segments whenever it has at most 16) is loaded once and
  // kept in registers for both passes: one round trip to memory instead of two, with the
  // same arithmetic.
  float mv0[4], lv0[4];
  f32x4 ov0[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int w = w0 + q + 4 * j;
    const bool ok = live(w);
    mv0[j] = ok ? pml[(w - w0) * stride_ml] : kNegBig;
    lv0[j] = ok ? pml[(w - w0) * stride_ml + 1] : 0.f;
    ov0[j] = ok ? *reinterpret_cast<const f32x4*>(po + (w - w0) * stride_o)
                : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  float M = kNegBig;
#pragma unroll
  for (int j = 0; j < 4; ++j) M = fmaxf(M, mv0[j]);
  for (int base = w0 + q + 16; base <= w1; base += 16) {
    float mv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int w = base + 4 * j;
      mv[j] = live(w) ? pml[(w - w0) * stride_ml] : kNegBig;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) M = fmaxf(M, mv[j]);
  }
  float l = 0.f;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float f = exp2f(mv0[j] - M);
    l += f * lv0[j];
    o += f * ov0[j];
  }
  for (int base = w0 + q + 16; base <= w1; base += 16) {
    float mv[4], lv[4];
    f32x4 ov[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int w = base + 4 * j;
      const bool ok = live(w);
      mv[j] = ok ? pml[(w - w0) * stride_ml] : kNegBig;
      lv[j] = ok ? pml[(w - w0) * stride_ml + 1] : 0.f;
      ov[j] = ok ? *reinterpret_cast<const f32x4*>(po + (w - w0) * stride_o)
                 : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float f = exp2f(mv[j] - M);
      l += f * lv[j];
      o += f * ov[j];
    }
  }
  __shared__ float s_ml[4][2];
  __shared__ f32x4 s_o[4][64];
  if (lane == 0) {
    s_ml[q][0] = M;
    s_ml[q][1] = l;
  }
  s_o[q][lane] = o;
  __syncthreads();
  if (q != 0) return;
  float Mt = s_ml[0][0];
#pragma unroll
  for (int k = 1; k < 4; ++k) Mt = fmaxf(Mt, s_ml[k][0]);
  float lt = 0.f;
  f32x4 ot = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float f = exp2f(s_ml[k][0] - Mt);
    lt += f * s_ml[k][1];
    ot += f * s_o[k][lane];
  }
  const float inv = 1.0f / lt;
  const uint32_t gw[2] = {gate_bits.x, gate_bits.y};
  uint32_t w[2];
  for (int j = 0; j < 2; ++j) {
    const float g0 = npn::sigmoid(npn::bf16_to_f32((uint16_t)(gw[j] & 0xFFFFu)));
    const float g1 = npn::sigmoid(npn::bf16_to_f32((uint16_t)(gw[j] >> 16)));
    w[j] = npn::f32_to_bf16(ot[2 * j] * inv * g0) |
           ((uint32_t)npn::f32_to_bf16(ot[2 * j + 1] * inv * g1) << 16);
  }
  *reinterpret_cast<uint2*>(a.out + oi) = make_uint2(w[0], w[1]);
}

// The same merge with one wave per query row (four rows per block) walking all of the pair's
// segments itself: for batches whose pairs have a few segments each (the host picks it when
// there are at least 64 pairs, about 8 segments per pair or fewer), a quarter as many blocks
// and no LDS exchange. Segments are loaded four at a time; the first four stay in registers
// for both the max pass and the sum pass.
__global__ __launch_bounds__(256) void gqa_merge_rows_kernel(MergeArgs a) {
  const int q = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int grp = a.Hq / a.Hkv;
  const int r = blockIdx.x * 4 + q;  // query row of the pair, t * grp + head; a.R >= T * grp
  if (r >= a.T * grp) return;        // wave-uniform; the kernel has no block barrier
  const int pr = blockIdx.y;
  const int b = pr / a.Hkv, g = pr - b * a.Hkv;
  const int S = a.pstart[a.npairs];
  const int64_t W = attn_wgs(S);
  const int x0 = a.pstart[pr], x1 = a.pstart[pr + 1] - 1;
  const int w0 = (int)(((int64_t)(x0 + 1) * W - 1) / S);
  const int w1 = (int)(((int64_t)(x1 + 1) * W - 1) / S);
  const size_t stride_ml = (size_t)a.R * 2, stride_o = (size_t)a.R * DH;
  const float* pml = a.part_ml + ((size_t)(w0 + pr) * a.R + r) * 2;
  const float* po = a.part_o + ((size_t)(w0 + pr) * a.R + r) * DH + 4 * lane;
  auto live = [&](int w) { return w <= w1 && wg_first_step(w, S) < wg_first_step(w + 1, S); };
  const int t = r / grp, qh = g * grp + (r - t * grp);
  const size_t oi = (((size_t)b * a.T + t) * a.Hq + qh) * DH + 4 * lane;
  const uint2 gate_bits = *reinterpret_cast<const uint2*>(a.gate + oi);
  float mv0[4], lv0[4];
  f32x4 ov0[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int w = w0 + j;
    const bool ok = live(w);
    mv0[j] = ok ? pml[(w - w0) * stride_ml] : kNegBig;
    lv0[j] = ok ? pml[(w - w0) * stride_ml + 1] : 0.f;
    ov0[j] = ok ? *reinterpret_cast<const f32x4*>(po + (w - w0) * stride_o)
                : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  float M = kNegBig;
#pragma unroll
  for (int j = 0; j < 4; ++j) M = fmaxf(M, mv0[j]);
  for (int base = w0 + 4; base <= w1; base += 4) {
    float mv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int w = base + j;
      mv[j] = live(w) ? pml[(w - w0) * stride_ml] : kNegBig;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) M = fmaxf(M, mv[j]);
  }
  float l = 0.f;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float f = exp2f(mv0[j] - M);
    l += f * lv0[j];
    o += f * ov0[j];
  }
  for (int base = w0 + 4; base <= w1; base += 4) {
    float mv[4], lv[4];
    f32x4 ov[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int w = base + j;
      const bool ok = live(w);
      mv[j] = ok ? pml[(w - w0) * stride_ml] : kNegBig;
      lv[j] = ok ? pml[(w - w0) * stride_ml + 1] : 0.f;
      ov[j] = ok ? *reinterpret_cast<const f32x4*>(po + (w - w0) * stride_o)
                 : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float f = exp2f(mv[j] - M);
      l += f * lv[j];
      o += f * ov[j];
    }
  }
  const float inv = 1.0f / l;
  const uint32_t gw[2] = {gate_bits.x, gate_bits.y};
  uint32_t w[2];
  for (int j = 0; j < 2; ++j) {
    const float g0 = npn::sigmoid(npn::bf16_to_f32((uint16_t)(gw[j] & 0xFFFFu)));
    const float g1 = npn::sigmoid(npn::bf16_to_f32((uint16_t)(gw[j] >> 16)));
    w[j] = npn::f32_to_bf16(o[2 * j] * inv * g0) |
           ((uint32_t)npn::f32_to_bf16(o[2 * j + 1] * inv * g1) << 16);
  }
  *reinterpret_cast<uint2*>(a.out + oi) = make_uint2(w[0], w[1]);
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
  int grp, R, nrt, P;
  size_t q_bytes, po_bytes, pml_bytes, ps_bytes, total;
};

VerifyPlan plan(int B, int T, int Hq, int Hkv) {
  VerifyPlan p{};
  p.grp = Hq / Hkv;
  p.nrt = (T * p.grp + 15) / 16;
  p.R = p.nrt * 16;
  p.P = B * Hkv;
  const size_t slots = (size_t)kAttnWG + p.P;
  auto up = [](size_t x) { return (x + 255) & ~size_t(255); };
  p.q_bytes = up((size_t)p.P * p.R * DH * 2);
  p.po_bytes = up(slots * p.R * DH * 4);
  p.pml_bytes = up(slots * p.R * 2 * 4);
  p.ps_bytes = up((size_t)(p.P + 1) * 4);
  p.total = 2 * p.q_bytes + p.po_bytes + p.pml_bytes + p.ps_bytes;
  return p;
}

bool verify_shape_ok(int B, int T, int Hq, int Hkv, int s_max) {
  // s_max <= 2^23 keeps cache row offsets in 32 bits; the total step count in int32.
  // B * Hkv is the merge grid's y extent (<= 65535).
  return B >= 1 && (int64_t)B * Hkv <= 65535 && T >= 1 && Hkv >= 1 && Hq >= Hkv && Hq % Hkv == 0 &&
         T * (Hq / Hkv) <= 48 && s_max >= T && s_max <= (1 << 23) &&
         (int64_t)B * Hkv * ((s_max + KS - 1) / KS) < ((int64_t)1 << 31);
}

}  // namespace

extern "C" size_t npn_gqa_tail_verify_workspace_size(int B, int T, int q_heads, int kv_heads,
                                                     int s_max) {
  if (!verify_shape_ok(B, T, q_heads, kv_heads, s_max)) return 0;
  return plan(B, T, q_heads, kv_heads).total;
}

// The verify tail's launches; with app.key set the query-prep launch also appends the new
// K/V rows (the attention launch that follows reads them).
static int tail_verify_launch(const uint16_t* query, const uint16_t* gate, const float* q_norm,
                              RopeSrc rope, const AppendArgs& app, const uint16_t* cache_k,
                              const uint16_t* cache_v, const int32_t* kv_len, uint16_t* out,
                              int B, int T, int q_heads, int kv_heads, int s_max, void* workspace,
                              size_t workspace_bytes, void* stream) {
  NPN_REQUIRE(query && gate && q_norm && rope.cos && rope.sin && cache_k && cache_v && kv_len &&
                  out,
              NPN_ERR_NULL);
  NPN_REQUIRE(verify_shape_ok(B, T, q_heads, kv_heads, s_max), NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(cache_k) && NPN_ALIGNED16(cache_v) && NPN_ALIGNED16(workspace) &&
                  NPN_ALIGNED16(gate) && NPN_ALIGNED16(out),
              NPN_ERR_ALIGN);
  const VerifyPlan p = plan(B, T, q_heads, kv_heads);
  NPN_REQUIRE(workspace != nullptr && workspace_bytes >= p.total, NPN_ERR_WORKSPACE);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint16_t* qhi = reinterpret_cast<uint16_t*>(ws);
  uint16_t* qlo = reinterpret_cast<uint16_t*>(ws + p.q_bytes);
  float* po = reinterpret_cast<float*>(ws + 2 * p.q_bytes);
  float* pml = reinterpret_cast<float*>(ws + 2 * p.q_bytes + p.po_bytes);
  int32_t* pstart = reinterpret_cast<int32_t*>(ws + 2 * p.q_bytes + p.po_bytes + p.pml_bytes);

  const int rows = B * kv_heads * p.R;
  const int qblocks = (rows + 3) / 4;
  QPrepArgs qa{query, q_norm, rope, qhi, qlo, kv_len, pstart, B, T, q_heads, kv_heads, p.R,
               p.P, s_max, qblocks, app};
  const int ablocks = app.key != nullptr ? (B * T * kv_heads + 3) / 4 : 0;
  hipLaunchKernelGGL(gqa_qprep_kernel, dim3(1 + qblocks + ablocks), dim3(256), 0, s, qa);

  AttnArgs aa{qhi, qlo, cache_k, cache_v, kv_len, pstart, po, pml, kv_heads, s_max, T, p.grp, p.P};
  const dim3 grid(kAttnWG);
  if (p.nrt == 1) hipLaunchKernelGGL((gqa_attn_kernel<1, 2>), grid, dim3(64), 0, s, aa);
  else if (p.nrt == 2) hipLaunchKernelGGL((gqa_attn_kernel<2, 2>), grid, dim3(128), 0, s, aa);
  else hipLaunchKernelGGL((gqa_attn_kernel<3, 2>), grid, dim3(192), 0, s, aa);

  MergeArgs ma{po, pml, pstart, gate, out, T, q_heads, kv_heads, p.R, p.P};
  if (p.P >= kMergeRowsMinPairs)
    hipLaunchKernelGGL(gqa_merge_rows_kernel, dim3((T * p.grp + 3) / 4, p.P), dim3(256), 0, s,
                       ma);
  else
    hipLaunchKernelGGL(gqa_merge_kernel, dim3(T * p.grp, p.P), dim3(256), 0, s, ma);
  return npn_launch_status();
}

extern "C" int npn_gqa_tail_verify(const uint16_t* query, const uint16_t* gate,
                                   const float* q_norm, const float* cos, const float* sin,
                                   const uint16_t* cache_k, const uint16_t* cache_v,
                                   const int32_t* kv_len, uint16_t* out, int B, int T,
                                   int q_heads, int kv_heads, int s_max, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  AppendArgs none{};
  return tail_verify_launch(query, gate, q_norm, RopeSrc{cos, sin, 0}, none, cache_k, cache_v,
                            kv_len, out, B, T, q_heads, kv_heads, s_max, workspace,
                            workspace_bytes, stream);
}

extern "C" int npn_gqa_tail_verify_append(const uint16_t* query, const uint16_t* gate,
                                          const uint16_t* key, const uint16_t* value,
                                          const float* q_norm, const float* k_norm,
                                          const float* cos_table, const float* sin_table,
                                          int positions, uint16_t* cache_k, uint16_t* cache_v,
                                          const int32_t* kv_len, uint16_t* out, int B, int T,
                                          int q_heads, int kv_heads, int s_max, void* workspace,
                                          size_t workspace_bytes, void* stream) {
  NPN_REQUIRE(key && value && k_norm, NPN_ERR_NULL);
  NPN_REQUIRE(positions >= 1, NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(cos_table) && NPN_ALIGNED16(sin_table), NPN_ERR_ALIGN);
  const RopeSrc rope{cos_table, sin_table, positions};
  const AppendArgs app{key, value, k_norm, rope, cache_k, cache_v, kv_len, B, T, kv_heads, s_max};
  return tail_verify_launch(query, gate, q_norm, rope, app, cache_k, cache_v, kv_len, out, B, T,
                            q_heads, kv_heads, s_max, workspace, workspace_bytes, stream);
}

extern "C" int npn_gqa_kv_append(const uint16_t* key, const uint16_t* value, const float* k_norm,
                                 const float* cos, const float* sin, uint16_t* cache_k,
                                 uint16_t* cache_v, const int32_t* kv_len, int B, int T,
                                 int kv_heads, int s_max, void* stream) {
  NPN_REQUIRE(key && value && k_norm && cos && sin && cache_k && cache_v && kv_len, NPN_ERR_NULL);
  NPN_REQUIRE(B >= 1 && T >= 1 && kv_heads >= 1 && s_max >= T, NPN_ERR_SHAPE);
  AppendArgs aa{key, value, k_norm, RopeSrc{cos, sin, 0}, cache_k, cache_v, kv_len, B, T,
                kv_heads, s_max};
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
