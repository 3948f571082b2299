// Inter-layer glue of the verify step, fused into single passes over HBM
// (the decode loop contrib/qwen3.6-27b/static_decode.py:533-542):
//   residual RMSNorm  hidden' = bf16(hidden + delta);  normed = bf16((1 + w) * hidden' *
//                     rsqrt(mean(hidden'^2) + eps))          (rms_norm, static_decode.py:322-335)
//   SwiGLU            y = bf16(bf16(silu(gate)) * up)         (_mlp_layer, static_decode.py:951-963;
//                     gate, up and silu(gate) are bf16 tensors there, so two roundings)
//   DeltaNet split    in-proj row [qkv | z | a | b | pad] -> mixed_qkv, z (bf16), a, b (f32)
//                     (the slicing and casts of _deltanet_layer, static_decode.py:802-832)
//   GQA split         q/k/v-proj row [(query | gate) per q head | key per kv head | value per
//                     kv head] -> query, gate, key, value (_gqa_layer, static_decode.py:867-890)
// All four move 16-byte chunks (8 bf16) per lane; widths must be multiples of 8.
// The residual norm and the two splits also read their input straight from the fp32 split-K
// partials of the projection GEMM that produces it (npn_fp8_matmul_partials): each 8-value
// chunk is bf16(scale * (p_0 + p_1 + ... + p_{S-1})), summed from 0 in that order, which is
// exactly what the GEMM's own reduction writes, so the results are bit-identical and the
// reduction's launch and its bf16 round trip through HBM go away.
#include "npn_common.h"

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void unpack8(const u32x4 v, float (&f)[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f[2 * j] = __uint_as_float(v[j] << 16);
    f[2 * j + 1] = __uint_as_float(v[j] & 0xFFFF0000u);
  }
}

__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
  u32x4 v;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    v[j] = (uint32_t)npn::f32_to_bf16(f[2 * j]) | ((uint32_t)npn::f32_to_bf16(f[2 * j + 1]) << 16);
  return v;
}

// Input sources: 8 bf16 values of row m starting at column col (a multiple of 8).
struct BfSrc {  // a bf16 matrix with row stride ld
  const uint16_t* p;
  int ld;
  __device__ __forceinline__ u32x4 load(size_t m, int col) const {
    return *reinterpret_cast<const u32x4*>(p + m * ld + col);
  }
};
constexpr int kMaxSplit = 16;  // the GEMM plan's largest split-K factor
constexpr int kSplitBatch = 8;  // partials loaded per batch (unrolled)

struct PartSrc {  // fp32 split-K partials [S][M][ld] and the per-column scale, S <= kMaxSplit
  const float* p;
  const float* scale;
  int ld, S;
  size_t stride;  // M * ld
  __device__ __forceinline__ u32x4 load(size_t m, int col) const {
    // The partials are added in order s = 0 .. S-1 (as the GEMM's own reduction does); the
    // loads of each batch of 8 are issued before its first add (unrolled, predicated), so
    // one memory latency is paid per batch rather than per partial.
    const float* q = p + m * ld + col;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < S; s0 += kSplitBatch) {
      float4 a[kSplitBatch], b[kSplitBatch];
#pragma unroll
      for (int j = 0; j < kSplitBatch; ++j) {
        if (s0 + j < S) {
          a[j] = *reinterpret_cast<const float4*>(q + (s0 + j) * stride);
          b[j] = *reinterpret_cast<const float4*>(q + (s0 + j) * stride + 4);
        }
      }
#pragma unroll
      for (int j = 0; j < kSplitBatch; ++j) {
        if (s0 + j < S) {
          acc[0] += a[j].x; acc[1] += a[j].y; acc[2] += a[j].z; acc[3] += a[j].w;
          acc[4] += b[j].x; acc[5] += b[j].y; acc[6] += b[j].z; acc[7] += b[j].w;
        }
      }
    }
    const float4 s0 = *reinterpret_cast<const float4*>(scale + col);
    const float4 s1 = *reinterpret_cast<const float4*>(scale + col + 4);
    const float o[8] = {acc[0] * s0.x, acc[1] * s0.y, acc[2] * s0.z, acc[3] * s0.w,
                        acc[4] * s1.x, acc[5] * s1.y, acc[6] * s1.z, acc[7] * s1.w};
    return pack8(o);
  }
};

// ---- residual + (1 + w) RMSNorm: one 1024-thread workgroup per row; the row (<= 2 chunks of
// 8 per thread, H <= 16384) stays in registers between the sum of squares and the scaling,
// and with split-K partials (S row segments per chunk) many loads are in flight per row.
// Both input forms use this one layout, so their sums of squares associate identically.
// Every load of the row is issued before the first store (hidden_out may alias hidden_in).
constexpr int kNormThreads = 1024;
constexpr int kNormMaxChunks = 2;

template <class Src>
__global__ __launch_bounds__(kNormThreads) void residual_rmsnorm_kernel(
    const uint16_t* h_in, Src delta, bool has_delta, const float* __restrict__ weight,
    uint16_t* h_out, uint16_t* __restrict__ y, int H, float eps) {  // h_out may alias h_in
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int nc = H / 8;
  const size_t base = (size_t)row * H;
  u32x4 hv[kNormMaxChunks], dv[kNormMaxChunks];
#pragma unroll
  for (int k = 0; k < kNormMaxChunks; ++k) {
    const int c = tid + k * kNormThreads;
    if (c < nc) {
      hv[k] = *reinterpret_cast<const u32x4*>(h_in + base + 8 * c);
      if (has_delta) dv[k] = delta.load(row, 8 * c);
    }
  }
  float x[kNormMaxChunks][8];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kNormMaxChunks; ++k) {
    const int c = tid + k * kNormThreads;
    if (c < nc) {
      unpack8(hv[k], x[k]);
      if (has_delta) {
        float d[8];
        unpack8(dv[k], d);
#pragma unroll
        for (int j = 0; j < 8; ++j) x[k][j] = npn::bf16_to_f32(npn::f32_to_bf16(x[k][j] + d[j]));
        *reinterpret_cast<u32x4*>(h_out + base + 8 * c) = pack8(x[k]);
      } else if (h_out != h_in) {
        *reinterpret_cast<u32x4*>(h_out + base + 8 * c) = hv[k];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += x[k][j] * x[k][j];
    }
  }
  __shared__ float part[kNormThreads / 64];
  ss = npn::wave_sum(ss);
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kNormThreads / 64; ++w) tot += part[w];
  const float r = rsqrtf(tot / (float)H + eps);
#pragma unroll
  for (int k = 0; k < kNormMaxChunks; ++k) {
    const int c = tid + k * kNormThreads;
    if (c < nc) {
      const float4 w0 = *reinterpret_cast<const float4*>(weight + 8 * c);
      const float4 w1 = *reinterpret_cast<const float4*>(weight + 8 * c + 4);
      const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
      float o[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = (1.0f + wv[j]) * (x[k][j] * r);
      *reinterpret_cast<u32x4*>(y + base + 8 * c) = pack8(o);
    }
  }
}

// ---- SwiGLU: gu [M, 2I] = [gate | up] -> y [M, I]; one lane per 8 outputs (grid-stride).
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gu,
                                                       uint16_t* __restrict__ y, int M, int I) {
  const int cpr = I / 8;  // chunks per row
  const size_t n = (size_t)M * cpr;
  for (size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x; c < n;
       c += (size_t)gridDim.x * blockDim.x) {
    const size_t m = c / cpr, j = c - m * cpr;
    float g[8], u[8], o[8];
    unpack8(*reinterpret_cast<const u32x4*>(gu + m * 2 * I + 8 * j), g);
    unpack8(*reinterpret_cast<const u32x4*>(gu + m * 2 * I + I + 8 * j), u);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float s = npn::bf16_to_f32(npn::f32_to_bf16(npn::silu_bf16(g[k])));
      o[k] = s * u[k];
    }
    *reinterpret_cast<u32x4*>(y + m * I + 8 * j) = pack8(o);
  }
}

// ---- DeltaNet in-projection split. Row m of proj (stride ld): [qkv_n | z_n | hv | hv | ...].
template <class Src>
__global__ __launch_bounds__(256) void dn_split_kernel(Src proj,
                                                       uint16_t* __restrict__ mixed,
                                                       uint16_t* __restrict__ z,
                                                       float* __restrict__ a,
                                                       float* __restrict__ b, int M, int qkv_n,
                                                       int z_n, int hv) {
  const int cq = qkv_n / 8, cz = z_n / 8, ch = hv / 8;
  const int cpr = cq + cz + 2 * ch;
  const size_t n = (size_t)M * cpr;
  for (size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x; c < n;
       c += (size_t)gridDim.x * blockDim.x) {
    const size_t m = c / cpr;
    const int j = (int)(c - m * cpr);
    const u32x4 v = proj.load(m, 8 * j);
    if (j < cq) {
      *reinterpret_cast<u32x4*>(mixed + m * qkv_n + 8 * j) = v;
    } else if (j < cq + cz) {
      *reinterpret_cast<u32x4*>(z + m * z_n + 8 * (j - cq)) = v;
    } else {
      const bool isb = j >= cq + cz + ch;
      const int k = j - cq - cz - (isb ? ch : 0);
      float f[8];
      unpack8(v, f);
      float* dst = (isb ? b : a) + m * hv + 8 * k;
      *reinterpret_cast<float4*>(dst) = make_float4(f[0], f[1], f[2], f[3]);
      *reinterpret_cast<float4*>(dst + 4) = make_float4(f[4], f[5], f[6], f[7]);
    }
  }
}

// ---- GQA projection split. Row m of proj (stride ld): query/gate interleaved per q head
// (hd each), then key per kv head, then value per kv head.
template <class Src>
__global__ __launch_bounds__(256) void gqa_split_kernel(Src proj,
                                                        uint16_t* __restrict__ query,
                                                        uint16_t* __restrict__ gate,
                                                        uint16_t* __restrict__ key,
                                                        uint16_t* __restrict__ value, int M,
                                                        int hq, int hkv, int hd) {
  const int ch = hd / 8;
  const int cqg = 2 * hq * ch;  // query+gate chunks per row
  const int ckv = hkv * ch;
  const int cpr = cqg + 2 * ckv;
  const size_t n = (size_t)M * cpr;
  for (size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x; c < n;
       c += (size_t)gridDim.x * blockDim.x) {
    const size_t m = c / cpr;
    const int j = (int)(c - m * cpr);
    const u32x4 v = proj.load(m, 8 * j);
    uint16_t* dst;
    if (j < cqg) {
      const int h = j / (2 * ch), r = j - h * 2 * ch;
      dst = (r < ch ? query : gate) + (m * hq + h) * hd + 8 * (r < ch ? r : r - ch);
    } else if (j < cqg + ckv) {
      dst = key + m * hkv * hd + 8 * (j - cqg);
    } else {
      dst = value + m * hkv * hd + 8 * (j - cqg - ckv);
    }
    *reinterpret_cast<u32x4*>(dst) = v;
  }
}

// ---- RoPE rows of the verify positions: cos/sin [B, T, D] = table[kv_len[b] + t] for a
// table [P, D] built once (the reference's _init_rope, static_decode.py:489-502); positions
// past the table are clamped to its last row.
__global__ __launch_bounds__(256) void rope_rows_kernel(const float* __restrict__ tcos,
                                                        const float* __restrict__ tsin,
                                                        const int32_t* __restrict__ kv_len,
                                                        float* __restrict__ cos_out,
                                                        float* __restrict__ sin_out, int B, int T,
                                                        int D, int P) {
  const int d4 = D / 4;
  const size_t n = (size_t)B * T * d4;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t bt = i / d4;
    const int k = (int)(i - bt * d4);
    const int b = (int)(bt / T), t = (int)(bt - (size_t)b * T);
    long pos = (long)kv_len[b] + t;
    pos = pos < 0 ? 0 : (pos >= P ? P - 1 : pos);
    reinterpret_cast<float4*>(cos_out)[i] = reinterpret_cast<const float4*>(tcos + pos * D)[k];
    reinterpret_cast<float4*>(sin_out)[i] = reinterpret_cast<const float4*>(tsin + pos * D)[k];
  }
}

// ---- Commit of a verify step's acceptance to the per-sequence decode state (one lane per
// sequence): prev_accepted = accepted; kv_len += accepted + 1; committed += accepted + 1.
__global__ __launch_bounds__(256) void commit_kernel(const int32_t* __restrict__ accepted,
                                                     int32_t* __restrict__ prev_accepted,
                                                     int32_t* __restrict__ kv_len,
                                                     int32_t* __restrict__ committed, int B) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const int a = accepted[b];
  if (prev_accepted != nullptr) prev_accepted[b] = a;
  if (kv_len != nullptr) kv_len[b] += a + 1;
  if (committed != nullptr) committed[b] += a + 1;
}

int grid_for(size_t chunks) {
  const size_t blocks = (chunks + 255) / 256;
  return (int)(blocks < 4096 ? (blocks > 0 ? blocks : 1) : 4096);
}

// ---- hidden += bf16(scale * sum of split-K partials), no norm (the slice's last residual):
// one thread per 8 columns, the partials summed by PartSrc in the GEMM reduction's order.
__global__ __launch_bounds__(256) void residual_add_partials_kernel(
    const uint16_t* h_in, PartSrc delta, uint16_t* h_out, int M, int H) {  // h_out may alias h_in
  const int nc = H / 8;
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)M * nc) return;
  const size_t row = i / nc;
  const int col = 8 * (int)(i - row * nc);
  const u32x4 hv = *reinterpret_cast<const u32x4*>(h_in + row * H + col);
  const u32x4 dv = delta.load(row, col);
  float x[8], d[8];
  unpack8(hv, x);
  unpack8(dv, d);
#pragma unroll
  for (int j = 0; j < 8; ++j) x[j] = npn::bf16_to_f32(npn::f32_to_bf16(x[j] + d[j]));
  *reinterpret_cast<u32x4*>(h_out + row * H + col) = pack8(x);
}

}  // namespace

extern "C" int npn_residual_rmsnorm(const uint16_t* hidden_in, const uint16_t* delta,
                                    const float* weight, uint16_t* hidden_out,
                                    uint16_t* normed, int M, int H, float eps, void* stream) {
  NPN_REQUIRE(hidden_in && weight && normed && (delta == nullptr || hidden_out), NPN_ERR_NULL);
  NPN_REQUIRE(M >= 1 && H >= 8 && H % 8 == 0 && H / 8 <= kNormThreads * kNormMaxChunks,
              NPN_ERR_SHAPE);
  NPN_REQUIRE(eps >= 0.0f, NPN_ERR_VALUE);
  NPN_REQUIRE(NPN_ALIGNED16(hidden_in) && NPN_ALIGNED16(delta) && NPN_ALIGNED16(weight) &&
                  NPN_ALIGNED16(hidden_out) && NPN_ALIGNED16(normed),
              NPN_ERR_ALIGN);
  uint16_t* hout = hidden_out ? hidden_out : const_cast<uint16_t*>(hidden_in);
  hipLaunchKernelGGL(residual_rmsnorm_kernel<BfSrc>, dim3(M), dim3(kNormThreads), 0,
                     static_cast<hipStream_t>(stream), hidden_in, BfSrc{delta, H},
                     delta != nullptr, weight, hout, normed, H, eps);
  return npn_launch_status();
}

extern "C" int npn_residual_rmsnorm_partials(const uint16_t* hidden_in, const float* partial,
                                             int split_k, const float* scale,
                                             const float* weight, uint16_t* hidden_out,
                                             uint16_t* normed, int M, int H, float eps,
                                             void* stream) {
  NPN_REQUIRE(hidden_in && partial && scale && weight && hidden_out && normed, NPN_ERR_NULL);
  NPN_REQUIRE(M >= 1 && H >= 8 && H % 8 == 0 && H / 8 <= kNormThreads * kNormMaxChunks &&
                  split_k >= 1 && split_k <= kMaxSplit,
              NPN_ERR_SHAPE);
  NPN_REQUIRE(eps >= 0.0f, NPN_ERR_VALUE);
  NPN_REQUIRE(NPN_ALIGNED16(hidden_in) && NPN_ALIGNED16(partial) && NPN_ALIGNED16(scale) &&
                  NPN_ALIGNED16(weight) && NPN_ALIGNED16(hidden_out) && NPN_ALIGNED16(normed),
              NPN_ERR_ALIGN);
  const PartSrc src{partial, scale, H, split_k, (size_t)M * H};
  hipLaunchKernelGGL(residual_rmsnorm_kernel<PartSrc>, dim3(M), dim3(kNormThreads), 0,
                     static_cast<hipStream_t>(stream), hidden_in, src, true, weight, hidden_out,
                     normed, H, eps);
  return npn_launch_status();
}

extern "C" int npn_residual_add_partials(const uint16_t* hidden_in, const float* partial,
                                         int split_k, const float* scale, uint16_t* hidden_out,
                                         int M, int H, void* stream) {
  NPN_REQUIRE(hidden_in && partial && scale && hidden_out, NPN_ERR_NULL);
  NPN_REQUIRE(M >= 1 && H >= 8 && H % 8 == 0 && split_k >= 1 && split_k <= kMaxSplit &&
                  (int64_t)M * H < ((int64_t)1 << 40),
              NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(hidden_in) && NPN_ALIGNED16(partial) && NPN_ALIGNED16(scale) &&
                  NPN_ALIGNED16(hidden_out),
              NPN_ERR_ALIGN);
  const PartSrc src{partial, scale, H, split_k, (size_t)M * H};
  const int64_t n = (int64_t)M * (H / 8);
  hipLaunchKernelGGL(residual_add_partials_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256),
                     0, static_cast<hipStream_t>(stream), hidden_in, src, hidden_out, M, H);
  return npn_launch_status();
}

extern "C" int npn_silu_mul(const uint16_t* gate_up, uint16_t* out, int M, int I, void* stream) {
  NPN_REQUIRE(gate_up && out, NPN_ERR_NULL);
  NPN_REQUIRE(M >= 1 && I >= 8 && I % 8 == 0, NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(gate_up) && NPN_ALIGNED16(out), NPN_ERR_ALIGN);
  hipLaunchKernelGGL(silu_mul_kernel, dim3(grid_for((size_t)M * (I / 8))), dim3(256), 0,
                     static_cast<hipStream_t>(stream), gate_up, out, M, I);
  return npn_launch_status();
}

extern "C" int npn_deltanet_split(const uint16_t* proj, int ld, uint16_t* mixed_qkv, uint16_t* z,
                                  float* a_out, float* b_out, int M, int qkv_n, int z_n, int hv,
                                  void* stream) {
  NPN_REQUIRE(proj && mixed_qkv && z && a_out && b_out, NPN_ERR_NULL);
  NPN_REQUIRE(M >= 1 && qkv_n % 8 == 0 && z_n % 8 == 0 && hv % 8 == 0 && qkv_n > 0 && z_n > 0 &&
                  hv > 0 && ld % 8 == 0 && ld >= qkv_n + z_n + 2 * hv,
              NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(proj) && NPN_ALIGNED16(mixed_qkv) && NPN_ALIGNED16(z) &&
                  NPN_ALIGNED16(a_out) && NPN_ALIGNED16(b_out),
              NPN_ERR_ALIGN);
  const size_t chunks = (size_t)M * ((qkv_n + z_n + 2 * hv) / 8);
  hipLaunchKernelGGL(dn_split_kernel<BfSrc>, dim3(grid_for(chunks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), BfSrc{proj, ld}, mixed_qkv, z, a_out,
                     b_out, M, qkv_n, z_n, hv);
  return npn_launch_status();
}

extern "C" int npn_deltanet_split_partials(const float* partial, int split_k, const float* scale,
                                           int ld, uint16_t* mixed_qkv, uint16_t* z,
                                           float* a_out, float* b_out, int M, int qkv_n, int z_n,
                                           int hv, void* stream) {
  NPN_REQUIRE(partial && scale && mixed_qkv && z && a_out && b_out, NPN_ERR_NULL);
  NPN_REQUIRE(M >= 1 && qkv_n % 8 == 0 && z_n % 8 == 0 && hv % 8 == 0 && qkv_n > 0 && z_n > 0 &&
                  hv > 0 && ld % 8 == 0 && ld >= qkv_n + z_n + 2 * hv && split_k >= 1 &&
                  split_k <= kMaxSplit,
              NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(partial) && NPN_ALIGNED16(scale) && NPN_ALIGNED16(mixed_qkv) &&
                  NPN_ALIGNED16(z) && NPN_ALIGNED16(a_out) && NPN_ALIGNED16(b_out),
              NPN_ERR_ALIGN);
  const size_t chunks = (size_t)M * ((qkv_n + z_n + 2 * hv) / 8);
  const PartSrc src{partial, scale, ld, split_k, (size_t)M * ld};
  hipLaunchKernelGGL(dn_split_kernel<PartSrc>, dim3(grid_for(chunks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), src, mixed_qkv, z, a_out, b_out, M, qkv_n,
                     z_n, hv);
  return npn_launch_status();
}

extern "C" int npn_gqa_split(const uint16_t* proj, int ld, uint16_t* query, uint16_t* gate,
                             uint16_t* key, uint16_t* value, int M, int q_heads, int kv_heads,
                             int head_dim, void* stream) {
  NPN_REQUIRE(proj && query && gate && key && value, NPN_ERR_NULL);
  NPN_REQUIRE(M >= 1 && q_heads >= 1 && kv_heads >= 1 && head_dim >= 8 && head_dim % 8 == 0 &&
                  ld % 8 == 0 && ld >= 2 * (q_heads + kv_heads) * head_dim,
              NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(proj) && NPN_ALIGNED16(query) && NPN_ALIGNED16(gate) &&
                  NPN_ALIGNED16(key) && NPN_ALIGNED16(value),
              NPN_ERR_ALIGN);
  const size_t chunks = (size_t)M * (2 * (q_heads + kv_heads) * head_dim / 8);
  hipLaunchKernelGGL(gqa_split_kernel<BfSrc>, dim3(grid_for(chunks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), BfSrc{proj, ld}, query, gate, key, value,
                     M, q_heads, kv_heads, head_dim);
  return npn_launch_status();
}

extern "C" int npn_gqa_split_partials(const float* partial, int split_k, const float* scale,
                                      int ld, uint16_t* query, uint16_t* gate, uint16_t* key,
                                      uint16_t* value, int M, int q_heads, int kv_heads,
                                      int head_dim, void* stream) {
  NPN_REQUIRE(partial && scale && query && gate && key && value, NPN_ERR_NULL);
  NPN_REQUIRE(M >= 1 && q_heads >= 1 && kv_heads >= 1 && head_dim >= 8 && head_dim % 8 == 0 &&
                  ld % 8 == 0 && ld >= 2 * (q_heads + kv_heads) * head_dim && split_k >= 1 &&
                  split_k <= kMaxSplit,
              NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(partial) && NPN_ALIGNED16(scale) && NPN_ALIGNED16(query) &&
                  NPN_ALIGNED16(gate) && NPN_ALIGNED16(key) && NPN_ALIGNED16(value),
              NPN_ERR_ALIGN);
  const size_t chunks = (size_t)M * (2 * (q_heads + kv_heads) * head_dim / 8);
  const PartSrc src{partial, scale, ld, split_k, (size_t)M * ld};
  hipLaunchKernelGGL(gqa_split_kernel<PartSrc>, dim3(grid_for(chunks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), src, query, gate, key, value, M, q_heads,
                     kv_heads, head_dim);
  return npn_launch_status();
}

extern "C" int npn_rope_rows(const float* cos_table, const float* sin_table, int positions,
                             const int32_t* kv_len, float* cos_out, float* sin_out, int B, int T,
                             int dim, void* stream) {
  NPN_REQUIRE(cos_table && sin_table && kv_len && cos_out && sin_out, NPN_ERR_NULL);
  NPN_REQUIRE(B >= 1 && T >= 1 && dim >= 4 && dim % 4 == 0 && positions >= 1, NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(cos_table) && NPN_ALIGNED16(sin_table) && NPN_ALIGNED16(cos_out) &&
                  NPN_ALIGNED16(sin_out),
              NPN_ERR_ALIGN);
  const size_t n = (size_t)B * T * (dim / 4);
  hipLaunchKernelGGL(rope_rows_kernel, dim3(grid_for(n)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), cos_table, sin_table, kv_len, cos_out,
                     sin_out, B, T, dim, positions);
  return npn_launch_status();
}

extern "C" int npn_spec_commit(const int32_t* accepted, int32_t* prev_accepted, int32_t* kv_len,
                               int32_t* committed, int B, void* stream) {
  NPN_REQUIRE(accepted != nullptr, NPN_ERR_NULL);
  NPN_REQUIRE(B >= 1, NPN_ERR_SHAPE);
  hipLaunchKernelGGL(commit_kernel, dim3((B + 255) / 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), accepted, prev_accepted, kv_len, committed,
                     B);
  return npn_launch_status();
}
