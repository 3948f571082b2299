// Gated-DeltaNet decode/verify kernels for gfx950.
//
// Math (per sequence b, v-head h, token t; k-head = h / (Hv/Hk)), from the reference's
// fused block contrib/qwen3.6-27b/kernels/deltanet_full.py:1-37 and its CPU check
// contrib/qwen3.6-27b/kernels/tests/test_deltanet_full.py:20-54:
//   y      = silu(sum_j w[c,j] * window[c,j] + bias[c])   window = [conv_state(3) || x_t]
//   q, k   = L2-normalised per head (q also * 1/sqrt(128)); v = y[v-head slice]
//   g      = -exp(A_log[h]) * softplus(a[t,h] + dt_bias[h]);  beta = sigmoid(b[t,h])
//   S     *= exp(g);  delta = (v - S^T k) * beta;  S += k delta^T;  o = S^T q
//   out    = o * rsqrt(mean(o^2) + 1e-6) * norm_w * silu(z)                -> bf16
//
// Layout in HBM: S[b][h] is a 128x128 fp32 row-major tile, row = k index, column = v
// index (the reference's [B*Hv*128, 128] state, deltanet_full_batched.py:11-22).
// Checkpoints ckpt[b][t][h] use the same tile layout, so the T=1 checkpoint buffer is
// exactly the reference's new_state.
//
// Work decomposition: one 128-thread workgroup per (b, h); thread j owns state column
// v = j and keeps all 128 rows of it in VGPRs for the whole verify block, so the
// column sums S^T k and S^T q are thread-local. Each checkpoint row is one
// 256-byte coalesced store per wave. The only cross-thread reductions are the q/k
// L2 norms (before the loop) and the output RMS norm (after it). The per-token q, k, v
// and o vectors live in LDS, which keeps the kernel at 168 VGPRs: three waves per SIMD,
// so B*Hv = 1536 workgroups (B = 32, Hv = 48) are resident at once on 256 CUs.
#include "npn_common.h"

namespace {

constexpr int D = 128;
constexpr int kThreads = 128;
constexpr float kEps = 1e-6f;

struct DnArgs {
  const float* state;
  const int32_t* state_index;
  int state_T;
  const uint16_t* mixed_qkv;
  const uint16_t* conv_state;
  const float* conv_weight;
  const float* conv_bias;
  const float* a_out;
  const float* b_out;
  const uint16_t* z;
  const float* A_log;
  const float* dt_bias;
  const float* norm_weight;
  float* ckpt;
  uint16_t* out;
  int B, T, Hk, Hv;
};

// Depthwise causal conv (4 taps, oldest first) + bias + SiLU of channel c over T tokens.
template <int TMAX>
__device__ __forceinline__ void conv_channel(const uint16_t* __restrict__ cs,
                                             const uint16_t* __restrict__ x,
                                             const float* __restrict__ w,
                                             const float* __restrict__ bias, int c, int QKV,
                                             int T, float (&y)[TMAX]) {
  const float w0 = w[c * 4 + 0], w1 = w[c * 4 + 1], w2 = w[c * 4 + 2], w3 = w[c * 4 + 3];
  const float bc = bias[c];
  float s0 = npn::bf16_to_f32(cs[c * 3 + 0]);
  float s1 = npn::bf16_to_f32(cs[c * 3 + 1]);
  float s2 = npn::bf16_to_f32(cs[c * 3 + 2]);
#pragma unroll
  for (int t = 0; t < TMAX; ++t) {
    if (t < T) {
      const float xt = npn::bf16_to_f32(x[(size_t)t * QKV + c]);
      y[t] = npn::silu(w0 * s0 + w1 * s1 + w2 * s2 + w3 * xt + bc);
      s0 = s1;
      s1 = s2;
      s2 = xt;
    } else {
      y[t] = 0.0f;
    }
  }
}

template <int TMAX>
__global__ __launch_bounds__(kThreads, 3) void dn_verify_kernel(DnArgs a) {
  const int b = blockIdx.x / a.Hv;
  const int h = blockIdx.x - b * a.Hv;
  const int tid = threadIdx.x;
  const int lane = tid & (npn::kWave - 1);
  const int wid = tid >> 6;
  const int T = a.T;
  const int kh = h / (a.Hv / a.Hk);
  const int QKV = (2 * a.Hk + a.Hv) * D;
  const size_t tile = (size_t)D * D;

  // Per token: raw (un-normalised) conv outputs of q and k, which every thread reads in
  // full; v and o, which only their own thread uses, are parked here too so that the
  // 128-row state column is the only large live set (three waves per SIMD).
  __shared__ float s_q[TMAX][D];
  __shared__ float s_k[TMAX][D];
  __shared__ float s_v[TMAX][D];
  __shared__ float s_o[TMAX][D];
  __shared__ float s_rq[TMAX], s_rk[TMAX], s_ro[TMAX];
  __shared__ float s_decay[TMAX];
  __shared__ float s_beta[TMAX];

  // Initial state column (issued first so the loads overlap the prologue).
  const float* S0;
  if (a.state_index != nullptr) {
    int idx = a.state_index[b];
    idx = idx < 0 ? 0 : (idx >= a.state_T ? a.state_T - 1 : idx);
    S0 = a.state + (((size_t)b * a.state_T + idx) * a.Hv + h) * tile;
  } else {
    S0 = a.state + ((size_t)b * a.Hv + h) * tile;
  }
  float S[D];
#pragma unroll
  for (int k = 0; k < D; ++k) S[k] = S0[(size_t)k * D + tid];

  // Conv + SiLU for this thread's q, k (shared k-head) and v channels.
  {
    const uint16_t* xb = a.mixed_qkv + (size_t)b * T * QKV;
    const uint16_t* csb = a.conv_state + (size_t)b * QKV * 3;
    float y[TMAX];
    conv_channel<TMAX>(csb, xb, a.conv_weight, a.conv_bias, kh * D + tid, QKV, T, y);
#pragma unroll
    for (int t = 0; t < TMAX; ++t) s_q[t][tid] = y[t];
    conv_channel<TMAX>(csb, xb, a.conv_weight, a.conv_bias, (a.Hk + kh) * D + tid, QKV, T, y);
#pragma unroll
    for (int t = 0; t < TMAX; ++t) s_k[t][tid] = y[t];
    conv_channel<TMAX>(csb, xb, a.conv_weight, a.conv_bias, (2 * a.Hk + h) * D + tid, QKV, T, y);
#pragma unroll
    for (int t = 0; t < TMAX; ++t) s_v[t][tid] = y[t];
  }

  // Gates for every token (one thread per token).
  if (tid < T) {
    const size_t gi = ((size_t)b * T + tid) * a.Hv + h;
    const float g = -__expf(a.A_log[h]) * npn::softplus(a.a_out[gi] + a.dt_bias[h]);
    s_decay[tid] = __expf(g);
    s_beta[tid] = npn::sigmoid(a.b_out[gi]);
  }
  __syncthreads();

  // L2 norms of q_t and k_t over the 128 channels of the k-head: wave w reduces the tokens
  // t = w, w + 2, ...; the scales multiply the dot products and the update below.
  const float qscale = 0.08838834764831845f;  // 1/sqrt(128)
#pragma unroll
  for (int t = wid; t < TMAX; t += 2) {
    const float q0 = s_q[t][lane], q1 = s_q[t][lane + 64];
    const float k0 = s_k[t][lane], k1 = s_k[t][lane + 64];
    const float sq = npn::wave_sum(q0 * q0 + q1 * q1);
    const float sk = npn::wave_sum(k0 * k0 + k1 * k1);
    if (lane == 0) {
      s_rq[t] = rsqrtf(sq + kEps) * qscale;
      s_rk[t] = rsqrtf(sk + kEps);
    }
  }
  __syncthreads();

  // Recurrence over the T tokens; checkpoint after each. With k = rk * k_raw and
  // q = rq * q_raw: S^T k = rk * (S^T k_raw), S += k_raw (rk * delta), o = rq * (S^T q_raw).
  float* ck = a.ckpt + ((size_t)b * T * a.Hv + h) * tile + tid;
#pragma unroll
  for (int t = 0; t < TMAX; ++t) {
    if (t < T) {
      const float decay = s_decay[t];
      const float rk = s_rk[t];
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < D; ++k) {
        S[k] *= decay;
        acc[k & 3] = fmaf(S[k], s_k[t][k], acc[k & 3]);
      }
      const float kS = ((acc[0] + acc[1]) + (acc[2] + acc[3])) * rk;
      const float kd = (s_v[t][tid] - kS) * s_beta[t] * rk;
      asm volatile("" ::: "memory");
      float oc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < D; ++k) {
        S[k] = fmaf(s_k[t][k], kd, S[k]);
        oc[k & 3] = fmaf(S[k], s_q[t][k], oc[k & 3]);
      }
      s_o[t][tid] = ((oc[0] + oc[1]) + (oc[2] + oc[3])) * s_rq[t];
      asm volatile("" ::: "memory");
      // Nontemporal stores. Plain (write-allocating) stores make this kernel ~11% shorter,
      // but part of the 805 MB then drains from the memory-side cache during the GEMMs
      // that follow, and the whole step is ~1% slower (measured on MI355X).
      float* dst = ck + (size_t)t * a.Hv * tile;
#pragma unroll
      for (int k = 0; k < D; ++k) __builtin_nontemporal_store(S[k], dst + (size_t)k * D);
    }
  }

  // Gated RMSNorm of o_t over the 128 v columns (tokens t < T only: s_o[t] is written for
  // those alone).
  __syncthreads();
#pragma unroll
  for (int t = wid; t < TMAX; t += 2) {
    if (t < T) {
      const float o0 = s_o[t][lane], o1 = s_o[t][lane + 64];
      const float so = npn::wave_sum(o0 * o0 + o1 * o1);
      if (lane == 0) s_ro[t] = rsqrtf(so * (1.0f / D) + kEps);
    }
  }
  __syncthreads();
  const float nw = a.norm_weight[tid];
#pragma unroll
  for (int t = 0; t < TMAX; ++t) {
    if (t < T) {
      const size_t oi = (((size_t)b * T + t) * a.Hv + h) * D + tid;
      const float zz = npn::bf16_to_f32(a.z[oi]);
      a.out[oi] = npn::f32_to_bf16(s_o[t][tid] * s_ro[t] * nw * npn::silu(zz));
    }
  }
}

// conv_out[b][c][0..2] = last 3 columns of [conv_state[b][c][0..2] || x_0..x_a], a = accepted[b]
// (0 when accepted == nullptr: the single-token shift new_cs = conv_in[:, 1:]).
// conv_out may equal conv_state (in-place rollback): each thread owns one channel's three
// entries and loads all of them before it stores.
__global__ void dn_conv_window_kernel(const uint16_t* conv_state,
                                      const uint16_t* __restrict__ x,
                                      const int32_t* __restrict__ accepted,
                                      uint16_t* conv_out, int B, int T, int QKV) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)B * QKV) return;
  const int b = (int)(i / QKV);
  const int c = (int)(i - (size_t)b * QKV);
  int acc = accepted ? accepted[b] : 0;
  acc = acc < 0 ? 0 : (acc >= T ? T - 1 : acc);
  const uint16_t* cs = conv_state + ((size_t)b * QKV + c) * 3;
  uint16_t* dst = conv_out + ((size_t)b * QKV + c) * 3;
  uint16_t v[3];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int p = acc + 1 + j;  // position in [cs0, cs1, cs2, x0, x1, ...]
    v[j] = p < 3 ? cs[p] : x[((size_t)b * T + (p - 3)) * QKV + c];
  }
#pragma unroll
  for (int j = 0; j < 3; ++j) dst[j] = v[j];
}

// state_out[b] = ckpt[b][accepted[b]] (tile-contiguous copy, 16 bytes per thread).
__global__ void dn_state_gather_kernel(const float4* __restrict__ ckpt,
                                       const int32_t* __restrict__ accepted,
                                       float4* __restrict__ state_out, int T,
                                       size_t per_seq4) {
  const int b = blockIdx.y;
  int acc = accepted[b];
  acc = acc < 0 ? 0 : (acc >= T ? T - 1 : acc);
  const float4* src = ckpt + ((size_t)b * T + acc) * per_seq4;
  float4* dst = state_out + (size_t)b * per_seq4;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < per_seq4;
       i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

int check_heads(int k_heads, int v_heads) {
  if (k_heads <= 0 || v_heads <= 0 || v_heads % k_heads != 0 || v_heads > 4096) return NPN_ERR_SHAPE;
  return NPN_OK;
}

template <int TMAX>
void launch_verify(const DnArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(dn_verify_kernel<TMAX>, dim3(a.B * a.Hv), dim3(kThreads), 0, s, a);
}

int verify_impl(const DnArgs& a, hipStream_t s) {
  if (a.T <= 1) launch_verify<1>(a, s);
  else if (a.T <= 4) launch_verify<4>(a, s);
  else if (a.T <= 8) launch_verify<8>(a, s);
  else launch_verify<16>(a, s);
  return npn_launch_status();
}

}  // namespace

extern "C" int npn_deltanet_verify(const float* state, const int32_t* state_index, int state_T,
                                   const uint16_t* mixed_qkv, const uint16_t* conv_state,
                                   const float* conv_weight, const float* conv_bias,
                                   const float* a_out, const float* b_out, const uint16_t* z,
                                   const float* A_log, const float* dt_bias,
                                   const float* norm_weight, float* ckpt, uint16_t* out, int B,
                                   int T, int k_heads, int v_heads, void* stream) {
  NPN_REQUIRE(state && mixed_qkv && conv_state && conv_weight && conv_bias && a_out && b_out &&
                  z && A_log && dt_bias && norm_weight && ckpt && out,
              NPN_ERR_NULL);
  NPN_REQUIRE(B >= 1 && B <= 65536 && T >= 1 && T <= 16, NPN_ERR_SHAPE);
  int st = check_heads(k_heads, v_heads);
  if (st != NPN_OK) return st;
  NPN_REQUIRE(state_index == nullptr || (state_T >= 1 && state_T <= 64), NPN_ERR_SHAPE);
  NPN_REQUIRE(NPN_ALIGNED16(state) && NPN_ALIGNED16(ckpt), NPN_ERR_ALIGN);
  DnArgs a{state, state_index, state_T, mixed_qkv, conv_state, conv_weight, conv_bias,
           a_out,  b_out,       z,       A_log,     dt_bias,    norm_weight, ckpt,
           out,    B,           T,       k_heads,   v_heads};
  return verify_impl(a, static_cast<hipStream_t>(stream));
}

extern "C" int npn_deltanet_full_batched(const float* state, const uint16_t* mixed_qkv,
                                         const uint16_t* conv_state, const float* conv_weight,
                                         const float* conv_bias, const float* a_out,
                                         const float* b_out, const uint16_t* z,
                                         const float* A_log, const float* dt_bias,
                                         const float* norm_weight, float* new_state,
                                         uint16_t* new_conv_state, uint16_t* out, int B,
                                         int k_heads, int v_heads, void* stream) {
  NPN_REQUIRE(new_conv_state != nullptr, NPN_ERR_NULL);
  int st = npn_deltanet_verify(state, nullptr, 0, mixed_qkv, conv_state, conv_weight, conv_bias,
                               a_out, b_out, z, A_log, dt_bias, norm_weight, new_state, out, B,
                               1, k_heads, v_heads, stream);
  if (st != NPN_OK) return st;
  const int QKV = (2 * k_heads + v_heads) * D;
  const size_t n = (size_t)B * QKV;
  hipLaunchKernelGGL(dn_conv_window_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), conv_state, mixed_qkv, nullptr,
                     new_conv_state, B, 1, QKV);
  return npn_launch_status();
}

extern "C" int npn_deltanet_rollback(const float* ckpt, const uint16_t* mixed_qkv,
                                     const uint16_t* conv_state, const int32_t* accepted,
                                     float* state_out, uint16_t* conv_state_out, int B, int T,
                                     int k_heads, int v_heads, void* stream) {
  NPN_REQUIRE(mixed_qkv && conv_state && accepted && conv_state_out, NPN_ERR_NULL);
  NPN_REQUIRE(state_out == nullptr || ckpt != nullptr, NPN_ERR_NULL);
  NPN_REQUIRE(B >= 1 && B <= 65536 && T >= 1 && T <= 16, NPN_ERR_SHAPE);
  int st = check_heads(k_heads, v_heads);
  if (st != NPN_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (state_out != nullptr) {
    NPN_REQUIRE(NPN_ALIGNED16(ckpt) && NPN_ALIGNED16(state_out), NPN_ERR_ALIGN);
    const size_t per_seq4 = (size_t)v_heads * D * D / 4;
    const unsigned gx = (unsigned)((per_seq4 + 1023) / 1024 < 512 ? (per_seq4 + 1023) / 1024 : 512);
    hipLaunchKernelGGL(dn_state_gather_kernel, dim3(gx, B), dim3(256), 0, s,
                       reinterpret_cast<const float4*>(ckpt), accepted,
                       reinterpret_cast<float4*>(state_out), T, per_seq4);
  }
  const int QKV = (2 * k_heads + v_heads) * D;
  const size_t n = (size_t)B * QKV;
  hipLaunchKernelGGL(dn_conv_window_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     conv_state, mixed_qkv, accepted, conv_state_out, B, T, QKV);
  return npn_launch_status();
}
