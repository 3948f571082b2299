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
// Work decomposition: one workgroup per (b, h) whose waves hold the head's 128 state columns
// split into row parts (the verify kernel below); the workgroup size follows the batch, so
// small batches still stream the states through many waves.
#include "npn_common.h"

namespace {

constexpr int D = 128;
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
  int nsplit;  // workgroups per head, each storing 128 / nsplit of the head's columns
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

// Verify kernel: one workgroup of 128 * P threads per (b, h). Wave w holds state columns
// 64 (w & 1) .. + 63 and rows (w >> 1) * 128 / P .. + 128 / P of them in VGPRs for the whole
// verify block, so a head's state streams through 2 P waves. The column sums S^T k and
// S^T q of each token are added over the P row parts through LDS in part order; each
// checkpoint row is one 256-byte coalesced store per wave; the q / k L2 norms (before the
// loop) and the output RMS norm (after it) are wave reductions over the head's 128 channels.
// The per-token q, k, v and o vectors live in LDS.
// Small batches run nsplit (2 or 4) workgroups per head: each computes the whole head (the
// same operations in the same order, so the same bits) but stores only its 128 / nsplit
// columns of every checkpoint and output row. The checkpoint stores, which a CU issues at a
// limited rate, then spread over nsplit times as many CUs; a head's workgroups are heads
// blocks apart, so with heads % 8 == 0 they share an XCD (and its L2 copy of the state).
template <int TMAX, int P>
__global__ __launch_bounds__(128 * P) void dn_verify_kernel(DnArgs a) {
  constexpr int R = D / P;             // state rows per thread
  constexpr int NT = 128 * P;
  const int heads = a.B * a.Hv;
  const int split = blockIdx.x / heads;
  const int bh = blockIdx.x - split * heads;
  const int b = bh / a.Hv;
  const int h = bh - b * a.Hv;
  const int cspan = D / a.nsplit;
  const int cs0 = split * cspan;        // this workgroup stores columns [cs0, cs0 + cspan)
  const int tid = threadIdx.x;
  const int lane = tid & (npn::kWave - 1);
  const int wid = tid >> 6;
  const int c = (wid & 1) * 64 + lane;   // state column (v index)
  const bool c_mine = c >= cs0 && c < cs0 + cspan;
  const int part = wid >> 1;             // rows part * R .. part * R + R - 1
  const int r0 = part * R;
  const int T = a.T;
  const int kh = h / (a.Hv / a.Hk);
  const int QKV = (2 * a.Hk + a.Hv) * D;
  const size_t tile = (size_t)D * D;

  __shared__ float s_q[TMAX][D];
  __shared__ float s_k[TMAX][D];
  __shared__ float s_v[TMAX][D];
  __shared__ float s_o[TMAX][D];
  __shared__ float s_rq[TMAX], s_rk[TMAX], s_ro[TMAX];
  __shared__ float s_decay[TMAX];
  __shared__ float s_beta[TMAX];
  __shared__ float s_red[2][2][P][D];  // [S^T k | S^T q][token parity][row part][column]

  const float* S0;
  if (a.state_index != nullptr) {
    int idx = a.state_index[b];
    idx = idx < 0 ? 0 : (idx >= a.state_T ? a.state_T - 1 : idx);
    S0 = a.state + (((size_t)b * a.state_T + idx) * a.Hv + h) * tile;
  } else {
    S0 = a.state + ((size_t)b * a.Hv + h) * tile;
  }
  float S[R];
#pragma unroll
  for (int r = 0; r < R; ++r) S[r] = S0[(size_t)(r0 + r) * D + c];

  // Conv + SiLU of the head's q, k and v channels (3 * 128 channels over the workgroup).
  {
    const uint16_t* xb = a.mixed_qkv + (size_t)b * T * QKV;
    const uint16_t* csb = a.conv_state + (size_t)b * QKV * 3;
    for (int ch = tid; ch < 3 * D; ch += NT) {
      const int which = ch / D, i = ch - which * D;
      const int chan = which == 0 ? kh * D + i : (which == 1 ? (a.Hk + kh) * D + i : (2 * a.Hk + h) * D + i);
      float (*dst)[D] = which == 0 ? s_q : (which == 1 ? s_k : s_v);
      float y[TMAX];
      conv_channel<TMAX>(csb, xb, a.conv_weight, a.conv_bias, chan, QKV, T, y);
#pragma unroll
      for (int t = 0; t < TMAX; ++t) dst[t][i] = y[t];
    }
  }
  if (tid < T) {
    const size_t gi = ((size_t)b * T + tid) * a.Hv + h;
    const float g = -__expf(a.A_log[h]) * npn::softplus(a.a_out[gi] + a.dt_bias[h]);
    s_decay[tid] = __expf(g);
    s_beta[tid] = npn::sigmoid(a.b_out[gi]);
  }
  __syncthreads();

  const float qscale = 0.08838834764831845f;  // 1/sqrt(128)
  for (int t = wid; t < TMAX; t += 2 * P) {
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

  // o of token t from its P row-part sums (threads of part 0), in part order
  auto o_reduce = [&](int t) {
    float pr[P];
#pragma unroll
    for (int q = 0; q < P; ++q) pr[q] = s_red[1][t & 1][q][c];
    float o = 0.f;
#pragma unroll
    for (int q = 0; q < P; ++q) o += pr[q];
    s_o[t][c] = o * s_rq[t];
  };
  float* ck = a.ckpt + ((size_t)b * T * a.Hv + h) * tile + (size_t)r0 * D + c;
#pragma unroll
  for (int t = 0; t < TMAX; ++t) {
    if (t < T) {
      const float decay = s_decay[t];
      const float rk = s_rk[t];
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < R; ++r) {
        S[r] *= decay;
        acc[r & 3] = fmaf(S[r], s_k[t][r0 + r], acc[r & 3]);
      }
      s_red[0][t & 1][part][c] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
      // One barrier per token: it publishes token t's S^T k sums and token t - 1's S^T q
      // sums (each kind double-buffered by token parity, so token t + 1 writes the other
      // half while this token's halves are still being read).
      __syncthreads();
      if (t > 0 && part == 0) o_reduce(t - 1);
      float pr[P];
#pragma unroll
      for (int q = 0; q < P; ++q) pr[q] = s_red[0][t & 1][q][c];
      float kS = 0.f;
#pragma unroll
      for (int q = 0; q < P; ++q) kS += pr[q];
      const float kd = (s_v[t][c] - kS * rk) * s_beta[t] * rk;
      float oc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < R; ++r) {
        S[r] = fmaf(s_k[t][r0 + r], kd, S[r]);
        oc[r & 3] = fmaf(S[r], s_q[t][r0 + r], oc[r & 3]);
      }
      s_red[1][t & 1][part][c] = (oc[0] + oc[1]) + (oc[2] + oc[3]);
      // Nontemporal stores: write-allocating ones leave part of the checkpoints to drain from
      // the memory-side cache during the GEMMs that follow (the step measured ~1% slower).
      float* dst = ck + (size_t)t * a.Hv * tile;
      if (c_mine) {
#pragma unroll
        for (int r = 0; r < R; ++r) __builtin_nontemporal_store(S[r], dst + (size_t)r * D);
      }
    }
  }
  __syncthreads();
  if (part == 0) o_reduce(T - 1);

  // Gated RMSNorm of o_t over the 128 v columns (tokens t < T only).
  __syncthreads();
  for (int t = wid; t < TMAX; t += 2 * P) {
    if (t < T) {
      const float o0 = s_o[t][lane], o1 = s_o[t][lane + 64];
      const float so = npn::wave_sum(o0 * o0 + o1 * o1);
      if (lane == 0) s_ro[t] = rsqrtf(so * (1.0f / D) + kEps);
    }
  }
  __syncthreads();
  for (int idx = tid; idx < T * cspan; idx += NT) {
    const int t = idx / cspan, cc = cs0 + (idx - t * cspan);
    const size_t oi = (((size_t)b * T + t) * a.Hv + h) * D + cc;
    const float zz = npn::bf16_to_f32(a.z[oi]);
    a.out[oi] = npn::f32_to_bf16(s_o[t][cc] * s_ro[t] * a.norm_weight[cc] * npn::silu(zz));
  }
}

// conv_out[b][c][0..2] = last 3 columns of [conv_state[b][c][0..2] || x_0..x_a], a = accepted[b]
// (0 when accepted == nullptr: the single-token shift new_cs = conv_in[:, 1:]).
// conv_out may equal conv_state (in-place rollback): each thread owns one channel's three
// entries and loads all of them before it stores.
__device__ __forceinline__ void conv_window_at(const uint16_t* conv_state, const uint16_t* x,
                                               const int32_t* accepted, uint16_t* conv_out,
                                               int T, int QKV, size_t i) {
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

__global__ void dn_conv_window_kernel(const uint16_t* conv_state,
                                      const uint16_t* __restrict__ x,
                                      const int32_t* __restrict__ accepted,
                                      uint16_t* conv_out, int B, int T, int QKV) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)B * QKV) return;
  conv_window_at(conv_state, x, accepted, conv_out, T, QKV, i);
}

// The bookkeeping after acceptance in one launch: every DeltaNet layer's conv window rolled
// back in place (as dn_conv_window_kernel), and, in the last block, the per-sequence commit
// prev_accepted = a, kv_len += a + 1, committed += a + 1 (null pointers skipped), with
// a = accepted clamped into [0, T-1] exactly as the conv windows clamp it, so the windows and
// the KV length always count the same tokens. The two parts touch disjoint memory and only
// read `accepted`.
constexpr int kMaxRollbackLayers = 8;
struct RollbackCommitArgs {
  const uint16_t* mixed[kMaxRollbackLayers];
  uint16_t* conv[kMaxRollbackLayers];
  const int32_t* accepted;
  int32_t* prev_accepted;
  int32_t* kv_len;
  int32_t* committed;
  size_t per_layer;  // B * QKV windows per layer
  unsigned conv_blocks;
  int layers, B, T, QKV;
};

__global__ __launch_bounds__(256) void dn_rollback_commit_kernel(RollbackCommitArgs a) {
  if (blockIdx.x == a.conv_blocks) {
    for (int b = threadIdx.x; b < a.B; b += blockDim.x) {
      int acc = a.accepted[b];
      acc = acc < 0 ? 0 : (acc >= a.T ? a.T - 1 : acc);
      if (a.prev_accepted != nullptr) a.prev_accepted[b] = acc;
      if (a.kv_len != nullptr) a.kv_len[b] += acc + 1;
      if (a.committed != nullptr) a.committed[b] += acc + 1;
    }
    return;
  }
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)a.layers * a.per_layer) return;
  const int l = (int)(i / a.per_layer);
  conv_window_at(a.conv[l], a.mixed[l], a.accepted, a.conv[l], a.T, a.QKV, i - l * a.per_layer);
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

// Row parts per state column, from a sweep on MI355X (16 k / 48 v heads, T = 8, P = 1, 2, 4,
// 8): below 192 heads (B <= 3) eight parts (B = 1: 18.0 us against 31.8 us unsplit), below
// 1536 four (B = 8: 47.0 us against 56.7 us), and two from there (B = 32: 168 us against
// 183 us, 67 % of HBM peak).
int row_parts(int heads) { return heads < 192 ? 8 : (heads < 1536 ? 4 : 2); }

// Workgroups per head: enough that up to 128 heads still occupy about 192 CUs. Measured at
// 16/48 heads, T = 8, B = 1: 17.2 us with one workgroup per head, 15.9 us with four, 28.3 us
// with eight (two workgroups per CU, each computing its whole head).
int col_splits(int heads) { return heads <= 64 ? 4 : (heads <= 128 ? 2 : 1); }

template <int TMAX>
void launch_verify(DnArgs a, hipStream_t s) {
  const int heads = a.B * a.Hv;
  a.nsplit = col_splits(heads);
  const dim3 grid(heads * a.nsplit);
  switch (row_parts(heads)) {
    case 2: hipLaunchKernelGGL((dn_verify_kernel<TMAX, 2>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((dn_verify_kernel<TMAX, 4>), grid, dim3(512), 0, s, a); break;
    default: hipLaunchKernelGGL((dn_verify_kernel<TMAX, 8>), grid, dim3(1024), 0, s, a); break;
  }
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

extern "C" int npn_deltanet_rollback_commit(const uint16_t* const* mixed_qkv,
                                            uint16_t* const* conv_state, int layers,
                                            const int32_t* accepted, int32_t* prev_accepted,
                                            int32_t* kv_len, int32_t* committed, int B, int T,
                                            int k_heads, int v_heads, void* stream) {
  NPN_REQUIRE(accepted != nullptr && (layers == 0 || (mixed_qkv && conv_state)), NPN_ERR_NULL);
  NPN_REQUIRE(layers >= 0 && layers <= kMaxRollbackLayers && B >= 1 && B <= 65536 && T >= 1 &&
                  T <= 16,
              NPN_ERR_SHAPE);
  int st = check_heads(k_heads, v_heads);
  if (st != NPN_OK) return st;
  RollbackCommitArgs a{};
  for (int l = 0; l < layers; ++l) {
    NPN_REQUIRE(mixed_qkv[l] != nullptr && conv_state[l] != nullptr, NPN_ERR_NULL);
    a.mixed[l] = mixed_qkv[l];
    a.conv[l] = conv_state[l];
  }
  a.accepted = accepted;
  a.prev_accepted = prev_accepted;
  a.kv_len = kv_len;
  a.committed = committed;
  a.layers = layers;
  a.B = B;
  a.T = T;
  a.QKV = (2 * k_heads + v_heads) * D;
  a.per_layer = (size_t)B * a.QKV;
  a.conv_blocks = (unsigned)(((size_t)layers * a.per_layer + 255) / 256);
  hipLaunchKernelGGL(dn_rollback_commit_kernel, dim3(a.conv_blocks + 1), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return npn_launch_status();
}
