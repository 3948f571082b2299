/*
 * npn_spec_verify.h -- C ABI of the MI355X (gfx950) EAGLE3 verify-and-accept library.
 *
 * Shared library: neuron-pytorch-native_amd/libnpn_spec_verify.so
 *
 * Conventions (all entry points):
 *  - Plain device pointers, element counts and a HIP stream passed as void*
 *    (NULL = the default stream). No torch types cross this boundary.
 *  - bf16 tensors are passed as uint16_t* holding the raw bf16 bits; fp8 weights
 *    as int8_t* holding OCP e4m3fn bytes.
 *  - Outputs and workspaces are allocated by the caller; the library never
 *    allocates device memory. Pointers must be 16-byte aligned.
 *  - Every call validates shapes and pointers on the host, enqueues its kernels
 *    on `stream` and returns an npn_status. No call synchronises the stream.
 *  - Head dimension of the DeltaNet state is 128 (k and v); GQA head dim is 256
 *    with a 64-dim partial RoPE, as in the reference models.
 *  - Calls are re-entrant; concurrent calls on different streams must use
 *    different workspaces.
 */
#ifndef NPN_SPEC_VERIFY_H
#define NPN_SPEC_VERIFY_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum npn_status {
  NPN_OK = 0,
  NPN_ERR_NULL = 1,        /* a required pointer is NULL */
  NPN_ERR_SHAPE = 2,       /* a size is out of the supported range or inconsistent */
  NPN_ERR_ALIGN = 3,       /* a pointer is not 16-byte aligned */
  NPN_ERR_WORKSPACE = 4,   /* workspace missing or smaller than the size query returned */
  NPN_ERR_LAUNCH = 5,      /* the HIP runtime rejected a kernel launch */
  NPN_ERR_VALUE = 6,       /* an argument value is out of range (e.g. temperature) */
  NPN_ERR_SCRATCH = 7      /* the problem needs more than a no-allocation entry point's
                              fixed scratch */
} npn_status;

/* Human-readable text for a status code (static storage). */
const char* npn_status_string(int status);

/* Library ABI version (major*100 + minor). */
int npn_abi_version(void);

/* ---------------------------------------------------------------------------
 * Gated DeltaNet.
 * Shapes: QKV = 2*Hk*128 + Hv*128; Hv % Hk == 0.
 * ------------------------------------------------------------------------- */

/* torch.ops.deltanet.full_batched -- replaces the op registered at
 * contrib/qwen3.6-27b/kernels/deltanet_full_batched_ops.py:22-41 (and, with B=1,
 * deltanet::full at contrib/qwen3.6-27b/kernels/deltanet_full_ops.py:7-25).
 * One decode token per sequence:
 *   state       [B*Hv*128, 128] f32     mixed_qkv [B*QKV] bf16
 *   conv_state  [B*QKV, 3] bf16         conv_weight [QKV, 4] f32, conv_bias [QKV] f32
 *   a_out,b_out [B*Hv] f32              z [B*Hv, 128] bf16
 *   A_log, dt_bias [Hv] f32             norm_weight [128] f32
 * Outputs: new_state [B*Hv*128,128] f32, new_conv_state [B*QKV,3] bf16,
 *          out [B*Hv,128] bf16. */
int npn_deltanet_full_batched(const float* state, const uint16_t* mixed_qkv,
                              const uint16_t* conv_state, const float* conv_weight,
                              const float* conv_bias, const float* a_out, const float* b_out,
                              const uint16_t* z, const float* A_log, const float* dt_bias,
                              const float* norm_weight, float* new_state,
                              uint16_t* new_conv_state, uint16_t* out, int B, int k_heads,
                              int v_heads, void* stream);

/* torch.ops.deltanet.full_fp8 -- replaces the op registered at
 * contrib/qwen3.6-27b/kernels/deltanet_full_fp8_ops.py:7-32 (kernel deltanet_full_fp8.py;
 * called by the decode harness at B = 1 with fp8 weights, static_decode.py:784-797): the four
 * fp8 W8A16 in-projections of one decode token folded into deltanet::full.
 *   x [hidden] bf16 (one token of one sequence)
 *   qkv_w [hidden, QKV], z_w [hidden, Hv*128], a_w, b_w [hidden, Hv]: e4m3fn bytes, [K, N]
 *   qkv_s [QKV], z_s [Hv*128], a_s, b_s [Hv]: f32 per-output-channel scales
 *   mixed_qkv = bf16((x . qkv_w) * qkv_s), z = bf16((x . z_w) * z_s),
 *   a_out = (x . a_w) * a_s, b_out = (x . b_w) * b_s in f32 (not rounded), fp32 accumulation;
 * then the token step of npn_deltanet_full_batched with B = 1 (same state, conv and parameter
 * arguments, same outputs; new_conv_state must not overlap conv_state). mixed_qkv and z are
 * bit-identical to npn_fp8_matmul's outputs. hidden % 64 == 0; workspace of
 * npn_deltanet_full_fp8_workspace_size(hidden, k_heads, v_heads) bytes (0: unsupported sizes),
 * 16-byte aligned. Three launches: the qkv and z GEMMs (split-K partials, one launch where
 * their plans agree), one kernel that reduces them, shifts the conv window and computes a_out
 * and b_out, then the token step. */
size_t npn_deltanet_full_fp8_workspace_size(int hidden, int k_heads, int v_heads);
int npn_deltanet_full_fp8(const uint16_t* x, const float* state, const uint16_t* conv_state,
                          const float* conv_weight, const float* conv_bias, const float* A_log,
                          const float* dt_bias, const float* norm_weight, const int8_t* qkv_w,
                          const float* qkv_s, const int8_t* z_w, const float* z_s,
                          const int8_t* a_w, const float* a_s, const int8_t* b_w,
                          const float* b_s, float* new_state, uint16_t* new_conv_state,
                          uint16_t* out, int hidden, int k_heads, int v_heads, void* workspace,
                          size_t workspace_bytes, void* stream);

/* torch.ops.deltanet.verify_batched -- new op (no reference counterpart; it runs
 * the token step of deltanet_full_batched_ops.py:22-41 over T = K+1 verify
 * tokens and keeps every intermediate state, the trajectory of
 * contrib/qwen3.6-27b/kernels/tests/test_spec_verify_tensor_ops.py:47-51).
 *   state        initial state. If state_index == NULL: [B, Hv, 128, 128] f32.
 *                Otherwise a checkpoint buffer [B, state_T, Hv, 128, 128] and the
 *                initial state of sequence b is checkpoint state_index[b]
 *                (index-based rollback of the previous verify step, no copy).
 *   mixed_qkv    [B, T, QKV] bf16   conv_state [B, QKV, 3] bf16
 *   a_out, b_out [B, T, Hv] f32     z [B, T, Hv, 128] bf16
 * Outputs: ckpt [B, T, Hv, 128, 128] f32 (state after each token),
 *          out  [B, T, Hv, 128] bf16 (gated RMSNorm output per token).
 * 1 <= T <= 16. */
int npn_deltanet_verify(const float* state, const int32_t* state_index, int state_T,
                        const uint16_t* mixed_qkv, const uint16_t* conv_state,
                        const float* conv_weight, const float* conv_bias, const float* a_out,
                        const float* b_out, const uint16_t* z, const float* A_log,
                        const float* dt_bias, const float* norm_weight, float* ckpt,
                        uint16_t* out, int B, int T, int k_heads, int v_heads, void* stream);

/* torch.ops.deltanet.rollback -- new op: roll back to the accepted prefix
 * (contrib/qwen3.6-27b/kernels/tests/test_deltanet_spec_verify_rollback.py:64-68).
 *   accepted [B] int32 in [0, T-1] (number of accepted drafts).
 *   state_out [B, Hv, 128, 128] f32 = ckpt[b, accepted[b]] (may be NULL to skip
 *   the copy when the next verify uses state_index instead);
 *   conv_state_out [B, QKV, 3] bf16 = last 3 columns of [conv_state || x_0..x_a]
 *   (conv_state_out may equal conv_state: the rollback then happens in place).
 * Out-of-range accepted values are clamped into [0, T-1] on the device. */
int npn_deltanet_rollback(const float* ckpt, const uint16_t* mixed_qkv,
                          const uint16_t* conv_state, const int32_t* accepted,
                          float* state_out, uint16_t* conv_state_out, int B, int T,
                          int k_heads, int v_heads, void* stream);

/* torch.ops.deltanet.chunked_prefill -- replaces the op registered at
 * contrib/qwen3.6-27b/kernels/deltanet_chunked_ops.py:26-42 (kernel
 * deltanet_chunked_v2.py:46-105): the gated delta rule over a whole prompt of one
 * sequence, in chunks. Rows are head-major (row h*S + t):
 *   state [Hv*128, 128] f32; query, key [Hv*S, 128] f32 raw (L2-normalised inside as
 *   x * rsqrt(sum x^2 + 1e-6), q also scaled by 1/sqrt(128)); value [Hv*S, 128] f32;
 *   g, beta [Hv*S] f32 (log decay and update gate per token and head).
 * Outputs: out [Hv*S, 128] f32 (the raw attention output, before the gated norm),
 * new_state [Hv*128, 128] f32. Any S >= 1 (the reference kernel needs S % C == 0; a
 * last partial chunk is handled as zero-gate padding here). The workspace holds the
 * state-independent part of every chunk (T, the intra-chunk attention and the per-token
 * scales), npn_deltanet_chunked_workspace_size bytes (about 33 KiB per head and 64 tokens);
 * two kernels run on the stream. Sizes: 1 <= v_heads <= 65535, v_heads * S <= 2^26. */
size_t npn_deltanet_chunked_workspace_size(int v_heads, int S);
int npn_deltanet_chunked_prefill(const float* state, const float* query, const float* key,
                                 const float* value, const float* g, const float* beta,
                                 float* out, float* new_state, int v_heads, int S,
                                 void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * GQA attention tail. Head dim 256, partial RoPE on dims [0, 64).
 * ------------------------------------------------------------------------- */

/* torch.ops.gqa.tail -- replaces the op registered at
 * contrib/qwen3.6-27b/kernels/gqa_tail_ops.py:14-26 (one kv head per call):
 *   query, gate [B*Hq, 256] f32   q_norm [256] f32   cos, sin [64] f32
 *   cached_k, cached_v [B*S, 256] f32   mask [S] f32 (1 valid / 0 masked)
 * Output: out [B*Hq, 256] f32 = softmax(q'k/16 + (mask-1)*1e9) V * sigmoid(gate). */
int npn_gqa_tail(const float* query, const float* gate, const float* q_norm, const float* cos,
                 const float* sin, const float* cached_k, const float* cached_v,
                 const float* mask, float* out, int B, int q_heads, int S, void* stream);

/* Workspace bytes for npn_gqa_tail_verify with these sizes. */
size_t npn_gqa_tail_verify_workspace_size(int B, int T, int q_heads, int kv_heads, int s_max);

/* torch.ops.gqa.tail_verify -- new op: the gqa::tail math (gqa_tail_ops.py:14-26)
 * for T verify tokens per sequence over a bf16 KV cache (split-KV: the
 * sequences' 32-key steps are divided evenly over a fixed set of workgroups,
 * then a log-sum-exp merge).
 *   query, gate [B, T, Hq, 256] bf16   q_norm [256] f32
 *   cos, sin    [B, T, 64] f32 (RoPE of each query row's position)
 *   cache_k/v   [B, Hkv, s_max, 256] bf16, rows [0, kv_len[b]+T) valid
 *   kv_len      [B] int32, cache rows before the T verify rows (kv_len+T <= s_max)
 * Row (b,t,h) uses kv head h/(Hq/Hkv) and attends rows [0, kv_len[b]+t].
 * Output: out [B, T, Hq, 256] bf16. Limits: Hq/Hkv * T <= 48, s_max <= 2^23,
 * B * Hkv <= 65535. The workspace query returns 0 outside them. gate, out, the
 * caches and the workspace must be 16-byte aligned. */
int npn_gqa_tail_verify(const uint16_t* query, const uint16_t* gate, const float* q_norm,
                        const float* cos, const float* sin, const uint16_t* cache_k,
                        const uint16_t* cache_v, const int32_t* kv_len, uint16_t* out, int B,
                        int T, int q_heads, int kv_heads, int s_max, void* workspace,
                        size_t workspace_bytes, void* stream);

/* torch.ops.gqa.kv_append -- new op: the k-side glue of _gqa_layer
 * (contrib/qwen3.6-27b/static_decode.py:880-910) for T rows per sequence:
 * cache_k[b, g, kv_len[b]+t] = bf16(rope(bf16(rms_norm_1p(key[b,t,g], k_norm))));
 * cache_v[b, g, kv_len[b]+t] = value[b,t,g].
 *   key, value [B, T, Hkv, 256] bf16; k_norm [256] f32; cos, sin [B, T, 64] f32. */
int npn_gqa_kv_append(const uint16_t* key, const uint16_t* value, const float* k_norm,
                      const float* cos, const float* sin, uint16_t* cache_k, uint16_t* cache_v,
                      const int32_t* kv_len, int B, int T, int kv_heads, int s_max,
                      void* stream);

/* torch.ops.gqa.tail_verify_append -- new op: the whole k-side and attention of
 * _gqa_layer (contrib/qwen3.6-27b/static_decode.py:880-931) in the verify tail's
 * launches: npn_gqa_kv_append followed by npn_gqa_tail_verify, with the RoPE rows read
 * from the position tables (the reference's _init_rope, static_decode.py:489-502) at
 * row kv_len[b] + t clamped to [0, positions) -- the rows npn_rope_rows gathers. The
 * append runs in the query-prep launch, so this is two launches fewer than
 * npn_rope_rows + npn_gqa_kv_append + npn_gqa_tail_verify, whose results (out and the
 * appended cache rows) it equals bit for bit.
 *   key, value [B, T, Hkv, 256] bf16; k_norm [256] f32;
 *   cos_table, sin_table [positions, 64] f32 (16-byte aligned);
 *   other arguments, limits and workspace (npn_gqa_tail_verify_workspace_size) as
 *   npn_gqa_tail_verify; cache_k/v are written at rows kv_len[b]+t < s_max. */
int npn_gqa_tail_verify_append(const uint16_t* query, const uint16_t* gate, const uint16_t* key,
                               const uint16_t* value, const float* q_norm, const float* k_norm,
                               const float* cos_table, const float* sin_table, int positions,
                               uint16_t* cache_k, uint16_t* cache_v, const int32_t* kv_len,
                               uint16_t* out, int B, int T, int q_heads, int kv_heads, int s_max,
                               void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * FP8 W8A16 GEMM.
 * ------------------------------------------------------------------------- */

/* Workspace bytes for npn_fp8_matmul with these sizes (0 if none is needed). */
size_t npn_fp8_matmul_workspace_size(int M, int K, int N);

/* torch.ops.fp8.matmul -- replaces the op registered at
 * contrib/qwen3.6-27b/kernels/fp8_matmul_ops.py:14-21:
 *   x [M, K] bf16, w [K, N] e4m3fn bytes (pre-transposed), scale [N] f32
 *   out [M, N] bf16 = bf16((x . w) * scale), fp32 accumulation.
 * K % 64 == 0, N % 64 == 0, 1 <= M <= 4096 (the reference caps M at 128,
 * fp8_matmul.py:74). */
int npn_fp8_matmul(const uint16_t* x, const int8_t* w, const float* scale, uint16_t* out, int M,
                   int K, int N, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes for npn_fp8_matmul_swiglu (0 when the SwiGLU is fused into the GEMM
 * epilogue and nothing is needed). */
size_t npn_fp8_matmul_swiglu_workspace_size(int M, int K, int N);

/* torch.ops.fp8.matmul_swiglu -- new op: the MLP's gate/up projection and SwiGLU
 * (contrib/qwen3.6-27b/static_decode.py:951-963) in one call.
 *   w [K, N] = [gate | up] along N (N % 128 == 0), scale [N];
 *   out [M, N/2] bf16 = bf16(bf16(silu(g)) * u), [g | u] = bf16((x . w) * scale),
 * bit-identical to npn_fp8_matmul followed by npn_silu_mul. Shapes whose npn_fp8_matmul
 * plan is the wide kernel without split-K (64 < M, wide N) apply the SwiGLU in its epilogue
 * and never write [g | u]; others write [g | u] to the workspace. */
int npn_fp8_matmul_swiglu(const uint16_t* x, const int8_t* w, const float* scale, uint16_t* out,
                          int M, int K, int N, void* workspace, size_t workspace_bytes,
                          void* stream);

/* Row argmax of npn_fp8_matmul's output without writing it (an LM head's greedy decision,
 * the reference takes logits.argmax(-1) of the bf16 LM-head output,
 * contrib/qwen3.6-27b/static_decode.py:546, :1313). New op torch.ops.fp8.matmul_argmax.
 * Writes parts [M][G] of {float value; int32 column}: per row and column group, the largest
 * bf16((x . w) * scale) value and its column (NaN counts as the maximum; ties go to the lower
 * column), G = npn_fp8_matmul_argmax_groups(M, K, N). npn_argmax_parts reduces them to ids,
 * npn_accept_greedy_parts to a greedy acceptance. Shape rules as npn_fp8_matmul. */
int npn_fp8_matmul_argmax_groups(int M, int K, int N);
int npn_fp8_matmul_argmax(const uint16_t* x, const int8_t* w, const float* scale, void* parts,
                          int M, int K, int N, void* stream);

/* New op, no reference counterpart: out [M, N] bf16 = bf16((x . w) * scale) as
 * npn_fp8_matmul, and gmax [M][G] f32 = per row and column group (the groups of
 * npn_fp8_matmul_argmax, G = npn_fp8_matmul_argmax_groups(M, K, N)) the largest of the row's
 * bf16 outputs in the group, NaN ignored (-inf if the group has none). The plan never splits
 * K; out is bit-identical to npn_fp8_matmul's wherever that plan does not split either (the
 * vocabulary-wide N of an LM head). Shape rules as npn_fp8_matmul. */
int npn_fp8_matmul_rowmax(const uint16_t* x, const int8_t* w, const float* scale, uint16_t* out,
                          float* gmax, int M, int K, int N, void* stream);

/* Split-K factor S of the GEMM plan for these sizes (1: no split; 0: unsupported sizes). */
int npn_fp8_matmul_split_k(int M, int K, int N);

/* The GEMM plan for these sizes, host-only (no device work), for tests and tuning -- no
 * reference counterpart. info[4] receives: kind (0 narrow kernel on a tiles x split grid,
 * 1 narrow kernel in stream-K, 2 wide kernel on 256-row tiles, 3 wide kernel on 128-row
 * tiles), the split-K factor (stream-K: partial slots), the tile parameter (narrow: 16-row
 * blocks per tile; kind 2: 16-column tiles per wave; kind 3: 16-column units per workgroup)
 * and the workgroups launched. NPN_ERR_SHAPE for unsupported sizes. */
int npn_fp8_matmul_plan(int M, int K, int N, int* info);

/* torch.ops.fp8.matmul_partials -- new op, no reference counterpart: the GEMM of
 * npn_fp8_matmul without its reduction and scaling, for consumers that fuse them.
 *   partial [S][M][N] f32, S = npn_fp8_matmul_split_k(M, K, N): the unscaled products of x
 *   and w over S consecutive K ranges. npn_fp8_matmul's output is
 *   bf16(scale * (partial[0] + ... + partial[S-1])), summed from 0 in that order.
 * Shape rules as npn_fp8_matmul; no workspace. */
int npn_fp8_matmul_partials(const uint16_t* x, const int8_t* w, float* partial, int M, int K,
                            int N, void* stream);

/* ---------------------------------------------------------------------------
 * Acceptance. T = K+1 verify positions per sequence, vocabulary V.
 * Outputs: accepted [B] int32 in [0, K]; out_ids [B, T] int64: accepted drafts,
 * then the correction/bonus token, then -1.
 * Draft ids outside [0, V) are never accepted, by every acceptance call: greedy compares
 * them with an argmax, which is always in range, and rejection sampling counts such a
 * position as a rejection whatever its uniform and samples its token from the residual as
 * for any rejection. So every emitted id lies in [0, V), and no logit is read at an
 * out-of-range id (the device code makes no host round trip to check them).
 * ------------------------------------------------------------------------- */

/* Workspace bytes for the acceptance calls. */
size_t npn_accept_workspace_size(int B, int K, int V);

/* torch.ops.spec.accept_greedy -- new op. Greedy verify of the reference's
 * on-device argmax (contrib/qwen3.6-27b/static_decode.py:1313): first-index
 * tie-break, NaN counts as the maximum.
 *   target_logits [B, K+1, V] f32, draft_ids [B, K] int64. */
int npn_accept_greedy(const float* target_logits, const int64_t* draft_ids, int32_t* accepted,
                      int64_t* out_ids, int B, int K, int V, void* workspace,
                      size_t workspace_bytes, void* stream);

/* torch.ops.spec.accept_rejection -- new op. Rejection sampling (Leviathan et
 * al. 2023, Alg. 1) under an integer softmax contract, so the result is
 * bit-identical to a CPU restatement for the same logits and uniforms, and every
 * sum comes from one pass over the logits:
 *   s_v = t_v*inv_temperature (fp32); the vocabulary is cut into chunks of 64
 *   and blocks of 8192; m_c = max of chunk c's non-NaN s_v, M_b = max of block b's
 *   m_c, M = max_b M_b; E_v = floor(2^31 * exp_c(s_v - m_c)), F_c = floor(2^31 *
 *   exp_c(m_c - M_b)), G_b = floor(2^31 * exp_c(M_b - M)) with exp_c a fixed fp32
 *   Cody-Waite + degree-7 Taylor evaluation in fused multiply-adds; the weight of v
 *   is W_v = E_v * F_c * G_b and Z = sum_v W_v (exact integers, Z <= 2^113);
 *   U = floor(u * 2^24). Accept draft x iff U * Wq_x * Zp <= 2^24 * Wp_x * Zq. At
 *   the first rejection sample from R_v = max(0, Wp_v*Zq - Wq_v*Zp) (bonus: R_v =
 *   Wp_v of row K): the smallest v with 2^24 * sum_{w<=v} R_w > U_s * sum_w R_w
 *   (exact to 2^256).
 *   A row with no finite entry relative to its maximum (all NaN or -inf, or a +inf
 *   entry) has Z = 0 and passes the accept test; if the sampling row has no mass (a
 *   bonus row, or the residual after an out-of-range draft id where Wp*Zq == Wq*Zp
 *   everywhere) the token is the target row's argmax (NaN counts as the maximum, ties
 *   go to the lowest index).
 *   target_logits [B, K+1, V] f32, draft_logits [B, K, V] f32, draft_ids [B, K]
 *   int64, u_accept [B, K] f32 in [0,1), u_sample [B] f32 in [0,1),
 *   inv_temperature > 0 (logits are multiplied by it), V <= 2^20.
 * Three launches: the one pass over the logits (every row's block maxima M_b and sums S_b,
 * and the draft token's E*F; the chunk statistics stay on chip), the residual (or bonus) mass
 * per 64 and per 2048 entries of each sequence's sampling rows (each workgroup first works
 * the row totals and the decision out from the block statistics), and the inverse CDF (one
 * workgroup per sequence).
 * On return the workspace starts with every row's Z (unsigned 128-bit, low 64-bit word
 * first [R]) and, at byte offset 16R rounded up to a multiple of 256, every row's max
 * scaled logit M (float [R]); R = B*(2K+1) rows: target row (b, i) at b*(K+1)+i, then
 * draft row (b, i) at B*(K+1) + b*K + i. */
int npn_accept_rejection(const float* target_logits, const float* draft_logits,
                         const int64_t* draft_ids, const float* u_accept,
                         const float* u_sample, float inv_temperature, int32_t* accepted,
                         int64_t* out_ids, int B, int K, int V, void* workspace,
                         size_t workspace_bytes, void* stream);

/* Bytes of the fixed per-GPU scratch behind npn_accept_rejection_noalloc (4 MiB). */
#define NPN_ACCEPT_SCRATCH_BYTES (4u << 20)

/* npn_accept_rejection without a workspace argument and without any allocation. No
 * counterpart in the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The workspace
 * is a fixed device array of NPN_ACCEPT_SCRATCH_BYTES per GPU, held from the first call on
 * that GPU until the process ends; problems whose npn_accept_workspace_size(B, K, V) exceeds
 * it return NPN_ERR_SCRATCH (B = 32, K = 7, V = 151936 needs 2.6 MiB). Every call on a GPU
 * uses that GPU's one array, so calls that overlap on one GPU (concurrent streams, or
 * threads) race and must be serialised by the caller; each call writes every scratch word it
 * reads before reading it, so nothing needs clearing between calls. The stream's device
 * (the current device for the null stream) selects the array. The first call on a device
 * looks the array's address up (hipGetSymbolAddress); make it outside stream capture, after
 * which a call only enqueues kernels and may be captured in a HIP graph. Results are bit-identical to
 * npn_accept_rejection; the scratch is not readable through this interface. */
int npn_accept_rejection_noalloc(const float* target_logits, const float* draft_logits,
                                 const int64_t* draft_ids, const float* u_accept,
                                 const float* u_sample, float inv_temperature,
                                 int32_t* accepted, int64_t* out_ids, int B, int K, int V,
                                 void* stream);

/* ids [M] int64 (and values [M] f32 if non-NULL) = the best of each row's nparts partials,
 * in column order, under the same rule. */
int npn_argmax_parts(const void* parts, int nparts, int64_t* ids, float* values, int M,
                     void* stream);

/* torch.ops.spec.accept_greedy_fused -- new op: npn_accept_greedy with the target argmax taken
 * from npn_fp8_matmul_argmax partials of the LM head over the B*(K+1) verify rows (row
 * b*(K+1) + t), so no logits are written or read. Same outputs and rules as npn_accept_greedy;
 * K + 1 <= 16. */
int npn_accept_greedy_parts(const void* parts, int nparts, const int64_t* draft_ids,
                            int32_t* accepted, int64_t* out_ids, int B, int K, void* stream);

/* torch.ops.spec.accept_rejection_lm_head -- new op: npn_accept_rejection with the target
 * logits produced by the LM head in the same call. hidden [B*(K+1), H] bf16 (the final-normed
 * verify rows, row b*(K+1) + t), lm_head_w [H, V] e4m3fn bytes, lm_head_scale [V] f32:
 * target_logits [B*(K+1), V] bf16 is written (= npn_fp8_matmul's out). The contract's chunk
 * statistics of the target rows come from the GEMM's epilogue where that costs the GEMM no
 * extra round of workgroups (then the logit pass covers only the draft rows and the sampling
 * kernel re-reads only each sequence's sampling row), else from one pass over the bf16 target
 * rows with the draft rows (at B*(K+1) = 256 with a 248320-entry vocabulary the epilogue's
 * chunk-aligned column groups would need a sixth round). accepted / out_ids equal
 * npn_accept_rejection's on the fp32 cast of target_logits, bit for bit, with the same
 * draft logits, ids, uniforms and inv_temperature (> 0). V % 64 == 0, H % 64 == 0, the other
 * rules as npn_accept_rejection. Workspace: npn_accept_rejection_lm_head_workspace_size
 * (0: unsupported sizes); it starts with the rows' Z and M as npn_accept_rejection's does. */
size_t npn_accept_rejection_lm_head_workspace_size(int B, int K, int H, int V);
int npn_accept_rejection_lm_head(const uint16_t* hidden, const int8_t* lm_head_w,
                                 const float* lm_head_scale, const float* draft_logits,
                                 const int64_t* draft_ids, const float* u_accept,
                                 const float* u_sample, float inv_temperature,
                                 uint16_t* target_logits, int32_t* accepted, int64_t* out_ids,
                                 int B, int K, int H, int V, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Inter-layer glue of the verify step (the decode loop of
 * contrib/qwen3.6-27b/static_decode.py:533-542), each a single pass.
 * ------------------------------------------------------------------------- */

/* torch.ops.normfuse.rms_norm -- replaces the op registered at
 * contrib/qwen3.6-27b/kernels/rms_norm_nki_ops.py:7-13 (rms_norm,
 * static_decode.py:322-335) and fuses the residual add before it
 * (normfuse::residual_rms_norm, new):
 *   hidden_out = bf16(hidden_in + delta)            (skipped when delta == NULL)
 *   normed     = bf16((1 + weight) * h * rsqrt(mean(h^2) + eps)), h = hidden_out
 *   hidden_in/out, delta, normed [M, H] bf16; weight [H] f32. H % 8 == 0, H <= 16384.
 *   hidden_out may equal hidden_in; with delta == NULL it may be NULL. */
int npn_residual_rmsnorm(const uint16_t* hidden_in, const uint16_t* delta, const float* weight,
                         uint16_t* hidden_out, uint16_t* normed, int M, int H, float eps,
                         void* stream);

/* torch.ops.glue.silu_mul -- new op: the SwiGLU of _mlp_layer (static_decode.py:951-963),
 * out = bf16(bf16(silu(gate)) * up) for gate_up [M, 2I] bf16 = [gate | up]; out [M, I].
 * I % 8 == 0. */
int npn_silu_mul(const uint16_t* gate_up, uint16_t* out, int M, int I, void* stream);

/* torch.ops.glue.deltanet_split -- new op: the slicing and casts of _deltanet_layer
 * (static_decode.py:802-832) from one fused in-projection output:
 *   proj [M, ld] bf16 rows [qkv_n | z_n | hv (a) | hv (b) | unused]
 *   -> mixed_qkv [M, qkv_n] bf16, z [M, z_n] bf16, a_out, b_out [M, hv] f32.
 * qkv_n, z_n, hv, ld multiples of 8. */
int npn_deltanet_split(const uint16_t* proj, int ld, uint16_t* mixed_qkv, uint16_t* z,
                       float* a_out, float* b_out, int M, int qkv_n, int z_n, int hv,
                       void* stream);

/* torch.ops.glue.gqa_split -- new op: the per-head split of _gqa_layer
 * (static_decode.py:867-870, :880-890) from one fused q/k/v projection output:
 *   proj [M, ld] bf16 rows [(query | gate) x q_heads | key x kv_heads | value x kv_heads],
 *   each head_dim wide -> query, gate [M, q_heads, head_dim], key, value
 *   [M, kv_heads, head_dim] bf16. head_dim, ld multiples of 8. */
int npn_gqa_split(const uint16_t* proj, int ld, uint16_t* query, uint16_t* gate, uint16_t* key,
                  uint16_t* value, int M, int q_heads, int kv_heads, int head_dim, void* stream);

/* The same three glue ops reading their input from npn_fp8_matmul_partials output instead
 * of a bf16 projection (new ops: normfuse::residual_rms_norm_partials,
 * glue::deltanet_split_partials, glue::gqa_split_partials). Input row m is
 *   bf16(scale[n] * (partial[0][m][n] + ... + partial[split_k-1][m][n])),
 * bit-identical to npn_fp8_matmul's output, so each result equals npn_fp8_matmul followed by
 * the bf16 op. partial [split_k][M][ld] f32 (ld = H for the norm), scale [ld] f32,
 * 1 <= split_k <= 16; other arguments as in the bf16 forms. */
int npn_residual_rmsnorm_partials(const uint16_t* hidden_in, const float* partial, int split_k,
                                  const float* scale, const float* weight, uint16_t* hidden_out,
                                  uint16_t* normed, int M, int H, float eps, void* stream);
/* torch.ops.normfuse.residual_add_partials -- new op: the residual add that ends the
 * layer stack (static_decode.py:533-542, the last layer's hidden += mlp(normed)) with the
 * MLP's down-projection taken as split-K partials: hidden_out = bf16(hidden_in + delta),
 * delta as above, equal to npn_fp8_matmul followed by a bf16 add. hidden_out may alias
 * hidden_in. */
int npn_residual_add_partials(const uint16_t* hidden_in, const float* partial, int split_k,
                              const float* scale, uint16_t* hidden_out, int M, int H,
                              void* stream);
int npn_deltanet_split_partials(const float* partial, int split_k, const float* scale, int ld,
                                uint16_t* mixed_qkv, uint16_t* z, float* a_out, float* b_out,
                                int M, int qkv_n, int z_n, int hv, void* stream);
int npn_gqa_split_partials(const float* partial, int split_k, const float* scale, int ld,
                           uint16_t* query, uint16_t* gate, uint16_t* key, uint16_t* value,
                           int M, int q_heads, int kv_heads, int head_dim, void* stream);

/* torch.ops.gqa.rope_rows -- new op: the RoPE rows of the T verify positions,
 *   cos_out, sin_out [B, T, dim] f32 = table[kv_len[b] + t] for cos_table, sin_table
 *   [positions, dim] f32 built once, as the reference indexes its _init_rope table
 *   (static_decode.py:489-502). Positions past the table are clamped to its last row.
 *   dim % 4 == 0. */
int npn_rope_rows(const float* cos_table, const float* sin_table, int positions,
                  const int32_t* kv_len, float* cos_out, float* sin_out, int B, int T, int dim,
                  void* stream);

/* torch.ops.spec.commit_ -- new op: the bookkeeping after acceptance, in place, for
 * decode state kept at fixed addresses (HIP-graph replay):
 *   prev_accepted[b] = accepted[b]; kv_len[b] += accepted[b] + 1;
 *   committed[b] += accepted[b] + 1. Any of the three outputs may be NULL. */
int npn_spec_commit(const int32_t* accepted, int32_t* prev_accepted, int32_t* kv_len,
                    int32_t* committed, int B, void* stream);

/* torch.ops.deltanet.rollback_commit_ -- new op: the whole bookkeeping after acceptance in
 * one launch, for decode state at fixed addresses: every DeltaNet layer's conv window rolled
 * back in place (npn_deltanet_rollback with conv_state_out == conv_state and no state copy)
 * and npn_spec_commit. Same results as those calls; 1 launch instead of layers + 1.
 *   mixed_qkv, conv_state: host arrays of `layers` (0..8) device pointers, layer l's
 *   [B, T, QKV] bf16 verify inputs and its [B, QKV, 3] bf16 window (rolled back in place);
 *   accepted [B] int32; prev_accepted, kv_len, committed [B] int32 (each may be NULL).
 *   An accepted value outside [0, T-1] is clamped into it, on the device, for every output
 *   alike (windows, prev_accepted, kv_len, committed), so the conv windows and the KV length
 *   always count the same tokens; npn_spec_commit alone adds accepted as given. */
int npn_deltanet_rollback_commit(const uint16_t* const* mixed_qkv, uint16_t* const* conv_state,
                                 int layers, const int32_t* accepted, int32_t* prev_accepted,
                                 int32_t* kv_len, int32_t* committed, int B, int T, int k_heads,
                                 int v_heads, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NPN_SPEC_VERIFY_H */
