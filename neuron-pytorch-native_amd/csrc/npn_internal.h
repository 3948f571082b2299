// Entry points shared between this library's source files, not part of its C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace npn {

// The LM-head GEMM for rejection sampling (fp8_gemm.hip): out [M, N] = bf16((x . w) * scale),
// as npn_fp8_matmul computes it, and in the epilogue the acceptance contract's statistics of
// every output row in 64-column chunks (accept_contract.h): cmax[m][c] = max of the chunk's
// s = out * inv_temp (NaN ignored), csum[m][c] = sum of expfix(s - cmax[m][c]), with
// N / 64 chunks per row. K is never split. fp8_matmul_chunk_stats_ok tells whether the sizes
// are supported (N % 64 == 0 and the npn_fp8_matmul shape rules).
bool fp8_matmul_chunk_stats_ok(int M, int K, int N);
int fp8_matmul_chunk_stats(const uint16_t* x, const int8_t* w, const float* scale, uint16_t* out,
                           float* cmax, uint64_t* csum, float inv_temp, int M, int K, int N,
                           hipStream_t stream);

// Whether the statistics are better computed by a pass over plain logits: true when the plain
// GEMM's plan is the wide kernel without split-K and needs fewer rounds of workgroups than the
// plan with the statistics epilogue (whose column groups must hold whole 64-column chunks,
// 12 of the widest tile's 14 units), or when the epilogue plan is not available.
bool fp8_matmul_stats_pass_cheaper(int M, int K, int N);
// out [M, N] = npn_fp8_matmul's output, for shapes whose plan has no split-K (no workspace);
// NPN_ERR_SHAPE otherwise.
int fp8_matmul_unsplit(const uint16_t* x, const int8_t* w, const float* scale, uint16_t* out,
                       int M, int K, int N, hipStream_t stream);

}  // namespace npn
