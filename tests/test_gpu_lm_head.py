"""Greedy decision straight from the LM head (fp8::matmul_argmax, spec::accept_greedy_fused):
the reference takes logits.argmax(-1) of the bf16 LM-head output
(contrib/qwen3.6-27b/static_decode.py:546, :1313); here the GEMM reduces each row in its
epilogue and never writes the logits.

Bars:
  - against fp8::matmul + torch.argmax on the GPU (same GEMM accumulation, so the same bf16
    logits): ids and values bit-exact, ties to the lowest column, at the 27B vocabulary
    (N = 248320) through both GEMM kernels (M = 256: rounds of the wide kernel; M = 40);
  - against the oracle (fp64 product, bf16 rounding, first-index argmax) at a small size: the
    chosen logit is within one bf16 ulp of the oracle's maximum, and the ids agree wherever
    the oracle's top two are more than two ulps apart;
  - accept_greedy_fused == accept_greedy over the materialised logits, bit-exact.
"""
import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle.numerics import bf16_bits_to_f32, f32_to_bf16_bits

pytestmark = pytest.mark.gpu


def _gpu_weights(K, N, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn(K, N, generator=g, device="cuda") * 60).clamp(-448, 448)
    w = w.to(torch.float8_e4m3fn).view(torch.int8)
    sc = (torch.rand(N, 1, generator=g, device="cuda") + 0.5) * 1e-3
    return w, sc


@pytest.mark.parametrize("M,K,N", [(256, 5120, 248320), (40, 5120, 248320), (256, 1024, 4096),
                                   (13, 512, 1024)])
def test_matmul_argmax_equals_torch_argmax(ops, M, K, N):
    g = torch.Generator(device="cuda").manual_seed(M + N)
    x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    w, sc = _gpu_weights(K, N, M + K)
    vals, ids = ops.fp8.matmul_argmax(x, w, sc)
    logits = ops.fp8.matmul(x, w, sc).float()
    ref_vals, ref_ids = logits.max(dim=-1)
    torch.cuda.synchronize()
    assert torch.equal(ids, torch.argmax(logits, dim=-1))
    assert torch.equal(ids, ref_ids) and torch.equal(vals, ref_vals)


def test_matmul_argmax_matches_oracle(ops):
    M, K, N = 16, 512, 1024
    rng = np.random.default_rng(3)
    x = rng.standard_normal((M, K)).astype(np.float32)
    xb = f32_to_bf16_bits(x)
    w_bits = f32_to_bf16_bits(rng.standard_normal((N, K)).astype(np.float32) * 0.02)
    wq, sc = ofp8.quantize_fp8_per_channel(w_bits)
    ref = ofp8.fp8_matmul(xb, wq, sc)                       # float64 [M, N], before the cast
    rf = bf16_bits_to_f32(f32_to_bf16_bits(ref.astype(np.float32))).astype(np.float64)
    xt = torch.from_numpy(xb.view(np.int16)).cuda().view(torch.bfloat16)
    wt = torch.from_numpy(np.ascontiguousarray(wq).view(np.int8)).cuda()
    st = torch.from_numpy(np.asarray(sc, np.float32).reshape(N, 1)).cuda()
    vals, ids = ops.fp8.matmul_argmax(xt, wt, st)
    torch.cuda.synchronize()
    ids = ids.cpu().numpy()
    top = np.sort(rf, axis=1)
    for m in range(M):
        mx = top[m, -1]
        ulp = 2.0 ** (np.floor(np.log2(abs(mx))) - 7)
        assert abs(rf[m, ids[m]] - mx) <= ulp, m
        if top[m, -1] - top[m, -2] > 2 * ulp:
            assert ids[m] == int(np.argmax(rf[m])), m


def test_accept_greedy_fused(ops):
    B, K, H, V = 8, 7, 5120, 248320
    T = K + 1
    g = torch.Generator(device="cuda").manual_seed(9)
    hid = torch.randn(B * T, H, generator=g, device="cuda").to(torch.bfloat16)
    w, sc = _gpu_weights(H, V, 10)
    logits = ops.fp8.matmul(hid, w, sc).float().view(B, T, V)
    best = logits.argmax(-1)
    drafts = best[:, :K].clone()
    # sequence b keeps its first b drafts right, then goes wrong (b = K: all right)
    for b in range(B):
        if b < K:
            drafts[b, b] = (drafts[b, b] + 1) % V
    acc_f, ids_f = ops.spec.accept_greedy_fused(hid, w, sc, drafts)
    acc_r, ids_r = ops.spec.accept_greedy(logits.contiguous(), drafts)
    torch.cuda.synchronize()
    assert torch.equal(acc_f, acc_r) and torch.equal(ids_f, ids_r)
    assert acc_f.tolist() == [min(b, K) for b in range(B)]
