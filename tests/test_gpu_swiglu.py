"""The MLP's gate/up projection with the SwiGLU applied in the FP8 GEMM's epilogue
(fp8::matmul_swiglu) against fp8::matmul followed by glue::silu_mul
(contrib/qwen3.6-27b/static_decode.py:951-963: y = bf16(bf16(silu(gate)) * up)).

Bar: bit-exact. The epilogue forms g and u as the GEMM's own bf16 outputs and applies the
glue kernel's rounding, so every output must be identical. Shapes: the verify step's
gate/up projection (M = 256, K = 5120, N = 2 * 17408; 128-row workgroups of 9 gate units),
partial row blocks (M = 65, 100, 130, 200, 300, 320) and N = 2 * 13312 on the fused path; shapes whose
fp8::matmul plan splits K or is not the wide kernel (the GEMM writes [g | u] to the workspace
and the glue kernel runs). A whole verify step at M = 128 with and
without the fusion is bit-identical too.
"""
import pytest
import torch

from _util import fp8_weights

pytestmark = pytest.mark.gpu


def _inputs(M, K, N, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    w, sc = fp8_weights(N, K, seed)
    return x, w.cuda(), sc.reshape(N, 1).cuda()


def _bits(t):
    return t.contiguous().view(torch.int16)


@pytest.mark.parametrize("M,K,N,fused", [
    (256, 5120, 34816, True), (100, 1024, 34816, True), (200, 2048, 26624, True),
    (65, 640, 34816, True), (130, 512, 25600, True), (300, 512, 30720, True),
    (320, 1024, 34816, True), (100, 1024, 4096, False), (48, 1024, 2048, False),
    (8, 5120, 34816, False), (64, 2048, 34816, False), (8, 5120, 4096, False),
    (16, 256, 1024, False)])
def test_swiglu_fused_equals_unfused(ops, M, K, N, fused):
    """Fused shapes run the SwiGLU epilogue of the 128-row wide kernel (9, 5, 7 and 12 gate
    units per workgroup at M <= 300) or of the 256-row kernel (M = 320, two row passes); on
    unsplit plans the result is also compared with the 256-row kernel's GEMM
    (npn_fp8_matmul_rowmax) + the glue SwiGLU. Unfused shapes take the GEMM's partials
    through one reduce + SwiGLU kernel when the plan splits K (stream-K at N = 34816,
    split 16 at M = 8, N = 4096) and the plain GEMM + glue SwiGLU when it does not
    (K = 256)."""
    from npn_native import call, query, stream_of
    # which path the shape takes: the fused epilogue needs no workspace
    assert (query("npn_fp8_matmul_swiglu_workspace_size", M, K, N) == 0) == fused
    x, w, sc = _inputs(M, K, N, seed=M + N)
    out = torch.ops.fp8.matmul_swiglu(x, w, sc)
    ref = torch.ops.glue.silu_mul(torch.ops.fp8.matmul(x, w, sc))
    torch.cuda.synchronize()
    assert out.shape == (M, N // 2)
    assert torch.equal(_bits(out), _bits(ref))
    if fused:
        G = query("npn_fp8_matmul_argmax_groups", M, K, N)
        gu = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        gmax = torch.empty((M, G), dtype=torch.float32, device="cuda")
        call("npn_fp8_matmul_rowmax", x, w, sc, gu, gmax, M, K, N, stream_of(x))
        ref256 = torch.ops.glue.silu_mul(gu)
        torch.cuda.synchronize()
        assert torch.equal(_bits(out), _bits(ref256))


def test_swiglu_rejects_bad_shape(ops):
    x, w, sc = _inputs(128, 512, 192, seed=1)  # N % 128 != 0
    with pytest.raises(RuntimeError):
        torch.ops.fp8.matmul_swiglu(x, w, sc)


def test_step_swiglu_fused_equals_unfused(ops):
    from spec_verify_step import HIDDEN, VerifySlice, synthetic_logits
    B, K = 16, 7
    kv = [37 + 23 * i for i in range(B)]
    models = [VerifySlice(B, K, kv, 600, pattern="DG", seed=9, device="cuda", fuse_swiglu=f)
              for f in (True, False)]
    g = torch.Generator(device="cuda").manual_seed(4)
    x = torch.randn(B * (K + 1), HIDDEN, generator=g, device="cuda").to(torch.bfloat16)
    logits = synthetic_logits(B, K, 1000, 6, "cuda")
    outs = [m.step(x, *logits) for m in models]
    torch.cuda.synchronize()
    (h0, a0, i0), (h1, a1, i1) = outs
    assert torch.equal(_bits(h0), _bits(h1))
    assert torch.equal(a0, a1) and torch.equal(i0, i1)
