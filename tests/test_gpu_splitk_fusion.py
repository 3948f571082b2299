"""The split-K reduction of the FP8 GEMM fused into the glue ops that consume its output
(fp8::matmul_partials + normfuse::residual_rms_norm_partials / residual_add_partials /
glue::*_split_partials)
against fp8::matmul followed by the bf16 forms of the same ops.

Bar: bit-exact. The fused ops compute bf16(scale * (p_0 + ... + p_{S-1})) in the order of the
GEMM's own reduction, so every output must be identical. The partials themselves are pinned
by the same sum, formed in torch in that order, reproducing fp8::matmul bit for bit (also
for a shape the plan does not split, S = 1). Shapes are the verify step's projections at
M = B*T = 256: down (S = 8), out/o (S = 4), DeltaNet in (S = 2), GQA q/k/v (S = 2).
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


def _reduce_in_order(p, sc):
    acc = torch.zeros_like(p[0])
    for s in range(p.shape[0]):
        acc = acc + p[s]
    return (acc * sc.reshape(1, -1)).to(torch.bfloat16)


@pytest.mark.parametrize("M,K,N,S", [(256, 17408, 5120, 8), (256, 6144, 5120, 4),
                                     (256, 5120, 16512, 2), (256, 5120, 14336, 2),
                                     (256, 5120, 34816, 1), (8, 17408, 5120, 16),
                                     (64, 5120, 34816, 5)])
def test_partials_reduce_to_matmul(ops, M, K, N, S):
    x, w, sc = _inputs(M, K, N, K + N)
    p = ops.fp8.matmul_partials(x, w)
    ref = ops.fp8.matmul(x, w, sc)
    torch.cuda.synchronize()
    assert p.shape == (S, M, N) and p.dtype == torch.float32
    assert torch.equal(_bits(_reduce_in_order(p, sc)), _bits(ref))


@pytest.mark.parametrize("M,K", [(256, 17408), (256, 6144), (8, 17408), (13, 6144)])
def test_residual_rms_norm_partials(ops, M, K):
    """M = 8 and 13 run the narrow plan's split 16 (two batches of partial loads)."""
    H = 5120
    x, w, sc = _inputs(M, K, H, K)
    g = torch.Generator(device="cuda").manual_seed(7)
    hid = (torch.randn(M, H, generator=g, device="cuda") * 2).to(torch.bfloat16)
    nw = torch.randn(H, generator=g, device="cuda") * 0.1
    p = ops.fp8.matmul_partials(x, w)
    h_f, n_f = ops.normfuse.residual_rms_norm_partials(hid, p, sc, nw)
    h_r, n_r = ops.normfuse.residual_rms_norm(hid, ops.fp8.matmul(x, w, sc), nw)
    torch.cuda.synchronize()
    assert p.shape[0] > 1
    assert torch.equal(_bits(h_f), _bits(h_r))
    assert torch.equal(_bits(n_f), _bits(n_r))


@pytest.mark.parametrize("M,K", [(256, 17408), (256, 6144), (8, 17408), (13, 6144)])
def test_residual_add_partials(ops, M, K):
    """The stack's last residual add from the down-projection's partials equals fp8::matmul
    followed by a bf16 add."""
    H = 5120
    x, w, sc = _inputs(M, K, H, K + 1)
    g = torch.Generator(device="cuda").manual_seed(9)
    hid = (torch.randn(M, H, generator=g, device="cuda") * 2).to(torch.bfloat16)
    p = ops.fp8.matmul_partials(x, w)
    got = ops.normfuse.residual_add_partials(hid, p, sc)
    ref = hid + ops.fp8.matmul(x, w, sc)
    torch.cuda.synchronize()
    assert torch.equal(_bits(got), _bits(ref))


def test_deltanet_split_partials(ops):
    M, K, N = 256, 5120, 16512
    x, w, sc = _inputs(M, K, N, 11)
    p = ops.fp8.matmul_partials(x, w)
    fused = ops.glue.deltanet_split_partials(p, sc, 10240, 6144, 48)
    ref = ops.glue.deltanet_split(ops.fp8.matmul(x, w, sc), 10240, 6144, 48)
    torch.cuda.synchronize()
    assert p.shape[0] > 1
    for f, r in zip(fused, ref):
        assert f.dtype == r.dtype and f.shape == r.shape
        assert torch.equal(f.view(torch.int16) if f.dtype == torch.bfloat16 else f,
                           r.view(torch.int16) if r.dtype == torch.bfloat16 else r)


def test_gqa_split_partials(ops):
    M, K, N = 256, 5120, 14336
    x, w, sc = _inputs(M, K, N, 12)
    p = ops.fp8.matmul_partials(x, w)
    fused = ops.glue.gqa_split_partials(p, sc, 24, 4, 256)
    ref = ops.glue.gqa_split(ops.fp8.matmul(x, w, sc), 24, 4, 256)
    torch.cuda.synchronize()
    assert p.shape[0] > 1
    for f, r in zip(fused, ref):
        assert torch.equal(_bits(f), _bits(r))


def test_step_fused_equals_unfused(ops):
    """A whole verify step with the split-K reductions fused into their consumers and the KV
    append + RoPE rows fused into the attention's launches is bit-identical to one with
    neither."""
    from spec_verify_step import HIDDEN, VerifySlice, synthetic_logits
    kv = [37, 300, 5, 129]
    B, K = 4, 7
    models = [VerifySlice(B, K, kv, 400, pattern="DG", seed=5, device="cuda", fuse_splitk=f,
                          fuse_launches=f)
              for f in (True, False)]
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(B * (K + 1), HIDDEN, generator=g, device="cuda").to(torch.bfloat16)
    logits = synthetic_logits(B, K, 1000, 4, "cuda")
    outs = [m.step(x, *logits) for m in models]
    torch.cuda.synchronize()
    (h0, a0, i0), (h1, a1, i1) = outs
    assert torch.equal(_bits(h0), _bits(h1))
    assert torch.equal(a0, a1) and torch.equal(i0, i1)
