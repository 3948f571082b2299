"""GPU checks of the fused glue ops against the torch ops they replace
(contrib/qwen3.6-27b/static_decode.py:322-335 rms_norm, :533-542 residual adds,
:951-963 SwiGLU, :802-832 / :867-890 projection slicing).

Bars: slices, casts and the bf16 residual sum are data movement or one IEEE add, so they
are bit-exact. The normalised output and silu(gate) * up may differ from torch by one bf16
ulp where the fp32 sum of squares (different summation order) or exp lands next to a
rounding boundary: at most 1 ulp, on under 1 % of elements.
"""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _ulp_diff(a, b):
    ia = a.contiguous().view(torch.int16).int()
    ib = b.contiguous().view(torch.int16).int()
    return (ia - ib).abs()


def _rms_ref(h, w):
    hf = h.float()
    return ((1.0 + w) * (hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + 1e-6))).to(torch.bfloat16)


@pytest.mark.parametrize("M,H", [(256, 5120), (3, 1024), (1, 5120), (7, 16384)])
def test_residual_rms_norm(ops, M, H):
    g = torch.Generator(device="cuda").manual_seed(M + H)
    hid = (torch.randn(M, H, generator=g, device="cuda") * 3).to(torch.bfloat16)
    delta = torch.randn(M, H, generator=g, device="cuda").to(torch.bfloat16)
    w = torch.randn(H, generator=g, device="cuda") * 0.1
    h2, y = ops.normfuse.residual_rms_norm(hid, delta, w)
    y1 = ops.normfuse.rms_norm(hid, w)
    torch.cuda.synchronize()
    assert torch.equal(h2, hid + delta)
    for got, ref in ((y, _rms_ref(hid + delta, w)), (y1, _rms_ref(hid, w))):
        d = _ulp_diff(got, ref)
        assert d.max().item() <= 1 and (d > 0).float().mean().item() < 0.01


def test_silu_mul(ops):
    g = torch.Generator(device="cuda").manual_seed(5)
    gu = (torch.randn(256, 2 * 17408, generator=g, device="cuda") * 2).to(torch.bfloat16)
    got = ops.glue.silu_mul(gu)
    ref = F.silu(gu[:, :17408]) * gu[:, 17408:]
    torch.cuda.synchronize()
    d = _ulp_diff(got, ref)
    assert d.max().item() <= 1 and (d > 0).float().mean().item() < 0.01


def test_deltanet_split(ops):
    g = torch.Generator(device="cuda").manual_seed(6)
    proj = torch.randn(256, 16512, generator=g, device="cuda").to(torch.bfloat16)
    mixed, z, a, b = ops.glue.deltanet_split(proj, 10240, 6144, 48)
    torch.cuda.synchronize()
    assert torch.equal(mixed, proj[:, :10240])
    assert torch.equal(z, proj[:, 10240:16384])
    assert torch.equal(a, proj[:, 16384:16432].float())
    assert torch.equal(b, proj[:, 16432:16480].float())


@pytest.mark.parametrize("Hq,Hkv,M", [(24, 4, 256), (6, 1, 5)])
def test_gqa_split(ops, Hq, Hkv, M):
    g = torch.Generator(device="cuda").manual_seed(7)
    N = (2 * Hq + 2 * Hkv) * 256
    proj = torch.randn(M, N, generator=g, device="cuda").to(torch.bfloat16)
    q, gt, k, v = ops.glue.gqa_split(proj, Hq, Hkv, 256)
    torch.cuda.synchronize()
    qg = proj[:, :2 * Hq * 256].reshape(M, Hq, 512)
    kv = proj[:, 2 * Hq * 256:].reshape(M, 2, Hkv, 256)
    assert torch.equal(q, qg[..., :256]) and torch.equal(gt, qg[..., 256:])
    assert torch.equal(k, kv[:, 0]) and torch.equal(v, kv[:, 1])


def test_glue_rejects_bad_shapes(ops):
    x = torch.zeros(4, 12, dtype=torch.bfloat16, device="cuda")       # H % 8 != 0
    with pytest.raises(RuntimeError):
        ops.normfuse.rms_norm(x, torch.zeros(12, device="cuda"))
    with pytest.raises(RuntimeError):
        ops.glue.silu_mul(torch.zeros(4, 24, dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(RuntimeError):                                  # row too narrow
        ops.glue.deltanet_split(torch.zeros(2, 64, dtype=torch.bfloat16, device="cuda"), 32, 32, 8)
