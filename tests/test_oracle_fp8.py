"""CPU pinning of oracle/fp8.py.

- the e4m3fn known-answer table of contrib/qwen3.6-35b-a3b/kernels/tests/
  test_moe_w8_cpu.py:99-107 (incl. the OCP-only codes 0x78..0x7E and NaN at 0x7F);
- all 256 codes and round-to-nearest-even encoding against torch.float8_e4m3fn;
- the per-channel quantiser against the reference's quantize_fp8_per_channel steps
  (contrib/qwen3.6-27b/static_decode.py:283-304) written with torch ops;
- the matmul against an fp64 torch matmul of torch-dequantised weights, and against the
  reference kernel test's cpu_ref (contrib/qwen3.6-27b/kernels/tests/test_fp8_matmul.py:25-36,
  seed 0, FP8_MAX 240) within that test's own bar (max abs < 0.5).
"""
import numpy as np
import torch

from oracle import fp8 as of
from oracle.numerics import bf16_bits_to_f32
from _util import bits


def test_known_answers():
    raw = np.array([0x00, 0x01, 0x07, 0x08, 0x38, 0x77, 0x78, 0x7E, 0xB8], np.uint8)
    exp = np.array([0.0, 2.0 ** -9, 7 * 2.0 ** -9, 2.0 ** -6, 1.0, 240.0, 256.0, 448.0, -1.0])
    assert np.array_equal(of.decode_e4m3fn(raw).astype(np.float64), exp)
    assert np.isnan(of.decode_e4m3fn(np.array([0x7F, 0xFF], np.uint8))).all()


def test_all_codes_match_torch():
    codes = torch.arange(256, dtype=torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).float().numpy()
    got = of.decode_e4m3fn(codes.numpy())
    both_nan = np.isnan(ref) & np.isnan(got)
    assert np.array_equal(got[~both_nan], ref[~both_nan]) and (np.isnan(ref) == np.isnan(got)).all()


def test_encode_matches_torch_cast():
    rng = np.random.default_rng(0)
    vals = np.concatenate([rng.standard_normal(20000) * 50, rng.standard_normal(2000) * 0.01,
                           of.DECODE_LUT[:0x7F].astype(np.float64),            # exact codes
                           (of.DECODE_LUT[1:0x7F] + of.DECODE_LUT[:0x7E]) / 2])  # ties
    vals = np.clip(vals, -448, 448).astype(np.float32)
    ref = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(of.encode_e4m3fn(vals), ref)


def test_quantizer_matches_reference_steps():
    g = torch.Generator().manual_seed(0)
    w = (torch.randn(96, 256, generator=g) * 0.05).to(torch.bfloat16)
    for fp8_max in (240.0, 448.0):
        absmax = w.abs().amax(dim=-1).float().clamp_min(1e-12)
        scale = absmax / fp8_max
        inv = (1.0 / scale).to(torch.bfloat16).unsqueeze(-1)
        wq = (w * inv).clamp(-fp8_max, fp8_max).to(torch.float8_e4m3fn)
        ref_q = wq.t().contiguous().view(torch.int8).numpy()
        got_q, got_s = of.quantize_fp8_per_channel(bits(w), fp8_max=fp8_max)
        assert np.array_equal(got_s, scale.numpy())
        assert np.array_equal(got_q, ref_q)


def test_matmul_against_fp64_torch():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(13, 512, generator=g).to(torch.bfloat16)
    wq = (torch.randn(512, 384, generator=g) * 40).clamp(-448, 448).to(torch.float8_e4m3fn)
    scale = torch.rand(384, generator=g) * 0.01
    ref = (x.double() @ wq.double()) * scale.double()
    got = of.fp8_matmul(bits(x), wq.view(torch.int8).numpy(), scale.numpy())
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-12, atol=1e-12)


def test_close_to_reference_cpu_ref_seed0():
    """contrib/qwen3.6-27b/kernels/tests/test_fp8_matmul.py run_case(1, 5120, 4352) inputs;
    the reference dequantises to bf16 before the matmul, the kernel scales the fp32 sum."""
    torch.manual_seed(0)
    B, K, N = 1, 5120, 4352
    x = torch.randn(B, K, dtype=torch.bfloat16) * 0.5
    w = torch.randn(N, K, dtype=torch.bfloat16) * 0.05
    absmax = w.abs().amax(dim=-1).float().clamp_min(1e-12)
    scale = absmax / 240.0
    inv = (1.0 / scale).to(w.dtype).unsqueeze(-1)
    w_q = (w * inv).clamp(-240.0, 240.0).to(torch.float8_e4m3fn)
    cpu_ref = torch.nn.functional.linear(x, w_q.to(x.dtype) * scale.to(x.dtype).unsqueeze(-1))
    got = of.fp8_matmul(bits(x), w_q.t().contiguous().view(torch.int8).numpy(), scale.numpy())
    got_bf16 = bf16_bits_to_f32(bits(torch.from_numpy(got.astype(np.float32)).to(torch.bfloat16)))
    assert np.abs(got_bf16 - cpu_ref.float().numpy()).max() < 0.5
