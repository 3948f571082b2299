"""FP8 (OCP e4m3fn) W8A16 matmul oracle (test infrastructure only).

Restates, in numpy:
- e4m3fn decode from the bit layout, ``decode_e4m3fn``
  (``contrib/qwen3.6-35b-a3b/moe_w8.py:26-50``): exponent 15 is finite up to 448,
  only exponent=15/mantissa=7 is NaN;
- round-to-nearest-even encode to e4m3fn (what ``tensor.to(torch.float8_e4m3fn)``
  does for in-range values), used by the per-channel quantiser;
- ``quantize_fp8_per_channel`` (``contrib/qwen3.6-27b/static_decode.py:283-304``):
  scale = absmax_row / FP8_MAX; Wq = clamp(W * bf16(1/scale), +-FP8_MAX) -> e4m3fn,
  pre-transposed to [K, N] bytes. FP8_MAX is an argument: 240 in the reference
  (static_decode.py:280), 448 for the full OCP range;
- ``fp8::matmul`` (``contrib/qwen3.6-27b/kernels/fp8_matmul_ops.py:14-21``) as the
  kernel computes it (``contrib/qwen3.6-27b/kernels/fp8_matmul.py:143-169``):
  fp32 accumulation of x[M,K] . decode(Wq)[K,N], then * scale[N], then bf16.
  (The reference's cpu_ref, ``kernels/tests/test_fp8_matmul.py:33-36``, rounds the
  dequantised weight to bf16 first; the kernel does not, and this oracle follows
  the kernel. e4m3 -> bf16 is exact, so the two differ only by where the scale
  is rounded.)

Pinning (tests/test_oracle_fp8.py): the e4m3fn known-answer table of
``contrib/qwen3.6-35b-a3b/kernels/tests/test_moe_w8_cpu.py:99-107``; all 256 codes
against torch.float8_e4m3fn; encode against torch's cast on random and tie values;
the matmul against an fp64 torch matmul of torch-dequantised weights.
"""
import numpy as np

from .numerics import bf16_bits_to_f32, f32_to_bf16_bits


def decode_e4m3fn(raw):
    """uint8/int8 e4m3fn bytes -> float32 (NaN for 0x7F/0xFF)."""
    bits = np.asarray(raw).astype(np.uint8).astype(np.int32)
    sign = (bits >> 7) & 1
    exponent = (bits >> 3) & 0x0F
    mantissa = bits & 0x07
    sub = mantissa.astype(np.float64) * 2.0 ** -9
    nrm = (1.0 + mantissa / 8.0) * np.exp2(exponent.astype(np.float64) - 7.0)
    v = np.where(exponent == 0, sub, nrm)
    v = np.where((exponent == 15) & (mantissa == 7), np.nan, v)
    return np.where(sign == 1, -v, v).astype(np.float32)


_POS_CODES = np.arange(0x7F, dtype=np.uint8)                      # 0x00..0x7E, all finite
_POS_VALUES = decode_e4m3fn(_POS_CODES).astype(np.float64)


def encode_e4m3fn(x):
    """float -> e4m3fn bytes (uint8), round to nearest, ties to even code, sign kept on
    values that round to zero; values beyond 448 saturate to +-448 (callers clamp first,
    as the reference does)."""
    x = np.asarray(x, np.float64)
    a = np.minimum(np.abs(x), 448.0)
    idx = np.searchsorted(_POS_VALUES, a)                          # first value >= a
    idx = np.clip(idx, 1, len(_POS_VALUES) - 1)
    lo, hi = _POS_VALUES[idx - 1], _POS_VALUES[idx]
    pick_hi = (a - lo > hi - a) | ((a - lo == hi - a) & ((idx % 2) == 0))
    code = np.where(pick_hi, idx, idx - 1).astype(np.uint8)
    code = np.where(a == 0.0, 0, code).astype(np.uint8)
    return np.where(np.signbit(x), code | 0x80, code).astype(np.uint8)   # -0 stays -0 (0x80)


def quantize_fp8_per_channel(w_bits, fp8_max=448.0):
    """w [N, K] bf16 bits -> (wq [K, N] int8 bytes, scale [N] float32)
    (static_decode.py:283-304)."""
    w = bf16_bits_to_f32(w_bits)
    absmax = np.maximum(np.abs(w).max(axis=-1).astype(np.float32), np.float32(1e-12))
    scale = (absmax / np.float32(fp8_max)).astype(np.float32)
    inv_bf = bf16_bits_to_f32(f32_to_bf16_bits((np.float32(1.0) / scale).astype(np.float32)))
    prod = bf16_bits_to_f32(f32_to_bf16_bits((w * inv_bf[:, None]).astype(np.float32)))
    q = encode_e4m3fn(np.clip(prod, -fp8_max, fp8_max))
    return np.ascontiguousarray(q.T).view(np.int8), scale


# All 256 codes decoded once by decode_e4m3fn; large weights are decoded by table lookup.
DECODE_LUT = decode_e4m3fn(np.arange(256, dtype=np.uint8))


def fp8_matmul(x_bits, w_i8, scale):
    """x [M, K] bf16 bits, w [K, N] e4m3fn bytes, scale [N] (or [N,1]) f32 ->
    float64 [M, N] = (x . decode(w)) * scale, before the bf16 cast."""
    x = bf16_bits_to_f32(x_bits).astype(np.float64)
    w = DECODE_LUT[np.asarray(w_i8).view(np.uint8)].astype(np.float64)
    return (x @ w) * np.asarray(scale, np.float64).reshape(1, -1)
