"""bf16 bit conversions for the oracle (test infrastructure only).

bf16 tensors are carried as ``uint16`` arrays holding the raw bits, the same
bytes a torch ``bfloat16`` tensor stores. float32 -> bf16 rounds to nearest,
ties to even, which is what ``torch.Tensor.to(torch.bfloat16)`` does (the
reference casts with ``.to(torch.bfloat16)`` throughout, e.g.
``contrib/qwen3.6-27b/static_decode.py:778``).

Pinned by ``tests/test_oracle_numerics.py`` against torch's own bf16 cast on
random, tie, overflow and NaN inputs.
"""
import numpy as np


def bf16_bits_to_f32(bits):
    """uint16 bf16 bits -> float32 (exact)."""
    b = np.asarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16_bits(x):
    """float32 -> uint16 bf16 bits, round to nearest even; NaN stays NaN."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    rounded = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    out = rounded.astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        out = np.where(nan, ((u >> np.uint64(16)).astype(np.uint16) | np.uint16(0x0040)), out)
    return out


def round_to_bf16(x):
    """Round float values to the nearest bf16 and return them as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, dtype=np.float32)))


def silu(x):
    return x / (1.0 + np.exp(-x))


def sigmoid(x):
    return np.exp(-np.logaddexp(0.0, -np.asarray(x, np.float64)))


def softplus(x):
    """torch.nn.functional.softplus with beta=1, threshold=20."""
    x = np.asarray(x, dtype=np.float64)
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))
