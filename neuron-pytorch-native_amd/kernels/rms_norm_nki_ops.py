"""torch.ops.normfuse.rms_norm on gfx950 -- drop-in for the op registered at
contrib/qwen3.6-27b/kernels/rms_norm_nki_ops.py:7-13 (same name and schema):

  normfuse::rms_norm(x [..., H] bf16, weight [H] f32) -> [..., H] bf16
      = x * rsqrt(mean(x^2) + 1e-6) * (1 + weight)      (rms_norm, static_decode.py:322-335)

plus the residual form the decode loop applies before every norm
(contrib/qwen3.6-27b/static_decode.py:533-542), fused into the same pass:

  normfuse::residual_rms_norm(hidden, delta, weight, eps) -> (hidden + delta, rms_norm(...))
  normfuse::residual_rms_norm_partials(hidden, partials, scale, weight, eps): the same with
      delta taken from fp8::matmul_partials output (the GEMM reduction fused in)
  normfuse::residual_add_partials(hidden, partials, scale) -> hidden + delta, no norm (the
      residual add that ends the layer stack)

The reference op takes one token's [H] vector; this one takes any number of rows.
"""
import torch

from npn_native import call, require, stream_of

RMS_EPS = 1e-6


def _rows(x):
    H = x.shape[-1]
    return x.numel() // H, H


@torch.library.custom_op("normfuse::rms_norm", mutates_args=(), device_types="cuda")
def rms_norm(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    M, H = _rows(x)
    require(x, "x", torch.bfloat16)
    require(weight, "weight", torch.float32, numel=H)
    out = torch.empty_like(x)
    call("npn_residual_rmsnorm", x, None, weight, None, out, M, H, RMS_EPS, stream_of(x))
    return out


@rms_norm.register_fake
def _(x, weight):
    return torch.empty_like(x)


@torch.library.custom_op("normfuse::residual_rms_norm", mutates_args=(), device_types="cuda")
def residual_rms_norm(hidden: torch.Tensor, delta: torch.Tensor, weight: torch.Tensor,
                      eps: float = RMS_EPS) -> tuple[torch.Tensor, torch.Tensor]:
    """(bf16(hidden + delta), bf16((1 + weight) * h * rsqrt(mean(h^2) + eps))), h = the sum."""
    M, H = _rows(hidden)
    require(hidden, "hidden", torch.bfloat16)
    require(delta, "delta", torch.bfloat16, shape=tuple(hidden.shape))
    require(weight, "weight", torch.float32, numel=H)
    h_out = torch.empty_like(hidden)
    normed = torch.empty_like(hidden)
    call("npn_residual_rmsnorm", hidden, delta, weight, h_out, normed, M, H, float(eps),
         stream_of(hidden))
    return h_out, normed


@residual_rms_norm.register_fake
def _(hidden, delta, weight, eps=RMS_EPS):
    return torch.empty_like(hidden), torch.empty_like(hidden)


@torch.library.custom_op("normfuse::residual_rms_norm_partials", mutates_args=(),
                         device_types="cuda")
def residual_rms_norm_partials(hidden: torch.Tensor, partials: torch.Tensor, scale: torch.Tensor,
                               weight: torch.Tensor,
                               eps: float = RMS_EPS) -> tuple[torch.Tensor, torch.Tensor]:
    """residual_rms_norm with delta = bf16(scale * partials.sum(0)) (summed in order) taken
    from fp8::matmul_partials output [S, M, H]: bit-identical to fp8::matmul followed by
    residual_rms_norm."""
    M, H = _rows(hidden)
    require(hidden, "hidden", torch.bfloat16)
    if partials.dim() != 3 or tuple(partials.shape[1:]) != (M, H):
        raise RuntimeError(f"partials must be [S, {M}, {H}], got {tuple(partials.shape)}")
    require(partials, "partials", torch.float32)
    require(scale, "scale", torch.float32, numel=H)
    require(weight, "weight", torch.float32, numel=H)
    h_out = torch.empty_like(hidden)
    normed = torch.empty_like(hidden)
    call("npn_residual_rmsnorm_partials", hidden, partials, partials.shape[0], scale, weight,
         h_out, normed, M, H, float(eps), stream_of(hidden))
    return h_out, normed


@residual_rms_norm_partials.register_fake
def _(hidden, partials, scale, weight, eps=RMS_EPS):
    return torch.empty_like(hidden), torch.empty_like(hidden)


@torch.library.custom_op("normfuse::residual_add_partials", mutates_args=(), device_types="cuda")
def residual_add_partials(hidden: torch.Tensor, partials: torch.Tensor,
                         scale: torch.Tensor) -> torch.Tensor:
    """hidden + bf16(scale * partials.sum(0)) (summed in order) in bf16, with the partials
    of fp8::matmul_partials [S, M, H]: bit-identical to fp8::matmul followed by a bf16 add.
    The residual add that ends the layer stack (static_decode.py:533-542)."""
    M, H = _rows(hidden)
    require(hidden, "hidden", torch.bfloat16)
    if partials.dim() != 3 or tuple(partials.shape[1:]) != (M, H):
        raise RuntimeError(f"partials must be [S, {M}, {H}], got {tuple(partials.shape)}")
    require(partials, "partials", torch.float32)
    require(scale, "scale", torch.float32, numel=H)
    h_out = torch.empty_like(hidden)
    call("npn_residual_add_partials", hidden, partials, partials.shape[0], scale, h_out, M, H,
         stream_of(hidden))
    return h_out


@residual_add_partials.register_fake
def _(hidden, partials, scale):
    return torch.empty_like(hidden)
