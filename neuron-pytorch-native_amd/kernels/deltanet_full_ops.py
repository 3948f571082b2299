"""torch.ops.deltanet.full on gfx950 -- drop-in for the op registered at
contrib/qwen3.6-27b/kernels/deltanet_full_ops.py:7-25 (B = 1, unbatched shapes).
It runs the same HIP kernel as deltanet::full_batched with B = 1.
"""
import torch

from npn_native import call, require, stream_of
from deltanet_full_batched_ops import K_DIM, V_DIM, heads_from_shapes


@torch.library.custom_op("deltanet::full", mutates_args=(), device_types="cuda")
def deltanet_full(
    state: torch.Tensor,         # [V_HEADS*K_DIM, V_DIM] f32
    mixed_qkv: torch.Tensor,     # [QKV_DIM] bf16
    conv_state: torch.Tensor,    # [QKV_DIM, 3] bf16
    conv_weight: torch.Tensor,   # [QKV_DIM, 4] f32
    conv_bias: torch.Tensor,     # [QKV_DIM] f32
    a_out: torch.Tensor,         # [V_HEADS] f32
    b_out: torch.Tensor,         # [V_HEADS] f32
    z: torch.Tensor,             # [V_HEADS, V_DIM] bf16
    A_log: torch.Tensor,         # [V_HEADS] f32
    dt_bias: torch.Tensor,       # [V_HEADS] f32
    norm_weight: torch.Tensor,   # [V_DIM] f32
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Returns (new_state, new_conv_state, gated_output[V_HEADS, V_DIM] bf16)."""
    hk, hv = heads_from_shapes(conv_weight.shape[0], A_log.numel())
    qkv = conv_weight.shape[0]
    require(state, "state", torch.float32, shape=(hv * K_DIM, V_DIM))
    require(mixed_qkv, "mixed_qkv", torch.bfloat16, numel=qkv)
    require(conv_state, "conv_state", torch.bfloat16, shape=(qkv, 3))
    require(conv_weight, "conv_weight", torch.float32, shape=(qkv, 4))
    require(conv_bias, "conv_bias", torch.float32, numel=qkv)
    for t, n in ((a_out, "a_out"), (b_out, "b_out"), (A_log, "A_log"), (dt_bias, "dt_bias")):
        require(t, n, torch.float32, numel=hv)
    require(z, "z", torch.bfloat16, numel=hv * V_DIM)
    require(norm_weight, "norm_weight", torch.float32, numel=V_DIM)
    new_state = torch.empty_like(state)
    new_conv = torch.empty_like(conv_state)
    out = torch.empty((hv, V_DIM), dtype=torch.bfloat16, device=state.device)
    call("npn_deltanet_full_batched", state, mixed_qkv, conv_state, conv_weight, conv_bias,
         a_out, b_out, z, A_log, dt_bias, norm_weight, new_state, new_conv, out,
         1, hk, hv, stream_of(state))
    return new_state, new_conv, out


@deltanet_full.register_fake
def _(state, mixed_qkv, conv_state, conv_weight, conv_bias, a_out, b_out, z, A_log,
      dt_bias, norm_weight):
    return (torch.empty_like(state), torch.empty_like(conv_state),
            state.new_empty((A_log.shape[0], V_DIM), dtype=torch.bfloat16))
