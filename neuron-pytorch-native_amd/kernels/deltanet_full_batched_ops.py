"""torch.ops.deltanet.full_batched on gfx950 -- drop-in for the op registered at
contrib/qwen3.6-27b/kernels/deltanet_full_batched_ops.py:22-41 (same name, schema,
layouts and return values).

One decode token for B sequences, batch flattened into dim 0; the weights are shared.
Head counts come from the shapes: Hv = A_log.numel(), QKV = 2*Hk*128 + Hv*128, and
B = state.shape[0] // (Hv*128) (as deltanet_full_batched.py:59-60 derives B).
The HIP kernel is the verify kernel of deltanet_verify_ops with T = 1, followed by
the conv-window shift.
"""
import torch

from npn_native import call, require, stream_of

K_DIM = V_DIM = 128


def heads_from_shapes(qkv_dim, v_heads):
    """(k_heads, v_heads) from QKV = 2*Hk*128 + Hv*128."""
    rest = qkv_dim // K_DIM - v_heads
    if qkv_dim % K_DIM or rest <= 0 or rest % 2 or v_heads % (rest // 2):
        raise RuntimeError(f"cannot derive head counts from QKV={qkv_dim}, Hv={v_heads}")
    return rest // 2, v_heads


@torch.library.custom_op("deltanet::full_batched", mutates_args=(), device_types="cuda")
def deltanet_full_batched(
    state: torch.Tensor,         # [B*V_HEADS*K_DIM, V_DIM] f32
    mixed_qkv: torch.Tensor,     # [B*QKV_DIM] bf16
    conv_state: torch.Tensor,    # [B*QKV_DIM, 3] bf16
    conv_weight: torch.Tensor,   # [QKV_DIM, 4] f32 (shared)
    conv_bias: torch.Tensor,     # [QKV_DIM] f32 (shared)
    a_out: torch.Tensor,         # [B*V_HEADS] f32
    b_out: torch.Tensor,         # [B*V_HEADS] f32
    z: torch.Tensor,             # [B*V_HEADS, V_DIM] bf16
    A_log: torch.Tensor,         # [V_HEADS] f32 (shared)
    dt_bias: torch.Tensor,       # [V_HEADS] f32 (shared)
    norm_weight: torch.Tensor,   # [V_DIM] f32 (shared)
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Returns (new_state[B*V_HEADS*K_DIM,V_DIM] f32, new_conv_state[B*QKV_DIM,3] bf16,
    gated_output[B*V_HEADS, V_DIM] bf16)."""
    hv = A_log.numel()
    qkv = conv_weight.shape[0]
    hk, hv = heads_from_shapes(qkv, hv)
    B = state.shape[0] // (hv * K_DIM)
    require(state, "state", torch.float32, shape=(B * hv * K_DIM, V_DIM))
    require(mixed_qkv, "mixed_qkv", torch.bfloat16, numel=B * qkv)
    require(conv_state, "conv_state", torch.bfloat16, shape=(B * qkv, 3))
    require(conv_weight, "conv_weight", torch.float32, shape=(qkv, 4))
    require(conv_bias, "conv_bias", torch.float32, numel=qkv)
    require(a_out, "a_out", torch.float32, numel=B * hv)
    require(b_out, "b_out", torch.float32, numel=B * hv)
    require(z, "z", torch.bfloat16, numel=B * hv * V_DIM)
    require(A_log, "A_log", torch.float32, numel=hv)
    require(dt_bias, "dt_bias", torch.float32, numel=hv)
    require(norm_weight, "norm_weight", torch.float32, numel=V_DIM)
    new_state = torch.empty_like(state)
    new_conv = torch.empty_like(conv_state)
    out = torch.empty((B * hv, V_DIM), dtype=torch.bfloat16, device=state.device)
    call("npn_deltanet_full_batched", state, mixed_qkv, conv_state, conv_weight, conv_bias,
         a_out, b_out, z, A_log, dt_bias, norm_weight, new_state, new_conv, out,
         B, hk, hv, stream_of(state))
    return new_state, new_conv, out


@deltanet_full_batched.register_fake
def _(state, mixed_qkv, conv_state, conv_weight, conv_bias, a_out, b_out, z, A_log,
      dt_bias, norm_weight):
    B_hv = state.shape[0] // K_DIM
    return (torch.empty_like(state), torch.empty_like(conv_state),
            state.new_empty((B_hv, V_DIM), dtype=torch.bfloat16))
