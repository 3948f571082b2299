"""torch.ops.deltanet.full_fp8 on gfx950 -- drop-in for the op registered at
contrib/qwen3.6-27b/kernels/deltanet_full_fp8_ops.py:7-32 (same name, schema and return
values). The decode harness calls it for one sequence with fp8 weights
(contrib/qwen3.6-27b/static_decode.py:784-797): the four in-projections of one decode token
(in_proj_qkv, in_proj_z, in_proj_a, in_proj_b; W8A16, weights [HIDDEN, N] e4m3fn bytes with
per-output-channel scales) folded into deltanet::full.

As in the reference kernel (contrib/qwen3.6-27b/kernels/deltanet_full_fp8.py):
  mixed_qkv = bf16((x . qkv_w) * qkv_s)   rounded to bf16 before the conv  (:147-203)
  z         = bf16((x . z_w) * z_s)                                          (:232-277)
  a_out, b_out = (x . a_w) * a_s, (x . b_w) * b_s in float32, NOT rounded   (:280-337)
then the token step of deltanet::full. (The harness's bf16 path, static_decode.py:802-805,
rounds a_out and b_out to bf16 instead; the two differ by that rounding.)

One C call (npn_deltanet_full_fp8) launches the fp8 GEMMs for mixed_qkv and z, a thin fp32
projection kernel for a_out and b_out, and the DeltaNet token step; the intermediates live in
a workspace allocated here. Head counts come from the shapes: Hv = A_log.numel(),
QKV = qkv_w.shape[1] = 2*Hk*128 + Hv*128, HIDDEN = x.numel().
"""
import torch

from npn_native import call, query, require, stream_of
from deltanet_full_batched_ops import K_DIM, V_DIM, heads_from_shapes

_FP8_BYTES = (torch.int8, torch.uint8, torch.float8_e4m3fn)


def _require_fp8(t, name, shape):
    if t.dtype not in _FP8_BYTES:
        raise TypeError(f"{name} must hold fp8 bytes, got {t.dtype}")
    require(t, name, t.dtype, shape=shape)


@torch.library.custom_op("deltanet::full_fp8", mutates_args=(), device_types="cuda")
def deltanet_full_fp8(
    x: torch.Tensor,             # [1, HIDDEN] bf16
    state: torch.Tensor,         # [V_HEADS*K_DIM, V_DIM] f32
    conv_state: torch.Tensor,    # [QKV_DIM, 3] bf16
    conv_weight: torch.Tensor,   # [QKV_DIM, 4] f32
    conv_bias: torch.Tensor,     # [QKV_DIM] f32
    A_log: torch.Tensor,         # [V_HEADS] f32
    dt_bias: torch.Tensor,       # [V_HEADS] f32
    norm_weight: torch.Tensor,   # [V_DIM] f32
    qkv_w_T_i8: torch.Tensor,    # [HIDDEN, QKV_DIM] int8 (fp8 bytes)
    qkv_s: torch.Tensor,         # [QKV_DIM, 1] f32
    z_w_T_i8: torch.Tensor,      # [HIDDEN, Z_DIM] int8
    z_s: torch.Tensor,           # [Z_DIM, 1] f32
    a_w_T_i8: torch.Tensor,      # [HIDDEN, V_HEADS] int8
    a_s: torch.Tensor,           # [V_HEADS, 1] f32
    b_w_T_i8: torch.Tensor,      # [HIDDEN, V_HEADS] int8
    b_s: torch.Tensor,           # [V_HEADS, 1] f32
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Returns (new_state, new_conv_state, gated_output[V_HEADS, V_DIM] bf16)."""
    hv = A_log.numel()
    hidden = x.numel()
    qkv = qkv_w_T_i8.shape[1] if qkv_w_T_i8.dim() == 2 else -1
    hk, hv = heads_from_shapes(qkv, hv)
    require(x, "x", torch.bfloat16, numel=hidden)
    if x.dim() != 2 or x.shape[0] != 1:
        raise RuntimeError(f"x must be [1, HIDDEN] (one token of one sequence), got {tuple(x.shape)}")
    require(state, "state", torch.float32, shape=(hv * K_DIM, V_DIM))
    require(conv_state, "conv_state", torch.bfloat16, shape=(qkv, 3))
    require(conv_weight, "conv_weight", torch.float32, shape=(qkv, 4))
    require(conv_bias, "conv_bias", torch.float32, numel=qkv)
    for t, n in ((A_log, "A_log"), (dt_bias, "dt_bias")):
        require(t, n, torch.float32, numel=hv)
    require(norm_weight, "norm_weight", torch.float32, numel=V_DIM)
    for w, s, n, name in ((qkv_w_T_i8, qkv_s, qkv, "qkv"), (z_w_T_i8, z_s, hv * V_DIM, "z"),
                          (a_w_T_i8, a_s, hv, "a"), (b_w_T_i8, b_s, hv, "b")):
        _require_fp8(w, f"{name}_w_T_i8", (hidden, n))
        require(s, f"{name}_s", torch.float32, numel=n)
    n_ws = query("npn_deltanet_full_fp8_workspace_size", hidden, hk, hv)
    if n_ws == 0:
        raise RuntimeError(f"unsupported deltanet::full_fp8 sizes HIDDEN={hidden} (a multiple "
                           f"of 64 is required), Hk={hk}, Hv={hv}")
    ws = torch.empty(n_ws, dtype=torch.uint8, device=x.device)
    new_state = torch.empty_like(state)
    new_conv = torch.empty_like(conv_state)
    out = torch.empty((hv, V_DIM), dtype=torch.bfloat16, device=x.device)
    call("npn_deltanet_full_fp8", x, state, conv_state, conv_weight, conv_bias, A_log, dt_bias,
         norm_weight, qkv_w_T_i8, qkv_s, z_w_T_i8, z_s, a_w_T_i8, a_s, b_w_T_i8, b_s,
         new_state, new_conv, out, hidden, hk, hv, ws, n_ws, stream_of(x))
    return new_state, new_conv, out


@deltanet_full_fp8.register_fake
def _(x, state, conv_state, conv_weight, conv_bias, A_log, dt_bias, norm_weight, qkv_w_T_i8,
      qkv_s, z_w_T_i8, z_s, a_w_T_i8, a_s, b_w_T_i8, b_s):
    return (torch.empty_like(state), torch.empty_like(conv_state),
            state.new_empty((A_log.shape[0], V_DIM), dtype=torch.bfloat16))
