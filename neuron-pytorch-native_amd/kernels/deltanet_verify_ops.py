"""Multi-token verify ops for the gated-DeltaNet layer on gfx950.

New ops in the reference's conventions (flattened batch in dim 0, functional,
shared weights), extending deltanet::full_batched
(contrib/qwen3.6-27b/kernels/deltanet_full_batched_ops.py:22-41) from one token to
the T = K+1 tokens of a speculative verify block:

  deltanet::verify_batched(state, mixed_qkv, conv_state, conv_weight, conv_bias,
                           a_out, b_out, z, A_log, dt_bias, norm_weight)
      -> (ckpt [B*T*Hv*128, 128] f32, out [B*T*Hv, 128] bf16)
  deltanet::verify_from_ckpt(prev_ckpt, state_index, mixed_qkv, ...)
      -> same; the initial state of sequence b is prev_ckpt[b, state_index[b]]
         (index-based rollback: the previous step's accepted checkpoint is read in
         place, no state copy)
  deltanet::verify_from_ckpt_into(prev_ckpt, state_index, mixed_qkv, ..., ckpt_out)
      -> out; as verify_from_ckpt, writing the checkpoints into the caller's ckpt_out
         (persistent ping-pong buffers for a captured HIP graph of the step)
  deltanet::rollback(ckpt, mixed_qkv, conv_state, accepted)
      -> (state [B*Hv*128, 128] f32 = ckpt[b, accepted[b]],
          conv_state [B*QKV, 3] bf16 = last 3 of [conv_state || x_0..x_a])

ckpt[b, t] is the state after verify token t; with `accepted` drafts the
sequence continues from ckpt[b, accepted] -- the reference's traj[k-1] with
k = accepted + 1 (contrib/qwen3.6-27b/kernels/tests/test_deltanet_spec_verify_rollback.py:64-68).
T is derived from a_out: T = a_out.numel() // (B*Hv).
"""
import ctypes

import torch

from npn_native import call, require, stream_of
from deltanet_full_batched_ops import K_DIM, V_DIM, heads_from_shapes

MAX_T = 16


def _check_common(mixed_qkv, conv_state, conv_weight, conv_bias, a_out, b_out, z, A_log,
                  dt_bias, norm_weight, B):
    hk, hv = heads_from_shapes(conv_weight.shape[0], A_log.numel())
    qkv = conv_weight.shape[0]
    if B < 1:
        raise RuntimeError("batch size derived from the state shape is 0")
    if a_out.numel() % (B * hv):
        raise RuntimeError("a_out must hold B*T*Hv gate values")
    T = a_out.numel() // (B * hv)
    if not 1 <= T <= MAX_T:
        raise RuntimeError(f"verify length T={T} outside [1, {MAX_T}]")
    require(mixed_qkv, "mixed_qkv", torch.bfloat16, numel=B * T * qkv)
    require(conv_state, "conv_state", torch.bfloat16, shape=(B * qkv, 3))
    require(conv_weight, "conv_weight", torch.float32, shape=(qkv, 4))
    require(conv_bias, "conv_bias", torch.float32, numel=qkv)
    require(a_out, "a_out", torch.float32, numel=B * T * hv)
    require(b_out, "b_out", torch.float32, numel=B * T * hv)
    require(z, "z", torch.bfloat16, numel=B * T * hv * V_DIM)
    require(A_log, "A_log", torch.float32, numel=hv)
    require(dt_bias, "dt_bias", torch.float32, numel=hv)
    require(norm_weight, "norm_weight", torch.float32, numel=V_DIM)
    return hk, hv, T


def _verify(state, state_index, state_T, mixed_qkv, conv_state, conv_weight, conv_bias, a_out,
            b_out, z, A_log, dt_bias, norm_weight, B, hk, hv, T, ckpt=None):
    if ckpt is None:
        ckpt = torch.empty((B * T * hv * K_DIM, V_DIM), dtype=torch.float32,
                           device=mixed_qkv.device)
    out = torch.empty((B * T * hv, V_DIM), dtype=torch.bfloat16, device=mixed_qkv.device)
    call("npn_deltanet_verify", state, state_index, state_T, mixed_qkv, conv_state, conv_weight,
         conv_bias, a_out, b_out, z, A_log, dt_bias, norm_weight, ckpt, out, B, T, hk, hv,
         stream_of(mixed_qkv))
    return ckpt, out


@torch.library.custom_op("deltanet::verify_batched", mutates_args=(), device_types="cuda")
def deltanet_verify_batched(
    state: torch.Tensor,         # [B*V_HEADS*K_DIM, V_DIM] f32
    mixed_qkv: torch.Tensor,     # [B*T*QKV_DIM] bf16
    conv_state: torch.Tensor,    # [B*QKV_DIM, 3] bf16
    conv_weight: torch.Tensor,   # [QKV_DIM, 4] f32 (shared)
    conv_bias: torch.Tensor,     # [QKV_DIM] f32 (shared)
    a_out: torch.Tensor,         # [B*T*V_HEADS] f32
    b_out: torch.Tensor,         # [B*T*V_HEADS] f32
    z: torch.Tensor,             # [B*T*V_HEADS, V_DIM] bf16
    A_log: torch.Tensor,         # [V_HEADS] f32 (shared)
    dt_bias: torch.Tensor,       # [V_HEADS] f32 (shared)
    norm_weight: torch.Tensor,   # [V_DIM] f32 (shared)
) -> tuple[torch.Tensor, torch.Tensor]:
    hv = A_log.numel()
    B = state.shape[0] // (hv * K_DIM)
    hk, hv, T = _check_common(mixed_qkv, conv_state, conv_weight, conv_bias, a_out, b_out, z,
                              A_log, dt_bias, norm_weight, B)
    require(state, "state", torch.float32, shape=(B * hv * K_DIM, V_DIM))
    return _verify(state, None, 0, mixed_qkv, conv_state, conv_weight, conv_bias, a_out, b_out,
                   z, A_log, dt_bias, norm_weight, B, hk, hv, T)


@deltanet_verify_batched.register_fake
def _(state, mixed_qkv, conv_state, conv_weight, conv_bias, a_out, b_out, z, A_log, dt_bias,
      norm_weight):
    hv = A_log.shape[0]
    bt_hv = a_out.shape[0]
    return (state.new_empty((bt_hv * K_DIM, V_DIM)),
            state.new_empty((bt_hv, V_DIM), dtype=torch.bfloat16))


@torch.library.custom_op("deltanet::verify_from_ckpt", mutates_args=(), device_types="cuda")
def deltanet_verify_from_ckpt(
    prev_ckpt: torch.Tensor,     # [B*Tp*V_HEADS*K_DIM, V_DIM] f32 (previous verify's ckpt)
    state_index: torch.Tensor,   # [B] int32 in [0, Tp-1] (previous accepted lengths)
    mixed_qkv: torch.Tensor,
    conv_state: torch.Tensor,
    conv_weight: torch.Tensor,
    conv_bias: torch.Tensor,
    a_out: torch.Tensor,
    b_out: torch.Tensor,
    z: torch.Tensor,
    A_log: torch.Tensor,
    dt_bias: torch.Tensor,
    norm_weight: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    B = state_index.numel()
    hk, hv, T = _check_common(mixed_qkv, conv_state, conv_weight, conv_bias, a_out, b_out, z,
                              A_log, dt_bias, norm_weight, B)
    require(state_index, "state_index", torch.int32, numel=B)
    if prev_ckpt.shape[0] % (B * hv * K_DIM):
        raise RuntimeError("prev_ckpt must hold B*Tp*Hv*128 rows")
    Tp = prev_ckpt.shape[0] // (B * hv * K_DIM)
    require(prev_ckpt, "prev_ckpt", torch.float32, shape=(B * Tp * hv * K_DIM, V_DIM))
    return _verify(prev_ckpt, state_index, Tp, mixed_qkv, conv_state, conv_weight, conv_bias,
                   a_out, b_out, z, A_log, dt_bias, norm_weight, B, hk, hv, T)


@deltanet_verify_from_ckpt.register_fake
def _(prev_ckpt, state_index, mixed_qkv, conv_state, conv_weight, conv_bias, a_out, b_out, z,
      A_log, dt_bias, norm_weight):
    bt_hv = a_out.shape[0]
    return (prev_ckpt.new_empty((bt_hv * K_DIM, V_DIM)),
            prev_ckpt.new_empty((bt_hv, V_DIM), dtype=torch.bfloat16))


@torch.library.custom_op("deltanet::verify_from_ckpt_into", mutates_args=("ckpt_out",),
                         device_types="cuda")
def deltanet_verify_from_ckpt_into(
    prev_ckpt: torch.Tensor,
    state_index: torch.Tensor,
    mixed_qkv: torch.Tensor,
    conv_state: torch.Tensor,
    conv_weight: torch.Tensor,
    conv_bias: torch.Tensor,
    a_out: torch.Tensor,
    b_out: torch.Tensor,
    z: torch.Tensor,
    A_log: torch.Tensor,
    dt_bias: torch.Tensor,
    norm_weight: torch.Tensor,
    ckpt_out: torch.Tensor,      # [B*T*V_HEADS*K_DIM, V_DIM] f32, must not overlap prev_ckpt
) -> torch.Tensor:
    B = state_index.numel()
    hk, hv, T = _check_common(mixed_qkv, conv_state, conv_weight, conv_bias, a_out, b_out, z,
                              A_log, dt_bias, norm_weight, B)
    require(state_index, "state_index", torch.int32, numel=B)
    if prev_ckpt.shape[0] % (B * hv * K_DIM):
        raise RuntimeError("prev_ckpt must hold B*Tp*Hv*128 rows")
    Tp = prev_ckpt.shape[0] // (B * hv * K_DIM)
    require(prev_ckpt, "prev_ckpt", torch.float32, shape=(B * Tp * hv * K_DIM, V_DIM))
    require(ckpt_out, "ckpt_out", torch.float32, shape=(B * T * hv * K_DIM, V_DIM))
    p0, p1 = prev_ckpt.data_ptr(), prev_ckpt.data_ptr() + prev_ckpt.numel() * 4
    o0, o1 = ckpt_out.data_ptr(), ckpt_out.data_ptr() + ckpt_out.numel() * 4
    if p0 < o1 and o0 < p1:
        raise RuntimeError("ckpt_out must not overlap prev_ckpt")
    return _verify(prev_ckpt, state_index, Tp, mixed_qkv, conv_state, conv_weight, conv_bias,
                   a_out, b_out, z, A_log, dt_bias, norm_weight, B, hk, hv, T, ckpt=ckpt_out)[1]


@deltanet_verify_from_ckpt_into.register_fake
def _(prev_ckpt, state_index, mixed_qkv, conv_state, conv_weight, conv_bias, a_out, b_out, z,
      A_log, dt_bias, norm_weight, ckpt_out):
    return prev_ckpt.new_empty((a_out.shape[0], V_DIM), dtype=torch.bfloat16)


@torch.library.custom_op("deltanet::rollback", mutates_args=(), device_types="cuda")
def deltanet_rollback(
    ckpt: torch.Tensor,          # [B*T*V_HEADS*K_DIM, V_DIM] f32
    mixed_qkv: torch.Tensor,     # [B*T*QKV_DIM] bf16
    conv_state: torch.Tensor,    # [B*QKV_DIM, 3] bf16
    accepted: torch.Tensor,      # [B] int32 in [0, T-1]
) -> tuple[torch.Tensor, torch.Tensor]:
    B = accepted.numel()
    qkv = conv_state.shape[0] // B
    T = mixed_qkv.numel() // (B * qkv)
    hv_rows = ckpt.shape[0] // (B * T)
    hv = hv_rows // K_DIM
    hk = (qkv // K_DIM - hv) // 2
    require(accepted, "accepted", torch.int32, numel=B)
    require(ckpt, "ckpt", torch.float32, shape=(B * T * hv * K_DIM, V_DIM))
    require(mixed_qkv, "mixed_qkv", torch.bfloat16, numel=B * T * qkv)
    require(conv_state, "conv_state", torch.bfloat16, shape=(B * qkv, 3))
    heads_from_shapes(qkv, hv)
    state = torch.empty((B * hv * K_DIM, V_DIM), dtype=torch.float32, device=ckpt.device)
    new_conv = torch.empty_like(conv_state)
    call("npn_deltanet_rollback", ckpt, mixed_qkv, conv_state, accepted, state, new_conv,
         B, T, hk, hv, stream_of(ckpt))
    return state, new_conv


@deltanet_rollback.register_fake
def _(ckpt, mixed_qkv, conv_state, accepted):
    B = accepted.shape[0]
    qkv = conv_state.shape[0] // B
    T = mixed_qkv.shape[0] // (B * qkv)
    return ckpt.new_empty((ckpt.shape[0] // T, V_DIM)), torch.empty_like(conv_state)


@torch.library.custom_op("deltanet::conv_rollback", mutates_args=(), device_types="cuda")
def deltanet_conv_rollback(
    mixed_qkv: torch.Tensor,     # [B*T*QKV_DIM] bf16
    conv_state: torch.Tensor,    # [B*QKV_DIM, 3] bf16
    accepted: torch.Tensor,      # [B] int32 in [0, T-1]
    v_heads: int,
) -> torch.Tensor:
    """Conv-window rollback only, for index-based state rollback (verify_from_ckpt)."""
    B = accepted.numel()
    qkv = conv_state.shape[0] // B
    T = mixed_qkv.numel() // (B * qkv)
    hk, hv = heads_from_shapes(qkv, v_heads)
    require(accepted, "accepted", torch.int32, numel=B)
    require(mixed_qkv, "mixed_qkv", torch.bfloat16, numel=B * T * qkv)
    require(conv_state, "conv_state", torch.bfloat16, shape=(B * qkv, 3))
    new_conv = torch.empty_like(conv_state)
    call("npn_deltanet_rollback", None, mixed_qkv, conv_state, accepted, None, new_conv,
         B, T, hk, hv, stream_of(conv_state))
    return new_conv


@deltanet_conv_rollback.register_fake
def _(mixed_qkv, conv_state, accepted, v_heads):
    return torch.empty_like(conv_state)


@torch.library.custom_op("deltanet::conv_rollback_", mutates_args=("conv_state",),
                         device_types="cuda")
def deltanet_conv_rollback_(
    mixed_qkv: torch.Tensor,     # [B*T*QKV_DIM] bf16
    conv_state: torch.Tensor,    # [B*QKV_DIM, 3] bf16, rolled back in place
    accepted: torch.Tensor,      # [B] int32 in [0, T-1]
    v_heads: int,
) -> None:
    """deltanet::conv_rollback writing the new window over conv_state (fixed addresses)."""
    B = accepted.numel()
    qkv = conv_state.shape[0] // B
    T = mixed_qkv.numel() // (B * qkv)
    hk, hv = heads_from_shapes(qkv, v_heads)
    require(accepted, "accepted", torch.int32, numel=B)
    require(mixed_qkv, "mixed_qkv", torch.bfloat16, numel=B * T * qkv)
    require(conv_state, "conv_state", torch.bfloat16, shape=(B * qkv, 3))
    call("npn_deltanet_rollback", None, mixed_qkv, conv_state, accepted, None, conv_state,
         B, T, hk, hv, stream_of(conv_state))


@deltanet_conv_rollback_.register_fake
def _(mixed_qkv, conv_state, accepted, v_heads):
    return None


@torch.library.custom_op("deltanet::rollback_commit_",
                         mutates_args=("conv_states", "prev_accepted", "kv_len", "committed"),
                         device_types="cuda")
def deltanet_rollback_commit_(
    mixed_qkvs: list[torch.Tensor],   # per DeltaNet layer: [B*T*QKV_DIM] bf16
    conv_states: list[torch.Tensor],  # per DeltaNet layer: [B*QKV_DIM, 3] bf16, in place
    accepted: torch.Tensor,           # [B] int32 in [0, T-1] (clamped into it on the device)
    prev_accepted: torch.Tensor,      # [B] int32, set to accepted
    kv_len: torch.Tensor,             # [B] int32, += accepted + 1
    committed: torch.Tensor,          # [B] int32, += accepted + 1
    v_heads: int,
    verify_T: int = -1,               # T; -1: from the layers' shapes (required without layers)
) -> None:
    """deltanet::conv_rollback_ over every layer plus spec::commit_, in one launch. accepted is
    clamped into [0, T-1] for every output alike, so the windows and kv_len count the same
    tokens."""
    B = accepted.numel()
    if len(mixed_qkvs) != len(conv_states) or len(conv_states) > 8:
        raise RuntimeError("rollback_commit_: one mixed_qkv per conv_state, at most 8 layers")
    for t, n in ((accepted, "accepted"), (prev_accepted, "prev_accepted"), (kv_len, "kv_len"),
                 (committed, "committed")):
        require(t, n, torch.int32, numel=B)
    hk, hv, T = 1, v_heads, 1
    for mixed, conv in zip(mixed_qkvs, conv_states):
        qkv = conv.shape[0] // B
        T = mixed.numel() // (B * qkv)
        hk, hv = heads_from_shapes(qkv, v_heads)
        require(mixed, "mixed_qkv", torch.bfloat16, numel=B * T * qkv)
        require(conv, "conv_state", torch.bfloat16, shape=(B * qkv, 3))
    if len({(m.numel(), c.shape) for m, c in zip(mixed_qkvs, conv_states)}) > 1:
        raise RuntimeError("rollback_commit_: every layer must have the same shapes")
    if verify_T != -1:
        if conv_states and verify_T != T:
            raise RuntimeError(f"rollback_commit_: verify_T {verify_T} but the layers hold T={T}")
        T = verify_T
    elif not conv_states:
        raise RuntimeError("rollback_commit_: without layers, verify_T must be given")
    n = len(conv_states)
    mp = (ctypes.c_void_p * max(n, 1))(*[m.data_ptr() for m in mixed_qkvs])
    cp = (ctypes.c_void_p * max(n, 1))(*[c.data_ptr() for c in conv_states])
    call("npn_deltanet_rollback_commit", mp, cp, n, accepted, prev_accepted, kv_len, committed,
         B, T, hk, hv, stream_of(accepted))


@deltanet_rollback_commit_.register_fake
def _(mixed_qkvs, conv_states, accepted, prev_accepted, kv_len, committed, v_heads, verify_T=-1):
    return None
