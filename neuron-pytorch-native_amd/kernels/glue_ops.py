"""Glue ops of the verify step, each one pass on gfx950 (new ops; they replace chains of
torch elementwise kernels in the reference's decode layers):

  glue::silu_mul(gate_up [M, 2I] bf16) -> [M, I] bf16 = bf16(bf16(silu(gate)) * up)
      (_mlp_layer, contrib/qwen3.6-27b/static_decode.py:951-963)
  glue::deltanet_split(proj [M, ld] bf16, qkv_n, z_n, hv)
      -> mixed_qkv [M, qkv_n] bf16, z [M, z_n] bf16, a [M, hv] f32, b [M, hv] f32
      (the slices and casts of _deltanet_layer, static_decode.py:802-832)
  glue::gqa_split(proj [M, ld] bf16, q_heads, kv_heads, head_dim)
      -> query, gate [M, q_heads, head_dim], key, value [M, kv_heads, head_dim] bf16
      (_gqa_layer, static_decode.py:867-870, :880-890)
  glue::deltanet_split_partials, glue::gqa_split_partials: the same, reading the projection
      as fp8::matmul_partials output [S, M, ld] f32 plus its scale; bit-identical to
      fp8::matmul followed by the bf16 form
"""
import torch

from npn_native import call, require, stream_of


@torch.library.custom_op("glue::silu_mul", mutates_args=(), device_types="cuda")
def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    M, I2 = gate_up.shape
    require(gate_up, "gate_up", torch.bfloat16)
    if I2 % 16:
        raise RuntimeError(f"gate_up width {I2} must be a multiple of 16")
    out = gate_up.new_empty((M, I2 // 2))
    call("npn_silu_mul", gate_up, out, M, I2 // 2, stream_of(gate_up))
    return out


@silu_mul.register_fake
def _(gate_up):
    return gate_up.new_empty((gate_up.shape[0], gate_up.shape[1] // 2))


@torch.library.custom_op("glue::deltanet_split", mutates_args=(), device_types="cuda")
def deltanet_split(proj: torch.Tensor, qkv_n: int, z_n: int,
                   hv: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    M, ld = proj.shape
    require(proj, "proj", torch.bfloat16)
    mixed = proj.new_empty((M, qkv_n))
    z = proj.new_empty((M, z_n))
    a = torch.empty((M, hv), dtype=torch.float32, device=proj.device)
    b = torch.empty((M, hv), dtype=torch.float32, device=proj.device)
    call("npn_deltanet_split", proj, ld, mixed, z, a, b, M, qkv_n, z_n, hv, stream_of(proj))
    return mixed, z, a, b


@deltanet_split.register_fake
def _(proj, qkv_n, z_n, hv):
    M = proj.shape[0]
    f32 = torch.float32
    return (proj.new_empty((M, qkv_n)), proj.new_empty((M, z_n)),
            proj.new_empty((M, hv), dtype=f32), proj.new_empty((M, hv), dtype=f32))


@torch.library.custom_op("glue::gqa_split", mutates_args=(), device_types="cuda")
def gqa_split(proj: torch.Tensor, q_heads: int, kv_heads: int,
              head_dim: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    M, ld = proj.shape
    require(proj, "proj", torch.bfloat16)
    query = proj.new_empty((M, q_heads, head_dim))
    gate = proj.new_empty((M, q_heads, head_dim))
    key = proj.new_empty((M, kv_heads, head_dim))
    value = proj.new_empty((M, kv_heads, head_dim))
    call("npn_gqa_split", proj, ld, query, gate, key, value, M, q_heads, kv_heads, head_dim,
         stream_of(proj))
    return query, gate, key, value


@gqa_split.register_fake
def _(proj, q_heads, kv_heads, head_dim):
    M = proj.shape[0]
    return (proj.new_empty((M, q_heads, head_dim)), proj.new_empty((M, q_heads, head_dim)),
            proj.new_empty((M, kv_heads, head_dim)), proj.new_empty((M, kv_heads, head_dim)))


def _partials(partials, scale, name="partials"):
    if partials.dim() != 3:
        raise RuntimeError(f"{name} must be [S, M, N], got {tuple(partials.shape)}")
    S, M, ld = partials.shape
    require(partials, name, torch.float32)
    require(scale, "scale", torch.float32, numel=ld)
    return S, M, ld


@torch.library.custom_op("glue::deltanet_split_partials", mutates_args=(), device_types="cuda")
def deltanet_split_partials(partials: torch.Tensor, scale: torch.Tensor, qkv_n: int, z_n: int,
                            hv: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                              torch.Tensor]:
    S, M, ld = _partials(partials, scale)
    bf = torch.bfloat16
    mixed = torch.empty((M, qkv_n), dtype=bf, device=partials.device)
    z = torch.empty((M, z_n), dtype=bf, device=partials.device)
    a = torch.empty((M, hv), dtype=torch.float32, device=partials.device)
    b = torch.empty((M, hv), dtype=torch.float32, device=partials.device)
    call("npn_deltanet_split_partials", partials, S, scale, ld, mixed, z, a, b, M, qkv_n, z_n,
         hv, stream_of(partials))
    return mixed, z, a, b


@deltanet_split_partials.register_fake
def _(partials, scale, qkv_n, z_n, hv):
    M = partials.shape[1]
    bf = torch.bfloat16
    return (partials.new_empty((M, qkv_n), dtype=bf), partials.new_empty((M, z_n), dtype=bf),
            partials.new_empty((M, hv)), partials.new_empty((M, hv)))


@torch.library.custom_op("glue::gqa_split_partials", mutates_args=(), device_types="cuda")
def gqa_split_partials(partials: torch.Tensor, scale: torch.Tensor, q_heads: int, kv_heads: int,
                       head_dim: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                               torch.Tensor]:
    S, M, ld = _partials(partials, scale)
    bf = torch.bfloat16
    dev = partials.device
    query = torch.empty((M, q_heads, head_dim), dtype=bf, device=dev)
    gate = torch.empty((M, q_heads, head_dim), dtype=bf, device=dev)
    key = torch.empty((M, kv_heads, head_dim), dtype=bf, device=dev)
    value = torch.empty((M, kv_heads, head_dim), dtype=bf, device=dev)
    call("npn_gqa_split_partials", partials, S, scale, ld, query, gate, key, value, M, q_heads,
         kv_heads, head_dim, stream_of(partials))
    return query, gate, key, value


@gqa_split_partials.register_fake
def _(partials, scale, q_heads, kv_heads, head_dim):
    M = partials.shape[1]
    bf = torch.bfloat16
    return (partials.new_empty((M, q_heads, head_dim), dtype=bf),
            partials.new_empty((M, q_heads, head_dim), dtype=bf),
            partials.new_empty((M, kv_heads, head_dim), dtype=bf),
            partials.new_empty((M, kv_heads, head_dim), dtype=bf))
