"""GQA attention-tail ops on gfx950.

torch.ops.gqa.tail -- drop-in for the op registered at
contrib/qwen3.6-27b/kernels/gqa_tail_ops.py:14-26 (same name, schema and f32 layouts;
one kv head per call, mask shared over the batch). B = cached_k.shape[0] // S with
S = mask.shape[-1]; q heads per kv head = query.shape[0] // B.

New ops for the T-token verify step (same conventions, bf16 KV cache):
  gqa::tail_verify(query [B,T,Hq,256] bf16, gate [B,T,Hq,256] bf16, q_norm [256] f32,
                   cos [B,T,64] f32, sin [B,T,64] f32,
                   cache_k [B,Hkv,S,256] bf16, cache_v [B,Hkv,S,256] bf16,
                   kv_len [B] int32) -> out [B,T,Hq,256] bf16
      Row (b, t, h) attends cache rows [0, kv_len[b] + t] with kv head h // (Hq/Hkv);
      the T verify rows must already be in the cache at kv_len[b] .. kv_len[b]+T-1.
  gqa::kv_append(key [B,T,Hkv,256] bf16, value [B,T,Hkv,256] bf16, k_norm [256] f32,
                 cos [B,T,64] f32, sin [B,T,64] f32, cache_k, cache_v, kv_len [B] int32)
      -> (), writes rows kv_len[b]+t of both caches in place (the k-side RMSNorm +
      partial RoPE + cache write of _gqa_layer, contrib/qwen3.6-27b/static_decode.py:880-910).
  gqa::tail_verify_append(query, gate, key, value, q_norm, k_norm,
                          cos_table [P,64] f32, sin_table [P,64] f32, cache_k, cache_v, kv_len)
      -> out [B,T,Hq,256] bf16: kv_append then tail_verify in the tail's own launches (the
      append rides in the query-prep launch), with the RoPE rows read from the position
      tables at kv_len[b] + t (clamped to the table) as rope_rows gathers them; equal bit
      for bit to rope_rows + kv_append + tail_verify.
"""
import torch

from npn_native import call, query as size_query, require, stream_of

HEAD_DIM = 256
ROPE_DIM = 64


@torch.library.custom_op("gqa::tail", mutates_args=(), device_types="cuda")
def gqa_tail(
    query: torch.Tensor,    # [B*Q_HEADS, HEAD_DIM] f32 (projected, pre-norm)
    gate: torch.Tensor,      # [B*Q_HEADS, HEAD_DIM] f32 (raw)
    q_norm: torch.Tensor,    # [1, HEAD_DIM] f32
    cos: torch.Tensor,       # [1, ROPE_DIM] f32
    sin: torch.Tensor,       # [1, ROPE_DIM] f32
    cached_k: torch.Tensor,  # [B*S, HEAD_DIM] f32 (already KV-written)
    cached_v: torch.Tensor,  # [B*S, HEAD_DIM] f32
    mask: torch.Tensor,      # [1, S] f32
) -> torch.Tensor:
    """Returns attn_out [B*Q_HEADS, HEAD_DIM] f32 = o * sigmoid(gate), pre-o_proj."""
    S = mask.shape[-1]
    B = cached_k.shape[0] // S
    hq = query.shape[0] // B
    require(query, "query", torch.float32, shape=(B * hq, HEAD_DIM))
    require(gate, "gate", torch.float32, shape=(B * hq, HEAD_DIM))
    require(q_norm, "q_norm", torch.float32, numel=HEAD_DIM)
    require(cos, "cos", torch.float32, numel=ROPE_DIM)
    require(sin, "sin", torch.float32, numel=ROPE_DIM)
    require(cached_k, "cached_k", torch.float32, shape=(B * S, HEAD_DIM))
    require(cached_v, "cached_v", torch.float32, shape=(B * S, HEAD_DIM))
    require(mask, "mask", torch.float32, numel=S)
    out = torch.empty_like(query)
    call("npn_gqa_tail", query, gate, q_norm, cos, sin, cached_k, cached_v, mask, out,
         B, hq, S, stream_of(query))
    return out


@gqa_tail.register_fake
def _(query, gate, q_norm, cos, sin, cached_k, cached_v, mask):
    return torch.empty_like(query)


def tail_verify_workspace(B, T, hq, hkv, s_max, device):
    n = size_query("npn_gqa_tail_verify_workspace_size", B, T, hq, hkv, s_max)
    if n == 0:
        raise RuntimeError(f"unsupported tail_verify shape B={B} T={T} Hq={hq} Hkv={hkv} S={s_max}")
    return torch.empty(n, dtype=torch.uint8, device=device)


@torch.library.custom_op("gqa::tail_verify", mutates_args=(), device_types="cuda")
def gqa_tail_verify(
    query: torch.Tensor,    # [B, T, Hq, 256] bf16
    gate: torch.Tensor,      # [B, T, Hq, 256] bf16
    q_norm: torch.Tensor,    # [256] f32
    cos: torch.Tensor,       # [B, T, 64] f32
    sin: torch.Tensor,       # [B, T, 64] f32
    cache_k: torch.Tensor,   # [B, Hkv, S, 256] bf16
    cache_v: torch.Tensor,   # [B, Hkv, S, 256] bf16
    kv_len: torch.Tensor,    # [B] int32
) -> torch.Tensor:
    B, T, hq, dh = query.shape
    hkv, s_max = cache_k.shape[1], cache_k.shape[2]
    if dh != HEAD_DIM:
        raise RuntimeError(f"head dim must be {HEAD_DIM}")
    require(query, "query", torch.bfloat16)
    require(gate, "gate", torch.bfloat16, shape=query.shape)
    require(q_norm, "q_norm", torch.float32, numel=HEAD_DIM)
    require(cos, "cos", torch.float32, shape=(B, T, ROPE_DIM))
    require(sin, "sin", torch.float32, shape=(B, T, ROPE_DIM))
    require(cache_k, "cache_k", torch.bfloat16, shape=(B, hkv, s_max, HEAD_DIM))
    require(cache_v, "cache_v", torch.bfloat16, shape=(B, hkv, s_max, HEAD_DIM))
    require(kv_len, "kv_len", torch.int32, numel=B)
    ws = tail_verify_workspace(B, T, hq, hkv, s_max, query.device)
    out = torch.empty_like(query)
    call("npn_gqa_tail_verify", query, gate, q_norm, cos, sin, cache_k, cache_v, kv_len, out,
         B, T, hq, hkv, s_max, ws, ws.numel(), stream_of(query))
    return out


@gqa_tail_verify.register_fake
def _(query, gate, q_norm, cos, sin, cache_k, cache_v, kv_len):
    return torch.empty_like(query)


@torch.library.custom_op("gqa::kv_append", mutates_args=("cache_k", "cache_v"),
                         device_types="cuda")
def gqa_kv_append(
    key: torch.Tensor,       # [B, T, Hkv, 256] bf16 (k projection, pre-norm)
    value: torch.Tensor,     # [B, T, Hkv, 256] bf16
    k_norm: torch.Tensor,    # [256] f32
    cos: torch.Tensor,       # [B, T, 64] f32
    sin: torch.Tensor,       # [B, T, 64] f32
    cache_k: torch.Tensor,   # [B, Hkv, S, 256] bf16 (written in place)
    cache_v: torch.Tensor,   # [B, Hkv, S, 256] bf16 (written in place)
    kv_len: torch.Tensor,    # [B] int32
) -> None:
    B, T, hkv, dh = key.shape
    s_max = cache_k.shape[2]
    require(key, "key", torch.bfloat16, shape=(B, T, hkv, HEAD_DIM))
    require(value, "value", torch.bfloat16, shape=(B, T, hkv, HEAD_DIM))
    require(k_norm, "k_norm", torch.float32, numel=HEAD_DIM)
    require(cos, "cos", torch.float32, shape=(B, T, ROPE_DIM))
    require(sin, "sin", torch.float32, shape=(B, T, ROPE_DIM))
    require(cache_k, "cache_k", torch.bfloat16, shape=(B, hkv, s_max, HEAD_DIM))
    require(cache_v, "cache_v", torch.bfloat16, shape=(B, hkv, s_max, HEAD_DIM))
    require(kv_len, "kv_len", torch.int32, numel=B)
    call("npn_gqa_kv_append", key, value, k_norm, cos, sin, cache_k, cache_v, kv_len,
         B, T, hkv, s_max, stream_of(key))


@gqa_kv_append.register_fake
def _(key, value, k_norm, cos, sin, cache_k, cache_v, kv_len):
    return None


@torch.library.custom_op("gqa::tail_verify_append", mutates_args=("cache_k", "cache_v"),
                         device_types="cuda")
def gqa_tail_verify_append(
    query: torch.Tensor,      # [B, T, Hq, 256] bf16
    gate: torch.Tensor,       # [B, T, Hq, 256] bf16
    key: torch.Tensor,        # [B, T, Hkv, 256] bf16 (k projection, pre-norm)
    value: torch.Tensor,      # [B, T, Hkv, 256] bf16
    q_norm: torch.Tensor,     # [256] f32
    k_norm: torch.Tensor,     # [256] f32
    cos_table: torch.Tensor,  # [P, 64] f32
    sin_table: torch.Tensor,  # [P, 64] f32
    cache_k: torch.Tensor,    # [B, Hkv, S, 256] bf16 (rows kv_len[b]+t written in place)
    cache_v: torch.Tensor,    # [B, Hkv, S, 256] bf16 (rows kv_len[b]+t written in place)
    kv_len: torch.Tensor,     # [B] int32
) -> torch.Tensor:
    B, T, hq, dh = query.shape
    hkv, s_max = cache_k.shape[1], cache_k.shape[2]
    P = cos_table.shape[0]
    if dh != HEAD_DIM:
        raise RuntimeError(f"head dim must be {HEAD_DIM}")
    require(query, "query", torch.bfloat16)
    require(gate, "gate", torch.bfloat16, shape=query.shape)
    require(key, "key", torch.bfloat16, shape=(B, T, hkv, HEAD_DIM))
    require(value, "value", torch.bfloat16, shape=(B, T, hkv, HEAD_DIM))
    require(q_norm, "q_norm", torch.float32, numel=HEAD_DIM)
    require(k_norm, "k_norm", torch.float32, numel=HEAD_DIM)
    require(cos_table, "cos_table", torch.float32, shape=(P, ROPE_DIM))
    require(sin_table, "sin_table", torch.float32, shape=(P, ROPE_DIM))
    require(cache_k, "cache_k", torch.bfloat16, shape=(B, hkv, s_max, HEAD_DIM))
    require(cache_v, "cache_v", torch.bfloat16, shape=(B, hkv, s_max, HEAD_DIM))
    require(kv_len, "kv_len", torch.int32, numel=B)
    ws = tail_verify_workspace(B, T, hq, hkv, s_max, query.device)
    out = torch.empty_like(query)
    call("npn_gqa_tail_verify_append", query, gate, key, value, q_norm, k_norm, cos_table,
         sin_table, P, cache_k, cache_v, kv_len, out, B, T, hq, hkv, s_max, ws, ws.numel(),
         stream_of(query))
    return out


@gqa_tail_verify_append.register_fake
def _(query, gate, key, value, q_norm, k_norm, cos_table, sin_table, cache_k, cache_v, kv_len):
    return torch.empty_like(query)


@torch.library.custom_op("gqa::rope_rows", mutates_args=(), device_types="cuda")
def rope_rows(cos_table: torch.Tensor, sin_table: torch.Tensor, kv_len: torch.Tensor,
              T: int) -> tuple[torch.Tensor, torch.Tensor]:
    """New op: cos, sin [B, T, dim] f32 = rows kv_len[b] + t of tables [P, dim] built once
    (the reference's _init_rope table, contrib/qwen3.6-27b/static_decode.py:489-502);
    positions past the table are clamped to its last row."""
    P, dim = cos_table.shape
    B = kv_len.numel()
    require(cos_table, "cos_table", torch.float32, shape=(P, dim))
    require(sin_table, "sin_table", torch.float32, shape=(P, dim))
    require(kv_len, "kv_len", torch.int32, numel=B)
    cos = torch.empty((B, T, dim), dtype=torch.float32, device=cos_table.device)
    sin = torch.empty_like(cos)
    call("npn_rope_rows", cos_table, sin_table, P, kv_len, cos, sin, B, T, dim,
         stream_of(cos_table))
    return cos, sin


@rope_rows.register_fake
def _(cos_table, sin_table, kv_len, T):
    shape = (kv_len.numel(), T, cos_table.shape[1])
    return cos_table.new_empty(shape), cos_table.new_empty(shape)
