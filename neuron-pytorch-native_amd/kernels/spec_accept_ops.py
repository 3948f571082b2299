"""Speculative-decode acceptance ops on gfx950 (new ops; the reference's sampler lives in
an un-vendored vLLM-Neuron fork and its on-device greedy path is a plain argmax,
contrib/qwen3.6-27b/static_decode.py:1313).

  spec::accept_greedy(target_logits [B, K+1, V] f32, draft_ids [B, K] int64)
      -> (accepted [B] int32, out_ids [B, K+1] int64)
  spec::accept_rejection(target_logits [B, K+1, V] f32, draft_logits [B, K, V] f32,
                         draft_ids [B, K] int64, u_accept [B, K] f32, u_sample [B] f32,
                         inv_temperature: float = 1.0)
      -> (accepted [B] int32, out_ids [B, K+1] int64)

  spec::accept_rejection_lm_head(hidden [B*(K+1), H] bf16, lm_head_w [H, V] fp8 bytes,
                                 lm_head_scale [V] f32, draft_logits, draft_ids, u_accept,
                                 u_sample, inv_temperature)
      -> (accepted, out_ids, target_logits [B, K+1, V] bf16)

accepted[b] is the number of accepted drafts (0..K); out_ids[b] holds those drafts,
then the correction (or bonus) token, then -1. Rejection sampling follows Leviathan
et al. 2023 (Alg. 1) under the library's integer softmax contract (chunk-relative exponentials
with exact chunk factors, so one pass over the logits gives every sum), so its decisions
are bit-identical to the CPU restatement for the same logits and uniforms.
"""
import torch

from npn_native import call, query, require, stream_of


def _workspace(B, K, V, device):
    n = query("npn_accept_workspace_size", B, K, V)
    if n == 0:
        raise RuntimeError(f"unsupported acceptance shape B={B} K={K} V={V}")
    return torch.empty(n, dtype=torch.uint8, device=device)


@torch.library.custom_op("spec::accept_greedy", mutates_args=(), device_types="cuda")
def accept_greedy(target_logits: torch.Tensor,
                  draft_ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    B, T, V = target_logits.shape
    K = T - 1
    require(target_logits, "target_logits", torch.float32, shape=(B, T, V))
    require(draft_ids, "draft_ids", torch.int64, shape=(B, K))
    ws = _workspace(B, K, V, target_logits.device)
    accepted = torch.empty(B, dtype=torch.int32, device=target_logits.device)
    out_ids = torch.empty((B, T), dtype=torch.int64, device=target_logits.device)
    call("npn_accept_greedy", target_logits, draft_ids, accepted, out_ids, B, K, V, ws,
         ws.numel(), stream_of(target_logits))
    return accepted, out_ids


@accept_greedy.register_fake
def _(target_logits, draft_ids):
    B, T, _ = target_logits.shape
    return (target_logits.new_empty((B,), dtype=torch.int32),
            target_logits.new_empty((B, T), dtype=torch.int64))


@torch.library.custom_op("spec::accept_rejection", mutates_args=(), device_types="cuda")
def accept_rejection(target_logits: torch.Tensor, draft_logits: torch.Tensor,
                     draft_ids: torch.Tensor, u_accept: torch.Tensor, u_sample: torch.Tensor,
                     inv_temperature: float = 1.0) -> tuple[torch.Tensor, torch.Tensor]:
    B, T, V = target_logits.shape
    K = T - 1
    require(target_logits, "target_logits", torch.float32, shape=(B, T, V))
    require(draft_logits, "draft_logits", torch.float32, shape=(B, K, V))
    require(draft_ids, "draft_ids", torch.int64, shape=(B, K))
    require(u_accept, "u_accept", torch.float32, shape=(B, K))
    require(u_sample, "u_sample", torch.float32, numel=B)
    if not inv_temperature > 0.0:
        raise ValueError("inv_temperature must be > 0")
    ws = _workspace(B, K, V, target_logits.device)
    accepted = torch.empty(B, dtype=torch.int32, device=target_logits.device)
    out_ids = torch.empty((B, T), dtype=torch.int64, device=target_logits.device)
    call("npn_accept_rejection", target_logits, draft_logits, draft_ids, u_accept, u_sample,
         float(inv_temperature), accepted, out_ids, B, K, V, ws, ws.numel(),
         stream_of(target_logits))
    return accepted, out_ids


@accept_rejection.register_fake
def _(target_logits, draft_logits, draft_ids, u_accept, u_sample, inv_temperature=1.0):
    B, T, _ = target_logits.shape
    return (target_logits.new_empty((B,), dtype=torch.int32),
            target_logits.new_empty((B, T), dtype=torch.int64))


@torch.library.custom_op("spec::commit_", mutates_args=("prev_accepted", "kv_len", "committed"),
                         device_types="cuda")
def commit_(accepted: torch.Tensor, prev_accepted: torch.Tensor, kv_len: torch.Tensor,
            committed: torch.Tensor) -> None:
    """New op: after acceptance, in place: prev_accepted = accepted, kv_len += accepted + 1,
    committed += accepted + 1 (all int32 [B]), for decode state at fixed addresses."""
    B = accepted.numel()
    for t, n in ((accepted, "accepted"), (prev_accepted, "prev_accepted"), (kv_len, "kv_len"),
                 (committed, "committed")):
        require(t, n, torch.int32, numel=B)
    call("npn_spec_commit", accepted, prev_accepted, kv_len, committed, B, stream_of(accepted))


@commit_.register_fake
def _(accepted, prev_accepted, kv_len, committed):
    return None


@torch.library.custom_op("spec::accept_greedy_fused", mutates_args=(), device_types="cuda")
def accept_greedy_fused(hidden: torch.Tensor, lm_head_w: torch.Tensor, lm_head_scale: torch.Tensor,
                        draft_ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """New op: greedy acceptance straight from the LM head: hidden [B*(K+1), H] bf16 (the
    final-normed verify rows, row b*(K+1) + t), lm_head_w [H, V] fp8 bytes, lm_head_scale
    [V] f32, draft_ids [B, K] int64 -> (accepted [B] int32, out_ids [B, K+1] int64), the
    same as accept_greedy(fp8::matmul(hidden, w, scale).float().view(B, K+1, V), draft_ids)
    but without writing or reading the logits."""
    from fp8_matmul_ops import argmax_parts
    B, K = draft_ids.shape
    require(draft_ids, "draft_ids", torch.int64, shape=(B, K))
    if hidden.shape[0] != B * (K + 1):
        raise RuntimeError(f"hidden must have B*(K+1) = {B * (K + 1)} rows, got {hidden.shape[0]}")
    parts = argmax_parts(hidden, lm_head_w, lm_head_scale)
    accepted = torch.empty(B, dtype=torch.int32, device=hidden.device)
    out_ids = torch.empty((B, K + 1), dtype=torch.int64, device=hidden.device)
    call("npn_accept_greedy_parts", parts, parts.shape[1], draft_ids, accepted, out_ids, B, K,
         stream_of(hidden))
    return accepted, out_ids


@accept_greedy_fused.register_fake
def _(hidden, lm_head_w, lm_head_scale, draft_ids):
    B, K = draft_ids.shape
    return (hidden.new_empty((B,), dtype=torch.int32),
            hidden.new_empty((B, K + 1), dtype=torch.int64))


@torch.library.custom_op("spec::accept_rejection_lm_head", mutates_args=(), device_types="cuda")
def accept_rejection_lm_head(hidden: torch.Tensor, lm_head_w: torch.Tensor,
                             lm_head_scale: torch.Tensor, draft_logits: torch.Tensor,
                             draft_ids: torch.Tensor, u_accept: torch.Tensor,
                             u_sample: torch.Tensor, inv_temperature: float = 1.0
                             ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """New op: rejection sampling with the target logits made by the LM head in the same
    call: hidden [B*(K+1), H] bf16 (row b*(K+1) + t), lm_head_w [H, V] e4m3fn bytes,
    lm_head_scale [V] f32 -> (accepted [B] int32, out_ids [B, K+1] int64, target_logits
    [B, K+1, V] bf16). The GEMM's epilogue produces the target rows' chunk statistics, so
    only each sequence's sampling row is read back. Equal, bit for bit, to
    accept_rejection(fp8::matmul(hidden, w, scale).float().view(B, K+1, V), ...)."""
    B, K, V = draft_logits.shape
    T = K + 1
    require(hidden, "hidden", torch.bfloat16)
    if hidden.dim() != 2 or hidden.shape[0] != B * T:
        raise RuntimeError(f"hidden must be [B*(K+1), H] = [{B * T}, H], got {tuple(hidden.shape)}")
    H = hidden.shape[1]
    require(lm_head_w, "lm_head_w", torch.int8, shape=(H, V))
    require(lm_head_scale, "lm_head_scale", torch.float32, numel=V)
    require(draft_logits, "draft_logits", torch.float32, shape=(B, K, V))
    require(draft_ids, "draft_ids", torch.int64, shape=(B, K))
    require(u_accept, "u_accept", torch.float32, shape=(B, K))
    require(u_sample, "u_sample", torch.float32, numel=B)
    if not inv_temperature > 0.0:
        raise ValueError("inv_temperature must be > 0")
    n = query("npn_accept_rejection_lm_head_workspace_size", B, K, H, V)
    if n == 0:
        raise RuntimeError(f"unsupported sizes B={B} K={K} H={H} V={V}")
    ws = torch.empty(n, dtype=torch.uint8, device=hidden.device)
    logits = torch.empty((B, T, V), dtype=torch.bfloat16, device=hidden.device)
    accepted = torch.empty(B, dtype=torch.int32, device=hidden.device)
    out_ids = torch.empty((B, T), dtype=torch.int64, device=hidden.device)
    call("npn_accept_rejection_lm_head", hidden, lm_head_w, lm_head_scale, draft_logits,
         draft_ids, u_accept, u_sample, float(inv_temperature), logits, accepted, out_ids, B, K,
         H, V, ws, ws.numel(), stream_of(hidden))
    return accepted, out_ids, logits


@accept_rejection_lm_head.register_fake
def _(hidden, lm_head_w, lm_head_scale, draft_logits, draft_ids, u_accept, u_sample,
      inv_temperature=1.0):
    B, K, V = draft_logits.shape
    return (hidden.new_empty(B, dtype=torch.int32), hidden.new_empty((B, K + 1), dtype=torch.int64),
            hidden.new_empty((B, K + 1, V), dtype=torch.bfloat16))
