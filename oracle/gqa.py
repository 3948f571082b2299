"""GQA attention-tail oracle: decode tail, T-token verify tail, KV append (test infrastructure only).

Restates, in numpy float64:
- ``gqa::tail`` (``contrib/qwen3.6-27b/kernels/gqa_tail_ops.py:14-26``) as computed by
  ``gqa_tail_ref`` (``contrib/qwen3.6-27b/kernels/gqa_tail_ref.py:31-70``):
  q' = (1+w)*q*rsqrt(mean(q^2)+1e-6); partial RoPE on dims [:64] with rotate_half
  inside those 64; s = q'.k/sqrt(256) + (mask-1)*1e9; softmax; o = P.V; out = o*sigmoid(gate).
- the T-token verify form of the same tail: row (b, t, head) attends cache rows
  [0, kv_len[b] + t] (causal over the T appended rows), RoPE cos/sin per row.
- the k-side glue that fills the cache before the tail, ``_gqa_layer``
  (``contrib/qwen3.6-27b/static_decode.py:880-910``): k = bf16(rms_norm(k)),
  k = bf16(rope(k)), rows written at their positions; v copied.
- the RoPE table of ``_init_rope`` (``contrib/qwen3.6-27b/static_decode.py:489-502``),
  computed in float32 like the reference.

Pinning (tests/test_oracle_gqa.py): torch ``scaled_dot_product_attention`` with an
explicit boolean mask on CPU (fp64), a brute-force fp64 loop on tiny shapes, the
append-after-attention equivalence of
``contrib/qwen3.6-35b-a3b/kernels/tests/test_gqa_stateful_cache_cpu.py:9-40``
(cache written by kv_append then attended == attention over a cloned cache), the
decode tail == verify tail at T=1 with a prefix mask, and torch's own rotate_half
RoPE on random vectors.
"""
import numpy as np

from .numerics import bf16_bits_to_f32, f32_to_bf16_bits, sigmoid

RMS_EPS = 1e-6
ROPE_DIM = 64


def rope_cos_sin(positions, theta=1e7, rope_dim=ROPE_DIM):
    """cos/sin rows for integer positions, float32 like the reference table
    (static_decode.py:489-502): inv_freq = 1/theta^(arange(0,d,2)/d) rounded to fp32,
    freqs = fp32(pos * inv_freq), emb = cat(f, f). The kernels take these tables as inputs;
    tests feed the same table to the device and the oracle."""
    inv_freq = (1.0 / (float(theta) ** (np.arange(0, rope_dim, 2, dtype=np.float64) / rope_dim))).astype(np.float32)
    pos = np.asarray(positions, dtype=np.float32)
    freqs = (pos[..., None] * inv_freq).astype(np.float32)
    emb = np.concatenate([freqs, freqs], axis=-1)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def rms_norm_1p(x, w):
    """(1 + w) * x * rsqrt(mean(x^2) + eps) over the last axis (gqa_tail_ref.py:31-34)."""
    x = np.asarray(x, np.float64)
    return (1.0 + np.asarray(w, np.float64)) * (x / np.sqrt((x * x).mean(-1, keepdims=True) + RMS_EPS))


def rope_partial(x, cos, sin):
    """Rotary on x[..., :64] with rotate_half = cat(-x[32:64], x[:32]); rest passes
    (gqa_tail_ref.py:37-46). cos/sin broadcast against x[..., :64]."""
    x = np.asarray(x, np.float64)
    r = x[..., :ROPE_DIM]
    h = ROPE_DIM // 2
    rot = np.concatenate([-r[..., h:], r[..., :h]], axis=-1)
    out = x.copy()
    out[..., :ROPE_DIM] = r * np.asarray(cos, np.float64) + rot * np.asarray(sin, np.float64)
    return out


def _softmax_rows(s):
    m = s.max(-1, keepdims=True)
    e = np.exp(s - m)
    return e / e.sum(-1, keepdims=True)


def gqa_tail(query, gate, q_norm, cos, sin, cached_k, cached_v, mask):
    """Reference ``gqa::tail`` semantics on its own flat layouts, one kv head per group:
    query, gate [B*Hq, Dh]; q_norm [1, Dh]; cos, sin [1, 64]; cached_k/v [B*S, Dh];
    mask [1, S] (1 valid, 0 masked). Returns float64 [B*Hq, Dh] (gqa_tail_ref.py:49-70)."""
    S = mask.shape[-1]
    Dh = query.shape[-1]
    B = cached_k.shape[0] // S
    Hq = query.shape[0] // B
    q = rms_norm_1p(np.asarray(query, np.float64).reshape(B, Hq, Dh), np.reshape(q_norm, (Dh,)))
    q = rope_partial(q, np.reshape(cos, (ROPE_DIM,)), np.reshape(sin, (ROPE_DIM,)))
    k = np.asarray(cached_k, np.float64).reshape(B, S, Dh)
    v = np.asarray(cached_v, np.float64).reshape(B, S, Dh)
    neg = (1.0 - np.asarray(mask, np.float64).reshape(1, 1, S)) * -1e9
    s = np.einsum("bhd,bsd->bhs", q, k) / np.sqrt(Dh) + neg
    o = np.einsum("bhs,bsd->bhd", _softmax_rows(s), v)
    g = sigmoid(np.asarray(gate, np.float64).reshape(B, Hq, Dh))
    return (o * g).reshape(B * Hq, Dh)


def gqa_tail_verify(query, gate, q_norm, cos, sin, cache_k, cache_v, kv_len):
    """T-token verify tail.
    query, gate  [B, T, Hq, Dh] bf16 bits; q_norm [Dh] f32; cos, sin [B, T, 64] f32;
    cache_k/v    [B, Hkv, Smax, Dh] bf16 bits, rows [0, kv_len[b]+T) valid;
    kv_len       [B] int, the number of cache rows before the T verify rows.
    Row (b, t, qh) uses kv head qh // (Hq/Hkv) and attends rows [0, kv_len[b]+t].
    Returns float64 [B, T, Hq, Dh] (before the bf16 cast)."""
    qf = bf16_bits_to_f32(query).astype(np.float64)
    gf = bf16_bits_to_f32(gate).astype(np.float64)
    B, T, Hq, Dh = qf.shape
    Hkv = cache_k.shape[1]
    grp = Hq // Hkv
    q = rms_norm_1p(qf, q_norm)
    q = rope_partial(q, np.asarray(cos)[:, :, None, :], np.asarray(sin)[:, :, None, :])
    out = np.empty((B, T, Hq, Dh), np.float64)
    for b in range(B):
        L = int(kv_len[b]) + T
        k = bf16_bits_to_f32(cache_k[b, :, :L]).astype(np.float64)    # [Hkv, L, Dh]
        v = bf16_bits_to_f32(cache_v[b, :, :L]).astype(np.float64)
        for g in range(Hkv):
            qb = q[b, :, g * grp:(g + 1) * grp]                        # [T, grp, Dh]
            s = np.einsum("thd,ld->thl", qb, k[g]) / np.sqrt(Dh)
            lim = int(kv_len[b]) + np.arange(T)                        # last valid row per t
            valid = np.arange(L)[None, :] <= lim[:, None]              # [T, L]
            s = np.where(valid[:, None, :], s, -np.inf)
            o = np.einsum("thl,ld->thd", _softmax_rows(s), v[g])
            out[b, :, g * grp:(g + 1) * grp] = o * sigmoid(gf[b, :, g * grp:(g + 1) * grp])
    return out


def gqa_kv_append(key, value, k_norm, cos, sin, cache_k, cache_v, kv_len):
    """Write the T verify rows into the cache, in place, and return (cache_k, cache_v).
    key, value [B, T, Hkv, Dh] bf16 bits (projection output); k_norm [Dh] f32.
    Row kv_len[b]+t of head g gets bf16(rope(bf16(rms_norm_1p(key))));
    value rows are copied (static_decode.py:880-910). Rounding to bf16 happens
    after the norm and after the RoPE, like the reference's two ``.to(x.dtype)``."""
    kf = bf16_bits_to_f32(key).astype(np.float32)
    xf = kf.astype(np.float32)
    var = (xf * xf).mean(-1, keepdims=True, dtype=np.float32)
    normed = ((np.float32(1.0) + np.asarray(k_norm, np.float32)) * (xf * (np.float32(1.0) / np.sqrt(var + np.float32(RMS_EPS))))).astype(np.float32)
    k1 = bf16_bits_to_f32(f32_to_bf16_bits(normed))
    c = np.asarray(cos, np.float32)[:, :, None, :]
    s = np.asarray(sin, np.float32)[:, :, None, :]
    r = k1[..., :ROPE_DIM]
    h = ROPE_DIM // 2
    rot = np.concatenate([-r[..., h:], r[..., :h]], axis=-1)
    k2 = k1.copy()
    k2[..., :ROPE_DIM] = (r * c + rot * s).astype(np.float32)
    kbits = f32_to_bf16_bits(k2)
    B, T = key.shape[:2]
    for b in range(B):
        p0 = int(kv_len[b])
        for t in range(T):
            cache_k[b, :, p0 + t] = kbits[b, t]
            cache_v[b, :, p0 + t] = value[b, t]
    return cache_k, cache_v
