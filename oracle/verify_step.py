"""Oracle of the verify-and-accept step of a hybrid slice (test infrastructure only).

Composes the op oracles the way the reference's decode harness composes its ops
(contrib/qwen3.6-27b/static_decode.py: _deltanet_layer :753-847, _gqa_layer :849-949,
_mlp_layer :951-963, rms_norm :322-335), for T verify tokens, rounding to bf16 at the
same points as the device path (every op output and residual add is bf16).

Layer dicts hold numpy arrays: fp8 weights as ([K, N] uint8/int8 bytes, [N] f32 scale),
norms and DeltaNet parameters as float32, the decode state (DeltaNet state [B,Hv,128,128]
and conv state bits [B,QKV,3]; GQA cache bits [B,Hkv,S,256]) and kv_len [B].

Pinning: tests/test_oracle_layers.py checks deltanet_mixer, gqa_mixer, mlp_branch,
rms_norm_1p_bits and the DeltaNet / KV state they leave against HF transformers' Qwen3.5
decoder layers (tests/golden/layers_hf.npz, made by tests/golden/make_layer_fixture.py):
against HF run with bf16 rounding at the harness's op boundaries to 2e-3 relative (most
outputs bit-identical), against HF in float32 to the bf16 noise of those roundings, and with
plausible mistakes planted in this oracle failing. The end-to-end GPU test compares the
device step against it over two consecutive steps (tests/test_gpu_verify_step.py).
"""
import numpy as np

from . import accept as oa
from . import deltanet as od
from . import fp8 as of
from . import gqa as og
from .numerics import bf16_bits_to_f32, f32_to_bf16_bits

HIDDEN = 5120
RMS_EPS = 1e-6


def bf16(x):
    """Round to bf16, returned as bits."""
    return f32_to_bf16_bits(np.asarray(x, np.float32))


def rms_norm_1p_bits(x_bits, w):
    x = bf16_bits_to_f32(x_bits).astype(np.float32)
    n = x * (np.float32(1.0) / np.sqrt((x * x).mean(-1, keepdims=True, dtype=np.float32) + np.float32(RMS_EPS)))
    return bf16((np.float32(1.0) + np.asarray(w, np.float32)) * n)


FP8_WEIGHTS = ("in_proj", "out_proj", "qkv_proj", "o_proj", "gate_up", "down")


def decode_weights(layers):
    """Decode every fp8 weight of the layer dicts to float32 [K, N] once (in place). Every
    e4m3fn value is exact in float32; a static model keeps them decoded across steps."""
    for L in layers:
        for nm in FP8_WEIGHTS:
            if nm in L and L[nm][0].dtype != np.float32:
                w, s = L[nm]
                L[nm] = (of.DECODE_LUT[np.asarray(w).view(np.uint8)].astype(np.float32), s)
    return layers


def linear(x_bits, wq):
    """bf16(x . W * scale). Raw fp8 bytes go through the pinned float64 oracle; decoded
    float32 weights (decode_weights) use a float32 product, whose relative error
    (about K * 2^-24 <= 1e-3 * 2^-9 for K <= 17408) is far below the bf16 rounding of the
    output."""
    w, s = wq
    s = np.asarray(s, np.float32).reshape(1, -1)
    if w.dtype == np.float32:
        x = bf16_bits_to_f32(x_bits).astype(np.float32)
        return bf16((x @ w) * s)
    return bf16(of.fp8_matmul(x_bits, w, s.reshape(-1)))


def add(a_bits, b_bits):
    return bf16(bf16_bits_to_f32(a_bits) + bf16_bits_to_f32(b_bits))


def deltanet_layer(L, x, B, T, hk, hv):
    return add(x, deltanet_mixer(L, x, B, T, hk, hv))


def deltanet_mixer(L, x, B, T, hk, hv):
    """The DeltaNet sublayer's output before the residual add (out_proj output bits);
    leaves (ckpt, mixed) in L["pending"] for the rollback."""
    h = rms_norm_1p_bits(x, L["in_norm"])
    proj = linear(h, L["in_proj"])
    qkv = (2 * hk + hv) * 128
    val = hv * 128
    mixed = proj[:, :qkv].reshape(B, T, qkv)
    z = proj[:, qkv:qkv + val].reshape(B, T, hv, 128)
    a = bf16_bits_to_f32(proj[:, qkv + val:qkv + val + hv]).reshape(B, T, hv)
    b = bf16_bits_to_f32(proj[:, qkv + val + hv:qkv + val + 2 * hv]).reshape(B, T, hv)
    ckpt, out = od.deltanet_verify(L["state"], mixed, L["conv_state"], L["conv_w"], L["conv_b"],
                                   a, b, z, L["A_log"], L["dt_bias"], L["norm_w"], hk, hv)
    L["pending"] = (ckpt, mixed)
    return linear(bf16(out.reshape(B * T, val)), L["out_proj"])


def gqa_layer(L, x, B, T, hq, hkv, kv_len, cos, sin):
    return add(x, gqa_mixer(L, x, B, T, hq, hkv, kv_len, cos, sin))


def gqa_mixer(L, x, B, T, hq, hkv, kv_len, cos, sin):
    """The attention sublayer's output before the residual add (o_proj output bits); the T
    key/value rows are written into L's cache at kv_len."""
    h = rms_norm_1p_bits(x, L["in_norm"])
    proj = linear(h, L["qkv_proj"])
    qg = proj[:, :hq * 512].reshape(B, T, hq, 512)
    query, gate = qg[..., :256], qg[..., 256:]
    kv = proj[:, hq * 512:].reshape(B, T, 2, hkv, 256)
    og.gqa_kv_append(kv[:, :, 0], kv[:, :, 1], L["k_norm"], cos, sin, L["cache_k"], L["cache_v"],
                     kv_len)
    attn = og.gqa_tail_verify(query, gate, L["q_norm"], cos, sin, L["cache_k"], L["cache_v"], kv_len)
    return linear(bf16(attn.reshape(B * T, hq * 256)), L["o_proj"])


def mlp(L, x, inter):
    return add(x, mlp_branch(L, x, inter))


def mlp_branch(L, x, inter):
    """SwiGLU as _mlp_layer (static_decode.py:951-963), before the residual add: gate, up
    and silu(gate) are bf16 tensors, so silu(gate) is rounded to bf16 before the product."""
    h = rms_norm_1p_bits(x, L["post_norm"])
    gu = bf16_bits_to_f32(linear(h, L["gate_up"])).astype(np.float32)
    g, u = gu[:, :inter], gu[:, inter:]
    s = bf16_bits_to_f32(bf16(g / (np.float32(1.0) + np.exp(-g)))).astype(np.float32)
    act = bf16(s * u)
    return linear(act, L["down"])


def verify_step(layers, x_bits, kv_len, B, T, target, draft, draft_ids, u_accept, u_sample,
                cos, sin, dn_heads=(16, 48), gqa_heads=(24, 4), inter=17408,
                layer_inputs=None, layer_outputs=None):
    """One verify + accept + rollback step. Returns (hidden bits [B*T, H], accepted, out_ids);
    layer states are updated in place (DeltaNet state = ckpt[accepted], conv rolled back,
    GQA caches written); kv_len is returned advanced as the 4th value.

    layer_inputs (optional): the residual stream entering each sublayer (mixer, then MLP,
    per layer), as bits; sublayer j then starts from layer_inputs[j] instead of sublayer
    j-1's output (teacher forcing, so a comparison measures each sublayer's own error
    instead of re-rounded differences carried through bf16 sublayers).
    layer_outputs (optional list): each sublayer's output is appended."""
    x = np.asarray(x_bits, np.uint16)
    j = 0
    for L in layers:
        for part in ("mixer", "mlp"):
            if layer_inputs is not None:
                x = np.asarray(layer_inputs[j], np.uint16)
            if part == "mlp":
                x = mlp(L, x, inter)
            elif L["kind"] == "D":
                x = deltanet_layer(L, x, B, T, *dn_heads)
            else:
                x = gqa_layer(L, x, B, T, *gqa_heads, kv_len, cos, sin)
            if layer_outputs is not None:
                layer_outputs.append(x)
            j += 1
    accepted, out_ids = oa.accept_rejection(target, draft, draft_ids, u_accept, u_sample, 1.0)
    for L in layers:
        if L["kind"] == "D":
            ckpt, mixed = L.pop("pending")
            L["state"], L["conv_state"] = od.deltanet_rollback(ckpt, mixed, L["conv_state"], accepted)
    return x, accepted, out_ids, np.asarray(kv_len) + accepted + 1
