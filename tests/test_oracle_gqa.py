"""CPU pinning of oracle/gqa.py.

- gqa_tail against the inline mirror of _gqa_layer's tail that gqa_tail_ref's own check
  uses (contrib/qwen3.6-27b/kernels/gqa_tail_ref.py:73-102: seed 0, B=8, S=128, position
  100, bar 1e-4), restated with torch ops;
- gqa_tail_verify against torch scaled_dot_product_attention (fp64, explicit boolean mask)
  and a brute-force per-row loop on tiny shapes;
- decode tail == verify tail at T=1 with a prefix mask;
- append-after-attention (contrib/qwen3.6-35b-a3b/kernels/tests/
  test_gqa_stateful_cache_cpu.py:9-40): rows written by gqa_kv_append then attended ==
  attention over a cache written by plain torch ops;
- RoPE: rope_partial against torch rotate_half on random vectors, and the cos/sin table
  against the reference's fp32 table recipe.
"""
import math

import numpy as np
import torch
import torch.nn.functional as F

from oracle import gqa as og
from oracle.numerics import bf16_bits_to_f32
from _util import bits, gqa_verify_inputs


def test_tail_matches_layer_mirror_seed0():
    torch.manual_seed(0)
    B, S, HQ = 8, 128, 6
    query = torch.randn(B, HQ, 256)
    gate = torch.randn(B, HQ, 256)
    q_norm = torch.randn(256) * 0.1
    cos = torch.randn(64)
    sin = torch.randn(64)
    ck = torch.randn(B, S, 256)
    cv = torch.randn(B, S, 256)
    mask = (torch.arange(S) <= 100).float()
    got = og.gqa_tail(query.reshape(B * HQ, 256).numpy(), gate.reshape(B * HQ, 256).numpy(),
                      q_norm.numpy(), cos.numpy(), sin.numpy(), ck.reshape(B * S, 256).numpy(),
                      cv.reshape(B * S, 256).numpy(), mask.reshape(1, S).numpy())
    # mirror of the reference layer's tail (query already projected, cache already written)
    x = query.double()
    qn = (1.0 + q_norm.double()) * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6))
    rot, pas = qn[..., :64], qn[..., 64:]
    rh = torch.cat((-rot[..., 32:], rot[..., :32]), -1)
    qr = torch.cat((rot * cos.double() + rh * sin.double(), pas), -1)
    sc = torch.matmul(qr, ck.double().transpose(1, 2)) / 16.0 + (1.0 - mask.double()) * -1e9
    ao = torch.matmul(F.softmax(sc, -1), cv.double()) * torch.sigmoid(gate.double())
    assert np.abs(got - ao.reshape(B * HQ, 256).numpy()).max() < 1e-4


def _sdpa_verify(d):
    q = bf16_bits_to_f32(bits(d["query"])).astype(np.float64)
    B, T, Hq, Dh = q.shape
    Hkv = d["cache_k"].shape[1]
    grp = Hq // Hkv
    qn = og.rope_partial(og.rms_norm_1p(q, d["q_norm"].numpy()),
                         d["cos"].numpy()[:, :, None, :], d["sin"].numpy()[:, :, None, :])
    out = np.empty_like(qn)
    for b in range(B):
        L = int(d["kv_len"][b]) + T
        k = torch.from_numpy(bf16_bits_to_f32(bits(d["cache_k"][b, :, :L])).astype(np.float64))
        v = torch.from_numpy(bf16_bits_to_f32(bits(d["cache_v"][b, :, :L])).astype(np.float64))
        k = k.repeat_interleave(grp, 0)                                  # [Hq, L, Dh]
        v = v.repeat_interleave(grp, 0)
        qq = torch.from_numpy(qn[b]).transpose(0, 1)                     # [Hq, T, Dh]
        mask = torch.arange(L)[None, :] <= (int(d["kv_len"][b]) + torch.arange(T))[:, None]
        o = F.scaled_dot_product_attention(qq, k, v, attn_mask=mask)
        out[b] = o.transpose(0, 1).numpy()
    gate = bf16_bits_to_f32(bits(d["gate"])).astype(np.float64)
    return out / (1 + np.exp(-gate))


def test_verify_matches_sdpa():
    d = gqa_verify_inputs(2, 4, 6, 2, [0, 37], 64, seed=5)
    got = og.gqa_tail_verify(bits(d["query"]), bits(d["gate"]), d["q_norm"].numpy(),
                             d["cos"].numpy(), d["sin"].numpy(), bits(d["cache_k"]),
                             bits(d["cache_v"]), d["kv_len"].numpy())
    np.testing.assert_allclose(got, _sdpa_verify(d), rtol=1e-10, atol=1e-12)


def test_verify_brute_force_row():
    d = gqa_verify_inputs(1, 3, 4, 1, [5], 16, seed=6)
    got = og.gqa_tail_verify(bits(d["query"]), bits(d["gate"]), d["q_norm"].numpy(),
                             d["cos"].numpy(), d["sin"].numpy(), bits(d["cache_k"]),
                             bits(d["cache_v"]), d["kv_len"].numpy())
    q = bf16_bits_to_f32(bits(d["query"]))[0].astype(np.float64)
    K = bf16_bits_to_f32(bits(d["cache_k"]))[0, 0].astype(np.float64)
    V = bf16_bits_to_f32(bits(d["cache_v"]))[0, 0].astype(np.float64)
    g = bf16_bits_to_f32(bits(d["gate"]))[0].astype(np.float64)
    w = d["q_norm"].numpy().astype(np.float64)
    for t in range(3):
        for h in range(4):
            x = q[t, h]
            xn = (1 + w) * x / math.sqrt((x * x).mean() + 1e-6)
            c, s = d["cos"].numpy()[0, t].astype(np.float64), d["sin"].numpy()[0, t].astype(np.float64)
            r = xn.copy()
            for i in range(64):
                partner = -xn[i + 32] if i < 32 else xn[i - 32]
                r[i] = xn[i] * c[i] + partner * s[i]
            sc = [float(r @ K[j]) / 16.0 for j in range(5 + t + 1)]
            m = max(sc)
            p = [math.exp(v - m) for v in sc]
            o = sum(pi * V[j] for j, pi in enumerate(p)) / sum(p)
            ref = o / (1 + np.exp(-g[t, h]))
            np.testing.assert_allclose(got[0, t, h], ref, rtol=1e-10, atol=1e-12)


def test_decode_tail_equals_verify_t1():
    d = gqa_verify_inputs(3, 1, 6, 1, [10, 20, 30], 64, seed=7)
    pos = 25
    d["kv_len"][:] = pos
    cos, sin = og.rope_cos_sin(np.array([pos]))
    d["cos"] = torch.from_numpy(np.broadcast_to(cos, (3, 1, 64)).copy())
    d["sin"] = torch.from_numpy(np.broadcast_to(sin, (3, 1, 64)).copy())
    ver = og.gqa_tail_verify(bits(d["query"]), bits(d["gate"]), d["q_norm"].numpy(),
                             d["cos"].numpy(), d["sin"].numpy(), bits(d["cache_k"]),
                             bits(d["cache_v"]), d["kv_len"].numpy())
    S = 64
    mask = (np.arange(S) <= pos).astype(np.float32).reshape(1, S)
    dec = og.gqa_tail(bf16_bits_to_f32(bits(d["query"])).reshape(3 * 6, 256),
                      bf16_bits_to_f32(bits(d["gate"])).reshape(3 * 6, 256), d["q_norm"].numpy(),
                      cos, sin, bf16_bits_to_f32(bits(d["cache_k"])).reshape(3 * S, 256),
                      bf16_bits_to_f32(bits(d["cache_v"])).reshape(3 * S, 256), mask)
    np.testing.assert_allclose(ver.reshape(18, 256), dec, rtol=1e-9, atol=1e-12)


def test_append_then_attend_equals_cloned_cache():
    B, T, Hkv, S = 2, 3, 2, 32
    g = torch.Generator().manual_seed(8)
    key = torch.randn(B, T, Hkv, 256, generator=g).to(torch.bfloat16)
    value = torch.randn(B, T, Hkv, 256, generator=g).to(torch.bfloat16)
    k_norm = torch.randn(256, generator=g) * 0.1
    d = gqa_verify_inputs(B, T, 4, Hkv, [4, 17], S, seed=9)
    ck, cv = bits(d["cache_k"]).copy(), bits(d["cache_v"]).copy()
    og.gqa_kv_append(bits(key), bits(value), k_norm.numpy(), d["cos"].numpy(), d["sin"].numpy(),
                     ck, cv, d["kv_len"].numpy())
    # plain torch: _gqa_layer's rms_norm (bf16 out) + apply_rope (bf16 out) + row writes
    ref_k, ref_v = d["cache_k"].clone(), d["cache_v"].clone()
    xf = key.float()
    n = ((1.0 + k_norm) * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6))).to(torch.bfloat16)
    rot = n[..., :64]
    rh = torch.cat((-rot[..., 32:], rot[..., :32]), -1)
    c, s = d["cos"].unsqueeze(2), d["sin"].unsqueeze(2)
    kr = torch.cat((rot * c + rh * s, n[..., 64:].float()), -1).to(torch.bfloat16)
    for b in range(B):
        p0 = int(d["kv_len"][b])
        ref_k[b, :, p0:p0 + T] = kr[b].transpose(0, 1)
        ref_v[b, :, p0:p0 + T] = value[b].transpose(0, 1)
    assert np.array_equal(cv, bits(ref_v))
    diff = np.abs(ck.astype(np.int32) - bits(ref_k).astype(np.int32))
    assert diff.max() <= 1 and (diff > 0).mean() < 0.01     # fp32 rsqrt vs 1/sqrt: 1 ulp at most
    untouched = np.ones(S, bool)
    for b in range(B):
        p0 = int(d["kv_len"][b])
        m = untouched.copy()
        m[p0:p0 + T] = False
        assert np.array_equal(ck[b][:, m], bits(d["cache_k"])[b][:, m])


def test_rope_against_torch_rotate_half():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 256))
    cos, sin = og.rope_cos_sin(np.arange(5) * 977)
    got = og.rope_partial(x, cos, sin)
    xt = torch.from_numpy(x)
    rot = xt[..., :64]
    rh = torch.cat((-rot[..., 32:], rot[..., :32]), -1)
    ref = torch.cat((rot * torch.from_numpy(cos).double() + rh * torch.from_numpy(sin).double(),
                     xt[..., 64:]), -1)
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-14)
    # table: reference recipe in torch fp32
    inv = 1.0 / (1e7 ** (torch.arange(0, 64, 2).float() / 64))
    fr = torch.outer(torch.arange(5).float() * 977, inv)
    emb = torch.cat([fr, fr], -1)
    # inv_freq may differ by 1 fp32 ulp between the two recipes: angle error <= pos * 2^-23
    tol = 4 * 977 * 2.0 ** -23 + 1e-6
    np.testing.assert_allclose(cos, emb.cos().numpy(), rtol=0, atol=tol)
    np.testing.assert_allclose(sin, emb.sin().numpy(), rtol=0, atol=tol)
