#!/usr/bin/env python3
"""Writes tests/golden/layers_hf.npz: T-token verify vectors of whole decoder layers computed
with HF transformers' Qwen3.5 modules (third-party; transformers 5.15.0:
Qwen3_5DecoderLayer with Qwen3_5GatedDeltaNet / Qwen3_5Attention / Qwen3_5MLP / Qwen3_5RMSNorm,
and their DynamicCache), used to pin the layer composition of oracle/verify_step.py.

Each case is a two-layer stack (a DeltaNet layer, then an attention layer, each with its MLP)
at reduced widths with the real head sizes (128 for DeltaNet, 256 for attention, 64 RoPE
dims), run in float32 on T verify tokens that continue a decode state:
  - the DeltaNet layer starts from a nonzero recurrent state and conv window, seeded into HF's
    cache (update_conv_state / update_recurrent_state), so HF takes its cached multi-token
    path (causal_conv1d over [cached window | new tokens], torch_chunk_gated_delta_rule with
    the initial state);
  - the attention layer starts from a KV prefix of P rows seeded into the cache (update), with
    an additive causal mask over the P + T keys and HF's rotary table at positions P..P+T-1.
Weights are built once as e4m3fn codes [K, N] with power-of-two per-channel scales, so the
dequantised weight decode(code) * 2^e is exact in float32 and bf16 and the HF linear layers
compute exactly the product the fp8 path computes. The projections keep the fused layouts of
the oracle ([qkv | z | a | b], [(query | gate) x Hq | key x Hkv | value x Hkv], [gate | up]),
split into HF's separate nn.Linear weights here. HF's conv1d has no bias; the conv bias of the
reference kernel is attached to it as a Parameter (causal_conv1d_fn passes conv1d.bias).

Each case runs twice:
  - float32 throughout ("dn/...", "at/..."): the output of each decoder layer
    (Qwen3_5DecoderLayer.forward), each mixer's output (forward hook on linear_attn /
    self_attn), the DeltaNet recurrent state and conv window after the T tokens, the appended
    key/value rows, and HF's cos/sin;
  - with bf16 rounding at the op boundaries of the reference's decode harness
    (contrib/qwen3.6-27b/static_decode.py: rms_norm :322-335, _deltanet_layer :753-847,
    _gqa_layer :849-949, _mlp_layer :951-963), applied to HF's modules by forward hooks
    ("r/..."): the outputs of the input / post-attention norms, of every projection
    (in_proj_qkv/z/a/b, out_proj, q/k/v/o_proj, gate/up/down_proj), of the gated norm, of
    silu(gate), of k_norm and of the key RoPE, and the inputs of o_proj, down_proj and the
    post-attention norm (the bf16 residual stream). Everything between those points (conv,
    l2norm, gates, the delta rule, attention softmax) stays float32 as in HF. This run
    records each mixer's output, the MLP's input and output per layer, the states and the
    appended rows.

Needs transformers; the tests read only the .npz it writes:
    python tests/golden/make_layer_fixture.py
"""
import os

import numpy as np
import torch
from transformers.cache_utils import DynamicCache
from transformers.models.qwen3_5 import modeling_qwen3_5 as hf
from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "layers_hf.npz")

H, HK, HV, D = 256, 1, 3, 128          # hidden, DeltaNet k / v heads (ratio 3), head dim
HQ, HKV, DH = 4, 2, 256                # attention q / kv heads (ratio 2), head dim
INTER = 512
QKV, VAL = (2 * HK + HV) * D, HV * D


def bits(t):
    return t.detach().to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def fp8_weight(n_out, k_in, g):
    """W ~ N(0, 0.02) [n_out, k_in] -> (codes [K, N] uint8 e4m3fn, scale [N] f32 = 2^e,
    dequantised [n_out, k_in] f32 = decode(code) * scale, exact)."""
    w = torch.randn(n_out, k_in, generator=g) * 0.02
    e = torch.floor(torch.log2(w.abs().amax(dim=1).clamp_min(1e-12) / 448.0))
    scale = torch.pow(2.0, e)
    q = (w / scale[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    deq = q.float() * scale[:, None]
    codes = q.view(torch.uint8).t().contiguous().numpy()
    return codes, scale.numpy().astype(np.float32), deq


def config():
    return Qwen3_5TextConfig(
        hidden_size=H, intermediate_size=INTER, num_hidden_layers=2,
        num_attention_heads=HQ, num_key_value_heads=HKV, head_dim=DH,
        linear_num_key_heads=HK, linear_num_value_heads=HV, linear_key_head_dim=D,
        linear_value_head_dim=D, linear_conv_kernel_dim=4, rms_norm_eps=1e-6,
        hidden_act="silu", attention_bias=False, max_position_embeddings=4096,
        layer_types=["linear_attention", "full_attention"],
        rope_parameters={"rope_type": "default", "rope_theta": 1e7, "partial_rotary_factor": 0.25},
        attn_implementation="eager")


def rnd(t):
    return t.to(torch.bfloat16).float()


def round_at_op_boundaries(dn, at, got):
    """Forward hooks that round to bf16 where the reference's decode harness holds bf16
    tensors, and capture into `got` each mixer's output, the residual stream entering each
    MLP (the post-attention norm's input, rounded: the harness's bf16 residual add) and each
    MLP's output."""
    hs = []

    def out_r(m, i, o):
        return rnd(o)

    def in_r(m, args):
        return (rnd(args[0]),) + tuple(args[1:])

    for nm, L in (("dn", dn), ("at", at)):
        hs.append(L.input_layernorm.register_forward_hook(out_r))
        hs.append(L.post_attention_layernorm.register_forward_pre_hook(
            lambda m, args, nm=nm: (got.__setitem__(f"{nm}/mlp_in", rnd(args[0])) or
                                    (got[f"{nm}/mlp_in"],) + tuple(args[1:]))))
        hs.append(L.post_attention_layernorm.register_forward_hook(out_r))
        mlp = L.mlp
        for mod in (mlp.gate_proj, mlp.up_proj, mlp.act_fn, mlp.down_proj):
            hs.append(mod.register_forward_hook(out_r))
        hs.append(mlp.down_proj.register_forward_pre_hook(in_r))
        hs.append(mlp.register_forward_hook(
            lambda m, i, o, nm=nm: got.__setitem__(f"{nm}/mlp_out", o)))
    la = dn.linear_attn
    for mod in (la.in_proj_qkv, la.in_proj_z, la.in_proj_a, la.in_proj_b, la.norm, la.out_proj):
        hs.append(mod.register_forward_hook(out_r))
    hs.append(la.register_forward_hook(lambda m, i, o: got.__setitem__("dn/mixer", o)))
    sa = at.self_attn
    for mod in (sa.q_proj, sa.k_proj, sa.v_proj, sa.k_norm, sa.o_proj):
        hs.append(mod.register_forward_hook(out_r))
    hs.append(sa.o_proj.register_forward_pre_hook(in_r))
    hs.append(sa.register_forward_hook(lambda m, i, o: got.__setitem__("at/mixer", o[0])))
    return hs


def case(B, T, P, seed, rec):
    """Adds case (B, T, P) to rec; the weights (under "w/") come from a fixed seed and are
    shared by every case, the decode state and inputs from `seed`."""
    g = torch.Generator().manual_seed(1234)
    cfg = config()
    dn = hf.Qwen3_5DecoderLayer(cfg, 0).float().eval()
    at = hf.Qwen3_5DecoderLayer(cfg, 1).float().eval()
    w = {}
    with torch.no_grad():
        for nm, L in (("dn", dn), ("at", at)):
            w_in = torch.randn(H, generator=g) * 0.1
            w_post = torch.randn(H, generator=g) * 0.1
            L.input_layernorm.weight.copy_(w_in)
            L.post_attention_layernorm.weight.copy_(w_post)
            w[f"{nm}/in_norm"], w[f"{nm}/post_norm"] = w_in.numpy(), w_post.numpy()
            c, s, deq = fp8_weight(2 * INTER, H, g)                       # [gate | up]
            L.mlp.gate_proj.weight.copy_(deq[:INTER])
            L.mlp.up_proj.weight.copy_(deq[INTER:])
            w[f"{nm}/gate_up"], w[f"{nm}/gate_up_scale"] = c, s
            c, s, deq = fp8_weight(H, INTER, g)
            L.mlp.down_proj.weight.copy_(deq)
            w[f"{nm}/down"], w[f"{nm}/down_scale"] = c, s
        la = dn.linear_attn
        c, s, deq = fp8_weight(QKV + VAL + 2 * HV, H, g)                  # [qkv | z | a | b]
        la.in_proj_qkv.weight.copy_(deq[:QKV])
        la.in_proj_z.weight.copy_(deq[QKV:QKV + VAL])
        la.in_proj_a.weight.copy_(deq[QKV + VAL:QKV + VAL + HV])
        la.in_proj_b.weight.copy_(deq[QKV + VAL + HV:])
        w["dn/in_proj"], w["dn/in_proj_scale"] = c, s
        c, s, deq = fp8_weight(H, VAL, g)
        la.out_proj.weight.copy_(deq)
        w["dn/out_proj"], w["dn/out_proj_scale"] = c, s
        conv_w = torch.randn(QKV, 4, generator=g) * 0.5
        conv_b = torch.randn(QKV, generator=g) * 0.1
        la.conv1d.weight.copy_(conv_w[:, None, :])
        la.conv1d.bias = torch.nn.Parameter(conv_b.clone())
        A_log = torch.randn(HV, generator=g) * 0.5
        dt_bias = torch.randn(HV, generator=g)
        norm_w = torch.randn(D, generator=g) * 0.1 + 1.0
        la.A_log.copy_(A_log)
        la.dt_bias.copy_(dt_bias)
        la.norm.weight.copy_(norm_w)
        w.update({"dn/conv_w": conv_w.numpy(), "dn/conv_b": conv_b.numpy(),
                    "dn/A_log": A_log.numpy(), "dn/dt_bias": dt_bias.numpy(),
                    "dn/norm_w": norm_w.numpy()})
        sa = at.self_attn
        c, s, deq = fp8_weight(HQ * 2 * DH + 2 * HKV * DH, H, g)          # [q+gate | k | v]
        sa.q_proj.weight.copy_(deq[:HQ * 2 * DH])
        sa.k_proj.weight.copy_(deq[HQ * 2 * DH:HQ * 2 * DH + HKV * DH])
        sa.v_proj.weight.copy_(deq[HQ * 2 * DH + HKV * DH:])
        w["at/qkv_proj"], w["at/qkv_proj_scale"] = c, s
        c, s, deq = fp8_weight(H, HQ * DH, g)
        sa.o_proj.weight.copy_(deq)
        w["at/o_proj"], w["at/o_proj_scale"] = c, s
        q_norm = torch.randn(DH, generator=g) * 0.1
        k_norm = torch.randn(DH, generator=g) * 0.1
        sa.q_norm.weight.copy_(q_norm)
        sa.k_norm.weight.copy_(k_norm)
        w["at/q_norm"], w["at/k_norm"] = q_norm.numpy(), k_norm.numpy()

        for k, v in w.items():
            if f"w/{k}" in rec:
                assert np.array_equal(rec[f"w/{k}"], v)
            rec[f"w/{k}"] = v
        out = {}
        g = torch.Generator().manual_seed(seed)
        # decode state: DeltaNet state and conv window, KV prefix (bf16 values)
        S0 = torch.randn(B, HV, D, D, generator=g) * 0.02
        conv3 = torch.randn(B, QKV, 3, generator=g).to(torch.bfloat16).float()
        kpre = torch.randn(B, HKV, P, DH, generator=g).to(torch.bfloat16).float()
        vpre = torch.randn(B, HKV, P, DH, generator=g).to(torch.bfloat16).float()
        x0 = torch.randn(B, T, H, generator=g).to(torch.bfloat16).float()
        out.update({"S0": S0.numpy(), "conv_state": bits(conv3), "cache_k": bits(kpre),
                    "cache_v": bits(vpre), "x0": bits(x0.reshape(B * T, H)),
                    "shape": np.array([B, T, P])})

        cache = DynamicCache(config=cfg)
        # the cached window holds the last 4 pre-conv inputs; only the last 3 reach the
        # outputs of the new tokens (kernel width 4)
        cache.update_conv_state(torch.cat([torch.zeros(B, QKV, 1), conv3], -1), 0)
        cache.update_recurrent_state(S0.clone(), 0)
        cache.update(kpre.clone(), vpre.clone(), 1)

        rot = hf.Qwen3_5TextRotaryEmbedding(cfg)
        pos = (P + torch.arange(T)).unsqueeze(0).expand(B, T)
        cos, sin = rot(x0, pos)
        out["cos"], out["sin"] = cos.numpy(), sin.numpy()
        mask = torch.full((T, P + T), float("-inf"))
        for t in range(T):
            mask[t, :P + t + 1] = 0.0
        mask = mask[None, None].expand(B, 1, T, P + T)

        mix = {}
        dn.linear_attn.register_forward_hook(lambda m, i, o: mix.__setitem__("dn", o))
        at.self_attn.register_forward_hook(lambda m, i, o: mix.__setitem__("at", o[0]))
        y0 = dn(x0, position_embeddings=(cos, sin), past_key_values=cache)
        x1 = y0.to(torch.bfloat16).float()        # the bf16 residual stream between layers
        y1 = at(x1, position_embeddings=(cos, sin), attention_mask=mask, past_key_values=cache)
        out.update({"dn/out": y0.reshape(B * T, H).numpy(),
                    "dn/mixer": mix["dn"].reshape(B * T, H).numpy(),
                    "at/in": bits(x1.reshape(B * T, H)),
                    "at/out": y1.reshape(B * T, H).numpy(),
                    "at/mixer": mix["at"].reshape(B * T, H).numpy(),
                    "S_final": cache.layers[0].recurrent_states[0].numpy(),
                    "conv_final": cache.layers[0].conv_states[0][..., 1:].numpy(),
                    "k_new": cache.layers[1].keys[:, :, P:].numpy(),
                    "v_new": cache.layers[1].values[:, :, P:].numpy()})
        # self-check of the hook bookkeeping (not of the oracle): the DecoderLayer output is
        # residual + mixer + MLP(post-norm) as HF composes it
        h = x0 + mix["dn"]
        chk = h + dn.mlp(dn.post_attention_layernorm(h))
        assert torch.allclose(chk, y0, rtol=0, atol=1e-5)

        # the same two layers with bf16 rounding at the reference harness's op boundaries
        cache = DynamicCache(config=cfg)
        cache.update_conv_state(torch.cat([torch.zeros(B, QKV, 1), conv3], -1), 0)
        cache.update_recurrent_state(S0.clone(), 0)
        cache.update(kpre.clone(), vpre.clone(), 1)
        got = {}
        handles = round_at_op_boundaries(dn, at, got)
        rope = hf.apply_rotary_pos_emb

        def rope_rounding_k(q, k, c, s_, unsqueeze_dim=1):
            qe, ke = rope(q, k, c, s_, unsqueeze_dim)
            return qe, rnd(ke)

        hf.apply_rotary_pos_emb = rope_rounding_k
        try:
            dn(x0, position_embeddings=(cos, sin), past_key_values=cache)
            x1r = rnd(got["dn/mlp_in"] + got["dn/mlp_out"])     # the harness's bf16 residual add
            at(x1r, position_embeddings=(cos, sin), attention_mask=mask, past_key_values=cache)
        finally:
            hf.apply_rotary_pos_emb = rope
            for hd in handles:
                hd.remove()
        for k in ("dn/mixer", "dn/mlp_in", "dn/mlp_out", "at/mixer", "at/mlp_in", "at/mlp_out"):
            out[f"r/{k}"] = bits(got[k].reshape(B * T, H))
        out["r/at/in"] = bits(x1r.reshape(B * T, H))
        out["r/S_final"] = cache.layers[0].recurrent_states[0].numpy()
        out["r/conv_final"] = bits(cache.layers[0].conv_states[0][..., 1:])
        out["r/k_new"] = bits(cache.layers[1].keys[:, :, P:])
        out["r/v_new"] = bits(cache.layers[1].values[:, :, P:])
    rec.update({f"b{B}p{P}/{k}": v for k, v in out.items()})


def main():
    rec = {}
    case(2, 8, 37, seed=5, rec=rec)
    case(1, 8, 3, seed=6, rec=rec)
    np.savez_compressed(OUT, **rec)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
