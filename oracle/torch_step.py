"""Batched PyTorch CPU (float32) restatement of the verify step: the CPU baseline that the
bench times beside the GPU step (test infrastructure only).

The composition and the bf16 rounding points are those of oracle/verify_step.py (which follows
contrib/qwen3.6-27b/static_decode.py: rms_norm :322-335, _deltanet_layer :753-847,
_gqa_layer :849-949, _mlp_layer :951-963), but the step runs batched over all B sequences in
float32 on torch's CPU kernels (BLAS GEMMs, vectorised elementwise ops, all host threads),
the way a CPU implementation of the step would run, instead of the float64 per-sequence
oracle:
- projections: bf16(x @ W * s), the fp8 weights decoded to float32 once (a static model
  keeps them decoded);
- DeltaNet: the width-4 conv over [window | tokens] (unfold), l2-normalised q, k, the gates,
  the delta rule on [B, Hv, 128, 128] float32 states, all T checkpoints kept, the gated
  RMSNorm (test_deltanet_full.py:20-54 per token);
- attention: keys normed, roped and rounded as the cache append does, then per sequence the
  T queries against its kv_len + T rows (scaled_dot_product_attention in float32 with the
  causal tail mask, kv heads shared by groups of q heads), times sigmoid(gate);
- acceptance: rejection sampling on float64 softmax probabilities. u is read as
  floor(u * 2^24) / 2^24 and the token is drawn by the same inverse-CDF rule as the
  integer contract of oracle/accept.py, so the decisions agree with it except where the two
  sides of an accept test lie within float64 rounding of each other;
- rollback: state = checkpoint[accepted], conv window = the last 3 of [window | tokens
  0..accepted], KV lengths += accepted + 1.

Pinned by tests/test_oracle_torch_step.py against oracle/verify_step.py (sublayer outputs on
the HF-pinned layer fixture, states, cache rows) and oracle/accept.py (decisions).
"""
import math

import torch
import torch.nn.functional as F

RMS_EPS = 1e-6
U_ONE = float(1 << 24)
D = 128


def bf16r(x):
    return x.to(torch.bfloat16).float()


def decode_fp8(w):
    """[K, N] e4m3fn bytes (int8 or uint8 tensor) -> float32 [K, N] (exact)."""
    return w.contiguous().view(torch.float8_e4m3fn).float()


def rms_norm_1p(x, w):
    return bf16r(x * (1.0 / torch.sqrt(x.pow(2).mean(-1, keepdim=True) + RMS_EPS)) * (1.0 + w))


def linear(x, wq):
    w, s = wq
    return bf16r((x @ w) * s)


def deltanet_mixer(L, h, B, T, hk, hv):
    """h: the layer's input residual [B*T, H] (bf16 values in float32). Returns the mixer
    output [B*T, H] and (ckpt [B, T, Hv, D, D], mixed [B, T, QKV]) for the rollback."""
    qkv, val = (2 * hk + hv) * D, hv * D
    proj = linear(rms_norm_1p(h, L["in_norm"]), L["in_proj"])
    mixed = proj[:, :qkv].reshape(B, T, qkv)
    z = proj[:, qkv:qkv + val].reshape(B, T, hv, D)
    a = proj[:, qkv + val:qkv + val + hv].reshape(B, T, hv)
    b = proj[:, qkv + val + hv:qkv + val + 2 * hv].reshape(B, T, hv)
    seq = torch.cat([L["conv_state"], mixed.transpose(1, 2)], -1)          # [B, QKV, 3+T]
    y = (seq.unfold(-1, 4, 1) * L["conv_w"][None, :, None, :]).sum(-1)      # [B, QKV, T]
    y = F.silu(y + L["conv_b"][None, :, None]).transpose(1, 2)               # [B, T, QKV]
    grp = hv // hk
    q = y[..., :hk * D].reshape(B, T, hk, D)
    k = y[..., hk * D:2 * hk * D].reshape(B, T, hk, D)
    v = y[..., 2 * hk * D:].reshape(B, T, hv, D)
    q = q / torch.sqrt(q.pow(2).sum(-1, keepdim=True) + RMS_EPS) * (1.0 / math.sqrt(D))
    k = k / torch.sqrt(k.pow(2).sum(-1, keepdim=True) + RMS_EPS)
    q = q.repeat_interleave(grp, dim=2)
    k = k.repeat_interleave(grp, dim=2)
    decay = torch.exp(-torch.exp(L["A_log"]) * F.softplus(a + L["dt_bias"]))  # [B, T, Hv]
    beta = torch.sigmoid(b)
    # (sequence, head) pairs as one batch of N = B * Hv [D, D] states
    N = B * hv
    S = L["state"].reshape(N, D, D).clone()
    ckpt = torch.empty(B, T, hv, D, D)
    out = torch.empty(B, T, hv, D)
    for t in range(T):
        S.mul_(decay[:, t].reshape(N, 1, 1))
        kt = k[:, t].reshape(N, 1, D)
        kv = torch.bmm(kt, S).reshape(B, hv, D)                              # S^T k
        delta = ((v[:, t] - kv) * beta[:, t, :, None]).reshape(N, 1, D)
        S.baddbmm_(kt.transpose(1, 2), delta)                                 # S += k delta^T
        out[:, t] = torch.bmm(q[:, t].reshape(N, 1, D), S).reshape(B, hv, D)  # S^T q
        ckpt[:, t] = S.reshape(B, hv, D, D)
    o = out * torch.rsqrt(out.pow(2).mean(-1, keepdim=True) + RMS_EPS) * L["norm_w"] * F.silu(z)
    return linear(bf16r(o.reshape(B * T, val)), L["out_proj"]), (ckpt, mixed)


def _rope(x, cos, sin):
    r = x[..., :64]
    rot = torch.cat([-r[..., 32:], r[..., :32]], -1)
    return torch.cat([r * cos + rot * sin, x[..., 64:]], -1)


def gqa_mixer(L, h, B, T, hq, hkv, kv_len, cos, sin):
    """h [B*T, H]; kv_len [B] (int tensor); cos, sin [B, T, 64]. Appends the T rows to
    L["cache_k"] / L["cache_v"] ([B, Hkv, S, 256] bf16) and returns the mixer output."""
    dh = 256
    proj = linear(rms_norm_1p(h, L["in_norm"]), L["qkv_proj"])
    qg = proj[:, :hq * 2 * dh].reshape(B, T, hq, 2 * dh)
    query, gate = qg[..., :dh], qg[..., dh:]
    kv = proj[:, hq * 2 * dh:].reshape(B, T, 2, hkv, dh)
    key, value = kv[:, :, 0], kv[:, :, 1]
    c, s = cos[:, :, None, :], sin[:, :, None, :]
    k1 = bf16r(key * (1.0 / torch.sqrt(key.pow(2).mean(-1, keepdim=True) + RMS_EPS))
               * (1.0 + L["k_norm"]))
    k2 = _rope(k1, c, s).to(torch.bfloat16)                                  # [B, T, Hkv, dh]
    qn = query * torch.rsqrt(query.pow(2).mean(-1, keepdim=True) + RMS_EPS) * (1.0 + L["q_norm"])
    qr = _rope(qn, c, s)                                                     # [B, T, Hq, dh]
    out = torch.empty(B, T, hq, dh)
    grp = hq // hkv
    for bi in range(B):
        p0 = int(kv_len[bi])
        L["cache_k"][bi, :, p0:p0 + T] = k2[bi].transpose(0, 1)
        L["cache_v"][bi, :, p0:p0 + T] = value[bi].transpose(0, 1).to(torch.bfloat16)
        n = p0 + T
        kk = L["cache_k"][bi, :, :n].float()                                 # [Hkv, n, dh]
        vv = L["cache_v"][bi, :, :n].float()
        mask = torch.arange(n)[None, :] <= (p0 + torch.arange(T))[:, None]   # [T, n]
        qb = qr[bi].transpose(0, 1)                                          # [Hq, T, dh]
        o = F.scaled_dot_product_attention(
            qb.reshape(hkv, grp * T, dh), kk, vv,
            attn_mask=mask.repeat(grp, 1)[None], scale=1.0 / math.sqrt(dh))
        out[bi] = o.reshape(hq, T, dh).transpose(0, 1)
    out = out * torch.sigmoid(gate)
    return linear(bf16r(out.reshape(B * T, hq * dh)), L["o_proj"])


def mlp_branch(L, h, inter):
    hn = rms_norm_1p(h, L["post_norm"])
    gu = linear(hn, L["gate_up"])
    g, u = gu[:, :inter], gu[:, inter:]
    return linear(bf16r(bf16r(F.silu(g)) * u), L["down"])


def accept_rejection(target, draft, draft_ids, u_accept, u_sample):
    """target [B, K+1, V], draft [B, K, V] float32, draft_ids [B, K], u [B, K], us [B] ->
    (accepted [B] int32, out_ids [B, K+1] int64) at temperature 1."""
    B, T, V = target.shape
    K = T - 1
    p = torch.softmax(target.double(), -1)
    q = torch.softmax(draft.double(), -1)
    ids = draft_ids.long()
    px = p[:, :K].gather(-1, ids[..., None])[..., 0]
    qx = q.gather(-1, ids[..., None])[..., 0]
    U = torch.floor(u_accept.double() * U_ONE) / U_ONE
    rejected = U * qx > px                                                   # [B, K]
    first = torch.where(rejected.any(1), rejected.int().argmax(1), torch.full((B,), K))
    accepted = first.to(torch.int32)
    out = torch.full((B, T), -1, dtype=torch.int64)
    Us = torch.floor(u_sample.double() * U_ONE) / U_ONE
    for b in range(B):
        a = int(first[b])
        out[b, :a] = ids[b, :a]
        w = (p[b, a] - q[b, a]).clamp_min(0.0) if a < K else p[b, K]
        c = torch.cumsum(w, 0)
        out[b, a] = int(torch.searchsorted(c, Us[b] * c[-1], right=True).clamp_max(V - 1))
    return accepted, out


class TorchCpuStep:
    """The verify step over layer dicts of CPU tensors (float32 weights decoded once; norms and
    DeltaNet parameters float32; state [B, Hv, D, D] float32, conv_state [B, QKV, 3] float32
    holding bf16 values, caches [B, Hkv, S, 256] bf16)."""

    def __init__(self, layers, B, T, dn_heads=(16, 48), gqa_heads=(24, 4), inter=17408):
        self.layers, self.B, self.T = layers, B, T
        self.dn_heads, self.gqa_heads, self.inter = dn_heads, gqa_heads, inter

    def step(self, x, kv_len, cos, sin, target, draft, draft_ids, u_accept, u_sample,
             layer_inputs=None, layer_outputs=None):
        """x [B*T, H] (bf16 values, float32). Returns (hidden, accepted, out_ids); the layer
        states are rolled back in place and kv_len (int64 tensor) advanced in place.
        layer_inputs / layer_outputs: as oracle.verify_step.verify_step."""
        B, T = self.B, self.T
        h = x
        pending = []
        j = 0
        for L in self.layers:
            for part in ("mixer", "mlp"):
                if layer_inputs is not None:
                    h = layer_inputs[j]
                if part == "mlp":
                    d = mlp_branch(L, h, self.inter)
                elif L["kind"] == "D":
                    d, pend = deltanet_mixer(L, h, B, T, *self.dn_heads)
                    pending.append((L, pend))
                else:
                    d = gqa_mixer(L, h, B, T, *self.gqa_heads, kv_len, cos, sin)
                h = bf16r(h + d)
                if layer_outputs is not None:
                    layer_outputs.append(h)
                j += 1
        accepted, out_ids = accept_rejection(target, draft, draft_ids, u_accept, u_sample)
        acc = accepted.long()
        bidx = torch.arange(B)
        for L, (ckpt, mixed) in pending:
            L["state"] = ckpt[bidx, acc]
            seq = torch.cat([L["conv_state"], mixed.transpose(1, 2)], -1)
            L["conv_state"] = torch.stack([seq[b, :, int(acc[b]) + 1:int(acc[b]) + 4]
                                           for b in range(B)])
        kv_len += acc + 1
        return h, accepted, out_ids
