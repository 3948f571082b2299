#!/usr/bin/env python3
"""Writes tests/golden/deltanet_hf.npz: multi-token gated-DeltaNet vectors computed with
HF transformers' Qwen3.5 reference functions (third-party; transformers 5.15.0), used
to pin oracle/deltanet.py.

  conv      transformers ... qwen3_5.modeling_qwen3_5.causal_conv1d_update (activation silu)
  recurrence torch_recurrent_gated_delta_rule(use_qk_l2norm_in_kernel=True), run on every
            prefix 1..T to get the state after each token
  output    Qwen3_5RMSNormGated on fp32 inputs (weight * rmsnorm(o) * silu(z))

Gates follow the reference kernel: g = -exp(A_log) * softplus(a + dt_bias), beta = sigmoid(b)
(contrib/qwen3.6-27b/kernels/deltanet_full.py:174-212). Needs transformers; the tests
read only the .npz it writes: python tests/golden/make_deltanet_fixture.py
"""
import os

import numpy as np
import torch
import torch.nn.functional as F
from transformers.models.qwen3_5 import modeling_qwen3_5 as hf

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "deltanet_hf.npz")


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def case(B, T, Hk, Hv, D, seed):
    g = torch.Generator().manual_seed(seed)
    QKV = (2 * Hk + Hv) * D
    state = torch.randn(B, Hv, D, D, generator=g) * 0.05
    mixed = torch.randn(B, T, QKV, generator=g).to(torch.bfloat16)
    conv_state = torch.randn(B, QKV, 3, generator=g).to(torch.bfloat16)
    conv_w = torch.randn(QKV, 4, generator=g) * 0.5
    conv_b = torch.randn(QKV, generator=g) * 0.1
    a = torch.randn(B, T, Hv, generator=g)
    b = torch.randn(B, T, Hv, generator=g)
    z = torch.randn(B, T, Hv, D, generator=g).to(torch.bfloat16)
    A_log = torch.randn(Hv, generator=g) * 0.5
    dt_bias = torch.randn(Hv, generator=g)
    norm_w = torch.randn(D, generator=g) * 0.1 + 1.0

    cs = conv_state.float().clone()
    y = hf.causal_conv1d_update(mixed.float().transpose(1, 2), cs, conv_w, conv_b, "silu")
    y = y.transpose(1, 2)                                             # [B, T, QKV]
    q = y[..., :Hk * D].reshape(B, T, Hk, D)
    k = y[..., Hk * D:2 * Hk * D].reshape(B, T, Hk, D)
    v = y[..., 2 * Hk * D:].reshape(B, T, Hv, D)
    rep = Hv // Hk
    q = q.repeat_interleave(rep, dim=2)
    k = k.repeat_interleave(rep, dim=2)
    gate = -A_log.exp() * F.softplus(a + dt_bias)                      # [B, T, Hv]
    beta = torch.sigmoid(b)
    ckpt = torch.empty(B, T, Hv, D, D)
    core = None
    for t in range(1, T + 1):
        o, s = hf.torch_recurrent_gated_delta_rule(q[:, :t], k[:, :t], v[:, :t], gate[:, :t],
                                                   beta[:, :t], state.clone(), True,
                                                   use_qk_l2norm_in_kernel=True)
        ckpt[:, t - 1] = s
        core = o                                                      # [B, t, Hv, D]
    norm = hf.Qwen3_5RMSNormGated(D, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(norm_w)
        out = norm(core.reshape(-1, D), z.float().reshape(-1, D)).reshape(B, T, Hv, D)
    return dict(state=state.numpy(), mixed_qkv=bits(mixed), conv_state=bits(conv_state),
                conv_weight=conv_w.numpy(), conv_bias=conv_b.numpy(), a_out=a.numpy(),
                b_out=b.numpy(), z=bits(z), A_log=A_log.numpy(), dt_bias=dt_bias.numpy(),
                norm_weight=norm_w.numpy(), ckpt=ckpt.numpy(), out=out.numpy(),
                conv_final=bits(cs.to(torch.bfloat16)), heads=np.array([Hk, Hv, D]))


def main():
    cases = {"d16": case(2, 5, 2, 4, 16, seed=7), "d32": case(1, 8, 1, 3, 32, seed=8)}
    flat = {f"{name}/{k}": v for name, d in cases.items() for k, v in d.items()}
    np.savez_compressed(OUT, **flat)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
