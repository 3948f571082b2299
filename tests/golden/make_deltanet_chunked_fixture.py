#!/usr/bin/env python3
"""Writes tests/golden/deltanet_chunked_hf.npz: chunked gated-DeltaNet prefill vectors
computed with HF transformers' torch_chunk_gated_delta_rule (third-party; transformers
5.15.0, qwen3_next.modeling_qwen3_next), used to pin
oracle/deltanet_chunked.py.

Inputs per case (op layouts, head-major rows h*S + t): raw q, k [Hv*S, 128], v [Hv*S, 128],
g, beta [Hv*S, 1] with the model's gates g = -exp(A_log) * softplus(a + dt),
beta = sigmoid(b) (contrib/qwen3.6-27b/static_decode.py:628-629), initial state
[Hv*128, 128]. HF is run with use_qk_l2norm_in_kernel=True (its l2norm is
x * rsqrt(sum x^2 + 1e-6), as the reference kernel normalises) in float32.
Needs transformers; the tests read only the .npz it writes:
    python tests/golden/make_deltanet_chunked_fixture.py
"""
import os

import numpy as np
import torch
import torch.nn.functional as F
from transformers.models.qwen3_next import modeling_qwen3_next as hf

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "deltanet_chunked_hf.npz")
D = 128


def case(Hv, S, C, seed):
    g_ = torch.Generator().manual_seed(seed)
    q = torch.randn(S, Hv, D, generator=g_)
    k = torch.randn(S, Hv, D, generator=g_)
    v = torch.randn(S, Hv, D, generator=g_)
    A_log = torch.randn(Hv, generator=g_)
    dt = torch.randn(Hv, generator=g_) * 0.1
    a = torch.randn(S, Hv, generator=g_)
    b = torch.randn(S, Hv, generator=g_)
    g = -torch.exp(A_log) * F.softplus(a + dt)
    beta = torch.sigmoid(b)
    state = torch.randn(Hv, D, D, generator=g_) * 0.05
    out, fs = hf.torch_chunk_gated_delta_rule(
        q[None], k[None], v[None], g[None], beta[None], chunk_size=C,
        initial_state=state[None].clone(), output_final_state=True,
        use_qk_l2norm_in_kernel=True)
    hm = lambda t: t.transpose(0, 1).reshape(Hv * S, -1).contiguous().numpy().astype(np.float32)
    return {
        "q": hm(q), "k": hm(k), "v": hm(v), "g": hm(g[..., None]), "beta": hm(beta[..., None]),
        "state": state.reshape(Hv * D, D).numpy().astype(np.float32),
        "out": hm(out[0].float()), "new_state": fs[0].reshape(Hv * D, D).float().numpy(),
        "C": np.int64(C),
    }


def main():
    arrays = {}
    for i, (Hv, S, C, seed) in enumerate([(2, 48, 16, 0), (1, 100, 64, 1), (1, 37, 16, 2),
                                          (1, 70, 32, 3)]):
        for name, a in case(Hv, S, C, seed).items():
            arrays[f"c{i}_{name}"] = a
    np.savez_compressed(OUT, **arrays)
    print("wrote", OUT, sorted({k.split('_')[0] for k in arrays}))


if __name__ == "__main__":
    main()
