"""Pins oracle/torch_step.py (the batched torch CPU float32 step the bench times as its CPU
baseline) against the numpy oracle (oracle/verify_step.py, oracle/accept.py):
- the whole step on the two HF-pinned layers of tests/golden/layers_hf.npz (a DeltaNet and an
  attention layer with their MLPs, B = 2 and 1, T = 8, nonzero states, KV prefix): every
  sublayer output within 2e-3 relative (float32 against float64 arithmetic between the same
  bf16 rounding points), rolled-back DeltaNet states within 1e-5, conv windows and appended
  cache rows within 2e-3, accepted lengths and tokens identical;
- rejection-sampling decisions (float64 probabilities) identical to the integer contract on
  correlated random logits, and the contract's special cases p == q (all accepted) and
  q(x) > 0 = p(x) (rejected).
"""
import numpy as np
import pytest
import torch

from oracle import accept as oa
from oracle import torch_step as ts
from oracle import verify_step as vs
from oracle.numerics import bf16_bits_to_f32 as b2f
from test_oracle_layers import FIXTURE, HKV, INTER, weights, with_state, rel

HEADS = dict(dn_heads=(1, 3), gqa_heads=(4, 2), inter=INTER)


def f32(bits):
    return torch.from_numpy(b2f(bits).astype(np.float32))


def torch_layers(fx, case):
    out = []
    for nm in ("dn", "at"):
        L, B, T, P = with_state(fx, case, weights(fx, nm))
        d = {"kind": L["kind"]}
        for k, v in L.items():
            if k == "kind":
                continue
            if isinstance(v, tuple):
                d[k] = (ts.decode_fp8(torch.from_numpy(v[0])), torch.from_numpy(v[1]))
            elif k == "conv_state":
                d[k] = f32(v)
            elif k in ("cache_k", "cache_v"):
                d[k] = torch.from_numpy(v.view(np.int16).copy()).view(torch.bfloat16)
            elif k == "state":
                d[k] = torch.from_numpy(v.astype(np.float32))
            else:
                d[k] = torch.from_numpy(np.asarray(v, np.float32))
        out.append(d)
    return out


def logits(B, K, V, seed, rho=0.8):
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(B, K + 1, V, generator=g)
    d = rho * t[:, :K] + (1 - rho * rho) ** 0.5 * torch.randn(B, K, V, generator=g)
    ids = torch.multinomial(torch.softmax(d, -1).reshape(B * K, V), 1, generator=g).reshape(B, K)
    return t, d, ids, torch.rand(B, K, generator=g), torch.rand(B, generator=g)


@pytest.mark.parametrize("case", ["b2p37", "b1p3"])
def test_step_matches_numpy_oracle(case):
    fx = dict(np.load(FIXTURE))
    B, T, P = (int(v) for v in fx[f"{case}/shape"])
    olayers = [with_state(fx, case, weights(fx, nm))[0] for nm in ("dn", "at")]
    tlayers = torch_layers(fx, case)
    x = fx[f"{case}/x0"]
    cos, sin = fx[f"{case}/cos"], fx[f"{case}/sin"]
    lg = logits(B, T - 1, 700, seed=B + P)
    outs = []
    _, oacc, oids, okv = vs.verify_step(olayers, x, np.full(B, P), B, T,
                                        *(v.numpy() for v in lg), cos, sin, layer_outputs=outs,
                                        **HEADS)
    # teacher forcing with the oracle's own residual stream, as the GPU step tests do
    ins = [x] + outs[:-1]
    touts = []
    kv = torch.full((B,), P, dtype=torch.int64)
    step = ts.TorchCpuStep(tlayers, B, T, **HEADS)
    _, tacc, tids = step.step(f32(x), kv, torch.from_numpy(cos), torch.from_numpy(sin), *lg,
                              layer_inputs=[f32(i) for i in ins], layer_outputs=touts)
    for i, (got, ref) in enumerate(zip(touts, outs)):
        d_ref = b2f(ref) - b2f(ins[i])
        d_got = got.numpy() - b2f(ins[i])
        assert rel(d_got, d_ref) < 2e-3, f"sublayer {i}"
    assert np.array_equal(tacc.numpy(), oacc) and np.array_equal(tids.numpy(), oids)
    assert np.array_equal(kv.numpy(), okv)
    D, G = olayers
    tD, tG = tlayers
    assert rel(tD["state"].numpy(), D["state"]) < 1e-5
    assert rel(tD["conv_state"].numpy(), b2f(D["conv_state"])) < 2e-3
    for nm in ("cache_k", "cache_v"):
        got = tG[nm].float().numpy()[:, :, P:P + T]
        assert rel(got, b2f(G[nm][:, :, P:P + T])) < 2e-3, nm


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_rejection_decisions_match_integer_contract(seed):
    lg = logits(48, 7, 3000, seed=seed)
    acc, ids = ts.accept_rejection(*lg)
    oacc, oids = oa.accept_rejection(*(v.numpy() for v in lg), 1.0)
    assert np.array_equal(acc.numpy(), oacc)
    assert np.array_equal(ids.numpy(), oids)
    assert 0 < acc.float().mean() < 7


def test_rejection_special_cases():
    t, _, ids, u, us = logits(8, 7, 500, seed=9)
    acc, _ = ts.accept_rejection(t, t[:, :7].clone(), ids, u, us)          # p == q
    assert (acc == 7).all()
    d = t[:, :7].clone()
    t2 = t.clone()
    t2[:, :7].scatter_(-1, ids[..., None], float("-inf"))                     # p(x) = 0 < q(x)
    acc, out = ts.accept_rejection(t2, d, ids, u, us)
    assert (acc == 0).all()
    assert (out[:, 0] != ids[:, 0]).all()
