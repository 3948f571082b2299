"""End-to-end GPU parity of the verify step (neuron-pytorch-native_amd/spec_verify_step.py:
fp8 projections, fused residual norms, DeltaNet verify, GQA append + verify attention,
SwiGLU, rejection sampling, rollback) against the oracle composition
(oracle/verify_step.py) on the same weights, states, caches, logits and uniforms, over two
consecutive steps, so the second step starts from the index-based DeltaNet rollback and the
advanced KV lengths of the first.

A 2-layer slice (one DeltaNet and one GQA layer, each with its MLP) at whole-model widths,
B = 2, K = 7, short caches, vocabulary 1000. Each sublayer (mixer, MLP) of the oracle starts
from the device's residual stream entering it (teacher forcing): through bf16-rounded
sublayers, rare one-ulp differences in one output perturb every element of the next
projection a little, and its bf16 rounding turns that into one-ulp differences in a large
share of elements, so free-running hiddens drift apart by about a bf16 ulp whatever the
kernels' accuracy (measured: 3e-4 after the first sublayer, 2e-3 after the second, 4.5e-3
after four); forcing measures each sublayer's own error.
Bars: accepted lengths and token ids bit-exact; each sublayer's output, the DeltaNet states
after rollback, conv windows and the appended cache rows within 2e-3 relative
(tests/_util.py). The elementwise term allows one bf16 ulp per bf16 rounding on a value's
path, since a flip of any of them shifts what follows by up to an ulp (2^-7 relative at the
bottom of a binade): conv windows are copies of one rounded projection output (ONE_ULP);
sublayer outputs (projection, silu, product, down projection, residual sum) and appended key
rows (projection, norm, RoPE) pass through up to four (CHAIN_ULPS = 4 ulps). For a sublayer
output (input + delta) the ulps are taken of |input| + |delta|, the operands' magnitude,
which is larger than the output's where the two cancel. A wiring mistake
(wrong slice, weight or layout) shows as O(1) errors under either bar.
Cache rows outside the appended ones keep their values from before the step.
"""
import numpy as np
import pytest
import torch

from oracle import verify_step as ovs
from oracle.numerics import bf16_bits_to_f32
from _util import assert_rel_close, bits

pytestmark = pytest.mark.gpu

ONE_ULP = 2.0 ** -7
CHAIN_ULPS = 4 * ONE_ULP


def _oracle_layers(model, B):
    from spec_verify_step import DN_HV, DN_QKV
    layers = []
    for L in model.layers:
        d = {"kind": L["kind"], "in_norm": L["in_norm"].cpu().numpy(),
             "post_norm": L["post_norm"].cpu().numpy()}
        for nm in ovs.FP8_WEIGHTS:
            if nm in L:
                d[nm] = (L[nm][0].cpu().numpy(), L[nm][1].cpu().numpy().reshape(-1))
        if L["kind"] == "D":
            for nm in ("conv_w", "conv_b", "A_log", "dt_bias", "norm_w"):
                d[nm] = L[nm].cpu().numpy()
            d["state"] = L["state"].cpu().double().numpy().reshape(B, DN_HV, 128, 128)
            d["conv_state"] = bits(L["conv_state"]).reshape(B, DN_QKV, 3).copy()
        else:
            d["q_norm"], d["k_norm"] = L["q_norm"].cpu().numpy(), L["k_norm"].cpu().numpy()
            d["cache_k"] = bits(L["cache_k"]).copy()
            d["cache_v"] = bits(L["cache_v"]).copy()
        layers.append(d)
    return ovs.decode_weights(layers)


def test_two_steps_match_oracle(ops):
    from spec_verify_step import DN_HV, DN_QKV, HIDDEN, VerifySlice, rope_tables, synthetic_logits
    B, K, V = 2, 7, 1000
    T = K + 1
    kv0 = [37, 90]
    model = VerifySlice(B, K, kv0, 128, pattern="DG", seed=3, device="cuda")
    olayers = _oracle_layers(model, B)
    okv = np.array(kv0)
    for step in range(2):
        g = torch.Generator(device="cuda").manual_seed(100 + step)
        x = torch.randn(B * T, HIDDEN, generator=g, device="cuda").to(torch.bfloat16)
        logits = synthetic_logits(B, K, V, 200 + step, "cuda")
        kv_before = model.kv_len.cpu().numpy().copy()
        assert np.array_equal(kv_before, okv)
        pos = model.kv_len.long().unsqueeze(1) + torch.arange(T, device="cuda")
        cos, sin = rope_tables(pos)
        caches_before = {nm: bits(L[nm]).copy() for L in model.layers if L["kind"] == "G"
                         for nm in ("cache_k", "cache_v")}
        trace = []
        h, acc, ids = model.step(x, *logits, trace=trace)
        torch.cuda.synchronize()
        assert len(trace) == 2 * len(model.layers) + 1 and torch.equal(trace[-1], h)

        tgt, drf, dids, u, us = (t.cpu().numpy() for t in logits)
        outs = []
        _, oacc, oids, okv = ovs.verify_step(olayers, bits(x), okv, B, T, tgt, drf, dids, u, us,
                                             cos.cpu().numpy(), sin.cpu().numpy(),
                                             layer_inputs=[bits(t) for t in trace[:-1]],
                                             layer_outputs=outs)
        tag = f"step {step}"
        assert np.array_equal(acc.cpu().numpy(), oacc), tag
        assert np.array_equal(ids.cpu().numpy(), oids), tag
        assert np.array_equal(model.kv_len.cpu().numpy(), okv), tag
        for i, (got, ref) in enumerate(zip(trace[1:], outs)):
            # output = input + delta: the delta's ulp flips scale with |delta|, which exceeds
            # |output| where the two cancel, so the ulp term uses |input| + |delta|
            hin = trace[i].float().cpu().numpy().astype(np.float64)
            ref = bf16_bits_to_f32(ref)
            assert_rel_close(got.float().cpu().numpy(), ref, out_unit=CHAIN_ULPS,
                             scale=np.abs(hin) + np.abs(ref - hin),
                             name=f"{tag} sublayer {i} output")
        for L, d in zip(model.layers, olayers):
            if L["kind"] == "D":
                ck = L["ckpt"].reshape(B, T, DN_HV, 128, 128)
                st = torch.stack([ck[b, int(oacc[b])] for b in range(B)]).double().cpu().numpy()
                assert_rel_close(st, d["state"], name=f"{tag} DeltaNet state")
                assert_rel_close(bf16_bits_to_f32(bits(L["conv_state"]).reshape(B, DN_QKV, 3)),
                                 bf16_bits_to_f32(d["conv_state"]), out_unit=ONE_ULP,
                                 name=f"{tag} conv window")
            else:
                for nm in ("cache_k", "cache_v"):
                    got, ref = bits(L[nm]), d[nm]
                    rows = np.zeros(got.shape[2], bool)
                    for b in range(B):
                        new = slice(int(kv_before[b]), int(kv_before[b]) + T)
                        assert_rel_close(bf16_bits_to_f32(got[b, :, new]),
                                         bf16_bits_to_f32(ref[b, :, new]), out_unit=CHAIN_ULPS,
                                         name=f"{tag} {nm} rows b={b}")
                        keep = np.ones(got.shape[2], bool)
                        keep[new] = False
                        before = caches_before[nm]
                        assert np.array_equal(got[b][:, keep], before[b][:, keep]), f"{tag} {nm}"
