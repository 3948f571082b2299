"""End-to-end GPU parity of the verify step (neuron-pytorch-native_amd/spec_verify_step.py:
fp8 projections, fused residual norms, DeltaNet verify, GQA append + verify attention,
SwiGLU, rejection sampling, rollback) against the oracle composition
(oracle/verify_step.py) on the same weights, states, caches, logits and uniforms, over two
consecutive steps, so the second step starts from the index-based DeltaNet rollback and the
advanced KV lengths of the first.

Two workloads:
- a 2-layer slice (one DeltaNet and one GQA layer, each with its MLP) at whole-model widths,
  B = 2, K = 7, short caches, vocabulary 1000, every sequence checked;
- the whole verify workload: the 4-layer slice (3 DeltaNet + 1 GQA), B = 32, K = 7,
  vocabulary 151936, KV lengths U{4096..32768} (including 4096 and 32768). Acceptance of
  all 32 sequences is checked against the oracle, and three of them (the shortest and
  longest caches and one drawn at random) through every sublayer, state and cache row; the
  sequences of the step are independent, so the oracle runs on those three alone.
Each sublayer (mixer, MLP) of the oracle starts
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

from oracle import accept as oa
from oracle import verify_step as ovs
from oracle.numerics import bf16_bits_to_f32
from _util import assert_rel_close, bits

pytestmark = pytest.mark.gpu

ONE_ULP = 2.0 ** -7
CHAIN_ULPS = 4 * ONE_ULP


def _oracle_layers(model, B, sel):
    """Oracle layer dicts for sequences `sel` of the device model (weights shared)."""
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
            st = L["state"].reshape(B, DN_HV, 128, 128)[sel]
            d["state"] = st.cpu().double().numpy()
            d["conv_state"] = bits(L["conv_state"].reshape(B, DN_QKV, 3)[sel]).copy()
        else:
            d["q_norm"], d["k_norm"] = L["q_norm"].cpu().numpy(), L["k_norm"].cpu().numpy()
            d["cache_k"] = bits(L["cache_k"][sel]).copy()
            d["cache_v"] = bits(L["cache_v"][sel]).copy()
        layers.append(d)
    return ovs.decode_weights(layers)


def _rows(t, B, T, sel):
    """Rows of sequences `sel` from a [B*T, ...] tensor."""
    return t.reshape(B, T, *t.shape[1:])[sel].reshape(len(sel) * T, *t.shape[1:])


def run_two_steps(B, K, V, kv0, s_max, pattern, seed, sel):
    from spec_verify_step import DN_HV, DN_QKV, HIDDEN, VerifySlice, rope_tables, synthetic_logits
    T = K + 1
    sel = torch.as_tensor(sel, device="cuda")
    ns = len(sel)
    model = VerifySlice(B, K, kv0, s_max, pattern=pattern, seed=seed, device="cuda")
    olayers = _oracle_layers(model, B, sel)
    okv = np.asarray(kv0)[sel.cpu().numpy()]
    for step in range(2):
        g = torch.Generator(device="cuda").manual_seed(100 + step)
        x = torch.randn(B * T, HIDDEN, generator=g, device="cuda").to(torch.bfloat16)
        logits = synthetic_logits(B, K, V, 200 + step, "cuda")
        kv_before = model.kv_len[sel].cpu().numpy().copy()
        assert np.array_equal(kv_before, okv)
        pos = model.kv_len.long().unsqueeze(1) + torch.arange(T, device="cuda")
        cos, sin = rope_tables(pos)
        caches_before = {nm: bits(L[nm][sel]).copy() for L in model.layers if L["kind"] == "G"
                         for nm in ("cache_k", "cache_v")}
        trace = []
        h, acc, ids = model.step(x, *logits, trace=trace)
        torch.cuda.synchronize()
        assert len(trace) == 2 * len(model.layers) + 1 and torch.equal(trace[-1], h)
        tag = f"step {step}"

        tgt, drf, dids, u, us = (t.cpu().numpy() for t in logits)
        if ns < B:  # acceptance of every sequence
            aacc, aids = oa.accept_rejection(tgt, drf, dids, u, us, 1.0)
            assert np.array_equal(acc.cpu().numpy(), aacc), tag
            assert np.array_equal(ids.cpu().numpy(), aids), tag
        s_np = sel.cpu().numpy()
        outs = []
        _, oacc, oids, okv = ovs.verify_step(
            olayers, bits(_rows(x, B, T, sel)), okv, ns, T, tgt[s_np], drf[s_np], dids[s_np],
            u[s_np], us[s_np], cos[sel].cpu().numpy(), sin[sel].cpu().numpy(),
            dn_heads=(16, 48), gqa_heads=(24, 4),
            layer_inputs=[bits(_rows(t, B, T, sel)) for t in trace[:-1]], layer_outputs=outs)
        assert np.array_equal(acc[sel].cpu().numpy(), oacc), tag
        assert np.array_equal(ids[sel].cpu().numpy(), oids), tag
        assert np.array_equal(model.kv_len[sel].cpu().numpy(), okv), tag
        for i, (got, ref) in enumerate(zip(trace[1:], outs)):
            # output = input + delta: the delta's ulp flips scale with |delta|, which exceeds
            # |output| where the two cancel, so the ulp term uses |input| + |delta|
            hin = _rows(trace[i], B, T, sel).float().cpu().numpy().astype(np.float64)
            ref = bf16_bits_to_f32(ref)
            assert_rel_close(_rows(got, B, T, sel).float().cpu().numpy(), ref,
                             out_unit=CHAIN_ULPS, scale=np.abs(hin) + np.abs(ref - hin),
                             name=f"{tag} sublayer {i} output")
        for L, d in zip(model.layers, olayers):
            if L["kind"] == "D":
                ck = L["ckpt"].reshape(B, T, DN_HV, 128, 128)
                st = torch.stack([ck[int(sel[j]), int(oacc[j])] for j in range(ns)])
                assert_rel_close(st.double().cpu().numpy(), d["state"],
                                 name=f"{tag} DeltaNet state")
                cw = bits(L["conv_state"].reshape(B, DN_QKV, 3)[sel])
                assert_rel_close(bf16_bits_to_f32(cw), bf16_bits_to_f32(d["conv_state"]),
                                 out_unit=ONE_ULP, name=f"{tag} conv window")
            else:
                for nm in ("cache_k", "cache_v"):
                    got, ref = bits(L[nm][sel]), d[nm]
                    for j in range(ns):
                        new = slice(int(kv_before[j]), int(kv_before[j]) + T)
                        assert_rel_close(bf16_bits_to_f32(got[j, :, new]),
                                         bf16_bits_to_f32(ref[j, :, new]), out_unit=CHAIN_ULPS,
                                         name=f"{tag} {nm} rows of sequence {int(sel[j])}")
                        keep = np.ones(got.shape[2], bool)
                        keep[new] = False
                        before = caches_before[nm]
                        assert np.array_equal(got[j][:, keep], before[j][:, keep]), f"{tag} {nm}"


def test_two_steps_match_oracle(ops):
    run_two_steps(2, 7, 1000, [37, 90], 128, "DG", seed=3, sel=[0, 1])


@pytest.mark.timeout(900)
def test_two_steps_whole_workload(ops):
    """B = 32, K = 7, the 4-layer slice, V = 151936, KV lengths U{4096..32768}."""
    B, K = 32, 7
    rng = np.random.default_rng(7)
    kv0 = rng.integers(4096, 32769, size=B)
    kv0[3], kv0[20] = 4096, 32768
    mid = int(rng.integers(0, B))
    sel = sorted({3, 20, mid if mid not in (3, 20) else 11})
    run_two_steps(B, K, 151936, kv0.tolist(), 32768 + 2 * (K + 1), "DDDG", seed=11, sel=sel)
