"""GPU parity of the GQA attention-tail ops against the oracle (oracle/gqa.py).

gqa::tail at the reference's shapes (seed 0, B=8, 6 q heads, S=128, position 100, as
contrib/qwen3.6-27b/kernels/gqa_tail_ref.py:73-102); gqa::tail_verify at reduced and full
verify shapes (24 q / 4 kv heads, T=8) with KV lengths that cross chunk boundaries, kv_len=0,
T=1 and other head groupings; gqa::kv_append bit-exact against the oracle's bf16 rounding
order (at most 1 bf16 ulp where fp32 rsqrt rounding differs).
"""
import numpy as np
import pytest
import torch

from oracle import gqa as og
from _util import BF16_U, assert_rel_close, bits, gqa_verify_inputs

pytestmark = pytest.mark.gpu


def test_tail_reference_shapes(ops):
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
    ref = og.gqa_tail(query.reshape(B * HQ, 256).numpy(), gate.reshape(B * HQ, 256).numpy(),
                      q_norm.numpy(), cos.numpy(), sin.numpy(), ck.reshape(B * S, 256).numpy(),
                      cv.reshape(B * S, 256).numpy(), mask.reshape(1, S).numpy())
    got = ops.gqa.tail(query.reshape(B * HQ, 256).cuda(), gate.reshape(B * HQ, 256).cuda(),
                       q_norm.reshape(1, 256).cuda(), cos.reshape(1, 64).cuda(),
                       sin.reshape(1, 64).cuda(), ck.reshape(B * S, 256).cuda(),
                       cv.reshape(B * S, 256).cuda(), mask.reshape(1, S).cuda())
    torch.cuda.synchronize()
    assert_rel_close(got.cpu().double().numpy(), ref, name="gqa.tail")


def _run_verify(ops, d):
    out = ops.gqa.tail_verify(*[d[k].cuda() for k in
                                ("query", "gate", "q_norm", "cos", "sin", "cache_k", "cache_v",
                                 "kv_len")])
    torch.cuda.synchronize()
    return out.float().cpu().double().numpy()


def _oracle_verify(d):
    return og.gqa_tail_verify(bits(d["query"]), bits(d["gate"]), d["q_norm"].numpy(),
                              d["cos"].numpy(), d["sin"].numpy(), bits(d["cache_k"]),
                              bits(d["cache_v"]), d["kv_len"].numpy())


@pytest.mark.parametrize("B,T,Hq,Hkv,kv_lens,s_max", [
    (2, 8, 24, 4, [37, 600], 1024),          # full head layout, short caches
    (2, 8, 24, 4, [504, 1023 - 8], 1024),    # rows straddling the 512-key chunk edge, full cache
    (3, 8, 24, 4, [0, 1, 2000], 2048),       # empty prior cache
    (1, 1, 6, 1, [300], 512),                # decode-like T=1, one 16-row tile
    (2, 4, 8, 2, [100, 33], 256),            # 16 rows per kv head
    (1, 5, 12, 2, [1500], 1536),             # 30 rows: two tiles with padding
])
def test_tail_verify_matches_oracle(ops, B, T, Hq, Hkv, kv_lens, s_max):
    d = gqa_verify_inputs(B, T, Hq, Hkv, kv_lens, s_max, seed=B * 7 + T)
    assert_rel_close(_run_verify(ops, d), _oracle_verify(d), out_unit=BF16_U, name="tail_verify")


def test_tail_verify_many_short_ragged_pairs(ops):
    """160 (sequence, kv head) pairs with 0..300 cached rows: more 32-key steps than
    attention workgroups, so workgroup ranges start and end inside pairs and one
    workgroup covers several consecutive pairs."""
    B = 40
    kv = np.random.default_rng(41).integers(0, 301, size=B).tolist()
    d = gqa_verify_inputs(B, 8, 24, 4, kv, 320, seed=41)
    assert_rel_close(_run_verify(ops, d), _oracle_verify(d), out_unit=BF16_U, name="ragged")


def test_tail_verify_many_pairs_padded_rows_and_one_long_pair(ops):
    """80 pairs (the per-row merge), 30 query rows per pair in a 32-row tile, and one pair
    with a 4000-row cache among short ones, so that most attention workgroups work on that
    pair and its merge walks hundreds of segments."""
    B = 40
    kv = np.random.default_rng(43).integers(0, 60, size=B)
    kv[7] = 4000
    d = gqa_verify_inputs(B, 5, 12, 2, kv.tolist(), 4096, seed=43)
    assert_rel_close(_run_verify(ops, d), _oracle_verify(d), out_unit=BF16_U, name="padded")


def test_tail_verify_full_width_long(ops):
    """Config-2-like: 24/4 heads, T=8, KV lengths 4096..8192 (oracle-affordable)."""
    d = gqa_verify_inputs(2, 8, 24, 4, [4096, 8000], 8200, seed=2)
    assert_rel_close(_run_verify(ops, d), _oracle_verify(d), out_unit=BF16_U, name="tail_verify")


def test_tail_verify_full_width_longest(ops):
    """24/4 heads, T=8, at the top of the verify workloads' KV range (32768 rows), next to
    a sequence in the middle of it, in one launch."""
    d = gqa_verify_inputs(2, 8, 24, 4, [32768 - 8, 17000], 32768, seed=5)
    assert_rel_close(_run_verify(ops, d), _oracle_verify(d), out_unit=BF16_U, name="tail_verify")


def test_kv_append_then_attend_equals_cloned_cache(ops):
    """Append-after-attention equivalence (contrib/qwen3.6-35b-a3b/kernels/tests/
    test_gqa_stateful_cache_cpu.py:9-40): rows written by kv_append match the oracle's
    bf16 rounding order and leave every other row untouched."""
    B, T, Hkv, s_max = 2, 8, 4, 512
    g = torch.Generator().manual_seed(3)
    key = torch.randn(B, T, Hkv, 256, generator=g).to(torch.bfloat16)
    value = torch.randn(B, T, Hkv, 256, generator=g).to(torch.bfloat16)
    k_norm = torch.randn(256, generator=g) * 0.1
    kv_len = torch.tensor([5, 300], dtype=torch.int32)
    d = gqa_verify_inputs(B, T, 24, Hkv, kv_len.numpy(), s_max, seed=4)
    ck = d["cache_k"].clone()
    cv = d["cache_v"].clone()
    ck_dev, cv_dev = ck.cuda(), cv.cuda()
    ops.gqa.kv_append(key.cuda(), value.cuda(), k_norm.cuda(), d["cos"].cuda(), d["sin"].cuda(),
                      ck_dev, cv_dev, kv_len.cuda())
    torch.cuda.synchronize()
    rk, rv = og.gqa_kv_append(bits(key), bits(value), k_norm.numpy(), d["cos"].numpy(),
                              d["sin"].numpy(), bits(ck).copy(), bits(cv).copy(), kv_len.numpy())
    gk, gv = bits(ck_dev.cpu()), bits(cv_dev.cpu())
    assert np.array_equal(gv, rv)
    diff = np.abs(gk.astype(np.int32) - rk.astype(np.int32))
    assert diff.max() <= 1, f"kv_append key rows differ by {diff.max()} bf16 ulps"
    assert (diff > 0).mean() < 0.01


@pytest.mark.parametrize("P", [600, 310])
def test_tail_verify_append_equals_separate_ops(ops, P):
    """gqa::tail_verify_append (append in the query-prep launch, RoPE rows from the position
    tables) against rope_rows + kv_append + tail_verify: output and both caches bit for bit,
    with kv_len 0, one mid-cache and one ending at s_max, and (P = 310) positions past the
    table clamped to its last row as rope_rows clamps them."""
    from oracle.gqa import rope_cos_sin
    B, T, Hq, Hkv, s_max = 3, 8, 24, 4, 600
    g = torch.Generator().manual_seed(21)
    kv_len = torch.tensor([0, 300, s_max - T], dtype=torch.int32)
    d = gqa_verify_inputs(B, T, Hq, Hkv, kv_len.numpy(), s_max, seed=22)
    key = torch.randn(B, T, Hkv, 256, generator=g).to(torch.bfloat16).cuda()
    value = torch.randn(B, T, Hkv, 256, generator=g).to(torch.bfloat16).cuda()
    k_norm = (torch.randn(256, generator=g) * 0.1).cuda()
    tc, ts = rope_cos_sin(np.arange(P)[:, None], theta=1e7)
    tc = torch.from_numpy(tc.reshape(P, 64)).cuda()
    ts = torch.from_numpy(ts.reshape(P, 64)).cuda()
    q, gate, qn = d["query"].cuda(), d["gate"].cuda(), d["q_norm"].cuda()
    kvl = kv_len.cuda()
    ck1, cv1 = d["cache_k"].cuda(), d["cache_v"].cuda()
    ck2, cv2 = ck1.clone(), cv1.clone()
    cos, sin = ops.gqa.rope_rows(tc, ts, kvl, T)
    ops.gqa.kv_append(key, value, k_norm, cos, sin, ck1, cv1, kvl)
    ref = ops.gqa.tail_verify(q, gate, qn, cos, sin, ck1, cv1, kvl)
    out = ops.gqa.tail_verify_append(q, gate, key, value, qn, k_norm, tc, ts, ck2, cv2, kvl)
    torch.cuda.synchronize()
    assert torch.equal(ck2, ck1) and torch.equal(cv2, cv1)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
