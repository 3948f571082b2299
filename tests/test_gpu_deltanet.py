"""GPU parity of the gated-DeltaNet ops against the oracle (oracle/deltanet.py).

Covers deltanet::full / full_batched (the reference's per-rank decode shapes, seed 11 as in
contrib/qwen3.6-27b/kernels/tests/test_deltanet_full.py:58-73), deltanet::verify_batched at
the single-layer workload (B=1, T=5, 4/4 heads) and full width (16/48 heads, T=8), index-based
and copy-based rollback, a B=32 full-size run checked on sampled sequences, and the
column-split launch of small batches against the unsplit one, bit for bit.
Bar: 2e-3 relative (tests/_util.py); conv windows are data movement and must be bit-exact.
"""
import numpy as np
import pytest
import torch

from oracle import deltanet as od
from _util import (assert_rel_close, bits, deltanet_flat_device, deltanet_inputs,
                   deltanet_oracle_args, BF16_U)

pytestmark = pytest.mark.gpu


def _verify_gpu(ops, d):
    f = deltanet_flat_device(d)
    ckpt, out = ops.deltanet.verify_batched(
        f["state"], f["mixed_qkv"], f["conv_state"], f["conv_weight"], f["conv_bias"],
        f["a_out"], f["b_out"], f["z"], f["A_log"], f["dt_bias"], f["norm_weight"])
    torch.cuda.synchronize()
    B, Hv, D, _ = d["state"].shape
    T = d["mixed_qkv"].shape[1]
    return (ckpt.cpu().double().numpy().reshape(B, T, Hv, D, D),
            out.float().cpu().double().numpy().reshape(B, T, Hv, D))


@pytest.mark.parametrize("B,T,Hk,Hv,gates", [
    (1, 5, 4, 4, "config0"),     # single layer verify + greedy workload
    (2, 8, 16, 48, "random"),    # full width, K=7
    (3, 4, 4, 12, "random"),     # reference per-rank heads (TP=4 share)
    (2, 16, 2, 6, "random"),     # longest verify block supported
    (4, 1, 1, 3, "random"),
])
def test_verify_matches_oracle(ops, B, T, Hk, Hv, gates):
    d = deltanet_inputs(B, T, Hk, Hv, seed=11 + B + T, gates=gates)
    ck, out = od.deltanet_verify(*deltanet_oracle_args(d), Hk, Hv)
    gck, gout = _verify_gpu(ops, d)
    assert_rel_close(gck, ck, name="ckpt")
    assert_rel_close(gout, out, out_unit=BF16_U, name="out")


def test_verify_large_state_scale(ops):
    """State magnitudes like a long prefill (std 1) keep the same relative bar."""
    d = deltanet_inputs(1, 8, 16, 48, seed=5, state_std=1.0)
    ck, out = od.deltanet_verify(*deltanet_oracle_args(d), 16, 48)
    gck, gout = _verify_gpu(ops, d)
    assert_rel_close(gck, ck, name="ckpt")
    assert_rel_close(gout, out, out_unit=BF16_U, name="out")


@pytest.mark.parametrize("B", [1, 8])
def test_full_batched_reference_shapes(ops, B):
    """deltanet::full_batched at the reference's per-rank shapes (Hk=4, Hv=12, state std 0.1,
    seed 11; test_deltanet_full_batched.py:60-75); conv state bit-exact."""
    d = deltanet_inputs(B, 1, 4, 12, seed=11, state_std=0.1)
    f = deltanet_flat_device(d)
    ns, ncs, o = ops.deltanet.full_batched(
        f["state"], f["mixed_qkv"], f["conv_state"], f["conv_weight"], f["conv_bias"],
        f["a_out"], f["b_out"], f["z"], f["A_log"], f["dt_bias"], f["norm_weight"])
    torch.cuda.synchronize()
    s_ref, cs_ref, o_ref = od.deltanet_token_step(
        d["state"].numpy(), bits(d["mixed_qkv"])[:, 0], bits(d["conv_state"]),
        d["conv_weight"].numpy(), d["conv_bias"].numpy(), d["a_out"].numpy()[:, 0],
        d["b_out"].numpy()[:, 0], bits(d["z"])[:, 0], d["A_log"].numpy(),
        d["dt_bias"].numpy(), d["norm_weight"].numpy(), 4, 12)
    assert_rel_close(ns.cpu().double().numpy().reshape(s_ref.shape), s_ref, name="state")
    assert np.array_equal(bits(ncs).reshape(cs_ref.shape), cs_ref)
    assert_rel_close(o.float().cpu().double().numpy().reshape(o_ref.shape), o_ref,
                     out_unit=BF16_U, name="out")
    if B == 1:
        s1, c1, o1 = ops.deltanet.full(
            f["state"], f["mixed_qkv"], f["conv_state"].reshape(-1, 3), f["conv_weight"],
            f["conv_bias"], f["a_out"], f["b_out"], f["z"], f["A_log"], f["dt_bias"],
            f["norm_weight"])
        torch.cuda.synchronize()
        assert torch.equal(s1, ns) and torch.equal(c1, ncs) and torch.equal(o1, o)


def test_rollback_copy_and_index(ops):
    """Copy rollback == ckpt[b, a_b]; conv window bit-exact; index-based next verify ==
    verify from the copied state (no copy needed)."""
    B, T, Hk, Hv = 4, 8, 16, 48
    d = deltanet_inputs(B, T, Hk, Hv, seed=21)
    f = deltanet_flat_device(d)
    ckpt, _ = ops.deltanet.verify_batched(
        f["state"], f["mixed_qkv"], f["conv_state"], f["conv_weight"], f["conv_bias"],
        f["a_out"], f["b_out"], f["z"], f["A_log"], f["dt_bias"], f["norm_weight"])
    acc = torch.tensor([0, 7, 3, 5], dtype=torch.int32)
    state, conv = ops.deltanet.rollback(ckpt, f["mixed_qkv"], f["conv_state"], acc.cuda())
    conv_only = ops.deltanet.conv_rollback(f["mixed_qkv"], f["conv_state"], acc.cuda(), Hv)
    torch.cuda.synchronize()
    ck = ckpt.reshape(B, T, Hv * 128, 128)
    for b in range(B):
        assert torch.equal(state.reshape(B, Hv * 128, 128)[b], ck[b, int(acc[b])])
    _, cs_ref = od.deltanet_rollback(np.zeros((B, T, 1, 1, 1)), bits(d["mixed_qkv"]),
                                     bits(d["conv_state"]), acc.numpy())
    assert np.array_equal(bits(conv).reshape(cs_ref.shape), cs_ref)
    assert torch.equal(conv, conv_only)

    # next verify step: from the copied state vs straight from the checkpoints
    d2 = deltanet_inputs(B, T, Hk, Hv, seed=22)
    f2 = deltanet_flat_device(d2)
    args = (f2["mixed_qkv"], conv, f2["conv_weight"], f2["conv_bias"], f2["a_out"],
            f2["b_out"], f2["z"], f2["A_log"], f2["dt_bias"], f2["norm_weight"])
    ck_copy, out_copy = ops.deltanet.verify_batched(state, *args)
    ck_idx, out_idx = ops.deltanet.verify_from_ckpt(ckpt, acc.cuda(), *args)
    torch.cuda.synchronize()
    assert torch.equal(ck_copy, ck_idx) and torch.equal(out_copy, out_idx)


def test_rollback_clamps_out_of_range(ops):
    """accepted / state_index outside [0, T-1] act as their clamped values (the kernels
    clamp on the device instead of reading out of bounds)."""
    B, T, Hk, Hv = 4, 8, 4, 12
    d = deltanet_inputs(B, T, Hk, Hv, seed=23)
    f = deltanet_flat_device(d)
    ckpt, _ = ops.deltanet.verify_batched(
        f["state"], f["mixed_qkv"], f["conv_state"], f["conv_weight"], f["conv_bias"],
        f["a_out"], f["b_out"], f["z"], f["A_log"], f["dt_bias"], f["norm_weight"])
    wild = torch.tensor([-2, 9, 3, 100], dtype=torch.int32)
    clamped = wild.clamp(0, T - 1)
    s_w, c_w = ops.deltanet.rollback(ckpt, f["mixed_qkv"], f["conv_state"], wild.cuda())
    s_c, c_c = ops.deltanet.rollback(ckpt, f["mixed_qkv"], f["conv_state"], clamped.cuda())
    d2 = deltanet_inputs(B, T, Hk, Hv, seed=24)
    f2 = deltanet_flat_device(d2)
    args = (f2["mixed_qkv"], c_c, f2["conv_weight"], f2["conv_bias"], f2["a_out"],
            f2["b_out"], f2["z"], f2["A_log"], f2["dt_bias"], f2["norm_weight"])
    ck_w, out_w = ops.deltanet.verify_from_ckpt(ckpt, wild.cuda(), *args)
    ck_c, out_c = ops.deltanet.verify_from_ckpt(ckpt, clamped.cuda(), *args)
    torch.cuda.synchronize()
    assert torch.equal(s_w, s_c) and torch.equal(c_w, c_c)
    assert torch.equal(ck_w, ck_c) and torch.equal(out_w, out_c)
    _, cs_ref = od.deltanet_rollback(np.zeros((B, T, 1, 1, 1)), bits(d["mixed_qkv"]),
                                     bits(d["conv_state"]), clamped.numpy())
    assert np.array_equal(bits(c_w).reshape(cs_ref.shape), cs_ref)


def test_full_size_b32_sampled(ops):
    """B=32, T=8, 16/48 heads (921.7 MB of state traffic): every sequence is independent,
    so three sampled sequences are checked against the oracle run on their slices."""
    B, T, Hk, Hv = 32, 8, 16, 48
    d = deltanet_inputs(B, T, Hk, Hv, seed=32)
    gck, gout = _verify_gpu(ops, d)
    for b in (0, 17, 31):
        sl = {k: (v[b:b + 1] if k in ("state", "mixed_qkv", "conv_state", "a_out", "b_out", "z")
                  else v) for k, v in d.items()}
        ck, out = od.deltanet_verify(*deltanet_oracle_args(sl), Hk, Hv)
        assert_rel_close(gck[b:b + 1], ck, name=f"ckpt[b={b}]")
        assert_rel_close(gout[b:b + 1], out, out_unit=BF16_U, name=f"out[b={b}]")


@pytest.mark.parametrize("B,parts", [(8, 4), (16, 2), (1, 8), (3, 8)])
def test_row_split_batches_sampled(ops, B, parts):
    """Batches that run the row-split kernel (each state column's rows split over `parts`
    wave pairs: B*Hv = 384 -> 4, 768 -> 2, 48 and 144 -> 8), full width, T = 8; sampled sequences
    against the oracle."""
    Hk, Hv, T = 16, 48, 8
    d = deltanet_inputs(B, T, Hk, Hv, seed=40 + B)
    gck, gout = _verify_gpu(ops, d)
    for b in sorted({0, B // 2, B - 1}):
        sl = {k: (v[b:b + 1] if k in ("state", "mixed_qkv", "conv_state", "a_out", "b_out", "z")
                  else v) for k, v in d.items()}
        ck, out = od.deltanet_verify(*deltanet_oracle_args(sl), Hk, Hv)
        assert_rel_close(gck[b:b + 1], ck, name=f"ckpt[b={b}]")
        assert_rel_close(gout[b:b + 1], out, out_unit=BF16_U, name=f"out[b={b}]")


def test_column_split_launch_is_bit_identical(ops):
    """Up to 128 heads a head runs as 4 (up to 64 heads) or 2 workgroups that each compute the
    whole head and store a quarter or half of its columns; from 129 heads one workgroup per
    head. All three launches use 8 row parts below 192 heads, so a sequence's checkpoints
    and outputs must come out bit for bit the same at B = 1 (48 heads, 4 splits), B = 2
    (96 heads, 2 splits) and B = 3 (144 heads, unsplit). The split launch itself is checked
    against the oracle by test_row_split_batches_sampled at B = 1."""
    Hk, Hv, T = 16, 48, 8
    d = deltanet_inputs(3, T, Hk, Hv, seed=77)
    ck3, out3 = _verify_gpu(ops, d)
    for B in (1, 2):
        sl = {k: (v[:B] if k in ("state", "mixed_qkv", "conv_state", "a_out", "b_out", "z")
                  else v) for k, v in d.items()}
        ck, out = _verify_gpu(ops, sl)
        assert np.array_equal(ck, ck3[:B]), f"ckpt B={B}"
        assert np.array_equal(out, out3[:B]), f"out B={B}"


def test_rejects_bad_shapes(ops):
    d = deltanet_inputs(1, 2, 4, 12, seed=1)
    f = deltanet_flat_device(d)
    with pytest.raises(RuntimeError):
        ops.deltanet.verify_batched(f["state"][:-1], f["mixed_qkv"], f["conv_state"],
                                    f["conv_weight"], f["conv_bias"], f["a_out"], f["b_out"],
                                    f["z"], f["A_log"], f["dt_bias"], f["norm_weight"])
    with pytest.raises((RuntimeError, TypeError)):
        ops.deltanet.verify_batched(f["state"].double(), f["mixed_qkv"], f["conv_state"],
                                    f["conv_weight"], f["conv_bias"], f["a_out"], f["b_out"],
                                    f["z"], f["A_log"], f["dt_bias"], f["norm_weight"])
