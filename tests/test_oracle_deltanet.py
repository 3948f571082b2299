"""CPU pinning of oracle/deltanet.py.

- golden vectors from HF transformers' Qwen3.5 gated-delta-rule functions
  (tests/golden/deltanet_hf.npz, written by tests/golden/make_deltanet_fixture.py);
- closed forms: beta = 0 and decay = 1 leave S unchanged; one token from S = 0 gives
  S = beta k v^T and o = beta v (k.q);
- T-token verify == T chained single-token steps (state and conv window), so the
  checkpoint bookkeeping is the token step's;
- the rollback invariant of contrib/qwen3.6-27b/kernels/tests/
  test_deltanet_spec_verify_rollback.py:20-22 with the real recurrence: after any sequence
  of (verify T, accept a) steps the restored state equals a clean replay over the accepted
  tokens (seeds 0-4, like the reference test).
"""
import os

import numpy as np
import pytest

from oracle import deltanet as od
from oracle.numerics import f32_to_bf16_bits

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "deltanet_hf.npz")


def _golden(name):
    d = np.load(GOLDEN)
    return {k.split("/")[1]: d[k] for k in d.files if k.startswith(name + "/")}


@pytest.mark.parametrize("name", ["d16", "d32"])
def test_matches_hf_reference_functions(name):
    g = _golden(name)
    hk, hv, _ = (int(x) for x in g["heads"])
    ck, out = od.deltanet_verify(g["state"], g["mixed_qkv"], g["conv_state"], g["conv_weight"],
                                 g["conv_bias"], g["a_out"], g["b_out"], g["z"], g["A_log"],
                                 g["dt_bias"], g["norm_weight"], hk, hv)
    assert np.linalg.norm(ck - g["ckpt"]) / np.linalg.norm(g["ckpt"]) < 1e-5
    assert np.linalg.norm(out - g["out"]) / np.linalg.norm(g["out"]) < 1e-5
    T = g["mixed_qkv"].shape[1]
    cs = od.conv_state_after(g["conv_state"], g["mixed_qkv"], np.full(len(g["state"]), T - 1))
    assert np.array_equal(cs, g["conv_final"])


def _inputs(B, T, Hk, Hv, D, seed):
    rng = np.random.default_rng(seed)
    QKV = (2 * Hk + Hv) * D
    return dict(
        state=rng.standard_normal((B, Hv, D, D)) * 0.05,
        mixed_qkv=f32_to_bf16_bits(rng.standard_normal((B, T, QKV))),
        conv_state=f32_to_bf16_bits(rng.standard_normal((B, QKV, 3))),
        conv_weight=rng.standard_normal((QKV, 4)).astype(np.float32) * 0.5,
        conv_bias=rng.standard_normal(QKV).astype(np.float32) * 0.1,
        a_out=rng.standard_normal((B, T, Hv)).astype(np.float32),
        b_out=rng.standard_normal((B, T, Hv)).astype(np.float32),
        z=f32_to_bf16_bits(rng.standard_normal((B, T, Hv, D))),
        A_log=rng.standard_normal(Hv).astype(np.float32) * 0.5,
        dt_bias=rng.standard_normal(Hv).astype(np.float32),
        norm_weight=(rng.standard_normal(D) * 0.1 + 1).astype(np.float32),
    )


def _args(d):
    return (d["state"], d["mixed_qkv"], d["conv_state"], d["conv_weight"], d["conv_bias"],
            d["a_out"], d["b_out"], d["z"], d["A_log"], d["dt_bias"], d["norm_weight"])


def test_no_write_no_decay_keeps_state():
    d = _inputs(2, 3, 1, 2, 16, seed=1)
    d["b_out"][:] = -1e4       # beta = sigmoid(-1e4) = 0
    d["A_log"][:] = -1e4       # g = -exp(-1e4) * softplus(.) = 0 -> decay 1
    ck, _ = od.deltanet_verify(*_args(d), 1, 2)
    for t in range(3):
        assert np.array_equal(ck[:, t], d["state"])


def test_single_token_from_zero_state():
    d = _inputs(1, 1, 1, 1, 16, seed=2)
    d["state"][:] = 0.0
    ck, _ = od.deltanet_verify(*_args(d), 1, 1)
    seq = od.conv_window(d["conv_state"], d["mixed_qkv"])
    y = od.conv_silu(seq, d["conv_weight"], d["conv_bias"], 0)[0]
    q, k, v = y[:16], y[16:32], y[32:]
    k = k / np.sqrt((k * k).sum() + 1e-6)
    _, beta = od.gates(d["a_out"], d["b_out"], d["A_log"], d["dt_bias"])
    S = beta[0, 0, 0] * np.outer(k, v)
    np.testing.assert_allclose(ck[0, 0, 0], S, rtol=1e-12, atol=1e-15)


def test_verify_equals_chained_token_steps():
    B, T, Hk, Hv, D = 2, 6, 2, 6, 16
    d = _inputs(B, T, Hk, Hv, D, seed=3)
    ck, out = od.deltanet_verify(*_args(d), Hk, Hv)
    s, cs = d["state"], d["conv_state"]
    for t in range(T):
        s, cs, o = od.deltanet_token_step(s, d["mixed_qkv"][:, t], cs, d["conv_weight"],
                                          d["conv_bias"], d["a_out"][:, t], d["b_out"][:, t],
                                          d["z"][:, t], d["A_log"], d["dt_bias"],
                                          d["norm_weight"], Hk, Hv)
        np.testing.assert_allclose(ck[:, t], s, rtol=1e-12, atol=1e-14)
        np.testing.assert_allclose(out[:, t], o, rtol=1e-12, atol=1e-14)
        _, cs_roll = od.deltanet_rollback(ck, d["mixed_qkv"], d["conv_state"], np.full(B, t))
        assert np.array_equal(cs_roll, cs)


@pytest.mark.parametrize("seed", range(5))
def test_rollback_invariant_clean_replay(seed):
    """Reference bookkeeping test (N = K+1 = 4, 12 steps, 1..N tokens committed per step)
    with the gated-DeltaNet recurrence in place of the scalar fold."""
    rng = np.random.default_rng(seed)
    Hk, Hv, D, N = 1, 2, 16, 4
    base = _inputs(1, 1, Hk, Hv, D, seed=100 + seed)
    state, conv = base["state"], base["conv_state"]
    committed = []                                   # per committed token: (x, a, b, z)
    for _ in range(12):
        d = _inputs(1, N, Hk, Hv, D, seed=int(rng.integers(1 << 30)))
        ck, _ = od.deltanet_verify(state, d["mixed_qkv"], conv, base["conv_weight"],
                                   base["conv_bias"], d["a_out"], d["b_out"], d["z"],
                                   base["A_log"], base["dt_bias"], base["norm_weight"], Hk, Hv)
        acc = int(rng.integers(0, N))                # accepted drafts; acc + 1 tokens commit
        state, conv = od.deltanet_rollback(ck, d["mixed_qkv"], conv, np.array([acc]))
        committed += [(d["mixed_qkv"][:, t], d["a_out"][:, t], d["b_out"][:, t], d["z"][:, t])
                      for t in range(acc + 1)]
        s, cs = base["state"], base["conv_state"]
        for x, a, b, z in committed:
            s, cs, _ = od.deltanet_token_step(s, x, cs, base["conv_weight"], base["conv_bias"],
                                              a, b, z, base["A_log"], base["dt_bias"],
                                              base["norm_weight"], Hk, Hv)
        np.testing.assert_allclose(state, s, rtol=1e-10, atol=1e-13)
        assert np.array_equal(conv, cs)


def test_rollback_rejects_out_of_range():
    d = _inputs(1, 2, 1, 1, 16, seed=4)
    ck, _ = od.deltanet_verify(*_args(d), 1, 1)
    with pytest.raises(ValueError):
        od.deltanet_rollback(ck, d["mixed_qkv"], d["conv_state"], np.array([2]))
