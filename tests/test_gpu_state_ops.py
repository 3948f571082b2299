"""GPU checks of the small per-step state ops against the torch computations they replace
(spec_verify_step.py: rope_tables indexed by position, the out-of-place conv rollback, and
the in-place bookkeeping of accepted lengths). All bit-exact: gathers, copies and integer
adds."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_rope_rows_match_tables(ops):
    from spec_verify_step import rope_tables
    P, T = 300, 8
    tc, ts = rope_tables(torch.arange(P, device="cuda"))
    kv = torch.tensor([0, 17, 291, 250, 299, 400], dtype=torch.int32, device="cuda")
    cos, sin = ops.gqa.rope_rows(tc, ts, kv, T)
    pos = (kv.long().unsqueeze(1) + torch.arange(T, device="cuda")).clamp(max=P - 1)
    rc, rs = rope_tables(pos)
    torch.cuda.synchronize()
    assert torch.equal(cos, rc) and torch.equal(sin, rs)
    # in range, the rows equal the per-step computation at the unclamped positions
    ok = (kv.long() + T <= P)
    rc2, rs2 = rope_tables(kv.long().unsqueeze(1) + torch.arange(T, device="cuda"))
    assert torch.equal(cos[ok], rc2[ok]) and torch.equal(sin[ok], rs2[ok])


def test_conv_rollback_in_place(ops):
    B, T, QKV = 5, 8, 10240
    g = torch.Generator(device="cuda").manual_seed(1)
    mixed = torch.randn(B * T * QKV, generator=g, device="cuda").to(torch.bfloat16)
    conv = torch.randn(B * QKV, 3, generator=g, device="cuda").to(torch.bfloat16)
    acc = torch.tensor([0, 7, 3, 1, 5], dtype=torch.int32, device="cuda")
    ref = ops.deltanet.conv_rollback(mixed, conv, acc, 48)
    inplace = conv.clone()
    ops.deltanet.conv_rollback_(mixed, inplace, acc, 48)
    torch.cuda.synchronize()
    assert torch.equal(inplace.view(torch.int16), ref.view(torch.int16))


def test_commit(ops):
    acc = torch.tensor([0, 7, 3, 1], dtype=torch.int32, device="cuda")
    prev = torch.full((4,), -5, dtype=torch.int32, device="cuda")
    kv = torch.tensor([10, 20, 30, 40], dtype=torch.int32, device="cuda")
    com = torch.tensor([1, 2, 3, 4], dtype=torch.int32, device="cuda")
    ops.spec.commit_(acc, prev, kv, com)
    torch.cuda.synchronize()
    assert prev.tolist() == [0, 7, 3, 1]
    assert kv.tolist() == [11, 28, 34, 42]
    assert com.tolist() == [2, 10, 7, 6]


@pytest.mark.parametrize("layers", [0, 1, 3])
def test_rollback_commit_equals_separate_ops(ops, layers):
    """deltanet::rollback_commit_ (every layer's conv window in place + the commit, one
    launch) against conv_rollback_ per layer and commit_, bit for bit, with accepted values
    out of range on both sides: clamped into [0, T-1] for the windows and for the commit
    alike (commit_ alone adds its input as given, so it gets the clamped values)."""
    B, T, QKV = 5, 8, 10240
    g = torch.Generator(device="cuda").manual_seed(7 + layers)
    mixed = [torch.randn(B * T * QKV, generator=g, device="cuda").to(torch.bfloat16)
             for _ in range(layers)]
    conv = [torch.randn(B * QKV, 3, generator=g, device="cuda").to(torch.bfloat16)
            for _ in range(layers)]
    acc = torch.tensor([0, 7, 3, -2, 9], dtype=torch.int32, device="cuda")
    state = [torch.tensor(v, dtype=torch.int32, device="cuda")
             for v in ([1, 2, 3, 4, 5], [100, 200, 300, 400, 500], [0, 0, 7, 7, 9])]
    ref_conv = [c.clone() for c in conv]
    ref_state = [s.clone() for s in state]
    for m, c in zip(mixed, ref_conv):
        ops.deltanet.conv_rollback_(m, c, acc, 48)
    ops.spec.commit_(acc.clamp(0, T - 1), *ref_state)
    ops.deltanet.rollback_commit_(mixed, conv, acc, *state, 48, T)
    torch.cuda.synchronize()
    for c, r in zip(conv, ref_conv):
        assert torch.equal(c.view(torch.int16), r.view(torch.int16))
    for s, r in zip(state, ref_state):
        assert torch.equal(s, r)
