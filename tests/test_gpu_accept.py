"""GPU parity of spec::accept_greedy and spec::accept_rejection against the oracle
(oracle/accept.py): accepted lengths and token ids must be bit-exact.

Greedy: the tie and ownership cases of contrib/qwen3.6-35b-a3b/kernels/tests/
test_decode_sharded_lm_cpu.py:29-46 (forced winners, equal maxima inside and across
8192-wide chunks, all-zero rows) plus NaN rows; the single-layer workload (5 positions,
V = 32000, draft = argmax with p = 0.5).
Rejection: the verify workload's distributions (V = 151936, draft logits 0.8 t + 0.6 eps)
and small vocabularies where rejection and residual sampling happen often; every row's
normaliser Z and maximum m (left in the workspace) bit-exact against the oracle's
row_weights, with -inf and NaN logits and a partial last chunk.
"""
import numpy as np
import pytest
import torch

from oracle import accept as oa

pytestmark = pytest.mark.gpu


def _greedy(ops, target, draft):
    acc, out = ops.spec.accept_greedy(target.cuda(), draft.cuda())
    torch.cuda.synchronize()
    return acc.cpu().numpy(), out.cpu().numpy()


def test_greedy_single_layer_workload(ops):
    g = torch.Generator().manual_seed(0)
    target = torch.randn(1, 5, 32000, generator=g)
    am = target.argmax(-1)[0, :4]
    coin = torch.rand(4, generator=g) < 0.5
    rnd = torch.randint(0, 32000, (4,), generator=g)
    draft = torch.where(coin, am, rnd).reshape(1, 4)
    acc, out = _greedy(ops, target, draft)
    racc, rout = oa.accept_greedy(target.numpy(), draft.numpy())
    assert np.array_equal(acc, racc) and np.array_equal(out, rout)


def test_greedy_ties_nan_and_chunk_edges(ops):
    B, T, V = 12, 3, 40000
    g = torch.Generator().manual_seed(20260717)
    target = torch.randn(B, T, V, generator=g)
    for r in range(8):
        target[r, 0, r * 4096 + 11] = 100 + r           # winners in different chunks
    target[8, 0, 7] = 200; target[8, 0, 13] = 200        # tie inside a chunk
    target[9, 0, 63] = 300; target[9, 0, 8192 + 5] = 300  # tie across chunks
    target[9, 1, 8191] = 50; target[9, 1, 8192] = 50    # tie at the chunk edge
    target[10] = 0                                        # all-zero rows
    target[11, 0, 9000] = float("nan")
    target[11, 0, 30000] = float("nan")                   # first NaN wins (torch.argmax)
    tid = target.argmax(-1)
    draft = tid[:, :T - 1].clone()
    draft[3, 1] = (draft[3, 1] + 1) % V                   # one mismatch
    acc, out = _greedy(ops, target, draft)
    racc, rout = oa.accept_greedy(target.numpy(), draft.numpy())
    assert np.array_equal(out[:, 0], tid[:, 0].numpy())
    assert np.array_equal(acc, racc) and np.array_equal(out, rout)


def _rejection_inputs(B, K, V, seed, rho=0.8):
    g = torch.Generator().manual_seed(seed)
    target = torch.randn(B, K + 1, V, generator=g)
    draft = rho * target[:, :K] + (1 - rho * rho) ** 0.5 * torch.randn(B, K, V, generator=g)
    probs = torch.softmax(draft, -1).reshape(B * K, V)
    ids = torch.multinomial(probs, 1, generator=g).reshape(B, K)
    u = torch.rand(B, K, generator=g)
    us = torch.rand(B, generator=g)
    return target.contiguous(), draft.contiguous(), ids, u, us


def _rejection(ops, target, draft, ids, u, us, inv_t=1.0):
    acc, out = ops.spec.accept_rejection(target.cuda(), draft.cuda(), ids.cuda(), u.cuda(),
                                         us.cuda(), inv_t)
    torch.cuda.synchronize()
    return acc.cpu().numpy(), out.cpu().numpy()


@pytest.mark.parametrize("B,K,V,seed,inv_t", [
    (4, 7, 151936, 0, 1.0),
    (16, 7, 1000, 1, 1.0),
    (8, 3, 17, 2, 1.0),
    (8, 7, 50000, 3, 0.7),
])
def test_rejection_bit_exact(ops, B, K, V, seed, inv_t):
    target, draft, ids, u, us = _rejection_inputs(B, K, V, seed)
    acc, out = _rejection(ops, target, draft, ids, u, us, inv_t)
    racc, rout = oa.accept_rejection(target.numpy(), draft.numpy(), ids.numpy(), u.numpy(),
                                     us.numpy(), inv_t)
    assert np.array_equal(acc, racc), (acc, racc)
    assert np.array_equal(out, rout)


def test_rejection_equal_distributions_always_accept(ops):
    target, _, ids, u, us = _rejection_inputs(6, 5, 3000, 9)
    acc, out = _rejection(ops, target, target[:, :5].contiguous(), ids, u, us)
    assert (acc == 5).all()
    assert np.array_equal(out[:, :5], ids.numpy())


@pytest.mark.parametrize("V", [1000, 151936])
def test_rejection_residual_with_exact_ties(ops, V):
    """Drafts equal to their target rows but for two swapped entries a and c (target 5 at a
    and 1 at c, the draft the reverse), the draft token at c and u near 1: the first draft
    is rejected, and the residual's weights tie exactly (p_v Zq = q_v Zp) at every entry but
    a and c, so the residual has all its mass at a. Entries that are -inf in both rows tie
    at zero. Every tie must be decided exactly, as the oracle decides it."""
    B, K = 3, 2
    g = torch.Generator().manual_seed(77)
    target = torch.randn(B, K + 1, V, generator=g)
    target[:, :, 10:40] = float("-inf")
    draft = target[:, :K].clone()
    a, c = V // 2 + 3, V // 3 + 1
    target[:, 0, a], target[:, 0, c] = 5.0, 1.0
    draft[:, 0, a], draft[:, 0, c] = 1.0, 5.0
    ids = torch.full((B, K), c, dtype=torch.int64)
    u = torch.full((B, K), 0.999)
    us = torch.rand(B, generator=g)
    acc, out = _rejection(ops, target, draft, ids, u, us)
    racc, rout = oa.accept_rejection(target.numpy(), draft.numpy(), ids.numpy(), u.numpy(),
                                     us.numpy())
    assert (acc == 0).all() and (out[:, 0] == a).all()
    assert np.array_equal(acc, racc) and np.array_equal(out, rout)


@pytest.mark.parametrize("B,K,V,seed,inv_t", [(3, 2, 151936, 4, 1.0), (2, 3, 20001, 5, 0.7)])
def test_rejection_row_sums_bit_exact(ops, B, K, V, seed, inv_t):
    from npn_native import call, query, stream_of
    target, draft, ids, u, us = _rejection_inputs(B, K, V, seed)
    target[0, 0, 17] = float("-inf")
    target[B - 1, K, V - 1] = float("nan")
    draft[0, K - 1, :100] = float("-inf")
    draft[B - 1, 0, 3] = float("nan")
    t, d = target.cuda(), draft.cuda()
    ws = torch.zeros(query("npn_accept_workspace_size", B, K, V), dtype=torch.uint8,
                     device="cuda")
    acc = torch.empty(B, dtype=torch.int32, device="cuda")
    out = torch.empty((B, K + 1), dtype=torch.int64, device="cuda")
    call("npn_accept_rejection", t, d, ids.cuda(), u.cuda(), us.cuda(), inv_t, acc, out,
         B, K, V, ws, ws.numel(), stream_of(t))
    torch.cuda.synchronize()
    R = B * (2 * K + 1)
    off = (16 * R + 255) // 256 * 256
    zw = ws[:16 * R].cpu().numpy().view(np.uint64).reshape(R, 2)   # u128, low word first
    z = [int(lo) | (int(hi) << 64) for lo, hi in zw]
    m = ws[off:off + 4 * R].cpu().numpy().view(np.float32)
    rows = [target[b, i].numpy() for b in range(B) for i in range(K + 1)]
    rows += [draft[b, i].numpy() for b in range(B) for i in range(K)]
    for r, logits in enumerate(rows):
        _, Z, mr = oa.row_weights(logits, inv_t)
        assert int(z[r]) == Z, f"row {r}: Z {int(z[r])} vs oracle {Z}"
        assert m[r].view(np.uint32) == np.float32(mr).view(np.uint32), f"row {r}: max"
    racc, rout = oa.accept_rejection(target.numpy(), draft.numpy(), ids.numpy(), u.numpy(),
                                     us.numpy(), inv_t)
    assert np.array_equal(acc.cpu().numpy(), racc)
    assert np.array_equal(out.cpu().numpy(), rout)


@pytest.mark.parametrize("V", [50, 151936])
def test_rejection_empty_bonus_rows(ops, V):
    """Bonus rows without mass (all NaN, all -inf, a +inf entry) emit the row's argmax, a
    valid token id (NaN first, then +inf, ties to the lowest index), as the oracle does;
    a row whose NaN entries sit among finite ones still samples by inverse CDF."""
    B, K = 5, 3
    g = torch.Generator().manual_seed(31)
    target = torch.randn(B, K + 1, V, generator=g)
    draft = target[:, :K].clone()                       # p == q: every draft accepted
    ids = torch.randint(0, V, (B, K), generator=g)
    u, us = torch.rand(B, K, generator=g), torch.rand(B, generator=g)
    target[0, K] = float("nan")
    target[1, K] = float("-inf")
    target[2, K, V // 3] = float("inf")
    target[2, K, V - 1] = float("inf")
    target[3, K, 7] = float("nan")
    target[3, K, V - 2] = float("nan")
    target[4, K] = float("-inf")
    target[4, K, V - 1] = float("nan")                  # NaN wins over -inf
    acc, out = _rejection(ops, target, draft, ids, u, us)
    racc, rout = oa.accept_rejection(target.numpy(), draft.numpy(), ids.numpy(), u.numpy(),
                                     us.numpy())
    assert (acc == K).all()
    assert np.array_equal(acc, racc) and np.array_equal(out, rout)
    assert out[0, K] == 0 and out[1, K] == 0 and out[2, K] == V // 3 and out[4, K] == V - 1
    assert ((out[:, K] >= 0) & (out[:, K] < V)).all()


@pytest.mark.parametrize("V", [40, 151936])
def test_out_of_range_draft_ids(ops, V):
    """Draft ids -1, V and -2^40 are never accepted: rejection sampling counts the position
    as a rejection whatever the uniform and samples it from the residual (here p == q for
    some sequences, an empty residual, so the target row's argmax), greedy rejects them, and
    every emitted id lies in [0, V) -- bit-exact against the oracle."""
    B, K = 6, 3
    g = torch.Generator().manual_seed(41)
    target = torch.randn(B, K + 1, V, generator=g)
    draft = target[:, :K].clone()
    draft[3:] = 0.8 * target[3:, :K] + 0.6 * torch.randn(3, K, V, generator=g)
    ids = torch.randint(0, V, (B, K), generator=g)
    ids[0, 0], ids[1, 1], ids[2, 2] = -1, V, -(1 << 40)
    ids[3, 0], ids[4, 2], ids[5, 1] = V, -1, V + 7
    u = torch.zeros(B, K)
    us = torch.rand(B, generator=g)
    acc, out = _rejection(ops, target, draft, ids, u, us)
    racc, rout = oa.accept_rejection(target.numpy(), draft.numpy(), ids.numpy(), u.numpy(),
                                     us.numpy())
    assert acc.tolist()[:3] == [0, 1, 2]
    assert np.array_equal(acc, racc) and np.array_equal(out, rout)
    assert ((out >= -1) & (out < V)).all()
    gacc, gout = _greedy(ops, target, ids)
    racc, rout = oa.accept_greedy(target.numpy(), ids.numpy())
    assert np.array_equal(gacc, racc) and np.array_equal(gout, rout)
    assert ((gout >= -1) & (gout < V)).all()
