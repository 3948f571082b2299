"""CPU pinning of oracle/accept.py.

Greedy: argmax_first against torch.argmax on the tie/ownership cases of
contrib/qwen3.6-35b-a3b/kernels/tests/test_decode_sharded_lm_cpu.py:29-46 and NaN rows;
accept_greedy on constructed draft sequences.

Rejection sampling (no reference vectors exist; pinned against the mathematics):
- fma32 (the fp32 fused multiply-add the contract is written in): equal to the C library's
  fmaf on random operands and on a constructed double-rounding case, where rounding the
  float64 sum to nearest first gives the wrong fp32 result;
- expfix: E(0) = 2^31, monotone, within max(2 quanta, 2^-21 relative) of floor(2^31 exp(x)),
  0 at and below -32 and for -inf and NaN;
- the exact distribution of the first emitted token implied by the integer contract
  (acceptance probabilities counted over all 2^24 uniforms, residual picked by counting
  uniforms per token) equals p = E^p / Z^p within 2^-22 (Leviathan et al. 2023, Thm 1);
- _inverse_cdf selects the right token on both sides of every boundary uniform;
- a chi-square test of the full accept_rejection output against p;
- p == q accepts every draft; q(x) > 0 = p(x) always rejects and resamples from the
  positive part of p - q.
"""
import numpy as np
import pytest
import torch

from oracle import accept as oa

U = 1 << 24


def test_argmax_ties_and_ownership():
    generator = torch.Generator().manual_seed(20260717)
    logits = torch.randn(37, 256, generator=generator)
    for rank in range(8):
        logits[rank, rank * 32 + 11] = 100 + rank
    logits[8, 7] = 200
    logits[8, 13] = 200
    logits[9, 63] = 300
    logits[9, 192] = 300
    logits[10] = 0
    assert np.array_equal(oa.argmax_first(logits.numpy()), logits.argmax(-1).numpy())


def test_argmax_nan_first():
    x = torch.randn(3, 50)
    x[0, 7] = float("nan")
    x[0, 30] = float("nan")
    x[1, 49] = float("nan")
    assert np.array_equal(oa.argmax_first(x.numpy()), x.argmax(-1).numpy())


def test_accept_greedy_cases():
    t = torch.randn(3, 5, 100).numpy()
    tid = t.argmax(-1)
    d = tid[:, :4].copy()
    d[1, 2] = (d[1, 2] + 1) % 100      # mismatch at position 2
    d[2, 0] = (d[2, 0] + 1) % 100      # immediate mismatch
    acc, out = oa.accept_greedy(t, d)
    assert acc.tolist() == [4, 2, 0]
    assert out[0].tolist() == tid[0].tolist()
    assert out[1].tolist() == tid[1, :3].tolist() + [-1, -1]
    assert out[2].tolist() == [tid[2, 0], -1, -1, -1, -1]


def _libm_fmaf():
    import ctypes
    import ctypes.util
    libm = ctypes.CDLL(ctypes.util.find_library("m") or "libm.so.6")
    f = libm.fmaf
    f.restype = ctypes.c_float
    f.argtypes = [ctypes.c_float] * 3
    return f


def test_fma32_matches_libm_fmaf():
    fmaf = _libm_fmaf()
    rng = np.random.default_rng(3)
    a = (rng.standard_normal(4000) * 4.0 ** rng.integers(-6, 6, 4000)).astype(np.float32)
    b = (rng.standard_normal(4000) * 4.0 ** rng.integers(-6, 6, 4000)).astype(np.float32)
    c = (rng.standard_normal(4000) * 4.0 ** rng.integers(-6, 6, 4000)).astype(np.float32)
    # operand ranges of the contract: x in [-32, 0] against log2(e), and Horner steps
    x = -rng.uniform(0, 32, 4000).astype(np.float32)
    a = np.concatenate([a, x, rng.uniform(-0.35, 0.35, 4000).astype(np.float32)])
    b = np.concatenate([b, np.full(4000, oa.L2E), np.full(4000, oa.TAYLOR[2])])
    c = np.concatenate([c, np.full(4000, oa.MAGIC), np.full(4000, oa.TAYLOR[3])])
    got = oa.fma32(a, b, c)
    ref = np.array([fmaf(float(p), float(q), float(r)) for p, q, r in zip(a, b, c)], np.float32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # 641 * 6700417 = 2^32 + 1: a*b = 2^-24 + 2^-56, so 1 + a*b lies just above the fp32
    # midpoint 1 + 2^-24; the float64 sum rounds onto the midpoint and then to even (1.0)
    a1, b1, one = np.float32(641 * 2.0 ** -28), np.float32(6700417 * 2.0 ** -28), np.float32(1)
    assert np.float32(np.float64(a1) * np.float64(b1) + 1.0) == one
    for s in (1.0, -1.0):
        want = fmaf(float(s * a1), float(b1), float(s * one))
        assert want == s * (1 + 2.0 ** -23)
        assert oa.fma32(np.float32(s * a1), b1, np.float32(s * one)) == np.float32(want)


def test_expfix_properties():
    x = np.sort(-np.random.default_rng(0).exponential(4.0, 100000).astype(np.float32))
    E = oa.expfix(x)
    assert E.dtype == np.uint32
    assert oa.expfix(np.float32([0.0, -0.0]))[0] == 1 << 31
    assert np.all(np.diff(E.astype(np.int64)) >= 0)                    # monotone in x
    ref = np.floor(np.exp(x.astype(np.float64)) * 2.0 ** 31)
    # within 2 quanta (2^-30 absolute) or 2^-21 relative, whichever is larger
    assert np.all(np.abs(E - ref) <= np.maximum(2.0, ref * 2.0 ** -21))
    assert np.all(oa.expfix(np.float32([-32.0, -40.0, -1e30, -np.inf, np.nan])) == 0)
    # the smallest nonzero E: 2^31 exp(x) >= 1 from x = -31 ln 2 = -21.487 on
    assert oa.expfix(np.float32([-21.4]))[0] == 1 and oa.expfix(np.float32([-21.6]))[0] == 0


def _first_token_distribution(t_row, d_row):
    """Exact P(first emitted token = v) for K = 1 under the integer contract, with the draft
    token drawn from the contract's own q = E^q / Z^q."""
    Ep, Zp, _ = oa.row_weights(t_row)
    Eq, Zq, _ = oa.row_weights(d_row)
    V = len(Ep)
    p_acc = np.zeros(V)
    for x in range(V):
        if Eq[x] == 0:
            p_acc[x] = 1.0
            continue
        n = (int(Ep[x]) * Zq * U) // (int(Eq[x]) * Zp) + 1               # U*Eq*Zp <= 2^24*Ep*Zq
        p_acc[x] = min(U, n) / U
    q = np.array([int(e) for e in Eq], dtype=object) / Zq
    reject = float(sum(q[x] * (1 - p_acc[x]) for x in range(V)))
    R = [max(0, int(ep) * Zq - int(eq) * Zp) for ep, eq in zip(Ep, Eq)]
    S = sum(R)
    frac = np.zeros(V)
    if S:
        c_prev = 0
        for v, r in enumerate(R):
            c = c_prev + r
            lo = -(-(c_prev * U) // S)            # smallest U_s with 2^24 * c_prev <= U_s * S ... picks v
            hi = -(-(c * U) // S)
            frac[v] = (min(hi, U) - min(lo, U)) / U
            if r and lo < U:                      # boundary uniforms select v / the token before
                assert oa._inverse_cdf(R, lo) == v
                if lo > 0:
                    assert oa._inverse_cdf(R, lo - 1) < v
            c_prev = c
    dist = np.array([float(q[v]) * p_acc[v] for v in range(V)]) + reject * frac
    p = np.array([int(e) for e in Ep], dtype=np.float64) / Zp
    return dist, p


@pytest.mark.parametrize("seed,V", [(0, 5), (1, 17), (2, 40), (3, 3)])
def test_exact_output_distribution_is_p(seed, V):
    rng = np.random.default_rng(seed)
    t = (rng.standard_normal(V) * 2).astype(np.float32)
    d = (0.8 * t + 0.6 * rng.standard_normal(V) * 2).astype(np.float32)
    dist, p = _first_token_distribution(t, d)
    assert abs(dist.sum() - 1.0) < 2.0 ** -20
    assert np.max(np.abs(dist - p)) < 2.0 ** -22


def test_chi_square_full_function():
    rng = np.random.default_rng(11)
    V, N = 8, 20000
    t_row = rng.standard_normal(V).astype(np.float32)
    d_row = (0.5 * t_row + rng.standard_normal(V)).astype(np.float32)
    q = np.exp(d_row - d_row.max()); q /= q.sum()
    target = np.broadcast_to(np.stack([t_row, t_row]), (N, 2, V)).copy()
    draft = np.broadcast_to(d_row, (N, 1, V)).copy()
    ids = rng.choice(V, size=(N, 1), p=q)
    u = rng.random((N, 1)).astype(np.float32)
    us = rng.random(N).astype(np.float32)
    _, out = oa.accept_rejection(target, draft, ids, u, us)
    counts = np.bincount(out[:, 0], minlength=V)
    p = np.exp(t_row - t_row.max()); p /= p.sum()
    chi2 = float(((counts - N * p) ** 2 / (N * p)).sum())
    assert chi2 < 24.3      # chi-square, 7 degrees of freedom, p = 0.001


def test_equal_distributions_always_accept():
    rng = np.random.default_rng(4)
    t = rng.standard_normal((6, 4, 30)).astype(np.float32)
    ids = rng.integers(0, 30, (6, 3))
    u = (1 - 2.0 ** -24) * np.ones((6, 3), np.float32)    # largest uniform
    acc, out = oa.accept_rejection(t, t[:, :3].copy(), ids, u, rng.random(6).astype(np.float32))
    assert (acc == 3).all() and np.array_equal(out[:, :3], ids)


def test_zero_target_mass_always_rejects():
    rng = np.random.default_rng(5)
    V = 12
    t = rng.standard_normal((4, 2, V)).astype(np.float32)
    d = t[:, :1].copy()
    x = 3
    t[:, 0, x] = -1e4                                         # p(x) = 0 under the contract
    u = np.full((4, 1), 2.0 ** -24, np.float32)               # smallest positive uniform
    acc, out = oa.accept_rejection(t, d, np.full((4, 1), x), u, rng.random(4).astype(np.float32))
    assert (acc == 0).all()
    Ep, Zp, _ = oa.row_weights(t[0, 0])
    Eq, Zq, _ = oa.row_weights(d[0, 0])
    positive = [int(ep) * Zq > int(eq) * Zp for ep, eq in zip(Ep, Eq)]
    assert all(positive[v] for v in out[:, 0]) and x not in out[:, 0]


def _all_accepting_inputs(B, K, V, seed):
    """Draft logits equal to the target's (p == q, so every draft is accepted, U < 2^24)."""
    g = np.random.default_rng(seed)
    target = g.standard_normal((B, K + 1, V)).astype(np.float32)
    draft = target[:, :K].copy()
    ids = g.integers(0, V, (B, K))
    u = g.random((B, K)).astype(np.float32)
    us = g.random(B).astype(np.float32)
    return target, draft, ids, u, us


def test_empty_bonus_row_takes_the_greedy_token():
    """A bonus row with no mass (all NaN, all -inf, or holding +inf: every E is 0) has no
    sampling distribution; the token is then the row's argmax as torch.argmax defines it
    (first NaN, else first +inf, else index 0 of an all -inf row)."""
    B, K, V = 4, 3, 50
    target, draft, ids, u, us = _all_accepting_inputs(B, K, V, 11)
    target[0, K] = np.nan                              # all NaN -> first NaN, index 0
    target[1, K] = -np.inf                             # all -inf -> index 0
    target[2, K, 17] = np.inf                          # +inf among finite values -> 17
    target[2, K, 33] = np.inf
    target[3, K, 5] = np.nan                           # NaN among finite values:
    target[3, K, 9] = np.nan                           # m ignores it, mass stays > 0
    for b in range(3):
        assert oa.row_weights(target[b, K])[1] == 0
    assert oa.row_weights(target[3, K])[1] > 0
    acc, out = oa.accept_rejection(target, draft, ids, u, us)
    assert (acc == K).all()
    assert np.array_equal(out[:, :K], ids)
    assert out[0, K] == 0 and out[1, K] == 0 and out[2, K] == 17
    # a row with mass samples by inverse CDF and never picks a NaN entry (E = 0 there)
    assert out[3, K] not in (5, 9)
    assert out[3, K] == oa._inverse_cdf([int(e) for e in oa.row_weights(target[3, K])[0]],
                                        oa.uniform_fix(us[3]))


def test_out_of_range_draft_ids_are_rejected():
    """Draft ids -1 and V are never accepted: rejection sampling stops at them whatever the
    uniform (u = 0 accepts every valid draft) and samples that position from the residual,
    greedy rejects them as an argmax is always in range, and no emitted id leaves [0, V)."""
    B, K, V = 4, 3, 40
    target, draft, ids, u, us = _all_accepting_inputs(B, K, V, 13)
    u[:] = 0.0
    ids[0, 0] = -1
    ids[1, 1] = V
    ids[2, 2] = -(1 << 40)
    acc, out = oa.accept_rejection(target, draft, ids, u, us)
    assert acc.tolist() == [0, 1, 2, K]
    assert np.array_equal(out[3, :K], ids[3])
    assert ((out >= -1) & (out < V)).all()
    for b in range(3):
        a = int(acc[b])
        assert np.array_equal(out[b, :a], ids[b, :a]) and (out[b, a + 1:] == -1).all()
        # p == q: the residual has no mass, so the token is the target row's argmax
        assert out[b, a] == oa.argmax_first(target[b, a])
    # with p != q the residual after an out-of-range id is sampled as after any rejection
    g = np.random.default_rng(14)
    draft2 = (0.8 * target[:, :K] + 0.6 * g.standard_normal((B, K, V))).astype(np.float32)
    acc2, out2 = oa.accept_rejection(target, draft2, np.full((B, K), V), u, us)
    assert (acc2 == 0).all()
    for b in range(B):
        Ep, Zp, _ = oa.row_weights(target[b, 0])
        Eq, Zq, _ = oa.row_weights(draft2[b, 0])
        R = [max(0, int(ep) * Zq - int(eq) * Zp) for ep, eq in zip(Ep, Eq)]
        assert out2[b, 0] == oa._inverse_cdf(R, oa.uniform_fix(us[b]))
    gacc, gout = oa.accept_greedy(target, np.where(ids < 0, -1, np.minimum(ids, V)))
    assert gacc[0] == 0 and gacc[1] <= 1 and ((gout >= -1) & (gout < V)).all()


def test_empty_rows_pass_the_accept_test():
    """Z = 0 in a target or a draft row makes both sides of the accept test 0."""
    B, K, V = 2, 3, 40
    target, draft, ids, u, us = _all_accepting_inputs(B, K, V, 12)
    draft[0, 1] = np.nan                               # empty draft row at position 1
    target[1, 0] = -np.inf                             # empty target row at position 0
    draft[1, 0] = target[1, 0] + 0                     # keep q(x) = p(x) elsewhere
    u[:] = np.float32(0.999)
    acc, _ = oa.accept_rejection(target, draft, ids, u, us)
    assert (acc == K).all()


def test_multichunk_weights_follow_softmax():
    """Rows over several 8192-entry blocks of 64-entry chunks whose maxima differ: inside
    block 1 one chunk 6 below, one 8 above (the row maximum) and one 40 below (factor F = 0);
    block 2 6 below the others and block 3, a partial one, 40 below (factor G = 0). The
    contract's p = W / Z equals float64 softmax(s) to its precision (2^-19 relative + 2^-29
    absolute), Z is exactly the sum of the weights, the top chunk's weights are E * 2^62 (both
    of its factors 2^31) and the far chunk and block get weight 0. A factor taken against the
    wrong maximum, a chunk or block left out of Z, or a level skipped moves p by orders of
    magnitude more than the bound."""
    rng = np.random.default_rng(5)
    C, BL = oa.CHUNK, oa.BLOCK
    V = 3 * BL + 500
    t = rng.normal(0.0, 2.0, V).astype(np.float32)
    b1 = BL
    t[b1 + C:b1 + 2 * C] -= 6.0          # a chunk below the others of block 1
    t[b1 + 2 * C:b1 + 3 * C] += 8.0      # the row maximum lives in chunk 2 of block 1
    t[b1 + 3 * C:b1 + 4 * C] -= 40.0     # a chunk whose factor is 0
    t[2 * BL:3 * BL] -= 6.0              # a block below the others
    t[3 * BL:] -= 40.0                   # a (partial) block whose factor is 0
    for inv_t in (1.0, 0.7):
        W, Z, M = oa.row_weights(t, inv_t)
        assert Z == int(W.sum())
        s = (t * np.float32(inv_t)).astype(np.float32).astype(np.float64)
        ref = np.exp(s - s.max())
        ref /= ref.sum()
        p = np.array([int(w) / Z for w in W.tolist()])
        # each factor is exp to ~2^-21 relative plus one unit of flooring: |dp| is at most
        # about 3 * 2^-21 p + 3 * 2^62 / Z, with Z >= 2^93 (the row maximum's own weight)
        assert np.all(np.abs(p - ref) <= 2.0 ** -19 * ref + 2.0 ** -29)
        assert np.all(W[b1 + 3 * C:b1 + 4 * C] == 0) and np.all(W[3 * BL:] == 0)
        assert np.all(W[2 * BL:3 * BL] > 0)
        _, m, S, E = oa.row_chunks(t, inv_t)
        assert M == m.max() and np.argmax(m) == b1 // C + 2
        top = W[b1 + 2 * C:b1 + 3 * C]
        assert np.array_equal(top, E[b1 + 2 * C:b1 + 3 * C].astype(object) << 62)
        # the levels: every chunk factor refers to its block's maximum, every block to M
        m2, F, Mb, Sb, E2 = oa.row_blocks(t, inv_t)
        assert np.array_equal(E2, E) and np.array_equal(m2, m)
        cpb = BL // C
        for b in range(len(Mb)):
            assert Mb[b] == m[b * cpb:(b + 1) * cpb].max()
            assert Sb[b] == sum(int(F[c]) * int(S[c]) for c in range(b * cpb, min(len(m), (b + 1) * cpb)))


def test_multichunk_p_equals_q_accepts_and_residual_is_valid():
    """Rows spanning several chunks: p == q always accepts; a rejection samples a token with
    p > q (the residual's support)."""
    rng = np.random.default_rng(6)
    V, K = 2 * oa.CHUNK + 300, 3
    t = rng.normal(0, 1.5, (2, K + 1, V)).astype(np.float32)
    ids = rng.integers(0, V, (2, K))
    u = rng.random((2, K)).astype(np.float32)
    us = rng.random(2).astype(np.float32)
    acc, _ = oa.accept_rejection(t, t[:, :K].copy(), ids, u, us)
    assert (acc == K).all()
    d = t[:, :K].copy()
    d[:, :, :oa.CHUNK] += 4.0                       # q puts its mass on chunk 0
    ids[:] = 5                                      # drafts from the region q favours
    acc, out = oa.accept_rejection(t, d, ids, np.full((2, K), 0.999, np.float32), us)
    for b in range(2):
        a = int(acc[b])
        if a < K:
            Wp, Zp, _ = oa.row_weights(t[b, a])
            Wq, Zq, _ = oa.row_weights(d[b, a])
            x = int(out[b, a])
            assert int(Wp[x]) * Zq > int(Wq[x]) * Zp
