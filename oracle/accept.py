"""Acceptance oracle: greedy and rejection sampling (test infrastructure only).

Greedy (pinned against the reference):
- per position argmax with first-index (lowest id) tie-breaking, exactly
  ``logits.argmax(-1)`` (``contrib/qwen3.6-27b/static_decode.py:1313``) and the
  vocab-sharded exact top-1 (``contrib/qwen3.6-35b-a3b/static_decode_35b.py:1532-1570``,
  CPU check ``contrib/qwen3.6-35b-a3b/kernels/tests/test_decode_sharded_lm_cpu.py:7-46``).
  NaN counts as the maximum (first NaN wins), as torch.argmax does.
- accepted a = number of leading drafts equal to the target argmax of the
  position before them; emitted tokens = argmax(t[0..a]).

Rejection sampling (textbook: Leviathan et al. 2023, Alg. 1; Chen et al. 2023).
The reference's sampler lives in an un-vendored vLLM-Neuron fork (pinned at
65ef8b7 on vLLM 0.21, named in ``contrib/qwen3.6-35b-a3b/VLLM_NEURON_ASSESSMENT.md:7-10``);
no reference test or vector covers it, so against the reference it is
"parity unpinned". It is pinned here against the mathematics instead:
exact enumeration of the output distribution on tiny vocabularies, a chi-square
test that emitted tokens follow p, and the special cases p == q (always accept)
and q(x) > 0 = p(x) (always reject, residual = p restricted to p > q)
(tests/test_oracle_accept.py).

Integer softmax contract (shared bit-for-bit with ``csrc/spec_accept.hip``), built so
that one pass over the logits gives every sum, in three levels: each vocabulary chunk's
values are referred to the chunk's own maximum, each chunk to its block's maximum and each
block to the row maximum, by exact integer factors:
- s_v = t_v * inv_temp (fp32 multiply). The vocabulary is cut into chunks of CHUNK = 64
  entries and blocks of BLOCK = 8192 entries (128 chunks); m_c = max of the non-NaN s_v of
  chunk c (-inf if none), M_b = max of block b's m_c, M = max_b M_b. (64 divides every
  column group of the LM-head GEMM, whose epilogue produces m_c and S_c of the target rows
  while their logits are still in registers; the block level lets one pass over plain
  logits write only 20 bytes per block.)
- E_v = floor(2^31 * exp_c(s_v - m_c)) for v in chunk c (fp32 subtraction; NaN gives 0),
  F_c = floor(2^31 * exp_c(m_c - M_b)) for c in block b, G_b = floor(2^31 * exp_c(M_b - M)),
  each at most 2^31, with exp_c the fp32 Cody-Waite reduction + degree-7 Taylor polynomial
  below, evaluated with correctly rounded fp32 fused multiply-adds (IEEE-754
  fusedMultiplyAdd), so every step is one IEEE-754 operation that CPU and GPU round
  identically.
- The weight of v is W_v = E_v * F_c * G_b (an integer of at most 2^93) and the row's total
  is Z = sum_v W_v = sum_b G_b * S_b with S_b = sum_{c in b} F_c * S_c and
  S_c = sum_{v in c} E_v, in exact integers (order-independent; Z <= V * 2^93 <= 2^113 for
  V <= 2^20). W_v / Z approximates softmax(s)_v to about 2^-29 relative for every entry
  within 21 of its chunk maximum, in a chunk within 21 of its block maximum, in a block
  within 21 of M.
- p(v) = W^p_v / Z_p, q(v) = W^q_v / Z_q. Uniforms u are read as U = floor(u * 2^24).
- Accept draft x at position i iff U * W^q_x * Z_p <= 2^24 * W^p_x * Z_q
  (integers below 2^231).
- At the first rejection sample from R_v = max(0, W^p_v Z_q - W^q_v Z_p); if all
  K drafts are accepted sample the bonus from R_v = W^p_v of row K. The token is
  the smallest v with 2^24 * sum_{w<=v} R_w > U_s * sum_w R_w (integers below 2^251).
- Draft ids outside [0, V) are never accepted: such a position is a rejection whatever the
  uniform, and its token is sampled from the residual R as for any rejection (greedy
  acceptance rejects them too, since an argmax is always in range). Emitted ids therefore
  always lie in [0, V).
- Rows without mass: Z = 0 when no entry is finite relative to the maximum (all NaN or
  -inf, or a +inf entry). Such a target or draft row passes the accept test (both sides
  are 0). A residual after a test that failed always has mass (sum_v (W^p_v Z_q - W^q_v Z_p)
  = 0 with a negative term at the rejected token), so only a bonus row, or the residual
  after an out-of-range draft id when W^p Z_q == W^q Z_p everywhere, can be empty; the
  token is then the greedy one, argmax of the target row (NaN counts as the maximum, first
  index on ties).
"""
import numpy as np

# ---- fp32 fused multiply-add --------------------------------------------------------

def fma32(a, b, c):
    """fp32 a*b + c with one rounding (IEEE-754 fusedMultiplyAdd, round to nearest even),
    elementwise. a*b is exact in float64 (24 + 24 significant bits); the float64 sum is
    rounded to odd (round to nearest, then the neighbour with an odd last bit when the
    TwoSum error is nonzero), which makes its rounding to fp32 the correctly rounded result
    since 53 >= 24 + 2 (Boldo & Melquiond, "Emulation of FMA and correctly rounded sums:
    proved algorithms using rounding to odd", IEEE Trans. Computers 57(4), 2008)."""
    a = np.asarray(a, np.float32).astype(np.float64)
    b = np.asarray(b, np.float32).astype(np.float64)
    c = np.asarray(c, np.float32).astype(np.float64)
    p = a * b
    s = p + c
    bp = s - p
    err = (p - (s - bp)) + (c - bp)                                  # s + err == p + c exactly
    even = (s.view(np.int64) & 1) == 0
    toward = np.nextafter(s, np.where(err > 0, np.inf, -np.inf))
    return np.where((err != 0) & even, toward, s).astype(np.float32)


# ---- exp_c: Cody-Waite range reduction + Taylor polynomial, fp32 with FMA ------------

_F = np.float32
L2E = _F(1.4426950408889634)                     # log2(e) rounded to fp32
_LN2 = 0.6931471805599453
LN2_HI = np.array([_LN2], np.float32).view(np.uint32) & np.uint32(0xFFFFF000)
LN2_HI = LN2_HI.view(np.float32)[0]              # ln2 with the low 12 mantissa bits cleared
LN2_LO = _F(_LN2 - float(LN2_HI))                # remainder
MAGIC = _F(1.5 * 2.0 ** 23)                      # fma(x, L2E, MAGIC) rounds x*L2E to an integer
FIX_BITS = 31                                    # E = floor(2^31 * exp(x))
# Taylor coefficients 1/k! rounded to fp32, k = 7..0, each scaled by 2^FIX_BITS (exact:
# a power of two), so the polynomial evaluates 2^31 * exp(r) directly.
TAYLOR = [_F(_F(1.0 / f) * _F(2.0 ** FIX_BITS)) for f in (5040.0, 720.0, 120.0, 24.0, 6.0, 2.0, 1.0, 1.0)]
X_MIN = _F(-32.0)                                # at and below this 2^31*exp(x) < 1: E = 0
U_BITS = 24                                      # U = floor(u * 2^24)


def expfix(x):
    """E = floor(2^31 * exp_c(x)) for fp32 x <= 0, as uint32 (elementwise).

    Steps (all fp32, one rounding each; fma = fused multiply-add):
      x  = fmax(x, -32)                        (NaN -> -32)
      t  = fma(x, L2E, 1.5*2^23); kf = t - 1.5*2^23    (kf = round(x*log2 e), exact integer)
      r  = fma(-kf, LN2_HI, x); r = fma(-kf, LN2_LO, r)
      p  = Horner with fma over the coefficients 2^31/k!, k = 7..0   (p ~ 2^31 exp(r))
      E  = trunc(p * 2^kf), the scaling done exactly by adding kf to p's exponent field
           (kf * 2^23 added to the bit pattern; the low bits of t's pattern hold kf)
    """
    x = np.fmax(np.asarray(x, np.float32), X_MIN).astype(np.float32)
    t = fma32(x, L2E, MAGIC)
    kf = (t - MAGIC).astype(np.float32)
    r = fma32(-kf, LN2_HI, x)
    r = fma32(-kf, LN2_LO, r)
    p = np.full_like(r, TAYLOR[0])
    for c in TAYLOR[1:]:
        p = fma32(p, r, c)
    bits = (p.view(np.uint32) + (t.view(np.uint32) << np.uint32(23))).astype(np.uint32)
    return bits.view(np.float32).astype(np.uint32)


CHUNK = 64                                       # vocabulary entries per chunk
BLOCK = 8192                                     # vocabulary entries per block (128 chunks)


def row_chunks(logits_row, inv_temp=1.0):
    """(s fp32 [V], m [nch] fp32 chunk maxima, S [nch] python ints, E [V] uint32) of one row."""
    s = (np.asarray(logits_row, np.float32) * _F(inv_temp)).astype(np.float32)
    V = s.shape[0]
    nch = (V + CHUNK - 1) // CHUNK
    seg = np.full(nch * CHUNK, np.nan, np.float32)     # a partial last chunk padded with NaN
    seg[:V] = s
    seg = seg.reshape(nch, CHUNK)
    m = np.fmax.reduce(seg, axis=1, initial=_F(-np.inf)).astype(np.float32)  # NaN ignored
    with np.errstate(invalid="ignore"):                # -inf - -inf and NaN entries: E = 0
        E = expfix((seg - m[:, None]).astype(np.float32))
    S = E.sum(axis=1, dtype=np.uint64).tolist()        # each below 64 * 2^31 + 1
    return s, m, S, E.reshape(-1)[:V]


def row_blocks(logits_row, inv_temp=1.0):
    """(m [nch] chunk maxima, F [nch] uint32 chunk factors, Mb [nb] block maxima,
    Sb [nb] python ints, E [V] uint32) of one row: F_c = expfix(m_c - M_b),
    S_b = sum_{c in b} F_c * S_c."""
    _, m, S, E = row_chunks(logits_row, inv_temp)
    cpb = BLOCK // CHUNK
    nch = m.shape[0]
    nb = (nch + cpb - 1) // cpb
    mp = np.full(nb * cpb, -np.inf, np.float32)
    mp[:nch] = m
    Mb = np.fmax.reduce(mp.reshape(nb, cpb), axis=1, initial=_F(-np.inf)).astype(np.float32)
    with np.errstate(invalid="ignore"):
        F = expfix((m - np.repeat(Mb, cpb)[:nch]).astype(np.float32))
    Fi, Si = F.tolist(), S
    Sb = [sum(Fi[c] * Si[c] for c in range(b * cpb, min(nch, (b + 1) * cpb))) for b in range(nb)]
    return m, F, Mb, Sb, E


def row_weights(logits_row, inv_temp=1.0):
    """(W [V] python ints (object array), Z python int, M fp32) for one logits row under the
    contract: W_v = E_v * F_c * G_b (at most 2^93), Z = sum_b G_b * S_b, M the row max."""
    m, F, Mb, Sb, E = row_blocks(logits_row, inv_temp)
    M = np.fmax.reduce(Mb, initial=_F(-np.inf))
    with np.errstate(invalid="ignore"):
        G = expfix((Mb - M).astype(np.float32))
    Gi = G.tolist()
    Z = sum(g * sb for g, sb in zip(Gi, Sb))
    cpb = BLOCK // CHUNK
    FG = np.array([f * Gi[c // cpb] for c, f in enumerate(F.tolist())], dtype=object)
    W = E.astype(object) * np.repeat(FG, CHUNK)[:E.shape[0]]
    return W, Z, M


def uniform_fix(u):
    """U = floor(u * 2^24) for fp32 u in [0, 1)."""
    return int((np.float32(u) * _F(1 << U_BITS)).astype(np.float32).astype(np.uint32))


def _inverse_cdf(weights, U):
    """Smallest v with 2^24 * cumsum(weights)[v] > U * sum(weights); weights are python ints."""
    total = sum(weights)
    target = U * total
    c = 0
    for v, w in enumerate(weights):
        c += w
        if (c << U_BITS) > target:
            return v
    raise AssertionError("inverse CDF found no token (all-zero weights)")


def accept_rejection(target, draft, draft_ids, u_accept, u_sample, inv_temp=1.0):
    """target [B, K+1, V] f32, draft [B, K, V] f32, draft_ids [B, K] int,
    u_accept [B, K] f32, u_sample [B] f32 -> (accepted int32 [B], out_ids int64 [B, K+1]).
    out_ids[b, :a] = drafts, out_ids[b, a] = residual/bonus sample, rest = -1."""
    target = np.asarray(target, np.float32)
    draft = np.asarray(draft, np.float32)
    B, T, V = target.shape
    K = T - 1
    accepted = np.zeros(B, np.int32)
    out = np.full((B, T), -1, np.int64)
    for b in range(B):
        a = K
        for i in range(K):
            Ep, Zp, _ = row_weights(target[b, i], inv_temp)
            Eq, Zq, _ = row_weights(draft[b, i], inv_temp)
            x = int(draft_ids[b, i])
            if x < 0 or x >= V:                  # out-of-range draft id: a rejection
                a = i
                break
            U = uniform_fix(u_accept[b, i])
            if U * int(Eq[x]) * Zp > (int(Ep[x]) * Zq << U_BITS):
                a = i
                break
        accepted[b] = a
        out[b, :a] = np.asarray(draft_ids[b, :a], np.int64)
        Us = uniform_fix(u_sample[b])
        if a < K:
            Ep, Zp, _ = row_weights(target[b, a], inv_temp)
            Eq, Zq, _ = row_weights(draft[b, a], inv_temp)
            R = [max(0, ep * Zq - eq * Zp) for ep, eq in zip(Ep.tolist(), Eq.tolist())]
        else:
            Ep, _, _ = row_weights(target[b, K], inv_temp)
            R = Ep.tolist()
        if sum(R) == 0:
            # no sampling mass (only a bonus row whose logits are all NaN / -inf or hold +inf:
            # every E is 0): the row's greedy token, NaN counting as the maximum
            out[b, a] = int(argmax_first(target[b, a]))
        else:
            out[b, a] = _inverse_cdf(R, Us)
    return accepted, out


def argmax_first(logits):
    """argmax over the last axis, first index on ties, NaN counts as maximum."""
    return np.argmax(np.asarray(logits, np.float32), axis=-1).astype(np.int64)


def accept_greedy(target, draft_ids):
    """target [B, K+1, V] f32, draft_ids [B, K] -> (accepted int32 [B], out_ids int64 [B, K+1])."""
    tid = argmax_first(target)                                          # [B, K+1]
    B, T = tid.shape
    K = T - 1
    d = np.asarray(draft_ids, np.int64)
    match = d == tid[:, :K]
    accepted = np.where(match.all(axis=1), K, np.argmin(match, axis=1)).astype(np.int32)
    out = np.full((B, T), -1, np.int64)
    for b in range(B):
        a = int(accepted[b])
        out[b, :a + 1] = tid[b, :a + 1]
    return accepted, out
