"""CPU pinning of oracle/deltanet_chunked.py (the chunked prefill restatement).

- HF transformers' torch_chunk_gated_delta_rule vectors (tests/golden/deltanet_chunked_hf.npz,
  float32 there): out and final state within 2e-5 of the float64 oracle, chunk sizes 16,
  32 and 64, lengths that are and are not multiples of the chunk;
- the token-by-token recurrence (a different algorithm, float64): equal to 1e-12, with the
  model's strongly negative gates;
- closed forms: beta = 0 leaves only the decay, S_final = exp(sum g) S_0 per head, and
  out_t = q_t^T S_t; g = 0 with beta = 0 leaves the state unchanged;
- identical pad rows in a chunk (kernels/tests/test_doubling_pad_stability.py:1-19: the
  reference's doubling-product inverse blows up there) stay finite and equal to the
  recurrence.
"""
import os

import numpy as np
import pytest

from oracle import deltanet_chunked as oc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "deltanet_chunked_hf.npz")


def _inputs(Hv, S, seed, K=128, V=128):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((Hv * S, K))
    k = rng.standard_normal((Hv * S, K))
    v = rng.standard_normal((Hv * S, V))
    A_log = rng.standard_normal(Hv)
    dt = rng.standard_normal(Hv) * 0.1
    a = rng.standard_normal((Hv, S))
    g = (-np.exp(A_log)[:, None] * np.log1p(np.exp(a + dt[:, None]))).reshape(-1, 1)
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((Hv * S, 1))))
    state = rng.standard_normal((Hv * K, V)) * 0.05
    return state, q, k, v, g, beta


def test_against_hf_chunked_vectors():
    z = np.load(GOLDEN)
    for c in sorted({k.split("_")[0] for k in z.files}):
        f = lambda n: z[f"{c}_{n}"]
        out, st = oc.chunked_prefill(f("state"), f("q"), f("k"), f("v"), f("g"), f("beta"),
                                     int(f("C")))
        scale = np.abs(f("out")).max()
        assert np.abs(out - f("out")).max() <= 2e-5 * max(scale, 1.0), c
        assert np.abs(st - f("new_state")).max() <= 2e-5 * max(np.abs(f("new_state")).max(), 1.0), c


@pytest.mark.parametrize("Hv,S,C,seed", [(2, 64, 16, 0), (2, 100, 64, 1), (1, 37, 16, 2),
                                         (3, 130, 32, 3), (1, 1, 64, 4)])
def test_equals_recurrence(Hv, S, C, seed):
    args = _inputs(Hv, S, seed)
    o1, s1 = oc.chunked_prefill(*args, C)
    o2, s2 = oc.recurrent(*args)
    assert np.abs(o1 - o2).max() <= 1e-12
    assert np.abs(s1 - s2).max() <= 1e-12


def test_beta_zero_only_decays():
    state, q, k, v, g, beta = _inputs(2, 70, 5)
    beta[:] = 0.0
    out, st = oc.chunked_prefill(state, q, k, v, g, beta, 32)
    Hv, K, S = 2, 128, 70
    qn = oc.l2_normalize_rows(q.reshape(Hv, S, K)) / np.sqrt(K)
    s0 = state.reshape(Hv, K, K)
    gh = g.reshape(Hv, S)
    for h in range(Hv):
        decay = np.exp(np.cumsum(gh[h]))
        want = (qn[h] @ s0[h]) * decay[:, None]
        assert np.allclose(out.reshape(Hv, S, K)[h], want, rtol=1e-12, atol=1e-15)
        assert np.allclose(st.reshape(Hv, K, K)[h], s0[h] * decay[-1], rtol=1e-12, atol=1e-15)
    g[:] = 0.0
    _, st = oc.chunked_prefill(state, q, k, v, g, beta, 32)
    assert np.array_equal(st, state)


def test_identical_pad_rows_stay_stable():
    state, q, k, v, g, beta = _inputs(1, 128, 6)
    state[:] = 0.0
    q[15:], k[15:], v[15:] = q[15], k[15], v[15]
    g[15:], beta[15:] = g[15], beta[15]
    o1, s1 = oc.chunked_prefill(state, q, k, v, g, beta, 64)
    o2, s2 = oc.recurrent(state, q, k, v, g, beta)
    assert np.all(np.isfinite(s1))
    assert np.abs(s1 - s2).max() <= 1e-10 and np.abs(o1 - o2).max() <= 1e-10


def test_constants():
    m_incl, m_strict, eye = oc.constants(4)
    assert m_incl.tolist() == [[1, 0, 0, 0], [1, 1, 0, 0], [1, 1, 1, 0], [1, 1, 1, 1]]
    assert np.array_equal(m_strict, m_incl - eye)
