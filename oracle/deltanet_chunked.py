"""Chunked gated-DeltaNet prefill oracle (test infrastructure only).

Restates, in numpy float64, the op ``deltanet::chunked_prefill``
(``contrib/qwen3.6-27b/kernels/deltanet_chunked_ops.py:26-42``; kernel
``contrib/qwen3.6-27b/kernels/deltanet_chunked_v2.py:46-105``, host mirror
``contrib/qwen3.6-27b/kernels/deltanet_chunked_v2_ref.py:55-103``):

  state [Hv*K, V], query/key [Hv*S, K] raw, value [Hv*S, V], g/beta [Hv*S, 1], rows
  head-major (row h*S + t); chunk size C = m_incl.shape[0].
  -> (out [Hv*S, V] raw attention output before the gated norm, new_state [Hv*K, V])

Per head, with q and k L2-normalised inside as x * rsqrt(sum x^2 + 1e-6)
(``deltanet_chunked_v2.py:123-134``) and q scaled by 1/sqrt(K), each chunk of C tokens
(``deltanet_chunked_v2_ref.py:67-102``, ``chunked_prefill.py:113-174``):
  g_cum = cumsum(g); dm[a, b] = exp(g_cum[a] - g_cum[b]) for a >= b, else 0
  A_str = -(beta k) k^T * dm, strictly lower; T = (I - A_str)^-1
  U = T (beta v); W = T (beta k * exp(g_cum))
  v_new = U - W S;  out = (q * exp(g_cum)) S + ((q k^T) * dm, lower incl. diagonal) v_new
  S <- exp(g_cum[-1]) S + (k * exp(g_cum[-1] - g_cum))^T v_new
T is formed by forward substitution (the form of ``chunked_prefill.py:131-137``); the
reference's device kernel uses the doubling product (I + A)(I + A^2)(I + A^4)...
(``deltanet_chunked_v2_ref.py:40-52``), equal in exact arithmetic.

A last partial chunk is padded with beta = g = 0 tokens (no effect on the state, outputs
dropped), as ``chunked_prefill.py:67-76`` pads; the reference's device kernel instead
requires S to be a multiple of C (``deltanet_chunked_v2.py:71``).

``recurrent`` is the token-by-token gated delta rule on the same inputs
(``contrib/qwen3.6-27b/kernels/deltanet_full.py:1-37``: S <- S e^g; delta = (v - S^T k)
beta; S <- S + k delta^T; o = S^T q), the closed form the chunked one must equal.

Pinning (tests/test_oracle_deltanet_chunked.py): against ``recurrent`` in float64 (a
different algorithm), against HF transformers' torch_chunk_gated_delta_rule vectors
(tests/golden/deltanet_chunked_hf.npz), closed forms (beta = 0 only decays the state),
and identical pad rows (where the doubling product is documented to blow up,
``kernels/tests/test_doubling_pad_stability.py:1-19``).
"""
import numpy as np

NORM_EPS = 1e-6


def l2_normalize_rows(x):
    """x * rsqrt(sum(x^2) + 1e-6) over the last axis (deltanet_chunked_v2.py:123-134)."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + NORM_EPS)


def _heads(state, query, key, value, g, beta):
    K = query.shape[1]
    V = value.shape[1]
    Hv = state.shape[0] // K
    S = query.shape[0] // Hv
    f = lambda a, d: np.asarray(a, np.float64).reshape(Hv, S, d)
    return (np.asarray(state, np.float64).reshape(Hv, K, V), f(query, K), f(key, K),
            f(value, V), f(g, 1)[..., 0], f(beta, 1)[..., 0], Hv, S, K, V)


def recurrent(state, query, key, value, g, beta):
    """Token-by-token rule with the same input normalisation. Returns (out, new_state)
    in the op's layouts, float64."""
    St, q, k, v, g, b, Hv, S, K, V = _heads(state, query, key, value, g, beta)
    q = l2_normalize_rows(q) / np.sqrt(K)
    k = l2_normalize_rows(k)
    out = np.zeros((Hv, S, V))
    St = St.copy()
    for h in range(Hv):
        s = St[h]
        for t in range(S):
            s = s * np.exp(g[h, t])
            delta = (v[h, t] - k[h, t] @ s) * b[h, t]
            s = s + np.outer(k[h, t], delta)
            out[h, t] = q[h, t] @ s
        St[h] = s
    return out.reshape(Hv * S, V), St.reshape(Hv * K, V)


def _unit_lower_inverse(A):
    """(I - A)^-1 for strictly lower-triangular A, by forward substitution:
    row i of T is e_i + A[i, :i] T[:i]."""
    C = A.shape[0]
    T = np.eye(C)
    for i in range(1, C):
        T[i, :i] = A[i, :i] @ T[:i, :i]
    return T


def chunked_prefill(state, query, key, value, g, beta, C):
    """The op on numpy arrays (any float dtype in, float64 out)."""
    St, q, k, v, g, b, Hv, S, K, V = _heads(state, query, key, value, g, beta)
    q = l2_normalize_rows(q) / np.sqrt(K)
    k = l2_normalize_rows(k)
    n = -(-S // C)
    pad = n * C - S
    if pad:
        z = lambda a: np.concatenate([a, np.zeros(a.shape[:1] + (pad,) + a.shape[2:])], 1)
        q, k, v, g, b = z(q), z(k), z(v), z(g), z(b)
    lower = np.tril(np.ones((C, C)))
    strict = np.tril(np.ones((C, C)), -1)
    out = np.zeros((Hv, n * C, V))
    St = St.copy()
    for h in range(Hv):
        s = St[h]
        for c in range(n):
            sl = slice(c * C, (c + 1) * C)
            qc, kc, vc, gc, bc = q[h, sl], k[h, sl], v[h, sl], g[h, sl], b[h, sl]
            g_cum = np.cumsum(gc)
            dm = np.exp((g_cum[:, None] - g_cum[None, :]) * lower) * lower
            A = -((bc[:, None] * kc) @ kc.T) * dm * strict
            T = _unit_lower_inverse(A)
            U = T @ (bc[:, None] * vc)
            W = T @ (bc[:, None] * kc * np.exp(g_cum)[:, None])
            v_new = U - W @ s
            intra = (qc @ kc.T) * dm
            out[h, sl] = (qc * np.exp(g_cum)[:, None]) @ s + intra @ v_new
            tot = g_cum[-1]
            s = s * np.exp(tot) + (kc * np.exp(tot - g_cum)[:, None]).T @ v_new
        St[h] = s
    return out[:, :S].reshape(Hv * S, V), St.reshape(Hv * K, V)


def constants(C):
    """The [C, C] constants the reference op takes (m_incl: i >= j, m_strict: i > j, eye),
    deltanet_chunked_v2_ref.py:26-37."""
    i = np.arange(C)[:, None]
    j = np.arange(C)[None, :]
    return (i >= j).astype(np.float32), (i > j).astype(np.float32), np.eye(C, dtype=np.float32)
