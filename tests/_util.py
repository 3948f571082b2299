"""Shared seeded input generators and tolerance checks for the parity tests.

Tolerance (states and outputs, bf16 I/O with fp32 accumulation): relative error
2e-3, measured two ways on every compared tensor:
  - Frobenius: ||got - ref|| / ||ref|| <= 2e-3
  - elementwise: |got - ref| <= 2e-3 * max|ref| + u * |ref|, where u covers the output's
    own rounding: against an unrounded oracle u = 2^-8 for bf16 outputs (half an ulp, at
    most 2^-8 relative at the bottom of a binade), against an oracle rounded to bf16
    u = 2^-7 (where the accumulation order flips a rounding the two differ by one ulp, at
    most 2^-7 relative); u = 0 for fp32 outputs.
Integer and index results (accepted lengths, token ids, cache rows written by
data movement) are compared bit-exactly.
"""
import numpy as np
import torch

REL_TOL = 2e-3
BF16_U = 2.0 ** -8      # half a bf16 ulp, relative (bf16 output vs unrounded oracle)
BF16_ULP = 2.0 ** -7    # one bf16 ulp, relative (bf16 output vs oracle rounded to bf16)


def bits(t):
    """bf16 tensor -> numpy uint16 raw bits."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def f64(t):
    return t.detach().cpu().double().numpy()


def assert_rel_close(got, ref, tol=REL_TOL, out_unit=0.0, name="tensor", scale=None):
    """`scale` (default |ref|) is the per-element magnitude the out_unit term applies to;
    a sum whose operands are larger than the result passes their magnitude, since a
    rounding flip in an operand moves the sum by the operand's ulp."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, f"{name}: shape {got.shape} vs {ref.shape}"
    assert np.all(np.isfinite(got)), f"{name}: non-finite values"
    nref = np.linalg.norm(ref)
    fro = np.linalg.norm(got - ref) / max(nref, 1e-30)
    mag = np.abs(ref) if scale is None else np.asarray(scale, np.float64)
    bound = tol * np.abs(ref).max() + out_unit * mag
    excess = np.abs(got - ref) - bound
    worst = np.max(excess)
    assert fro <= tol, f"{name}: Frobenius relative error {fro:.3e} > {tol}"
    if worst > 0:
        at = np.unravel_index(np.argmax(excess), excess.shape)
        raise AssertionError(f"{name}: elementwise error exceeds bound by {worst:.3e} at "
                             f"{tuple(int(i) for i in at)} (got {got[at]:.6g}, ref {ref[at]:.6g}, "
                             f"magnitude {mag.reshape(excess.shape)[at] if mag.ndim else mag:.6g})")
    return fro


# ---- DeltaNet -------------------------------------------------------------------------

def deltanet_inputs(B, T, Hk, Hv, seed, state_std=0.02, gates="random"):
    """Seeded inputs for a T-token verify. gates="config0" uses A_log = dt_bias = 0
    (g = -softplus(N(0,1)), beta = sigmoid(N(0,1))), as in the single-layer workload."""
    g = torch.Generator().manual_seed(seed)
    D = 128
    QKV = (2 * Hk + Hv) * D
    d = dict(
        state=torch.randn(B, Hv, D, D, generator=g) * state_std,
        mixed_qkv=torch.randn(B, T, QKV, generator=g).to(torch.bfloat16),
        conv_state=torch.randn(B, QKV, 3, generator=g).to(torch.bfloat16),
        conv_weight=torch.randn(QKV, 4, generator=g) * 0.5,
        conv_bias=torch.randn(QKV, generator=g) * 0.1,
        a_out=torch.randn(B, T, Hv, generator=g),
        b_out=torch.randn(B, T, Hv, generator=g),
        z=torch.randn(B, T, Hv, D, generator=g).to(torch.bfloat16),
        A_log=torch.randn(Hv, generator=g) * 0.5,
        dt_bias=torch.randn(Hv, generator=g),
        norm_weight=torch.randn(D, generator=g) * 0.1 + 1.0,
    )
    if gates == "config0":
        d["A_log"] = torch.zeros(Hv)
        d["dt_bias"] = torch.zeros(Hv)
        d["norm_weight"] = torch.ones(D)
    return d


def deltanet_oracle_args(d):
    """Numpy arguments of oracle.deltanet.deltanet_verify for a deltanet_inputs dict."""
    return (d["state"].numpy(), bits(d["mixed_qkv"]), bits(d["conv_state"]),
            d["conv_weight"].numpy(), d["conv_bias"].numpy(), d["a_out"].numpy(),
            d["b_out"].numpy(), bits(d["z"]), d["A_log"].numpy(), d["dt_bias"].numpy(),
            d["norm_weight"].numpy())


def deltanet_flat_device(d, device="cuda"):
    """The reference's flattened layouts ([B*Hv*128,128] state, [B*...] vectors)."""
    B, Hv, D, _ = d["state"].shape
    T = d["mixed_qkv"].shape[1]
    return dict(
        state=d["state"].reshape(B * Hv * D, D).to(device),
        mixed_qkv=d["mixed_qkv"].reshape(-1).to(device),
        conv_state=d["conv_state"].reshape(-1, 3).to(device),
        conv_weight=d["conv_weight"].to(device),
        conv_bias=d["conv_bias"].to(device),
        a_out=d["a_out"].reshape(-1).to(device),
        b_out=d["b_out"].reshape(-1).to(device),
        z=d["z"].reshape(B * T * Hv, D).to(device),
        A_log=d["A_log"].to(device),
        dt_bias=d["dt_bias"].to(device),
        norm_weight=d["norm_weight"].to(device),
    )


# ---- GQA ------------------------------------------------------------------------------

def gqa_verify_inputs(B, T, Hq, Hkv, kv_lens, s_max, seed, theta=1e7):
    """Seeded verify-attention inputs; cache rows beyond kv_len+T are random too (never read
    as valid rows). cos/sin are the reference RoPE table rows at positions kv_len + t."""
    from oracle.gqa import rope_cos_sin
    g = torch.Generator().manual_seed(seed)
    kv_lens = np.asarray(kv_lens, np.int64)
    pos = kv_lens[:, None] + np.arange(T)[None, :]
    cos, sin = rope_cos_sin(pos, theta=theta)
    return dict(
        query=torch.randn(B, T, Hq, 256, generator=g).to(torch.bfloat16),
        gate=torch.randn(B, T, Hq, 256, generator=g).to(torch.bfloat16),
        q_norm=torch.randn(256, generator=g) * 0.1,
        cos=torch.from_numpy(cos),
        sin=torch.from_numpy(sin),
        cache_k=torch.randn(B, Hkv, s_max, 256, generator=g).to(torch.bfloat16),
        cache_v=torch.randn(B, Hkv, s_max, 256, generator=g).to(torch.bfloat16),
        kv_len=torch.from_numpy(kv_lens.astype(np.int32)),
    )


# ---- FP8 ------------------------------------------------------------------------------

def fp8_weights(N, K, seed, fp8_max=448.0, std=0.02):
    """W ~ N(0, std) [N, K], per-channel absmax quantised to e4m3fn (clip +-fp8_max),
    pre-transposed to [K, N] bytes; returns (w_i8 [K,N] torch.int8, scale [N] f32)."""
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(N, K, generator=g) * std).to(torch.bfloat16)
    # static_decode.py:283-304 with FP8_MAX as an argument (torch's e4m3fn cast; the
    # oracle's numpy quantiser is checked against this in test_oracle_fp8.py)
    absmax = w.abs().amax(dim=-1).float().clamp_min(1e-12)
    scale = absmax / fp8_max
    inv = (1.0 / scale).to(torch.bfloat16).unsqueeze(-1)
    wq = (w * inv).clamp(-fp8_max, fp8_max).to(torch.float8_e4m3fn)
    return wq.t().contiguous().view(torch.int8), scale.contiguous()
