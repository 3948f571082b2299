"""GPU parity of deltanet::full_fp8 (the four fp8 in-projections of one decode token folded
into deltanet::full; contrib/qwen3.6-27b/kernels/deltanet_full_fp8_ops.py:7-32) against the
oracle (oracle.deltanet.deltanet_full_fp8, pinned to HF's DeltaNet layer in
test_oracle_layers.py), at the reference's per-rank shapes (HIDDEN 5120, 4 k / 12 v heads,
seed 11 and state std 0.1 as contrib/qwen3.6-27b/kernels/tests/test_deltanet_full.py:58-73)
at full width (16 / 48 heads), and at 32 / 64 heads (where the qkv and z GEMMs take different
one-row plans and so run as two launches). Weights are the harness's per-channel quantisation of
N(0, 0.02) (static_decode.py:283-304).

Bars: state and gated output within 2e-3 relative (tests/_util.py); the new conv window's
newest column bit-identical to fp8::matmul's mixed_qkv on the GPU (the same GEMM) and its two
older columns to the input window's shift; repeated calls bit-identical.
"""
import numpy as np
import pytest
import torch

from oracle import deltanet as od
from _util import BF16_U, assert_rel_close, bits, fp8_weights

pytestmark = pytest.mark.gpu

HIDDEN, D = 5120, 128


def _inputs(hk, hv, seed, state_std=0.1):
    g = torch.Generator().manual_seed(seed)
    qkv = (2 * hk + hv) * D
    d = dict(
        x=torch.randn(1, HIDDEN, generator=g).to(torch.bfloat16),
        state=torch.randn(hv * D, D, generator=g) * state_std,
        conv_state=torch.randn(qkv, 3, generator=g).to(torch.bfloat16),
        conv_weight=torch.randn(qkv, 4, generator=g) * 0.5,
        conv_bias=torch.randn(qkv, generator=g) * 0.1,
        A_log=torch.randn(hv, generator=g) * 0.5,
        dt_bias=torch.randn(hv, generator=g),
        norm_weight=torch.randn(D, generator=g) * 0.1 + 1.0,
    )
    for i, (name, n) in enumerate((("qkv", qkv), ("z", hv * D), ("a", hv), ("b", hv))):
        w, s = fp8_weights(n, HIDDEN, seed=seed + 100 + i)
        d[f"{name}_w"], d[f"{name}_s"] = w, s.reshape(n, 1)
    return d


def _gpu_args(d):
    names = ("x", "state", "conv_state", "conv_weight", "conv_bias", "A_log", "dt_bias",
             "norm_weight", "qkv_w", "qkv_s", "z_w", "z_s", "a_w", "a_s", "b_w", "b_s")
    return [d[n].cuda() for n in names]


def _oracle(d, hk, hv):
    n = lambda k: d[k].numpy()
    w = lambda k: np.ascontiguousarray(d[k].numpy())
    return od.deltanet_full_fp8(
        bits(d["x"]).reshape(-1), n("state").reshape(hv, D, D).astype(np.float64),
        bits(d["conv_state"]), n("conv_weight"), n("conv_bias"), n("A_log"), n("dt_bias"),
        n("norm_weight"), w("qkv_w"), n("qkv_s").reshape(-1), w("z_w"), n("z_s").reshape(-1),
        w("a_w"), n("a_s").reshape(-1), w("b_w"), n("b_s").reshape(-1), hk, hv)


def _plan_kind(N):
    import ctypes
    import npn_native
    info = (ctypes.c_int * 4)()
    assert npn_native.lib().npn_fp8_matmul_plan(1, HIDDEN, N, info) == 0
    return tuple(info[:2])


# 32 / 64 heads: the qkv GEMM's one-row plan is stream-K (64 tiles) while z's is a tiles x
# split grid, so the two GEMMs run as separate launches instead of one
@pytest.mark.parametrize("hk,hv,seed", [(4, 12, 11), (16, 48, 12), (32, 64, 13)])
def test_full_fp8_matches_oracle(ops, hk, hv, seed):
    if hk == 32:
        assert _plan_kind((2 * hk + hv) * D)[0] == 1 and _plan_kind(hv * D)[0] == 0
    d = _inputs(hk, hv, seed)
    args = _gpu_args(d)
    ns, ncs, out = ops.deltanet.full_fp8(*args)
    mixed = ops.fp8.matmul(args[0], args[8], args[9])
    ns2, ncs2, out2 = ops.deltanet.full_fp8(*args)
    torch.cuda.synchronize()
    s_ref, cs_ref, o_ref = _oracle(d, hk, hv)
    assert_rel_close(ns.cpu().double().numpy().reshape(s_ref.shape), s_ref, name="state")
    assert_rel_close(out.float().cpu().double().numpy().reshape(o_ref.shape), o_ref,
                     out_unit=BF16_U, name="out")
    # conv window: the newest column is the GEMM's bf16 mixed_qkv, the older two the shift
    assert torch.equal(ncs[:, 2].contiguous().view(torch.int16),
                       mixed.reshape(-1).view(torch.int16))
    assert torch.equal(ncs[:, :2].cpu(), d["conv_state"][:, 1:])
    # the oracle's mixed_qkv (float64 products) agrees up to rare one-ulp bf16 flips
    assert np.mean(bits(ncs) == cs_ref) > 0.99
    assert torch.equal(ns, ns2) and torch.equal(ncs, ncs2) and torch.equal(out, out2)


def test_full_fp8_rejects_bad_arguments(ops):
    d = _inputs(4, 12, 3)
    args = _gpu_args(d)
    bad = list(args)
    bad[0] = args[0].reshape(2, HIDDEN // 2)                  # x must be one row
    with pytest.raises(RuntimeError):
        ops.deltanet.full_fp8(*bad)
    bad = list(args)
    bad[12] = args[12][:, :11].contiguous()                   # a_w narrower than Hv
    with pytest.raises(RuntimeError):
        ops.deltanet.full_fp8(*bad)
    bad = list(args)
    bad[9] = args[9].double()                                 # scale dtype
    with pytest.raises(TypeError):
        ops.deltanet.full_fp8(*bad)
    # the C ABI: the new conv window may not be written over the old one (it is written before
    # the token step reads the old one); a short workspace is refused
    from npn_native import call, query, stream_of
    n_ws = query("npn_deltanet_full_fp8_workspace_size", HIDDEN, 4, 12)
    ws = torch.empty(n_ws, dtype=torch.uint8, device="cuda")
    ns = torch.empty_like(args[1])
    out = torch.empty(12, D, dtype=torch.bfloat16, device="cuda")
    cs = args[2].clone()
    with pytest.raises(RuntimeError, match="status 6"):
        call("npn_deltanet_full_fp8", *args, ns, args[2], out, HIDDEN, 4, 12,
             ws, n_ws, stream_of(ws))
    # a partial overlap (the new window one row, 6 bytes, past the old one's start; and one
    # ending a row into it) is refused the same way
    qkv = args[2].shape[0]
    pad = torch.zeros(qkv + 2, 3, dtype=torch.bfloat16, device="cuda")
    pad[1:qkv + 1] = args[2]
    args_pad = list(args)
    args_pad[2] = pad[1:qkv + 1]
    for alias in (pad[2:qkv + 2], pad[0:qkv]):
        with pytest.raises(RuntimeError, match="status 6"):
            call("npn_deltanet_full_fp8", *args_pad, ns, alias, out, HIDDEN, 4, 12,
                 ws, n_ws, stream_of(ws))
    assert torch.equal(pad[1:qkv + 1], args[2])
    with pytest.raises(RuntimeError, match="status 4"):
        call("npn_deltanet_full_fp8", *args, ns, cs, out, HIDDEN, 4, 12, ws, n_ws - 256,
             stream_of(ws))
    torch.cuda.synchronize()
    assert torch.equal(cs, args[2])                           # nothing ran
