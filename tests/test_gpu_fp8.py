"""GPU parity of fp8::matmul against the oracle (oracle/fp8.py): bf16((x . decode(W)) * scale)
with fp32 accumulation, at the verify-step shapes (M = B*T in {8, 64, 256}, K = 5120,
N in {5120, 17408, 34816}) on sampled columns, the reference's per-rank decode shapes
(contrib/qwen3.6-27b/kernels/tests/test_fp8_matmul.py:217-236, seed 0), split-K, M
not a multiple of 16, and the OCP-only codes 0x78..0x7E (256..448).
The oracle's product is rounded to bf16 as the op's output is, so what remains is the
accumulation order (fp32 MFMA sums vs fp64): the 2e-3 bar, and elementwise one bf16 ulp
(2^-7 relative at most) where that order flips a rounding.
"""
import numpy as np
import pytest
import torch

from oracle import fp8 as of
from oracle.numerics import round_to_bf16
from _util import BF16_ULP, assert_rel_close, bits, fp8_weights

pytestmark = pytest.mark.gpu


def _check(ops, M, K, N, seed, cols=None, fp8_max=448.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w, scale = fp8_weights(N, K, seed + 1, fp8_max=fp8_max)
    got = ops.fp8.matmul(x.cuda(), w.cuda(), scale.reshape(N, 1).cuda())
    torch.cuda.synchronize()
    got = got.float().cpu().double().numpy()
    if cols is not None:
        sel = np.asarray(cols)
        ref = of.fp8_matmul(bits(x), w.numpy()[:, sel], scale.numpy()[sel])
        got = got[:, sel]
    else:
        ref = of.fp8_matmul(bits(x), w.numpy(), scale.numpy())
    assert_rel_close(got, round_to_bf16(ref), out_unit=BF16_ULP, name=f"fp8 M={M} K={K} N={N}")


@pytest.mark.parametrize("M", [1, 8, 13, 64, 100, 256])
def test_small_n(ops, M):
    _check(ops, M, 5120, 512, seed=M)


@pytest.mark.parametrize("M,N", [(8, 320), (40, 576), (64, 1088), (1, 64), (16, 1344)])
def test_partial_last_tile(ops, M, N):
    """N not a multiple of the narrow kernel's 256-column tile: the last tile's W reads past
    N are clamped and its columns past N never stored (K = 1024 also splits K in two)."""
    _check(ops, M, 1024, N, seed=N + M)


@pytest.mark.parametrize("M,K,N", [(8, 1024, 34816), (40, 2048, 17408), (64, 2048, 14336)])
def test_stream_k(ops, M, K, N):
    """Narrow shapes planned as stream-K (each workgroup an equal run of the tiles' k steps,
    a tile's partial sums in up to 8 slots, unused slots zeroed), every column checked."""
    import npn_native
    assert npn_native.query("npn_fp8_matmul_split_k", M, K, N) in (5, 7)
    _check(ops, M, K, N, seed=K + N)


@pytest.mark.parametrize("M,K,N", [(8, 17408, 5120), (16, 6144, 4608)])
def test_split_16(ops, M, K, N):
    """At most 16 rows with few 256-column tiles: split-K 16, every column checked."""
    import npn_native
    assert npn_native.query("npn_fp8_matmul_split_k", M, K, N) == 16
    _check(ops, M, K, N, seed=K + N)


# The nine (M, N) shapes of the FP8 projection workload at K = 5120, each with the plan it
# runs: (kind, split-K or stream-K slots, tile parameter, workgroups); kind 0 = narrow
# kernel on a tiles x split grid, 1 = narrow kernel in stream-K, 2 = wide kernel on 256-row
# tiles (tile parameter: column tiles per wave), 3 = wide kernel on 128-row tiles (tile
# parameter: units of 16 columns per workgroup).
CONFIG3_PLANS = {
    (8, 5120): (0, 16, 1, 320),
    (8, 17408): (1, 7, 1, 476),
    (8, 34816): (1, 5, 1, 512),
    (64, 5120): (0, 8, 4, 160),
    (64, 17408): (1, 7, 4, 476),
    (64, 34816): (1, 5, 4, 512),
    (256, 5120): (3, 4, 10, 256),
    (256, 17408): (3, 2, 18, 248),
    (256, 34816): (3, 1, 18, 248),
}


def _plan(M, K, N):
    import ctypes
    import npn_native
    info = (ctypes.c_int * 4)()
    assert npn_native.lib().npn_fp8_matmul_plan(M, K, N, info) == 0
    return tuple(info)


@pytest.mark.parametrize("M,N", sorted(CONFIG3_PLANS))
def test_config3_every_column(ops, M, N):
    """Every (M, N) of the projection workload at K = 5120, every column against the oracle
    (so every 256-column tile, stream-K slot boundary and wide column group is covered), with
    the plan each shape runs asserted first."""
    K = 5120
    assert _plan(M, K, N) == CONFIG3_PLANS[(M, N)]
    g = torch.Generator().manual_seed(M * 7 + N)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w, scale = fp8_weights(N, K, seed=N + 1)
    got = ops.fp8.matmul(x.cuda(), w.cuda(), scale.reshape(N, 1).cuda())
    torch.cuda.synchronize()
    got = got.float().cpu().double().numpy()
    wn, sn, xb = w.numpy(), scale.numpy(), bits(x)
    flips = 0
    for c0 in range(0, N, 8192):  # column blocks keep the fp64 weights near 300 MB
        c1 = min(N, c0 + 8192)
        ref = of.fp8_matmul(xb, wn[:, c0:c1], sn[c0:c1])
        rref = round_to_bf16(ref)
        assert_rel_close(got[:, c0:c1], rref, out_unit=BF16_ULP,
                         name=f"fp8 M={M} K={K} N={N} cols {c0}:{c1}")
        # where fp32 accumulation and the fp64 sum round differently, they land on adjacent
        # bf16 values, and only where the exact sum sits near a rounding midpoint (rare);
        # outputs near zero (cancellation) are left to the absolute bound above
        diff = got[:, c0:c1] != rref
        diff &= np.abs(rref) >= 1e-3 * np.abs(rref).max()
        r32 = rref.astype(np.float32)
        ulp = np.maximum(np.abs(np.nextafter(r32, np.float32(np.inf)) - rref),
                         np.abs(np.nextafter(r32, np.float32(-np.inf)) - rref))
        ulp = ulp * 2.0 ** 16                           # fp32 ulp -> bf16 ulp (16 fewer bits)
        assert np.all(np.abs(got[:, c0:c1] - rref)[diff] <= ulp[diff] * 1.0001)
        flips += int(diff.sum())
    assert flips <= 0.01 * M * N, f"{flips} of {M * N} outputs differ from the rounded oracle"


# One shape for every 128-row configuration (units per workgroup 4..24, i.e. 1..6 column
# tiles per long quarter, with and without the short quarters), without and with split-K,
# at row counts that leave the last 128-row tile partial (72, 130, 300).
ROWS128_SHAPES = [
    (72, 512, 9216, 1, 4), (72, 512, 17408, 1, 6), (72, 512, 25600, 1, 8),
    (72, 512, 33792, 1, 10), (300, 512, 14336, 1, 12), (130, 512, 25600, 1, 14),
    (300, 512, 19456, 1, 16), (130, 512, 33792, 1, 18), (300, 512, 24576, 1, 20),
    (300, 512, 27648, 1, 22), (300, 512, 30720, 1, 24),
    (72, 1024, 2048, 8, 4), (72, 1024, 5120, 4, 6), (72, 1024, 7168, 4, 8),
    (72, 1024, 9216, 4, 10), (72, 2048, 11264, 4, 12), (72, 2048, 13312, 4, 14),
    (300, 1024, 5120, 4, 16), (130, 2048, 9216, 4, 18), (300, 2048, 6144, 4, 20),
    (300, 2048, 7168, 4, 22)]


@pytest.mark.parametrize("M,K,N,S,U", ROWS128_SHAPES)
def test_rows128_plans(ops, M, K, N, S, U):
    """The wide kernel on 128-row tiles, one shape per configuration: the plan asserted,
    columns of the first, a middle and the last column group plus a random sample against
    the oracle, and, where K is not split, every output bit-identical to the 256-row kernel
    (npn_fp8_matmul_rowmax never takes the 128-row plans, and both sum every output's k
    steps in the same order)."""
    kind, split, units, _ = _plan(M, K, N)
    assert (kind, split, units) == (3, S, U)
    g = torch.Generator().manual_seed(M + K + N)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w, scale = fp8_weights(N, K, seed=N + 3)
    xd, wd, sd = x.cuda(), w.cuda(), scale.reshape(N, 1).cuda()
    got = ops.fp8.matmul(xd, wd, sd)
    if S == 1:
        from npn_native import call, query, stream_of
        G = query("npn_fp8_matmul_argmax_groups", M, K, N)
        ref = torch.empty_like(got)
        gmax = torch.empty((M, G), dtype=torch.float32, device="cuda")
        call("npn_fp8_matmul_rowmax", xd, wd, sd, ref, gmax, M, K, N, stream_of(xd))
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    torch.cuda.synchronize()
    rng = np.random.default_rng(N)
    span = 16 * U
    mid = (N // 2) // span * span
    cols = np.unique(np.concatenate([np.arange(span), np.arange(mid, mid + span),
                                     np.arange(N - span, N), rng.choice(N, 256, replace=False)]))
    ref = of.fp8_matmul(bits(x), w.numpy()[:, cols], scale.numpy()[cols])
    assert_rel_close(got.float().cpu().double().numpy()[:, cols], round_to_bf16(ref),
                     out_unit=BF16_ULP, name=f"fp8 rows128 M={M} K={K} N={N}")


@pytest.mark.parametrize("M,N", [(8, 5120), (64, 17408), (256, 34816)])
def test_verify_shapes_sampled(ops, M, N):
    rng = np.random.default_rng(M)
    cols = np.sort(rng.choice(N, 384, replace=False))
    _check(ops, M, 5120, N, seed=7, cols=cols)


@pytest.mark.parametrize("K,N", [(5120, 4352), (4352, 5120), (5120, 3072), (5120, 256),
                                 (1536, 5120), (5120, 2560)])
def test_reference_decode_shapes(ops, K, N):
    """B=1 per-rank shapes from the reference's kernel test, with its FP8_MAX = 240."""
    _check(ops, 1, K, N, seed=0, fp8_max=240.0)


def test_ocp_only_codes(ops):
    """Weights made only of the codes 0x78..0x7E (256..448, finite only in OCP e4m3fn)."""
    K, N = 128, 64
    codes = np.random.default_rng(0).integers(0x78, 0x7F, size=(K, N)).astype(np.uint8)
    codes[::3] |= 0x80
    w = torch.from_numpy(codes.view(np.int8))
    x = torch.randn(4, K, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    scale = torch.full((N,), 1.0 / 448.0)
    got = ops.fp8.matmul(x.cuda(), w.cuda(), scale.reshape(N, 1).cuda()).float().cpu().numpy()
    ref = of.fp8_matmul(bits(x), codes, scale.numpy())
    assert_rel_close(got, round_to_bf16(ref), out_unit=BF16_ULP, name="ocp codes")


def test_rejects_bad_shapes(ops):
    x = torch.randn(4, 100).to(torch.bfloat16).cuda()
    w = torch.zeros(100, 64, dtype=torch.int8).cuda()
    with pytest.raises(RuntimeError):
        ops.fp8.matmul(x, w, torch.ones(64, 1).cuda())
