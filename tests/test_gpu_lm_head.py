"""Greedy decision straight from the LM head (fp8::matmul_argmax, spec::accept_greedy_fused):
the reference takes logits.argmax(-1) of the bf16 LM-head output
(contrib/qwen3.6-27b/static_decode.py:546, :1313); here the GEMM reduces each row in its
epilogue and never writes the logits.

Bars:
  - against fp8::matmul + torch.argmax on the GPU (same GEMM accumulation, so the same bf16
    logits): ids and values bit-exact, ties to the lowest column, at the 27B vocabulary
    (N = 248320) through both GEMM kernels (M = 256: rounds of the wide kernel; M = 40);
  - against the oracle (fp64 product, bf16 rounding, first-index argmax) at a small size: the
    chosen logit is within one bf16 ulp of the oracle's maximum, and the ids agree wherever
    the oracle's top two are more than two ulps apart;
  - accept_greedy_fused == accept_greedy over the materialised logits, bit-exact;
  - the row-max epilogue (npn_fp8_matmul_rowmax): its logits bit-identical to fp8::matmul's,
    and the max over its row-group maxima equal to each row's max with NaN ignored, including
    rows made ±inf and NaN by an infinite activation;
  - accept_rejection_lm_head == accept_rejection over the fp32 cast of the same logits,
    bit-exact (accepted lengths, ids and the logits it returns), at the 27B verify batch
    (M = 256, wide kernel) and a small one (M = 64, narrow kernel), temperature 1 and 1/0.7;
  - the contract statistics its GEMM epilogue produces: every row's Z and M (left in the
    workspace) bit-identical to accept_rejection's and to the oracle's row_weights, through
    both GEMM kernels (M = 256 wide, M = 32 narrow), with +-inf and NaN logits in some rows;
  - the argmax epilogue with planted exact ties (copies of a row's best column at lower and
    higher columns, in other column groups) and NaN columns, through the wide kernel in rounds
    (M = 256, N = 248320), in one round (N = 34816) and the narrow kernel (M = 40), against
    fp8::matmul + torch.argmax.
"""
import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle.numerics import bf16_bits_to_f32, f32_to_bf16_bits

pytestmark = pytest.mark.gpu


def _gpu_weights(K, N, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn(K, N, generator=g, device="cuda") * 60).clamp(-448, 448)
    w = w.to(torch.float8_e4m3fn).view(torch.int8)
    sc = (torch.rand(N, 1, generator=g, device="cuda") + 0.5) * 1e-3
    return w, sc


@pytest.mark.parametrize("M,K,N", [(256, 5120, 248320), (40, 5120, 248320), (256, 1024, 4096),
                                   (13, 512, 1024), (13, 256, 320), (40, 256, 832)])
def test_matmul_argmax_equals_torch_argmax(ops, M, K, N):
    g = torch.Generator(device="cuda").manual_seed(M + N)
    x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    w, sc = _gpu_weights(K, N, M + K)
    vals, ids = ops.fp8.matmul_argmax(x, w, sc)
    logits = ops.fp8.matmul(x, w, sc).float()
    ref_vals, ref_ids = logits.max(dim=-1)
    torch.cuda.synchronize()
    assert torch.equal(ids, torch.argmax(logits, dim=-1))
    assert torch.equal(ids, ref_ids) and torch.equal(vals, ref_vals)


@pytest.mark.parametrize("M,K,N,nan_cols", [(256, 256, 248320, False), (256, 256, 248320, True),
                                            (256, 512, 34816, True), (40, 256, 151936, False),
                                            (40, 256, 151936, True)])
def test_matmul_argmax_ties_and_nan(ops, M, K, N, nan_cols):
    """Exact ties at the row maximum: the best columns of some rows copied (weights and scale)
    to lower and higher columns in other column groups, so the lowest copy must win; with
    nan_cols, two columns made NaN by an e4m3fn NaN weight, so every row takes the first."""
    g = torch.Generator(device="cuda").manual_seed(N + K + M)
    x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    w, sc = _gpu_weights(K, N, N)
    best = ops.fp8.matmul(x, w, sc).float().argmax(1)
    rng = np.random.default_rng(N + M)
    for m in rng.choice(M, min(M, 24), replace=False).tolist():
        j = int(best[m])
        for dst in (j // 3, (j + N) // 2, int(rng.integers(0, N))):
            if dst != j:
                w[:, dst] = w[:, j]
                sc[dst] = sc[j]
    if nan_cols:
        for c in (N // 3 + 5, 2 * N // 3 + 1):
            w[7, c] = 0x7F                             # e4m3fn NaN
    vals, ids = ops.fp8.matmul_argmax(x, w, sc)
    logits = ops.fp8.matmul(x, w, sc).float()
    torch.cuda.synchronize()
    assert torch.equal(ids, torch.argmax(logits, dim=-1))
    if nan_cols:
        assert (ids == N // 3 + 5).all() and torch.isnan(vals).all()
    else:
        assert torch.equal(vals, logits.max(dim=-1).values)
        ties = (logits == logits.max(dim=-1, keepdim=True).values).sum(1)
        assert (ties >= 2).sum() >= min(M, 24) // 2    # the planted ties are there


def test_matmul_argmax_matches_oracle(ops):
    M, K, N = 16, 512, 1024
    rng = np.random.default_rng(3)
    x = rng.standard_normal((M, K)).astype(np.float32)
    xb = f32_to_bf16_bits(x)
    w_bits = f32_to_bf16_bits(rng.standard_normal((N, K)).astype(np.float32) * 0.02)
    wq, sc = ofp8.quantize_fp8_per_channel(w_bits)
    ref = ofp8.fp8_matmul(xb, wq, sc)                       # float64 [M, N], before the cast
    rf = bf16_bits_to_f32(f32_to_bf16_bits(ref.astype(np.float32))).astype(np.float64)
    xt = torch.from_numpy(xb.view(np.int16)).cuda().view(torch.bfloat16)
    wt = torch.from_numpy(np.ascontiguousarray(wq).view(np.int8)).cuda()
    st = torch.from_numpy(np.asarray(sc, np.float32).reshape(N, 1)).cuda()
    vals, ids = ops.fp8.matmul_argmax(xt, wt, st)
    torch.cuda.synchronize()
    ids = ids.cpu().numpy()
    top = np.sort(rf, axis=1)
    for m in range(M):
        mx = top[m, -1]
        ulp = 2.0 ** (np.floor(np.log2(abs(mx))) - 7)
        assert abs(rf[m, ids[m]] - mx) <= ulp, m
        if top[m, -1] - top[m, -2] > 2 * ulp:
            assert ids[m] == int(np.argmax(rf[m])), m


def test_accept_greedy_fused(ops):
    B, K, H, V = 8, 7, 5120, 248320
    T = K + 1
    g = torch.Generator(device="cuda").manual_seed(9)
    hid = torch.randn(B * T, H, generator=g, device="cuda").to(torch.bfloat16)
    w, sc = _gpu_weights(H, V, 10)
    logits = ops.fp8.matmul(hid, w, sc).float().view(B, T, V)
    best = logits.argmax(-1)
    drafts = best[:, :K].clone()
    # sequence b keeps its first b drafts right, then goes wrong (b = K: all right)
    for b in range(B):
        if b < K:
            drafts[b, b] = (drafts[b, b] + 1) % V
    acc_f, ids_f = ops.spec.accept_greedy_fused(hid, w, sc, drafts)
    acc_r, ids_r = ops.spec.accept_greedy(logits.contiguous(), drafts)
    torch.cuda.synchronize()
    assert torch.equal(acc_f, acc_r) and torch.equal(ids_f, ids_r)
    assert acc_f.tolist() == [min(b, K) for b in range(B)]


def _rowmax(x, w, sc):
    from npn_native import call, query, stream_of
    M, K = x.shape
    N = w.shape[1]
    G = query("npn_fp8_matmul_argmax_groups", M, K, N)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    gmax = torch.empty((M, G), dtype=torch.float32, device=x.device)
    call("npn_fp8_matmul_rowmax", x, w, sc, out, gmax, M, K, N, stream_of(x))
    return out, gmax


@pytest.mark.parametrize("M,K,N", [(256, 5120, 151936), (40, 5120, 248320), (13, 128, 1024),
                                   (13, 128, 320), (40, 256, 832)])
def test_matmul_rowmax(ops, M, K, N):
    """Shapes where fp8::matmul's own plan does not split K either (so its sums are the
    same); the host plan tests pin which shapes split."""
    g = torch.Generator(device="cuda").manual_seed(M + 3 * N)
    x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    w, sc = _gpu_weights(K, N, M + 7)
    # row 0: x[0, 0] = +inf, with W row 0 zero on columns 0..99 -> those logits NaN (inf * 0),
    # the others +-inf; row 1: -inf the same way
    x[0, 0] = float("inf")
    x[1, 0] = float("-inf")
    w[0, :100] = 0
    out, gmax = _rowmax(x, w, sc)
    ref = ops.fp8.matmul(x, w, sc)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    rf = ref.float()
    want = torch.where(torch.isnan(rf), torch.full_like(rf, float("-inf")), rf).amax(1)
    assert torch.equal(gmax.amax(1), want)
    assert torch.isnan(rf[0, :100]).all() and want[0] == float("inf")


@pytest.mark.parametrize("B,V,inv_t", [(32, 151936, 1.0), (8, 151936, 1.0 / 0.7),
                                       (32, 248320, 1.0)])
def test_accept_rejection_lm_head(ops, B, V, inv_t):
    K, H = 7, 5120
    T = K + 1
    g = torch.Generator(device="cuda").manual_seed(B + V)
    hid = torch.randn(B * T, H, generator=g, device="cuda").to(torch.bfloat16)
    w, sc = _gpu_weights(H, V, B + 11)
    logits = ops.fp8.matmul(hid, w, sc).float().view(B, T, V)
    draft = 0.8 * logits[:, :K] + 0.6 * torch.randn(B, K, V, generator=g, device="cuda")
    ids = torch.multinomial(torch.softmax(draft * inv_t, -1).reshape(B * K, V), 1,
                            generator=g).reshape(B, K)
    u = torch.rand(B, K, generator=g, device="cuda")
    us = torch.rand(B, generator=g, device="cuda")
    acc_f, ids_f, lg = ops.spec.accept_rejection_lm_head(hid, w, sc, draft.contiguous(), ids, u,
                                                         us, inv_t)
    acc_r, ids_r = ops.spec.accept_rejection(logits.contiguous(), draft.contiguous(), ids, u, us,
                                             inv_t)
    torch.cuda.synchronize()
    assert torch.equal(lg.float(), logits)
    assert torch.equal(acc_f, acc_r), (acc_f.tolist(), acc_r.tolist())
    assert torch.equal(ids_f, ids_r)
    assert 0 < acc_f.float().mean() < K  # neither all accepted nor all rejected


def _zm(ws, R):
    """Every row's Z (unsigned 128-bit, low word first) and M from a rejection workspace."""
    off = (16 * R + 255) // 256 * 256
    zw = ws[:16 * R].cpu().numpy().view(np.uint64).reshape(R, 2)
    z = [int(lo) | (int(hi) << 64) for lo, hi in zw]
    m = ws[off:off + 4 * R].cpu().numpy().view(np.float32)
    return z, m


@pytest.mark.parametrize("B,V,inv_t", [(32, 248320, 1.0), (4, 151936, 1.0 / 0.7),
                                       (32, 16384, 1.0 / 0.7)])
def test_lm_head_chunk_stats_bit_exact(ops, B, V, inv_t):
    """The LM-head form's rows' Z and M against accept_rejection's and the oracle's. The shapes
    take both routes: the plain GEMM then a statistics pass (B = 32, V = 248320, where the
    chunk-aligned epilogue plan would need an extra round of workgroups) and the statistics
    written by the GEMM epilogue (the narrow kernel at B = 4; the wide kernel at B = 32,
    V = 16384, where both plans fit one round)."""
    from oracle import accept as oa
    from npn_native import call, query, stream_of
    K, H = 7, 1024
    T = K + 1
    g = torch.Generator(device="cuda").manual_seed(B * 3 + V)
    hid = torch.randn(B * T, H, generator=g, device="cuda").to(torch.bfloat16)
    hid[1, 5] = float("inf")                     # rows of +-inf and NaN logits
    hid[T + 2, 7] = float("nan")
    w, sc = _gpu_weights(H, V, B + 5)
    logits = ops.fp8.matmul(hid, w, sc).float().view(B, T, V).contiguous()
    draft = (0.8 * logits[:, :K].nan_to_num(0.0, 50.0, -50.0)
             + 0.6 * torch.randn(B, K, V, generator=g, device="cuda")).contiguous()
    ids = torch.randint(0, V, (B, K), generator=g, device="cuda")
    u = torch.rand(B, K, generator=g, device="cuda")
    us = torch.rand(B, generator=g, device="cuda")
    R = B * (2 * K + 1)
    st = stream_of(hid)
    n_lm = query("npn_accept_rejection_lm_head_workspace_size", B, K, H, V)
    n_pl = query("npn_accept_workspace_size", B, K, V)
    ws_lm = torch.empty(n_lm, dtype=torch.uint8, device="cuda")
    ws_pl = torch.empty(n_pl, dtype=torch.uint8, device="cuda")
    lg = torch.empty((B, T, V), dtype=torch.bfloat16, device="cuda")
    acc = [torch.empty(B, dtype=torch.int32, device="cuda") for _ in range(2)]
    out = [torch.empty((B, T), dtype=torch.int64, device="cuda") for _ in range(2)]
    call("npn_accept_rejection_lm_head", hid, w, sc, draft, ids, u, us, float(inv_t), lg,
         acc[0], out[0], B, K, H, V, ws_lm, n_lm, st)
    call("npn_accept_rejection", logits, draft, ids, u, us, float(inv_t), acc[1], out[1],
         B, K, V, ws_pl, n_pl, st)
    torch.cuda.synchronize()
    torch.testing.assert_close(lg.float(), logits, rtol=0, atol=0, equal_nan=True)
    z_lm, m_lm = _zm(ws_lm, R)
    z_pl, m_pl = _zm(ws_pl, R)
    assert z_lm == z_pl
    assert np.array_equal(m_lm.view(np.uint32), m_pl.view(np.uint32))
    assert torch.equal(acc[0], acc[1]) and torch.equal(out[0], out[1])
    # the oracle, for the rows holding +-inf / NaN and a spread of others
    lc, dc = logits.cpu().numpy(), draft.cpu().numpy()
    for r in sorted({0, 1, T + 2, B * T - 1, B * T, R - 1, (B * T) // 2}):
        row = lc.reshape(B * T, V)[r] if r < B * T else dc.reshape(B * K, V)[r - B * T]
        _, Z, M = oa.row_weights(row, inv_t)
        assert z_lm[r] == Z, f"row {r}"
        assert m_lm[r].view(np.uint32) == np.float32(M).view(np.uint32), f"row {r}"
