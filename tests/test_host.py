"""Host-side checks that need no GPU: the C-ABI library loads and exports every entry
point include/npn_spec_verify.h declares (no compute calls), the host-only size queries and
status texts, shape propagation of every registered op under FakeTensorMode, and that the
ops refuse CPU tensors instead of falling back to a CPU path."""
import os
import re

import pytest
import torch

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "npn_spec_verify.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(npn_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    import npn_native
    lib = npn_native.lib()
    names = _declared()
    assert len(names) >= 29
    for n in names:
        assert hasattr(lib, n), f"{n} declared in the header but not exported"
    assert set(names) == set(npn_native.SIGNATURES)


def test_status_strings_and_version():
    import npn_native
    lib = npn_native.lib()
    assert lib.npn_abi_version() == 102
    assert lib.npn_status_string(0) == b"ok"
    for code in range(1, 7):
        assert lib.npn_status_string(code) not in (b"ok", b"unknown status")
    assert lib.npn_status_string(99) == b"unknown status"


def test_size_queries():
    import npn_native
    q = npn_native.query
    assert q("npn_gqa_tail_verify_workspace_size", 16, 8, 24, 4, 32776) > 0
    assert q("npn_gqa_tail_verify_workspace_size", 16, 8, 24, 4, 4) == 0        # s_max < T
    assert q("npn_gqa_tail_verify_workspace_size", 1, 9, 24, 4, 1024) == 0      # 54 rows > 48
    assert q("npn_accept_workspace_size", 32, 7, 151936) > 0
    assert q("npn_accept_workspace_size", 32, 0, 151936) == 0
    assert q("npn_fp8_matmul_workspace_size", 8, 5120, 17408) >= 0
    assert q("npn_fp8_matmul_workspace_size", 8, 100, 17408) == 0
    # chunked prefill: one 34,048-byte record per (head, 64-token chunk), partial chunks count
    assert q("npn_deltanet_chunked_workspace_size", 48, 4096) == 48 * 64 * 34048
    assert q("npn_deltanet_chunked_workspace_size", 3, 65) == 3 * 2 * 34048
    assert q("npn_deltanet_chunked_workspace_size", 0, 64) == 0
    assert q("npn_deltanet_chunked_workspace_size", 1, (1 << 22) + 1) == 0     # 32-bit offsets
    # full_fp8: mixed_qkv and z (bf16), a and b (f32), each 256-byte aligned, then the split-K
    # partials [S][N] f32 of the qkv and z GEMMs
    fixed = 10240 * 2 + 6144 * 2 + 256 + 256
    parts = sum(q("npn_fp8_matmul_split_k", 1, 5120, n) * n * 4 for n in (10240, 6144))
    assert q("npn_deltanet_full_fp8_workspace_size", 5120, 16, 48) == fixed + parts
    assert q("npn_deltanet_full_fp8_workspace_size", 5100, 16, 48) == 0        # hidden % 64
    assert q("npn_deltanet_full_fp8_workspace_size", 5120, 5, 48) == 0         # Hv % Hk


def test_ops_register_and_propagate_shapes():
    import npn_ops  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode
    B, T, Hk, Hv, D = 2, 8, 16, 48, 128
    QKV = (2 * Hk + Hv) * D
    with FakeTensorMode():
        f32, bf = torch.float32, torch.bfloat16
        st = torch.empty(B * Hv * D, D, dtype=f32)
        args = (torch.empty(B * T * QKV, dtype=bf), torch.empty(B * QKV, 3, dtype=bf),
                torch.empty(QKV, 4), torch.empty(QKV), torch.empty(B * T * Hv),
                torch.empty(B * T * Hv), torch.empty(B * T * Hv, D, dtype=bf), torch.empty(Hv),
                torch.empty(Hv), torch.empty(D))
        ck, out = torch.ops.deltanet.verify_batched(st, *args)
        assert ck.shape == (B * T * Hv * D, D) and out.shape == (B * T * Hv, D)
        y = torch.ops.fp8.matmul(torch.empty(64, 5120, dtype=bf),
                                 torch.empty(5120, 17408, dtype=torch.int8), torch.empty(17408, 1))
        assert y.shape == (64, 17408) and y.dtype == bf
        q = torch.empty(B, T, 24, 256, dtype=bf)
        o = torch.ops.gqa.tail_verify(q, q, torch.empty(256), torch.empty(B, T, 64),
                                      torch.empty(B, T, 64), torch.empty(B, 4, 100, 256, dtype=bf),
                                      torch.empty(B, 4, 100, 256, dtype=bf),
                                      torch.empty(B, dtype=torch.int32))
        assert o.shape == q.shape
        acc, ids = torch.ops.spec.accept_greedy(torch.empty(B, T, 1000),
                                                torch.empty(B, T - 1, dtype=torch.int64))
        assert acc.shape == (B,) and ids.shape == (B, T)
        x = torch.empty(16, 5120, dtype=bf)
        h2, nrm = torch.ops.normfuse.residual_rms_norm(x, x, torch.empty(5120))
        assert h2.shape == nrm.shape == x.shape
        assert torch.ops.normfuse.rms_norm(x, torch.empty(5120)).shape == x.shape
        assert torch.ops.glue.silu_mul(torch.empty(16, 64, dtype=bf)).shape == (16, 32)
        m, zz, a, b = torch.ops.glue.deltanet_split(torch.empty(16, 16512, dtype=bf), 10240, 6144, 48)
        assert (m.shape, zz.shape, a.shape, a.dtype) == ((16, 10240), (16, 6144), (16, 48), f32)
        q, gt, k, v = torch.ops.glue.gqa_split(torch.empty(16, 14336, dtype=bf), 24, 4, 256)
        assert q.shape == gt.shape == (16, 24, 256) and k.shape == v.shape == (16, 4, 256)
        p = torch.ops.fp8.matmul_partials(torch.empty(256, 17408, dtype=bf),
                                          torch.empty(17408, 5120, dtype=torch.int8))
        assert p.shape == (8, 256, 5120) and p.dtype == f32
        h = torch.empty(256, 5120, dtype=bf)
        h2, nrm = torch.ops.normfuse.residual_rms_norm_partials(h, p, torch.empty(5120),
                                                                torch.empty(5120))
        assert h2.shape == nrm.shape == h.shape and nrm.dtype == bf
        m, zz, a, b = torch.ops.glue.deltanet_split_partials(torch.empty(2, 16, 16512),
                                                             torch.empty(16512), 10240, 6144, 48)
        assert (m.shape, m.dtype, zz.shape, a.shape, a.dtype) == ((16, 10240), bf, (16, 6144),
                                                                  (16, 48), f32)
        q, gt, k, v = torch.ops.glue.gqa_split_partials(torch.empty(2, 16, 14336),
                                                        torch.empty(14336), 24, 4, 256)
        assert q.shape == gt.shape == (16, 24, 256) and k.shape == v.shape == (16, 4, 256)
        assert q.dtype == bf
        vals, ids = torch.ops.fp8.matmul_argmax(torch.empty(256, 5120, dtype=bf),
                                                torch.empty(5120, 248320, dtype=torch.int8),
                                                torch.empty(248320))
        assert vals.shape == ids.shape == (256,) and ids.dtype == torch.int64
        acc, oid = torch.ops.spec.accept_greedy_fused(torch.empty(B * T, 5120, dtype=bf),
                                                      torch.empty(5120, 4096, dtype=torch.int8),
                                                      torch.empty(4096),
                                                      torch.empty(B, T - 1, dtype=torch.int64))
        assert acc.shape == (B,) and oid.shape == (B, T)
        c, sn = torch.ops.gqa.rope_rows(torch.empty(100, 64), torch.empty(100, 64),
                                        torch.empty(B, dtype=torch.int32), T)
        assert c.shape == sn.shape == (B, T, 64) and c.dtype == f32
        i8 = torch.int8
        ns, nc, g = torch.ops.deltanet.full_fp8(
            torch.empty(1, 5120, dtype=bf), torch.empty(Hv * D, D), torch.empty(QKV, 3, dtype=bf),
            torch.empty(QKV, 4), torch.empty(QKV), torch.empty(Hv), torch.empty(Hv),
            torch.empty(D), torch.empty(5120, QKV, dtype=i8), torch.empty(QKV, 1),
            torch.empty(5120, Hv * D, dtype=i8), torch.empty(Hv * D, 1),
            torch.empty(5120, Hv, dtype=i8), torch.empty(Hv, 1), torch.empty(5120, Hv, dtype=i8),
            torch.empty(Hv, 1))
        assert ns.shape == (Hv * D, D) and nc.shape == (QKV, 3) and g.shape == (Hv, D)
        assert g.dtype == bf and nc.dtype == bf


def test_fp8_split_k_plan():
    """Split-K factors the GEMM plan picks at the verify step's M = 256 (host code only)."""
    from npn_native import query
    assert query("npn_fp8_matmul_split_k", 256, 17408, 5120) == 8
    assert query("npn_fp8_matmul_split_k", 256, 6144, 5120) == 4
    assert query("npn_fp8_matmul_split_k", 256, 5120, 16512) == 2
    assert query("npn_fp8_matmul_split_k", 256, 5120, 14336) == 2
    assert query("npn_fp8_matmul_split_k", 256, 5120, 34816) == 1
    assert query("npn_fp8_matmul_split_k", 256, 100, 5120) == 0
    # argmax mode never splits K; the LM head's vocabulary runs in rounds of 256 workgroups
    # of the widest tiles (14 units of 16 columns: ceil(15520 / 14) = 1109 groups)
    assert query("npn_fp8_matmul_argmax_groups", 256, 5120, 248320) == 1109
    # below 65 rows: 256-column tiles of 4 column slices (2 at 33..64 rows), and the grid
    # kept at or under 576 workgroups (1152 up to 16 rows)
    assert query("npn_fp8_matmul_argmax_groups", 16, 5120, 248320) == 248320 // 64
    assert query("npn_fp8_matmul_argmax_groups", 32, 5120, 248320) == 248320 // 64
    assert query("npn_fp8_matmul_argmax_groups", 40, 5120, 248320) == 248320 // 128
    for m in (8, 32, 64):
        # stream-K (partial slots per tile): 136 tiles over 512 workgroups, 68 over 476
        assert query("npn_fp8_matmul_split_k", m, 5120, 34816) == 5
        assert query("npn_fp8_matmul_split_k", m, 5120, 17408) == 7
        assert query("npn_fp8_matmul_split_k", m, 5120, 14336) == 7
        # a tiles x split grid: 20 tiles split 8 (16 up to 16 rows)
        assert query("npn_fp8_matmul_split_k", m, 5120, 5120) == (16 if m <= 16 else 8)
        assert query("npn_fp8_matmul_split_k", m, 17408, 5120) == (16 if m <= 16 else 8)
    assert query("npn_fp8_matmul_workspace_size", 64, 5120, 34816) == 5 * 64 * 34816 * 4
    assert query("npn_fp8_matmul_split_k", 8, 256, 1024) == 1           # 8 k steps
    assert query("npn_fp8_matmul_split_k", 8, 512, 1024) == 2


def test_ops_refuse_cpu_tensors():
    """No CPU fallback: the ops are registered for HIP devices only."""
    import npn_ops  # noqa: F401
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    w = torch.zeros(64, 64, dtype=torch.int8)
    with pytest.raises((NotImplementedError, RuntimeError)):
        torch.ops.fp8.matmul(x, w, torch.ones(64, 1))


def test_call_refuses_mixed_devices():
    """The C-ABI takes raw pointers: tensors on two devices are refused before any call."""
    import npn_native
    a, b = torch.zeros(4), torch.zeros(4, device="meta")
    with pytest.raises(RuntimeError, match="span devices"):
        npn_native.call("npn_silu_mul", a, b, 1, 4, None)


def test_rope_tables_match_oracle():
    """The step's table generator (torch fp32, as the reference's _init_rope) and the
    oracle's agree: inv_freq to 1 fp32 ulp, cos/sin tightly where position * ulp is small."""
    import numpy as np
    from oracle.gqa import rope_cos_sin
    from spec_verify_step import rope_tables
    pos = torch.arange(0, 2048, 7).reshape(1, -1)
    c, s = rope_tables(pos)
    rc, rs = rope_cos_sin(pos.numpy())
    np.testing.assert_allclose(c.numpy(), rc, rtol=0, atol=2e-4)
    np.testing.assert_allclose(s.numpy(), rs, rtol=0, atol=2e-4)
    inv_t = 1.0 / (1e7 ** (torch.arange(0, 64, 2).float() / 64))
    inv_o = (1.0 / (1e7 ** (np.arange(0, 64, 2) / 64.0))).astype(np.float32)
    ulps = np.abs(inv_t.numpy().view(np.int32) - inv_o.view(np.int32))
    assert ulps.max() <= 1
