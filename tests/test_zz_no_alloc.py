"""GPU check of npn_accept_rejection_noalloc (the rejection acceptance entry point that takes
no workspace and allocates nothing: its kernels use a fixed per-GPU device array) against
npn_accept_rejection with a caller-allocated workspace, through the C ABI.

Two calls in a row share the array: the verify workload (B = 32, K = 7, V = 151936), then a
smaller problem whose rows and chunks sit where the first call left its values, so a read of
a scratch word the second call did not write would change its result. Accepted lengths and
token ids must be bit-identical to the workspace entry point's (and to the oracle's). A
problem whose workspace exceeds the fixed scratch is refused on the host
(NPN_ERR_SCRATCH), before any launch.
"""
import numpy as np
import pytest
import torch

from oracle import accept as oa

pytestmark = pytest.mark.gpu

NPN_ERR_SCRATCH = 7


def _inputs(B, K, V, seed, rho=0.8):
    g = torch.Generator().manual_seed(seed)
    target = torch.randn(B, K + 1, V, generator=g)
    draft = rho * target[:, :K] + (1 - rho * rho) ** 0.5 * torch.randn(B, K, V, generator=g)
    ids = torch.multinomial(torch.softmax(draft, -1).reshape(B * K, V), 1,
                            generator=g).reshape(B, K)
    u, us = torch.rand(B, K, generator=g), torch.rand(B, generator=g)
    return [t.contiguous().cuda() for t in (target, draft, ids, u, us)]


def _with_workspace(B, K, V, args, inv_t):
    from npn_native import call, query, stream_of
    ws = torch.empty(query("npn_accept_workspace_size", B, K, V), dtype=torch.uint8,
                     device="cuda")
    acc = torch.empty(B, dtype=torch.int32, device="cuda")
    out = torch.empty((B, K + 1), dtype=torch.int64, device="cuda")
    call("npn_accept_rejection", *args, inv_t, acc, out, B, K, V, ws, ws.numel(),
         stream_of(args[0]))
    return acc, out


def _noalloc(B, K, V, args, inv_t):
    from npn_native import call, stream_of
    acc = torch.full((B,), -7, dtype=torch.int32, device="cuda")
    out = torch.full((B, K + 1), -7, dtype=torch.int64, device="cuda")
    call("npn_accept_rejection_noalloc", *args, inv_t, acc, out, B, K, V, stream_of(args[0]))
    return acc, out


def test_noalloc_matches_workspace_entry_point(ops):
    for B, K, V, seed, inv_t in ((32, 7, 151936, 41, 1.0), (3, 2, 1000, 42, 0.7)):
        print(f"noalloc case B={B} K={K} V={V} seed={seed}", flush=True)
        args = _inputs(B, K, V, seed)
        acc_n, out_n = _noalloc(B, K, V, args, inv_t)
        acc_w, out_w = _with_workspace(B, K, V, args, inv_t)
        torch.cuda.synchronize()
        assert torch.equal(acc_n, acc_w), (B, K, V)
        assert torch.equal(out_n, out_w), (B, K, V)
        racc, rout = oa.accept_rejection(*(t.cpu().numpy() for t in args), inv_t)
        assert np.array_equal(acc_n.cpu().numpy(), racc)
        assert np.array_equal(out_n.cpu().numpy(), rout)


def test_noalloc_refuses_problems_beyond_the_scratch(ops):
    import ctypes
    from npn_native import lib, query
    B, K, V = 4096, 15, 1 << 20
    assert query("npn_accept_workspace_size", B, K, V) > 4 << 20
    dummy = torch.empty(16, dtype=torch.uint8, device="cuda")
    p = ctypes.c_void_p(dummy.data_ptr())
    status = lib().npn_accept_rejection_noalloc(p, p, p, p, p, 1.0, p, p, B, K, V, None)
    assert status == NPN_ERR_SCRATCH
    assert "scratch" in lib().npn_status_string(status).decode()


def test_noalloc_under_graph_capture(ops):
    """The entry point captured in a HIP graph (after one eager call on the device, which
    looks up the scratch address), replayed on three new input sets copied into the captured
    buffers with eager work and synchronisations between replays: every replay bit-identical
    to npn_accept_rejection on the same inputs."""
    B, K, V, inv_t = 8, 7, 151936, 1.0
    static = _inputs(B, K, V, 50)
    _noalloc(B, K, V, static, inv_t)                     # eager first call on this device
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        acc_g = torch.full((B,), -7, dtype=torch.int32, device="cuda")
        out_g = torch.full((B, K + 1), -7, dtype=torch.int64, device="cuda")
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        from npn_native import call, stream_of
        call("npn_accept_rejection_noalloc", *static, inv_t, acc_g, out_g, B, K, V,
             stream_of(static[0]))
    for seed in (51, 52, 53):
        print(f"noalloc graph replay seed={seed}", flush=True)
        new = _inputs(B, K, V, seed)
        for dst, src in zip(static, new):
            dst.copy_(src)
        acc_w, out_w = _with_workspace(B, K, V, new, inv_t)   # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(acc_g, acc_w), seed
        assert torch.equal(out_g, out_w), seed
