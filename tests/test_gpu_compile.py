"""The drop-in ops under torch.compile(fullgraph=True).

The reference runs its decode step as a compiled static graph in which each of its kernels is
an opaque custom call (contrib/qwen3.6-27b/kernels/fp8_matmul_ops.py:3-7, called from
contrib/qwen3.6-27b/static_decode.py:318, :834, :924, :1313). Here dynamo must trace the same
op names through their register_fake implementations without a graph break, and the compiled
function must compute exactly what the eager ops compute. The aot_eager backend runs the
captured graph op by op without generating code, so only this library's kernels compute.
"""
import pytest
import torch

from _util import deltanet_flat_device, deltanet_inputs, fp8_weights

pytestmark = pytest.mark.gpu


def _decode_like(x, w, sc, nw, dn, q, gate, qn, cos, sin, ck, cv, mask, logits, drafts):
    """One of each reference op the decode graph calls, in one function."""
    ops = torch.ops
    y = ops.fp8.matmul(x, w, sc)                                   # projection
    normed = ops.normfuse.rms_norm(y, nw)                          # the harness's rms_norm
    ns, ncs, o = ops.deltanet.full_batched(*dn)                    # DeltaNet decode token
    att = ops.gqa.tail(q, gate, qn, cos, sin, ck, cv, mask)        # GQA attention tail
    acc, ids = ops.spec.accept_greedy(logits, drafts)              # argmax acceptance
    return normed, ns, ncs, o, att, acc, ids


def _inputs():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(8, 1024, generator=g).to(torch.bfloat16).cuda()
    w, sc = fp8_weights(2048, 1024, seed=6)
    nw = (torch.randn(2048, generator=g) * 0.1).cuda()
    d = deltanet_inputs(2, 1, 4, 12, seed=7)
    f = deltanet_flat_device(d)
    dn = [f[k] for k in ("state", "mixed_qkv", "conv_state", "conv_weight", "conv_bias",
                         "a_out", "b_out", "z", "A_log", "dt_bias", "norm_weight")]
    B, HQ, S = 2, 6, 96
    q = torch.randn(B * HQ, 256, generator=g).cuda()
    gate = torch.randn(B * HQ, 256, generator=g).cuda()
    qn = (torch.randn(1, 256, generator=g) * 0.1).cuda()
    cos, sin = torch.randn(1, 64, generator=g).cuda(), torch.randn(1, 64, generator=g).cuda()
    ck = torch.randn(B * S, 256, generator=g).cuda()
    cv = torch.randn(B * S, 256, generator=g).cuda()
    mask = (torch.arange(S) <= 70).float().reshape(1, S).cuda()
    logits = torch.randn(2, 5, 3000, generator=g).cuda()
    drafts = logits[:, :4].argmax(-1)
    drafts[1, 2] = 7
    return (x, w.cuda(), sc.reshape(-1, 1).cuda(), nw, dn, q, gate, qn, cos, sin, ck, cv, mask,
            logits, drafts.contiguous())


def test_compiled_fullgraph_equals_eager(ops):
    import torch._dynamo
    torch._dynamo.reset()
    args = _inputs()
    eager = _decode_like(*args)
    compiled = torch.compile(_decode_like, fullgraph=True, backend="aot_eager")(*args)
    torch.cuda.synchronize()
    assert len(compiled) == len(eager)
    for a, b in zip(compiled, eager):
        assert a.shape == b.shape and a.dtype == b.dtype
        assert torch.equal(a.view(-1).view(torch.uint8) if a.is_floating_point() else a,
                           b.view(-1).view(torch.uint8) if b.is_floating_point() else b)


def test_compiled_graph_holds_the_custom_ops(ops):
    """The captured graph calls the library's ops themselves (no decomposition into torch
    ops, no graph break)."""
    import torch._dynamo
    torch._dynamo.reset()
    graphs = []

    def backend(gm, example_inputs):
        graphs.append(gm)
        return gm.forward

    args = _inputs()
    torch.compile(_decode_like, fullgraph=True, backend=backend)(*args)
    torch.cuda.synchronize()
    assert len(graphs) == 1
    targets = {str(n.target) for n in graphs[0].graph.nodes if n.op == "call_function"}
    for name in ("fp8.matmul", "normfuse.rms_norm", "deltanet.full_batched", "gqa.tail",
                 "spec.accept_greedy"):
        assert any(name in t for t in targets), (name, sorted(targets))
