#!/usr/bin/env python3
"""Benchmark: EAGLE3 verify+accept step on one MI355X.

Workload (the verify-step metric's configuration): a random-init 4-layer slice of the
27B hybrid at whole-model widths (3 gated-DeltaNet layers + 1 GQA layer, each with its
MLP, FP8 W8A16 projections), B = 32 sequences, K = 7 chain drafts (T = 8 verify tokens),
KV lengths U{4096..32768}, rejection-sampling acceptance at temperature 1 over
[32, 8, 151936] target and [32, 7, 151936] draft logits (draft = 0.8 t + 0.6 eps),
then rollback (DeltaNet checkpoint index, conv windows, KV lengths).

A step = layers + acceptance + rollback on inputs resident in HBM. Reported:
  value        committed tokens/s = sum_b (a_b + 1) / t_step
  roofline     the dominant kernel's algorithmic bytes (or FLOPs) per launch over its
               mean launch time (HIP events on the launch stream, over the timed steps)
  cpu_baseline the CPU oracle (numpy) on one sampled sequence of the same step

  python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu-baseline]
"""
import argparse
import gc
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "neuron-pytorch-native_amd")
sys.path[:0] = [ROOT, PKG, os.path.join(PKG, "kernels")]

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
B, K, V = 32, 7, 151936
T = K + 1


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--per-op", action="store_true", help="print per-op timings to stderr")
    p.add_argument("--no-graph", action="store_true",
                   help="time eager steps instead of HIP graph replays of the step")
    p.add_argument("--lm-head", action="store_true",
                   help="time the LM head + greedy acceptance over the 27B vocabulary, fused "
                        "(argmax in the GEMM epilogue) against logits + accept_greedy")
    p.add_argument("--prefill", action="store_true",
                   help="time the chunked gated-DeltaNet prefill (deltanet::chunked_prefill) "
                        "over the 27B layer's 48 v-heads x 4096 prompt tokens")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run a plain 1 GiB device copy 5 times (scales HBM byte counters)")
    return p.parse_args()


COPY_BYTES = 1 << 30
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.txt")


def copy_calibration():
    """A plain device-to-device copy of COPY_BYTES, the reference for FETCH_SIZE / WRITE_SIZE."""
    import torch
    src = torch.empty(COPY_BYTES // 4, dtype=torch.int32, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "launches": 5}))


def measured_traffic(op):
    """HBM bytes per launch of an op's kernels from the committed counter summary, or None.
    Lines read: 'traffic <op> <bytes>' (FETCH_SIZE + WRITE_SIZE per launch, each scaled by
    the plain-copy calibration)."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic" and parts[1] == op:
                    return int(float(parts[2]))
    except OSError:
        pass
    return None


def kv_lengths(seed):
    import numpy as np
    return np.random.default_rng(seed).integers(4096, 32769, size=B).astype(np.int32)


def algorithmic(name, kv_len_mean_rows):
    """(bound, units per launch, unit) for an op name of the step."""
    if name == "deltanet.verify":
        per_seq = 48 * 128 * 128 * 4 * (1 + T) + T * 10240 * 2 + 2 * T * 48 * 4 \
            + 2 * T * 48 * 128 * 2 + 10240 * 3 * 2
        shared = 10240 * 4 * 4 + 10240 * 4 + 2 * 48 * 4 + 128 * 4
        return "hbm", B * per_seq + shared, "B"
    if name == "gqa.tail_verify":
        kv = B * 4 * (kv_len_mean_rows + T) * 256 * 2 * 2
        return "hbm", kv + 3 * B * T * 24 * 256 * 2 + 2 * B * T * 64 * 4, "B"
    if name == "spec.accept_rejection":
        return "hbm", (B * (2 * K + 1) * V + 2 * B * V) * 4, "B"
    if name.startswith("fp8.matmul["):
        m, k, n = (int(v) for v in name[len("fp8.matmul["):-1].split("x"))
        return "mfma", 2 * m * n * k, "FLOP"
    return None, None, None


def cpu_baseline(model, x, logits, budget_s=10.0):
    """Time the numpy oracle on whole sequences of the same step (same weights, KV lengths,
    inputs and logits), one after another until about budget_s of CPU work (at least one).
    The fp8 weights are decoded to float32 once, outside the timed region, as a CPU
    implementation of a static model would keep them."""
    import numpy as np
    import torch
    from oracle import verify_step as ovs
    from oracle.gqa import rope_cos_sin
    from spec_verify_step import DN_HV, DN_QKV
    weights = []
    for L in model.layers:
        d = {"kind": L["kind"], "in_norm": L["in_norm"].cpu().numpy(),
             "post_norm": L["post_norm"].cpu().numpy()}
        for nm in ovs.FP8_WEIGHTS:
            if nm in L:
                d[nm] = (L[nm][0].cpu().numpy(), L[nm][1].cpu().numpy().reshape(-1))
        weights.append(d)
    ovs.decode_weights(weights)
    total, tokens, done = 0.0, 0, []
    for b in range(B):
        L_b = int(model.kv_len[b].item())
        layers = []
        for L, w in zip(model.layers, weights):
            d = dict(w)
            if L["kind"] == "D":
                for nm in ("conv_w", "conv_b", "A_log", "dt_bias", "norm_w"):
                    d[nm] = L[nm].cpu().numpy()
                rng = np.random.default_rng(b)
                d["state"] = rng.standard_normal((1, DN_HV, 128, 128)) * 0.02
                d["conv_state"] = rng.integers(0, 1 << 15, (1, DN_QKV, 3)).astype(np.uint16) & 0x3FFF
            else:
                d["q_norm"], d["k_norm"] = L["q_norm"].cpu().numpy(), L["k_norm"].cpu().numpy()
                rows = L_b + T
                for nm in ("cache_k", "cache_v"):
                    d[nm] = L[nm][b:b + 1, :, :rows].contiguous().cpu().view(torch.int16).numpy().view(np.uint16)
            layers.append(d)
        xb = x[b * T:(b + 1) * T].cpu().view(torch.int16).numpy().view(np.uint16)
        tgt, drf, ids, u, us = (t[b:b + 1].cpu().numpy() for t in logits)
        cos, sin = rope_cos_sin(L_b + np.arange(T)[None, :])
        t0 = time.perf_counter()
        _, acc, _, _ = ovs.verify_step(layers, xb, np.array([L_b]), 1, T, tgt, drf, ids, u, us,
                                       cos, sin)
        total += time.perf_counter() - t0
        tokens += int(acc[0]) + 1
        done.append(L_b)
        if total >= budget_s:
            break
    cores = len(os.sched_getaffinity(0))
    return {"value": round(tokens / total, 4), "unit": "tokens/s", "cores": cores,
            "kind": "port",
            "sample": f"{len(done)} of {B} sequences (kv_len {', '.join(map(str, done))}) "
                      f"through the same 4-layer step, {total:.1f} s; numpy oracle, fp8 "
                      f"weights decoded to float32 once before timing, BLAS on {cores} threads"}


LM_VOCAB = 248320  # Qwen3.6-27B vocabulary (static_decode.py:107)
# untimed calls per variant before its timed ones, at least: with 3 the shader clock has not
# settled for the first variant (measured: fused 0.808 ms per call after 3, 0.772 after 64)
LM_MIN_WARMUP = 64


def lm_head_bench(args):
    """LM head [B*T, 5120] x [5120, 248320] fp8 + greedy acceptance: fused (row argmax in the
    GEMM epilogue, no logits) vs the GEMM writing bf16 logits, a float cast and
    accept_greedy. Two weight copies (2.5 GB) alternate so the weights come from HBM."""
    import torch
    from spec_verify_step import HIDDEN, random_fp8_linear
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(args.seed)
    ws = [random_fp8_linear(LM_VOCAB, HIDDEN, g, dev) for _ in range(2)]
    x = torch.randn(B * T, HIDDEN, generator=g, device=dev).to(torch.bfloat16)
    drafts = torch.randint(0, LM_VOCAB, (B, K), generator=g, device=dev)

    def fused(i):
        w, sc = ws[i % 2]
        return torch.ops.spec.accept_greedy_fused(x, w, sc, drafts)

    def unfused(i):
        w, sc = ws[i % 2]
        logits = torch.ops.fp8.matmul(x, w, sc).float().view(B, T, LM_VOCAB)
        return torch.ops.spec.accept_greedy(logits, drafts)

    res = {}
    warmup = max(args.warmup, LM_MIN_WARMUP)
    for name, fn in (("fused", fused), ("unfused", unfused)):
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s_ev.record()
        for i in range(args.steps):
            fn(i)
        e_ev.record()
        torch.cuda.synchronize()
        res[name] = s_ev.elapsed_time(e_ev) / args.steps
    a_f, o_f = fused(0)
    a_u, o_u = unfused(0)
    flops = 2.0 * B * T * HIDDEN * LM_VOCAB
    print(json.dumps({
        "workload": f"LM head [{B * T}x{HIDDEN}]x[{HIDDEN}x{LM_VOCAB}] fp8 + greedy acceptance, "
                    f"B={B}, K={K}",
        "fused_ms": round(res["fused"], 4), "unfused_ms": round(res["unfused"], 4),
        "fused_tflops": round(flops / res["fused"] / 1e9, 1),
        "weights_gb": round(HIDDEN * LM_VOCAB / 1e9, 3),
        "identical": bool(torch.equal(a_f, a_u) and torch.equal(o_f, o_u)),
        "steps": args.steps, "warmup": warmup}))


PF_HEADS, PF_TOKENS, PF_CHUNK, PF_DIM = 48, 4096, 64, 128
# untimed calls before the timed ones, at least: a call is 0.3 ms, and a few of them leave the
# shader clock below its settled rate (measured: 0.331 ms per call after 3, 0.314 after 64)
PF_MIN_WARMUP = 64
FP32_PEAK_TFLOPS = 157.3       # MI355X dense fp32 MFMA


def prefill_flops_per_chunk(C=PF_CHUNK, d=PF_DIM):
    """Algorithmic FLOPs of one chunk of one head in the chunked form: A (strictly lower) and
    the intra attention (lower) over d, the unit-lower inverse by substitution, k S and q S,
    v_new = T Z and intra v_new (lower), and the state update k^T v_new."""
    strict, lower = C * (C - 1) // 2, C * (C + 1) // 2
    inverse = sum((i - j - 1) for i in range(C) for j in range(i)) * 2
    return (2 * d * strict + 2 * d * lower + inverse + 2 * 2 * C * d * d
            + 2 * 2 * d * lower + 2 * C * d * d)


def prefill_bench(args):
    """deltanet::chunked_prefill on [48 * 4096, 128] fp32 q, k, v (the 27B layer's v-heads over
    a 4096-token prompt, k already repeated to the v-heads), random inputs with the model's
    gate ranges. One head is checked against the float64 oracle; the oracle is timed on a
    bounded CPU sample (one head, 512 tokens)."""
    import numpy as np
    import torch
    import npn_ops  # noqa: F401  (registers torch.ops.deltanet.chunked_prefill)
    from oracle import deltanet_chunked as oc
    dev = "cuda"
    Hv, S = PF_HEADS, PF_TOKENS
    g = torch.Generator(device=dev).manual_seed(args.seed)
    st = torch.randn(Hv * PF_DIM, PF_DIM, generator=g, device=dev) * 0.05
    q, k, v = (torch.randn(Hv * S, PF_DIM, generator=g, device=dev) for _ in range(3))
    a_log = torch.randn(Hv, 1, generator=g, device=dev)
    dt = torch.randn(Hv, 1, generator=g, device=dev) * 0.1
    a_in = torch.randn(Hv, S, generator=g, device=dev)
    gate = (-torch.exp(a_log) * torch.nn.functional.softplus(a_in + dt)).reshape(-1, 1)
    beta = torch.sigmoid(torch.randn(Hv * S, 1, generator=g, device=dev))
    consts = [torch.from_numpy(x).to(dev) for x in oc.constants(PF_CHUNK)]

    def run():
        return torch.ops.deltanet.chunked_prefill(st, q, k, v, gate, beta, *consts)

    warmup = max(args.warmup, PF_MIN_WARMUP)
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s_ev.record()
    for _ in range(args.steps):
        run()
    e_ev.record()
    torch.cuda.synchronize()
    ms = s_ev.elapsed_time(e_ev) / args.steps
    out, new_state = run()
    # parity on head 0 (float64 oracle, the op's 2e-3 relative bar)
    h0 = slice(0, S)
    args0 = [x.detach().cpu().numpy() for x in (st[:PF_DIM], q[h0], k[h0], v[h0], gate[h0],
                                                beta[h0])]
    o_ref, s_ref = oc.chunked_prefill(*args0, PF_CHUNK)
    err = max(float(np.abs(out[h0].cpu().numpy() - o_ref).max() / np.abs(o_ref).max()),
              float(np.abs(new_state[:PF_DIM].cpu().numpy() - s_ref).max()
                    / np.abs(s_ref).max()))
    nch = -(-S // PF_CHUNK)
    flops = prefill_flops_per_chunk() * nch * Hv
    achieved = flops / ms / 1e9
    line = {
        "metric": "chunked prefill prompt tokens/s (one DeltaNet layer, 48 v-heads)",
        "value": round(S / ms * 1e3, 1), "unit": "tokens/s", "ms_per_call": round(ms, 4),
        "higher_is_better": True, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"deltanet::chunked_prefill, {Hv} v-heads x {S} tokens, "
                               f"head dim {PF_DIM}, chunk {PF_CHUNK}"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": FP32_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / FP32_PEAK_TFLOPS, 4),
                     "traffic": None, "scope": "both kernels of the op",
                     "flop_per_chunk_head": prefill_flops_per_chunk(),
                     "bf16_executed_frac": round(3 * achieved / BF16_PEAK_TFLOPS, 4)},
        "products": "fp32 results; matrix products as split bf16 (hi*hi + hi*lo + lo*hi, fp32 "
                    "accumulation), the triangular inverse in fp32",
        "max_rel_err_head0": err, "steps": args.steps, "warmup": warmup,
    }
    if not args.no_cpu_baseline:
        n_tok = 512
        t0 = time.perf_counter()
        reps = 0
        while True:
            oc.chunked_prefill(*(x[:n_tok] if x.shape[0] == S else x for x in args0), PF_CHUNK)
            reps += 1
            if time.perf_counter() - t0 > 5.0:
                break
        cpu_s = (time.perf_counter() - t0) / reps
        line["cpu_baseline"] = {
            "value": round(n_tok / cpu_s / Hv, 2), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"oracle/deltanet_chunked.py (numpy float64) on 1 head x {n_tok} tokens, "
                      f"scaled to {Hv} heads"}
    print(json.dumps(line))


def main():
    args = parse()
    if args.prefill:
        prefill_bench(args)
        return
    if args.copy_calibration:
        copy_calibration()
        return
    if args.lm_head:
        lm_head_bench(args)
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); the verify step is "
              f"measured on a single MI355X", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    from spec_verify_step import HIDDEN, OpTimer, VerifySlice, synthetic_logits

    dev = "cuda"
    torch.manual_seed(args.seed)
    kv_lens = kv_lengths(args.seed)
    # cache rows: the warmup, the graph-timed steps and the per-op eager pass each append T
    s_max = int(kv_lens.max()) + T * (2 * (args.warmup + args.steps) + 6)
    model = VerifySlice(B, K, kv_lens, s_max, pattern="DDDG", seed=args.seed, device=dev)
    g = torch.Generator(device=dev).manual_seed(args.seed + 1)
    x = torch.randn(B * T, HIDDEN, generator=g, device=dev).to(torch.bfloat16)
    logits = synthetic_logits(B, K, V, args.seed + 2, dev)
    kv_start = model.kv_len.clone()

    # Python's garbage collector stays off from here to the end of the per-op pass: a full
    # collection (tens of ms) inside an op's event bracket drains the GPU queue and shows up
    # as that op's time.
    gc.collect()
    gc.disable()
    # Warmup: eager steps (the first starts from the initial DeltaNet state); then the state
    # moves to fixed buffers and the step is captured as HIP graphs (two checkpoint-buffer
    # parities), replayed in the timed region.
    model.step(x, *logits)
    for _ in range(max(args.warmup - 1, 0)):
        model.step(x, *logits)
    model.make_persistent()
    use_graph = not args.no_graph
    if use_graph:
        model.capture(x, *logits)
        for _ in range(args.warmup):
            model.replay()
    run = model.replay if use_graph else (lambda: model.step(x, *logits))
    torch.cuda.synchronize()
    model.committed.zero_()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    tokens = int(model.committed.sum().item())
    ms_per_step = elapsed * 1e3 / args.steps

    # Per-op launch times: HIP events around every op launch on the launch stream, over an
    # eager pass of the same number of steps (same kernels and sizes as the replays), after
    # two untimed eager steps: the first eager allocations after the graph captures may call
    # hipMalloc, which waits for the queued work inside an op's event bracket.
    for _ in range(2):
        model.step(x, *logits)
    torch.cuda.synchronize()
    kv0 = float(model.kv_len.float().mean().item())
    timer = OpTimer()
    model.timer = timer
    model.committed.zero_()
    for _ in range(args.steps):
        model.step(x, *logits)
    torch.cuda.synchronize()
    model.timer = lambda name, fn, *a: fn(*a)
    gc.enable()
    ops = timer.summary()
    # mean prior cache rows seen by the attention over the timed eager steps
    kv_mean_rows = kv0 + float(model.committed.float().mean().item()) * (args.steps - 1) / (2 * args.steps)

    # dominant kernel by total time in the timed steps
    priced = [k for k in ops if algorithmic(k, kv_mean_rows)[0] is not None]
    dom = max(priced, key=lambda k: ops[k]["total_ms"])
    top = max(ops, key=lambda k: ops[k]["total_ms"])
    if top != dom:
        print(f"note: op {top} has the most time but no algorithmic byte/flop count; "
              f"roofline reported for {dom}", file=sys.stderr)
    bound, units, unit = algorithmic(dom, kv_mean_rows)
    mean_s = ops[dom]["mean_ms"] * 1e-3
    if bound == "mfma":
        achieved = units / mean_s / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": BF16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK_TFLOPS, 4), "traffic": None}
    else:
        achieved = units / mean_s / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None}
    roof["traffic"] = measured_traffic(dom)
    roof["kernel"] = dom
    roof["mean_launch_ms"] = round(ops[dom]["mean_ms"], 4)
    roof["units_per_launch"] = units

    if args.per_op:
        for k, v in sorted(ops.items(), key=lambda kv: -kv[1]["total_ms"]):
            bnd, u, un = algorithmic(k, kv_mean_rows)
            rate = ""
            if bnd == "hbm":
                rate = f"{u / (v['mean_ms'] * 1e-3) / 1e9:8.1f} GB/s"
            elif bnd == "mfma":
                rate = f"{u / (v['mean_ms'] * 1e-3) / 1e12:8.1f} TFLOP/s"
            print(f"{k:40s} x{v['launches'] // args.steps:2d}/step {v['mean_ms']:8.4f} ms "
                  f"{v['total_ms'] / args.steps:8.4f} ms/step {rate}", file=sys.stderr)

    cpu = None
    if not args.no_cpu_baseline:
        model.kv_len = kv_start
        cpu = cpu_baseline(model, x, logits)

    line = {
        "metric": "verify-step tokens/s (B=32,K=7) + achieved HBM GB/s vs MI355X peak",
        "value": round(tokens / elapsed, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, N(0,1) activations and logits)",
        "config": {"workload": "EAGLE3 verify+accept+rollback, 4-layer Qwen3.6-27B-width slice "
                               "(3 gated-DeltaNet + 1 GQA, FP8 W8A16 projections), rejection "
                               "sampling at T=1",
                   "batch": B, "draft_len": K, "verify_tokens": T, "vocab": V,
                   "kv_len": "U{4096..32768}", "parallelism": "single GPU"},
        "verified_tokens_per_s": round(B * T * args.steps / elapsed, 1),
        "committed_per_seq": round(tokens / (B * args.steps), 3),
        "timing": ("HIP graph replays of the whole step (two captured graphs, one per "
                   "DeltaNet checkpoint-buffer parity)" if use_graph else "eager steps")
                  + "; per-op launch times from HIP events over an eager pass of as many steps",
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
