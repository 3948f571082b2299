#!/usr/bin/env python3
"""Benchmark: EAGLE3 verify+accept step on one MI355X.

Workload (the verify-step metric's configuration): a random-init 4-layer slice of the
27B hybrid at whole-model widths (3 gated-DeltaNet layers + 1 GQA layer, each with its
MLP, FP8 W8A16 projections), B = 32 sequences, K = 7 chain drafts (T = 8 verify tokens),
KV lengths U{4096..32768}, rejection-sampling acceptance at temperature 1 over
[32, 8, 151936] target and [32, 7, 151936] draft logits (draft = 0.8 t + 0.6 eps),
then rollback (DeltaNet checkpoint index, conv windows, KV lengths).

A step = layers + acceptance + rollback on inputs resident in HBM; consecutive steps use
8 pre-generated logits / uniform sets in turn. Reported:
  value        committed tokens/s = sum_b (a_b + 1) / t_step
  roofline     the dominant kernel family by time per step (every FP8 GEMM shape is one
               family) and its op with the most time: algorithmic bytes (or FLOPs) per
               launch over the mean launch time (HIP events on the launch stream)
  kernels      the same figures for every op of the step
  parity       the numpy oracle on two sequences of the first step, from the same initial
               state, teacher-forced: accepted lengths and ids bit-exact, sublayer outputs
               and states within 2e-3 (the bench exits 1 if not)
  cpu_baseline the batched torch float32 step (oracle/torch_step.py) on the whole first
               step on the host's cores, with the CPU model and thread count

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
N_SETS = 8                     # logits / uniform sets the timed steps use in turn


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--batch", type=int, default=32,
                   help="sequences per step (the workload's B = 32; other values are side runs "
                        "of the same step, labelled with their B)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--per-op", action="store_true", help="print per-op timings to stderr")
    p.add_argument("--no-graph", action="store_true",
                   help="time eager steps instead of HIP graph replays of the step")
    p.add_argument("--lm-head", action="store_true",
                   help="time the LM head + greedy acceptance over the 27B vocabulary, fused "
                        "(argmax in the GEMM epilogue) against logits + accept_greedy, and the "
                        "same for rejection sampling (row maxima in the epilogue)")
    p.add_argument("--prefill", action="store_true",
                   help="time the chunked gated-DeltaNet prefill (deltanet::chunked_prefill) "
                        "over the 27B layer's 48 v-heads x 4096 prompt tokens")
    p.add_argument("--config", type=int, choices=(1, 2, 3),
                   help="one kernel at its workload's shapes: 1 DeltaNet verify at B = 1, 8, "
                        "32; 2 GQA verify attention at B = 16; 3 the FP8 GEMM at nine shapes")
    p.add_argument("--full-fp8", action="store_true",
                   help="time deltanet::full_fp8 (one decode token, fp8 in-projections) at the "
                        "reference's per-rank heads (4/12) and full width (16/48)")
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


def dn_verify_bytes(nseq, hv=48, hk=16, t=T):
    """Algorithmic HBM bytes of one DeltaNet verify launch over nseq sequences: the fp32 state
    read once and t checkpoints written, the bf16 projection rows (q, k, v channels, z) read
    and the output written, the a / b gate inputs, the conv window read, and the per-layer
    constants (conv weights and bias, A_log, dt_bias, norm weight)."""
    qkv = (2 * hk + hv) * 128
    per_seq = hv * 128 * 128 * 4 * (1 + t) + t * qkv * 2 + 2 * t * hv * 4 \
        + 2 * t * hv * 128 * 2 + qkv * 3 * 2
    shared = qkv * 4 * 4 + qkv * 4 + 2 * hv * 4 + 128 * 4
    return nseq * per_seq + shared


def gqa_verify_bytes(kv_lens, hq=24, hkv=4, t=T, dh=256):
    """Algorithmic HBM bytes of one verify-attention launch: every sequence's K and V rows
    [0, kv_len + t) read once (bf16), the query, gate and output rows, and the RoPE rows."""
    rows = sum(int(k) + t for k in kv_lens)
    nseq = len(kv_lens)
    return rows * hkv * dh * 2 * 2 + 3 * nseq * t * hq * dh * 2 + 2 * nseq * t * 64 * 4


def algorithmic(name, kv_len_mean_rows):
    """(bound, units per launch, unit) for an op name of the step; (None, None, None) for
    ops without a count (the glue: norms, splits, RoPE rows, rollback)."""
    if name == "deltanet.verify":
        return "hbm", dn_verify_bytes(B), "B"
    if name == "gqa.tail_verify":
        return "hbm", gqa_verify_bytes([kv_len_mean_rows] * B), "B"
    if name == "gqa.tail_verify_append":  # + the new K/V rows read and written to the cache
        return "hbm", gqa_verify_bytes([kv_len_mean_rows] * B) + 4 * B * T * 4 * 256 * 2, "B"
    if name == "spec.accept_rejection":
        return "hbm", (B * (2 * K + 1) * V + 2 * B * V) * 4, "B"
    if name.startswith(("fp8.matmul[", "fp8.matmul_swiglu[")):
        m, k, n = (int(v) for v in name[name.index("[") + 1:-1].split("x"))
        return "mfma", 2 * m * n * k, "FLOP"
    return None, None, None


def family(name):
    """Kernel family of an op: every FP8 projection shape is one family (one GEMM kernel
    design at several shapes); the others are their own."""
    return "fp8 GEMM" if name.startswith("fp8.") else name


def rate(bound, units, seconds):
    """(achieved, peak, unit) of `units` algorithmic bytes or FLOPs done in `seconds`."""
    if bound == "mfma":
        return units / seconds / 1e12, BF16_PEAK_TFLOPS, "TFLOP/s"
    return units / seconds / 1e9, HBM_PEAK_GBS, "GB/s"


def kernel_table(ops, steps, kv_mean_rows):
    """Per-op rows, by time per step: launches per step, mean launch ms, and for priced ops
    the achieved rate and its fraction of the roofline that bounds the op."""
    rows = []
    for k, v in sorted(ops.items(), key=lambda kv: -kv[1]["total_ms"]):
        row = {"op": k, "per_step": v["launches"] // steps, "mean_ms": round(v["mean_ms"], 4),
               "ms_per_step": round(v["total_ms"] / steps, 4)}
        bound, units, _ = algorithmic(k, kv_mean_rows)
        if bound is not None:
            achieved, peak, unit = rate(bound, units, v["mean_ms"] * 1e-3)
            row.update(bound=bound, achieved=round(achieved, 1), unit=unit,
                       frac=round(achieved / peak, 4))
        rows.append(row)
    return rows


def roofline(ops, steps, kv_mean_rows):
    """The roofline object: the kernel family with the most time per step among priced ops,
    and within it the op with the most time (its mean launch, the dominant kernel); the
    family's aggregate rate beside it."""
    priced = [k for k in ops if algorithmic(k, kv_mean_rows)[0] is not None]
    fam_ms = {}
    for k in priced:
        fam_ms[family(k)] = fam_ms.get(family(k), 0.0) + ops[k]["total_ms"]
    fam = max(fam_ms, key=fam_ms.get)
    members = [k for k in priced if family(k) == fam]
    dom = max(members, key=lambda k: ops[k]["total_ms"])
    bound, units, _ = algorithmic(dom, kv_mean_rows)
    achieved, peak, unit = rate(bound, units, ops[dom]["mean_ms"] * 1e-3)
    digits = 2 if bound == "mfma" else 1
    roof = {"bound": bound, "achieved": round(achieved, digits), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": measured_traffic(dom),
            "kernel": dom, "mean_launch_ms": round(ops[dom]["mean_ms"], 4),
            "units_per_launch": units}
    roof["traffic_source"] = (
        "profiles/hbm_traffic.txt: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE per dispatch, "
        "scaled by a plain 1 GiB copy" if roof["traffic"] is not None else None)
    fam_units = sum(algorithmic(k, kv_mean_rows)[1] * ops[k]["launches"] for k in members)
    fa, _, _ = rate(bound, fam_units, fam_ms[fam] * 1e-3)
    roof["family"] = {"name": fam, "ops": len(members),
                      "ms_per_step": round(fam_ms[fam] / steps, 4),
                      "achieved": round(fa, digits), "frac": round(fa / peak, 4)}
    return roof


def snapshot(model, kv_rows):
    """The decode state on the host before the first step: DeltaNet states and conv windows,
    and the first kv_rows rows of every cache."""
    snap = []
    for L in model.layers:
        if L["kind"] == "D":
            snap.append({"state": L["state"].cpu(), "conv_state": L["conv_state"].cpu()})
        else:
            snap.append({nm: L[nm][:, :, :kv_rows].cpu() for nm in ("cache_k", "cache_v")})
    return snap


def host_weights(model, decode):
    """Per layer: the fp8 projections as decode(bytes) with their [N] scales, and the other
    parameters as CPU tensors."""
    out = []
    for L in model.layers:
        d = {"kind": L["kind"]}
        for nm, v in L.items():
            if nm in ("in_proj", "out_proj", "qkv_proj", "o_proj", "gate_up", "down"):
                d[nm] = (decode(v[0].cpu()), v[1].cpu().reshape(-1))
            elif nm in ("in_norm", "post_norm", "conv_w", "conv_b", "A_log", "dt_bias",
                        "norm_w", "q_norm", "k_norm"):
                d[nm] = v.cpu()
        out.append(d)
    return out


def oracle_parity(model, snap, kv_start, inputs, trace, first, sample):
    """The numpy oracle on sequences `sample` of the first step, from the same initial state
    (snap), teacher-forced with the GPU's residual stream entering each sublayer (trace):
    accepted lengths and token ids must be bit-identical, each sublayer output and the
    rolled-back DeltaNet states within 2e-3 relative (Frobenius)."""
    import numpy as np
    import torch
    from oracle import verify_step as ovs
    from oracle.numerics import bf16_bits_to_f32
    from spec_verify_step import DN_HV, DN_QKV
    from spec_verify_step import rope_tables

    def bits(t):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)

    def rel(a, b):
        return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))

    t0 = time.perf_counter()
    ws = host_weights(model, lambda w: w.numpy())
    sel = list(sample)
    kv = kv_start.cpu().numpy()[sel]
    layers = []
    for w, sn in zip(ws, snap):
        d = {k: (v[0], v[1].numpy()) if isinstance(v, tuple) else
             (v.numpy() if torch.is_tensor(v) else v) for k, v in w.items()}
        if w["kind"] == "D":
            d["state"] = sn["state"].reshape(B, DN_HV, 128, 128)[sel].double().numpy()
            d["conv_state"] = bits(sn["conv_state"].reshape(B, DN_QKV, 3)[sel]).copy()
        else:
            for nm in ("cache_k", "cache_v"):
                d[nm] = bits(sn[nm][sel]).copy()
        layers.append(d)
    ovs.decode_weights(layers)
    pos = torch.as_tensor(kv)[:, None] + torch.arange(T)
    cos, sin = (t.numpy() for t in rope_tables(pos))
    rows = lambda t: t.reshape(B, T, -1)[sel].reshape(len(sel) * T, -1)
    tgt, drf, ids, u, us = (t.cpu().numpy()[sel] for t in inputs)
    outs = []
    _, acc, out_ids, _ = ovs.verify_step(layers, bits(rows(trace[0])), kv, len(sel), T, tgt, drf,
                                         ids, u, us, cos, sin,
                                         layer_inputs=[bits(rows(t)) for t in trace[:-1]],
                                         layer_outputs=outs)
    sub = max(rel(rows(g).float().numpy(), bf16_bits_to_f32(r)) for g, r in zip(trace[1:], outs))
    st = max(rel(gs, d["state"]) for gs, d in zip(first["states"], (l for l in layers if l["kind"] == "D")))
    exact = bool(np.array_equal(first["accepted"].numpy()[sel], acc)
                 and np.array_equal(first["out_ids"].numpy()[sel], out_ids))
    return {"sequences": sel, "kv_len": kv.tolist(), "accepted_and_ids_bit_exact": exact,
            "max_sublayer_rel_err": float(f"{sub:.3e}"), "max_state_rel_err": float(f"{st:.3e}"),
            "tolerance": 2e-3, "ok": exact and sub <= 2e-3 and st <= 2e-3,
            "oracle": "oracle/verify_step.py (numpy), teacher-forced with the GPU's residual "
                      "stream entering each sublayer",
            "oracle_s": round(time.perf_counter() - t0, 1)}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_share():
    """(threads, affinity cores, cgroup CPU quota or None): the cores this process may run
    on (os.sched_getaffinity), capped by the cgroup v2 quota in /sys/fs/cgroup/cpu.max."""
    affinity = len(os.sched_getaffinity(0))
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()[:2]
        if q != "max":
            quota = max(1, int(int(q) // int(period)))
    except (OSError, ValueError):
        pass
    return (min(affinity, quota) if quota else affinity), affinity, quota


def cpu_baseline(model, snap, kv_start, x, inputs, first, budget_s=20.0):
    """The batched torch CPU float32 step (oracle/torch_step.py) on the whole workload (all B
    sequences, the same weights, initial state, inputs and logits as the first GPU step),
    repeated from the same initial state until about budget_s (at most 3 runs). The fp8
    weights are decoded to float32 once, before timing, as a CPU implementation of a static
    model keeps them."""
    import torch
    from oracle import torch_step as ts
    from spec_verify_step import rope_tables
    # one thread per core this process may run on: its CPU affinity, capped by a cgroup CPU
    # quota where one is set (a container's share of a larger host)
    threads, affinity, quota = cpu_share()
    torch.set_num_threads(threads)
    ws = host_weights(model, ts.decode_fp8)
    xc = x.cpu().float()
    tgt, drf, ids, u, us = (t.cpu() for t in inputs)
    kv0 = kv_start.cpu().long()
    cos, sin = rope_tables(kv0[:, None] + torch.arange(T))
    times = []
    while True:
        layers = []
        for w, sn in zip(ws, snap):
            d = dict(w)
            if w["kind"] == "D":
                d["state"] = sn["state"].reshape(B, -1, 128, 128).clone()
                d["conv_state"] = sn["conv_state"].reshape(B, -1, 3).float()
            else:
                d["cache_k"], d["cache_v"] = sn["cache_k"].clone(), sn["cache_v"].clone()
            layers.append(d)
        kv = kv0.clone()
        step = ts.TorchCpuStep(layers, B, T)
        t0 = time.perf_counter()
        _, acc, out_ids = step.step(xc, kv, cos, sin, tgt, drf, ids, u, us)
        times.append(time.perf_counter() - t0)
        print(f"cpu baseline: step {len(times)} took {times[-1]:.1f} s", file=sys.stderr,
              flush=True)
        if sum(times) >= budget_s or len(times) >= 3:
            break
    per_step = sum(times) / len(times)
    tokens = int((acc.long() + 1).sum())
    same = int(((acc == first["accepted"]) & (out_ids == first["out_ids"]).all(1)).sum())
    return {"value": round(tokens / per_step, 2), "unit": "tokens/s", "cores": threads,
            "kind": "port", "cpu": cpu_model(), "threads": threads,
            "affinity_cores": affinity, "cgroup_cpu_quota": quota,
            "sample": f"the whole first step (all {B} sequences, {tokens} committed tokens) from "
                      f"the same initial state and inputs, {len(times)} run(s), "
                      f"{per_step:.2f} s per step; oracle/torch_step.py, batched torch float32 "
                      f"on the CPU, fp8 weights decoded to float32 once before timing",
            "decisions_equal_to_gpu": f"{same}/{B}"}


CFG_MIN_WARMUP = 64      # untimed calls first, so the shader clock has settled


def time_calls(fn, n, warmup, replays=5):
    """Mean ms per call of fn(i), i = 0..n-1: after max(warmup, CFG_MIN_WARMUP) untimed
    calls, the n calls are captured in one HIP graph and the graph is replayed `replays`
    times between HIP events, so the figure is the GPU's time per call (launches included)
    rather than the host's time to issue a call from Python."""
    import torch
    for i in range(max(warmup, CFG_MIN_WARMUP)):
        fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s_ev.record()
    for _ in range(replays):
        g.replay()
    e_ev.record()
    torch.cuda.synchronize()
    return s_ev.elapsed_time(e_ev) / (n * replays)


def hbm_row(nbytes, ms):
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"bytes": int(nbytes), "achieved": round(gbs, 1), "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4)}


def config1_bench(args):
    """Full-width DeltaNet verify (16 k / 48 v heads of 128, T = 8) at B = 1, 8, 32, as the
    step runs it: deltanet::verify_from_ckpt_into reads each sequence's state from the previous
    checkpoint buffer at its accepted index (U{0..7}) and writes the T new checkpoints into the
    other buffer (the two alternate), then deltanet::conv_rollback_ rolls the conv windows
    back. q, k, v channels are bf16 N(0,1) (L2-normalised in the kernel), beta = sigmoid(N(0,1)),
    g = -softplus(N(0,1)) (A_log = dt_bias = 0), states fp32 N(0, 0.02)."""
    import torch
    import npn_ops  # noqa: F401
    dev, Hk, Hv, D = "cuda", 16, 48, 128
    QKV = (2 * Hk + Hv) * D
    rows = []
    for nb in (1, 8, 32):
        g = torch.Generator(device=dev).manual_seed(args.seed + nb)
        ck = [torch.randn(nb * T * Hv * D, D, generator=g, device=dev) * 0.02 for _ in range(2)]
        mixed = torch.randn(nb * T * QKV, generator=g, device=dev).to(torch.bfloat16)
        conv = torch.randn(nb * QKV, 3, generator=g, device=dev).to(torch.bfloat16)
        cw = torch.randn(QKV, 4, generator=g, device=dev) * 0.5
        cb = torch.randn(QKV, generator=g, device=dev) * 0.1
        a_in = torch.randn(nb * T * Hv, generator=g, device=dev)
        b_in = torch.randn(nb * T * Hv, generator=g, device=dev)
        z = torch.randn(nb * T * Hv, D, generator=g, device=dev).to(torch.bfloat16)
        zeros = torch.zeros(Hv, device=dev)
        nw = torch.randn(D, generator=g, device=dev) * 0.1 + 1.0
        acc = torch.randint(0, T, (nb,), generator=g, device=dev, dtype=torch.int32)

        def verify(i):
            return torch.ops.deltanet.verify_from_ckpt_into(
                ck[i % 2], acc, mixed, conv, cw, cb, a_in, b_in, z, zeros, zeros, nw,
                ck[1 - i % 2])

        def rollback(i):
            torch.ops.deltanet.conv_rollback_(mixed, conv, acc, Hv)

        ms_v = time_calls(verify, args.steps, args.warmup)
        ms_r = time_calls(rollback, args.steps, args.warmup)
        row = {"B": nb, "heads": nb * Hv, "verify_ms": round(ms_v, 4),
               "rollback_ms": round(ms_r, 4)}
        row.update(hbm_row(dn_verify_bytes(nb), ms_v))
        rows.append(row)
        del ck
    print(json.dumps({
        "workload": "DeltaNet verify, 16 k / 48 v heads of 128, T = 8, state checkpoints per "
                    "position, index rollback to U{0..7}",
        "kernel": "deltanet.verify (dn_verify_kernel), conv rollback separately",
        "bound": "hbm", "peak": HBM_PEAK_GBS, "rows": rows, "steps": args.steps,
        "warmup": max(args.warmup, CFG_MIN_WARMUP)}))


def full_fp8_bytes(hk, hv, hidden=5120, d=128):
    """Algorithmic bytes of one deltanet::full_fp8 call: the four fp8 weight matrices and their
    scales, x, the state in and out, the conv window in and out, the conv weight and bias,
    A_log, dt_bias, norm weight and the bf16 output."""
    qkv, zn = (2 * hk + hv) * d, hv * d
    n = qkv + zn + 2 * hv
    return (hidden * n + 4 * n + 2 * hidden + 2 * hv * d * d * 4 + qkv * 3 * 2 * 2
            + qkv * 5 * 4 + 2 * hv * 4 + d * 4 + hv * d * 2)


def full_fp8_bench(args):
    """deltanet::full_fp8: one decode token of one sequence through the four fp8
    in-projections (HIDDEN 5120 -> qkv, z, a, b) and the DeltaNet token step, at the
    reference's per-rank heads (4 k / 12 v) and full width (16 / 48). Weights are e4m3 codes
    of N(0, 0.02) quantised per channel (clip +-448), x bf16 N(0,1), states fp32 N(0, 0.1);
    four copies of the weights and states are used in turn (360 MB at full width, above the
    256 MB memory-side cache), so the weights come from HBM."""
    import torch
    import npn_ops  # noqa: F401
    dev, H, D = "cuda", 5120, 128
    rows = []
    for hk, hv in ((4, 12), (16, 48)):
        qkv = (2 * hk + hv) * D
        g = torch.Generator(device=dev).manual_seed(args.seed + hv)

        def weights(n):
            w = (torch.randn(n, H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
            sc = w.abs().amax(-1).float().clamp_min(1e-12) / 448.0
            q = (w * (1.0 / sc).to(torch.bfloat16)[:, None]).clamp(-448, 448)
            return q.to(torch.float8_e4m3fn).view(torch.int8).t().contiguous(), sc.reshape(n, 1)

        shared = [torch.randn(1, H, generator=g, device=dev).to(torch.bfloat16),
                  None,
                  torch.randn(qkv, 3, generator=g, device=dev).to(torch.bfloat16),
                  torch.randn(qkv, 4, generator=g, device=dev) * 0.5,
                  torch.randn(qkv, generator=g, device=dev) * 0.1,
                  torch.randn(hv, generator=g, device=dev) * 0.5,
                  torch.randn(hv, generator=g, device=dev),
                  torch.randn(D, generator=g, device=dev) * 0.1 + 1.0]
        sets = []
        for _ in range(4):
            a = list(shared)
            a[1] = torch.randn(hv * D, D, generator=g, device=dev) * 0.1
            for n in (qkv, hv * D, hv, hv):
                a += list(weights(n))
            sets.append(a)

        def call(i):
            return torch.ops.deltanet.full_fp8(*sets[i % 4])

        ms = time_calls(call, args.steps, args.warmup)
        row = {"k_heads": hk, "v_heads": hv, "ms": round(ms, 4)}
        row.update(hbm_row(full_fp8_bytes(hk, hv), ms))
        rows.append(row)
        del sets
    print(json.dumps({
        "workload": "deltanet::full_fp8, one decode token of one sequence, HIDDEN 5120, fp8 "
                    "in-projections (qkv, z, a, b) + DeltaNet token step",
        "kernel": "deltanet.full_fp8 (fp8_gemm_narrow_kernel: qkv + z in one launch, "
                  "dn_fp8_inproj_finish_kernel, dn_verify_kernel)", "bound": "hbm", "peak": HBM_PEAK_GBS, "rows": rows,
        "steps": args.steps, "warmup": max(args.warmup, CFG_MIN_WARMUP)}))


def config2_bench(args):
    """GQA verify attention: B = 16, T = 8 causal query rows, 24 q / 4 kv heads of 256, partial
    RoPE (64 dims, theta 1e7), bf16 N(0,1) KV cache with per-sequence lengths U{4096..32768}
    in contiguous per-sequence blocks; bf16 output, fp32 softmax."""
    import numpy as np
    import torch
    import npn_ops  # noqa: F401
    from spec_verify_step import rope_tables
    dev, nb, hq, hkv, dh = "cuda", 16, 24, 4, 256
    kv = np.random.default_rng(args.seed).integers(4096, 32769, size=nb)
    s_max = int(kv.max()) + T
    g = torch.Generator(device=dev).manual_seed(args.seed)
    q = torch.randn(nb, T, hq, dh, generator=g, device=dev).to(torch.bfloat16)
    gate = torch.randn(nb, T, hq, dh, generator=g, device=dev).to(torch.bfloat16)
    qn = torch.randn(dh, generator=g, device=dev) * 0.1
    ck = torch.randn(nb, hkv, s_max, dh, generator=g, device=dev).to(torch.bfloat16)
    cv = torch.randn(nb, hkv, s_max, dh, generator=g, device=dev).to(torch.bfloat16)
    kvl = torch.as_tensor(kv, dtype=torch.int32, device=dev)
    cos, sin = rope_tables(kvl.long()[:, None] + torch.arange(T, device=dev))

    def attn(i):
        return torch.ops.gqa.tail_verify(q, gate, qn, cos, sin, ck, cv, kvl)

    ms = time_calls(attn, args.steps, args.warmup)
    row = {"B": nb, "kv_len": kv.tolist(), "ms": round(ms, 4)}
    row.update(hbm_row(gqa_verify_bytes(kv), ms))
    print(json.dumps({
        "workload": "GQA verify attention, B = 16, T = 8, 24 q / 4 kv heads of 256, kv "
                    "U{4096..32768}", "kernel": "gqa.tail_verify", "bound": "hbm",
        "peak": HBM_PEAK_GBS, "rows": [row], "steps": args.steps,
        "warmup": max(args.warmup, CFG_MIN_WARMUP)}))


def config3_bench(args):
    """FP8 W8A16 GEMM (fp8::matmul, bf16 out) at M = B*T in {8, 64, 256}, K = 5120,
    N in {5120, 17408, 34816}: e4m3 weights from N(0, 0.02) per-channel absmax-quantised
    (clip +-448), fp32 per-channel scales, bf16 N(0,1) activations. Enough weight copies
    (at least 2, over 600 MB in all) are used in turn that the weights come from HBM."""
    import torch
    import npn_ops  # noqa: F401
    from spec_verify_step import random_fp8_linear
    dev, Kd = "cuda", 5120
    rows = []
    for n in (5120, 17408, 34816):
        g = torch.Generator(device=dev).manual_seed(args.seed + n)
        copies = max(2, -(-600_000_000 // (Kd * n)))
        ws = [random_fp8_linear(n, Kd, g, dev) for _ in range(copies)]
        for m in (8, 64, 256):
            x = torch.randn(m, Kd, generator=g, device=dev).to(torch.bfloat16)

            def mm(i):
                w, sc = ws[i % copies]
                return torch.ops.fp8.matmul(x, w, sc)

            ms = time_calls(mm, max(args.steps, 2 * copies), args.warmup)
            flops = 2.0 * m * n * Kd
            tf = flops / (ms * 1e-3) / 1e12
            row = {"M": m, "K": Kd, "N": n, "ms": round(ms, 4), "tflops": round(tf, 1),
                   "mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4), "weight_copies": copies}
            hb = hbm_row(Kd * n + n * 4 + m * Kd * 2 + m * n * 2, ms)
            row.update({"hbm_gbs": hb["achieved"], "hbm_frac": hb["frac"],
                        "bound": "hbm" if m <= 64 else "mfma"})
            rows.append(row)
        del ws
    print(json.dumps({
        "workload": "FP8 W8A16 GEMM, M in {8, 64, 256}, K = 5120, N in {5120, 17408, 34816}",
        "kernel": "fp8.matmul", "peaks": {"hbm_gbs": HBM_PEAK_GBS,
                                          "bf16_mfma_tflops": BF16_PEAK_TFLOPS},
        "rows": rows, "steps": args.steps, "warmup": max(args.warmup, CFG_MIN_WARMUP)}))


LM_VOCAB = 248320  # Qwen3.6-27B vocabulary (static_decode.py:107)
# untimed calls per variant before its timed ones, at least: with 3 the shader clock has not
# settled for the first variant (measured: fused 0.808 ms per call after 3, 0.772 after 64)
LM_MIN_WARMUP = 64
LM_ROUNDS = 5       # alternating timing rounds per path in --lm-head


def lm_head_bench(args):
    """LM head [B*T, 5120] x [5120, 248320] fp8 + greedy acceptance: fused (row argmax in the
    GEMM epilogue, no logits) vs the GEMM writing bf16 logits, a float cast and
    accept_greedy; the same for rejection sampling; and the bare GEMM for reference. Two weight
    copies (2.5 GB) alternate so the weights come from HBM."""
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

    def gemm(i):  # the bare LM-head GEMM writing bf16 logits, for reference
        w, sc = ws[i % 2]
        return torch.ops.fp8.matmul(x, w, sc)

    warmup = max(args.warmup, LM_MIN_WARMUP)
    a_f, o_f = fused(0)
    a_u, o_u = unfused(0)

    # Rejection sampling at temperature 1 over the same LM head: the fused op (the GEMM writes
    # bf16 logits and, in its epilogue, the contract's 64-column chunk statistics, so only the
    # draft rows get a statistics pass and of the target rows only the sampling rows are read
    # back) against the GEMM, a float cast and accept_rejection.
    draft = torch.randn(B, K, LM_VOCAB, generator=g, device=dev)
    rids = torch.randint(0, LM_VOCAB, (B, K), generator=g, device=dev)
    u = torch.rand(B, K, generator=g, device=dev)
    us = torch.rand(B, generator=g, device=dev)

    def rej_fused(i):
        w, sc = ws[i % 2]
        return torch.ops.spec.accept_rejection_lm_head(x, w, sc, draft, rids, u, us, 1.0)[:2]

    def rej_unfused(i):
        w, sc = ws[i % 2]
        logits = torch.ops.fp8.matmul(x, w, sc).float().view(B, T, LM_VOCAB)
        return torch.ops.spec.accept_rejection(logits, draft, rids, u, us, 1.0)

    # Every path warmed up, then LM_ROUNDS rounds that time each path in turn (args.steps
    # calls each); the median round per path. Back-to-back runs of one path drift with the
    # clock by several percent, so paths timed in separate blocks are not comparable.
    paths = (("gemm", gemm), ("fused", fused), ("unfused", unfused), ("rej_fused", rej_fused),
             ("rej_unfused", rej_unfused))
    for _, fn in paths:
        for i in range(warmup):
            fn(i)
    torch.cuda.synchronize()
    times = {name: [] for name, _ in paths}
    for _ in range(LM_ROUNDS):
        for name, fn in paths:
            s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s_ev.record()
            for i in range(args.steps):
                fn(i)
            e_ev.record()
            torch.cuda.synchronize()
            times[name].append(s_ev.elapsed_time(e_ev) / args.steps)
    res = {name: sorted(v)[len(v) // 2] for name, v in times.items()}
    ra_f, ro_f = rej_fused(0)
    ra_u, ro_u = rej_unfused(0)
    flops = 2.0 * B * T * HIDDEN * LM_VOCAB
    print(json.dumps({
        "workload": f"LM head [{B * T}x{HIDDEN}]x[{HIDDEN}x{LM_VOCAB}] fp8 + greedy acceptance, "
                    f"B={B}, K={K}",
        "gemm_ms": round(res["gemm"], 4),
        "fused_ms": round(res["fused"], 4), "unfused_ms": round(res["unfused"], 4),
        "fused_tflops": round(flops / res["fused"] / 1e9, 1),
        "weights_gb": round(HIDDEN * LM_VOCAB / 1e9, 3),
        "identical": bool(torch.equal(a_f, a_u) and torch.equal(o_f, o_u)),
        "rejection": {
            "workload": "the same LM head + rejection sampling at temperature 1 against "
                        f"[{B}, {K}, {LM_VOCAB}] fp32 draft logits",
            "fused_ms": round(res["rej_fused"], 4), "unfused_ms": round(res["rej_unfused"], 4),
            "fused_over_gemm": round(res["rej_fused"] / res["gemm"], 4),
            "identical": bool(torch.equal(ra_f, ra_u) and torch.equal(ro_f, ro_u))},
        "steps": args.steps, "warmup": warmup, "rounds": LM_ROUNDS}))


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
    if args.full_fp8:
        full_fp8_bench(args)
        return
    if args.config:
        (config1_bench, config2_bench, config3_bench)[args.config - 1](args)
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); the verify step is "
              f"measured on a single MI355X", file=sys.stderr)
        sys.exit(2)
    global B
    if not 1 <= args.batch <= 256:
        print(f"--batch must be in [1, 256] (got {args.batch})", file=sys.stderr)
        sys.exit(2)
    B = args.batch
    import torch
    from spec_verify_step import HIDDEN, OpTimer, VerifySlice, synthetic_logits

    def note(msg):
        print(msg, file=sys.stderr, flush=True)

    dev = "cuda"
    torch.manual_seed(args.seed)
    kv_lens = kv_lengths(args.seed)
    # cache rows: the warmup, the graph-timed steps and the per-op eager pass each append T
    s_max = int(kv_lens.max()) + T * (2 * (args.warmup + args.steps) + 6)
    model = VerifySlice(B, K, kv_lens, s_max, pattern="DDDG", seed=args.seed, device=dev)
    g = torch.Generator(device=dev).manual_seed(args.seed + 1)
    x = torch.randn(B * T, HIDDEN, generator=g, device=dev).to(torch.bfloat16)
    # N_SETS pre-generated logits / draft / uniform sets, used in turn by consecutive steps
    sets = [synthetic_logits(B, K, V, args.seed + 2 + i, dev) for i in range(N_SETS)]
    kv_start = model.kv_len.clone()
    check = not args.no_cpu_baseline
    snap = snapshot(model, int(kv_lens.max()) + T) if check else None

    # Python's garbage collector stays off from here to the end of the per-op pass: a full
    # collection (tens of ms) inside an op's event bracket drains the GPU queue and shows up
    # as that op's time.
    gc.collect()
    gc.disable()
    # Warmup: eager steps (the first starts from the initial DeltaNet state and is the one
    # checked against the CPU); then the state moves to fixed buffers and the step is
    # captured as one HIP graph per input set, replayed in turn in the timed region.
    trace = [] if check else None
    _, acc0, ids0 = model.step(x, *sets[0], trace=trace)
    first = None
    if check:
        sample = sorted({int(kv_start.argmin()), int(kv_start.argmax())})
        ck = [L["ckpt"].reshape(B, T, -1, 128, 128) for L in model.layers if L["kind"] == "D"]
        first = {"accepted": acc0.cpu(), "out_ids": ids0.cpu(), "trace": [t.cpu() for t in trace],
                 "states": [torch.stack([c[b, int(acc0[b])] for b in sample]).double().cpu()
                            .numpy() for c in ck]}
        trace = None
    for i in range(1, max(args.warmup, 1)):
        model.step(x, *sets[i % N_SETS])
    model.make_persistent()
    use_graph = not args.no_graph
    if use_graph:
        model.capture(x, sets)
        for _ in range(args.warmup):
            model.replay()
    step_no = [0]

    def eager():
        model.step(x, *sets[step_no[0] % N_SETS])
        step_no[0] += 1

    run = model.replay if use_graph else eager
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
    note(f"timed {args.steps} steps: {ms_per_step:.4f} ms per step")

    # Per-op launch times: HIP events around every op launch on the launch stream, over an
    # eager pass of the same number of steps over the same input sets (same kernels and
    # sizes as the replays), after two untimed eager steps: the first eager allocations after
    # the graph captures may call hipMalloc, which waits for the queued work inside an op's
    # event bracket.
    for _ in range(2):
        eager()
    torch.cuda.synchronize()
    kv0 = float(model.kv_len.float().mean().item())
    timer = OpTimer()
    model.timer = timer
    model.committed.zero_()
    for _ in range(args.steps):
        eager()
    torch.cuda.synchronize()
    model.timer = lambda name, fn, *a: fn(*a)
    gc.enable()
    ops = timer.summary()
    # mean prior cache rows seen by the attention over the timed eager steps
    kv_mean_rows = kv0 + float(model.committed.float().mean().item()) * (args.steps - 1) / (2 * args.steps)
    table = kernel_table(ops, args.steps, kv_mean_rows)
    roof = roofline(ops, args.steps, kv_mean_rows)
    if args.per_op:
        for r in table:
            rt = f"{r['achieved']:9.1f} {r['unit']} ({r['frac']:.3f})" if "frac" in r else ""
            note(f"{r['op']:40s} x{r['per_step']:2d}/step {r['mean_ms']:8.4f} ms "
                 f"{r['ms_per_step']:8.4f} ms/step {rt}")

    cpu = parity = None
    if check:
        model.graphs = model.graph_outputs = None   # release the graphs' memory pools
        note("parity: numpy oracle on the shortest- and longest-cache sequences of the first step")
        parity = oracle_parity(model, snap, kv_start, sets[0], first["trace"], first, sample)
        note(f"parity: {parity}")
        note("cpu baseline: batched torch float32 step on the host")
        cpu = cpu_baseline(model, snap, kv_start, x, sets[0], first)

    line = {
        "metric": f"verify-step tokens/s (B={B},K={K}) + achieved HBM GB/s vs MI355X peak",
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
        "data": f"synthetic (random-init weights, N(0,1) activations; {N_SETS} logits / "
                f"uniform sets used in turn by consecutive steps)",
        "config": {"workload": "EAGLE3 verify+accept+rollback, 4-layer Qwen3.6-27B-width slice "
                               "(3 gated-DeltaNet + 1 GQA, FP8 W8A16 projections), rejection "
                               "sampling at T=1",
                   "batch": B, "draft_len": K, "verify_tokens": T, "vocab": V,
                   "kv_len": "U{4096..32768}", "parallelism": "single GPU"},
        "verified_tokens_per_s": round(B * T * args.steps / elapsed, 1),
        "committed_per_seq": round(tokens / (B * args.steps), 3),
        "timing": ("HIP graph replays of the whole step (one captured graph per input set, "
                   "alternating DeltaNet checkpoint buffers)" if use_graph else "eager steps")
                  + "; per-op launch times from HIP events over an eager pass of as many steps",
        "roofline": roof,
        "kernels": table,
        "cpu_baseline": cpu,
        "parity": parity,
    }
    print(json.dumps(line), flush=True)
    if parity is not None and not parity["ok"]:
        note("parity check FAILED: the GPU step differs from the oracle")
        sys.exit(1)


if __name__ == "__main__":
    main()
