"""EAGLE3 verify-and-accept step of a Qwen3.6 hybrid slice on gfx950.

The caller side of the ops, mirroring the reference's decode harness
(contrib/qwen3.6-27b/static_decode.py: _deltanet_layer :753-847, _gqa_layer :849-949,
_mlp_layer :951-963, rms_norm :322-335, _init_rope :489-502) for T = K+1 verify tokens
per sequence instead of one:

  x [B*T, 5120] --(per layer)--> input RMSNorm(1+w)
      DeltaNet layer: fp8 in-proj [qkv | z | a | b] -> deltanet::verify_from_ckpt -> fp8 out-proj
      GQA layer:      fp8 [q+gate | k | v] -> gqa::tail_verify_append (k norm + RoPE + KV
                      append in the attention's query-prep launch) -> fp8 o-proj
    -> residual -> post RMSNorm(1+w) -> fp8 gate/up -> SiLU * up -> fp8 down -> residual
  logits -> spec::accept_rejection (or accept_greedy)
  rollback: DeltaNet state = checkpoint[accepted] (read in place by the next step),
            conv window rolled back, KV length += accepted + 1.

Dimensions are the 27B model's whole-model widths on one GPU: hidden 5120, DeltaNet 16 k /
48 v heads of 128, GQA 24 q / 4 kv heads of 256 with a 64-dim partial RoPE (theta 1e7),
MLP intermediate 17408. Weights are random (e4m3fn, per-output-channel fp32 scales).
"""
import math

import torch

import npn_ops  # noqa: F401  (registers the torch.ops)
from fp8_matmul_ops import split_k as fp8_split_k

HIDDEN = 5120
DN_HK, DN_HV, DN_D = 16, 48, 128
DN_QKV = (2 * DN_HK + DN_HV) * DN_D       # 10240
DN_VAL = DN_HV * DN_D                     # 6144
GQA_HQ, GQA_HKV, GQA_DH = 24, 4, 256
GQA_QG = GQA_HQ * 2 * GQA_DH              # 12288 (query and gate interleaved per head)
INTER = 17408
ROPE_DIM, ROPE_THETA = 64, 1e7
DN_IN_N = DN_QKV + DN_VAL + 2 * DN_HV     # 16480 = qkv | z | a | b
DN_IN_PAD = ((DN_IN_N + 63) // 64) * 64   # 16512 (the GEMM takes N % 64 == 0)


def rope_tables(positions):
    """cos/sin [..., 64] at integer positions, fp32 as the reference table (:489-502)."""
    inv_freq = 1.0 / (ROPE_THETA ** (torch.arange(0, ROPE_DIM, 2, device=positions.device,
                                                  dtype=torch.float32) / ROPE_DIM))
    freqs = positions.float().unsqueeze(-1) * inv_freq
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos().contiguous(), emb.sin().contiguous()


def random_fp8_linear(n_out, k_in, gen, device, std=0.02, fp8_max=448.0, pad_to=None):
    """W ~ N(0, std) [n_out, k_in] -> (w [K, N] int8 e4m3fn bytes, scale [N, 1] f32), the
    reference's per-channel absmax quantisation (static_decode.py:283-304) with FP8_MAX=448."""
    w = torch.randn(n_out, k_in, generator=gen, device=device, dtype=torch.float32) * std
    w = w.to(torch.bfloat16)
    absmax = w.abs().amax(dim=-1).float().clamp_min(1e-12)
    scale = absmax / fp8_max
    inv = (1.0 / scale).to(torch.bfloat16).unsqueeze(-1)
    wq = (w * inv).clamp(-fp8_max, fp8_max).to(torch.float8_e4m3fn)
    del w
    wt = wq.t().contiguous().view(torch.int8)
    scale = scale.reshape(-1, 1).contiguous()
    if pad_to is not None and pad_to > n_out:
        wt = torch.cat([wt, torch.zeros(k_in, pad_to - n_out, dtype=torch.int8, device=device)], 1)
        scale = torch.cat([scale, torch.ones(pad_to - n_out, 1, device=device)], 0)
    return wt.contiguous(), scale.contiguous()


class OpTimer:
    """Records a pair of HIP events around each op launch on the current stream, keyed by
    op name; `summary()` (after a synchronize) gives per-name launch counts and mean ms."""

    def __init__(self):
        self.events = {}

    def __call__(self, name, fn, *args):
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        out = fn(*args)
        e.record()
        self.events.setdefault(name, []).append((s, e))
        return out

    def summary(self):
        res = {}
        for k, ev in self.events.items():
            ms = [s.elapsed_time(e) for s, e in ev]
            res[k] = {"launches": len(ms), "mean_ms": sum(ms) / len(ms), "total_ms": sum(ms)}
        return res


def _untimed(name, fn, *args):
    return fn(*args)


def fp8_linear(x, wq, timer=_untimed, name="fp8.matmul"):
    w, s = wq
    return timer(name, torch.ops.fp8.matmul, x, w, s)


def fp8_project(x, wq, timer=_untimed, name="fp8.matmul", fuse=True):
    """A projection whose consumer is a glue op with a *_partials form: when the GEMM plan
    splits K, returns (fp32 partials, scale) for that consumer to reduce (bit-identical to
    fp8.matmul's own reduction); otherwise the bf16 output."""
    w, s = wq
    if fuse and fp8_split_k(x.shape[0], x.shape[1], w.shape[1]) > 1:
        return timer(name, torch.ops.fp8.matmul_partials, x, w), s
    return timer(name, torch.ops.fp8.matmul, x, w, s)


class VerifySlice:
    """Random-init slice of `pattern` layers ('D' DeltaNet, 'G' GQA) plus per-layer MLPs,
    with the decode state of B sequences."""

    def __init__(self, B, K, kv_lens, s_max, pattern="DDDG", seed=0, device="cuda",
                 fuse_splitk=True, fuse_swiglu=True, fuse_launches=True):
        self.B, self.K, self.T = B, K, K + 1
        self.fuse_splitk = fuse_splitk
        self.fuse_swiglu = fuse_swiglu
        self.fuse_launches = fuse_launches
        self.pattern = pattern
        self.device = device
        self.s_max = s_max
        g = torch.Generator(device=device).manual_seed(seed)
        self.layers = []
        for kind in pattern:
            L = {"kind": kind,
                 "in_norm": (torch.randn(HIDDEN, generator=g, device=device) * 0.1),
                 "post_norm": (torch.randn(HIDDEN, generator=g, device=device) * 0.1),
                 "gate_up": random_fp8_linear(2 * INTER, HIDDEN, g, device),
                 "down": random_fp8_linear(HIDDEN, INTER, g, device)}
            if kind == "D":
                L["in_proj"] = random_fp8_linear(DN_IN_N, HIDDEN, g, device, pad_to=DN_IN_PAD)
                L["out_proj"] = random_fp8_linear(HIDDEN, DN_VAL, g, device)
                L["conv_w"] = torch.randn(DN_QKV, 4, generator=g, device=device) * 0.5
                L["conv_b"] = torch.randn(DN_QKV, generator=g, device=device) * 0.1
                L["A_log"] = torch.randn(DN_HV, generator=g, device=device) * 0.5
                L["dt_bias"] = torch.randn(DN_HV, generator=g, device=device)
                L["norm_w"] = torch.randn(DN_D, generator=g, device=device) * 0.1 + 1.0
                # decode state: one initial state per sequence; after a step the state is
                # the previous step's checkpoint buffer plus the accepted index
                L["state"] = torch.randn(B * DN_HV * DN_D, DN_D, generator=g, device=device) * 0.02
                L["ckpt"] = None
                L["conv_state"] = torch.randn(B * DN_QKV, 3, generator=g,
                                              device=device).to(torch.bfloat16)
            else:
                L["qkv_proj"] = random_fp8_linear(GQA_QG + 2 * GQA_HKV * GQA_DH, HIDDEN, g, device)
                L["o_proj"] = random_fp8_linear(HIDDEN, GQA_HQ * GQA_DH, g, device)
                L["q_norm"] = torch.randn(GQA_DH, generator=g, device=device) * 0.1
                L["k_norm"] = torch.randn(GQA_DH, generator=g, device=device) * 0.1
                shape = (B, GQA_HKV, s_max, GQA_DH)
                L["cache_k"] = torch.randn(shape, generator=g, device=device).to(torch.bfloat16)
                L["cache_v"] = torch.randn(shape, generator=g, device=device).to(torch.bfloat16)
            self.layers.append(L)
        self.kv_len = torch.as_tensor(kv_lens, dtype=torch.int32, device=device).clone()
        # RoPE table of every cache position, built once (the reference's _init_rope); each
        # step gathers the rows of its T positions.
        self.rope_cos, self.rope_sin = rope_tables(torch.arange(s_max, device=device))
        self.prev_accepted = None
        self.timer = _untimed
        self.persistent = False
        self.parity = 0
        self.graphs = None

    # ---- layers: each takes the normed input and returns the residual delta -------------
    def _deltanet(self, L, h):
        B, T = self.B, self.T
        proj = fp8_project(h, L["in_proj"], self.timer, f"fp8.matmul[{B * T}x{HIDDEN}x{DN_IN_PAD}]",
                           self.fuse_splitk)
        if isinstance(proj, tuple):
            mixed, z, a, b = self.timer("glue.deltanet_split",
                                        torch.ops.glue.deltanet_split_partials, *proj, DN_QKV,
                                        DN_VAL, DN_HV)
        else:
            mixed, z, a, b = self.timer("glue.deltanet_split", torch.ops.glue.deltanet_split,
                                        proj, DN_QKV, DN_VAL, DN_HV)
        mixed = mixed.reshape(-1)
        args = (mixed, L["conv_state"], L["conv_w"], L["conv_b"], a.reshape(-1), b.reshape(-1),
                z.reshape(B * T * DN_HV, DN_D), L["A_log"], L["dt_bias"], L["norm_w"])
        if self.persistent:  # previous checkpoints in ckbuf[parity], new ones into the other
            p = self.parity
            ckpt = L["ckbuf"][1 - p]
            out = self.timer("deltanet.verify", torch.ops.deltanet.verify_from_ckpt_into,
                             L["ckbuf"][p], self.prev_accepted, *args, ckpt)
        elif L["ckpt"] is None:
            ckpt, out = self.timer("deltanet.verify", torch.ops.deltanet.verify_batched,
                                   L["state"], *args)
        else:
            ckpt, out = self.timer("deltanet.verify", torch.ops.deltanet.verify_from_ckpt,
                                   L["ckpt"], self.prev_accepted, *args)
        L["pending"] = (ckpt, mixed)
        return fp8_project(out.reshape(B * T, DN_VAL), L["out_proj"], self.timer,
                           f"fp8.matmul[{B * T}x{DN_VAL}x{HIDDEN}]", self.fuse_splitk)

    def _gqa(self, L, h, cos, sin):
        B, T = self.B, self.T
        proj = fp8_project(h, L["qkv_proj"], self.timer,
                           f"fp8.matmul[{B * T}x{HIDDEN}x{GQA_QG + 2 * GQA_HKV * GQA_DH}]",
                           self.fuse_splitk)
        if isinstance(proj, tuple):
            query, gate, key, value = self.timer("glue.gqa_split",
                                                 torch.ops.glue.gqa_split_partials, *proj,
                                                 GQA_HQ, GQA_HKV, GQA_DH)
        else:
            query, gate, key, value = self.timer("glue.gqa_split", torch.ops.glue.gqa_split,
                                                 proj, GQA_HQ, GQA_HKV, GQA_DH)
        query = query.reshape(B, T, GQA_HQ, GQA_DH)
        gate = gate.reshape(B, T, GQA_HQ, GQA_DH)
        key = key.reshape(B, T, GQA_HKV, GQA_DH)
        value = value.reshape(B, T, GQA_HKV, GQA_DH)
        if cos is None:  # append, RoPE rows from the tables and attention in one op
            attn = self.timer("gqa.tail_verify_append", torch.ops.gqa.tail_verify_append,
                              query, gate, key, value, L["q_norm"], L["k_norm"], self.rope_cos,
                              self.rope_sin, L["cache_k"], L["cache_v"], self.kv_len)
        else:
            self.timer("gqa.kv_append", torch.ops.gqa.kv_append, key, value, L["k_norm"], cos,
                       sin, L["cache_k"], L["cache_v"], self.kv_len)
            attn = self.timer("gqa.tail_verify", torch.ops.gqa.tail_verify, query, gate,
                              L["q_norm"], cos, sin, L["cache_k"], L["cache_v"], self.kv_len)
        return fp8_project(attn.reshape(B * T, GQA_HQ * GQA_DH), L["o_proj"], self.timer,
                           f"fp8.matmul[{B * T}x{GQA_HQ * GQA_DH}x{HIDDEN}]", self.fuse_splitk)

    def _mlp(self, L, h):
        M = h.shape[0]
        if self.fuse_swiglu:
            w, sc = L["gate_up"]
            act = self.timer(f"fp8.matmul_swiglu[{M}x{HIDDEN}x{2 * INTER}]",
                             torch.ops.fp8.matmul_swiglu, h, w, sc)
        else:
            gu = fp8_linear(h, L["gate_up"], self.timer, f"fp8.matmul[{M}x{HIDDEN}x{2 * INTER}]")
            act = self.timer("glue.silu_mul", torch.ops.glue.silu_mul, gu)
        return fp8_project(act, L["down"], self.timer, f"fp8.matmul[{M}x{INTER}x{HIDDEN}]",
                           self.fuse_splitk)

    def _add_norm(self, hidden, d, weight):
        """(hidden + d, its (1+w) RMSNorm); d is a bf16 delta or (partials, scale)."""
        if isinstance(d, tuple):
            return self.timer("normfuse.residual_rms_norm",
                              torch.ops.normfuse.residual_rms_norm_partials, hidden, *d, weight)
        return self.timer("normfuse.residual_rms_norm", torch.ops.normfuse.residual_rms_norm,
                          hidden, d, weight)

    def forward(self, x, cos=None, sin=None, trace=None):
        """x [B*T, 5120] bf16 -> hidden after the slice (the verify positions' features).
        Per layer, as the reference's decode loop (static_decode.py:533-542):
          normed = rms_norm(hidden); hidden += layer(normed);
          normed = rms_norm(hidden); hidden += mlp(normed)
        with every residual add fused into the norm that follows it. Explicit cos/sin rows
        (or fuse_launches=False) select the separate rope_rows / kv_append / tail_verify ops,
        whose results the fused op equals bit for bit. If `trace` is a list,
        the residual stream entering each sublayer (mixer, then MLP, per layer) and the final
        hidden are appended to it."""
        if cos is None and not self.fuse_launches and "G" in self.pattern:
            cos, sin = self.timer("gqa.rope_rows", torch.ops.gqa.rope_rows, self.rope_cos,
                                  self.rope_sin, self.kv_len, self.T)
        layers = self.layers
        hidden = x
        normed = self.timer("normfuse.rms_norm", torch.ops.normfuse.rms_norm, x,
                            layers[0]["in_norm"])
        for i, L in enumerate(layers):
            if trace is not None:
                trace.append(hidden)
            d = self._deltanet(L, normed) if L["kind"] == "D" else self._gqa(L, normed, cos, sin)
            hidden, normed = self._add_norm(hidden, d, L["post_norm"])
            if trace is not None:
                trace.append(hidden)
            last = i + 1 == len(layers)
            d = self._mlp(L, normed)
            if not last:
                hidden, normed = self._add_norm(hidden, d, layers[i + 1]["in_norm"])
            elif isinstance(d, tuple):
                hidden = self.timer("normfuse.residual_add",
                                    torch.ops.normfuse.residual_add_partials, hidden, *d)
            else:
                hidden = hidden + d
        if trace is not None:
            trace.append(hidden)
        return hidden

    def accept_and_rollback(self, accepted):
        """Commit `accepted` drafts per sequence: DeltaNet continues from checkpoint
        [accepted] (in place, next step), conv windows roll back, KV lengths advance. With
        state at fixed addresses and fuse_launches, the conv rollbacks of every DeltaNet layer
        and the commit are one launch (deltanet::rollback_commit_)."""
        if self.persistent and self.fuse_launches:
            dn = [L for L in self.layers if L["kind"] == "D"]
            pend = [L.pop("pending") for L in dn]
            self.timer("deltanet.rollback_commit", torch.ops.deltanet.rollback_commit_,
                       [m for _, m in pend], [L["conv_state"] for L in dn], accepted,
                       self.prev_accepted, self.kv_len, self.committed, DN_HV)
            self.parity ^= 1
            return
        for L in self.layers:
            if L["kind"] == "D":
                ckpt, mixed = L.pop("pending")
                if self.persistent:  # window rolled back over the fixed buffer
                    self.timer("deltanet.conv_rollback", torch.ops.deltanet.conv_rollback_,
                               mixed, L["conv_state"], accepted, DN_HV)
                else:
                    L["conv_state"] = self.timer("deltanet.conv_rollback",
                                                 torch.ops.deltanet.conv_rollback, mixed,
                                                 L["conv_state"], accepted, DN_HV)
                    L["ckpt"] = ckpt
        if self.persistent:
            self.timer("spec.commit", torch.ops.spec.commit_, accepted, self.prev_accepted,
                       self.kv_len, self.committed)
            self.parity ^= 1
        else:
            self.prev_accepted = accepted
            self.kv_len = self.kv_len + accepted + 1

    # ---- fixed-address state and HIP graphs of the step -----------------------------------
    def make_persistent(self):
        """After at least one eager step: keep the decode state in fixed buffers updated in
        place (conv windows, previous accepted lengths, KV lengths, a committed-token
        counter) with two checkpoint buffers per DeltaNet layer used in turn -- each step
        reads the previous step's checkpoints from one and writes its own into the other --
        so that a step can be captured once per buffer parity and replayed."""
        if self.prev_accepted is None:
            raise RuntimeError("run one eager step before make_persistent()")
        for L in self.layers:
            if L["kind"] == "D":
                L["ckbuf"] = [L.pop("ckpt"), None]
                L["ckbuf"][1] = torch.empty_like(L["ckbuf"][0])
        self.committed = torch.zeros(self.B, dtype=torch.int32, device=self.device)
        self.parity = 0
        self.persistent = True

    def capture(self, x, input_sets, greedy=False):
        """Capture the step as one HIP graph per entry of `input_sets`, each a tuple
        (target_logits, draft_logits, draft_ids, u_accept, u_sample) of tensors that keep
        their addresses (as does x). Consecutive graphs use the two checkpoint buffers in
        turn, so the number of sets must be even; replay() runs them in order, cyclically.
        Capturing runs nothing: the parity flips once per graph and ends where it started."""
        if len(input_sets) == 0 or len(input_sets) % 2:
            raise ValueError("capture needs an even, nonzero number of input sets")
        if not self.persistent:
            self.make_persistent()
        self.graphs, self.graph_outputs = [], []
        self.graph_parity0 = self.parity
        for inputs in input_sets:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                outs = self.step(x, *inputs, greedy=greedy)
            self.graphs.append(g)
            self.graph_outputs.append(outs)
        self.next_graph = 0

    def replay(self):
        """One step by graph replay; returns that graph's (hidden, accepted, out_ids) tensors
        (overwritten by the next replay of the same graph)."""
        i = self.next_graph
        if (self.graph_parity0 + i) % 2 != self.parity:
            raise RuntimeError("graph replay out of step with the checkpoint-buffer parity")
        self.graphs[i].replay()
        self.parity ^= 1
        self.next_graph = (i + 1) % len(self.graphs)
        return self.graph_outputs[i]

    def step(self, x, target_logits, draft_logits, draft_ids, u_accept, u_sample, greedy=False,
             trace=None):
        """One verify + accept + rollback step. Returns (hidden, accepted, out_ids)."""
        h = self.forward(x, trace=trace)
        if greedy:
            accepted, out_ids = self.timer("spec.accept_greedy", torch.ops.spec.accept_greedy,
                                           target_logits, draft_ids)
        else:
            accepted, out_ids = self.timer("spec.accept_rejection",
                                           torch.ops.spec.accept_rejection, target_logits,
                                           draft_logits, draft_ids, u_accept, u_sample, 1.0)
        self.accept_and_rollback(accepted)
        return h, accepted, out_ids


def synthetic_logits(B, K, V, seed, device, rho=0.8):
    """Target logits [B, K+1, V] ~ N(0,1); draft logits [B, K, V] = rho*t + sqrt(1-rho^2)*eps;
    draft ids sampled from softmax(draft); uniforms [B, K] and [B]."""
    g = torch.Generator(device=device).manual_seed(seed)
    target = torch.randn(B, K + 1, V, generator=g, device=device)
    draft = rho * target[:, :K] + math.sqrt(1 - rho * rho) * torch.randn(B, K, V, generator=g,
                                                                         device=device)
    ids = torch.multinomial(torch.softmax(draft, -1).reshape(B * K, V), 1,
                            generator=g).reshape(B, K)
    u = torch.rand(B, K, generator=g, device=device)
    us = torch.rand(B, generator=g, device=device)
    return target.contiguous(), draft.contiguous(), ids, u, us
