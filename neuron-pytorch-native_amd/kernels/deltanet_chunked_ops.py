"""torch.ops.deltanet.chunked_prefill on gfx950 -- drop-in for the op registered at
contrib/qwen3.6-27b/kernels/deltanet_chunked_ops.py:26-42 (same name and schema):

  deltanet::chunked_prefill(state [Hv*128, 128] f32, query [Hv*S, 128] f32 (raw),
      key [Hv*S, 128] f32 (raw), value [Hv*S, 128] f32, g [Hv*S, 1] f32, beta [Hv*S, 1] f32,
      m_incl [C, C] f32, m_strict [C, C] f32, eye [C, C] f32)
      -> (output [Hv*S, 128] f32 raw (before the gated norm), new_state [Hv*128, 128] f32)

Rows are head-major (row h*S + t). q and k are L2-normalised inside and q is scaled by
1/sqrt(128), as the reference kernel does (contrib/qwen3.6-27b/kernels/deltanet_chunked_v2.py:
123-160). The [C, C] constants exist for the reference's device compiler (no iota there);
they are checked for shape only: the kernel chunks by 64 tokens whatever C is (the result is
the same up to rounding), and takes any S (a last partial chunk is zero-gate padding; the
reference kernel needs S % C == 0).
"""
import torch

from npn_native import call, require, stream_of
from npn_native import query as query_size

D = 128


@torch.library.custom_op("deltanet::chunked_prefill", mutates_args=(), device_types="cuda")
def chunked_prefill(state: torch.Tensor, query: torch.Tensor, key: torch.Tensor,
                    value: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
                    m_incl: torch.Tensor, m_strict: torch.Tensor,
                    eye: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    if state.dim() != 2 or state.shape[1] != D or state.shape[0] % D != 0:
        raise RuntimeError(f"state must be [Hv*{D}, {D}], got {tuple(state.shape)}")
    Hv = state.shape[0] // D
    rows = query.shape[0]
    if rows % Hv != 0 or rows == 0:
        raise RuntimeError(f"query rows {rows} are not a positive multiple of Hv={Hv}")
    S = rows // Hv
    require(state, "state", torch.float32, shape=(Hv * D, D))
    for name, t in (("query", query), ("key", key), ("value", value)):
        require(t, name, torch.float32, shape=(Hv * S, D))
    require(g, "g", torch.float32, numel=Hv * S)
    require(beta, "beta", torch.float32, numel=Hv * S)
    C = m_incl.shape[0] if m_incl.dim() == 2 else 0
    for name, t in (("m_incl", m_incl), ("m_strict", m_strict), ("eye", eye)):
        if t.dim() != 2 or tuple(t.shape) != (C, C) or C < 1:
            raise RuntimeError(f"{name} must be [C, C], got {tuple(t.shape)}")
    n_ws = query_size("npn_deltanet_chunked_workspace_size", Hv, S)
    if n_ws == 0:
        raise RuntimeError(f"unsupported chunked prefill size Hv={Hv} S={S}")
    ws = torch.empty(n_ws, dtype=torch.uint8, device=state.device)
    out = torch.empty((Hv * S, D), dtype=torch.float32, device=state.device)
    new_state = torch.empty((Hv * D, D), dtype=torch.float32, device=state.device)
    call("npn_deltanet_chunked_prefill", state, query, key, value, g, beta, out, new_state,
         Hv, S, ws, n_ws, stream_of(state))
    return out, new_state


@chunked_prefill.register_fake
def _(state, query, key, value, g, beta, m_incl, m_strict, eye):
    return torch.empty_like(query), torch.empty_like(state)
