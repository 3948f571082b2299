"""torch.ops.fp8.matmul on gfx950 -- drop-in for the op registered at
contrib/qwen3.6-27b/kernels/fp8_matmul_ops.py:14-21 (same name, schema and layouts):

  fp8::matmul(x [B, K] bf16, w_fp8_T_i8 [K, N] int8 (OCP e4m3fn bytes), scale [N, 1] f32)
      -> [B, N] bf16 = bf16((x . w) * scale), fp32 accumulation

The reference kernel caps B at 128 (contrib/qwen3.6-27b/kernels/fp8_matmul.py:74); this
one takes 1 <= B <= 4096 so the verify step can pass all B*T rows in one call.
K and N must be multiples of 64.
"""
import torch

from npn_native import call, query, require, stream_of


@torch.library.custom_op("fp8::matmul", mutates_args=(), device_types="cuda")
def fp8_matmul(
    x: torch.Tensor,           # [B, K] bf16
    w_fp8_T_i8: torch.Tensor,  # [K, N] int8 (fp8 bytes; reinterpreted in kernel)
    scale: torch.Tensor,       # [N, 1] f32 (per-output-channel dequant scale)
) -> torch.Tensor:
    """Returns [B, N] bf16 = x @ w.T."""
    M, K = x.shape
    Kw, N = w_fp8_T_i8.shape
    if Kw != K:
        raise RuntimeError(f"x has K={K} but the weight has K={Kw}")
    require(x, "x", torch.bfloat16, shape=(M, K))
    if w_fp8_T_i8.dtype not in (torch.int8, torch.uint8, torch.float8_e4m3fn):
        raise TypeError(f"w_fp8_T_i8 must hold fp8 bytes, got {w_fp8_T_i8.dtype}")
    require(w_fp8_T_i8, "w_fp8_T_i8", w_fp8_T_i8.dtype, shape=(K, N))
    require(scale, "scale", torch.float32, numel=N)
    n_ws = query("npn_fp8_matmul_workspace_size", M, K, N)
    if n_ws == 0 and not (K % 64 == 0 and N % 64 == 0 and 1 <= M <= 4096):
        raise RuntimeError(f"unsupported fp8 matmul shape M={M} K={K} N={N}")
    ws = torch.empty(max(n_ws, 1), dtype=torch.uint8, device=x.device)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    call("npn_fp8_matmul", x, w_fp8_T_i8, scale, out, M, K, N, ws, n_ws, stream_of(x))
    return out


@fp8_matmul.register_fake
def _(x, w_fp8_T_i8, scale):
    return x.new_empty((x.shape[0], w_fp8_T_i8.shape[1]))


def split_k(M, K, N):
    """Split-K factor of the GEMM plan for these sizes (1: the GEMM writes bf16 itself)."""
    return query("npn_fp8_matmul_split_k", M, K, N)


@torch.library.custom_op("fp8::matmul_partials", mutates_args=(), device_types="cuda")
def fp8_matmul_partials(x: torch.Tensor, w_fp8_T_i8: torch.Tensor) -> torch.Tensor:
    """New op: the GEMM of fp8::matmul without its reduction and scale, [S, M, N] f32 with
    S = split_k(M, K, N); fp8::matmul(x, w, scale) == bf16(scale * partials.sum(0)) summed
    in order. The *_partials glue ops consume it."""
    M, K = x.shape
    Kw, N = w_fp8_T_i8.shape
    if Kw != K:
        raise RuntimeError(f"x has K={K} but the weight has K={Kw}")
    require(x, "x", torch.bfloat16, shape=(M, K))
    if w_fp8_T_i8.dtype not in (torch.int8, torch.uint8, torch.float8_e4m3fn):
        raise TypeError(f"w_fp8_T_i8 must hold fp8 bytes, got {w_fp8_T_i8.dtype}")
    require(w_fp8_T_i8, "w_fp8_T_i8", w_fp8_T_i8.dtype, shape=(K, N))
    S = split_k(M, K, N)
    if S == 0:
        raise RuntimeError(f"unsupported fp8 matmul shape M={M} K={K} N={N}")
    out = torch.empty((S, M, N), dtype=torch.float32, device=x.device)
    call("npn_fp8_matmul_partials", x, w_fp8_T_i8, out, M, K, N, stream_of(x))
    return out


@fp8_matmul_partials.register_fake
def _(x, w_fp8_T_i8):
    M, K = x.shape
    N = w_fp8_T_i8.shape[1]
    return x.new_empty((split_k(M, K, N), M, N), dtype=torch.float32)


def _check_gemm_args(x, w_fp8_T_i8):
    M, K = x.shape
    Kw, N = w_fp8_T_i8.shape
    if Kw != K:
        raise RuntimeError(f"x has K={K} but the weight has K={Kw}")
    require(x, "x", torch.bfloat16, shape=(M, K))
    if w_fp8_T_i8.dtype not in (torch.int8, torch.uint8, torch.float8_e4m3fn):
        raise TypeError(f"w_fp8_T_i8 must hold fp8 bytes, got {w_fp8_T_i8.dtype}")
    require(w_fp8_T_i8, "w_fp8_T_i8", w_fp8_T_i8.dtype, shape=(K, N))
    return M, K, N


def argmax_parts(x, w_fp8_T_i8, scale):
    """Per-(row, column group) argmax partials of bf16((x . w) * scale), [M, G, 2] int32
    (value bits, column), for npn_argmax_parts / npn_accept_greedy_parts."""
    M, K, N = _check_gemm_args(x, w_fp8_T_i8)
    require(scale, "scale", torch.float32, numel=N)
    G = query("npn_fp8_matmul_argmax_groups", M, K, N)
    if G == 0:
        raise RuntimeError(f"unsupported fp8 matmul shape M={M} K={K} N={N}")
    parts = torch.empty((M, G, 2), dtype=torch.int32, device=x.device)
    call("npn_fp8_matmul_argmax", x, w_fp8_T_i8, scale, parts, M, K, N, stream_of(x))
    return parts


@torch.library.custom_op("fp8::matmul_argmax", mutates_args=(), device_types="cuda")
def fp8_matmul_argmax(x: torch.Tensor, w_fp8_T_i8: torch.Tensor,
                      scale: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """New op: (values f32 [M], ids int64 [M]) = max and argmax over each row of
    fp8::matmul(x, w, scale) (bf16 values; NaN is the maximum; ties to the lower column),
    without writing the [M, N] output -- the LM head's greedy decision
    (contrib/qwen3.6-27b/static_decode.py:546, :1313)."""
    parts = argmax_parts(x, w_fp8_T_i8, scale)
    M, G = parts.shape[0], parts.shape[1]
    ids = torch.empty(M, dtype=torch.int64, device=x.device)
    values = torch.empty(M, dtype=torch.float32, device=x.device)
    call("npn_argmax_parts", parts, G, ids, values, M, stream_of(x))
    return values, ids


@fp8_matmul_argmax.register_fake
def _(x, w_fp8_T_i8, scale):
    M = x.shape[0]
    return x.new_empty((M,), dtype=torch.float32), x.new_empty((M,), dtype=torch.int64)


@torch.library.custom_op("fp8::matmul_swiglu", mutates_args=(), device_types="cuda")
def fp8_matmul_swiglu(x: torch.Tensor, w_fp8_T_i8: torch.Tensor,
                      scale: torch.Tensor) -> torch.Tensor:
    """New op: the MLP's gate/up projection and SwiGLU in one call
    (contrib/qwen3.6-27b/static_decode.py:951-963). w = [gate | up] along N; returns
    [M, N/2] bf16 = bf16(bf16(silu(g)) * u) for [g | u] = fp8::matmul(x, w, scale),
    bit-identical to fp8::matmul followed by glue::silu_mul."""
    M, K, N = _check_gemm_args(x, w_fp8_T_i8)
    require(scale, "scale", torch.float32, numel=N)
    if N % 128 != 0 or not (K % 64 == 0 and 1 <= M <= 4096):
        raise RuntimeError(f"unsupported fp8 matmul_swiglu shape M={M} K={K} N={N}")
    n_ws = query("npn_fp8_matmul_swiglu_workspace_size", M, K, N)
    ws = torch.empty(max(n_ws, 1), dtype=torch.uint8, device=x.device)
    out = torch.empty((M, N // 2), dtype=torch.bfloat16, device=x.device)
    call("npn_fp8_matmul_swiglu", x, w_fp8_T_i8, scale, out, M, K, N, ws, n_ws, stream_of(x))
    return out


@fp8_matmul_swiglu.register_fake
def _(x, w_fp8_T_i8, scale):
    return x.new_empty((x.shape[0], w_fp8_T_i8.shape[1] // 2), dtype=torch.bfloat16)


def fp8_linear(x, w_fp8_T_i8, scale):
    """x [..., K] bf16 -> [..., N], as the reference's fp8_linear
    (contrib/qwen3.6-27b/static_decode.py:307-319)."""
    flat = x.reshape(-1, x.shape[-1])
    return torch.ops.fp8.matmul(flat, w_fp8_T_i8, scale).reshape(*x.shape[:-1], -1)
