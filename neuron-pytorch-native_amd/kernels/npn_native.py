"""ctypes binding of libnpn_spec_verify.so (the C ABI declared in include/npn_spec_verify.h).

This is the only place Python crosses into native code. Each op module calls
``call(name, *args)``: tensors are passed as raw device pointers, ints as C ints,
and a non-zero npn_status becomes a RuntimeError carrying the library's text.
There is no fallback: if the library is missing the first call raises.
"""
import ctypes
import os

import torch

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "libnpn_spec_verify.so")

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_Z = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/npn_spec_verify.h one to one.
SIGNATURES = {
    "npn_status_string": (ctypes.c_char_p, [_I]),
    "npn_abi_version": (_I, []),
    "npn_deltanet_full_batched": (_I, [_P] * 14 + [_I, _I, _I, _P]),
    "npn_deltanet_verify": (_I, [_P, _P, _I] + [_P] * 12 + [_I, _I, _I, _I, _P]),
    "npn_deltanet_rollback": (_I, [_P] * 6 + [_I, _I, _I, _I, _P]),
    "npn_gqa_tail": (_I, [_P] * 9 + [_I, _I, _I, _P]),
    "npn_gqa_tail_verify_workspace_size": (_Z, [_I] * 5),
    "npn_gqa_tail_verify": (_I, [_P] * 9 + [_I] * 5 + [_P, _Z, _P]),
    "npn_gqa_kv_append": (_I, [_P] * 8 + [_I] * 4 + [_P]),
    "npn_gqa_tail_verify_append": (_I, [_P] * 8 + [_I] + [_P] * 4 + [_I] * 5 + [_P, _Z, _P]),
    "npn_fp8_matmul_workspace_size": (_Z, [_I] * 3),
    "npn_fp8_matmul": (_I, [_P] * 4 + [_I] * 3 + [_P, _Z, _P]),
    "npn_accept_workspace_size": (_Z, [_I] * 3),
    "npn_accept_greedy": (_I, [_P] * 4 + [_I] * 3 + [_P, _Z, _P]),
    "npn_accept_rejection": (_I, [_P] * 5 + [_F] + [_P] * 2 + [_I] * 3 + [_P, _Z, _P]),
    "npn_accept_rejection_noalloc": (_I, [_P] * 5 + [_F] + [_P] * 2 + [_I] * 3 + [_P]),
    "npn_residual_rmsnorm": (_I, [_P] * 5 + [_I, _I, _F, _P]),
    "npn_silu_mul": (_I, [_P, _P, _I, _I, _P]),
    "npn_deltanet_split": (_I, [_P, _I] + [_P] * 4 + [_I] * 4 + [_P]),
    "npn_gqa_split": (_I, [_P, _I] + [_P] * 4 + [_I] * 4 + [_P]),
    "npn_fp8_matmul_split_k": (_I, [_I] * 3),
    "npn_fp8_matmul_plan": (_I, [_I] * 3 + [_P]),
    "npn_fp8_matmul_partials": (_I, [_P] * 3 + [_I] * 3 + [_P]),
    "npn_residual_rmsnorm_partials": (_I, [_P, _P, _I] + [_P] * 4 + [_I, _I, _F, _P]),
    "npn_residual_add_partials": (_I, [_P, _P, _I, _P, _P, _I, _I, _P]),
    "npn_deltanet_split_partials": (_I, [_P, _I, _P, _I] + [_P] * 4 + [_I] * 4 + [_P]),
    "npn_gqa_split_partials": (_I, [_P, _I, _P, _I] + [_P] * 4 + [_I] * 4 + [_P]),
    "npn_rope_rows": (_I, [_P, _P, _I] + [_P] * 3 + [_I] * 3 + [_P]),
    "npn_spec_commit": (_I, [_P] * 4 + [_I, _P]),
    "npn_deltanet_rollback_commit": (_I, [_P, _P, _I] + [_P] * 4 + [_I] * 4 + [_P]),
    "npn_fp8_matmul_argmax_groups": (_I, [_I] * 3),
    "npn_fp8_matmul_argmax": (_I, [_P] * 4 + [_I] * 3 + [_P]),
    "npn_argmax_parts": (_I, [_P, _I, _P, _P, _I, _P]),
    "npn_accept_greedy_parts": (_I, [_P, _I] + [_P] * 3 + [_I, _I, _P]),
    "npn_fp8_matmul_swiglu_workspace_size": (_Z, [_I] * 3),
    "npn_fp8_matmul_swiglu": (_I, [_P] * 4 + [_I] * 3 + [_P, _Z, _P]),
    "npn_fp8_matmul_rowmax": (_I, [_P] * 5 + [_I] * 3 + [_P]),
    "npn_accept_rejection_lm_head_workspace_size": (_Z, [_I] * 4),
    "npn_accept_rejection_lm_head": (_I, [_P] * 7 + [_F] + [_P] * 3 + [_I] * 4 + [_P, _Z, _P]),
    "npn_deltanet_chunked_workspace_size": (_Z, [_I, _I]),
    "npn_deltanet_chunked_prefill": (_I, [_P] * 8 + [_I, _I, _P, _Z, _P]),
    "npn_deltanet_full_fp8_workspace_size": (_Z, [_I] * 3),
    "npn_deltanet_full_fp8": (_I, [_P] * 19 + [_I] * 3 + [_P, _Z, _P]),
}

_lib = None


def lib():
    """Load the library once and declare every entry point's C signature."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built: run `make -C {PKG_DIR}` (hipcc, gfx950) first")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def _arg(a):
    if isinstance(a, torch.Tensor):
        return a.data_ptr()
    return a


def stream_of(t):
    """Handle of torch's current HIP stream on t's device (the caller's stream)."""
    return torch.cuda.current_stream(t.device).cuda_stream


def call(name, *args):
    """Call an npn_* entry point; raise RuntimeError on a non-zero status.

    Every tensor argument must sit on one device: the kernels dereference the raw pointers
    on the device of the stream they are launched on."""
    devices = {a.device for a in args if isinstance(a, torch.Tensor)}
    if len(devices) > 1:
        raise RuntimeError(f"{name}: tensor arguments span devices {sorted(map(str, devices))}")
    status = getattr(lib(), name)(*[_arg(a) for a in args])
    if status != 0:
        text = lib().npn_status_string(status).decode()
        raise RuntimeError(f"{name} failed with status {status}: {text}")


def query(name, *args):
    """Call a size-query entry point and return its value."""
    return int(getattr(lib(), name)(*args))


def require(t, name, dtype, numel=None, shape=None):
    """Reference-style argument checks: CUDA device, dtype, contiguity, size."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be on a HIP device, got {t.device}")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
    if numel is not None and t.numel() != numel:
        raise RuntimeError(f"{name} must have {numel} elements, got {t.numel()} {tuple(t.shape)}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise RuntimeError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
