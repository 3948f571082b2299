"""Import every op module once, registering all torch.ops of the library:

  torch.ops.deltanet.{full, full_batched, full_fp8, verify_batched, verify_from_ckpt,
                      rollback, conv_rollback, chunked_prefill}
  torch.ops.gqa.{tail, tail_verify, kv_append}
  torch.ops.fp8.{matmul, matmul_partials, matmul_argmax, matmul_swiglu}
  torch.ops.spec.{accept_greedy, accept_rejection}
  torch.ops.normfuse.{rms_norm, residual_rms_norm}
  torch.ops.glue.{silu_mul, deltanet_split, gqa_split}

(The reference registers its ops by importing each *_ops module,
contrib/qwen3.6-27b/static_decode.py:29-34; importing the modules one by one works
the same way here.)
"""
import deltanet_full_ops  # noqa: F401
import deltanet_full_batched_ops  # noqa: F401
import deltanet_full_fp8_ops  # noqa: F401
import deltanet_verify_ops  # noqa: F401
import deltanet_chunked_ops  # noqa: F401
import gqa_tail_ops  # noqa: F401
import fp8_matmul_ops  # noqa: F401
import spec_accept_ops  # noqa: F401
import rms_norm_nki_ops  # noqa: F401
import glue_ops  # noqa: F401
