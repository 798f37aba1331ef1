"""Sliding-window helpers and the log-sum-exp reduce launcher.

Mirrors the host-facing pieces of kernels/pa_decode_swa.py:

* ``get_sw_max_context_partition_num`` -- kernels/pa_decode_swa.py:832-840
* ``pa_decode_sw_reduce``               -- the launch of ``compile_pa_decode_sw_reduce``
                                           (kernels/pa_decode_swa.py:843-1183)

The sliding-window decode itself runs through ``pa_decode_ps_launch`` (the
partition kernel takes the window as an argument), for every block size.
"""

from __future__ import annotations

import torch

from . import _lib

KV_COMPUTE_BLOCK = 256


def _cdiv(a: int, b: int) -> int:
    return (a + b - 1) // b


def get_sw_max_context_partition_num(
    sliding_window: int,
    context_partition_size: int = KV_COMPUTE_BLOCK,
    query_length: int = 1,
) -> int:
    """Partitions that can hold keys of a sliding window (kernels/pa_decode_swa.py:832-840)."""
    if sliding_window <= 0:
        return 0
    return _cdiv(sliding_window + query_length - 1, context_partition_size) + 1


_OUT_DTYPES = {"bf16": _lib.PA_FP8_BF16, "f16": _lib.PA_FP8_F16, "f32": _lib.PA_FP8_F32}


def _reduce_args(output_5d, exp_sums, max_logits, temporary_output, max_parts, output_dtype_str) -> _lib.ReduceArgs:
    a = _lib.ReduceArgs()
    a.output = output_5d.data_ptr()
    a.exp_sums = exp_sums.data_ptr()
    a.max_logits = max_logits.data_ptr()
    a.tmp_out = temporary_output.data_ptr()
    a.stride_o_seq, a.stride_o_len, a.stride_o_head, a.stride_o_group = (output_5d.stride(i) for i in range(4))
    a.stride_es_seq, a.stride_es_head, a.stride_es_part = (exp_sums.stride(i) for i in range(3))
    a.stride_to_seq, a.stride_to_head, a.stride_to_part, a.stride_to_group = (temporary_output.stride(i) for i in range(4))
    a.batch_size = output_5d.shape[0]
    a.query_length = output_5d.shape[1]
    a.num_kv_heads = output_5d.shape[2]
    a.query_group_size = output_5d.shape[3]
    a.head_dim = output_5d.shape[4]
    a.max_context_partition_num = max_parts
    a.out_dtype = _OUT_DTYPES[output_dtype_str]
    return a


def pa_decode_sw_reduce(
    output: torch.Tensor,
    exp_sums: torch.Tensor,
    max_logits: torch.Tensor,
    temporary_output: torch.Tensor,
    *,
    query_length: int,
    query_group_size: int,
    stream=None,
) -> None:
    """Merge partials [B, Hkv, P, ql*g(, D)] into ``output`` [B*ql, Hq, D] in place.

    out = sum_z w_z * tmp_out_z, w_z = s_z e^(m_z - M) / sum_z s_z e^(m_z - M)
    (kernels/pa_decode_swa.py:954-1130).
    """
    batch_size, num_kv_heads, max_parts, eqgs = exp_sums.shape
    head_size = temporary_output.shape[-1]
    if eqgs != query_length * query_group_size:
        raise ValueError("exp_sums last dim must equal query_length * query_group_size")
    if exp_sums.dtype != torch.float32 or max_logits.dtype != torch.float32 or temporary_output.dtype != torch.bfloat16:
        raise ValueError("exp_sums / max_logits must be float32 and temporary_output bfloat16")
    if exp_sums.stride(3) != 1 or exp_sums.stride() != max_logits.stride() or temporary_output.stride(4) != 1:
        raise ValueError("partials need unit last strides and exp_sums / max_logits must share strides")
    out_str = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}.get(output.dtype)
    if out_str is None:
        raise ValueError(f"Unsupported output dtype {output.dtype}")
    output_5d = output.view(batch_size, query_length, num_kv_heads, query_group_size, head_size)
    s = stream if stream is not None else torch.cuda.current_stream(output.device)
    handle = s.cuda_stream if hasattr(s, "cuda_stream") else int(s)
    _lib.lse_reduce(_reduce_args(output_5d, exp_sums, max_logits, temporary_output, max_parts, out_str), handle)
