"""Merge of the split works' partials of the persistent decode path.

The reference launcher ends its persistent path with
``aiter.ops.attention.pa_reduce_v1(partial_output[ql:], partial_lse[ql:],
reduce_indptr, reduce_final_map, reduce_partial_map, ql, output, None)``
(kernels/pa_decode_fp8.py:3189-3200).  aiter is not part of the reference
tree, so this is our own kernel with that call signature; the arithmetic is the
log-sum-exp merge of partial softmaxes:

    rows s_j = reduce_partial_map[j] + qi,  j in [reduce_indptr[g], reduce_indptr[g+1])
    LSE      = log sum_j exp(partial_lse[s_j, h])
    out[qo_start + qi, h, :] = sum_j exp(partial_lse[s_j, h] - LSE) * partial_output[s_j, h, :]

with ``(qo_start, qo_end) = reduce_final_map[g]``.
"""

from __future__ import annotations

import torch

from . import _lib

_OUT_DTYPES = {torch.bfloat16: _lib.PA_FP8_BF16, torch.float16: _lib.PA_FP8_F16, torch.float32: _lib.PA_FP8_F32}


def _reduce_v1_args(
    partial_output: torch.Tensor,
    partial_lse: torch.Tensor,
    reduce_indptr: torch.Tensor,
    reduce_final_map: torch.Tensor,
    reduce_partial_map: torch.Tensor,
    max_seqlen_q: int,
    final_output: torch.Tensor,
    final_lse: torch.Tensor = None,
) -> _lib.ReduceV1Args:
    if partial_output.dim() != 4 or partial_output.dtype != torch.float32:
        raise ValueError(f"partial_output must be float32 [rows, 1, heads, head_dim], got {tuple(partial_output.shape)}")
    rows, _, heads, head_dim = partial_output.shape
    if partial_lse.dim() != 4 or partial_lse.dtype != torch.float32 or tuple(partial_lse.shape) != (rows, 1, heads, 1):
        raise ValueError(f"partial_lse must be float32 [{rows}, 1, {heads}, 1], got {tuple(partial_lse.shape)}")
    if partial_output.stride(3) != 1:
        raise ValueError("partial_output needs a unit last stride")
    if final_output.dim() != 3 or final_output.shape[1] != heads or final_output.shape[2] != head_dim:
        raise ValueError(f"final_output must be [tokens, {heads}, {head_dim}], got {tuple(final_output.shape)}")
    if final_output.dtype not in _OUT_DTYPES or final_output.stride(2) != 1:
        raise ValueError(f"final_output must be bf16 / f16 / f32 with a unit last stride, got {final_output.dtype}")
    for name, t in (("reduce_indptr", reduce_indptr), ("reduce_partial_map", reduce_partial_map)):
        if t.dtype != torch.int32 or t.dim() != 1 or not t.is_contiguous():
            raise ValueError(f"`{name}` must be a contiguous 1-D int32 tensor")
    groups = reduce_indptr.shape[0] - 1
    if reduce_final_map.dtype != torch.int32 or not reduce_final_map.is_contiguous() or reduce_final_map.numel() < 2 * max(groups, 0):
        raise ValueError("`reduce_final_map` must be a contiguous int32 [groups, 2] tensor")
    if final_lse is not None and (final_lse.dtype != torch.float32 or final_lse.dim() != 2
                                  or tuple(final_lse.shape) != (final_output.shape[0], heads)):
        raise ValueError(f"final_lse must be float32 [{final_output.shape[0]}, {heads}]")
    a = _lib.ReduceV1Args()
    a.output = final_output.data_ptr()
    a.final_lse = final_lse.data_ptr() if final_lse is not None else None
    a.partial_output = partial_output.data_ptr()
    a.partial_lse = partial_lse.data_ptr()
    a.reduce_indptr = reduce_indptr.data_ptr()
    a.reduce_final_map = reduce_final_map.data_ptr()
    a.reduce_partial_map = reduce_partial_map.data_ptr()
    a.stride_po_row, a.stride_po_head = partial_output.stride(0), partial_output.stride(2)
    a.stride_pl_row, a.stride_pl_head = partial_lse.stride(0), partial_lse.stride(2)
    a.stride_out_row, a.stride_out_head = final_output.stride(0), final_output.stride(1)
    if final_lse is not None:
        a.stride_lse_row, a.stride_lse_head = final_lse.stride(0), final_lse.stride(1)
    a.num_groups = max(groups, 0)
    a.num_heads = heads
    a.head_dim = head_dim
    a.max_qlen = int(max_seqlen_q)
    a.partial_rows = rows
    a.output_rows = final_output.shape[0]
    a.partial_map_len = reduce_partial_map.shape[0]
    a.out_dtype = _OUT_DTYPES[final_output.dtype]
    return a


def pa_reduce_v1(
    partial_output: torch.Tensor,
    partial_lse: torch.Tensor,
    reduce_indptr: torch.Tensor,
    reduce_final_map: torch.Tensor,
    reduce_partial_map: torch.Tensor,
    max_seqlen_q: int,
    final_output: torch.Tensor,
    final_lse: torch.Tensor = None,
    stream=None,
) -> None:
    """Write the merged rows of every split group into ``final_output`` in place.

    ``partial_output`` [rows, 1, Hq, D] f32 and ``partial_lse`` [rows, 1, Hq, 1] f32
    start at the row the partial map's 0 refers to.  Groups with no partials and
    rows not named by ``reduce_final_map`` are left untouched.  ``final_lse``
    ([tokens, Hq] f32), when given, receives each merged row's log-sum-exp.
    """
    args = _reduce_v1_args(partial_output, partial_lse, reduce_indptr, reduce_final_map, reduce_partial_map,
                           max_seqlen_q, final_output, final_lse)
    s = stream if stream is not None else torch.cuda.current_stream(final_output.device)
    _lib.reduce_v1(args, s.cuda_stream if hasattr(s, "cuda_stream") else int(s))
