"""``get_pa_metadata_v1`` worklist scheduler -- host API.

Same signatures and buffer contract as kernels/pa_metadata.py:

* ``get_pa_metadata_info_v1`` -- kernels/pa_metadata.py:53-79
* ``get_pa_metadata_v1``      -- kernels/pa_metadata.py:450-524

The schedule itself runs on the device (pa_fp8_metadata_v1 in libpa_fp8.so).
work_info layout (8 x int32 per work):
  [0] batch  [1] partial_qo_loc (-1 = direct)  [2] qo_start  [3] qo_end
  [4] kv_start  [5] kv_end (cumulative partition indices)  [6] 0
  [7] (qhead_end << 16) | (qhead_start & 0xFFFF)
"""

from __future__ import annotations

import torch

from . import _lib

_WORK_INFO_FIELDS = 8


def get_pa_metadata_info_v1(batch_size: int, num_head_k: int = 1, num_cu: int = None):
    """(shape, dtype) of work_metadata_ptrs, work_indptr, work_info_set,
    reduce_indptr, reduce_final_map, reduce_partial_map (kernels/pa_metadata.py:53-79)."""
    if num_cu is None:
        num_cu = torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    max_work = (batch_size + num_cu - 1) * num_head_k
    max_split_tiles = min(batch_size + num_cu - 1, (num_cu - 1) * 2)
    return (
        ((2,), torch.uint64),
        ((num_cu + 1,), torch.int32),
        ((max_work, _WORK_INFO_FIELDS), torch.int32),
        ((batch_size + 1,), torch.int32),
        ((batch_size, 2), torch.int32),
        ((max_split_tiles,), torch.int32),
    )


def _is_pow2(x: int) -> bool:
    return x > 0 and (x & (x - 1)) == 0


def get_pa_metadata_v1(
    seqlens_qo_indptr: torch.Tensor,
    pages_kv_indptr: torch.Tensor,
    context_lens: torch.Tensor,
    num_heads_per_head_k: int,
    num_heads_k: int,
    is_causal: bool,
    work_metadata_ptrs: torch.Tensor,
    work_indptr: torch.Tensor,
    work_info: torch.Tensor,
    reduce_indptr: torch.Tensor,
    reduce_final_map: torch.Tensor,
    reduce_partial_map: torch.Tensor,
    kv_granularity: int = 16,
    block_size: int = 16,
    max_seqlen_qo: int = -1,
    uni_seqlen_qo: int = -1,
    fast_mode: bool = True,
    topk: int = -1,
    max_split_per_batch: int = -1,
    num_cu: int = None,
) -> None:
    """Fill the worklist buffers in place (kernels/pa_metadata.py:450-524).

    Causal, non-sparse, uniform query length only (the reference asserts the
    same, :481-483).  ``pages_kv_indptr`` is accepted for signature
    compatibility; the schedule counts ``ceil(context_len / kv_granularity)``
    partitions per sequence.
    """
    assert is_causal, "pa_metadata only supports causal"
    assert topk == -1, "pa_metadata does not support sparse (topk)"
    assert uni_seqlen_qo >= 1, "pa_metadata requires uniform qo length"
    dev = context_lens.device
    if num_cu is None:
        num_cu = torch.cuda.get_device_properties(dev).multi_processor_count
    assert _is_pow2(kv_granularity), "kv_granularity must be power of 2"
    assert num_cu % num_heads_k == 0, "num_cu must be divisible by num_heads_k"
    num_batches = context_lens.shape[0]
    for name, t in (("seqlens_qo_indptr", seqlens_qo_indptr), ("context_lens", context_lens),
                    ("work_indptr", work_indptr), ("work_info", work_info), ("reduce_indptr", reduce_indptr),
                    ("reduce_final_map", reduce_final_map), ("reduce_partial_map", reduce_partial_map)):
        if t.dtype != torch.int32 or not t.is_contiguous() or t.device != dev:
            raise ValueError(f"`{name}` must be a contiguous int32 tensor on {dev}")
    if seqlens_qo_indptr.numel() < num_batches + 1 or work_indptr.numel() < num_cu + 1:
        raise ValueError("seqlens_qo_indptr / work_indptr too small")
    if reduce_indptr.numel() < num_batches + 1 or reduce_final_map.numel() < 2 * num_batches:
        raise ValueError("reduce_indptr / reduce_final_map too small")
    if work_info.numel() % _WORK_INFO_FIELDS:
        raise ValueError("work_info must hold 8 int32 per work")
    # The schedule can need every row get_pa_metadata_info_v1 sizes (kernels/pa_metadata.py:
    # 63-72); the device marks an overflow only in work_indptr[0], which the decode would
    # read as a truncated worklist, so smaller buffers are refused here (no device read).
    max_work = (num_batches + num_cu - 1) * num_heads_k
    max_split = min(num_batches + num_cu - 1, 2 * (num_cu - 1))
    if work_info.numel() // _WORK_INFO_FIELDS < max_work:
        raise ValueError(f"work_info holds {work_info.numel() // _WORK_INFO_FIELDS} works; the schedule may need "
                         f"{max_work} ((batch + num_cu - 1) * num_heads_k, get_pa_metadata_info_v1)")
    if reduce_partial_map.numel() < max_split:
        raise ValueError(f"reduce_partial_map holds {reduce_partial_map.numel()} entries; the schedule may need "
                         f"{max_split} (min(batch + num_cu - 1, 2 * (num_cu - 1)), get_pa_metadata_info_v1)")
    if work_metadata_ptrs is not None and work_metadata_ptrs.numel() >= 2:
        # device fills (capturable into a graph), not host-to-device copies
        ptrs = work_metadata_ptrs.view(torch.int64)
        ptrs[0:1].fill_(work_indptr.data_ptr())
        ptrs[1:2].fill_(work_info.data_ptr())
    a = _lib.MetadataArgs()
    a.seqlens_qo_indptr = seqlens_qo_indptr.data_ptr()
    a.context_lens = context_lens.data_ptr()
    a.work_indptr = work_indptr.data_ptr()
    a.work_info = work_info.data_ptr()
    a.reduce_indptr = reduce_indptr.data_ptr()
    a.reduce_final_map = reduce_final_map.data_ptr()
    a.reduce_partial_map = reduce_partial_map.data_ptr()
    a.num_batches = num_batches
    a.gqa = num_heads_per_head_k
    a.num_heads_k = num_heads_k
    a.num_cu = num_cu
    a.kv_granularity = kv_granularity
    a.query_length = uni_seqlen_qo
    a.max_work = work_info.numel() // _WORK_INFO_FIELDS
    a.max_split_tiles = reduce_partial_map.numel()
    _lib.metadata_v1(a, torch.cuda.current_stream(dev).cuda_stream)
