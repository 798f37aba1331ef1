"""ctypes binding of libpa_fp8.so (the C ABI declared in include/pa_fp8.h).

The library is required: importing this module when it has not been built
raises, and there is no CPU or PyTorch fallback for any kernel.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

_HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("PA_FP8_LIB", str(_HERE / "libpa_fp8.so")))

PA_FP8_ABI_VERSION = 10
PA_FP8_BF16, PA_FP8_F16, PA_FP8_F32 = 0, 1, 2
PA_FP8_CACHE_ELEM, PA_FP8_CACHE_FP8_TENSOR, PA_FP8_CACHE_FP8_TOKEN = 0, 1, 2
PA_FP8_KV_FLASH, PA_FP8_KV_X_PACKED, PA_FP8_KV_X_TRANS = 0, 1, 2
PA_FP8_V_TRANS, PA_FP8_V_4D = 0, 1
PA_FP8_ERR_SCRATCH = 10
PA_FP8_NOALLOC_SCRATCH_BYTES = 32 << 20

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("exp_sums", _vp),
        ("max_logits", _vp),
        ("tmp_out", _vp),
        ("query", _vp),
        ("key_cache", _vp),
        ("value_cache", _vp),
        ("block_tables", _vp),
        ("context_lengths", _vp),
        ("key_scale", _vp),
        ("value_scale", _vp),
        ("stride_q_seq", _i64),
        ("stride_q_head", _i64),
        ("stride_k_block", _i64),
        ("stride_k_head", _i64),
        ("stride_v_block", _i64),
        ("stride_v_head", _i64),
        ("stride_es_seq", _i64),
        ("stride_es_head", _i64),
        ("stride_es_part", _i64),
        ("stride_to_seq", _i64),
        ("stride_to_head", _i64),
        ("stride_to_part", _i64),
        ("stride_to_group", _i64),
        ("stride_bt_seq", _i64),
        ("stride_ks_block", _i64),
        ("stride_ks_head", _i64),
        ("batch_size", _i32),
        ("num_kv_heads", _i32),
        ("query_group_size", _i32),
        ("query_length", _i32),
        ("head_dim", _i32),
        ("block_size", _i32),
        ("num_blocks", _i32),
        ("max_blocks_per_seq", _i32),
        ("max_context_partition_num", _i32),
        ("sliding_window", _i32),
        ("per_token_kv", _i32),
        ("query_dtype", _i32),
        ("softmax_scale", _f32),
        ("direct_output", _i32),
        ("out_dtype", _i32),
        ("output", _vp),
        ("stride_o_seq", _i64),
        ("stride_o_len", _i64),
        ("stride_o_head", _i64),
        ("stride_o_group", _i64),
        ("waves_per_slot", _i32),
        ("value_layout", _i32),
        ("slots_per_wave", _i32),
    ]


class ReduceArgs(ctypes.Structure):
    _fields_ = [
        ("output", _vp),
        ("exp_sums", _vp),
        ("max_logits", _vp),
        ("tmp_out", _vp),
        ("stride_o_seq", _i64),
        ("stride_o_len", _i64),
        ("stride_o_head", _i64),
        ("stride_o_group", _i64),
        ("stride_es_seq", _i64),
        ("stride_es_head", _i64),
        ("stride_es_part", _i64),
        ("stride_to_seq", _i64),
        ("stride_to_head", _i64),
        ("stride_to_part", _i64),
        ("stride_to_group", _i64),
        ("batch_size", _i32),
        ("num_kv_heads", _i32),
        ("query_group_size", _i32),
        ("query_length", _i32),
        ("head_dim", _i32),
        ("max_context_partition_num", _i32),
        ("out_dtype", _i32),
        ("reserved", _i32),
    ]


class WorklistArgs(ctypes.Structure):
    _fields_ = [
        ("output", _vp),
        ("partial_output", _vp),
        ("partial_lse", _vp),
        ("query", _vp),
        ("key_cache", _vp),
        ("value_cache", _vp),
        ("context_lengths", _vp),
        ("key_scale", _vp),
        ("value_scale", _vp),
        ("work_indptr", _vp),
        ("work_info", _vp),
        ("kv_page_indices", _vp),
        ("kv_indptr", _vp),
        ("partition_indptr", _vp),
        ("stride_q_seq", _i64),
        ("stride_q_head", _i64),
        ("stride_k_block", _i64),
        ("stride_k_head", _i64),
        ("stride_v_block", _i64),
        ("stride_v_head", _i64),
        ("stride_out_seq", _i64),
        ("stride_out_head", _i64),
        ("stride_po_row", _i64),
        ("stride_pl_row", _i64),
        ("stride_ks_block", _i64),
        ("stride_ks_head", _i64),
        ("batch_size", _i32),
        ("num_kv_heads", _i32),
        ("query_group_size", _i32),
        ("query_length", _i32),
        ("head_dim", _i32),
        ("block_size", _i32),
        ("num_blocks", _i32),
        ("num_pages", _i32),
        ("num_cu", _i32),
        ("max_work", _i32),
        ("partial_rows", _i32),
        ("output_rows", _i32),
        ("per_token_kv", _i32),
        ("query_dtype", _i32),
        ("out_dtype", _i32),
        ("softmax_scale", _f32),
        ("bin_groups", _i32),
        ("value_layout", _i32),
    ]


class ReduceV1Args(ctypes.Structure):
    _fields_ = [
        ("output", _vp),
        ("final_lse", _vp),
        ("partial_output", _vp),
        ("partial_lse", _vp),
        ("reduce_indptr", _vp),
        ("reduce_final_map", _vp),
        ("reduce_partial_map", _vp),
        ("stride_po_row", _i64),
        ("stride_po_head", _i64),
        ("stride_pl_row", _i64),
        ("stride_pl_head", _i64),
        ("stride_out_row", _i64),
        ("stride_out_head", _i64),
        ("stride_lse_row", _i64),
        ("stride_lse_head", _i64),
        ("num_groups", _i32),
        ("num_heads", _i32),
        ("head_dim", _i32),
        ("max_qlen", _i32),
        ("partial_rows", _i32),
        ("output_rows", _i32),
        ("partial_map_len", _i32),
        ("out_dtype", _i32),
    ]


class MetadataArgs(ctypes.Structure):
    _fields_ = [
        ("seqlens_qo_indptr", _vp),
        ("context_lens", _vp),
        ("work_indptr", _vp),
        ("work_info", _vp),
        ("reduce_indptr", _vp),
        ("reduce_final_map", _vp),
        ("reduce_partial_map", _vp),
        ("num_batches", _i32),
        ("gqa", _i32),
        ("num_heads_k", _i32),
        ("num_cu", _i32),
        ("kv_granularity", _i32),
        ("query_length", _i32),
        ("max_work", _i32),
        ("max_split_tiles", _i32),
        ("partition_indptr", _vp),
        ("uniform_context", _vp),
        ("bin_groups", _i32),
        ("bin_weight", _i32 * 4),
        ("partial_count", _vp),
        ("pack", _i32),
    ]


class RopeCacheArgs(ctypes.Structure):
    _fields_ = [
        ("query", _vp),
        ("key", _vp),
        ("value", _vp),
        ("positions", _vp),
        ("cos_cache", _vp),
        ("sin_cache", _vp),
        ("slot_mapping", _vp),
        ("key_cache", _vp),
        ("value_cache", _vp),
        ("query_out", _vp),
        ("key_out", _vp),
        ("key_scale", _vp),
        ("value_scale", _vp),
        ("stride_q_token", _i64),
        ("stride_q_head", _i64),
        ("stride_k_token", _i64),
        ("stride_k_head", _i64),
        ("stride_v_token", _i64),
        ("stride_v_head", _i64),
        ("stride_qo_token", _i64),
        ("stride_qo_head", _i64),
        ("stride_ko_token", _i64),
        ("stride_ko_head", _i64),
        ("stride_cos_pos", _i64),
        ("stride_sin_pos", _i64),
        ("stride_kc_block", _i64),
        ("stride_kc_head", _i64),
        ("stride_kc_token", _i64),
        ("stride_vc_block", _i64),
        ("stride_vc_head", _i64),
        ("stride_vc_token", _i64),
        ("stride_ks_block", _i64),
        ("stride_ks_head", _i64),
        ("num_tokens", _i32),
        ("num_q_heads", _i32),
        ("num_kv_heads", _i32),
        ("head_dim", _i32),
        ("block_size", _i32),
        ("num_blocks", _i32),
        ("max_pos", _i32),
        ("elem_dtype", _i32),
        ("cache_format", _i32),
        ("kv_layout", _i32),
        ("reuse_freqs_front_part", _i32),
        ("positions_i64", _i32),
        ("slots_i64", _i32),
        ("reserved", _i32),
    ]


EXPORTED_SYMBOLS = (
    "pa_fp8_decode_partitions",
    "pa_fp8_decode_partitions_noalloc",
    "pa_fp8_lse_reduce",
    "pa_fp8_decode_worklist",
    "pa_fp8_reduce_v1",
    "pa_fp8_metadata_v1",
    "pa_fp8_metadata_multi",
    "pa_fp8_rope_cache",
    "pa_fp8_hw_reciprocal",
    "pa_fp8_status_string",
    "pa_fp8_abi_version",
)


class PaFp8Error(RuntimeError):
    """A libpa_fp8 entry point returned a non-zero status."""

    def __init__(self, func: str, status: int, text: str):
        super().__init__(f"{func} failed with status {status}: {text}")
        self.status = status


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"libpa_fp8.so not found at {LIB_PATH}; build it with `python flydsl_amd/build.py` "
            "(there is no fallback implementation)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    lib.pa_fp8_abi_version.argtypes = []
    lib.pa_fp8_abi_version.restype = ctypes.c_int
    ver = lib.pa_fp8_abi_version()
    if ver != PA_FP8_ABI_VERSION:
        raise ImportError(f"libpa_fp8.so ABI version {ver} != expected {PA_FP8_ABI_VERSION}; rebuild the library")
    lib.pa_fp8_decode_partitions.argtypes = [ctypes.POINTER(DecodeArgs), _vp]
    lib.pa_fp8_decode_partitions.restype = ctypes.c_int
    lib.pa_fp8_decode_partitions_noalloc.argtypes = [ctypes.POINTER(DecodeArgs), _vp]
    lib.pa_fp8_decode_partitions_noalloc.restype = ctypes.c_int
    lib.pa_fp8_lse_reduce.argtypes = [ctypes.POINTER(ReduceArgs), _vp]
    lib.pa_fp8_lse_reduce.restype = ctypes.c_int
    lib.pa_fp8_decode_worklist.argtypes = [ctypes.POINTER(WorklistArgs), _vp]
    lib.pa_fp8_decode_worklist.restype = ctypes.c_int
    lib.pa_fp8_reduce_v1.argtypes = [ctypes.POINTER(ReduceV1Args), _vp]
    lib.pa_fp8_reduce_v1.restype = ctypes.c_int
    lib.pa_fp8_metadata_v1.argtypes = [ctypes.POINTER(MetadataArgs), _vp]
    lib.pa_fp8_metadata_v1.restype = ctypes.c_int
    lib.pa_fp8_metadata_multi.argtypes = [ctypes.POINTER(MetadataArgs), ctypes.c_int32, _vp]
    lib.pa_fp8_metadata_multi.restype = ctypes.c_int
    lib.pa_fp8_rope_cache.argtypes = [ctypes.POINTER(RopeCacheArgs), _vp]
    lib.pa_fp8_rope_cache.restype = ctypes.c_int
    lib.pa_fp8_hw_reciprocal.argtypes = [_vp, _vp, ctypes.c_int64, _vp]
    lib.pa_fp8_hw_reciprocal.restype = ctypes.c_int
    lib.pa_fp8_status_string.argtypes = [ctypes.c_int]
    lib.pa_fp8_status_string.restype = ctypes.c_char_p
    return lib


LIB = _load()


def check(func: str, status: int) -> None:
    if status != 0:
        raise PaFp8Error(func, status, LIB.pa_fp8_status_string(status).decode())


def decode_partitions(args: DecodeArgs, stream: int) -> None:
    check("pa_fp8_decode_partitions", LIB.pa_fp8_decode_partitions(ctypes.byref(args), _vp(stream)))


def decode_partitions_noalloc(args: DecodeArgs, stream: int) -> None:
    check("pa_fp8_decode_partitions_noalloc", LIB.pa_fp8_decode_partitions_noalloc(ctypes.byref(args), _vp(stream)))


def lse_reduce(args: ReduceArgs, stream: int) -> None:
    check("pa_fp8_lse_reduce", LIB.pa_fp8_lse_reduce(ctypes.byref(args), _vp(stream)))


def decode_worklist(args: WorklistArgs, stream: int) -> None:
    check("pa_fp8_decode_worklist", LIB.pa_fp8_decode_worklist(ctypes.byref(args), _vp(stream)))


def reduce_v1(args: ReduceV1Args, stream: int) -> None:
    check("pa_fp8_reduce_v1", LIB.pa_fp8_reduce_v1(ctypes.byref(args), _vp(stream)))


def metadata_v1(args: MetadataArgs, stream: int) -> None:
    check("pa_fp8_metadata_v1", LIB.pa_fp8_metadata_v1(ctypes.byref(args), _vp(stream)))


def metadata_multi(args, stream: int) -> None:
    """Several schedules in one launch: ``args`` is a ctypes array of MetadataArgs."""
    check("pa_fp8_metadata_multi", LIB.pa_fp8_metadata_multi(args, len(args), _vp(stream)))


def rope_cache(args: RopeCacheArgs, stream: int) -> None:
    check("pa_fp8_rope_cache", LIB.pa_fp8_rope_cache(ctypes.byref(args), _vp(stream)))


def hw_reciprocal(x_ptr: int, y_ptr: int, n: int, stream: int) -> None:
    """y[i] = v_rcp_f32(x[i]) on the device (float32 buffers of n elements)."""
    check("pa_fp8_hw_reciprocal", LIB.pa_fp8_hw_reciprocal(_vp(x_ptr), _vp(y_ptr), n, _vp(stream)))
