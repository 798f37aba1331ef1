"""The C ABI: libpa_fp8.so loads without a GPU, exports every function
include/pa_fp8.h declares, its argument structs have the layout the ctypes
binding assumes, and argument validation returns the documented status codes
(these calls return before any device work)."""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "pa_fp8.h"


@pytest.fixture(scope="module")
def lib():
    import importlib.util

    # The recipe is loaded by path: importing it through the package would run
    # flydsl_amd/__init__.py, which needs the library it builds.
    spec = importlib.util.spec_from_file_location("_flydsl_amd_build", ROOT / "flydsl_amd" / "build.py")
    fbuild = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(fbuild)
    if not fbuild.LIB_PATH.exists():
        fbuild.build()
    from flydsl_amd import _lib

    return _lib


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^[A-Za-z_][\w \*]*?\b(pa_fp8_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_expected_api():
    assert declared_functions() == sorted(
        ["pa_fp8_decode_partitions", "pa_fp8_decode_partitions_noalloc", "pa_fp8_lse_reduce", "pa_fp8_decode_worklist", "pa_fp8_reduce_v1",
         "pa_fp8_metadata_v1", "pa_fp8_metadata_multi", "pa_fp8_rope_cache", "pa_fp8_hw_reciprocal",
         "pa_fp8_status_string", "pa_fp8_abi_version"]
    )


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib.LIB_PATH)], capture_output=True, text=True, check=True)
    exported = set(re.findall(r"\bT\s+(\w+)$", out.stdout, flags=re.M))
    for name in declared_functions():
        assert name in exported, name
        assert hasattr(lib.LIB, name)
    assert set(lib.EXPORTED_SYMBOLS) == set(declared_functions())


def test_abi_version(lib):
    assert lib.LIB.pa_fp8_abi_version() == lib.PA_FP8_ABI_VERSION
    assert f"#define PA_FP8_ABI_VERSION {lib.PA_FP8_ABI_VERSION}" in HEADER.read_text()


STRUCTS = {
    "pa_fp8_decode_args": "DecodeArgs",
    "pa_fp8_reduce_args": "ReduceArgs",
    "pa_fp8_worklist_args": "WorklistArgs",
    "pa_fp8_reduce_v1_args": "ReduceV1Args",
    "pa_fp8_metadata_args": "MetadataArgs",
    "pa_fp8_rope_cache_args": "RopeCacheArgs",
}


def test_struct_layouts_match_header(lib, tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "pa_fp8.h"', "int main(void) {"]
    for cname, pyname in STRUCTS.items():
        cls = getattr(lib, pyname)
        lines.append(f'printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        s, f, v = line.split()
        got[(s, f)] = int(v)
    for cname, pyname in STRUCTS.items():
        cls = getattr(lib, pyname)
        assert got[(cname, "sizeof")] == ctypes.sizeof(cls), cname
        for field, _ in cls._fields_:
            assert got[(cname, field)] == getattr(cls, field).offset, (cname, field)


def _decode_args(lib, **over):
    a = lib.DecodeArgs()
    a.batch_size, a.num_kv_heads, a.query_group_size, a.query_length = 0, 8, 4, 1
    a.head_dim, a.block_size, a.max_context_partition_num = 128, 16, 8
    for k, v in over.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize(
    "over,status",
    [
        ({}, 0),  # an empty batch is a no-op
        ({"head_dim": 64}, 0),
        ({"head_dim": 192}, 0),
        ({"head_dim": 256}, 0),
        ({"head_dim": 96}, 2),
        ({"head_dim": 320}, 2),
        ({"block_size": 8}, 3),
        ({"block_size": 48}, 3),
        ({"query_group_size": 65}, 0),  # more than 64 rows run as row chunks
        ({"query_length": 8, "query_group_size": 16}, 0),
        ({"query_group_size": 65536}, 4),
        ({"query_length": 300, "query_group_size": 256}, 4),
        ({"value_layout": 1}, 0),
        ({"value_layout": 2}, 9),
        ({"max_context_partition_num": 0}, 7),
        ({"query_dtype": 2}, 6),
        ({"num_kv_heads": 0}, 5),
        ({"direct_output": 1}, 7),
        ({"waves_per_slot": 3}, 5),
        ({"batch_size": 3}, 1),  # null pointers
        # the chained layout: one 16-row group, head_dim 128, the trans_v layout
        ({"slots_per_wave": 2}, 0),
        ({"slots_per_wave": 2, "waves_per_slot": 4}, 0),
        ({"slots_per_wave": -1}, 5),
        ({"slots_per_wave": 2, "query_group_size": 32}, 5),
        ({"slots_per_wave": 2, "head_dim": 64}, 5),
        ({"slots_per_wave": 2, "value_layout": 1}, 5),
        # several slots written to the output: only workgroups that hold every slot
        ({"direct_output": 1, "slots_per_wave": 2, "waves_per_slot": 4}, 0),
        ({"direct_output": 1, "slots_per_wave": 2, "waves_per_slot": 2}, 7),
        ({"direct_output": 1, "slots_per_wave": 0, "waves_per_slot": 8}, 7),
        ({"direct_output": 1, "slots_per_wave": 8, "waves_per_slot": 1, "batch_size": 3}, 1),  # null pointers
    ],
)
def test_decode_validation_codes(lib, over, status):
    assert lib.LIB.pa_fp8_decode_partitions(ctypes.byref(_decode_args(lib, **over)), None) == status


def test_null_args_and_status_strings(lib):
    assert lib.LIB.pa_fp8_decode_partitions(None, None) == 1
    assert lib.LIB.pa_fp8_lse_reduce(None, None) == 1
    assert lib.LIB.pa_fp8_metadata_v1(None, None) == 1
    assert lib.LIB.pa_fp8_decode_worklist(None, None) == 1
    assert lib.LIB.pa_fp8_reduce_v1(None, None) == 1
    assert lib.LIB.pa_fp8_rope_cache(None, None) == 1
    for code in range(0, 11):
        assert lib.LIB.pa_fp8_status_string(code)
    assert b"scratch" in lib.LIB.pa_fp8_status_string(lib.PA_FP8_ERR_SCRATCH)
    with pytest.raises(lib.PaFp8Error, match="status 2"):
        lib.check("pa_fp8_decode_partitions", 2)


def test_noalloc_validation_codes(lib):
    """The allocation-free decode returns before any device work on these."""
    assert lib.LIB.pa_fp8_decode_partitions_noalloc(None, None) == 1
    a = _decode_args(lib)  # empty batch
    assert lib.LIB.pa_fp8_decode_partitions_noalloc(ctypes.byref(a), None) == 0
    a.out_dtype = 3
    assert lib.LIB.pa_fp8_decode_partitions_noalloc(ctypes.byref(a), None) == 6
    # 4096 x 8 heads x 8 slots x 4 rows of partials need 69 MB: more than the scratch
    big = _decode_args(lib, batch_size=4096)
    assert lib.LIB.pa_fp8_decode_partitions_noalloc(ctypes.byref(big), None) == lib.PA_FP8_ERR_SCRATCH
    assert lib.LIB.pa_fp8_decode_partitions_noalloc(ctypes.byref(_decode_args(lib, head_dim=96)), None) == 2


def test_reduce_and_metadata_validation(lib):
    r = lib.ReduceArgs()
    r.batch_size, r.num_kv_heads, r.query_group_size, r.query_length, r.head_dim = 0, 8, 4, 1, 128
    r.max_context_partition_num, r.out_dtype = 8, 0
    assert lib.LIB.pa_fp8_lse_reduce(ctypes.byref(r), None) == 0
    r.out_dtype = 7
    assert lib.LIB.pa_fp8_lse_reduce(ctypes.byref(r), None) == 6
    r.out_dtype, r.head_dim = 0, 320
    assert lib.LIB.pa_fp8_lse_reduce(ctypes.byref(r), None) == 2
    m = lib.MetadataArgs()
    m.num_batches, m.gqa, m.num_heads_k, m.num_cu, m.kv_granularity, m.query_length = 4, 4, 8, 12, 256, 1
    assert lib.LIB.pa_fp8_metadata_v1(ctypes.byref(m), None) == 5  # 12 bins not a multiple of 8 heads
    m.num_cu, m.kv_granularity = 16, 100
    assert lib.LIB.pa_fp8_metadata_v1(ctypes.byref(m), None) == 5  # granularity not a power of two
    m.kv_granularity = 256
    assert lib.LIB.pa_fp8_metadata_v1(ctypes.byref(m), None) == 1  # null buffers


def test_metadata_accepts_null_for_empty_buffers(lib):
    """One bin per kv head gives get_pa_metadata_info_v1 a zero-entry
    reduce_partial_map (min(B + cu - 1, 2 (cu - 1)) = 0), and torch gives an empty
    tensor a NULL data pointer: the scheduler must take it (every write to it is
    bounded by max_split_tiles).  Without a GPU the call then fails at the launch,
    never at the argument check."""
    m = lib.MetadataArgs()
    m.num_batches, m.gqa, m.num_heads_k, m.num_cu, m.kv_granularity, m.query_length = 3, 4, 1, 1, 256, 1
    buf = (ctypes.c_int32 * 64)()
    for name in ("seqlens_qo_indptr", "context_lens", "work_indptr", "work_info", "reduce_indptr", "reduce_final_map"):
        setattr(m, name, ctypes.cast(buf, ctypes.c_void_p).value)
    m.max_work, m.max_split_tiles = 3, 0
    assert lib.LIB.pa_fp8_metadata_v1(ctypes.byref(m), None) != 1
    m.max_split_tiles = 2  # a buffer with entries must not be NULL
    assert lib.LIB.pa_fp8_metadata_v1(ctypes.byref(m), None) == 1


def test_metadata_null_query_offsets_mean_uniform_query_length(lib):
    """A NULL seqlens_qo_indptr stands for b * query_length (what get_pa_metadata
    passes); it is refused with a shape error when that would overflow int32."""
    m = lib.MetadataArgs()
    m.num_batches, m.gqa, m.num_heads_k, m.num_cu, m.kv_granularity, m.query_length = 3, 4, 1, 2, 256, 4
    buf = (ctypes.c_int32 * 64)()
    for name in ("context_lens", "work_indptr", "work_info", "reduce_indptr", "reduce_final_map", "reduce_partial_map"):
        setattr(m, name, ctypes.cast(buf, ctypes.c_void_p).value)
    m.seqlens_qo_indptr = None
    m.max_work, m.max_split_tiles = 4, 2
    assert lib.LIB.pa_fp8_metadata_v1(ctypes.byref(m), None) not in (1, 5)
    m.num_batches, m.query_length = 1 << 20, 4096
    assert lib.LIB.pa_fp8_metadata_v1(ctypes.byref(m), None) == 5


def _worklist_args(lib, **over):
    a = lib.WorklistArgs()
    a.batch_size, a.num_kv_heads, a.query_group_size, a.query_length = 0, 1, 8, 1
    a.head_dim, a.block_size, a.num_cu, a.num_blocks = 128, 1024, 8, 4
    for k, v in over.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize(
    "over,status",
    [
        ({}, 0),  # an empty batch is a no-op
        ({"batch_size": 2, "num_cu": 0}, 0),  # no workgroups: nothing to launch
        ({"head_dim": 96}, 2),
        ({"head_dim": 256}, 0),
        ({"block_size": 1000}, 3),
        ({"query_length": 5, "query_group_size": 16}, 0),  # row chunks
        ({"query_length": 5, "query_group_size": 16384}, 4),
        ({"value_layout": 1}, 0),
        ({"value_layout": 5}, 9),
        ({"query_dtype": 2}, 6),
        ({"out_dtype": 5}, 6),
        ({"num_cu": -1}, 5),
        ({"batch_size": 2}, 1),  # null pointers
    ],
)
def test_worklist_validation_codes(lib, over, status):
    assert lib.LIB.pa_fp8_decode_worklist(ctypes.byref(_worklist_args(lib, **over)), None) == status


def test_reduce_v1_validation(lib):
    r = lib.ReduceV1Args()
    r.num_groups, r.num_heads, r.head_dim, r.max_qlen, r.partial_map_len = 0, 8, 128, 1, 4
    assert lib.LIB.pa_fp8_reduce_v1(ctypes.byref(r), None) == 0  # no groups: no-op
    r.head_dim = 64
    assert lib.LIB.pa_fp8_reduce_v1(ctypes.byref(r), None) == 0
    r.head_dim = 258
    assert lib.LIB.pa_fp8_reduce_v1(ctypes.byref(r), None) == 2
    r.head_dim, r.num_groups, r.out_dtype = 128, 3, 9
    assert lib.LIB.pa_fp8_reduce_v1(ctypes.byref(r), None) == 6
    r.out_dtype = 0
    assert lib.LIB.pa_fp8_reduce_v1(ctypes.byref(r), None) == 0  # no partial rows: nothing to merge
    r.partial_rows = 4
    assert lib.LIB.pa_fp8_reduce_v1(ctypes.byref(r), None) == 1  # null buffers
    r.max_qlen = 0
    assert lib.LIB.pa_fp8_reduce_v1(ctypes.byref(r), None) == 5


def _rope_args(lib, **over):
    """Zero tokens and fake (never dereferenced) 16-byte aligned pointers: validation only."""
    a = lib.RopeCacheArgs()
    for i, name in enumerate(["query", "key", "value", "positions", "cos_cache", "sin_cache", "slot_mapping",
                              "key_cache", "value_cache", "query_out", "key_out", "key_scale", "value_scale"]):
        setattr(a, name, 0x10000 + 0x100 * i)
    a.num_tokens, a.num_q_heads, a.num_kv_heads, a.head_dim = 0, 8, 1, 128
    a.block_size, a.num_blocks, a.max_pos = 16, 4, 64
    a.stride_q_token, a.stride_q_head = 8 * 128, 128
    a.stride_kc_block, a.stride_kc_head, a.stride_vc_block, a.stride_vc_head = 2048, 2048, 2048, 2048
    a.elem_dtype, a.cache_format, a.kv_layout = lib.PA_FP8_BF16, lib.PA_FP8_CACHE_FP8_TOKEN, lib.PA_FP8_KV_X_TRANS
    for k, v in over.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize(
    "over,status",
    [
        ({}, 0),  # no tokens: nothing to launch
        ({"head_dim": 72}, 2),
        ({"head_dim": 2048}, 2),
        ({"elem_dtype": 2}, 6),
        ({"cache_format": 3}, 9),
        ({"kv_layout": 3}, 9),
        ({"block_size": 8}, 9),  # trans_v V needs block_size % 16 == 0
        ({"block_size": 8, "kv_layout": 1}, 0),  # 4-D V takes any block size
        ({"num_tokens": -1}, 5),
        ({"num_kv_heads": 0}, 5),
        ({"max_pos": 0}, 5),
        ({"query": 0x10008}, 5),  # 16-bit rows must be 16-byte aligned
        ({"stride_q_head": 100}, 5),
        ({"key_cache": 0x10004}, 5),  # fp8 runs of 8 head dims: 8-byte aligned
        ({"key_scale": 0}, 1),
        ({"key_scale": 0, "cache_format": 0, "key_cache": 0x10000, "value_cache": 0x10000}, 0),
        ({"slot_mapping": 0}, 0),  # empty per-token tensors are fine without tokens
        ({"slot_mapping": 0, "num_tokens": 1}, 1),
        ({"cos_cache": 0}, 1),
    ],
)
def test_rope_cache_validation_codes(lib, over, status):
    assert lib.LIB.pa_fp8_rope_cache(ctypes.byref(_rope_args(lib, **over)), None) == status


def test_hw_reciprocal_validation_codes(lib):
    # checked before any device call; an empty range is a no-op
    assert lib.LIB.pa_fp8_hw_reciprocal(None, None, -1, None) == 5  # PA_FP8_ERR_SHAPE
    assert lib.LIB.pa_fp8_hw_reciprocal(None, None, 4, None) == 1  # PA_FP8_ERR_NULL_POINTER
    assert lib.LIB.pa_fp8_hw_reciprocal(None, None, 0, None) == 0
