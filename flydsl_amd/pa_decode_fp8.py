"""Drop-in host API of the FP8 paged-attention decode path (gfx950 / MI355X).

Same names, arguments, return tags and error behaviour as the reference
launcher module kernels/pa_decode_fp8.py:

* ``pa_decode_ps_launch``     -- kernels/pa_decode_fp8.py:2812-3202
* ``get_pa_metadata``         -- kernels/pa_decode_fp8.py:1729-1859
* ``get_recommended_splits``  -- kernels/pa_decode_fp8.py:1922-1949

Every kernel is a hand-written HIP kernel in libpa_fp8.so reached through the
C ABI of include/pa_fp8.h; tensors are plain torch device tensors.
"""

from __future__ import annotations

import functools
import math
from collections import OrderedDict

import torch

from . import _lib
from .pa_decode_swa import _reduce_args, get_sw_max_context_partition_num  # noqa: F401
from .pa_metadata import get_pa_metadata_info_v1, get_pa_metadata_v1
from .pa_reduce import _reduce_v1_args

KV_COMPUTE_BLOCK = 256  # tokens per context partition (kernels/pa_decode_fp8.py:36)
# Worklist bins per CU: one per workgroup of the worklist kernel that fits a CU, so
# every bin's share of the batch runs from start to end.  The reference schedules 3
# (kernels/pa_decode_fp8.py:37-40).  Two 4-wave workgroups of the register-streaming
# kernel fit a CU (query rows per kv head ql * g <= 32); three of the LDS-staged one
# (ql * g > 32: three waves per SIMD, a 52.5 KiB ring each).
_PA_METADATA_GRID_OVERSUB = 2
_PA_METADATA_GRID_OVERSUB_STAGED = 3
_REFERENCE_BINS_PER_CU = 3  # the reference's _PA_METADATA_GRID_OVERSUB (kernels/pa_decode_fp8.py:37-40)


# Quota weights of the bin groups, first-dispatched group first.  Workgroups that
# share a CU progress at different rates (the one dispatched first issues ahead of
# the others): with even quotas, c5's three per CU ran 287 / 308 / 329 us and
# c3's two per CU 145 / 153 us.  The weights are the fastest of a sweep
# (three per CU: 108..145 for the first group; two per CU: 105..120).
_BIN_WEIGHTS = {2: (105, 100), 3: (115, 107, 100)}


def _metadata_bins_per_cu(query_length: int, query_group_size: int, head_dim: int = 128) -> int:
    """Worklist workgroups that fit a CU: at head_dim 128 and below two of the
    register-streaming kernel and three of the LDS-staged one; at 192 one and two
    (one wave per SIMD, a 76 KiB ring); at 256 one of either."""
    staged = query_length * query_group_size > 32
    if head_dim <= 128:
        return _PA_METADATA_GRID_OVERSUB_STAGED if staged else _PA_METADATA_GRID_OVERSUB
    if head_dim <= 192:
        return 2 if staged else 1
    return 1
_PA_DECODE_PS_SMALL_BLOCK_SIZES = (16, 64)  # kernels/pa_decode_fp8.py:1955
HEAD_DIM = 128
# Head dims the decode kernels are built for: the multiples of 64 up to 256 (the
# reference accepts every multiple of 64, kernels/pa_decode_fp8.py:969-970, :2084-2085).
HEAD_DIMS = (64, 128, 192, 256)
_MAX_QUERY_ROWS = 65535  # query_length * group size per kv head (the merge's grid)

_PACKED_FP8_QUERY_DTYPES = tuple(
    dt
    for dt in (torch.uint8, getattr(torch, "float8_e4m3fnuz", None), getattr(torch, "float8_e4m3fn", None))
    if dt is not None
)
_FP8_CACHE_DTYPES = tuple(
    dt for dt in (torch.uint8, torch.int8, getattr(torch, "float8_e4m3fn", None)) if dt is not None
)


def _cdiv(a: int, b: int) -> int:
    return (a + b - 1) // b


@functools.lru_cache(maxsize=16)
def _cu_count(device_index: int) -> int:
    return torch.cuda.get_device_properties(device_index).multi_processor_count


def _device_cu_count(dev: torch.device) -> int:
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    return _cu_count(idx)


def get_recommended_splits(
    num_sequences: int,
    num_kv_heads: int,
    split_kv_blocks: int = 1,
    *,
    sliding_window: int = 0,
    context_partition_size: int = KV_COMPUTE_BLOCK,
    query_length: int = 1,
) -> int:
    """Recommended ``max_context_partition_num`` (kernels/pa_decode_fp8.py:1922-1949).

    Sliding window: ``cdiv(sliding_window + query_length - 1, partition) + 1``.
    Otherwise ``clamp(cdiv(2*CUs, max(1, seqs*kv_heads*split)) * split, 4, 8)``.
    """
    if sliding_window > 0:
        return _cdiv(sliding_window + query_length - 1, context_partition_size) + 1
    num_sm = _cu_count(torch.cuda.current_device()) * 2
    denom = max(1, num_sequences * num_kv_heads * split_kv_blocks)
    n = _cdiv(num_sm, denom) * split_kv_blocks
    return max(4, min(n, 8))


def _is_current_stream_capturing() -> bool:
    if not torch.cuda.is_available():
        return False
    try:
        return torch.cuda.is_current_stream_capturing()
    except RuntimeError:
        return False


def _prepare_scale_tensor(name: str, scale, *, device: torch.device, is_graph_capturing: bool) -> torch.Tensor:
    """float / tensor -> f32 device tensor (kernels/pa_decode_fp8.py:1871-1895)."""
    if isinstance(scale, torch.Tensor):
        if is_graph_capturing:
            if scale.device != device:
                raise ValueError(f"CUDA graph capture requires `{name}` to already be on {device}, got {scale.device}.")
            if scale.dtype != torch.float32:
                raise ValueError(f"CUDA graph capture requires `{name}` to already be float32, got {scale.dtype}.")
            return scale
        return scale.to(device=device, dtype=torch.float32)
    if is_graph_capturing:
        raise ValueError(
            f"CUDA graph capture requires `{name}` to be passed as a pre-created float32 tensor on the target device."
        )
    return torch.tensor([float(scale or 1.0)], device=device, dtype=torch.float32)


def _get_query_input_dtype(query: torch.Tensor) -> str:
    if query.dtype in _PACKED_FP8_QUERY_DTYPES:
        return "packed_fp8"
    if query.dtype == torch.bfloat16:
        return "bf16"
    if query.dtype == torch.float16:
        return "f16"
    raise ValueError(
        f"Unsupported query dtype for pa_decode_ps_launch: {query.dtype}. Expected packed FP8/uint8, bf16, or f16."
    )


def _get_output_dtype_str(output: torch.Tensor) -> str:
    if output.dtype == torch.bfloat16:
        return "bf16"
    if output.dtype == torch.float16:
        return "f16"
    if output.dtype == torch.float32:
        return "f32"
    raise ValueError(
        f"Unsupported output dtype for pa_decode_ps_launch reduce: {output.dtype}. Expected bf16, f16, or f32."
    )


def _check_int32(name: str, t: torch.Tensor, ndim: int) -> None:
    if t.dtype != torch.int32 or t.dim() != ndim:
        raise ValueError(f"`{name}` must be a {ndim}-D int32 tensor, got {tuple(t.shape)} {t.dtype}")


def _check_cache_layouts(key_cache: torch.Tensor, value_cache: torch.Tensor, head_size: int):
    """(block_size, trans_v) of the caches: K [nb, Hkv, D/16, bs, 16] and V either
    trans_v [nb, Hkv, bs/16, D, 16] or 4-D [nb, Hkv, D, bs] (trans_v = V.ndim == 5,
    kernels/pa_decode_fp8.py:2841), each contiguous within a (block, kv head) tile."""
    if key_cache.dim() != 5:
        raise ValueError(f"key_cache must be [num_blocks, kv_heads, head_dim/16, block_size, 16], got {tuple(key_cache.shape)}")
    if key_cache.element_size() != 1 or value_cache.element_size() != 1:
        raise ValueError("key_cache / value_cache must hold one-byte fp8 e4m3fn values (uint8 / float8_e4m3fn view)")
    nb, hkv, dc, bs, x = key_cache.shape
    if x != 16 or dc * 16 != head_size:
        raise ValueError(f"key_cache inner dims {tuple(key_cache.shape[2:])} do not match head_dim {head_size}")
    if key_cache.stride()[2:] != (bs * 16, 16, 1):
        raise ValueError("key_cache must be contiguous within each (block, kv head) tile")
    trans_v = value_cache.dim() == 5
    if trans_v:
        if tuple(value_cache.shape) != (nb, hkv, bs // 16, head_size, 16):
            raise ValueError(f"value_cache {tuple(value_cache.shape)} is not the trans_v layout of key_cache")
        if value_cache.stride()[2:] != (head_size * 16, 16, 1):
            raise ValueError("value_cache must be contiguous within each (block, kv head) tile")
    else:
        if tuple(value_cache.shape) != (nb, hkv, head_size, bs):
            raise ValueError(f"value_cache {tuple(value_cache.shape)} is not [num_blocks, kv_heads, head_dim, block_size]")
        if value_cache.stride()[2:] != (bs, 1):
            raise ValueError("value_cache must be contiguous within each (block, kv head) tile")
    return bs, trans_v


def _u8(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.uint8 else t.view(torch.uint8)


def _decode_args(
    *,
    query,
    key_cache,
    value_cache,
    block_tables,
    context_lengths,
    key_scale,
    value_scale,
    per_token_kv,
    exp_sums,
    max_logits,
    temporary_output,
    query_length,
    query_group_size,
    max_parts,
    sliding_window,
    softmax_scale,
) -> _lib.DecodeArgs:
    a = _lib.DecodeArgs()
    if exp_sums is not None:
        a.exp_sums = exp_sums.data_ptr()
        a.max_logits = max_logits.data_ptr()
        a.tmp_out = temporary_output.data_ptr()
        a.stride_es_seq, a.stride_es_head, a.stride_es_part = exp_sums.stride(0), exp_sums.stride(1), exp_sums.stride(2)
        a.stride_to_seq, a.stride_to_head = temporary_output.stride(0), temporary_output.stride(1)
        a.stride_to_part, a.stride_to_group = temporary_output.stride(2), temporary_output.stride(3)
    a.query = query.data_ptr()
    a.key_cache = key_cache.data_ptr()
    a.value_cache = value_cache.data_ptr()
    a.block_tables = block_tables.data_ptr()
    a.context_lengths = context_lengths.data_ptr()
    a.key_scale = key_scale.data_ptr()
    a.value_scale = value_scale.data_ptr()
    a.stride_q_seq, a.stride_q_head = query.stride(0), query.stride(1)
    a.stride_k_block, a.stride_k_head = key_cache.stride(0), key_cache.stride(1)
    a.stride_v_block, a.stride_v_head = value_cache.stride(0), value_cache.stride(1)
    a.stride_bt_seq = block_tables.stride(0)
    if per_token_kv:
        a.stride_ks_block, a.stride_ks_head = key_scale.stride(0), key_scale.stride(1)
    a.batch_size = context_lengths.shape[0]
    a.num_kv_heads = key_cache.shape[1]
    a.query_group_size = query_group_size
    a.query_length = query_length
    a.head_dim = query.shape[-1]
    a.block_size = key_cache.shape[-2]
    a.num_blocks = key_cache.shape[0]
    a.max_blocks_per_seq = block_tables.shape[1]
    a.max_context_partition_num = max_parts
    a.sliding_window = sliding_window
    a.per_token_kv = 1 if per_token_kv else 0
    a.query_dtype = _lib.PA_FP8_F16 if query.dtype == torch.float16 else _lib.PA_FP8_BF16
    a.softmax_scale = float(softmax_scale)
    a.value_layout = _lib.PA_FP8_V_TRANS if value_cache.dim() == 5 else _lib.PA_FP8_V_4D
    return a


def _check_intermediates(exp_sums, max_logits, temporary_output, shape, head_size):
    if tuple(exp_sums.shape) != shape or exp_sums.dtype != torch.float32 or exp_sums.stride(3) != 1:
        raise ValueError(f"exp_sums must be float32 {shape} with a unit last stride")
    if tuple(max_logits.shape) != shape or max_logits.dtype != torch.float32 or max_logits.stride(3) != 1:
        raise ValueError(f"max_logits must be float32 {shape} with a unit last stride")
    if exp_sums.stride() != max_logits.stride():
        raise ValueError("exp_sums and max_logits must share strides")
    if (
        tuple(temporary_output.shape) != shape + (head_size,)
        or temporary_output.dtype != torch.bfloat16
        or temporary_output.stride(4) != 1
    ):
        raise ValueError(f"temporary_output must be bfloat16 {shape + (head_size,)} with a unit last stride")


def _validate_scale(name: str, scale: torch.Tensor, per_token: bool, key_cache: torch.Tensor) -> None:
    nb, hkv, _, bs, _ = key_cache.shape
    if per_token:
        if scale.dim() != 4 or tuple(scale.shape) != (nb, hkv, bs, 1) or scale.stride(2) != 1:
            raise ValueError(f"per-token `{name}` must be float32 [num_blocks, kv_heads, block_size, 1], got {tuple(scale.shape)}")
    elif scale.numel() != 1:
        raise ValueError(f"per-tensor `{name}` must hold one value, got {tuple(scale.shape)}")


class _Plan:
    """Prepared launch of one decode step: the C-ABI argument blocks plus the
    tensors they point into that the launcher allocated itself.

    Split-context paths: ``dargs`` (partition kernel) and ``rargs`` (LSE reduce;
    None when the partition kernel writes the output directly).  Persistent
    path: ``wargs`` (worklist kernel) and ``vargs`` (reduce of split works).
    ``cacheable`` is False when the plan holds metadata the launcher derived from
    context-length values, which a later call with the same tensors may change."""

    __slots__ = ("dargs", "rargs", "wargs", "vargs", "tag", "keepalive", "max_parts", "cacheable", "launches")

    def __init__(self, tag, keepalive, max_parts=None, dargs=None, rargs=None, wargs=None, vargs=None, cacheable=True):
        self.dargs, self.rargs, self.wargs, self.vargs = dargs, rargs, wargs, vargs
        self.tag, self.keepalive, self.max_parts, self.cacheable = tag, keepalive, max_parts, cacheable
        self.launches = [
            (fn, a)
            for fn, a in ((_lib.decode_partitions, dargs), (_lib.lse_reduce, rargs), (_lib.decode_worklist, wargs),
                          (_lib.reduce_v1, vargs))
            if a is not None
        ]

    def launch(self, stream_handle: int) -> str:
        for fn, a in self.launches:
            fn(a, stream_handle)
        return self.tag


# Default partition count when the caller passes max_context_partition_num=0,
# together with the waves per workgroup of the one-row-group layout.  Eight waves
# resident per CU (two per SIMD) keep enough K/V loads in flight: either two
# 4-wave workgroups per CU, or -- when the (sequence, kv head) pairs are at most
# one per CU -- one 8-wave workgroup per slot, which needs fewer slots (no
# partials, no reduce at one slot).  Slots hold at most _MAX_SLOT_TOKENS of the
# longest possible sequence, so ragged batches stay balanced.
# (get_recommended_splits keeps the reference formula for callers that ask for it.)
_TARGET_WORKGROUPS_PER_CU = 2
_MAX_SLOT_TOKENS = 8192


def _auto_partitions(dev, batch_size, num_kv_heads, max_tokens, sliding_window, query_length, head_dim=HEAD_DIM):
    return _auto_layout(dev, batch_size, num_kv_heads, max_tokens, sliding_window, query_length, head_dim)[0]


def _auto_layout(dev, batch_size, num_kv_heads, max_tokens, sliding_window, query_length, head_dim=HEAD_DIM):
    """(partition slots, waves per slot) for the launcher's default.  Eight-wave
    slots exist for head_dim 128 only; other head dims size the grid for four."""
    cus = _device_cu_count(dev)
    pairs = max(1, batch_size * num_kv_heads)
    span = min(max_tokens, sliding_window + query_length) if sliding_window > 0 else max_tokens
    tiles = max(1, _cdiv(span, KV_COMPUTE_BLOCK) + (1 if sliding_window > 0 else 0))
    least = _cdiv(span, _MAX_SLOT_TOKENS)
    p8 = max(1, min(max(_cdiv(cus, pairs), least), tiles))
    if pairs * p8 <= cus and head_dim == HEAD_DIM:
        return p8, 8
    fill = _cdiv(cus * _TARGET_WORKGROUPS_PER_CU, pairs)
    return max(1, min(max(fill, least), tiles)), 4


# Resident waves per CU of the register-streaming layout (two per SIMD), and the
# most steps a chain of slots may give one wave (it bounds the longest wave of a
# ragged batch, whose slots the host cannot see).
_WAVES_PER_CU = 8
_CHAIN_MAX_STEPS = 32


def _slot_layout(dev, batch_size, num_kv_heads, max_parts, head_dim=HEAD_DIM, eqgs=1, v4=False,
                 max_slot_tokens=None):
    """(waves per workgroup, slots per wave, merged) of the partition kernel.

    One-row-group layouts take the fewest waves per slot (1, 2, 4 or 8) whose grid
    fills the GPU at eight resident waves per CU: a wave then streams more steps and
    a slot needs no merge of its waves' states.  Measured on c2 at 8 slots per
    sequence, 99.7 / 101.8 / 106.6 / 136.0 us per step at 1 / 2 / 4 / 8 waves; c4 at
    17 slots, 61.3 / 63.2 / 73.8 / 97.2 us.

    When one wave per slot fills the GPU, and workgroups of W <= 8 waves, one per
    (sequence, kv head), fill it too, each wave of such a workgroup runs consecutive
    slots in turn (the chained layout, slots per wave > 0), its loads running on
    across slot boundaries, and the workgroup merges its own partials into the output
    (``merged``: no reduce launch) -- as long as a wave's chain stays within
    _CHAIN_MAX_STEPS steps of the longest possible slot (``max_slot_tokens``).  c2 at
    8 slots: 94.0 us (99.6 with one slot per one-wave workgroup and the reduce); c4 at
    17 slots: 54.3 us (62.2).  Otherwise slots that may be long (ragged batches, whose
    lengths the host cannot see) get one wave per _CHAIN_MAX_STEPS steps, up to 8:
    c3 at 8 slots (up to 64 steps each) 302.1 us with two waves, 308.1 with one."""
    if head_dim != HEAD_DIM or eqgs > 16:
        return 4, 0, False
    target = _WAVES_PER_CU * _device_cu_count(dev)
    pairs = max(1, batch_size * num_kv_heads)
    slots = pairs * max_parts
    choices = (4, 8) if v4 else (1, 2, 4, 8)
    waves = next((c for c in choices if slots * c >= target), choices[-1])
    if v4 or waves > 1 or max_parts == 1:
        return waves, 0, False
    steps = max(1, _cdiv(max_slot_tokens, 64)) if max_slot_tokens else 1
    wg = next((c for c in (1, 2, 4, 8) if pairs * c >= target), None)
    if wg is not None and _cdiv(max_parts, wg) * steps <= _CHAIN_MAX_STEPS:
        return wg, _cdiv(max_parts, wg), True
    return next((c for c in (1, 2, 4, 8) if c * _CHAIN_MAX_STEPS >= steps), 8), 0, False


def _waves_per_slot(dev, batch_size, num_kv_heads, max_parts, head_dim=HEAD_DIM):
    """Waves per workgroup of the one-row-group layout (see _slot_layout)."""
    return _slot_layout(dev, batch_size, num_kv_heads, max_parts, head_dim)[0]


def _max_slot_tokens(max_tokens, max_parts, sliding_window, query_length):
    """Tokens of the longest slot any sequence of at most max_tokens tokens can have."""
    span = min(max_tokens, sliding_window + query_length) if sliding_window > 0 else max_tokens
    tiles = _cdiv(span, KV_COMPUTE_BLOCK) + (1 if sliding_window > 0 else 0)
    return _cdiv(tiles, max_parts) * KV_COMPUTE_BLOCK


_PLAN_CACHE: "OrderedDict[tuple, _Plan]" = OrderedDict()
_PLAN_CACHE_SIZE = 64


def _tkey(t):
    if t is None:
        return None
    if isinstance(t, torch.Tensor):
        return (t.data_ptr(), tuple(t.shape), t.stride(), t.dtype, t.device)
    return ("scalar", float(t or 1.0))


def _partitioned_plan(
    output,
    query,
    key_cache,
    value_cache,
    context_lengths,
    block_tables,
    softmax_scale,
    key_scale,
    value_scale,
    per_token_kv,
    sliding_window,
    max_parts,
    exp_sums,
    max_logits,
    temporary_output,
    is_graph_capturing,
    path_name,
    tag,
) -> _Plan:
    dev = query.device
    batch_size = context_lengths.shape[0]
    num_query_heads = query.shape[1]
    num_kv_heads = key_cache.shape[1]
    head_size = query.shape[-1]
    query_group_size = num_query_heads // num_kv_heads
    query_length = query.shape[0] // batch_size
    eqgs = query_length * query_group_size
    shape = (batch_size, num_kv_heads, max_parts, eqgs)
    if is_graph_capturing and (exp_sums is None or max_logits is None or temporary_output is None):
        raise ValueError(
            "CUDA graph capture requires preallocated `exp_sums`, `max_logits`, "
            f"and `temporary_output` for the {path_name} path."
        )
    output_5d = output.view(batch_size, query_length, num_kv_heads, query_group_size, head_size)
    max_tokens = block_tables.shape[1] * key_cache.shape[-2]
    waves, spw, merged = _slot_layout(dev, batch_size, num_kv_heads, max_parts, head_size, eqgs,
                                      value_cache.dim() != 5,
                                      _max_slot_tokens(max_tokens, max_parts, sliding_window, query_length))
    given_es, given_ml, given_to = exp_sums is not None, max_logits is not None, temporary_output is not None
    if merged and not (given_es or given_ml or given_to):
        # Workgroups would hold every slot of their (sequence, kv head) and merge
        # partials nobody reads: one slot per sequence on the same workgroups gives the
        # output (to rounding: no bf16 slot rows in between) without the slot
        # boundaries and the merge.  c2 at the harness's 8 slots: 84 us against 92.
        max_parts = 1
        waves, spw, merged = _slot_layout(dev, batch_size, num_kv_heads, 1, head_size, eqgs, value_cache.dim() != 5)
        shape = (batch_size, num_kv_heads, 1, eqgs)
    # One slot per sequence: the kernel writes the output itself.  On the small-block
    # path the reference fills caller-passed partials even at one slot (its reduce
    # then reads them), so those calls keep the partials; its fused sliding-window
    # kernel writes the output directly (kernels/pa_decode_fp8.py:2923, :2977-2979).
    direct = max_parts == 1 and (sliding_window > 0 or not (given_es or given_ml or given_to))
    if direct:
        # one slot per sequence: the partition kernel writes the output itself
        exp_sums = max_logits = temporary_output = None
    else:
        # every slot (including empty ones) is written by the kernel, so no fill is needed
        if exp_sums is None:
            exp_sums = torch.empty(shape, device=dev, dtype=torch.float32)
        if max_logits is None:
            max_logits = torch.empty(shape, device=dev, dtype=torch.float32)
        if temporary_output is None:
            temporary_output = torch.empty(shape + (head_size,), device=dev, dtype=torch.bfloat16)
        _check_intermediates(exp_sums, max_logits, temporary_output, shape, head_size)
    own = tuple(t for t, given in ((exp_sums, given_es), (max_logits, given_ml), (temporary_output, given_to))
                if t is not None and not given)
    dargs = _decode_args(
        query=query,
        key_cache=_u8(key_cache),
        value_cache=_u8(value_cache),
        block_tables=block_tables,
        context_lengths=context_lengths,
        key_scale=key_scale,
        value_scale=value_scale,
        per_token_kv=per_token_kv,
        exp_sums=exp_sums,
        max_logits=max_logits,
        temporary_output=temporary_output,
        query_length=query_length,
        query_group_size=query_group_size,
        max_parts=max_parts,
        sliding_window=sliding_window,
        softmax_scale=softmax_scale,
    )
    out_dtype = _get_output_dtype_str(output)
    dargs.waves_per_slot, dargs.slots_per_wave = waves, spw
    if direct or merged:
        # the kernel writes the output: one slot per sequence, or workgroups that hold
        # every slot of their (sequence, kv head) and merge the partials they wrote
        dargs.direct_output = 1
        dargs.out_dtype = {"bf16": _lib.PA_FP8_BF16, "f16": _lib.PA_FP8_F16, "f32": _lib.PA_FP8_F32}[out_dtype]
        dargs.output = output_5d.data_ptr()
        dargs.stride_o_seq, dargs.stride_o_len, dargs.stride_o_head, dargs.stride_o_group = (
            output_5d.stride(i) for i in range(4)
        )
        rargs = None
    else:
        rargs = _reduce_args(output_5d, exp_sums, max_logits, temporary_output, max_parts, out_dtype)
    return _Plan(tag, own, max_parts, dargs=dargs, rargs=rargs)


_METADATA_KEYS = ("work_indptr", "work_info_flat", "partition_indptr", "reduce_indptr", "reduce_final_map",
                  "reduce_partial_map", "partial_output", "partial_lse")
_SCHEDULE_KEYS = ("work_indptr", "work_info_flat", "reduce_indptr", "reduce_final_map", "reduce_partial_map",
                  "partial_output", "partial_lse", "num_sm")


def _worklist_plan(
    output,
    query,
    key_cache,
    value_cache,
    context_lengths,
    kv_page_indices,
    kv_indptr,
    metadata,
    softmax_scale,
    key_scale,
    value_scale,
    per_token_kv,
    is_graph_capturing,
) -> _Plan:
    """Persistent path (kernels/pa_decode_fp8.py:3123-3202): the worklist decode
    over ``metadata`` and the merge of the split works' partials."""
    dev = query.device
    batch_size = context_lengths.shape[0]
    num_query_heads = query.shape[1]
    num_kv_heads = key_cache.shape[1]
    head_size = query.shape[-1]
    query_length = query.shape[0] // batch_size
    block_size = key_cache.shape[-2]
    if kv_page_indices is None or kv_indptr is None:
        raise ValueError(
            f"pa_decode_ps_launch: block_size={block_size} runs the persistent worklist path, which reads pages "
            "through `kv_page_indices` and `kv_indptr`."
        )
    _check_int32("kv_page_indices", kv_page_indices, 1)
    _check_int32("kv_indptr", kv_indptr, 1)
    if kv_indptr.shape[0] != batch_size + 1 or not kv_indptr.is_contiguous() or not kv_page_indices.is_contiguous():
        raise ValueError(f"kv_indptr must be a contiguous [{batch_size + 1}] tensor and kv_page_indices contiguous")
    own = None  # metadata the launcher built itself (kept alive by the plan, which is not cached)
    if metadata is None:
        if is_graph_capturing:
            raise ValueError(
                "CUDA graph capture requires precomputed `metadata`; "
                "call `get_pa_metadata()` before capture and pass it via `metadata=`."
            )
        metadata = own = get_pa_metadata(query, key_cache, context_lengths, kv_indptr, num_query_heads, num_kv_heads)
    missing = [k for k in _METADATA_KEYS + ("num_sm",) if k not in metadata]
    if missing:
        raise ValueError(f"metadata is missing {missing}; build it with get_pa_metadata()")
    # get_pa_metadata's own schedule for this kernel when present, else the reference's
    sched = metadata.get("tuned") or metadata
    missing = [k for k in _SCHEDULE_KEYS if k not in sched]
    if missing:
        raise ValueError(f"metadata['tuned'] is missing {missing}; build it with get_pa_metadata()")
    num_sm = int(sched["num_sm"])
    work_indptr, work_info = sched["work_indptr"], sched["work_info_flat"]
    partition_indptr = metadata["partition_indptr"]
    po, pl = sched["partial_output"], sched["partial_lse"]
    for name, t in [(k, sched[k]) for k in ("work_indptr", "work_info_flat", "reduce_indptr", "reduce_final_map",
                                          "reduce_partial_map")] + [("partition_indptr", partition_indptr)]:
        if t.dtype != torch.int32 or not t.is_contiguous() or t.device != dev:
            raise ValueError(f"metadata[{name!r}] must be a contiguous int32 tensor on {dev}")
    if work_indptr.numel() != num_sm + 1 or work_info.numel() % 8 != 0:
        raise ValueError(f"metadata work_indptr has {work_indptr.numel()} entries for num_sm={num_sm}")
    if partition_indptr.numel() != batch_size + 1:
        raise ValueError(f"metadata partition_indptr must have {batch_size + 1} entries")
    if (po.dim() != 4 or po.dtype != torch.float32 or tuple(po.shape[1:]) != (1, num_query_heads, head_size)
            or po.stride()[1:] != (num_query_heads * head_size, head_size, 1) or po.shape[0] < query_length):
        raise ValueError(f"metadata partial_output must be float32 [rows, 1, {num_query_heads}, {head_size}], rows >= ql")
    if pl.dim() != 4 or pl.dtype != torch.float32 or tuple(pl.shape) != (po.shape[0], 1, num_query_heads, 1):
        raise ValueError(f"metadata partial_lse must be float32 [{po.shape[0]}, 1, {num_query_heads}, 1]")
    out_dtype = _get_output_dtype_str(output)

    w = _lib.WorklistArgs()
    w.output = output.data_ptr()
    w.partial_output = po.data_ptr()
    w.partial_lse = pl.data_ptr()
    w.query = query.data_ptr()
    w.key_cache = key_cache.data_ptr()
    w.value_cache = value_cache.data_ptr()
    w.context_lengths = context_lengths.data_ptr()
    w.key_scale = key_scale.data_ptr()
    w.value_scale = value_scale.data_ptr()
    w.work_indptr = work_indptr.data_ptr()
    w.work_info = work_info.data_ptr()
    w.kv_page_indices = kv_page_indices.data_ptr()
    w.kv_indptr = kv_indptr.data_ptr()
    w.partition_indptr = partition_indptr.data_ptr()
    w.bin_groups = int(sched.get("bin_groups", 0))  # the schedule's quota groups, by dispatch round
    w.stride_q_seq, w.stride_q_head = query.stride(0), query.stride(1)
    w.stride_k_block, w.stride_k_head = key_cache.stride(0), key_cache.stride(1)
    w.stride_v_block, w.stride_v_head = value_cache.stride(0), value_cache.stride(1)
    w.stride_out_seq, w.stride_out_head = output.stride(0), output.stride(1)
    w.stride_po_row, w.stride_pl_row = po.stride(0), pl.stride(0)
    if per_token_kv:
        w.stride_ks_block, w.stride_ks_head = key_scale.stride(0), key_scale.stride(1)
    w.batch_size = batch_size
    w.num_kv_heads = num_kv_heads
    w.query_group_size = num_query_heads // num_kv_heads
    w.query_length = query_length
    w.head_dim = head_size
    w.block_size = block_size
    w.num_blocks = key_cache.shape[0]
    w.num_pages = kv_page_indices.shape[0]
    w.num_cu = num_sm
    w.max_work = work_info.numel() // 8
    w.partial_rows = po.shape[0]
    w.output_rows = output.shape[0]
    w.per_token_kv = 1 if per_token_kv else 0
    w.query_dtype = _lib.PA_FP8_F16 if query.dtype == torch.float16 else _lib.PA_FP8_BF16
    w.out_dtype = {"bf16": _lib.PA_FP8_BF16, "f16": _lib.PA_FP8_F16, "f32": _lib.PA_FP8_F32}[out_dtype]
    w.softmax_scale = float(softmax_scale)
    w.value_layout = _lib.PA_FP8_V_TRANS if value_cache.dim() == 5 else _lib.PA_FP8_V_4D
    # no partial rows past the first query_length: nothing was split, so there is nothing to merge
    v = None
    if po.shape[0] > query_length:
        v = _reduce_v1_args(po[query_length:], pl[query_length:], sched["reduce_indptr"],
                            sched["reduce_final_map"], sched["reduce_partial_map"], query_length, output)
    # A cached plan holds pointers only: every caller tensor it reads is part of the
    # cache key (pointer, shape, strides), so a later call hits the plan only with
    # tensors at the same addresses; it keeps nothing of the caller alive.
    return _Plan("ps_split_reduce", (own,), wargs=w, vargs=v, cacheable=own is None)


def _mkey(metadata):
    if metadata is None:
        return None

    def one(d):
        return tuple((k, _tkey(d[k])) for k in _METADATA_KEYS if k in d) + (
            ("num_sm", d.get("num_sm")), ("bin_groups", d.get("bin_groups")))

    t = metadata.get("tuned")
    return one(metadata) + (("uniform_context", bool(metadata.get("uniform_context", False))),
                            ("tuned", one(t) if t else None))


def pa_decode_ps_launch(
    output: torch.Tensor,
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    context_lengths: torch.Tensor,
    kv_page_indices: torch.Tensor,
    kv_indptr: torch.Tensor,
    softmax_scale: float,
    key_scale: torch.Tensor = None,
    value_scale: torch.Tensor = None,
    *,
    sliding_window: int = 0,
    metadata: dict = None,
    block_tables: torch.Tensor = None,
    max_context_partition_num: int = 0,
    exp_sums: torch.Tensor = None,
    max_logits: torch.Tensor = None,
    temporary_output: torch.Tensor = None,
    stream=None,
) -> str:
    """Paged-attention decode over an fp8 e4m3fn KV cache (kernels/pa_decode_fp8.py:2812-3202).

    Routing follows the reference:

    * ``sliding_window > 0``: sliding-window split-context path (partition
      kernel + log-sum-exp reduce; every block size), reading ``block_tables``;
    * block sizes 16 / 64: small-block path.  Given ``metadata`` (from
      ``get_pa_metadata``) of a ragged batch and ``kv_page_indices`` /
      ``kv_indptr`` it runs the worklist kernel over that schedule, which
      balances the batch; otherwise the split-context partition kernel reading
      ``block_tables``;
    * other block sizes: the persistent path -- the worklist kernel over
      ``metadata`` (computed with ``get_pa_metadata`` when absent, which
      synchronises once) reading pages through ``kv_page_indices`` /
      ``kv_indptr``, then the merge of the split works' partials.

    ``output`` is written in place.  A call whose tensors (pointers, shapes,
    strides, dtypes), metadata tensors, scalars and stream all match an earlier
    call reuses that call's prepared argument blocks (and the intermediates it
    allocated), so steady-state decode pays two C calls.  Plans built on
    metadata the launcher computed itself are not reused, because that metadata
    depends on the context-length values.

    Returns the path tag: "ps_sw_partitioned" / "ps_sw_fused_partitioned",
    "ps_small_block" or "ps_split_reduce".
    """
    dev = query.device
    s = stream if stream is not None else torch.cuda.current_stream(dev)
    stream_handle = s.cuda_stream if hasattr(s, "cuda_stream") else int(s)
    is_graph_capturing = _is_current_stream_capturing()
    key = None
    if not is_graph_capturing:
        key = (
            stream_handle,
            _tkey(output),
            _tkey(query),
            _tkey(key_cache),
            _tkey(value_cache),
            _tkey(context_lengths),
            _tkey(block_tables),
            _tkey(key_scale),
            _tkey(value_scale),
            float(softmax_scale),
            int(sliding_window),
            int(max_context_partition_num),
            _tkey(exp_sums),
            _tkey(max_logits),
            _tkey(temporary_output),
            _tkey(kv_page_indices),
            _tkey(kv_indptr),
            _mkey(metadata),
        )
        plan = _PLAN_CACHE.get(key)
        if plan is not None:
            _PLAN_CACHE.move_to_end(key)
            return plan.launch(stream_handle)
    plan = _build_plan(
        output, query, key_cache, value_cache, context_lengths, softmax_scale, key_scale, value_scale,
        sliding_window, block_tables, max_context_partition_num, exp_sums, max_logits, temporary_output,
        is_graph_capturing, kv_page_indices=kv_page_indices, kv_indptr=kv_indptr, metadata=metadata,
    )
    if key is not None and plan.cacheable:
        _PLAN_CACHE[key] = plan
        if len(_PLAN_CACHE) > _PLAN_CACHE_SIZE:
            _PLAN_CACHE.popitem(last=False)
    return plan.launch(stream_handle)


def _build_plan(
    output, query, key_cache, value_cache, context_lengths, softmax_scale, key_scale, value_scale,
    sliding_window, block_tables, max_context_partition_num, exp_sums, max_logits, temporary_output,
    is_graph_capturing, kv_page_indices=None, kv_indptr=None, metadata=None,
) -> _Plan:
    if query.dim() != 3:
        raise ValueError(f"query must be [num_seqs*query_length, num_heads, head_dim], got {tuple(query.shape)}")
    num_query_heads = query.shape[1]
    num_kv_heads = key_cache.shape[1]
    query_input_dtype = _get_query_input_dtype(query)
    dev = query.device
    given_scales = (key_scale, value_scale)
    key_scale = _prepare_scale_tensor("key_scale", key_scale, device=dev, is_graph_capturing=is_graph_capturing)
    value_scale = _prepare_scale_tensor("value_scale", value_scale, device=dev, is_graph_capturing=is_graph_capturing)
    # Scales the launcher made itself: a float becomes a new tensor of that value
    # (the cache key holds the value), a tensor of another device or dtype a
    # converted copy, which must not be reused once the caller's tensor changes.
    made = tuple(s for s, g in zip((key_scale, value_scale), given_scales) if s is not g)
    copied = any(isinstance(g, torch.Tensor) and s is not g for s, g in zip((key_scale, value_scale), given_scales))
    plan = _build_plan_checked(
        output, query, key_cache, value_cache, context_lengths, softmax_scale, key_scale, value_scale,
        sliding_window, block_tables, max_context_partition_num, exp_sums, max_logits, temporary_output,
        is_graph_capturing, query_input_dtype, kv_page_indices, kv_indptr, metadata,
    )
    if made:
        plan.keepalive = tuple(plan.keepalive) + made
    if copied:
        plan.cacheable = False
    return plan


def _build_plan_checked(
    output, query, key_cache, value_cache, context_lengths, softmax_scale, key_scale, value_scale,
    sliding_window, block_tables, max_context_partition_num, exp_sums, max_logits, temporary_output,
    is_graph_capturing, query_input_dtype, kv_page_indices, kv_indptr, metadata,
) -> _Plan:
    num_query_heads = query.shape[1]
    num_kv_heads = key_cache.shape[1]
    dev = query.device
    if query_input_dtype == "packed_fp8":
        raise ValueError(
            "`pa_decode_ps_launch` no longer accepts host query_scale and only supports "
            "bf16/f16 query inputs with kernel-internal query scale computation."
        )
    head_size = query.shape[-1]
    if head_size not in HEAD_DIMS:
        raise ValueError(f"Unsupported head_dim={head_size}; this build supports {', '.join(map(str, HEAD_DIMS))}.")
    if num_query_heads % num_kv_heads != 0:
        raise ValueError("Query heads must be divisible by KV heads")
    _check_int32("context_lengths", context_lengths, 1)
    batch_size = context_lengths.shape[0]
    if batch_size == 0 or query.shape[0] % batch_size != 0:
        raise ValueError(f"query rows {query.shape[0]} are not a multiple of batch size {batch_size}")
    if tuple(output.shape) != tuple(query.shape):
        raise ValueError(f"output shape {tuple(output.shape)} must equal query shape {tuple(query.shape)}")
    _get_output_dtype_str(output)
    if query.stride(2) != 1 or not output.is_contiguous():
        raise ValueError("query needs a unit last stride and output must be contiguous")
    block_size, trans_v = _check_cache_layouts(key_cache, value_cache, head_size)
    if block_size < 16 or block_size & (block_size - 1):
        raise ValueError(f"pa_decode_ps_launch: unsupported block_size={block_size}; expected a power of two >= 16.")
    per_token_kv = key_scale.ndim > 1
    _validate_scale("key_scale", key_scale, per_token_kv, key_cache)
    _validate_scale("value_scale", value_scale, value_scale.ndim > 1, key_cache)
    if (value_scale.ndim > 1) != per_token_kv:
        raise ValueError("key_scale and value_scale must both be per-tensor or both per-token")
    query_length = query.shape[0] // batch_size
    query_group_size = num_query_heads // num_kv_heads
    if query_length * query_group_size > _MAX_QUERY_ROWS:
        raise ValueError(f"query_length * (num_query_heads // num_kv_heads) must be <= {_MAX_QUERY_ROWS}")
    for name, t in (("query", query), ("key_cache", key_cache), ("value_cache", value_cache), ("output", output),
                    ("context_lengths", context_lengths), ("key_scale", key_scale), ("value_scale", value_scale)):
        if t.device != dev:
            raise ValueError(f"`{name}` is on {t.device}, expected {dev}")
    small = block_size in _PA_DECODE_PS_SMALL_BLOCK_SIZES
    # Block sizes other than 16 / 64 take the persistent path, as in the reference.
    # The small-block path also runs the worklist kernel when the caller hands
    # in get_pa_metadata's schedule with the flat page list and no split-context
    # partials, and the batch is ragged or the caller asks for several slots: the
    # schedule balances ragged batches across CUs, which fixed partition slots
    # cannot, and on an equal-length batch it holds whole sequences, as one slot
    # does.  Equal-length batches keep the partition kernel at one slot or the
    # automatic count, and at a larger count when workgroups of one (sequence, kv
    # head) each fill the GPU (the partition route then runs one slot per sequence,
    # see _partitioned_plan): it skips the worklist reads (c2 at the harness's 8
    # slots: 84.0 us against 85.7 on the worklist).  The tag stays "ps_small_block".
    # A caller that passes
    # exp_sums / max_logits / temporary_output gets them filled in the reference's
    # partition-slot format, as the reference's small-block route (which ignores
    # metadata) fills them: that call runs the partition kernel at the caller's
    # partition count (kernels/pa_decode_fp8.py:3010-3121).
    caller_partials = exp_sums is not None or max_logits is not None or temporary_output is not None
    uniform = metadata is not None and bool(metadata.get("uniform_context", False))
    one_slot = max_context_partition_num <= 1
    if uniform and not one_slot and not caller_partials and block_tables is not None and block_tables.dim() == 2:
        one_slot = _slot_layout(dev, batch_size, num_kv_heads, max_context_partition_num, head_size,
                                query_length * query_group_size, not trans_v,
                                _max_slot_tokens(block_tables.shape[1] * block_size, max_context_partition_num,
                                                 sliding_window, query_length))[2]
    balanced_worklist = (metadata is not None and kv_page_indices is not None and kv_indptr is not None
                         and not caller_partials and not (uniform and one_slot))
    if small and sliding_window <= 0 and not trans_v:
        # the reference's small-block kernel reads trans_v only (kernels/pa_decode_fp8.py:2082-2083)
        raise NotImplementedError("compile_pa_decode_ps: trans_v=False not yet supported.")
    if sliding_window <= 0 and (not small or balanced_worklist):
        if small:
            # The reference requires preallocated partials under capture on this path
            # because its kernel writes them (kernels/pa_decode_fp8.py:3030-3034); the
            # worklist route writes none and allocates nothing, so it is capturable
            # without them (the partition route below keeps the reference's rule).
            plan = _worklist_plan(output, query, key_cache, value_cache, context_lengths, kv_page_indices, kv_indptr,
                                  metadata, softmax_scale, key_scale, value_scale, per_token_kv, is_graph_capturing)
            plan.tag = "ps_small_block"
            return plan
        return _worklist_plan(output, query, key_cache, value_cache, context_lengths, kv_page_indices, kv_indptr,
                              metadata, softmax_scale, key_scale, value_scale, per_token_kv, is_graph_capturing)
    if block_tables is None:
        raise ValueError(
            f"pa_decode_ps_launch: block_size={block_size} requires `block_tables` "
            "(per-sequence physical block index table)."
        )
    _check_int32("block_tables", block_tables, 2)
    if block_tables.shape[0] != batch_size or block_tables.stride(1) != 1 or block_tables.device != dev:
        raise ValueError("block_tables must be [num_seqs, max_blocks] on the query device with a unit last stride")

    if max_context_partition_num == 0:
        if exp_sums is not None:
            # the caller sized the partials: the reference sizes them with
            # get_recommended_splits and launches that many slots (:2890-2896, :3024-3029)
            max_context_partition_num = exp_sums.shape[2] if exp_sums.dim() == 4 else 0
        else:
            max_context_partition_num = _auto_partitions(
                dev, batch_size, num_kv_heads, block_tables.shape[1] * block_size, sliding_window, query_length,
                head_size,
            )
    if max_context_partition_num < 1 or max_context_partition_num > 65535:
        raise ValueError(f"max_context_partition_num={max_context_partition_num} out of range [1, 65535]")
    if sliding_window > 0:
        tag = "ps_sw_fused_partitioned" if max_context_partition_num <= 1 else "ps_sw_partitioned"
        path = "sliding-window"
    else:
        tag, path = "ps_small_block", "small-block PS"
    return _partitioned_plan(output, query, key_cache, value_cache, context_lengths, block_tables, softmax_scale,
                             key_scale, value_scale, per_token_kv, sliding_window, max_context_partition_num,
                             exp_sums, max_logits, temporary_output, is_graph_capturing, path, tag)


def _schedule_layout(batch_size: int, num_kv_heads: int, num_sm: int) -> list:
    """int32 element counts of one schedule's buffers: work_indptr, work_info (flat),
    reduce_indptr, reduce_final_map (flat), reduce_partial_map."""
    infos = get_pa_metadata_info_v1(batch_size, num_kv_heads, num_cu=num_sm)
    return [int(torch.Size(shape).numel()) for shape, _ in infos[1:]]


@functools.lru_cache(maxsize=64)
def _metadata_layout(batch_size, num_kv_heads, gqa, query_length, head_size, cus, partition_size, tuned):
    """What get_pa_metadata's launches share for one shape: the schedules (num_sm,
    bin groups), the int32 element counts and 16-byte aligned offsets of the pieces
    of its one allocation, and the scheduler argument blocks with every field but the
    pointers filled (as bytes, copied per call)."""
    num_sm = (cus * _REFERENCE_BINS_PER_CU // num_kv_heads) * num_kv_heads  # kernels/pa_decode_fp8.py:1769-1771
    if num_sm <= 0 or partition_size <= 0 or partition_size & (partition_size - 1):
        raise ValueError(
            f"get_pa_metadata needs num_kv_heads <= {_REFERENCE_BINS_PER_CU} * CUs and a power-of-two partition_size"
        )
    schedules = [(num_sm, 0)]
    if tuned:
        bins_per_cu = _metadata_bins_per_cu(query_length, gqa, head_size)
        t_sm = (cus * bins_per_cu // num_kv_heads) * num_kv_heads
        # quotas weighted by dispatch round, when every round holds whole groups of bins
        # and the parallel scheduler runs (the serial one, past 4096 batches, splits evenly)
        t_groups = bins_per_cu if (t_sm == cus * bins_per_cu and t_sm % (bins_per_cu * num_kv_heads) == 0
                                   and batch_size <= 4096 and bins_per_cu in _BIN_WEIGHTS) else 0
        if t_sm > 0:
            schedules.append((t_sm, t_groups))
    # Every int32 output in one allocation: four counters first (the reference
    # schedule's split partials, uniform_context, the tuned schedule's split
    # partials), so one three-int read returns what the host needs; then each
    # schedule's buffers and partition_indptr, in 16-byte aligned pieces.
    sizes = [4]
    for s_sm, _ in schedules:
        sizes += _schedule_layout(batch_size, num_kv_heads, s_sm)
    sizes.append(batch_size + 1)  # partition_indptr
    offs = [0]
    for n in sizes:
        offs.append(offs[-1] + (n + 3) // 4 * 4)
    args = (_lib.MetadataArgs * len(schedules))()
    for k, (s_sm, s_groups) in enumerate(schedules):
        a = args[k]
        a.seqlens_qo_indptr = None  # the scheduler's b * query_length: no offsets tensor to build
        a.num_batches = batch_size
        a.gqa = gqa
        a.num_heads_k = num_kv_heads
        a.num_cu = s_sm
        a.kv_granularity = partition_size
        a.query_length = query_length
        a.max_work = sizes[2 + 5 * k] // 8
        a.max_split_tiles = sizes[5 + 5 * k]
        a.bin_groups = s_groups
        for g, wgt in enumerate(_BIN_WEIGHTS.get(s_groups, ())):
            a.bin_weight[g] = wgt
    if len(schedules) > 1:
        args[1].pack = 1  # this build's packing schedule where it applies (the reference's stays sequential)
    return tuple(schedules), tuple(sizes), tuple(offs), bytes(args)


def get_pa_metadata(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    context_lengths: torch.Tensor,
    kv_indptr: torch.Tensor,
    num_query_heads: int,
    num_kv_heads: int,
    partition_size: int = KV_COMPUTE_BLOCK,
    *,
    graph_safe: bool = None,
    tuned: bool = True,
):
    """Worklist metadata for the persistent decode (kernels/pa_decode_fp8.py:1729-1859).

    The keys the reference returns hold the reference's schedule, byte for byte:
    ``get_pa_metadata_v1`` over ``num_sm = (CUs * 3 // kv_heads) * kv_heads`` bins
    with even quotas (:1764-1771), ``partition_indptr`` and the partial buffers
    sized for its split partials.  work_info kv ranges are cumulative
    ``partition_size``-token partition indices.

    With ``tuned`` (the default) the dict also holds ``"tuned"``: this build's
    schedule for its worklist kernel, which ``pa_decode_ps_launch`` runs when
    present -- one bin per resident workgroup (2 per CU for the register-streaming
    kernel, 3 for the LDS-staged one that query_length * num_query_heads /
    num_kv_heads > 32 selects) with quotas weighted by dispatch round
    (``bin_groups``, ``bin_weight``), and its own partial buffers.  Both schedules
    come from one scheduler launch.

    By default it synchronises once to size the partial buffers, as the reference
    does on ``reduce_indptr[-1]`` (:1832).  With ``graph_safe`` (the default while
    the current stream is being captured into a graph) it reads nothing back: the
    partial buffers are sized for the scheduler's bound on split partials
    (``reduce_partial_map``'s length, kernels/pa_metadata.py:66-72), and
    ``uniform_context`` is False.  Everything it launches is then capturable, so a
    graph can hold the schedule and the decode together and be replayed over new
    context lengths.  The reference's ``get_pa_metadata`` cannot be captured.
    """
    if graph_safe is None:
        graph_safe = _is_current_stream_capturing()
    dev = query.device
    batch_size = context_lengths.shape[0]
    query_length = query.shape[0] // batch_size
    head_size = query.shape[-1]
    gqa = num_query_heads // num_kv_heads
    schedules, sizes, offs, template = _metadata_layout(
        batch_size, num_kv_heads, gqa, query_length, head_size, _device_cu_count(dev), partition_size, bool(tuned))
    tuned = len(schedules) > 1
    ctx = context_lengths if context_lengths.dtype == torch.int32 else context_lengths.to(torch.int32)
    ctx = ctx.contiguous()
    buf = torch.empty(offs[-1], dtype=torch.int32, device=dev)
    # The launch goes out first: its pointers are the pieces' offsets into the one
    # allocation, and the pieces' tensors are made while the scheduler runs.
    base = buf.data_ptr()
    args = (_lib.MetadataArgs * len(schedules)).from_buffer_copy(template)
    ctx_ptr = ctx.data_ptr()
    for k in range(len(schedules)):
        a, o = args[k], offs[1 + 5 * k: 6 + 5 * k]
        a.context_lens = ctx_ptr
        a.work_indptr = base + 4 * o[0]
        a.work_info = base + 4 * o[1]
        a.reduce_indptr = base + 4 * o[2]
        a.reduce_final_map = base + 4 * o[3]
        a.reduce_partial_map = base + 4 * o[4]
        a.partial_count = base + 4 * (2 * k)  # counts[2k]
    # the first schedule also writes the derived per-batch values
    args[0].partition_indptr = base + 4 * offs[-2]
    args[0].uniform_context = base + 4  # counts[1]
    _lib.metadata_multi(args, torch.cuda.current_stream(dev).cuda_stream)
    piece = [buf[offs[k]: offs[k] + sizes[k]] for k in range(len(sizes))]
    counts, partition_indptr = piece[0], piece[-1]
    sched_bufs = [piece[1 + 5 * k: 6 + 5 * k] for k in range(len(schedules))]

    # the dicts are built while the scheduler runs; only the partial buffers wait for
    # the host read below
    def entry(k):
        wi, winfo, ri, rfm, rpm = sched_bufs[k]
        return {
            "work_indptr": wi,
            "work_info_flat": winfo,
            "reduce_indptr": ri,
            "reduce_final_map": rfm.view(batch_size, 2),
            "reduce_partial_map": rpm,
            "num_sm": schedules[k][0],
        }

    entries = [entry(k) for k in range(len(schedules))]
    md = entries[0]
    md.update({
        "partition_indptr": partition_indptr,
        "stride_po_partial": query_length * num_query_heads * head_size,
        "stride_pl_partial": query_length * num_query_heads,
        "stride_po_ql": num_query_heads * head_size,
        "stride_pl_ql": num_query_heads,
        "query_length": query_length,
    })
    if tuned:
        t = entries[1]
        t["bin_groups"] = schedules[1][1]
        t["bin_weight"] = _BIN_WEIGHTS.get(schedules[1][1])
        md["tuned"] = t
    if graph_safe:
        # no host read: room for every partial a schedule can emit
        nparts = [int(b[4].numel()) for b in sched_bufs]
        uniform = False
    else:
        # one host read (the reference reads reduce_indptr[-1] here too): the split
        # partial counts and whether every sequence has the same context length
        host = counts[:3].cpu().tolist()
        nparts = [host[0], host[2]][: len(schedules)]
        uniform = bool(host[1])
    for e, n in zip(entries, nparts):
        rows = (n + 1) * query_length
        e["partial_output"] = torch.empty((rows, 1, num_query_heads, head_size), dtype=torch.float32, device=dev)
        e["partial_lse"] = torch.empty((rows, 1, num_query_heads, 1), dtype=torch.float32, device=dev)
    # equal context lengths: at one slot or the automatic count the small-block path
    # keeps its partition kernel (one balanced slot per sequence) instead of the worklist
    md["uniform_context"] = uniform
    return md


def softmax_scale_for(head_dim: int = HEAD_DIM) -> float:
    return 1.0 / math.sqrt(head_dim)
