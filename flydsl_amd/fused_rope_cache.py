"""Fused NeoX RoPE + paged KV-cache writer (kernels/fused_rope_cache_kernel.py).

``build_fused_rope_cache_module`` has the reference's build signature
(kernels/fused_rope_cache_kernel.py:52-63) and returns a launcher with the
reference's call signature (:477-493):

    launch(Q, K, V, Positions, CosCache, SinCache, SlotMapping,
           KeyCache, ValueCache, Q_out, K_out, num_tokens, KScale, VScale, stream=None)

One launch of the gfx950 kernel ``pa_fp8_rope_cache`` (libpa_fp8.so) writes
``Q_out = rope(Q)``, ``K_out = rope(K)`` and, for every token whose slot is
non-negative, ``rope(K)`` and ``V`` into the paged cache.

Layouts (chosen by ``flash_layout`` and, for the non-flash layout, by the
value cache's rank, the same rule ``pa_decode_ps_launch`` uses):

* ``flash_layout=True``:  K, V ``[num_blocks, block_size, KH, D]``
* ``flash_layout=False``: K ``[num_blocks, KH, D/16, block_size, 16]`` and
  V ``[num_blocks, KH, D, block_size]`` (4-D) or
  V ``[num_blocks, KH, block_size/16, D, 16]`` (5-D, trans_v -- the layout the
  decode kernels read; not offered by the reference writer).

Cache formats:

* ``apply_scale=False``: the cache has the element dtype and receives the
  rotated K / V unchanged;
* ``apply_scale=True`` with ``[1]`` float32 scales: fp8 e4m3fn codes of
  ``x * (1 / scale)`` (reference :270-296);
* ``apply_scale=True`` with ``[num_blocks, KH, block_size, 1]`` float32 scales
  (per-token, the decode kernels' per-token format): the writer computes
  ``scale = amax / 448`` over each (token, kv head) vector (0 -> 1), stores it
  in the scale tensor at the token's slot and writes the codes of
  ``x / scale`` (the quantiser of tests/kernels/test_pa.py:334-376).

Head dims: those the reference admits (its vector-width rule, and a multiple
of 16 without the flash layout), up to 1024.  Multiples of 16 run one kernel
over 16-byte vectors; other (flash-layout) head dims a kernel that reads and
writes element by element, with the same arithmetic.

Differences from the reference, each an error where the reference would
silently misbehave: Positions / SlotMapping
must have the dtype ``pos_dtype`` names; every tensor is checked for shape,
dtype, device and alignment before the launch.  Positions outside
``[0, CosCache.shape[0])`` are clamped into it and slots past the cache are
skipped, so no input can make the kernel access memory outside its tensors.
"""

from __future__ import annotations

from collections import OrderedDict

import torch

from . import _lib

_X = 16  # x-pack factor of the non-flash key cache (kernels/fused_rope_cache_kernel.py:84)
_ELEM = {"bf16": (torch.bfloat16, _lib.PA_FP8_BF16), "f16": (torch.float16, _lib.PA_FP8_F16)}
_FP8_CACHE_DTYPES = tuple(dt for dt in (torch.uint8, getattr(torch, "float8_e4m3fn", None)) if dt is not None)
_POS_DTYPES = {"i32": torch.int32, "i64": torch.int64}

_ARGS_CACHE_SIZE = 64  # prepared argument blocks kept per launcher


def _tkey(t):
    if isinstance(t, torch.Tensor):
        return (t.data_ptr(), tuple(t.shape), t.stride(), t.dtype, t.device)
    return ("obj", id(t))


def _rows(name, t, tokens, heads, head_dim, dtype, vec16=True):
    """A [>= tokens, heads, head_dim] tensor with contiguous rows -> (token stride, head stride).

    ``vec16``: rows read and written as 16-byte vectors must be 16-byte aligned."""
    if not isinstance(t, torch.Tensor) or t.dim() != 3:
        raise ValueError(f"{name} must be a 3-D tensor [tokens, heads, head_dim]")
    if t.shape[0] < tokens or t.shape[1] != heads or t.shape[2] != head_dim:
        raise ValueError(f"{name} has shape {tuple(t.shape)}; expected [>= {tokens}, {heads}, {head_dim}]")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if t.stride(2) != 1:
        raise ValueError(f"{name} must be contiguous along head_dim")
    if vec16 and (t.data_ptr() % 16 or t.stride(0) % 8 or t.stride(1) % 8):
        raise ValueError(f"{name} rows must be 16-byte aligned (pointer and strides)")
    return t.stride(0), t.stride(1)


def _index(name, t, tokens, dtype):
    if not isinstance(t, torch.Tensor) or t.dim() != 1:
        raise ValueError(f"{name} must be a 1-D tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype} (pos_dtype), got {t.dtype}")
    if t.shape[0] < tokens or (t.shape[0] > 1 and t.stride(0) != 1):
        raise ValueError(f"{name} must hold >= {tokens} contiguous entries, got shape {tuple(t.shape)}")


def _check_contiguous_tail(name, t, dims):
    """Dims ``dims..`` of ``t`` must be packed row-major (contiguous inside a (block, head) tile)."""
    expect = 1
    for d in range(t.dim() - 1, dims - 1, -1):
        if t.shape[d] != 1 and t.stride(d) != expect:
            raise ValueError(f"{name} must be contiguous inside each (block, head) tile")
        expect *= t.shape[d]


class _Spec:
    __slots__ = (
        "head_dim", "num_q_heads", "num_kv_heads", "block_size", "flash_layout", "dtype", "elem",
        "apply_scale", "reuse", "pos_dtype",
    )


def _pack_args(spec, Q, K, V, Positions, CosCache, SinCache, SlotMapping, KeyCache, ValueCache, Q_out, K_out,
               num_tokens, KScale, VScale):
    """Validate every tensor against the build parameters and fill the C argument block."""
    T = int(num_tokens)
    if T < 0:
        raise ValueError(f"num_tokens must be >= 0, got {num_tokens}")
    D, QH, KH, bs = spec.head_dim, spec.num_q_heads, spec.num_kv_heads, spec.block_size
    # head dims off the 16-dim grid (flash layout only) are read and written element by element
    vec16 = D % 16 == 0
    a = _lib.RopeCacheArgs()
    a.stride_q_token, a.stride_q_head = _rows("Q", Q, T, QH, D, spec.dtype, vec16)
    a.stride_k_token, a.stride_k_head = _rows("K", K, T, KH, D, spec.dtype, vec16)
    a.stride_v_token, a.stride_v_head = _rows("V", V, T, KH, D, spec.dtype, vec16)
    a.stride_qo_token, a.stride_qo_head = _rows("Q_out", Q_out, T, QH, D, spec.dtype, vec16)
    a.stride_ko_token, a.stride_ko_head = _rows("K_out", K_out, T, KH, D, spec.dtype, vec16)
    pos_dt = _POS_DTYPES[spec.pos_dtype]
    _index("Positions", Positions, T, pos_dt)
    _index("SlotMapping", SlotMapping, T, pos_dt)

    cols = D // 2 if spec.reuse else D
    for name, t in (("CosCache", CosCache), ("SinCache", SinCache)):
        if not isinstance(t, torch.Tensor) or t.dim() != 2 or t.shape[1] != cols or t.shape[0] < 1:
            shape = tuple(t.shape) if isinstance(t, torch.Tensor) else type(t).__name__
            raise ValueError(f"{name} must be [max_pos, {cols}] (reuse_freqs_front_part={spec.reuse}), got {shape}")
        if t.dtype != spec.dtype:
            raise ValueError(f"{name} must be {spec.dtype} (the element dtype), got {t.dtype}")
        if t.stride(1) != 1 or (vec16 and (t.data_ptr() % 16 or t.stride(0) % 8)):
            raise ValueError(f"{name} rows must be contiguous and 16-byte aligned")
    if CosCache.shape[0] != SinCache.shape[0]:
        raise ValueError("CosCache and SinCache must have the same number of positions")
    a.stride_cos_pos, a.stride_sin_pos = CosCache.stride(0), SinCache.stride(0)

    # cache layout
    if spec.flash_layout:
        for name, c in (("KeyCache", KeyCache), ("ValueCache", ValueCache)):
            if c.dim() != 4 or tuple(c.shape[1:]) != (bs, KH, D):
                raise ValueError(f"{name} must be [num_blocks, {bs}, {KH}, {D}] (flash layout), got {tuple(c.shape)}")
            if c.stride(3) != 1:
                raise ValueError(f"{name} must be contiguous along head_dim")
        layout = _lib.PA_FP8_KV_FLASH
        a.stride_kc_block, a.stride_kc_token, a.stride_kc_head = KeyCache.stride()[:3]
        a.stride_vc_block, a.stride_vc_token, a.stride_vc_head = ValueCache.stride()[:3]
    else:
        if KeyCache.dim() != 5 or tuple(KeyCache.shape[1:]) != (KH, D // _X, bs, _X):
            raise ValueError(
                f"KeyCache must be [num_blocks, {KH}, {D // _X}, {bs}, {_X}] (non-flash layout), "
                f"got {tuple(KeyCache.shape)}"
            )
        _check_contiguous_tail("KeyCache", KeyCache, 2)
        if ValueCache.dim() == 4:
            if tuple(ValueCache.shape[1:]) != (KH, D, bs):
                raise ValueError(f"ValueCache must be [num_blocks, {KH}, {D}, {bs}], got {tuple(ValueCache.shape)}")
            layout = _lib.PA_FP8_KV_X_PACKED
        elif ValueCache.dim() == 5:
            if bs % 16:
                raise ValueError(f"the 5-D (trans_v) value cache needs block_size % 16 == 0, got {bs}")
            if tuple(ValueCache.shape[1:]) != (KH, bs // 16, D, 16):
                raise ValueError(
                    f"ValueCache must be [num_blocks, {KH}, {bs // 16}, {D}, 16] (trans_v), got {tuple(ValueCache.shape)}"
                )
            layout = _lib.PA_FP8_KV_X_TRANS
        else:
            raise ValueError(f"ValueCache must be 4-D or 5-D (trans_v) for the non-flash layout, got {ValueCache.dim()}-D")
        _check_contiguous_tail("ValueCache", ValueCache, 2)
        a.stride_kc_block, a.stride_kc_head = KeyCache.stride()[:2]
        a.stride_vc_block, a.stride_vc_head = ValueCache.stride()[:2]
        a.stride_kc_token = a.stride_vc_token = 0
    if KeyCache.shape[0] != ValueCache.shape[0] or KeyCache.shape[0] < 1:
        raise ValueError("KeyCache and ValueCache must have the same (non-zero) number of blocks")
    num_blocks = KeyCache.shape[0]

    # cache format and scales
    if spec.apply_scale:
        for name, c in (("KeyCache", KeyCache), ("ValueCache", ValueCache)):
            if c.dtype not in _FP8_CACHE_DTYPES:
                raise ValueError(f"apply_scale=True writes fp8 e4m3fn codes: {name} must be float8_e4m3fn or uint8")
        for name, s in (("KScale", KScale), ("VScale", VScale)):
            if not isinstance(s, torch.Tensor) or s.dtype != torch.float32:
                raise ValueError(f"{name} must be a float32 tensor when apply_scale=True")
        per_token = KScale.dim() > 1
        if per_token != (VScale.dim() > 1):
            raise ValueError("KScale and VScale must both be per-tensor [1] or both per-token [num_blocks, KH, bs, 1]")
        if per_token:
            for name, s in (("KScale", KScale), ("VScale", VScale)):
                if s.dim() != 4 or tuple(s.shape) != (num_blocks, KH, bs, 1) or (bs > 1 and s.stride(2) != 1):
                    raise ValueError(
                        f"per-token {name} must be [{num_blocks}, {KH}, {bs}, 1] with unit token stride, "
                        f"got {tuple(s.shape)}"
                    )
            if KScale.stride()[:2] != VScale.stride()[:2]:
                raise ValueError("per-token KScale and VScale must share block / head strides")
            fmt = _lib.PA_FP8_CACHE_FP8_TOKEN
            a.stride_ks_block, a.stride_ks_head = KScale.stride()[:2]
        else:
            if KScale.numel() != 1 or VScale.numel() != 1:
                raise ValueError("per-tensor KScale / VScale must hold exactly one element")
            fmt = _lib.PA_FP8_CACHE_FP8_TENSOR
        a.key_scale, a.value_scale = KScale.data_ptr(), VScale.data_ptr()
    else:
        for name, c in (("KeyCache", KeyCache), ("ValueCache", ValueCache)):
            if c.dtype != spec.dtype:
                raise ValueError(f"apply_scale=False writes {spec.dtype}: {name} is {c.dtype}")
        fmt = _lib.PA_FP8_CACHE_ELEM
    esize = 2 if fmt == _lib.PA_FP8_CACHE_ELEM else 1
    used = 3 if spec.flash_layout else 2  # block, (token,) head strides
    for name, c in (("KeyCache", KeyCache), ("ValueCache", ValueCache)):
        if vec16 and (c.data_ptr() % (8 * esize) or any(st % 8 for st in c.stride()[:used])):
            raise ValueError(f"{name} must be aligned to 8 elements (pointer and block / head strides)")

    a.query, a.key, a.value = Q.data_ptr(), K.data_ptr(), V.data_ptr()
    a.positions, a.slot_mapping = Positions.data_ptr(), SlotMapping.data_ptr()
    a.cos_cache, a.sin_cache = CosCache.data_ptr(), SinCache.data_ptr()
    a.key_cache, a.value_cache = KeyCache.data_ptr(), ValueCache.data_ptr()
    a.query_out, a.key_out = Q_out.data_ptr(), K_out.data_ptr()
    a.num_tokens, a.num_q_heads, a.num_kv_heads, a.head_dim = T, QH, KH, D
    a.block_size, a.num_blocks, a.max_pos = bs, num_blocks, CosCache.shape[0]
    a.elem_dtype, a.cache_format, a.kv_layout = spec.elem, fmt, layout
    a.reuse_freqs_front_part = int(spec.reuse)
    a.positions_i64 = a.slots_i64 = int(spec.pos_dtype == "i64")
    return a


def build_fused_rope_cache_module(
    head_dim: int = 64,
    rotary_dim: int = -1,
    num_q_heads: int = 8,
    num_kv_heads: int = 1,
    block_size: int = 16,
    is_neox: bool = True,
    flash_layout: bool = True,
    dtype_str: str = "bf16",
    apply_scale: bool = False,
    reuse_freqs_front_part: bool = True,
    pos_dtype: str = "i32",
):
    """Fused RoPE + KV-cache launcher (kernels/fused_rope_cache_kernel.py:52-512).

    Build-time checks raise as the reference's do (:64-98): NotImplementedError
    for GPT-J style rotation or partial rotary_dim, ValueError for other dtypes
    and head sizes.
    """
    if rotary_dim == -1:
        rotary_dim = head_dim
    if not is_neox:
        raise NotImplementedError("Only NeoX-style RoPE is supported")
    if rotary_dim != head_dim:
        raise NotImplementedError("Partial rotation not yet supported")
    if dtype_str not in _ELEM:
        raise ValueError(f"dtype_str must be 'bf16' or 'f16', got {dtype_str!r}")
    # the reference's vector-width rule (:79-96): one wave of 64 lanes covers a head
    # vector, ceil(head_dim / 64) elements per lane, in both halves
    vec = max(1, (head_dim + 63) // 64)
    if head_dim % vec != 0:
        raise ValueError(f"head_dim must be a multiple of the vector width {vec}, got {head_dim}")
    if rotary_dim % 2 != 0:
        raise ValueError(f"rotary_dim must be even, got {rotary_dim}")
    if (head_dim // 2) % vec != 0:
        raise ValueError(f"head_dim / 2 must be a multiple of the vector width {vec}, got {head_dim // 2}")
    if not flash_layout and head_dim % _X != 0:
        raise ValueError(f"head_dim must be a multiple of the x-pack factor {_X} without the flash layout, got {head_dim}")
    if not 2 <= head_dim <= 1024:
        raise ValueError(f"head_dim must be in [2, 1024], got {head_dim}")
    if pos_dtype not in _POS_DTYPES:
        raise ValueError(f"pos_dtype must be 'i32' or 'i64', got {pos_dtype!r}")
    if num_q_heads < 1 or num_kv_heads < 1 or block_size < 1:
        raise ValueError("num_q_heads, num_kv_heads and block_size must be positive")

    spec = _Spec()
    spec.head_dim, spec.num_q_heads, spec.num_kv_heads = int(head_dim), int(num_q_heads), int(num_kv_heads)
    spec.block_size, spec.flash_layout = int(block_size), bool(flash_layout)
    spec.dtype, spec.elem = _ELEM[dtype_str]
    spec.apply_scale, spec.reuse, spec.pos_dtype = bool(apply_scale), bool(reuse_freqs_front_part), pos_dtype
    cache: "OrderedDict[tuple, _lib.RopeCacheArgs]" = OrderedDict()

    def launch_fused_rope_cache(
        Q, K, V, Positions, CosCache, SinCache, SlotMapping, KeyCache, ValueCache, Q_out, K_out, num_tokens,
        KScale, VScale, stream=None,
    ):
        tensors = (Q, K, V, Positions, CosCache, SinCache, SlotMapping, KeyCache, ValueCache, Q_out, K_out)
        dev = Q.device
        if dev.type != "cuda":
            raise ValueError("the fused RoPE + KV-cache writer runs on the GPU: Q must be a CUDA tensor")
        for t in tensors:
            if t.device != dev:
                raise ValueError(f"all tensors must be on {dev}; found one on {t.device}")
        if spec.apply_scale:
            for s in (KScale, VScale):
                if isinstance(s, torch.Tensor) and s.device != dev:
                    raise ValueError(f"KScale / VScale must be on {dev}")
        s = stream if stream is not None else torch.cuda.current_stream(dev)
        handle = s.cuda_stream if hasattr(s, "cuda_stream") else int(s)
        key = (tuple(_tkey(t) for t in tensors), int(num_tokens))
        if spec.apply_scale:
            key += (_tkey(KScale), _tkey(VScale))
        args = cache.get(key)
        if args is None:
            args = _pack_args(spec, *tensors, num_tokens, KScale, VScale)
            cache[key] = args
            if len(cache) > _ARGS_CACHE_SIZE:
                cache.popitem(last=False)
        else:
            cache.move_to_end(key)
        _lib.rope_cache(args, handle)

    launch_fused_rope_cache.spec = spec
    return launch_fused_rope_cache
