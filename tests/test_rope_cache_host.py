"""Host logic of the fused RoPE + KV-cache launcher (no GPU): build-time checks,
tensor validation and the argument block handed to pa_fp8_rope_cache."""

from __future__ import annotations

import pytest
import torch

from flydsl_amd import _lib
from flydsl_amd import fused_rope_cache as frc


def _tensors(T=4, QH=8, KH=2, D=128, bs=16, nb=6, layout="flash", fp8=False, per_token=False, reuse=True,
             pos_dtype=torch.int32):
    bf = torch.bfloat16
    cache_dt = torch.float8_e4m3fn if fp8 else bf
    if layout == "flash":
        kc = torch.zeros(nb, bs, KH, D, dtype=cache_dt)
        vc = torch.zeros(nb, bs, KH, D, dtype=cache_dt)
    else:
        kc = torch.zeros(nb, KH, D // 16, bs, 16, dtype=cache_dt)
        vc = torch.zeros((nb, KH, D, bs) if layout == "x4" else (nb, KH, bs // 16, D, 16), dtype=cache_dt)
    cols = D // 2 if reuse else D
    ks = torch.zeros(nb, KH, bs, 1) if per_token else torch.ones(1)
    vs = torch.zeros(nb, KH, bs, 1) if per_token else torch.ones(1)
    return dict(
        Q=torch.zeros(T, QH, D, dtype=bf), K=torch.zeros(T, KH, D, dtype=bf), V=torch.zeros(T, KH, D, dtype=bf),
        Positions=torch.zeros(T, dtype=pos_dtype), CosCache=torch.zeros(64, cols, dtype=bf),
        SinCache=torch.zeros(64, cols, dtype=bf), SlotMapping=torch.zeros(T, dtype=pos_dtype), KeyCache=kc,
        ValueCache=vc, Q_out=torch.zeros(T, QH, D, dtype=bf), K_out=torch.zeros(T, KH, D, dtype=bf), num_tokens=T,
        KScale=ks, VScale=vs,
    )


def _spec(**kw):
    launch = frc.build_fused_rope_cache_module(**{**dict(head_dim=128, num_q_heads=8, num_kv_heads=2), **kw})
    return launch.spec


def _pack(spec, t):
    return frc._pack_args(spec, *t.values())


def test_build_time_checks_follow_the_reference():
    with pytest.raises(NotImplementedError):
        frc.build_fused_rope_cache_module(is_neox=False)
    with pytest.raises(NotImplementedError):
        frc.build_fused_rope_cache_module(head_dim=128, rotary_dim=64)
    with pytest.raises(ValueError):
        frc.build_fused_rope_cache_module(dtype_str="f32")
    with pytest.raises(ValueError):
        frc.build_fused_rope_cache_module(pos_dtype="i16")
    assert callable(frc.build_fused_rope_cache_module(head_dim=64))


# head dims the reference's vector-width rule admits (kernels/fused_rope_cache_kernel.py:79-96):
# width w = ceil(D / 64); D and D / 2 multiples of w; D a multiple of 16 without the flash layout
@pytest.mark.parametrize("D,flash,ok", [
    (2, True, True), (8, True, True), (20, True, True), (62, True, True), (72, True, True),
    (100, True, True), (200, True, True), (900, True, True), (1024, True, True), (1024, False, True),
    (72, False, False),   # not a multiple of 16 without the flash layout
    (66, True, False),    # w = 2, D / 2 = 33
    (130, True, False),   # w = 3, 130 % 3
    (160, True, False),   # w = 3, 160 % 3, although a multiple of 16
    (1008, True, False),  # w = 16, D / 2 = 504
    (63, True, False),    # rotary_dim odd
    (1040, True, False),  # past 1024
])
def test_head_dim_rule(D, flash, ok):
    if ok:
        assert callable(frc.build_fused_rope_cache_module(head_dim=D, flash_layout=flash))
    else:
        with pytest.raises(ValueError):
            frc.build_fused_rope_cache_module(head_dim=D, flash_layout=flash)


def test_off_grid_head_dim_takes_element_alignment():
    """Head dims off the 16-dim grid are read element by element: rows, tables and
    caches need only element alignment (a 16-dim head keeps the 16-byte rule)."""
    D, QH, KH, T = 20, 5, 2, 5
    launch = frc.build_fused_rope_cache_module(head_dim=D, num_q_heads=QH, num_kv_heads=KH)
    qkv = torch.zeros(T, (QH + 2 * KH) * D, dtype=torch.bfloat16)
    q = qkv[:, : QH * D].view(T, QH, D)
    k = qkv[:, QH * D: (QH + KH) * D].view(T, KH, D)
    v = qkv[:, (QH + KH) * D:].view(T, KH, D)
    t = dict(Q=q, K=k, V=v, Positions=torch.zeros(T, dtype=torch.int32),
             CosCache=torch.zeros(16, D // 2, dtype=torch.bfloat16), SinCache=torch.zeros(16, D // 2, dtype=torch.bfloat16),
             SlotMapping=torch.arange(T, dtype=torch.int32),
             KeyCache=torch.zeros(4, 16, KH, D, dtype=torch.bfloat16), ValueCache=torch.zeros(4, 16, KH, D, dtype=torch.bfloat16),
             Q_out=torch.zeros(T, QH, D, dtype=torch.bfloat16), K_out=torch.zeros(T, KH, D, dtype=torch.bfloat16),
             num_tokens=T, KScale=None, VScale=None)
    a = _pack(launch.spec, t)
    assert (a.head_dim, a.stride_q_token, a.kv_layout) == (D, (QH + 2 * KH) * D, frc._lib.PA_FP8_KV_FLASH)
    assert a.stride_q_token % 8 != 0 and a.stride_q_head % 8 != 0  # 180 and 20 elements


@pytest.mark.parametrize(
    "layout,fp8,per_token,fmt,kv",
    [
        ("flash", False, False, _lib.PA_FP8_CACHE_ELEM, _lib.PA_FP8_KV_FLASH),
        ("flash", True, False, _lib.PA_FP8_CACHE_FP8_TENSOR, _lib.PA_FP8_KV_FLASH),
        ("x4", True, False, _lib.PA_FP8_CACHE_FP8_TENSOR, _lib.PA_FP8_KV_X_PACKED),
        ("x5", True, True, _lib.PA_FP8_CACHE_FP8_TOKEN, _lib.PA_FP8_KV_X_TRANS),
        ("x5", False, False, _lib.PA_FP8_CACHE_ELEM, _lib.PA_FP8_KV_X_TRANS),
    ],
)
def test_argument_block(layout, fp8, per_token, fmt, kv):
    spec = _spec(flash_layout=layout == "flash", apply_scale=fp8)
    t = _tensors(layout=layout, fp8=fp8, per_token=per_token)
    a = _pack(spec, t)
    assert (a.cache_format, a.kv_layout) == (fmt, kv)
    assert (a.num_tokens, a.num_q_heads, a.num_kv_heads, a.head_dim, a.block_size) == (4, 8, 2, 128, 16)
    assert (a.num_blocks, a.max_pos, a.elem_dtype) == (6, 64, _lib.PA_FP8_BF16)
    assert (a.stride_q_token, a.stride_q_head) == (8 * 128, 128)
    assert a.stride_kc_block == t["KeyCache"].stride(0) and a.stride_vc_block == t["ValueCache"].stride(0)
    if layout == "flash":  # [nb, bs, KH, D]: token stride KH*D, head stride D
        assert (a.stride_kc_token, a.stride_kc_head, a.stride_vc_token, a.stride_vc_head) == (256, 128, 256, 128)
    else:
        assert (a.stride_kc_head, a.stride_vc_head) == (t["KeyCache"].stride(1), t["ValueCache"].stride(1))
    if per_token:
        assert (a.stride_ks_block, a.stride_ks_head) == (2 * 16, 16)
    assert a.query == t["Q"].data_ptr() and a.key_cache == t["KeyCache"].data_ptr()
    assert a.reuse_freqs_front_part == 1 and a.positions_i64 == 0


def test_strided_views_and_int64_indices():
    spec = _spec(pos_dtype="i64", reuse_freqs_front_part=False)
    t = _tensors(pos_dtype=torch.int64, reuse=False)
    qkv = torch.zeros(4, (8 + 4) * 128, dtype=torch.bfloat16)
    t["Q"] = qkv[:, : 8 * 128].view(4, 8, 128)
    t["K"] = qkv[:, 8 * 128 : 10 * 128].view(4, 2, 128)
    t["V"] = qkv[:, 10 * 128 :].view(4, 2, 128)
    a = _pack(spec, t)
    assert (a.stride_q_token, a.stride_k_token, a.stride_v_token) == (12 * 128,) * 3
    assert a.positions_i64 == a.slots_i64 == 1 and a.reuse_freqs_front_part == 0


@pytest.mark.parametrize(
    "mutate,match",
    [
        (lambda t: t.update(Q=torch.zeros(4, 8, 64, dtype=torch.bfloat16)), "Q has shape"),
        (lambda t: t.update(K=torch.zeros(4, 2, 128, dtype=torch.float16)), "K must be"),
        (lambda t: t.update(V=torch.zeros(4, 2, 256, dtype=torch.bfloat16)[..., ::2]), "contiguous along head_dim"),
        (lambda t: t.update(Q_out=torch.zeros(3, 8, 128, dtype=torch.bfloat16)), "Q_out has shape"),
        (lambda t: t.update(Positions=torch.zeros(4, dtype=torch.int64)), "Positions must be torch.int32"),
        (lambda t: t.update(SlotMapping=torch.zeros(2, dtype=torch.int32)), "SlotMapping must hold"),
        (lambda t: t.update(CosCache=torch.zeros(64, 128, dtype=torch.bfloat16)), "CosCache must be"),
        (lambda t: t.update(SinCache=torch.zeros(64, 64, dtype=torch.float32)), "SinCache must be"),
        (lambda t: t.update(SinCache=torch.zeros(32, 64, dtype=torch.bfloat16)), "same number of positions"),
        (lambda t: t.update(KeyCache=torch.zeros(6, 2, 8, 16, 16, dtype=torch.bfloat16)), "KeyCache must be"),
        (lambda t: t.update(ValueCache=torch.zeros(5, 16, 2, 128, dtype=torch.bfloat16)), "same"),
        (lambda t: t.update(KeyCache=torch.zeros(6, 16, 2, 128, dtype=torch.uint8)), "apply_scale=False"),
        (lambda t: t.update(num_tokens=-1), "num_tokens"),
        (lambda t: t.update(num_tokens=5), "has shape"),
    ],
)
def test_validation_errors(mutate, match):
    spec = _spec()
    t = _tensors()
    mutate(t)
    with pytest.raises(ValueError, match=match):
        _pack(spec, t)


def test_fp8_and_layout_validation_errors():
    spec = _spec(flash_layout=False, apply_scale=True)
    t = _tensors(layout="x5", fp8=True)
    t["KScale"] = torch.zeros(6, 2, 16, 1)  # per-token K with per-tensor V
    with pytest.raises(ValueError, match="both"):
        _pack(spec, t)
    t = _tensors(layout="x5", fp8=True, per_token=True)
    t["VScale"] = torch.zeros(6, 2, 8, 1)
    with pytest.raises(ValueError, match="per-token VScale"):
        _pack(spec, t)
    t = _tensors(layout="x5", fp8=False)
    with pytest.raises(ValueError, match="float8_e4m3fn or uint8"):
        _pack(spec, t)
    t = _tensors(layout="x5", fp8=True)
    t["KScale"] = torch.ones(1, dtype=torch.float64)
    with pytest.raises(ValueError, match="float32"):
        _pack(spec, t)
    spec8 = _spec(flash_layout=False, block_size=8)
    t = _tensors(layout="x5", bs=16)
    t["KeyCache"] = torch.zeros(6, 2, 8, 8, 16, dtype=torch.bfloat16)
    t["ValueCache"] = torch.zeros(6, 2, 1, 128, 16, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="block_size % 16"):
        _pack(spec8, t)
    t = _tensors(layout="x5", fp8=True)
    t["ValueCache"] = torch.zeros(6, 2, 1, 128, 16, 1, dtype=torch.float8_e4m3fn)
    with pytest.raises(ValueError, match="4-D or 5-D"):
        _pack(spec, t)


def test_launch_requires_cuda_tensors():
    launch = frc.build_fused_rope_cache_module(head_dim=128, num_q_heads=8, num_kv_heads=2)
    with pytest.raises(ValueError, match="GPU"):
        launch(*_tensors().values())
