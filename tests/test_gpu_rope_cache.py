"""GPU parity of the fused RoPE + KV-cache writer (pa_fp8_rope_cache) against oracle/rope_cache.py.

Cases mirror the reference test's categories (tests/kernels/test_fused_rope_cache.py:502-760:
decode T=1, flash bf16 over the model shapes, non-flash, f16, i32/i64 positions,
half/full cos-sin tables, negative slots, fp8 cache) plus this build's trans_v
V layout, per-token fp8 scales, strided Q/K/V views, clamped positions,
out-of-cache slots, large prefill batches and a write-then-decode round trip.

The bar is bit-exact: Q_out, K_out, every cache byte and every written scale
equal the oracle's (same rounding after each element-dtype product and sum,
same fp8 encoding).  The reference test's own tolerances are checked too.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import quant as oq
from oracle import rope_cache as orc
from oracle.fp8 import e4m3_decode

pytestmark = pytest.mark.gpu

DEV = "cuda"
MAX_POS = 8192
TORCH_DT = {"bf16": torch.bfloat16, "f16": torch.float16}
FP8 = torch.float8_e4m3fn

MODELS = [
    ("Llama8B-TP1", 32, 8, 128),
    ("Llama8B-TP8", 4, 1, 128),
    ("Llama70B-TP1", 64, 8, 128),
    ("Llama70B-TP8", 8, 1, 128),
    ("Llama405B-TP1", 128, 8, 128),
    ("Llama405B-TP8", 16, 1, 128),
    ("Qwen72B-TP1", 64, 4, 128),
    ("GPTOSS-TP1", 64, 8, 64),
    ("GPTOSS-TP8", 8, 1, 64),
]


def _np(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint8 if t.element_size() == 1 else torch.int16).cpu().numpy().view(
        np.uint8 if t.element_size() == 1 else np.uint16
    )


def _cache_shapes(layout, nb, bs, KH, D):
    if layout == "flash":
        return (nb, bs, KH, D), (nb, bs, KH, D)
    k = (nb, KH, D // 16, bs, 16)
    return k, ((nb, KH, D, bs) if layout == "x4" else (nb, KH, bs // 16, D, 16))


def run_case(
    T, D, QH, KH, layout="flash", elem="bf16", fmt="elem", reuse=True, pos_dtype="i32", negative_slots=False,
    bs=16, num_blocks=None, slots=None, positions=None, fused_qkv=False, scale=(0.1, 0.1), seed=42, max_pos=MAX_POS,
    value_scale=1.0,
):
    """Launch the writer and compare every output with the oracle; returns the tensors."""
    from flydsl_amd.fused_rope_cache import build_fused_rope_cache_module

    dt = TORCH_DT[elem]
    g = torch.Generator().manual_seed(seed)
    nb = num_blocks or max(32, (T + bs - 1) // bs + 4)
    cols = D // 2 if reuse else D
    if fused_qkv:  # Q, K, V as strided views of one [T, (QH + 2KH) * D] projection output
        qkv = torch.randn(T, (QH + 2 * KH) * D, generator=g).to(dt).to(DEV)
        q = qkv[:, : QH * D].view(T, QH, D)
        k = qkv[:, QH * D : (QH + KH) * D].view(T, KH, D)
        v = qkv[:, (QH + KH) * D :].view(T, KH, D)
    else:
        q = torch.randn(T, QH, D, generator=g).to(dt).to(DEV)
        k = torch.randn(T, KH, D, generator=g).to(dt).to(DEV)
        v = (torch.randn(T, KH, D, generator=g) * value_scale).to(dt).to(DEV)
    cos = torch.randn(max_pos, cols, generator=g).to(dt).to(DEV)
    sin = torch.randn(max_pos, cols, generator=g).to(dt).to(DEV)
    if positions is None:
        positions = torch.randint(0, max_pos, (T,), generator=g, dtype=torch.int32)
    positions = torch.as_tensor(positions, dtype=torch.int32)
    if slots is None:
        slots = torch.arange(T, dtype=torch.int32)
        if negative_slots:
            slots[1::2] = -1
    slots = torch.as_tensor(slots, dtype=torch.int32)
    idx_dt = torch.int64 if pos_dtype == "i64" else torch.int32
    pos_t, slot_t = positions.to(idx_dt).to(DEV), slots.to(idx_dt).to(DEV)

    kshape, vshape = _cache_shapes(layout, nb, bs, KH, D)
    cache_dt = dt if fmt == "elem" else FP8
    kc = torch.zeros(kshape, dtype=cache_dt, device=DEV)
    vc = torch.zeros(vshape, dtype=cache_dt, device=DEV)
    if fmt == "fp8_token":
        ks = torch.zeros(nb, KH, bs, 1, dtype=torch.float32, device=DEV)
        vs = torch.zeros(nb, KH, bs, 1, dtype=torch.float32, device=DEV)
    else:
        ks = torch.tensor([scale[0]], dtype=torch.float32, device=DEV)
        vs = torch.tensor([scale[1]], dtype=torch.float32, device=DEV)
    q_out = torch.empty(T, QH, D, dtype=dt, device=DEV)
    k_out = torch.empty(T, KH, D, dtype=dt, device=DEV)

    launch = build_fused_rope_cache_module(
        head_dim=D, num_q_heads=QH, num_kv_heads=KH, block_size=bs, flash_layout=layout == "flash", dtype_str=elem,
        apply_scale=fmt != "elem", reuse_freqs_front_part=reuse, pos_dtype=pos_dtype,
    )
    print(f"rope_cache case T={T} D={D} QH={QH} KH={KH} layout={layout} elem={elem} fmt={fmt} reuse={reuse} "
          f"pos={pos_dtype} bs={bs} nb={nb}", flush=True)
    launch(q, k, v, pos_t, cos, sin, slot_t, kc, vc, q_out, k_out, T, ks, vs, stream=torch.cuda.current_stream())
    torch.cuda.synchronize()

    # oracle on the same inputs
    okc, ovc = orc.new_caches(nb, bs, KH, D, layout, fmt != "elem")
    oks = ovs = krcp = vrcp = None
    if fmt == "fp8_tensor":
        oks, ovs = np.float32(scale[0]), np.float32(scale[1])
        krcp, vrcp = hw_reciprocal([scale[0], scale[1]])
    elif fmt == "fp8_token":
        oks, ovs = np.zeros((nb, KH, bs, 1), np.float32), np.zeros((nb, KH, bs, 1), np.float32)
    pos_np = orc.low_word(pos_t.cpu().numpy())
    slot_np = orc.low_word(slot_t.cpu().numpy())
    oq_out, ok_out = orc.fused_rope_cache(
        _np(q), _np(k), _np(v), pos_np, _np(cos), _np(sin), slot_np, okc, ovc, elem=elem, layout=layout,
        block_size=bs, fmt=fmt, k_scale=oks, v_scale=ovs, k_rcp=krcp, v_rcp=vrcp,
    )
    np.testing.assert_array_equal(_bits(q_out), orc.elem_bits(oq_out, elem), err_msg="Q_out")
    np.testing.assert_array_equal(_bits(k_out), orc.elem_bits(ok_out, elem), err_msg="K_out")
    np.testing.assert_array_equal(_bits(kc), okc, err_msg="key cache")
    np.testing.assert_array_equal(_bits(vc), ovc, err_msg="value cache")
    if fmt == "fp8_token":
        np.testing.assert_array_equal(ks.cpu().numpy(), oks, err_msg="key scales")
        np.testing.assert_array_equal(vs.cpu().numpy(), ovs, err_msg="value scales")
    return dict(q=q, k=k, v=v, cos=cos, sin=sin, pos=positions, slots=slots, kc=kc, vc=vc, ks=ks, vs=vs,
                q_out=q_out, k_out=k_out, nb=nb, bs=bs, layout=layout, fmt=fmt, elem=elem)


def _reference_tolerances(r, atol):
    """The reference test's acceptance check (tests/kernels/test_fused_rope_cache.py:354-391)."""
    D = r["q"].shape[-1]
    dt = r["q"].dtype
    pos = r["pos"].long().to(DEV)
    cos = r["cos"][pos].unsqueeze(1)
    sin = r["sin"][pos].unsqueeze(1)
    if cos.shape[-1] == D // 2:
        cos, sin = torch.cat([cos, cos], -1), torch.cat([sin, sin], -1)

    def rot(x):
        x1, x2 = x[..., : D // 2], x[..., D // 2 :]
        return torch.cat([x1 * cos[..., : D // 2] - x2 * sin[..., : D // 2],
                          x2 * cos[..., D // 2 :] + x1 * sin[..., D // 2 :]], -1).to(dt)

    assert (r["q_out"].float() - rot(r["q"]).float()).abs().max().item() < atol
    assert (r["k_out"].float() - rot(r["k"]).float()).abs().max().item() < atol


# ---- reference categories -------------------------------------------------------------------


@pytest.mark.parametrize("name,QH,KH,D", MODELS, ids=[m[0] for m in MODELS])
def test_decode_flash(name, QH, KH, D):
    r = run_case(1, D, QH, KH)
    _reference_tolerances(r, 1e-2)


@pytest.mark.parametrize("T", [32, 128])
@pytest.mark.parametrize("name,QH,KH,D", MODELS, ids=[m[0] for m in MODELS])
def test_flash_bf16(T, name, QH, KH, D):
    run_case(T, D, QH, KH)


@pytest.mark.parametrize("layout", ["x4", "x5"])
@pytest.mark.parametrize("T", [1, 32, 128])
@pytest.mark.parametrize("name,QH,KH,D", [MODELS[0], MODELS[1], MODELS[3], MODELS[8]],
                         ids=["Llama8B-TP1", "Llama8B-TP8", "Llama70B-TP8", "GPTOSS-TP8"])
def test_nonflash_bf16(layout, T, name, QH, KH, D):
    run_case(T, D, QH, KH, layout=layout)


@pytest.mark.parametrize("layout", ["flash", "x4", "x5"])
@pytest.mark.parametrize("T", [1, 32])
def test_f16(layout, T):
    r = run_case(T, 128, 4, 1, layout=layout, elem="f16")
    _reference_tolerances(r, 5e-3)


@pytest.mark.parametrize("pos_dtype", ["i32", "i64"])
@pytest.mark.parametrize("T", [1, 32, 128])
def test_pos_dtype(pos_dtype, T):
    run_case(T, 128, 8, 1, pos_dtype=pos_dtype)


def test_i64_reads_the_low_word():
    # int64 indices above 2**32 alias their low word, as the reference's stride-2 int32 view does
    T = 8
    pos = torch.arange(T, dtype=torch.int64) * 3 + (1 << 32)
    slots = torch.arange(T, dtype=torch.int64) + (5 << 32)
    from flydsl_amd.fused_rope_cache import build_fused_rope_cache_module

    r = run_case(T, 128, 8, 1, pos_dtype="i64")  # values in range: same as int32
    launch = build_fused_rope_cache_module(head_dim=128, num_q_heads=8, num_kv_heads=1, pos_dtype="i64")
    kc = torch.zeros_like(r["kc"])
    vc = torch.zeros_like(r["vc"])
    qo = torch.empty_like(r["q_out"])
    ko = torch.empty_like(r["k_out"])
    launch(r["q"], r["k"], r["v"], pos.to(DEV), r["cos"], r["sin"], slots.to(DEV), kc, vc, qo, ko, T, r["ks"], r["vs"])
    torch.cuda.synchronize()
    okc, ovc = orc.new_caches(r["nb"], 16, 1, 128, "flash", False)
    oqo, oko = orc.fused_rope_cache(_np(r["q"]), _np(r["k"]), _np(r["v"]), orc.low_word(pos.numpy()), _np(r["cos"]),
                                    _np(r["sin"]), orc.low_word(slots.numpy()), okc, ovc, elem="bf16",
                                    layout="flash", block_size=16)
    np.testing.assert_array_equal(_bits(qo), orc.elem_bits(oqo, "bf16"))
    np.testing.assert_array_equal(_bits(kc), okc)
    np.testing.assert_array_equal(_bits(vc), ovc)


@pytest.mark.parametrize("reuse", [True, False], ids=["half_dim", "full_dim"])
@pytest.mark.parametrize("T", [1, 32])
@pytest.mark.parametrize("layout", ["flash", "x4"])
def test_reuse_freqs(reuse, T, layout):
    run_case(T, 128, 8, 1, layout=layout, reuse=reuse)


@pytest.mark.parametrize("T", [4, 32])
@pytest.mark.parametrize("layout", ["flash", "x4", "x5"])
def test_negative_slots(T, layout):
    r = run_case(T, 128, 8, 1, layout=layout, negative_slots=True)
    # skipped tokens leave their cache entries zero
    assert r["kc"].float().abs().sum().item() > 0
    assert int((r["slots"] >= 0).sum()) == (T + 1) // 2


@pytest.mark.parametrize("T", [1, 32])
@pytest.mark.parametrize("layout", ["flash", "x4", "x5"])
@pytest.mark.parametrize("QH,KH,D", [(8, 1, 64), (8, 1, 128), (32, 8, 128)], ids=["GPTOSS-TP8", "Llama-TP8", "Llama8B-TP1"])
def test_fp8_cache(T, layout, QH, KH, D):
    r = run_case(T, D, QH, KH, layout=layout, fmt="fp8_tensor")
    # the reference test's bound: dequantised error <= max|ref| / 8 (flash layout, tokens 0..T-1)
    if layout == "flash":
        kd = r["kc"].float() * r["ks"].float()
        ref = torch.zeros_like(kd)
        ref[: (T + 15) // 16].view(-1, KH, D)[:T] = r["k_out"].float()
        assert (kd - ref).abs().max().item() <= max(1e-3, ref.abs().max().item() / 8)


# ---- this build's additions --------------------------------------------------------------------


@pytest.mark.parametrize("scale", [(0.37, 1.3), (1.0, 1.0), (3.0e-3, 7.0), (3.0, 0.37)])
def test_fp8_scales_where_the_approximate_reciprocal_differs(scale):
    # the writer multiplies by v_rcp_f32(scale), as the reference does, also where it is
    # not the correctly rounded 1/scale
    run_case(64, 128, 8, 2, layout="x5", fmt="fp8_tensor", scale=scale)


def hw_reciprocal(xs):
    """v_rcp_f32 of each value, computed on the device (float32 numpy array)."""
    from flydsl_amd import _lib

    x = torch.tensor(np.asarray(xs, dtype=np.float32), device=DEV)
    y = torch.full_like(x, float("nan"))
    _lib.hw_reciprocal(x.data_ptr(), y.data_ptr(), x.numel(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def test_hw_reciprocal_within_one_ulp():
    # the primitive the writer's per-tensor codes rest on: within 1 ulp of 1/x over a
    # sweep of scales, exact at powers of two, and equal to the correctly rounded
    # quotient at the scales the CPU oracle tests use
    rng = np.random.default_rng(7)
    xs = np.concatenate([
        np.exp(rng.uniform(np.log(1e-6), np.log(1e6), 200000)).astype(np.float32),
        np.float32(2.0) ** np.arange(-40, 41, dtype=np.float32),
        np.array([0.1, 0.05, 0.25, 3.0, 0.37, 1.3, 7.0, 3.0e-3], np.float32),
    ])
    got = hw_reciprocal(xs).astype(np.float64)
    exact = 1.0 / xs.astype(np.float64)
    crr = (np.float32(1.0) / xs).astype(np.float64)  # correctly rounded
    ulp = np.spacing(crr.astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - exact) <= ulp), "v_rcp_f32 more than 1 ulp from 1/x"
    pow2 = slice(200000, 200000 + 81)
    np.testing.assert_array_equal(got[pow2], crr[pow2])
    tail = got[-8:]
    np.testing.assert_array_equal(tail[:3], crr[-8:-5])  # 0.1, 0.05, 0.25
    print(f"v_rcp_f32 differs from the correctly rounded 1/x on {int((got != crr).sum())} of {xs.size} "
          f"values; at 3.0: {got[-5] != crr[-5]}, at 0.37: {got[-4] != crr[-4]}", flush=True)


@pytest.mark.parametrize("layout", ["flash", "x4", "x5"])
@pytest.mark.parametrize("QH,KH,D", [(8, 1, 128), (32, 8, 128), (8, 1, 64), (16, 2, 256)])
def test_fp8_per_token(layout, QH, KH, D):
    run_case(48, D, QH, KH, layout=layout, fmt="fp8_token", slots=torch.randperm(32 * 16)[:48].int())


@pytest.mark.parametrize("D", [16, 32, 80, 96, 192, 256, 512])
@pytest.mark.parametrize("fmt", ["elem", "fp8_token"])
def test_other_head_dims(D, fmt):
    run_case(33, D, 6, 2, layout="x5", fmt=fmt)


@pytest.mark.parametrize("layout", ["flash", "x4", "x5"])
def test_fused_qkv_views(layout):
    run_case(40, 128, 32, 8, layout=layout, fused_qkv=True, fmt="fp8_tensor")


@pytest.mark.parametrize("bs", [1, 16, 64, 1024])
def test_block_sizes_random_slots(bs):
    layout = "x5" if bs % 16 == 0 else "x4"
    nb = max(4, 3000 // bs)
    slots = torch.randperm(nb * bs, generator=torch.Generator().manual_seed(bs))[:200].int()
    run_case(200, 128, 8, 2, layout=layout, bs=bs, num_blocks=nb, slots=slots, fmt="fp8_token")


def test_positions_clamped_and_slots_past_the_cache_skipped():
    T = 16
    pos = torch.tensor([0, 5, -3, 99, 100, 1 << 20, 7, 50, -1, 2, 3, 4, 98, 97, 1000, 1], dtype=torch.int32)
    slots = torch.tensor([0, 1, 2, 3, 16 * 6 - 1, 16 * 6, 16 * 6 + 5, 1 << 30, 8, 9, -7, 11, 12, 13, 14, 15],
                         dtype=torch.int32)
    run_case(T, 128, 8, 2, layout="x5", positions=pos, slots=slots, num_blocks=6, max_pos=100, fmt="fp8_token")


def test_large_prefill_batch():
    T = 4096
    slots = torch.randperm(5000, generator=torch.Generator().manual_seed(1))[:T].int()
    run_case(T, 128, 32, 8, layout="x5", fmt="fp8_tensor", slots=slots, num_blocks=5000 // 16)


def test_zero_tokens_is_a_no_op():
    from flydsl_amd.fused_rope_cache import build_fused_rope_cache_module

    launch = build_fused_rope_cache_module(head_dim=128, num_q_heads=8, num_kv_heads=1)
    t = lambda *s: torch.zeros(*s, dtype=torch.bfloat16, device=DEV)  # noqa: E731
    kc, vc = t(4, 16, 1, 128), t(4, 16, 1, 128)
    launch(t(0, 8, 128), t(0, 1, 128), t(0, 1, 128), torch.zeros(0, dtype=torch.int32, device=DEV), t(16, 64),
           t(16, 64), torch.zeros(0, dtype=torch.int32, device=DEV), kc, vc, t(0, 8, 128), t(0, 1, 128), 0,
           torch.ones(1, device=DEV), torch.ones(1, device=DEV))
    torch.cuda.synchronize()
    assert kc.abs().sum().item() == 0


def test_repeated_launches_reuse_argument_blocks():
    # the launcher caches prepared argument blocks per tensor set; new slot values on the same
    # tensors must still be honoured (the kernel reads them from device memory)
    from flydsl_amd.fused_rope_cache import build_fused_rope_cache_module

    r = run_case(8, 128, 8, 1, layout="x5", fmt="fp8_tensor")
    launch = build_fused_rope_cache_module(head_dim=128, num_q_heads=8, num_kv_heads=1, flash_layout=False,
                                           apply_scale=True)
    slot_t = torch.zeros(8, dtype=torch.int32, device=DEV)
    pos_t = r["pos"].to(DEV)
    kc = torch.zeros_like(r["kc"])
    vc = torch.zeros_like(r["vc"])
    qo, ko = torch.empty_like(r["q_out"]), torch.empty_like(r["k_out"])
    for step in range(3):
        slot_t.copy_(torch.arange(8, dtype=torch.int32) + 8 * step)
        launch(r["q"], r["k"], r["v"], pos_t, r["cos"], r["sin"], slot_t, kc, vc, qo, ko, 8, r["ks"], r["vs"])
    torch.cuda.synchronize()
    k_tok = oq.k_x_to_tok(_bits(kc))
    for step in range(3):
        for t in range(8):
            blk, p = divmod(8 * step + t, 16)
            np.testing.assert_array_equal(k_tok[blk, 0, p], _bits(r["kc"])[0, 0, :, t, :].reshape(-1))


@pytest.mark.parametrize("per_token", [False, True], ids=["per_tensor", "per_token"])
def test_write_then_decode(per_token):
    """Write a batch's K/V with the writer (x-packed K, trans_v V, fp8) and decode over it."""
    from flydsl_amd import pa_decode_ps_launch
    from flydsl_amd.fused_rope_cache import build_fused_rope_cache_module

    B, QH, KH, D, bs = 4, 16, 2, 128, 16
    ctx = [37, 300, 129, 513]
    g = torch.Generator().manual_seed(7)
    blocks = [math.ceil(c / bs) for c in ctx]
    nb = sum(blocks) + 3
    perm = torch.randperm(nb, generator=g)
    tables = torch.zeros(B, max(blocks), dtype=torch.int32)
    start = 0
    for b in range(B):
        tables[b, : blocks[b]] = perm[start : start + blocks[b]]
        start += blocks[b]
    # every token of every sequence, prefill-style, in one launch
    T = sum(ctx)
    slots = torch.cat([tables[b, torch.arange(ctx[b]) // bs].long() * bs + torch.arange(ctx[b]) % bs
                       for b in range(B)]).int()
    positions = torch.cat([torch.arange(c) for c in ctx]).int()
    k = torch.randn(T, KH, D, generator=g).bfloat16().to(DEV)
    v = torch.randn(T, KH, D, generator=g).bfloat16().to(DEV)
    q_tok = torch.randn(T, QH, D, generator=g).bfloat16().to(DEV)
    th = torch.arange(MAX_POS)[:, None].float() * (10000.0 ** (-torch.arange(D // 2).float() / (D // 2)))
    cos, sin = th.cos().bfloat16().to(DEV), th.sin().bfloat16().to(DEV)
    kc = torch.zeros(nb, KH, D // 16, bs, 16, dtype=FP8, device=DEV)
    vc = torch.zeros(nb, KH, bs // 16, D, 16, dtype=FP8, device=DEV)
    if per_token:
        ks = torch.zeros(nb, KH, bs, 1, device=DEV)
        vs = torch.zeros(nb, KH, bs, 1, device=DEV)
    else:
        ks = torch.tensor([0.02], device=DEV)
        vs = torch.tensor([0.015], device=DEV)
    q_out = torch.empty_like(q_tok)
    k_out = torch.empty_like(k)
    launch = build_fused_rope_cache_module(head_dim=D, num_q_heads=QH, num_kv_heads=KH, block_size=bs,
                                           flash_layout=False, apply_scale=True)
    launch(q_tok, k, v, positions.to(DEV), cos, sin, slots.to(DEV), kc, vc, q_out, k_out, T, ks, vs)
    # decode the last token of every sequence with its rotated query
    last = torch.tensor(np.cumsum(ctx) - 1)
    query = q_out[last.to(DEV)].contiguous()
    out = torch.empty_like(query)
    ctx_t = torch.tensor(ctx, dtype=torch.int32, device=DEV)
    pa_decode_ps_launch(out, query, kc, vc, ctx_t, None, None, 1.0 / math.sqrt(D), ks, vs,
                        block_tables=tables.to(DEV))
    torch.cuda.synchronize()
    # oracle: attention over the dequantised cache the writer produced (itself checked bit-exact above)
    k_tok = oq.k_x_to_tok(_bits(kc))
    v_tok = oq.v_4d_to_tok(oq.v_trans_to_4d(_bits(vc)))
    ksn, vsn = ks.cpu().numpy(), vs.cpu().numpy()
    for b in range(B):
        rows = slots[int(np.sum(ctx[:b])) : int(np.sum(ctx[: b + 1]))].long().numpy()
        blk, p = rows // bs, rows % bs
        kk = e4m3_decode(k_tok[blk, :, p])  # [ctx, KH, D]
        vv = e4m3_decode(v_tok[blk, :, p])
        if per_token:
            kk = kk * ksn[blk, :, p]
            vv = vv * vsn[blk, :, p]
        else:
            kk, vv = kk * ksn[0], vv * vsn[0]
        # the written keys are the rotated keys, to fp8 precision
        kref = _np(k_out)[int(np.sum(ctx[:b])) : int(np.sum(ctx[: b + 1]))]
        assert np.abs(kk - kref).max() <= np.abs(kref).max() / 8
        want = oatt.reference_masked_attention(_np(query)[b : b + 1], kk, vv, 1.0 / math.sqrt(D), True, 0)
        np.testing.assert_allclose(_np(out)[b : b + 1], want, atol=2e-2, rtol=2e-2)


def _runs(kind, T, bs, nb, seed):
    """Slot patterns around the staged V path (16-token groups of consecutive, 16-aligned slots)."""
    g = torch.Generator().manual_seed(seed)
    if kind == "aligned":
        return torch.arange(T, dtype=torch.int32) + 3 * bs
    if kind == "misaligned":
        return torch.arange(T, dtype=torch.int32) + 5
    if kind == "one_swap":
        s = torch.arange(T, dtype=torch.int32) + bs
        s[[17, 18]] = s[[18, 17]]
        return s
    if kind == "pages":  # every 16-token group in its own random page, aligned inside it
        groups = (T + 15) // 16
        starts = torch.randperm(nb * bs // 16, generator=g)[:groups].int() * 16
        return (starts.repeat_interleave(16)[:T] + torch.arange(T, dtype=torch.int32) % 16).int()
    if kind == "tail_negative":
        s = torch.arange(T, dtype=torch.int32)
        s[-3:] = -1
        return s
    raise ValueError(kind)


@pytest.mark.parametrize("kind", ["aligned", "misaligned", "one_swap", "pages", "tail_negative"])
@pytest.mark.parametrize("T", [50, 64, 200])
@pytest.mark.parametrize("layout,fmt", [("x5", "fp8_tensor"), ("x4", "fp8_token"), ("x5", "elem"), ("x4", "elem")])
def test_prefill_slot_runs(kind, T, layout, fmt):
    bs, nb = 32, 24
    run_case(T, 128, 8, 2, layout=layout, fmt=fmt, bs=bs, num_blocks=nb, slots=_runs(kind, T, bs, nb, T))


@pytest.mark.parametrize("D,QH,KH", [(64, 8, 1), (256, 4, 2), (96, 6, 2), (512, 2, 1)])
def test_prefill_runs_other_head_dims(D, QH, KH):
    # D=512 has 8 rows per workgroup (fewer than a 16-token group): element-wise V writes
    run_case(80, D, QH, KH, layout="x5", fmt="fp8_token", bs=16, num_blocks=12, slots=_runs("aligned", 80, 16, 12, 0))


# ---- head dims off the 16-dim grid (flash layout) ----------------------------------------------
# The reference admits any head dim its vector-width rule passes in the flash layout
# (kernels/fused_rope_cache_kernel.py:79-96): 72, 100, 200, 900, ... as well as the
# multiples of 16.  These run the element-wise kernel; same bit-exact bar.

NARROW_DIMS = [2, 8, 20, 40, 72, 100, 120, 200, 300, 900]


@pytest.mark.parametrize("D", NARROW_DIMS)
@pytest.mark.parametrize("fmt", ["elem", "fp8_tensor", "fp8_token"])
def test_flash_head_dims_off_the_16_grid(D, fmt):
    run_case(37, D, 6, 2, fmt=fmt, negative_slots=True)


@pytest.mark.parametrize("D", [20, 72, 200])
def test_flash_off_grid_f16_full_tables_i64(D):
    run_case(25, D, 4, 2, elem="f16", reuse=False, pos_dtype="i64", fmt="fp8_token", bs=24,
             slots=torch.randperm(8 * 24, generator=torch.Generator().manual_seed(D))[:25].int(), num_blocks=8)


@pytest.mark.parametrize("D", [20, 40, 72])
def test_flash_off_grid_strided_views(D):
    # Q / K / V as views of one projection output: token strides of (QH + 2 KH) * D
    # elements, not 16-byte multiples
    run_case(19, D, 6, 2, fused_qkv=True, fmt="fp8_tensor")


@pytest.mark.parametrize("D", [8, 72, 120])
def test_flash_off_grid_decode_tolerances(D):
    r = run_case(1, D, 8, 1)
    _reference_tolerances(r, 1e-2)


@pytest.mark.parametrize("seed", range(12))
def test_random_flash_off_grid_case(seed):
    """Random flash-layout launches at head dims off the 16-dim grid, bit-exact against
    the oracle: every element dtype and cache format, half / full tables, i32 / i64
    indices, page sizes 1-1024, strided views and skipped slots."""
    import random

    rnd = random.Random(7100 + seed)
    D = rnd.choice(NARROW_DIMS)
    bs = rnd.choice([1, 2, 8, 16, 24, 64, 256, 1024])
    KH = rnd.choice([1, 2, 4, 8])
    QH = KH * rnd.choice([1, 2, 4, 8])
    T = rnd.choice([1, 3, 16, 64, 200])
    nb = max(4, (T + bs - 1) // bs + rnd.randint(0, 4))
    g = torch.Generator().manual_seed(7100 + seed)
    slots = torch.randperm(nb * bs, generator=g)[:T].to(torch.int32)
    slots[torch.rand(T, generator=g) < 0.1] = -1
    run_case(T, D, QH, KH, elem=rnd.choice(["bf16", "f16"]), fmt=rnd.choice(["elem", "fp8_tensor", "fp8_token"]),
             reuse=rnd.random() < 0.5, pos_dtype=rnd.choice(["i32", "i64"]), bs=bs, num_blocks=nb, slots=slots,
             fused_qkv=rnd.random() < 0.3, seed=7100 + seed)


@pytest.mark.parametrize(
    "layout,bs,fmt,kind",
    [("flash", 24, "fp8_token", "random"), ("x4", 24, "elem", "random"), ("x5", 48, "fp8_tensor", "random"),
     ("x5", 48, "fp8_token", "aligned"), ("x4", 48, "elem", "aligned")],
)
def test_divisors_that_are_not_powers_of_two(layout, bs, fmt, kind):
    """12 query and 3 kv heads, head_dim 96 and 24- or 48-token pages: every index the
    kernel divides (row / heads, (token group, head) / kv heads, slot / block size and
    the staged segments' index / head_dim) has a divisor that is not a power of two."""
    T, nb = 150, 12
    if kind == "random":
        slots = torch.randperm(nb * bs, generator=torch.Generator().manual_seed(bs))[:T].int()
    else:  # consecutive slots from a 16-aligned start: the staged V writes
        slots = _runs("aligned", T, bs, nb, T)
    run_case(T, 96, 12, 3, layout=layout, fmt=fmt, bs=bs, num_blocks=nb, slots=slots)


# ---- seeded random cases -------------------------------------------------------------------


@pytest.mark.parametrize("seed", range(32))
def test_random_writer_case(seed):
    """Random valid writer launches, bit-exact against the oracle: token counts 1-600,
    head dims 16-512, GQA 1-8, every cache layout, element dtype and cache format,
    half / full tables, i32 / i64 indices, page sizes 1-1024, strided Q/K/V views,
    and unique random slots with some skipped (negative)."""
    import random

    rnd = random.Random(9000 + seed)
    layout = rnd.choice(["flash", "x4", "x5"])
    bs = rnd.choice([16, 32, 64, 256, 1024] if layout == "x5" else [1, 2, 8, 16, 64, 256, 1024])
    D = rnd.choice([16, 32, 64, 96, 128, 128, 192, 256, 512])
    KH = rnd.choice([1, 2, 4, 8])
    QH = KH * rnd.choice([1, 2, 4, 8])
    T = rnd.choice([1, 3, 16, 64, 200, 600])
    nb = max(4, (T + bs - 1) // bs + rnd.randint(0, 4))
    g = torch.Generator().manual_seed(9000 + seed)
    slots = torch.randperm(nb * bs, generator=g)[:T].to(torch.int32)
    slots[torch.rand(T, generator=g) < 0.1] = -1
    run_case(T, D, QH, KH, layout=layout, elem=rnd.choice(["bf16", "f16"]),
             fmt=rnd.choice(["elem", "fp8_tensor", "fp8_token"]), reuse=rnd.random() < 0.5,
             pos_dtype=rnd.choice(["i32", "i64"]), bs=bs, num_blocks=nb, slots=slots,
             fused_qkv=rnd.random() < 0.3, seed=9000 + seed)
