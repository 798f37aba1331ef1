"""Pins of the fused RoPE + KV-cache writer restatement (oracle/rope_cache.py).

* torch's own bf16 / f16 arithmetic on the reference test's formula
  (tests/kernels/test_fused_rope_cache.py:166-215: ``q1*cos - q2*sin`` and
  ``q2*cos + q1*sin`` on element-dtype tensors, each op rounded by torch)
  matches the restatement bit for bit; rounding only once at the end, or
  pairing d with d^1 (GPT-J style) instead of d + D/2, does not;
* in exact (float64) arithmetic the rotation is a plane rotation: identity at
  angle 0, (a, b) -> (-b, a) at a quarter turn, pair norms preserved, angles
  add, a turn and its inverse cancel;
* half-width tables equal full-width tables holding [c, c];
* every layout round-trips through the layout inverses of oracle/quant.py
  (pinned against the reference test's cache shapes), skipped slots stay untouched;
* fp8 codes equal torch's float8_e4m3fn cast of the scaled values and satisfy
  the reference test's dequantisation bound (max|ref| / 8).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quant as oq
from oracle import rope_cache as orc
from oracle.fp8 import e4m3_decode

TORCH_DT = {"bf16": torch.bfloat16, "f16": torch.float16}


def _rand(shape, elem, rng, scale=1.0):
    x = (rng.standard_normal(shape) * scale).astype(np.float32)
    return orc.round_elem(x, elem)


def _torch_rope(x, cos_rows, sin_rows, elem):
    """The reference test's torch model, evaluated in the element dtype by torch."""
    dt = TORCH_DT[elem]
    xt = torch.from_numpy(np.ascontiguousarray(x)).to(dt)
    c = torch.from_numpy(np.ascontiguousarray(cos_rows)).to(dt).unsqueeze(1)
    s = torch.from_numpy(np.ascontiguousarray(sin_rows)).to(dt).unsqueeze(1)
    D = xt.shape[-1]
    if c.shape[-1] == D // 2:
        c = torch.cat([c, c], dim=-1)
        s = torch.cat([s, s], dim=-1)
    x1, x2 = xt[..., : D // 2], xt[..., D // 2 :]
    out = torch.cat([x1 * c[..., : D // 2] - x2 * s[..., : D // 2], x2 * c[..., D // 2 :] + x1 * s[..., D // 2 :]], -1)
    return out.float().numpy()


@pytest.mark.parametrize("elem", ["bf16", "f16"])
@pytest.mark.parametrize("reuse", [True, False])
@pytest.mark.parametrize("T,H,D", [(1, 8, 64), (17, 4, 128), (5, 2, 256)])
def test_matches_torch_element_dtype_arithmetic(elem, reuse, T, H, D):
    rng = np.random.default_rng(T * 1000 + H * 10 + D)
    x = _rand((T, H, D), elem, rng, 3.0)
    cols = D // 2 if reuse else D
    c = _rand((T, cols), elem, rng)
    s = _rand((T, cols), elem, rng)
    want = _torch_rope(x, c, s, elem)
    got = orc.rope_neox(x, c, s, elem)
    np.testing.assert_array_equal(orc.elem_bits(got, elem), orc.elem_bits(want, elem))


@pytest.mark.parametrize("elem", ["bf16", "f16"])
def test_planted_mistakes_fail_the_torch_pin(elem):
    rng = np.random.default_rng(3)
    T, H, D = 64, 8, 128
    x = _rand((T, H, D), elem, rng, 3.0)
    c = _rand((T, D // 2), elem, rng)
    s = _rand((T, D // 2), elem, rng)
    want = orc.elem_bits(_torch_rope(x, c, s, elem), elem)
    # (1) one rounding at the end instead of after every product
    once = orc.elem_bits(orc.rope_neox(x, c, s, elem, round_steps=False), elem)
    assert (once != want).any()
    # (2) GPT-J pairing (d with d^1) instead of NeoX (d with d + D/2)
    perm = np.arange(D).reshape(2, D // 2).T.reshape(-1)  # interleave the halves
    inv = np.argsort(perm)
    gptj = orc.rope_neox(x[..., perm], c, s, elem)[..., inv]
    assert (orc.elem_bits(gptj, elem) != want).any()


def _angles(T, D, rng):
    return rng.uniform(-np.pi, np.pi, size=(T, D // 2))


def test_exact_rotation_closed_forms():
    rng = np.random.default_rng(11)
    T, H, D = 6, 3, 32
    x = rng.standard_normal((T, H, D))
    a, b = x[..., : D // 2], x[..., D // 2 :]
    # angle 0: identity
    np.testing.assert_array_equal(orc.rope_neox(x, np.ones((T, D // 2)), np.zeros((T, D // 2)), "f64"), x)
    # quarter turn: (a, b) -> (-b, a)
    q = orc.rope_neox(x, np.zeros((T, D // 2)), np.ones((T, D // 2)), "f64")
    np.testing.assert_array_equal(q, np.concatenate([-b, a], -1))
    # norms of every (d, d + D/2) pair preserved
    th = _angles(T, D, rng)
    y = orc.rope_neox(x, np.cos(th), np.sin(th), "f64")
    np.testing.assert_allclose(y[..., : D // 2] ** 2 + y[..., D // 2 :] ** 2, a**2 + b**2, rtol=1e-12)
    # angles add; a turn and its inverse cancel
    th2 = _angles(T, D, rng)
    yy = orc.rope_neox(y, np.cos(th2), np.sin(th2), "f64")
    np.testing.assert_allclose(yy, orc.rope_neox(x, np.cos(th + th2), np.sin(th + th2), "f64"), atol=1e-12)
    back = orc.rope_neox(y, np.cos(-th), np.sin(-th), "f64")
    np.testing.assert_allclose(back, x, atol=1e-12)
    # the rotation direction: first half gets a*cos - b*sin (angle +th maps (1, 0) to (cos, sin))
    e = np.zeros((1, 1, D))
    e[..., 0] = 1.0
    r = orc.rope_neox(e, np.cos(th[:1]), np.sin(th[:1]), "f64")
    assert r[0, 0, 0] == pytest.approx(np.cos(th[0, 0])) and r[0, 0, D // 2] == pytest.approx(np.sin(th[0, 0]))


@pytest.mark.parametrize("elem", ["bf16", "f16"])
def test_half_tables_equal_duplicated_full_tables(elem):
    rng = np.random.default_rng(5)
    x = _rand((9, 4, 64), elem, rng)
    c = _rand((9, 32), elem, rng)
    s = _rand((9, 32), elem, rng)
    half = orc.rope_neox(x, c, s, elem)
    full = orc.rope_neox(x, np.concatenate([c, c], -1), np.concatenate([s, s], -1), elem)
    np.testing.assert_array_equal(orc.elem_bits(half, elem), orc.elem_bits(full, elem))


def _write(layout, fmt, T=40, QH=4, KH=2, D=64, bs=16, nb=5, seed=0, slots=None):
    rng = np.random.default_rng(seed)
    q = _rand((T, QH, D), "bf16", rng)
    k = _rand((T, KH, D), "bf16", rng)
    v = _rand((T, KH, D), "bf16", rng)
    cos = _rand((100, D // 2), "bf16", rng)
    sin = _rand((100, D // 2), "bf16", rng)
    pos = rng.integers(0, 100, size=T)
    if slots is None:
        slots = rng.permutation(nb * bs)[:T]
    kc, vc = orc.new_caches(nb, bs, KH, D, layout, fmt != "elem")
    ks = vs = None
    if fmt == "fp8_tensor":
        ks, vs = np.float32(0.1), np.float32(0.05)
    elif fmt == "fp8_token":
        ks, vs = np.zeros((nb, KH, bs, 1), np.float32), np.zeros((nb, KH, bs, 1), np.float32)
    qo, ko = orc.fused_rope_cache(q, k, v, pos, cos, sin, slots, kc, vc, elem="bf16", layout=layout,
                                  block_size=bs, fmt=fmt, k_scale=ks, v_scale=vs)
    return dict(q=q, k=k, v=v, pos=pos, cos=cos, sin=sin, slots=slots, kc=kc, vc=vc, qo=qo, ko=ko, ks=ks, vs=vs,
                nb=nb, bs=bs, KH=KH, D=D)


def _token_major(w, layout):
    """Caches -> token-major [nb, H, bs, D] via the layout inverses of oracle/quant.py."""
    if layout == "flash":
        return w["kc"].transpose(0, 2, 1, 3), w["vc"].transpose(0, 2, 1, 3)
    k_tok = oq.k_x_to_tok(w["kc"])
    v4 = w["vc"] if layout == "x4" else oq.v_trans_to_4d(w["vc"])
    return k_tok, oq.v_4d_to_tok(v4)


@pytest.mark.parametrize("layout", orc.LAYOUTS)
def test_layouts_round_trip(layout):
    slots = np.array([3, -1, 17, 79, -5, 40, 33, 1000] + list(range(50, 60)))  # 1000: past the cache
    w = _write(layout, "elem", T=len(slots), slots=slots)
    k_tok, v_tok = _token_major(w, layout)
    written = np.zeros((w["nb"], w["bs"]), bool)
    for t, slot in enumerate(slots):
        if slot < 0 or slot >= w["nb"] * w["bs"]:
            continue
        blk, p = divmod(int(slot), w["bs"])
        written[blk, p] = True
        np.testing.assert_array_equal(k_tok[blk, :, p], orc.elem_bits(w["ko"][t], "bf16"))
        np.testing.assert_array_equal(v_tok[blk, :, p], orc.elem_bits(w["v"][t], "bf16"))
    assert not k_tok.transpose(0, 2, 1, 3)[~written].any()
    assert not v_tok.transpose(0, 2, 1, 3)[~written].any()


@pytest.mark.parametrize("layout", orc.LAYOUTS)
def test_fp8_per_tensor_codes(layout):
    w = _write(layout, "fp8_tensor", seed=1)
    k_tok, v_tok = _token_major(w, layout)
    for t, slot in enumerate(w["slots"]):
        blk, p = divmod(int(slot), w["bs"])
        for h in range(w["KH"]):
            for got, row, s in ((k_tok[blk, h, p], w["ko"][t, h], w["ks"]), (v_tok[blk, h, p], w["v"][t, h], w["vs"])):
                want = (torch.from_numpy(row.astype(np.float32)) * float(orc.reciprocal(s))).to(torch.float8_e4m3fn)
                np.testing.assert_array_equal(got, want.view(torch.uint8).numpy())
                # the reference test's bound: dequantised error <= max|ref| / 8
                err = np.abs(e4m3_decode(got) * s - row).max()
                assert err <= max(1e-3, np.abs(row).max() / 8)


@pytest.mark.parametrize("layout", orc.LAYOUTS)
def test_fp8_per_token_codes_and_scales(layout):
    w = _write(layout, "fp8_token", seed=2)
    k_tok, v_tok = _token_major(w, layout)
    for t, slot in enumerate(w["slots"]):
        blk, p = divmod(int(slot), w["bs"])
        for h in range(w["KH"]):
            for got, row, sc in ((k_tok[blk, h, p], w["ko"][t, h], w["ks"]), (v_tok[blk, h, p], w["v"][t, h], w["vs"])):
                s = sc[blk, h, p, 0]
                assert s == np.float32(np.abs(row).max()) / np.float32(448.0)
                want = (torch.from_numpy(row.astype(np.float32)) / float(s)).to(torch.float8_e4m3fn)
                np.testing.assert_array_equal(got, want.view(torch.uint8).numpy())
                # e4m3 keeps 3 mantissa bits: relative error <= 1/16 above the subnormal range
                deq = e4m3_decode(got) * s
                assert np.all(np.abs(deq - row) <= np.abs(row) / 16 + s * 2.0**-10)
    # untouched scale entries stay zero
    assert (w["ks"] == 0).sum() == w["ks"].size - len(w["slots"]) * w["KH"]


def test_reciprocal_and_low_word():
    assert orc.reciprocal(0.1) == np.float32(10.0)
    assert orc.reciprocal(0.25) == np.float32(4.0)
    rng = np.random.default_rng(0)
    for s in rng.uniform(1e-4, 10, size=200).astype(np.float32):
        r = orc.reciprocal(s)
        # correctly rounded: no float32 neighbour is closer to 1/s
        exact = 1.0 / float(s)
        for nb in (np.nextafter(r, np.float32(np.inf)), np.nextafter(r, np.float32(-np.inf))):
            assert abs(float(r) - exact) <= abs(float(nb) - exact)
    # a device reciprocal, when given, is the one the codes use
    assert orc.reciprocal(3.0, hw=np.float32(0.33333331)) == np.float32(0.33333331)
    np.testing.assert_array_equal(orc.low_word([5, -1, 2**32 + 7, -(2**32) + 3]), [5, -1, 7, 3])
