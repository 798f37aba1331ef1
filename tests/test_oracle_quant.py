"""Pins the quantisers (tests/utils.py:29-73 semantics, amax/448) and the paged
layouts (tests/kernels/test_pa.py:189-211, 419-429) by element-wise brute force."""

import numpy as np
import torch

from oracle import fp8 as ofp8
from oracle import quant as oq


def test_pertoken_quant_scale_and_extremes():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 7, 128)).astype(np.float32)
    x[0, 0] = 0.0
    codes, scale = oq.pertoken_quant(x)
    assert scale.shape == (5, 7, 1)
    assert scale[0, 0, 0] == 1.0  # all-zero row -> scale 1
    amax = np.abs(x).max(-1, keepdims=True)
    np.testing.assert_array_equal(scale[1:], (amax / np.float32(448.0))[1:])
    dec = ofp8.E4M3_DECODE[codes]
    # the largest magnitude of each row lands on +-448 exactly
    assert np.all(np.abs(dec[1:]).max(-1) == 448.0)
    # |x/scale - decode| within half an e4m3 ulp (relative 1/16), subnormals absolute 2**-10
    err = np.abs(x / scale - dec)
    bound = np.maximum(np.abs(dec) / 16.0, 2.0**-10)
    assert np.all(err <= bound + 1e-6)


def test_pertoken_quant_matches_torch_formula():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 4, 128)).astype(np.float32) * 3
    codes, scale = oq.pertoken_quant(x)
    xt = torch.from_numpy(x)
    amax = torch.maximum(xt.amax(-1, keepdim=True), -xt.amin(-1, keepdim=True))
    st = amax / torch.finfo(torch.float8_e4m3fn).max
    qt = (xt / st).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(scale, st.numpy())
    np.testing.assert_array_equal(codes, qt)


def test_per_tensor_quant():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 2, 16, 128)).astype(np.float32)
    codes, scale = oq.per_tensor_quant(x)
    assert scale.shape == (1,) and scale[0] == np.float32(np.abs(x).max() / np.float32(448.0))
    assert np.abs(ofp8.E4M3_DECODE[codes]).max() == 448.0
    z, s0 = oq.per_tensor_quant(np.zeros((2, 2), np.float32))
    assert s0[0] == 1.0 and np.all(z == 0)


def test_layouts_elementwise():
    rng = np.random.default_rng(3)
    nb, h, bs, d = 3, 2, 64, 128
    t = rng.integers(0, 255, size=(nb, h, bs, d), dtype=np.uint8)
    kx = oq.k_tok_to_x(t)
    v4 = oq.v_tok_to_4d(t)
    vt = oq.v_4d_to_trans(v4)
    assert kx.shape == (nb, h, d // 16, bs, 16) and vt.shape == (nb, h, bs // 16, d, 16)
    for (b, hh, tok, dd) in [(0, 0, 0, 0), (2, 1, 63, 127), (1, 0, 17, 33), (1, 1, 40, 100)]:
        assert kx[b, hh, dd // 16, tok, dd % 16] == t[b, hh, tok, dd]
        assert v4[b, hh, dd, tok] == t[b, hh, tok, dd]
        assert vt[b, hh, tok // 16, dd, tok % 16] == t[b, hh, tok, dd]
    assert np.array_equal(oq.k_x_to_tok(kx), t)
    assert np.array_equal(oq.v_4d_to_tok(oq.v_trans_to_4d(vt)), t)


def test_trans_v_matches_reference_shuffle_semantics():
    """shuffle_value_cache_layout = view(nb,h,d,bs/16,16).permute(0,1,3,2,4)."""
    rng = np.random.default_rng(4)
    v4 = rng.integers(0, 255, size=(2, 3, 128, 32), dtype=np.uint8)
    t = torch.from_numpy(v4).view(2, 3, 128, 2, 16).permute(0, 1, 3, 2, 4).contiguous().numpy()
    assert np.array_equal(oq.v_4d_to_trans(v4), t)


def test_scale_flat_layout():
    s = np.arange(2 * 3 * 4, dtype=np.float32).reshape(2, 3, 4, 1)
    f = oq.scale_flat(s, 2, 3, 4)
    assert f.shape == (3, 8)
    assert f[1, 4 + 2] == s[1, 1, 2, 0]
    assert np.all(oq.scale_flat(np.array([0.5], np.float32), 2, 3, 4) == 0.5)
