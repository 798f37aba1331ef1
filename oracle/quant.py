"""KV quantisers and paged KV-cache layouts in numpy (test infrastructure only).

Layouts (all per physical block ``b`` and kv head ``h``):

* token-major   ``x_tok[nb, H, bs, D]``           -- one D-vector per token
* K x-layout    ``k[nb, H, D/16, bs, 16]``        -- 16 consecutive head dims of one
                                                  token in 16 bytes
                                                  (tests/kernels/test_pa.py:189-195)
* V 4-D         ``v[nb, H, D, bs]``               (tests/kernels/test_pa.py:196)
* V trans_v     ``v[nb, H, bs/16, D, 16]``        -- 16 consecutive tokens of one head
                                                  dim in 16 bytes
                                                  (shuffle_value_cache_layout,
                                                  tests/kernels/test_pa.py:419-429)
* per-token scales ``s[nb, H, bs, 1]`` float32   (quantize_kv_cache_symmetric,
                                                  tests/kernels/test_pa.py:334-376)

Parity unpinned: ``per_tensor_quant`` (aiter's quantiser is absent, see there).
"""

from __future__ import annotations

import numpy as np

from .fp8 import E4M3_MAX, e4m3_decode, e4m3_encode


def pertoken_quant(x: np.ndarray, dtype_max: float = E4M3_MAX):
    """Per-row symmetric fp8 quantisation over the last axis.

    Follows tests/utils.py:29-73 (the in-repo analogue of aiter's
    ``pertoken_quant``): nan_to_num, amax = max(max, -min), scale = amax / max
    (0 -> 1), codes = e4m3(x / scale).  Returns (uint8 codes, float32 scales
    with a trailing singleton axis).
    """
    x = np.asarray(x, dtype=np.float32)
    x = np.nan_to_num(x, nan=0.0, posinf=dtype_max, neginf=-dtype_max).astype(np.float32)
    amax = np.maximum(x.max(axis=-1, keepdims=True), -x.min(axis=-1, keepdims=True))
    scale = (amax / np.float32(dtype_max)).astype(np.float32)
    scale[scale == 0] = 1.0
    scale = np.nan_to_num(scale, nan=1.0, posinf=1.0, neginf=1.0).astype(np.float32)
    codes = e4m3_encode((x / scale).astype(np.float32))
    return codes, scale


def per_tensor_quant(x: np.ndarray, dtype_max: float = E4M3_MAX):
    """Single-scale symmetric fp8 quantisation: scale = amax / 448 (0 -> 1).

    aiter's ``per_tensor_quant`` (tests/kernels/test_pa.py:20-26, :408-409) is not
    in the container; this follows the benchmark configurations' definition
    (scale = amax / 448, then the float8_e4m3fn cast).  Parity unpinned: no
    reference output of aiter's quantiser exists here.  The decode kernels consume
    whatever codes and scale they are given, so their parity does not rest on it.
    Returns (uint8 codes, float32 scale of shape [1]).
    """
    x = np.asarray(x, dtype=np.float32)
    amax = np.float32(np.max(np.abs(x))) if x.size else np.float32(0)
    scale = np.float32(amax / np.float32(dtype_max))
    if scale == 0 or not np.isfinite(scale):
        scale = np.float32(1.0)
    codes = e4m3_encode((x / scale).astype(np.float32))
    return codes, np.array([scale], dtype=np.float32)


# ---------------------------------------------------------------- layouts
def k_tok_to_x(k_tok: np.ndarray) -> np.ndarray:
    """[nb, H, bs, D] -> [nb, H, D/16, bs, 16]."""
    nb, h, bs, d = k_tok.shape
    return np.ascontiguousarray(k_tok.reshape(nb, h, bs, d // 16, 16).transpose(0, 1, 3, 2, 4))


def k_x_to_tok(k_x: np.ndarray) -> np.ndarray:
    nb, h, dc, bs, x = k_x.shape
    return np.ascontiguousarray(k_x.transpose(0, 1, 3, 2, 4).reshape(nb, h, bs, dc * x))


def v_tok_to_4d(v_tok: np.ndarray) -> np.ndarray:
    """[nb, H, bs, D] -> [nb, H, D, bs]."""
    return np.ascontiguousarray(v_tok.transpose(0, 1, 3, 2))


def v_4d_to_tok(v4: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(v4.transpose(0, 1, 3, 2))


def v_4d_to_trans(v4: np.ndarray) -> np.ndarray:
    """[nb, H, D, bs] -> [nb, H, bs/16, D, 16] (tests/kernels/test_pa.py:419-429)."""
    nb, h, d, bs = v4.shape
    return np.ascontiguousarray(v4.reshape(nb, h, d, bs // 16, 16).transpose(0, 1, 3, 2, 4))


def v_trans_to_4d(vt: np.ndarray) -> np.ndarray:
    nb, h, g, d, x = vt.shape
    return np.ascontiguousarray(vt.transpose(0, 1, 3, 2, 4).reshape(nb, h, d, g * x))


def quantize_kv_per_token(k_tok: np.ndarray, v_tok: np.ndarray):
    """Per-token-per-head quantisation of token-major K/V.

    Mirrors quantize_kv_cache_symmetric (tests/kernels/test_pa.py:334-376):
    one scale per (block, head, token) over the D axis.  Returns
    (k_x codes, k_scale[nb,H,bs,1], v_4d codes, v_scale[nb,H,bs,1]).
    """
    kq, ks = pertoken_quant(k_tok)
    vq, vs = pertoken_quant(v_tok)
    return k_tok_to_x(kq), ks, v_tok_to_4d(vq), vs


def quantize_kv_per_tensor(k_tok: np.ndarray, v_tok: np.ndarray):
    """Per-tensor quantisation (quantize_kv_cache_per_tensor,
    tests/kernels/test_pa.py:379-416).  Returns (k_x, k_scale[1], v_4d, v_scale[1])."""
    kq, ks = per_tensor_quant(k_tok)
    vq, vs = per_tensor_quant(v_tok)
    return k_tok_to_x(kq), ks, v_tok_to_4d(vq), vs


def scale_flat(scale: np.ndarray, num_blocks: int, num_heads: int, block_size: int) -> np.ndarray:
    """Scales as the reference oracle consumes them: [H, nb*bs]
    (key_scales_flat / expand, tests/kernels/test_pa.py:371-372, :412-413)."""
    scale = np.asarray(scale, dtype=np.float32)
    if scale.size == 1:
        return np.full((num_heads, num_blocks * block_size), scale.reshape(()), dtype=np.float32)
    s = scale.reshape(num_blocks, num_heads, block_size)
    return np.ascontiguousarray(s.transpose(1, 0, 2).reshape(num_heads, num_blocks * block_size))


def dequant_tok(codes_tok: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """Token-major codes [nb,H,bs,D] times their scale(s) -> float32."""
    vals = e4m3_decode(codes_tok)
    s = np.asarray(scale, dtype=np.float32)
    if s.size == 1:
        return vals * s.reshape(())
    return vals * s.reshape(codes_tok.shape[:3] + (1,))
