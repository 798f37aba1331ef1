"""CPU restatement of the fused NeoX RoPE + paged KV-cache writer (test infrastructure only).

Follows kernels/fused_rope_cache_kernel.py:106-429 and the reference test's
torch model of it, ``_rope_ref`` (tests/kernels/test_fused_rope_cache.py:166-235):

* rotation (NeoX, rotary_dim == D): head dim d pairs with d + D/2;
  ``out[d] = r(r(x[d]*c) - r(x[d+D/2]*s))`` and
  ``out[d+D/2] = r(r(x[d+D/2]*c') + r(x[d]*s'))`` where ``r`` rounds to the
  element dtype (bf16 / f16, round to nearest even) after every product and
  after the sum, as the reference's element-dtype arithmetic does (:214-247);
  ``(c, s) = cos/sin[pos, d]``, ``(c', s')`` the same for half-width tables
  (``reuse_freqs_front_part``, :190) or ``cos/sin[pos, d + D/2]`` for full ones;
* cache write (:252-429): tokens with ``slot >= 0`` go to block ``slot // bs``,
  position ``slot % bs``; K receives the rotated key, V the value;
* fp8 per-tensor (:270-296): codes of ``x * rcp`` (float32 product) with
  ``rcp = v_rcp_f32(scale)``, the hardware reciprocal (:282-283) -- see
  ``reciprocal``;
* fp8 per-token (this build's extension for the decode kernels' per-token
  format): ``pertoken_quant`` of each (token, kv head) vector.

Layouts (``layout``): "flash" K/V [nb, bs, H, D]; "x4" K [nb, H, D/16, bs, 16]
+ V [nb, H, D, bs]; "x5" K as "x4" + V [nb, H, bs/16, D, 16] (trans_v).

Pins (tests/test_oracle_rope_cache.py): torch's own bf16 / f16 arithmetic on
the reference test's formula; closed forms of plane rotations in float64
(identity, quarter turn, norm preservation, angle addition); layout inverses;
the fp8 codec's pins against torch's float8_e4m3fn cast.  The reference has no
golden vectors for this kernel.
"""

from __future__ import annotations

import numpy as np

from .fp8 import E4M3_MAX, bf16_round, e4m3_encode, f32_to_bf16_bits
from .quant import pertoken_quant

ELEMS = ("bf16", "f16", "f64")
LAYOUTS = ("flash", "x4", "x5")


def round_elem(x, elem: str) -> np.ndarray:
    """Round to the element dtype (values returned as float32; 'f64' = exact float64)."""
    if elem == "bf16":
        return bf16_round(np.asarray(x, dtype=np.float32))
    if elem == "f16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
    if elem == "f64":
        return np.asarray(x, dtype=np.float64)
    raise ValueError(elem)


def elem_bits(x, elem: str) -> np.ndarray:
    """float32 values of the element dtype -> their uint16 bit patterns."""
    if elem == "bf16":
        return f32_to_bf16_bits(x)
    if elem == "f16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)
    raise ValueError(elem)


def rope_neox(x, cos_rows, sin_rows, elem: str, round_steps: bool = True) -> np.ndarray:
    """NeoX rotation of ``x[T, H, D]`` by per-token tables ``cos_rows / sin_rows [T, D/2 or D]``.

    ``round_steps=False`` rounds only the final result (a planted mistake the
    pins must catch).  kernels/fused_rope_cache_kernel.py:214-247.
    """
    ftype = np.float64 if elem == "f64" else np.float32
    x = np.asarray(x, dtype=ftype)
    D = x.shape[-1]
    half = D // 2
    cos_rows = np.asarray(cos_rows, dtype=ftype)[:, None, :]
    sin_rows = np.asarray(sin_rows, dtype=ftype)[:, None, :]
    if cos_rows.shape[-1] == half:
        c1 = c2 = cos_rows
        s1 = s2 = sin_rows
    elif cos_rows.shape[-1] == D:
        c1, c2 = cos_rows[..., :half], cos_rows[..., half:]
        s1, s2 = sin_rows[..., :half], sin_rows[..., half:]
    else:
        raise ValueError("cos/sin rows must have D/2 or D columns")
    a, b = x[..., :half], x[..., half:]
    r = (lambda v: round_elem(v, elem)) if round_steps else (lambda v: v)
    first = round_elem(r(a * c1) - r(b * s1), elem)
    second = round_elem(r(b * c2) + r(a * s2), elem)
    return np.concatenate([first, second], axis=-1)


def reciprocal(scale, hw=None) -> np.float32:
    """The reciprocal the reference multiplies by: ``v_rcp_f32(scale)`` (:282-283).

    v_rcp_f32 is a hardware approximation within 1 ulp of 1/scale whose last bit
    no published formula fixes, so a checker passes the device's own value as
    ``hw`` (read back through ``pa_fp8_hw_reciprocal``); its 1-ulp bound and the
    scales where it is exact are pinned in tests/test_gpu_rope_cache.py.
    Without ``hw`` this is 1/scale correctly rounded, which v_rcp_f32 equals at
    powers of two and at the scales the CPU tests use (0.1 among them).
    """
    if hw is not None:
        return np.float32(hw)
    return np.float32(np.float32(1.0) / np.float32(scale))


def low_word(idx) -> np.ndarray:
    """int64 index tensors are read through their low 32-bit word (:182-186, :253-258)."""
    return (np.asarray(idx, dtype=np.int64) & 0xFFFFFFFF).astype(np.uint32).view(np.int32).astype(np.int64)


def new_caches(num_blocks: int, block_size: int, num_kv_heads: int, head_dim: int, layout: str, fp8: bool):
    """Zeroed K / V caches of ``layout`` (uint8 codes for fp8, uint16 bit patterns otherwise)."""
    dt = np.uint8 if fp8 else np.uint16
    nb, bs, H, D = num_blocks, block_size, num_kv_heads, head_dim
    if layout == "flash":
        return np.zeros((nb, bs, H, D), dt), np.zeros((nb, bs, H, D), dt)
    k = np.zeros((nb, H, D // 16, bs, 16), dt)
    if layout == "x4":
        return k, np.zeros((nb, H, D, bs), dt)
    if layout == "x5":
        return k, np.zeros((nb, H, bs // 16, D, 16), dt)
    raise ValueError(layout)


def _put(cache, kind: str, layout: str, blk: int, pos: int, h: int, row):
    D = row.shape[-1]
    if layout == "flash":
        cache[blk, pos, h, :] = row
    elif kind == "k":
        cache[blk, h, :, pos, :] = row.reshape(D // 16, 16)
    elif layout == "x4":
        cache[blk, h, :, pos] = row
    else:
        cache[blk, h, pos // 16, :, pos % 16] = row


def fused_rope_cache(
    q, k, v, positions, cos, sin, slots, key_cache, value_cache, *,
    elem: str, layout: str, block_size: int, fmt: str = "elem", k_scale=None, v_scale=None,
    k_rcp=None, v_rcp=None,
):
    """Restatement of one launch; returns (q_out, k_out) and writes the caches in place.

    q [T, QH, D], k / v [T, KH, D]: float32 values of ``elem``; positions /
    slots: per-token ints (already low-word decoded); cos / sin [max_pos, cols].
    ``fmt``: "elem" (caches hold uint16 bit patterns), "fp8_tensor" (uint8
    codes, ``k_scale`` / ``v_scale`` scalars) or "fp8_token" (uint8 codes,
    ``k_scale`` / ``v_scale`` arrays [nb, KH, bs, 1] written at each slot).
    ``k_rcp`` / ``v_rcp``: the device's v_rcp_f32 of the per-tensor scales
    (``reciprocal``).
    """
    T = q.shape[0]
    positions = np.clip(np.asarray(positions, dtype=np.int64)[:T], 0, cos.shape[0] - 1)
    cos_rows, sin_rows = np.asarray(cos)[positions], np.asarray(sin)[positions]
    q_out = rope_neox(q, cos_rows, sin_rows, elem)
    k_out = rope_neox(k, cos_rows, sin_rows, elem)
    nb = key_cache.shape[0]
    KH = k.shape[1]
    for t in range(T):
        slot = int(slots[t])
        if slot < 0 or slot // block_size >= nb:
            continue
        blk, pos = slot // block_size, slot % block_size
        for h in range(KH):
            krow, vrow = k_out[t, h], np.asarray(v[t, h], dtype=np.float32)
            if fmt == "elem":
                kc, vc = elem_bits(krow, elem), elem_bits(vrow, elem)
            elif fmt == "fp8_tensor":
                kc = e4m3_encode((krow * reciprocal(k_scale, k_rcp)).astype(np.float32))
                vc = e4m3_encode((vrow * reciprocal(v_scale, v_rcp)).astype(np.float32))
            elif fmt == "fp8_token":
                kc, ks = pertoken_quant(krow, E4M3_MAX)
                vc, vs = pertoken_quant(vrow, E4M3_MAX)
                k_scale[blk, h, pos, 0] = ks[0]
                v_scale[blk, h, pos, 0] = vs[0]
            else:
                raise ValueError(fmt)
            _put(key_cache, "k", layout, blk, pos, h, kc)
            _put(value_cache, "v", layout, blk, pos, h, vc)
    return q_out, k_out
