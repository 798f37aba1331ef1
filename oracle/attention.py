"""Attention oracle in numpy (test infrastructure only).

Restates the reference's torch oracle for the paged decode path:

* ``reference_masked_attention`` -- tests/kernels/test_pa.py:214-274
* ``torch_mha_extend``           -- tests/kernels/test_pa.py:277-331

plus the two pieces of the split-context contract that the decode kernels
expose to callers:

* ``partition_partial`` -- the per-(sequence, kv head, partition) partial
  ``(exp_sum, max_logit, normalised bf16 output)`` written by the small-block
  kernel (kernels/pa_decode_fp8.py:2291-2305, empty slot :2591-2598);
* ``lse_reduce`` -- the log-sum-exp merge of those partials
  (kernels/pa_decode_swa.py:954-1022).
"""

from __future__ import annotations

import math
from typing import Optional

import numpy as np

from .fp8 import bf16_round, e4m3_decode
from .quant import k_x_to_tok, v_4d_to_tok, v_trans_to_4d

CAUSAL_BIAS = np.float32(-3.4e38)  # tests/kernels/test_pa.py:236-238


def reference_masked_attention(
    query: np.ndarray,
    key: np.ndarray,
    value: np.ndarray,
    softmax_scale: float,
    is_causal: bool = True,
    sliding_window: int = 0,
) -> np.ndarray:
    """float32 masked attention; returns float32 [s_q, Hq, D] (before the cast).

    query [s_q, Hq, D]; key/value [s_k, Hkv, D].  q head ``h`` reads kv head
    ``h // (Hq/Hkv)`` (repeat_interleave, tests/kernels/test_pa.py:228-229).
    Causal: key k is visible to query q iff k <= q + (s_k - s_q), masked keys get
    a -3.4e38 bias (:231-239).  Sliding window: with query position
    ``p = s_k - s_q + q`` a key at position k is dropped (-inf) iff
    ``p - k >= sliding_window + 1`` (:241-266).
    """
    q = np.asarray(query, dtype=np.float32)
    k = np.asarray(key, dtype=np.float32)
    v = np.asarray(value, dtype=np.float32)
    s_q, hq, d = q.shape
    s_k, hkv, _ = k.shape
    g = hq // hkv
    qh = q.reshape(s_q, hkv, g, d).transpose(1, 2, 0, 3).reshape(hkv, g * s_q, d)
    kh = k.transpose(1, 2, 0)  # [hkv, d, s_k]
    logits = np.matmul(qh, kh).reshape(hkv, g, s_q, s_k) * np.float32(softmax_scale)
    if is_causal:
        qi = np.arange(s_q)[:, None]
        ki = np.arange(s_k)[None, :]
        masked = ki > qi + (s_k - s_q)
        logits = logits + np.where(masked, CAUSAL_BIAS, np.float32(0.0)).astype(np.float32)
    if sliding_window > 0:
        qpos = np.arange(s_k - s_q, s_k)[:, None]
        kpos = np.arange(s_k)[None, :]
        drop = (qpos - kpos) >= sliding_window + 1
        logits = np.where(drop, np.float32(-np.inf), logits)
    m = logits.max(axis=-1, keepdims=True)
    e = np.exp(logits - m, dtype=np.float32)
    p = e / e.sum(axis=-1, keepdims=True, dtype=np.float32)
    vh = v.transpose(1, 0, 2)  # [hkv, s_k, d]
    out = np.matmul(p.reshape(hkv, g * s_q, s_k), vh).reshape(hkv, g, s_q, d)
    return np.ascontiguousarray(out.transpose(2, 0, 1, 3).reshape(s_q, hq, d))


def gather_sequence(
    k_x: np.ndarray,
    v_cache: np.ndarray,
    block_table_row: np.ndarray,
    context_length: int,
    k_scale: np.ndarray,
    v_scale: np.ndarray,
):
    """Dequantised K/V [ctx, Hkv, D] float32 of one sequence.

    Token ``t`` lives in physical block ``block_table_row[t // bs]`` at slot
    ``t % bs`` (tests/kernels/test_pa.py:302-306); per-token scales are indexed
    [block, head, slot] (:308-314).  ``v_cache`` may be 4-D or trans_v 5-D.
    """
    if v_cache.ndim == 5:
        v_cache = v_trans_to_4d(v_cache)
    nb, hkv, d, bs = v_cache.shape
    t = np.arange(context_length)
    phys = np.asarray(block_table_row, dtype=np.int64)[t // bs]
    slot = t % bs
    # k_x [nb, H, D/16, bs, 16] -> codes [ctx, H, D/16, 16]
    kc = k_x[phys, :, :, slot, :].reshape(context_length, hkv, d)
    vc = v_cache[phys, :, :, slot]  # [ctx, H, D]
    kf = e4m3_decode(kc)
    vf = e4m3_decode(vc)
    ks = np.asarray(k_scale, dtype=np.float32)
    vs = np.asarray(v_scale, dtype=np.float32)
    if ks.size == 1:
        kf = kf * ks.reshape(())
    else:
        kf = kf * ks.reshape(nb, hkv, bs)[phys, :, slot][..., None]
    if vs.size == 1:
        vf = vf * vs.reshape(())
    else:
        vf = vf * vs.reshape(nb, hkv, bs)[phys, :, slot][..., None]
    return kf.astype(np.float32), vf.astype(np.float32)


def torch_mha_extend(
    query: np.ndarray,
    k_x: np.ndarray,
    v_cache: np.ndarray,
    block_tables: np.ndarray,
    context_lengths: np.ndarray,
    query_length: int,
    k_scale: np.ndarray,
    v_scale: np.ndarray,
    sliding_window: int = 0,
    batches: Optional[list] = None,
) -> np.ndarray:
    """Paged decode reference; returns bf16-rounded float32 [B*ql, Hq, D].

    ``query`` holds the (bf16) query values as float32.  ``batches`` restricts
    the computation to a subset of sequences (rows of other sequences are NaN).
    softmax_scale = 1/sqrt(D) as in tests/kernels/test_pa.py:289.
    """
    query = np.asarray(query, dtype=np.float32)
    d = query.shape[-1]
    softmax_scale = 1.0 / (d**0.5)
    bsz = len(context_lengths)
    out = np.full(query.shape, np.nan, dtype=np.float32)
    for b in range(bsz) if batches is None else batches:
        ctx = int(context_lengths[b])
        kf, vf = gather_sequence(k_x, v_cache, block_tables[b], ctx, k_scale, v_scale)
        qb = query[b * query_length : (b + 1) * query_length]
        o = reference_masked_attention(qb, kf, vf, softmax_scale, True, sliding_window)
        out[b * query_length : (b + 1) * query_length] = bf16_round(o)
    return out


# ---------------------------------------------------------- split contract
def visible_token_bounds(context_length: int, query_length: int, qi: int, sliding_window: int):
    """[lo, hi) of keys visible to query ``qi`` of a sequence.

    hi = ctx + 1 - ql + qi (kernels/pa_decode_fp8.py:2646), and with a sliding
    window lo = ctx - ql - sw + qi (kernels/pa_decode_swa.py:1619-1620).
    """
    hi = context_length + 1 - query_length + qi
    lo = context_length - query_length - sliding_window + qi if sliding_window > 0 else 0
    return max(lo, 0), max(hi, 0)


def partition_partial(
    q_rows: np.ndarray,
    k_seq: np.ndarray,
    v_seq: np.ndarray,
    tok_lo: int,
    tok_hi: int,
    context_length: int,
    query_length: int,
    group_size: int,
    softmax_scale: float,
    sliding_window: int = 0,
):
    """Partial of one (sequence, kv head, partition) slot, float64 math.

    q_rows [ql*g, D] (row r = qi*g + gi), k_seq/v_seq [ctx, D] of this kv head.
    Returns (exp_sum[rows], max_logit[rows], out_bf16[rows, D]); a row with no
    visible key in [tok_lo, tok_hi) gets (0, -inf, 0) like an empty slot
    (kernels/pa_decode_fp8.py:2591-2598).
    """
    rows, d = q_rows.shape
    es = np.zeros(rows, dtype=np.float32)
    ml = np.full(rows, -np.inf, dtype=np.float32)
    out = np.zeros((rows, d), dtype=np.float32)
    for r in range(rows):
        qi = r // group_size
        lo, hi = visible_token_bounds(context_length, query_length, qi, sliding_window)
        lo, hi = max(lo, tok_lo), min(hi, tok_hi)
        if hi <= lo:
            continue
        s = (k_seq[lo:hi].astype(np.float64) @ q_rows[r].astype(np.float64)) * softmax_scale
        m = s.max()
        p = np.exp(s - m)
        l = p.sum()
        es[r] = l
        ml[r] = m
        out[r] = bf16_round((p @ v_seq[lo:hi].astype(np.float64) / l).astype(np.float32))
    return es, ml, out


def lse_reduce(exp_sums: np.ndarray, max_logits: np.ndarray, tmp_out: np.ndarray) -> np.ndarray:
    """Merge P partials: out = sum_p w_p * tmp_out_p with
    w_p = s_p e^(m_p - M) / sum_p s_p e^(m_p - M), M = max_p m_p, a zero total
    weight treated as 1 (kernels/pa_decode_swa.py:990-1022).

    exp_sums/max_logits [P, rows], tmp_out [P, rows, D] -> float32 [rows, D].
    Rows where every partial is empty (M = -inf) give 0.
    """
    es = np.asarray(exp_sums, dtype=np.float64)
    ml = np.asarray(max_logits, dtype=np.float64)
    to = np.asarray(tmp_out, dtype=np.float64)
    gmax = ml.max(axis=0)
    safe = np.where(np.isfinite(gmax), gmax, 0.0)
    scale = np.where(np.isfinite(ml), np.exp(ml - safe[None, :]), 0.0)
    w = es * scale
    tot = w.sum(axis=0)
    tot = np.where(tot > 0, tot, 1.0)
    return (np.einsum("pr,prd->rd", w / tot[None, :], to)).astype(np.float32)


def softmax_scale_for(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)


def k_tok_from_x(k_x: np.ndarray) -> np.ndarray:
    return k_x_to_tok(k_x)


def v_tok_from_cache(v_cache: np.ndarray) -> np.ndarray:
    if v_cache.ndim == 5:
        v_cache = v_trans_to_4d(v_cache)
    return v_4d_to_tok(v_cache)
