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
  (kernels/pa_decode_swa.py:954-1022);

and the two halves of the persistent (worklist) path:

* ``worklist_decode`` -- per-work semantics of ``pa_decode_metadata_kenrel``
  (kernels/pa_decode_fp8.py:941-1721): direct rows or f32 partial rows plus
  their log-sum-exp;
* ``reduce_v1`` -- the merge of split works' partials that the reference
  delegates to aiter's ``pa_reduce_v1`` (call site kernels/pa_decode_fp8.py:3189-3200).
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


# ---------------------------------------------------------- worklist path
def range_attention(q_row, k_seq, v_seq, lo: int, hi: int, softmax_scale: float):
    """Softmax attention of one query row over keys [lo, hi), float64.

    Returns (l, m, o): exp sum relative to the max logit m (natural log units)
    and the normalised output; (0, -inf, zeros) when the range is empty.
    """
    d = v_seq.shape[-1]
    if hi <= lo:
        return 0.0, -np.inf, np.zeros(d, dtype=np.float64)
    s = (k_seq[lo:hi].astype(np.float64) @ np.asarray(q_row, dtype=np.float64)) * softmax_scale
    m = float(s.max())
    p = np.exp(s - m)
    l = float(p.sum())
    return l, m, (p @ v_seq[lo:hi].astype(np.float64)) / l


def worklist_decode(
    query: np.ndarray,
    seq_kv,
    context_lengths,
    query_length: int,
    group_size: int,
    softmax_scale: float,
    work_indptr,
    work_info,
    partition_indptr,
    partial_rows: int,
    partition_size: int = 256,
):
    """What the persistent decode writes for a worklist (kernels/pa_decode_fp8.py:941-1721).

    ``seq_kv(b)`` returns the dequantised (K, V) [ctx, Hkv, D] of sequence b.
    Workgroup c runs works [work_indptr[c], work_indptr[c+1]); work
    ``[batch, ploc, qo_start, qo_end, kv_start, kv_end, _, qhr]`` attends the
    keys of partitions [kv_start - partition_indptr[batch], kv_end - ...) of its
    sequence (256 tokens each, :1150-1166) under the causal bound
    tok < ctx + 1 - ql + qi (:1338-1341), for every query head of kv head
    ``(qhr & 0xffff) // g`` (:1168-1170).  ploc < 0 writes the normalised row to
    out[qo_start + qi, qhead]; ploc >= 0 writes it (f32) to partial row
    ploc + ql + qi with lse = m + log(l) (:1612-1643; l = 0 gives -inf).

    Returns (out [B*ql, Hq, D], partial_output [partial_rows, Hq, D],
    partial_lse [partial_rows, Hq]) as float64, NaN where nothing was written.
    """
    q = np.asarray(query, dtype=np.float64)
    rows, hq, d = q.shape
    out = np.full((rows, hq, d), np.nan)
    po = np.full((partial_rows, hq, d), np.nan)
    pl = np.full((partial_rows, hq), np.nan)
    wi = np.asarray(work_indptr, dtype=np.int64)
    winfo = np.asarray(work_info, dtype=np.int64).reshape(-1, 8)
    pind = np.asarray(partition_indptr, dtype=np.int64)
    cache = {}
    for c in range(len(wi) - 1):
        for w in range(int(wi[c]), int(wi[c + 1])):
            b, ploc, qo_start, _, kv_start, kv_end, _, qhr = (int(x) for x in winfo[w])
            h = (qhr & 0xFFFF) // group_size
            ctx = int(context_lengths[b])
            if b not in cache:
                cache[b] = seq_kv(b)
            k_seq, v_seq = cache[b]
            tok_lo = (kv_start - int(pind[b])) * partition_size
            tok_hi = min((kv_end - int(pind[b])) * partition_size, ctx)
            for qi in range(query_length):
                bound = ctx + 1 - query_length + qi
                for gi in range(group_size):
                    qhead = h * group_size + gi
                    l, m, o = range_attention(q[b * query_length + qi, qhead], k_seq[:, h], v_seq[:, h],
                                              max(tok_lo, 0), min(tok_hi, bound), softmax_scale)
                    if ploc < 0:
                        out[qo_start + qi, qhead] = o
                    else:
                        po[ploc + query_length + qi, qhead] = o
                        pl[ploc + query_length + qi, qhead] = m + math.log(l) if l > 0 else -np.inf
    return out, po, pl


def reduce_v1(partial_output, partial_lse, reduce_indptr, reduce_final_map, reduce_partial_map, max_qlen: int, out):
    """Merge of split works' partials into ``out`` in place (the role of aiter's
    pa_reduce_v1, called at kernels/pa_decode_fp8.py:3189-3200 on
    ``partial_output[ql:]``).  For group g with partials j in
    [reduce_indptr[g], reduce_indptr[g+1]) and rows s_j = reduce_partial_map[j] + qi:
    out[qo_start + qi, h] = sum_j exp(lse_j - LSE) * partial_j, LSE = log sum_j exp(lse_j);
    a row whose partials are all -inf gets 0.  Returns the merged LSE per written
    (row, head) as a dict.
    """
    po = np.asarray(partial_output, dtype=np.float64)
    pl = np.asarray(partial_lse, dtype=np.float64)
    ri = np.asarray(reduce_indptr, dtype=np.int64)
    fm = np.asarray(reduce_final_map, dtype=np.int64).reshape(-1, 2)
    pm = np.asarray(reduce_partial_map, dtype=np.int64)
    lses = {}
    for g in range(len(ri) - 1):
        j0, j1 = int(ri[g]), int(ri[g + 1])
        if j0 >= j1:
            continue
        qo_start, qo_end = int(fm[g, 0]), int(fm[g, 1])
        for qi in range(min(qo_end - qo_start, max_qlen)):
            srows = pm[j0:j1] + qi
            lse = pl[srows]  # [n, Hq]
            mx = lse.max(axis=0)
            safe = np.where(np.isfinite(mx), mx, 0.0)
            wgt = np.where(np.isfinite(lse), np.exp(lse - safe[None, :]), 0.0)
            tot = wgt.sum(axis=0)
            inv = np.where(tot > 0, 1.0 / np.where(tot > 0, tot, 1.0), 0.0)
            out[qo_start + qi] = np.einsum("nh,nhd->hd", wgt * inv[None, :], po[srows])
            lses[qo_start + qi] = np.where(tot > 0, safe + np.log(np.where(tot > 0, tot, 1.0)), -np.inf)
    return lses


def softmax_scale_for(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)


def k_tok_from_x(k_x: np.ndarray) -> np.ndarray:
    return k_x_to_tok(k_x)


def v_tok_from_cache(v_cache: np.ndarray) -> np.ndarray:
    if v_cache.ndim == 5:
        v_cache = v_trans_to_4d(v_cache)
    return v_4d_to_tok(v_cache)
