"""Integer planners of the paged decode path, restated in Python (test
infrastructure only).

Every function cites the reference lines it restates.  These are the oracle
for the bit-exact partition / block-table / worklist indexing of the HIP path.
"""

from __future__ import annotations

from typing import Callable, Dict, List, Optional, Sequence, Tuple

import numpy as np

KV_COMPUTE_BLOCK = 256  # kernels/pa_decode_fp8.py:36


def cdiv(a: int, b: int) -> int:
    return (a + b - 1) // b


# ------------------------------------------------------------ split counts
def get_recommended_splits(
    num_sequences: int,
    num_kv_heads: int,
    split_kv_blocks: int = 1,
    *,
    sliding_window: int = 0,
    context_partition_size: int = KV_COMPUTE_BLOCK,
    query_length: int = 1,
    num_cu: int = 256,
) -> int:
    """kernels/pa_decode_fp8.py:1922-1949 (CU count passed explicitly)."""
    if sliding_window > 0:
        return cdiv(sliding_window + query_length - 1, context_partition_size) + 1
    num_sm = num_cu * 2
    denom = max(1, num_sequences * num_kv_heads * split_kv_blocks)
    n = cdiv(num_sm, denom) * split_kv_blocks
    return max(4, min(n, 8))


def get_sw_max_context_partition_num(
    sliding_window: int, context_partition_size: int = KV_COMPUTE_BLOCK, query_length: int = 1
) -> int:
    """kernels/pa_decode_swa.py:832-840."""
    if sliding_window <= 0:
        return 0
    return cdiv(sliding_window + query_length - 1, context_partition_size) + 1


# ------------------------------------------------------- partition ranges
def small_block_partition_range(context_length: int, part_idx: int, max_parts: int) -> Tuple[int, int]:
    """256-token partitions [lo, hi) handled by grid slot ``part_idx``.

    kernels/pa_decode_fp8.py:2311-2320: T = ceil(ctx/256), pps = ceil(T/P),
    slot z covers [z*pps, min((z+1)*pps, T)); empty when lo >= hi.
    """
    t = cdiv(context_length, KV_COMPUTE_BLOCK)
    pps = cdiv(t, max_parts) if t > 0 else 0
    lo = part_idx * pps
    hi = min((part_idx + 1) * pps, t)
    return lo, max(lo, hi)


def sw_tail_start_tile(context_length: int, query_length: int, sliding_window: int) -> int:
    """First 256-token tile that any query of the sequence can see
    (kernels/pa_decode_swa.py:1359-1365)."""
    seq_start = max(context_length - query_length - sliding_window, 0)
    return seq_start // KV_COMPUTE_BLOCK


def sw_partition_range(
    context_length: int, part_idx: int, max_parts: int, query_length: int, sliding_window: int
) -> Tuple[int, int]:
    """Tiles [lo, hi) handled by sliding-window grid slot ``part_idx``.

    The reference maps slot z to the single tile ``tail_start_tile + z`` and
    leaves slots with z >= visible tiles empty (kernels/pa_decode_swa.py:1359-1368,
    :1493-1504, :1630-1636).  This build keeps that mapping whenever
    ``max_parts`` covers the visible tiles (always true with the recommended
    count) and otherwise spreads the visible tiles over the slots with the
    small-block rule (pps = ceil(visible / max_parts)), so no tile is dropped.
    """
    t = cdiv(context_length, KV_COMPUTE_BLOCK)
    tail = sw_tail_start_tile(context_length, query_length, sliding_window)
    visible = max(t - tail, 0)
    pps = cdiv(visible, max_parts) if visible > 0 else 0
    lo = tail + part_idx * pps
    hi = min(tail + (part_idx + 1) * pps, t)
    return lo, max(lo, hi)


def partition_token_range(
    context_length: int,
    part_idx: int,
    max_parts: int,
    query_length: int = 1,
    sliding_window: int = 0,
) -> Tuple[int, int]:
    """Token range [lo, hi) of a grid slot (empty when lo == hi)."""
    if sliding_window > 0:
        plo, phi = sw_partition_range(context_length, part_idx, max_parts, query_length, sliding_window)
    else:
        plo, phi = small_block_partition_range(context_length, part_idx, max_parts)
    lo = plo * KV_COMPUTE_BLOCK
    hi = min(phi * KV_COMPUTE_BLOCK, context_length)
    return lo, max(lo, hi)


def token_physical_slot(block_table_row: Sequence[int], token: int, block_size: int) -> Tuple[int, int]:
    """(physical block, slot) of a token (tests/kernels/test_pa.py:302-306;
    kernels/pa_decode_fp8.py:2421-2425 with 256/bs blocks per partition)."""
    return int(block_table_row[token // block_size]), token % block_size


# -------------------------------------------------------------- page data
def build_ps_page_data(block_tables_list: List[List[int]], context_lengths: Sequence[int], block_size: int):
    """kv_page_indices / kv_indptr (tests/kernels/test_pa.py:545-559)."""
    ctx = np.asarray(context_lengths, dtype=np.int64)
    actual = (ctx + block_size - 1) // block_size
    kv_indptr = np.zeros(len(ctx) + 1, dtype=np.int32)
    kv_indptr[1:] = np.cumsum(actual)
    pages: List[int] = []
    for b, n in enumerate(actual.tolist()):
        pages.extend(block_tables_list[b][:n])
    return np.asarray(pages, dtype=np.int32), kv_indptr


# ------------------------------------------------------ worklist scheduler
WORK_INFO_FIELDS = 8


def get_pa_metadata_info_v1(batch_size: int, num_head_k: int = 1, num_cu: int = 256):
    """Buffer shapes (kernels/pa_metadata.py:53-79)."""
    max_work = (batch_size + num_cu - 1) * num_head_k
    max_split_tiles = min(batch_size + num_cu - 1, (num_cu - 1) * 2)
    return (
        ((2,), "uint64"),
        ((num_cu + 1,), "int32"),
        ((max_work, WORK_INFO_FIELDS), "int32"),
        ((batch_size + 1,), "int32"),
        ((batch_size, 2), "int32"),
        ((max_split_tiles,), "int32"),
    )


POISON = -0x5A5A5A5B  # stands for the undefined bytes of torch.empty buffers


def get_pa_metadata_v1(
    seqlens_qo_indptr: Sequence[int],
    context_lens: Sequence[int],
    num_heads_per_head_k: int,
    num_heads_k: int,
    num_cu: int,
    kv_granularity: int = KV_COMPUTE_BLOCK,
    query_length: int = 1,
    quota_of: Optional[Callable[[int, int], int]] = None,
) -> Dict[str, np.ndarray]:
    """Serial CU x batch worklist scheduler (kernels/pa_metadata.py:145-420).

    ``quota_of(i, sum_blocks)``, when given, replaces the reference's even quota of
    bin i of a head (:203-206) -- for schedules that split the partitions
    unevenly over a head's bins; the state machine is otherwise the reference's.

    Buffers start POISON-filled (they are torch.empty in the reference) and are
    written exactly where the reference kernel writes, including its
    overwrite-safe unconditional stores; compare only the valid prefixes
    returned by :func:`metadata_valid_prefixes`.
    """
    assert kv_granularity > 0 and (kv_granularity & (kv_granularity - 1)) == 0  # :108
    assert num_cu % num_heads_k == 0  # :109
    sq = [int(x) for x in seqlens_qo_indptr]
    ctx = [int(x) for x in context_lens]
    nb = len(ctx)
    gqa = num_heads_per_head_k
    nspk = num_cu // num_heads_k
    ql = query_length
    shapes = get_pa_metadata_info_v1(nb, num_heads_k, num_cu)
    work_indptr = np.full(shapes[1][0], POISON, dtype=np.int64)
    work_info = np.full(shapes[2][0], POISON, dtype=np.int64)
    reduce_indptr = np.full(shapes[3][0], POISON, dtype=np.int64)
    reduce_final_map = np.full(shapes[4][0], POISON, dtype=np.int64)
    reduce_partial_map = np.full(shapes[5][0], POISON, dtype=np.int64)

    def num_part(b: int) -> int:
        return cdiv(ctx[b], kv_granularity)

    work_indptr[0] = 0  # :177-178
    reduce_indptr[0] = 0
    sum_blocks = sum(num_part(b) for b in range(nb))  # :180-198
    average, reminder = sum_blocks // nspk, sum_blocks % nspk  # :200-201

    def quota(cid: int) -> int:  # :203-206
        if quota_of is not None:
            return quota_of(cid % nspk, sum_blocks)
        return average + (1 if (cid % nspk) < reminder else 0)

    cid = 0
    num_works = 0
    lri = grt = 0
    for khead in range(num_heads_k):  # :212
        qhr = (((khead + 1) * gqa) << 16) | ((khead * gqa) & 0xFFFF)  # :213-215
        batch = kvblk = nsplit = pidx = kvbeg = 0
        kvend = num_part(0) if nb > 0 else 0
        remain = quota(cid)
        lri = grt = 0
        while cid < num_cu and batch < nb:  # :247-251
            remain_kv = (kvend - kvbeg) - kvblk
            do_finish = remain >= remain_kv
            qo_start, qo_end = sq[batch], sq[batch + 1]
            kv_start = kvbeg + kvblk
            # one work slot is written every iteration (:302-311)
            if do_finish:
                w_ploc = pidx if nsplit > 0 else -1
                w_kv_end = kvend
            else:
                w_ploc = pidx
                w_kv_end = min(kv_start + remain, kvend)
            base = num_works * WORK_INFO_FIELDS
            work_info.reshape(-1)[base : base + 8] = [batch, w_ploc, qo_start, qo_end, kv_start, w_kv_end, 0, qhr]
            # reduce maps (:313-343)
            do_reduce = do_finish and nsplit > 0
            num_splits = nsplit + 1
            reduce_indptr[grt + 1] = lri + num_splits
            reduce_final_map[grt] = [qo_start, qo_end]
            if do_reduce:
                for s in range(num_splits):
                    reduce_partial_map[lri + s] = pidx - (nsplit - s) * ql
            n_lri = lri + (num_splits if do_reduce else 0)
            n_grt = grt + (1 if do_reduce else 0)
            # next state (:270-300, :345-354)
            if do_finish:
                n_cid = cid
                n_pidx = pidx + ql if nsplit > 0 else pidx
                n_nworks = num_works + 1
                n_remain = remain - remain_kv
                n_batch = batch + 1
                n_kvblk = n_nsplit = 0
                n_kvbeg = kvend
                n_kvend = kvend + (num_part(n_batch) if n_batch < nb else 0)
            else:
                emit = remain > 0
                n_cid = cid + 1
                n_pidx = pidx + ql if emit else pidx
                n_nworks = num_works + 1 if emit else num_works
                n_kvblk = kvblk + remain if emit else kvblk
                n_nsplit = nsplit + 1 if emit else nsplit
                n_remain = quota(n_cid)
                n_batch, n_kvbeg, n_kvend = batch, kvbeg, kvend
            work_indptr[cid + 1] = n_nworks  # :356-365 (pre-update cid)
            cid, batch, kvblk, nsplit, num_works = n_cid, n_batch, n_kvblk, n_nsplit, n_nworks
            pidx, kvbeg, kvend, remain, lri, grt = n_pidx, n_kvbeg, n_kvend, n_remain, n_lri, n_grt
        if cid < num_cu:  # :382-387
            cid += 1
    for i in range(cid, num_cu + 1):  # :389-399
        work_indptr[i] = num_works
    for i in range(grt, nb + 1):  # :401-414
        reduce_indptr[i] = lri
    return {
        "work_indptr": work_indptr.astype(np.int32),
        "work_info": work_info.astype(np.int32),
        "reduce_indptr": reduce_indptr.astype(np.int32),
        "reduce_final_map": reduce_final_map.astype(np.int32),
        "reduce_partial_map": reduce_partial_map.astype(np.int32),
        "num_reduce_groups": np.int32(grt),
    }


def get_pa_metadata_packed(
    seqlens_qo_indptr: Sequence[int],
    context_lens: Sequence[int],
    num_heads_per_head_k: int,
    num_heads_k: int,
    num_cu: int,
    kv_granularity: int = KV_COMPUTE_BLOCK,
    query_length: int = 1,
    quota_of: Optional[Callable[[int, int], int]] = None,
) -> Optional[Dict[str, np.ndarray]]:
    """This build's packing schedule (no counterpart in the reference; the device
    version is pa_metadata.hip's pack kernel).  Same buffers and meaning as
    get_pa_metadata_v1, with the same per-bin quotas (``quota_of``, else even),
    but batches are placed whole where they fit:

    * sequences in order of (partitions descending, batch); bins in order of
      (quota descending, bin);
    * rank k < min(bins, B): sequence k goes whole into bin k (the rule below
      guarantees it fits), leaving a gap of quota - partitions;
    * the remaining sequences (ranks >= bins) are poured, in rank order, into the
      gaps in bin-rank order, split at gap boundaries; an empty one becomes one
      empty work in the last bin that has a gap (the last bin if none has);
    * a bin's works: its whole sequence, then its poured pieces in rank order;
    * a sequence with several pieces is split: split sequences form the reduce
      groups in batch order, their pieces taking consecutive partial rows in
      order of position.

    Returns None (the sequential fill applies) unless every sequence of rank
    k < min(bins, B) fits bin k, the total is 1 .. 2^31 - 1 partitions, every
    quota is below 2^19 partitions, no context length is negative, and B, bins
    per head <= 2048.
    """
    sq = [int(x) for x in seqlens_qo_indptr]
    ctx = [int(x) for x in context_lens]
    nb = len(ctx)
    gqa, nhk, ql = num_heads_per_head_k, num_heads_k, query_length
    n = num_cu // nhk
    if nb == 0 or nb > 2048 or n > 2048 or min(ctx) < 0:
        return None
    P = [cdiv(c, kv_granularity) for c in ctx]
    S = sum(P)
    if S < 1 or S > 0x7FFFFFFF:
        return None
    if quota_of is not None:
        Q = [quota_of(c, S) for c in range(n)]
    else:
        Q = [S // n + (1 if c < S % n else 0) for c in range(n)]
    if max(Q) >= 1 << 19:  # (the device ranks by 31-bit keys)
        return None
    order = sorted(range(nb), key=lambda b: (-P[b], b))
    bins = sorted(range(n), key=lambda c: (-Q[c], c))
    m = min(n, nb)
    if any(P[order[k]] > Q[bins[k]] for k in range(m)):
        return None
    works = [[] for _ in range(n)]  # (batch, p0, p1) in partitions of the batch
    gap = [0] * n  # by bin rank
    for k in range(n):
        c = bins[k]
        if k < m:
            works[c].append((order[k], 0, P[order[k]]))
            gap[k] = Q[c] - P[order[k]]
        else:
            gap[k] = Q[c]
    positive = [k for k in range(n) if gap[k] > 0]
    zero_bin = bins[positive[-1]] if positive else bins[n - 1]
    gi, room = 0, (gap[positive[0]] if positive else 0)
    pieces = {}
    for k in range(m, nb):
        b = order[k]
        if P[b] == 0:
            works[zero_bin].append((b, 0, 0))
            continue
        s = 0
        while s < P[b]:
            while room == 0:
                gi += 1
                room = gap[positive[gi]]
            take = min(room, P[b] - s)
            works[bins[positive[gi]]].append((b, s, s + take))
            room -= take
            s += take
    for c in range(n):
        for (b, p0, _) in works[c]:
            pieces.setdefault(b, []).append(p0)
    split = [b for b in range(nb) if len(pieces[b]) > 1]
    pidx_of, red_indptr, red_final, red_partial, base = {}, [0], [], [], 0
    for b in split:
        for p0 in sorted(pieces[b]):
            pidx_of[(b, p0)] = ql * base
            red_partial.append(ql * base)
            base += 1
        red_indptr.append(base)
        red_final.append((sq[b], sq[b + 1]))
    pind = [0]
    for x in P:
        pind.append(pind[-1] + x)
    W = sum(len(w) for w in works)
    work_indptr = np.zeros(num_cu + 1, dtype=np.int64)
    work_info = np.zeros((nhk * W, WORK_INFO_FIELDS), dtype=np.int64)
    row = 0
    for kh in range(nhk):
        qhr = (((kh + 1) * gqa) << 16) | ((kh * gqa) & 0xFFFF)
        for c in range(n):
            for (b, p0, p1) in works[c]:
                work_info[row] = [b, pidx_of.get((b, p0), -1), sq[b], sq[b + 1], pind[b] + p0, pind[b] + p1, 0, qhr]
                row += 1
            work_indptr[kh * n + c + 1] = row
    reduce_indptr = np.full(nb + 1, base, dtype=np.int64)
    reduce_indptr[: len(red_indptr)] = red_indptr
    return {
        "work_indptr": work_indptr.astype(np.int32),
        "work_info": work_info.astype(np.int32),
        "reduce_indptr": reduce_indptr.astype(np.int32),
        "reduce_final_map": np.array(red_final, dtype=np.int32).reshape(-1, 2),
        "reduce_partial_map": np.array(red_partial, dtype=np.int32),
        "num_reduce_groups": np.int32(len(split)),
    }


def metadata_valid_prefixes(md: Dict[str, np.ndarray]) -> Dict[str, np.ndarray]:
    """The bytes the reference defines: work_indptr (all), work_info up to
    work_indptr[-1], reduce_indptr (all), reduce_final_map up to the reduce
    group count, reduce_partial_map up to reduce_indptr[-1]."""
    nw = int(md["work_indptr"][-1])
    ngroups = int(md["num_reduce_groups"])
    nparts = int(md["reduce_indptr"][-1])
    return {
        "work_indptr": md["work_indptr"],
        "work_info": md["work_info"][:nw],
        "reduce_indptr": md["reduce_indptr"],
        "reduce_final_map": md["reduce_final_map"][:ngroups],
        "reduce_partial_map": md["reduce_partial_map"][:nparts],
    }
