"""Integer planners of the decode path: split counts, partition ranges,
sliding-window tiles, page data and the get_pa_metadata_v1 worklist.

Pinned by brute-force enumeration, invariants and a hand-worked example; the
Python and plain-C restatements of the scheduler are cross-checked bit-exact."""

import ctypes
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle import planners as op

ROOT = Path(__file__).resolve().parents[1]


# ------------------------------------------------------------- split counts
def test_recommended_splits_baseline_values():
    # MI355X: 256 CUs. Values of the five benchmark configurations.
    assert op.get_recommended_splits(4, 2, 16, num_cu=256) == 8
    assert op.get_recommended_splits(64, 8, 16, num_cu=256) == 8
    assert op.get_recommended_splits(128, 8, 16, num_cu=256) == 8
    assert op.get_recommended_splits(256, 4, 4, num_cu=256) == 4
    assert op.get_recommended_splits(32, 8, sliding_window=4096, query_length=1) == 17
    # the harness passes (sliding_window, 256, ql) positionally: seqs=0 -> denominator 1 -> 8
    assert op.get_recommended_splits(0, 256, 1, num_cu=256) == 8


def test_recommended_splits_clamp_and_form():
    for seqs in (0, 1, 3, 17, 64, 1000):
        for heads in (1, 2, 8):
            for split in (1, 4, 16):
                n = op.get_recommended_splits(seqs, heads, split, num_cu=256)
                assert 4 <= n <= 8
                raw = -(-512 // max(1, seqs * heads * split)) * split
                assert n == max(4, min(raw, 8))


def test_sw_partition_count_bounds_visible_tiles():
    for sw in (1, 100, 255, 256, 257, 4096):
        for ql in (1, 2, 4):
            bound = op.get_sw_max_context_partition_num(sw, 256, ql)
            assert bound == op.get_recommended_splits(1, 1, sliding_window=sw, query_length=ql)
            worst = 0
            for ctx in range(1, sw + ql + 2 * 256 + 3):
                tail = op.sw_tail_start_tile(ctx, ql, sw)
                worst = max(worst, op.cdiv(ctx, 256) - tail)
            assert worst <= bound  # every visible tile gets a slot
            assert worst >= bound - 1
    assert op.get_sw_max_context_partition_num(0) == 0


# --------------------------------------------------------- partition ranges
@pytest.mark.parametrize("max_parts", [1, 2, 3, 5, 8, 16])
def test_small_block_ranges_tile_exactly(max_parts):
    for ctx in list(range(0, 1200, 7)) + [4096, 4097, 32768]:
        t = op.cdiv(ctx, 256)
        covered = []
        pps = op.cdiv(t, max_parts) if t else 0
        seen_empty = False
        for z in range(max_parts):
            lo, hi = op.small_block_partition_range(ctx, z, max_parts)
            if lo == hi:
                seen_empty = True
                continue
            assert not seen_empty, "non-empty slot after an empty one"
            assert hi - lo <= pps
            covered.extend(range(lo, hi))
        assert covered == list(range(t))


def test_token_ranges_cover_visible_keys_once():
    for sw in (0, 50, 300):
        for ql in (1, 3):
            for ctx in range(ql, 900, 13):
                for parts in (1, 2, 4, 17):
                    toks = []
                    for z in range(parts):
                        lo, hi = op.partition_token_range(ctx, z, parts, ql, sw)
                        toks.extend(range(lo, hi))
                    assert len(toks) == len(set(toks))
                    need = set()
                    for qi in range(ql):
                        from oracle.attention import visible_token_bounds

                        a, b = visible_token_bounds(ctx, ql, qi, sw)
                        need.update(range(a, b))
                    assert need <= set(toks)
                    assert all(t < ctx for t in toks)


def test_sw_slots_match_reference_tile_mapping():
    """With the recommended slot count the mapping is tile tail+z, one tile each
    (kernels/pa_decode_swa.py:1359-1368)."""
    sw, ql = 4096, 1
    parts = op.get_sw_max_context_partition_num(sw, 256, ql)
    for ctx in (8192, 8193, 9000, 20000, 32768, 100, 4096, 4097):
        tail = op.sw_tail_start_tile(ctx, ql, sw)
        t = op.cdiv(ctx, 256)
        for z in range(parts):
            lo, hi = op.sw_partition_range(ctx, z, parts, ql, sw)
            if tail + z < t:
                assert (lo, hi) == (tail + z, tail + z + 1)
            else:
                assert lo == hi


def test_token_physical_slot():
    row = [7, 3, 9]
    assert op.token_physical_slot(row, 0, 16) == (7, 0)
    assert op.token_physical_slot(row, 17, 16) == (3, 1)
    assert op.token_physical_slot(row, 47, 16) == (9, 15)


def test_build_ps_page_data():
    tables = [[5, 6, 7, 8], [1, 2, 3, 4], [9, 10, 11, 12]]
    pages, indptr = op.build_ps_page_data(tables, [17, 1, 48], 16)
    assert indptr.tolist() == [0, 2, 3, 6]
    assert pages.tolist() == [5, 6, 1, 9, 10, 11]


# ----------------------------------------------------------- worklist
def test_metadata_info_shapes():
    info = op.get_pa_metadata_info_v1(128, 8, 768)
    assert [s for s, _ in info] == [(2,), (769,), (7160, 8), (129,), (128, 2), (895,)]


def test_metadata_hand_worked_example():
    """num_cu 4, 2 kv heads (2 bins each), ctx [300, 1000, 100] -> partitions
    [2, 4, 1] (sum 7, quota 4/3 by bin parity); worked by hand from the
    scheduler rules (kernels/pa_metadata.py:203-399)."""
    md = op.get_pa_metadata_v1([0, 1, 2, 3], [300, 1000, 100], 4, 2, 4, 256, 1)
    v = op.metadata_valid_prefixes(md)
    q0, q1 = (4 << 16) | 0, (8 << 16) | 4
    assert v["work_indptr"].tolist() == [0, 2, 4, 6, 8]
    assert v["work_info"].tolist() == [
        [0, -1, 0, 1, 0, 2, 0, q0],
        [1, 0, 1, 2, 2, 4, 0, q0],
        [1, 1, 1, 2, 4, 6, 0, q0],
        [2, -1, 2, 3, 6, 7, 0, q0],
        [0, -1, 0, 1, 0, 2, 0, q1],
        [1, 0, 1, 2, 2, 4, 0, q1],
        [1, 1, 1, 2, 4, 6, 0, q1],
        [2, -1, 2, 3, 6, 7, 0, q1],
    ]
    assert v["reduce_indptr"].tolist() == [0, 2, 2, 2]
    assert v["reduce_final_map"].tolist() == [[1, 2]]
    assert v["reduce_partial_map"].tolist() == [0, 1]


def _check_invariants(md, ctx, gqa, nhk, num_cu, gran, ql):
    v = op.metadata_valid_prefixes(md)
    wi = v["work_indptr"]
    assert wi[0] == 0 and np.all(np.diff(wi) >= 0)
    works = v["work_info"]
    assert len(works) == wi[-1]
    parts = [op.cdiv(c, gran) for c in ctx]
    starts = np.concatenate([[0], np.cumsum(parts)])
    total = int(starts[-1])
    nspk = num_cu // nhk
    avg, rem = total // nspk, total % nspk
    for cid in range(num_cu):
        load = sum(int(w[5] - w[4]) for w in works[wi[cid] : wi[cid + 1]])
        assert load <= avg + (1 if cid % nspk < rem else 0)
    for kh in range(nhk):
        qhr = (((kh + 1) * gqa) << 16) | ((kh * gqa) & 0xFFFF)
        hw = [w for w in works if w[7] == qhr]
        cover = []
        for w in hw:
            b = int(w[0])
            assert (w[2], w[3]) == (b * ql, (b + 1) * ql)
            assert starts[b] <= w[4] < w[5] <= starts[b + 1]
            cover.extend(range(int(w[4]), int(w[5])))
            nworks_b = sum(1 for x in hw if x[0] == b)
            assert (w[1] == -1) == (nworks_b == 1)
        assert cover == [t for b in range(len(ctx)) for t in range(int(starts[b]), int(starts[b + 1]))]


@pytest.mark.parametrize("seed", range(12))
def test_metadata_invariants_random(seed):
    rng = np.random.default_rng(seed)
    nhk = int(rng.choice([1, 2, 4, 8]))
    num_cu = nhk * int(rng.integers(1, 40))
    b = int(rng.integers(1, 60))
    ctx = [int(x) for x in rng.integers(1, 9000, size=b)]
    ql = int(rng.integers(1, 5))
    gqa = int(rng.choice([1, 4, 8]))
    md = op.get_pa_metadata_v1([i * ql for i in range(b + 1)], ctx, gqa, nhk, num_cu, 256, ql)
    _check_invariants(md, ctx, gqa, nhk, num_cu, 256, ql)


# ------------------------------------------------ C restatement agreement
@pytest.fixture(scope="module")
def c_oracle():
    so = ROOT / "oracle" / "_build" / "libpa_oracle.so"
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
    lib = ctypes.CDLL(str(so))
    P = ctypes.POINTER(ctypes.c_int32)
    lib.pa_metadata_v1_ref.argtypes = [P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int, P, P, ctypes.c_int, P, P, P, ctypes.c_int, P]
    lib.pa_metadata_v1_ref.restype = ctypes.c_int
    return lib


def run_c_metadata(lib, sq, ctx, gqa, nhk, num_cu, gran, ql):
    info = op.get_pa_metadata_info_v1(len(ctx), nhk, num_cu)
    arr = lambda shape: np.full(shape, op.POISON, dtype=np.int32)  # noqa: E731
    wi, winfo, ri, rfm, rpm = arr(info[1][0]), arr(info[2][0]), arr(info[3][0]), arr(info[4][0]), arr(info[5][0])
    ng = np.zeros(1, np.int32)
    P = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))  # noqa: E731
    sqa, ca = np.asarray(sq, np.int32), np.asarray(ctx, np.int32)
    rc = lib.pa_metadata_v1_ref(P(sqa), P(ca), len(ctx), gqa, nhk, num_cu, gran, ql, P(wi), P(winfo),
                                info[2][0][0], P(ri), P(rfm), P(rpm), info[5][0][0], P(ng))
    assert rc == 0
    return {"work_indptr": wi, "work_info": winfo, "reduce_indptr": ri, "reduce_final_map": rfm,
            "reduce_partial_map": rpm, "num_reduce_groups": ng[0]}


@pytest.mark.parametrize("seed", range(40))
def test_c_and_python_schedulers_agree(c_oracle, seed):
    rng = np.random.default_rng(100 + seed)
    nhk = int(rng.choice([1, 2, 4, 8]))
    num_cu = nhk * int(rng.integers(1, 100))
    b = int(rng.integers(1, 140))
    hi = int(rng.choice([300, 5000, 33000]))
    ctx = [int(x) for x in rng.integers(1, hi, size=b)]
    ql = int(rng.integers(1, 5))
    gqa = int(rng.choice([1, 4, 16]))
    gran = int(rng.choice([16, 256, 1024]))
    sq = [i * ql for i in range(b + 1)]
    py = op.metadata_valid_prefixes(op.get_pa_metadata_v1(sq, ctx, gqa, nhk, num_cu, gran, ql))
    cc = op.metadata_valid_prefixes(run_c_metadata(c_oracle, sq, ctx, gqa, nhk, num_cu, gran, ql))
    for key in py:
        np.testing.assert_array_equal(py[key], cc[key], err_msg=key)


def test_c3_shaped_schedule(c_oracle):
    """The benchmark's ragged shape: 128 sequences, 8 kv heads, 768 bins."""
    from flydsl_amd.workloads import CONFIGS, context_lengths_for

    ctx = context_lengths_for(CONFIGS["c3"])
    sq = list(range(129))
    md = op.get_pa_metadata_v1(sq, ctx, 4, 8, 768, 256, 1)
    _check_invariants(md, ctx, 4, 8, 768, 256, 1)
    cc = run_c_metadata(c_oracle, sq, ctx, 4, 8, 768, 256, 1)
    for key, val in op.metadata_valid_prefixes(md).items():
        np.testing.assert_array_equal(val, op.metadata_valid_prefixes(cc)[key])


def test_scheduler_with_uneven_quotas_covers_every_partition_once():
    """get_pa_metadata_v1 with per-bin quotas (quota_of): every head's works still
    cover each partition exactly once, in order, and each bin takes exactly its
    quota; with the reference's even quota passed explicitly the schedule is the
    reference's."""
    rng = np.random.default_rng(5)
    for _ in range(40):
        b = int(rng.integers(1, 200))
        nhk = int(rng.choice([1, 2, 4]))
        nspk = int(rng.integers(1, 30))
        ctx = [int(x) for x in rng.integers(1, 6000, size=b)]
        total = sum((c + 255) // 256 for c in ctx)
        if total < nspk:
            continue
        w = [int(x) for x in rng.integers(1, 5, size=nspk)]
        cw = np.concatenate([[0], np.cumsum(w)])

        def quota(i, s, cw=cw):
            return s * int(cw[i + 1]) // int(cw[-1]) - s * int(cw[i]) // int(cw[-1])

        md = op.get_pa_metadata_v1(list(range(b + 1)), ctx, 4, nhk, nspk * nhk, 256, 1, quota_of=quota)
        v = op.metadata_valid_prefixes(md)
        info, wi = v["work_info"], v["work_indptr"]
        for k in range(nhk):
            rows = info[(info[:, 7] & 0xFFFF) == 4 * k]
            assert (rows[:, 4] == np.concatenate([[0], rows[:-1, 5]])).all()  # contiguous, in order
            assert rows[-1, 5] == total
            for i in range(nspk):  # bin i of head k holds its quota
                c = k * nspk + i
                got = int((info[wi[c]:wi[c + 1], 5] - info[wi[c]:wi[c + 1], 4]).sum())
                assert got == quota(i, total)
        even = op.get_pa_metadata_v1(list(range(b + 1)), ctx, 4, nhk, nspk * nhk, 256, 1,
                                     quota_of=lambda i, s: s // nspk + (1 if i < s % nspk else 0))
        ref = op.get_pa_metadata_v1(list(range(b + 1)), ctx, 4, nhk, nspk * nhk, 256, 1)
        for key, val in op.metadata_valid_prefixes(ref).items():
            np.testing.assert_array_equal(op.metadata_valid_prefixes(even)[key], val)


# ------------------------------------------------ packing schedule (this build's own)
def _packed_case(rng):
    nhk = int(rng.choice([1, 2, 3, 4, 8]))
    nspk = int(rng.choice([1, 2, 5, 16, 64, 192]))
    b = int(rng.choice([1, 3, 40, 256, 700]))
    kind = rng.choice(["uniform", "narrow", "zeros", "equal"])
    if kind == "uniform":
        ctx = [int(x) for x in rng.integers(1, int(rng.choice([600, 9000])), size=b)]
    elif kind == "narrow":
        lo = int(rng.integers(1000, 4000))
        ctx = [int(x) for x in rng.integers(lo, 2 * lo, size=b)]
    elif kind == "zeros":
        ctx = [int(x) if rng.random() < 0.7 else 0 for x in rng.integers(1, 5000, size=b)]
    else:
        ctx = [int(rng.integers(1, 9000))] * b
    ws = [int(x) for x in rng.integers(90, 140, size=int(rng.choice([1, 2, 3])))]
    weights = sorted(ws, reverse=True) if nspk % len(ws) == 0 and len(ws) > 1 else None
    return nhk, nspk, b, ctx, weights


def _quota_fn(weights, nspk):
    if weights is None:
        return None
    m = nspk // len(weights)
    wc = lambda i: sum(w * min(max(i - g * m, 0), m) for g, w in enumerate(weights))  # noqa: E731

    def quota(i, total):
        return total * wc(i + 1) // wc(nspk) - total * wc(i) // wc(nspk)

    return quota


@pytest.mark.parametrize("seed", range(60))
def test_packing_schedule_invariants(seed):
    """The packing schedule (get_pa_metadata's tuned schedule where it applies),
    checked against what it must be rather than against a second copy of it:
    every partition of every sequence runs exactly once per head, every bin holds
    exactly its quota, sequence rank k < min(bins, B) runs whole in bin rank k (the
    rank orders recomputed here), a sequence is split exactly when it has several
    works and then takes consecutive partial rows in position order, reduce groups
    follow batch order, and the buffers' bounds hold.  When it does not apply, some
    rank k sequence is larger than its bin."""
    rng = np.random.default_rng(7000 + seed)
    nhk, nspk, b, ctx, weights = _packed_case(rng)
    ql, gqa = int(rng.integers(1, 5)), int(rng.choice([1, 4, 16]))
    num_cu = nhk * nspk
    sq = [i * ql for i in range(b + 1)]
    qf = _quota_fn(weights, nspk)
    md = op.get_pa_metadata_packed(sq, ctx, gqa, nhk, num_cu, 256, ql, quota_of=qf)
    P = [(c + 255) // 256 for c in ctx]
    S = sum(P)
    Q = [qf(c, S) for c in range(nspk)] if qf else [S // nspk + (1 if c < S % nspk else 0) for c in range(nspk)]
    order = sorted(range(b), key=lambda x: (-P[x], x))
    bins = sorted(range(nspk), key=lambda c: (-Q[c], c))
    m = min(nspk, b)
    if md is None:
        assert S < 1 or any(P[order[k]] > Q[bins[k]] for k in range(m))
        return
    assert all(P[order[k]] <= Q[bins[k]] for k in range(m))
    v = op.metadata_valid_prefixes(md)
    info, wi = v["work_info"], v["work_indptr"]
    pind = np.concatenate([[0], np.cumsum(P)])
    W = int(wi[nspk])
    max_work, max_split = (b + num_cu - 1) * nhk, min(b + num_cu - 1, 2 * (num_cu - 1))
    assert nhk * W <= max_work and int(v["reduce_indptr"][-1]) <= max_split
    works_of = {}
    for k in range(nhk):
        qhr = (((k + 1) * gqa) << 16) | ((k * gqa) & 0xFFFF)
        cover = np.zeros(S, np.int64)
        for c in range(nspk):
            rows = info[wi[k * nspk + c]:wi[k * nspk + c + 1]]
            assert (rows[:, 7] == qhr).all()
            assert int((rows[:, 5] - rows[:, 4]).sum()) == Q[c]  # the bin's quota
            for r in rows:
                bb = int(r[0])
                assert pind[bb] <= r[4] <= r[5] <= pind[bb + 1] and r[2] == sq[bb] and r[3] == sq[bb + 1]
                cover[r[4]:r[5]] += 1
                if k == 0:
                    works_of.setdefault(bb, []).append((int(r[4]), int(r[1]), c))
        assert (cover == 1).all()  # every partition exactly once
        assert int(wi[(k + 1) * nspk]) == (k + 1) * W
    for k in range(m):  # rank k runs whole in bin rank k
        bb = order[k]
        assert works_of[bb] == [(int(pind[bb]), -1, bins[k])]
    split = [bb for bb in range(b) if len(works_of[bb]) > 1]
    assert int(md["num_reduce_groups"]) == len(split)
    nxt = 0
    for g, bb in enumerate(split):  # groups in batch order, consecutive partial rows by position
        pieces = sorted(works_of[bb])
        assert [p for (_, p, _) in pieces] == [ql * (nxt + i) for i in range(len(pieces))]
        assert list(v["reduce_partial_map"][v["reduce_indptr"][g]:v["reduce_indptr"][g + 1]]) == \
            [p for (_, p, _) in pieces]
        assert tuple(v["reduce_final_map"][g]) == (sq[bb], sq[bb + 1])
        nxt += len(pieces)
    for bb in range(b):
        if len(works_of[bb]) == 1:
            assert works_of[bb][0][1] == -1
    assert int(v["reduce_indptr"][0]) == 0 and (md["reduce_indptr"][len(split):] == nxt).all()


def test_packing_schedule_benchmark_shapes():
    """c5's shape packs (fewer split works than the sequential fill over the same
    weighted quotas); c3's does not apply (its longest sequences outgrow every bin)."""
    from flydsl_amd.workloads import CONFIGS, context_lengths_for

    ctx = context_lengths_for(CONFIGS["c5"])
    qf = _quota_fn([115, 107, 100], 192)
    sq = [4 * i for i in range(len(ctx) + 1)]
    packed = op.get_pa_metadata_packed(sq, ctx, 16, 4, 768, 256, 4, quota_of=qf)
    seq = op.get_pa_metadata_v1(sq, ctx, 16, 4, 768, 256, 4, quota_of=qf)
    assert packed is not None
    split = lambda md: int((op.metadata_valid_prefixes(md)["work_info"][:, 1] >= 0).sum())  # noqa: E731
    assert split(packed) == 984 and split(seq) == 1520
    ctx3 = context_lengths_for(CONFIGS["c3"])
    assert op.get_pa_metadata_packed(list(range(129)), ctx3, 4, 8, 512, 256, 1,
                                     quota_of=_quota_fn([105, 100], 64)) is None


def test_packing_schedule_hand_example():
    """Two bins of 5 partitions, sequences of 4, 3 and 3 partitions: the 4 goes whole
    to bin 0, a 3 whole to bin 1, and the last 3 is poured into bin 0's 1 left and
    bin 1's 2 left (split, partial rows 0 and ql); its group is the only one."""
    gran = 256
    ctx = [3 * gran, 4 * gran, 3 * gran]  # batch 1 is the largest; batches 0 and 2 tie (batch order)
    md = op.get_pa_metadata_packed([0, 1, 2, 3], ctx, 1, 1, 2, gran, 1)
    v = op.metadata_valid_prefixes(md)
    # pind = [0, 3, 7, 10]; rank order: batch 1 (4), batch 0 (3), batch 2 (3)
    assert v["work_indptr"].tolist() == [0, 2, 4]
    assert v["work_info"][:, [0, 1, 4, 5]].tolist() == [[1, -1, 3, 7], [2, 0, 7, 8], [0, -1, 0, 3], [2, 1, 8, 10]]
    assert v["reduce_indptr"].tolist() == [0, 2, 2, 2]
    assert v["reduce_final_map"].tolist() == [[2, 3]] and v["reduce_partial_map"].tolist() == [0, 1]
