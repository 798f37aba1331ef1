"""Pins of the oracle's persistent-path restatement (worklist decode + reduce).

* split-then-merge over the get_pa_metadata_v1 schedule equals single-pass
  masked attention (the reference's torch path) for random shapes whose small
  bin counts force splits;
* every partial's log-sum-exp equals scipy's logsumexp of that work's visible
  logits, computed here from the raw keys;
* every output row is written (by a direct work or the reduce) and the partial
  rows the reduce reads are exactly the ones the works wrote;
* planted mistakes (reading the partials without the query_length row offset,
  dropping one partition of a work) are caught by the single-pass comparison.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
from scipy.special import logsumexp

from oracle import attention as oatt
from oracle import planners as oplan

D = 16  # the restatement is independent of head_dim; small keeps the loops fast


def _case(seed, batch, hkv, g, ql, ctx_hi, bins_per_head):
    rng = np.random.default_rng(seed)
    ctx = [int(x) for x in rng.integers(ql, ctx_hi + 1, size=batch)]
    q = rng.standard_normal((batch * ql, hkv * g, D))
    kv = {b: (rng.standard_normal((ctx[b], hkv, D)), rng.standard_normal((ctx[b], hkv, D))) for b in range(batch)}
    num_cu = hkv * bins_per_head
    sq = [b * ql for b in range(batch + 1)]
    md = oplan.get_pa_metadata_v1(sq, ctx, g, hkv, num_cu, 256, ql)
    parts = [oplan.cdiv(c, 256) for c in ctx]
    pind = np.concatenate([[0], np.cumsum(parts)]).astype(np.int32)
    nparts = int(md["reduce_indptr"][-1])
    return dict(ctx=ctx, q=q, kv=kv, md=md, pind=pind, rows=(nparts + 1) * ql, ql=ql, g=g, hkv=hkv, batch=batch)


def _single_pass(c):
    out = np.zeros_like(c["q"])
    ql = c["ql"]
    for b in range(c["batch"]):
        k, v = c["kv"][b]
        out[b * ql : (b + 1) * ql] = oatt.reference_masked_attention(
            c["q"][b * ql : (b + 1) * ql], k, v, 1 / math.sqrt(D), True, 0
        )
    return out


def _worklist(c, work_info=None):
    md = c["md"]
    return oatt.worklist_decode(
        c["q"], lambda b: c["kv"][b], c["ctx"], c["ql"], c["g"], 1 / math.sqrt(D), md["work_indptr"],
        md["work_info"] if work_info is None else work_info, c["pind"], c["rows"],
    )


CASES = [
    # seed, batch, hkv, g, ql, ctx_hi, bins per kv head
    (1, 3, 1, 8, 1, 1027, 3),
    (2, 5, 2, 4, 2, 3000, 3),
    (3, 4, 1, 16, 4, 1500, 5),
    (4, 6, 2, 1, 3, 2600, 7),
    (5, 2, 3, 2, 1, 5000, 11),
    (6, 7, 1, 4, 1, 700, 1),
]


@pytest.mark.parametrize("case", CASES)
def test_split_then_merge_equals_single_pass(case):
    c = _case(*case)
    out, po, pl = _worklist(c)
    md = c["md"]
    ql = c["ql"]
    oatt.reduce_v1(po[ql:], pl[ql:], md["reduce_indptr"], md["reduce_final_map"], md["reduce_partial_map"], ql, out)
    assert not np.isnan(out).any(), "an output row was written by neither a direct work nor the reduce"
    # the single-pass reference computes in float32 (as the reference torch path does)
    np.testing.assert_allclose(out, _single_pass(c), rtol=1e-5, atol=1e-6)


def test_cases_exercise_splits():
    # the comparison above only pins the reduce when works are actually split
    splits = [int(_case(*case)["md"]["reduce_indptr"][-1]) for case in CASES]
    assert all(s > 0 for s in splits[:5]) and splits[5] == 0, splits


@pytest.mark.parametrize("case", CASES[:5])
def test_partial_lse_is_logsumexp_of_visible_logits(case):
    c = _case(*case)
    _, po, pl = _worklist(c)
    md = c["md"]
    ql, g = c["ql"], c["g"]
    winfo = md["work_info"][: int(md["work_indptr"][-1])]
    checked = 0
    for b, ploc, _, _, kv_start, kv_end, _, qhr in winfo.tolist():
        if ploc < 0:
            continue
        h = (qhr & 0xFFFF) // g
        k, _ = c["kv"][b]
        lo = (kv_start - int(c["pind"][b])) * 256
        for qi in range(ql):
            hi = min((kv_end - int(c["pind"][b])) * 256, c["ctx"][b], c["ctx"][b] + 1 - ql + qi)
            for gi in range(g):
                qh = h * g + gi
                logits = [float(np.dot(k[t, h], c["q"][b * ql + qi, qh])) / math.sqrt(D) for t in range(lo, hi)]
                want = logsumexp(logits) if logits else -np.inf
                got = pl[ploc + ql + qi, qh]
                assert (got == want) if not logits else abs(got - want) < 1e-9
                checked += 1
    assert checked > 0


@pytest.mark.parametrize("case", CASES[:4])
def test_planted_mistakes_are_caught(case):
    c = _case(*case)
    md = c["md"]
    ql = c["ql"]
    ref = _single_pass(c)
    # (1) the reduce reading partials without the query_length row offset
    out, po, pl = _worklist(c)
    oatt.reduce_v1(po, pl, md["reduce_indptr"], md["reduce_final_map"], md["reduce_partial_map"], ql, out)
    assert np.isnan(out).any() or not np.allclose(out, ref, atol=1e-6)
    # (2) a work that drops its last partition
    wi = md["work_info"].copy()
    nw = int(md["work_indptr"][-1])
    long = [w for w in range(nw) if wi[w, 5] - wi[w, 4] >= 1 and wi[w, 1] < 0]
    if long:
        wi[long[0], 5] -= 1
        out, po, pl = _worklist(c, wi)
        oatt.reduce_v1(po[ql:], pl[ql:], md["reduce_indptr"], md["reduce_final_map"], md["reduce_partial_map"], ql, out)
        assert not np.allclose(out, ref, atol=1e-6)


def test_reduce_of_one_partial_is_identity():
    rng = np.random.default_rng(0)
    po = rng.standard_normal((6, 3, D))
    pl = rng.standard_normal((6, 3))
    out = np.full((4, 3, D), np.nan)
    # one group of one partial (rows 2..3 with ql 2), one empty group
    lse = oatt.reduce_v1(po, pl, [0, 1, 1], [[1, 3], [0, 0]], [2], 2, out)
    np.testing.assert_allclose(out[1:3], po[2:4])
    np.testing.assert_allclose(lse[1], pl[2])
    assert np.isnan(out[0]).all() and np.isnan(out[3]).all()


def test_reduce_all_empty_partials_gives_zero():
    po = np.ones((2, 1, D))
    pl = np.full((2, 1), -np.inf)
    out = np.full((1, 1, D), np.nan)
    lse = oatt.reduce_v1(po, pl, [0, 2], [[0, 1]], [0, 1], 1, out)
    assert np.all(out == 0.0) and np.isneginf(lse[0]).all()
