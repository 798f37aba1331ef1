"""GPU parity of the persistent (worklist) path: pa_decode_ps_launch on block
sizes other than 16 / 64 runs the worklist kernel over get_pa_metadata's
schedule, then the merge of split works (the reference's pa_reduce_v1 step).

Outputs are checked against the CPU oracle (atol 2e-2 / rtol 2e-2, bf16), and
every partial row the kernel writes against the oracle's per-work restatement
(pa_testlib.check_worklist_partials), which pins the work -> token range
mapping exactly.
"""

from __future__ import annotations


import numpy as np
import pytest
import torch

from flydsl_amd.workloads import CONFIGS, build_workload, scaled
from oracle import attention as oatt
from tests.pa_testlib import check_worklist_partials, compare_outputs, launch, metadata_with_bins, schedule_of

pytestmark = pytest.mark.gpu


def _spread(n: int, k: int):
    if n <= k:
        return list(range(n))
    return sorted({round(i * (n - 1) / (k - 1)) for i in range(k)})


# The reference's own persistent-path case set (tests/kernels/test_pa.py:1180-1205):
# 1024-token pages, heads (8,1) and (16,1), ql 1..4, ctx 1027 fixed or U[ql, 1027],
# batch 3 and 81, per-token and per-tensor scales.
@pytest.mark.parametrize("heads", [(8, 1), (16, 1)])
@pytest.mark.parametrize("ql", [1, 2, 3, 4])
@pytest.mark.parametrize("varlen", [False, True])
@pytest.mark.parametrize("batch", [3, 81])
@pytest.mark.parametrize("quant", ["per_token", "per_tensor"])
def test_reference_normal_accuracy_cases(heads, ql, varlen, batch, quant):
    hq, hkv = heads
    cfg = scaled(CONFIGS["c2"], name="normal_accuracy", batch=batch, num_q_heads=hq, num_kv_heads=hkv,
                 block_size=1024, query_length=ql, per_token=quant == "per_token",
                 ctx_kind="uniform" if varlen else "fixed", ctx_a=ql if varlen else 1027, ctx_b=1027)
    print(f"[worklist] heads {heads} ql {ql} varlen {varlen} batch {batch} {quant}", flush=True)
    w = build_workload(cfg, "cuda", seed=123)
    out, tag, _ = launch(w)
    assert tag == "ps_split_reduce"
    compare_outputs(w, out, range(batch) if batch <= 3 else _spread(batch, 9))


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c5"])
def test_baseline_configs_with_metadata(name):
    """The benchmark configurations (16 / 64-token pages) through the small-block
    path with get_pa_metadata's schedule, which runs the worklist kernel."""
    from flydsl_amd import get_pa_metadata

    cfg = CONFIGS[name]
    print(f"[worklist] {name} with metadata: {cfg.description}", flush=True)
    w = build_workload(cfg, "cuda")
    md = get_pa_metadata(w["query"], w["key_cache"], w["context_lengths"], w["kv_indptr"], cfg.num_q_heads,
                         cfg.num_kv_heads)
    assert md["uniform_context"] == (len(set(w["context_list"])) == 1)
    md["uniform_context"] = False  # run the worklist kernel on every config, c2 included
    out, tag, _ = launch(w, metadata=md)
    assert tag == "ps_small_block"
    # every sequence: the split ones (their rows come from the merge) and the whole ones
    split = split_sequences(schedule_of(md))
    print(f"[worklist] {name}: {len(split)} split sequences", flush=True)
    compare_outputs(w, out, range(cfg.batch))


def split_sequences(sched):
    """Batches with a work that writes partials (partial_qo_loc >= 0)."""
    nw = int(sched["work_indptr"][-1])
    info = sched["work_info_flat"][: 8 * nw].view(nw, 8).cpu().numpy()
    return {int(b) for b, p in zip(info[:, 0], info[:, 1]) if p >= 0}


# The reference's second case set (tests/kernels/test_pa.py:1207-1233, named
# sliding_window_accuracy; its window option is 0): 16- and 1024-token pages,
# heads (8,1) / (16,1), ql 1-4, per-token scales, context lengths U[ql, 8192],
# batch 128, uniform(-1, 1) draws, block tables drawn with replacement
# (:713-716).  Called as the reference's harness calls the launcher: the
# metadata of get_pa_metadata, max_context_partition_num 8 (:852-856) and the
# flat page list; 16-token pages also without metadata (the reference's
# small-block kernel ignores it).
@pytest.mark.parametrize("bs", [16, 1024])
@pytest.mark.parametrize("heads", [(8, 1), (16, 1)])
@pytest.mark.parametrize("ql", [1, 2, 3, 4])
def test_reference_sliding_window_accuracy_cases(bs, heads, ql):
    from flydsl_amd import get_pa_metadata

    hq, hkv = heads
    cfg = scaled(CONFIGS["c3"], name="sliding_window_accuracy", batch=128, num_q_heads=hq, num_kv_heads=hkv,
                 block_size=bs, query_length=ql, per_token=True, ctx_kind="uniform", ctx_a=ql, ctx_b=8192,
                 dist="uniform", bt_replace=True, num_physical_blocks=128 * ((16384 + bs - 1) // bs))
    print(f"[worklist] sliding_window_accuracy bs {bs} heads {heads} ql {ql}", flush=True)
    w = build_workload(cfg, "cuda", seed=123)
    md = get_pa_metadata(w["query"], w["key_cache"], w["context_lengths"], w["kv_indptr"], hq, hkv)
    out, tag, _ = launch(w, max_parts=8, metadata=md)
    assert tag == ("ps_small_block" if bs == 16 else "ps_split_reduce")
    check = sorted(set(_spread(cfg.batch, 12)) | set(sorted(split_sequences(schedule_of(md)))[:12]))
    compare_outputs(w, out, check)
    if bs == 16:
        out2, _, _ = launch(w, max_parts=8)  # the partition kernel, as the reference's small-block route
        compare_outputs(w, out2, _spread(cfg.batch, 12))


@pytest.mark.parametrize("name", ["c3", "c5"])
def test_dispatch_round_bin_remap_is_a_permutation(name):
    """get_pa_metadata's weighted schedule run with its workgroups remapped by
    dispatch round (bin_groups) and with workgroup c on bin c: each work runs
    exactly once either way and a work's arithmetic does not depend on the
    workgroup, so the outputs are bit-identical."""
    from flydsl_amd import get_pa_metadata

    cfg = CONFIGS[name]
    print(f"[worklist] {name} bin remap", flush=True)
    w = build_workload(cfg, "cuda")
    md = get_pa_metadata(w["query"], w["key_cache"], w["context_lengths"], w["kv_indptr"], cfg.num_q_heads,
                         cfg.num_kv_heads)
    md["uniform_context"] = False
    if md["tuned"]["bin_groups"] <= 1:
        pytest.skip("the device's CU count does not split into whole groups of bins")
    out_remap, _, _ = launch(w, metadata=md)
    out_plain, _, _ = launch(w, metadata=dict(md, tuned=dict(md["tuned"], bin_groups=0)))
    assert torch.equal(out_remap, out_plain)
    compare_outputs(w, out_remap, _spread(cfg.batch, 4))


WORKLIST_CASES = {
    "bs16_tok_g4": dict(base="c3", batch=6, ctx_kind="uniform", ctx_a=1, ctx_b=3000),
    "bs16_pt_mtp2_g8": dict(base="c2", batch=4, num_q_heads=16, num_kv_heads=2, query_length=2, ctx_kind="uniform",
                            ctx_a=2, ctx_b=2500),
    "bs64_tok_mtp4_g16": dict(base="c5", batch=3, ctx_kind="uniform", ctx_a=4, ctx_b=1500),
    "bs1024_tok": dict(base="c3", batch=3, block_size=1024, ctx_kind="uniform", ctx_a=1, ctx_b=2100),
    "bs32_ql2_g8": dict(base="c2", batch=3, num_q_heads=16, num_kv_heads=2, block_size=32, query_length=2,
                        ctx_kind="uniform", ctx_a=2, ctx_b=1200),
    "bs128_g1": dict(base="c2", batch=3, num_q_heads=4, num_kv_heads=4, block_size=128, ctx_kind="uniform",
                     ctx_a=1, ctx_b=900),
    "bs256_tok_mtp4_g16": dict(base="c5", batch=4, block_size=256, ctx_kind="uniform", ctx_a=4, ctx_b=3000),
    "bs512_mtp3_g4": dict(base="c2", batch=5, block_size=512, query_length=3, ctx_kind="uniform", ctx_a=3,
                          ctx_b=4000),
    "bs16_long_mtp4_g16": dict(base="c5", batch=2, block_size=16, ctx_kind="uniform", ctx_a=17000, ctx_b=40000),
    "bs64_long_mtp4_g16": dict(base="c5", batch=2, ctx_kind="uniform", ctx_a=16500, ctx_b=30000),
    "bs1024_long": dict(base="c2", batch=2, num_q_heads=16, num_kv_heads=2, block_size=1024, ctx_kind="uniform",
                        ctx_a=9000, ctx_b=20000),
    # one kv head: at one bin per head get_pa_metadata_info_v1 sizes reduce_partial_map to 0 entries
    "bs64_hkv1_mtp2_g8": dict(base="c5", batch=4, num_q_heads=8, num_kv_heads=1, query_length=2,
                              ctx_kind="uniform", ctx_a=2, ctx_b=2500),
    "bs256_hkv1_g1": dict(base="c2", batch=5, num_q_heads=1, num_kv_heads=1, block_size=256, ctx_kind="uniform",
                          ctx_a=1, ctx_b=3000),
}


@pytest.mark.parametrize("case", sorted(WORKLIST_CASES))
@pytest.mark.parametrize("bins_per_head", [1, 3, 16, 0, -1])
def test_worklist_partials_and_outputs(case, bins_per_head):
    """Ragged shapes over schedules with few bins (many splits), with
    get_pa_metadata's tuned schedule (bins_per_head 0) and with the reference's
    schedule it returns under the reference's keys (-1): every output row and
    every partial row checked."""
    kw = dict(WORKLIST_CASES[case])
    cfg = scaled(CONFIGS[kw.pop("base")], name=case, **kw)
    print(f"[worklist] {case} bins/head {bins_per_head}", flush=True)
    w = build_workload(cfg, "cuda", seed=7)
    if bins_per_head > 0:
        md = metadata_with_bins(w, bins_per_head * cfg.num_kv_heads)
    else:
        from flydsl_amd import get_pa_metadata

        md = get_pa_metadata(w["query"], w["key_cache"], w["context_lengths"], w["kv_indptr"], cfg.num_q_heads,
                             cfg.num_kv_heads, tuned=bins_per_head == 0)
        md["uniform_context"] = False
        sched = schedule_of(md)
        sched["partial_output"].fill_(float("nan"))
        sched["partial_lse"].fill_(float("nan"))
    out, tag, _ = launch(w, metadata=md)
    assert tag == ("ps_small_block" if cfg.block_size in (16, 64) else "ps_split_reduce")
    compare_outputs(w, out, range(cfg.batch))
    n = check_worklist_partials(w, schedule_of(md))
    if bins_per_head == 1:
        assert n == 0  # one bin per head holds every sequence whole: direct writes only
    print(f"[worklist] {case}: {n} partial rows checked", flush=True)


def test_worklist_output_dtypes_and_f16_query():
    cfg = scaled(CONFIGS["c3"], name="dtypes", batch=3, block_size=1024, query_length=2, ctx_kind="uniform",
                 ctx_a=2, ctx_b=3000)
    w = build_workload(cfg, "cuda", seed=11)
    md = metadata_with_bins(w, 2 * cfg.num_kv_heads)
    for dt in (torch.float32, torch.float16):
        out, tag, _ = launch(w, out_dtype=dt, metadata=md)
        assert out.dtype == dt and tag == "ps_split_reduce"
        compare_outputs(w, out, range(cfg.batch))
    out, _, _ = launch(w, query=w["query"].to(torch.float16), metadata=md)
    compare_outputs(w, out, range(cfg.batch))


def test_plan_cache_does_not_reuse_internal_metadata():
    """Without ``metadata`` the launcher schedules from the current context
    lengths on every call; changing them in place must change the schedule."""
    cfg = scaled(CONFIGS["c2"], name="recache", batch=4, block_size=1024, ctx_kind="uniform", ctx_a=1, ctx_b=4000)
    w = build_workload(cfg, "cuda", seed=5)
    out1, _, _ = launch(w)
    compare_outputs(w, out1, range(cfg.batch))
    shorter = [max(1, c // 3) for c in w["context_list"]]
    w["context_lengths"].copy_(torch.tensor(shorter, dtype=torch.int32))
    w["context_list"] = shorter
    out2, _, _ = launch(w)
    compare_outputs(w, out2, range(cfg.batch))


@pytest.mark.parametrize("hq", [8, 12])
@pytest.mark.parametrize("aligned", [True, False], ids=["vec16", "offset8"])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_pa_reduce_v1_api(out_dtype, aligned, hq):
    """The reduce on synthetic partials vs the oracle merge, with final_lse.  Groups
    of 0-19 partials (more than one batch of eight), head counts that are and are
    not multiples of 8, and partial rows offset by 8 bytes (the element-pair path)."""
    from flydsl_amd import pa_reduce_v1

    rng = np.random.default_rng(3)
    ql, groups = 2, 6
    counts = [0, 3, 1, 7, 2, 19]  # partials per group (0: a group with nothing to merge)
    nparts = sum(counts)
    rows = nparts * ql + 3
    po = rng.standard_normal((rows, 1, hq, 128)).astype(np.float32)
    pl = (rng.standard_normal((rows, 1, hq, 1)) * 4).astype(np.float32)
    pl[5, 0, 3, 0] = -np.inf  # an empty partial inside a group
    ri = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    rpm = (rng.permutation(nparts) * ql).astype(np.int32)
    rfm = np.array([[g * ql, (g + 1) * ql] for g in range(groups)], dtype=np.int32)
    dev = torch.device("cuda:0")
    out = torch.full((groups * ql, hq, 128), 7.0, dtype=out_dtype, device=dev)
    lse = torch.full((groups * ql, hq), 7.0, device=dev)
    t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    po_t = t(po)
    if not aligned:  # same values, data pointer 8 bytes past a 16-byte boundary
        buf = torch.empty(po.size + 2, dtype=torch.float32, device=dev)
        po_t = buf[2:].view(po.shape)
        po_t.copy_(t(po))
        assert po_t.data_ptr() % 16 == 8
    pa_reduce_v1(po_t, t(pl), t(ri), t(rfm), t(rpm), ql, out, lse)
    torch.cuda.synchronize()
    exp = np.full((groups * ql, hq, 128), 7.0)
    exp_lse = oatt.reduce_v1(po[:, 0], pl[:, 0, :, 0], ri, rfm, rpm, ql, exp)
    got = out.float().cpu().numpy()
    tol = 1e-5 if out_dtype == torch.float32 else 1e-2
    np.testing.assert_allclose(got, exp, atol=tol, rtol=tol)
    got_lse = lse.cpu().numpy()
    for row, v in exp_lse.items():
        np.testing.assert_allclose(got_lse[row], v, atol=1e-5, rtol=1e-5)
    assert np.all(got_lse[0:ql] == 7.0)  # group 0 has no partials: untouched
