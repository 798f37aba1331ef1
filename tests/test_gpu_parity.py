"""GPU parity: the HIP decode path vs the CPU oracle on identical seeded inputs.

Tolerance is the north-star contract: bf16 outputs within atol 2e-2 / rtol 2e-2
of the oracle (restatement of the reference's torch path), partition indexing
exact (see pa_testlib.check_partials).
"""

from __future__ import annotations

import math

import pytest
import torch

from flydsl_amd.workloads import CONFIGS, build_workload, scaled
from tests.pa_testlib import check_partials, compare_outputs, launch

pytestmark = pytest.mark.gpu


def _spread(n: int, k: int):
    if n <= k:
        return list(range(n))
    return sorted({round(i * (n - 1) / (k - 1)) for i in range(k)})


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
def test_baseline_config_outputs(name):
    """Every benchmark configuration at full size, every sequence against the oracle
    (the reference counts any mismatching element, tests/kernels/test_pa.py:626-641)."""
    cfg = CONFIGS[name]
    print(f"[parity] {name}: {cfg.description}", flush=True)
    w = build_workload(cfg, "cuda")
    out, tag, _ = launch(w)
    # one slot per sequence under a window is the reference's "fused" variant
    assert tag in (("ps_sw_partitioned", "ps_sw_fused_partitioned") if cfg.sliding_window else ("ps_small_block",))
    worst = compare_outputs(w, out, range(cfg.batch))
    print(f"[parity] {name}: max |diff| {worst:.3e}", flush=True)


SMALL_CASES = {
    "bs16_pt_g4": dict(base="c2", batch=5, ctx_kind="uniform", ctx_a=1, ctx_b=3000),
    "bs16_tok_g4": dict(base="c3", batch=6, ctx_kind="uniform", ctx_a=1, ctx_b=3000),
    "bs64_tok_mtp4_g16": dict(base="c5", batch=3, ctx_kind="uniform", ctx_a=4, ctx_b=1500),
    "sw_small": dict(base="c4", batch=4, sliding_window=300, ctx_kind="uniform", ctx_a=1, ctx_b=2000),
    "sw_mtp": dict(base="c4", batch=4, sliding_window=100, query_length=3, ctx_kind="uniform", ctx_a=3, ctx_b=900),
    # block sizes other than 16 / 64 reach the partition kernel through a window
    # (without one they run the worklist path, tests/test_gpu_worklist.py)
    "sw_ql2_g8_bs32": dict(base="c4", batch=3, num_q_heads=16, num_kv_heads=2, block_size=32, query_length=2,
                           sliding_window=700, ctx_kind="uniform", ctx_a=2, ctx_b=1200),
    "sw_g1_bs128": dict(base="c4", batch=3, num_q_heads=4, num_kv_heads=4, block_size=128, sliding_window=500,
                        ctx_kind="uniform", ctx_a=1, ctx_b=900),
    "sw_bs1024_tok": dict(base="c3", batch=3, block_size=1024, sliding_window=1500, ctx_kind="uniform", ctx_a=1,
                          ctx_b=2100),
    "mtp2_pt": dict(base="c2", batch=3, num_q_heads=16, num_kv_heads=2, query_length=4, ctx_kind="uniform",
                    ctx_a=4, ctx_b=1500),
    "mtp2_tok": dict(base="c3", batch=3, num_q_heads=16, num_kv_heads=2, query_length=4, ctx_kind="uniform",
                     ctx_a=4, ctx_b=1500),
    "mtp3_tok": dict(base="c5", batch=3, query_length=3, ctx_kind="uniform", ctx_a=3, ctx_b=1500),
    "mtp4_pt": dict(base="c5", batch=3, per_token=False, ctx_kind="uniform", ctx_a=4, ctx_b=1500),
    # 16-token pages and contexts past 16K tokens: a slot's pages outgrow the
    # 256-entry page window of the LDS-staged layout many times over, which is then
    # refilled; and 64-token pages past 256 pages (16K tokens)
    "mtp4_g16_bs16_long": dict(base="c5", batch=2, block_size=16, ctx_kind="uniform", ctx_a=17000, ctx_b=40000),
    "mtp4_g16_bs64_long": dict(base="c5", batch=2, ctx_kind="uniform", ctx_a=16500, ctx_b=30000),
}


@pytest.mark.parametrize("case", sorted(SMALL_CASES))
@pytest.mark.parametrize("max_parts", [1, 2, 3, 8])
def test_small_cases_with_partials(case, max_parts):
    """Ragged small shapes, every sequence and every partition slot checked.

    max_parts == 1 runs the direct-output mode (no partials, no reduce)."""
    kw = dict(SMALL_CASES[case])
    cfg = scaled(CONFIGS[kw.pop("base")], name=case, **kw)
    print(f"[parity] {case} P={max_parts}", flush=True)
    w = build_workload(cfg, "cuda", seed=7)
    out, _, partials = launch(w, max_parts=max_parts, with_partials=max_parts > 1)
    compare_outputs(w, out, range(cfg.batch))
    if max_parts > 1:
        check_partials(w, partials, max_parts, range(cfg.batch))


@pytest.mark.parametrize("name", ["c2", "c3", "c4"])
@pytest.mark.parametrize("max_parts", [1, 8])
def test_baseline_config_partition_counts(name, max_parts):
    """Full-size configs at the direct-output and the reference-default partition
    counts, every sequence against the oracle (c3: a ragged batch on the partition
    route, as a caller without metadata gets it)."""
    cfg = CONFIGS[name]
    print(f"[parity] {name} P={max_parts}", flush=True)
    w = build_workload(cfg, "cuda")
    out, _, _ = launch(w, max_parts=max_parts)
    compare_outputs(w, out, range(cfg.batch))


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("max_parts", [1, 4])
def test_output_dtypes(out_dtype, max_parts):
    cfg = scaled(CONFIGS["c2"], name="odt", batch=3, ctx_kind="uniform", ctx_a=5, ctx_b=700)
    w = build_workload(cfg, "cuda", seed=3)
    out, _, _ = launch(w, out_dtype=out_dtype, max_parts=max_parts)
    compare_outputs(w, out, range(cfg.batch))


def test_f16_query():
    cfg = scaled(CONFIGS["c3"], name="f16q", batch=3, ctx_kind="uniform", ctx_a=5, ctx_b=700)
    w = build_workload(cfg, "cuda", seed=5)
    out, _, _ = launch(w, query=w["query"].to(torch.float16))
    compare_outputs(w, out, range(cfg.batch))


@pytest.mark.parametrize("name", ["c3", "c4"])
def test_reference_call_pattern_with_recommended_partials(name):
    """The reference harness's call: max_context_partition_num=0 with exp_sums /
    max_logits / temporary_output preallocated for get_recommended_splits' count
    (kernels/pa_decode_fp8.py:3024-3049; 8 for c3, 17 for the c4 window).  The
    launcher takes the count from the buffers and fills every slot; each slot's
    partial is checked against the oracle's token range."""
    import torch

    from flydsl_amd import get_recommended_splits, pa_decode_ps_launch

    cfg = CONFIGS[name]
    print(f"[parity] {name}: reference call pattern", flush=True)
    w = build_workload(cfg, "cuda")
    if cfg.sliding_window:
        parts = get_recommended_splits(cfg.batch, cfg.num_kv_heads, sliding_window=cfg.sliding_window,
                                       query_length=cfg.query_length)
    else:
        parts = get_recommended_splits(cfg.batch, cfg.num_kv_heads, split_kv_blocks=256 // cfg.block_size)
    assert parts == (17 if cfg.sliding_window else 8)
    eqgs = cfg.query_length * cfg.group_size
    shape = (cfg.batch, cfg.num_kv_heads, parts, eqgs)
    partials = {"exp_sums": torch.full(shape, float("nan"), device="cuda"),
                "max_logits": torch.full(shape, float("nan"), device="cuda"),
                "temporary_output": torch.full(shape + (128,), float("nan"), dtype=torch.bfloat16, device="cuda")}
    out = torch.empty_like(w["query"])
    tag = pa_decode_ps_launch(out, w["query"], w["key_cache"], w["value_cache"], w["context_lengths"],
                              w["kv_page_indices"], w["kv_indptr"], 1.0 / math.sqrt(128), w["key_scale"],
                              w["value_scale"], sliding_window=cfg.sliding_window, block_tables=w["block_tables"],
                              max_context_partition_num=0, **partials)
    torch.cuda.synchronize()
    assert tag == ("ps_sw_partitioned" if cfg.sliding_window else "ps_small_block")
    compare_outputs(w, out, range(cfg.batch))
    check_partials(w, partials, parts, _spread(cfg.batch, 16))


@pytest.mark.parametrize("parts", [1, 8])
def test_caller_partials_with_metadata_on_a_ragged_batch(parts):
    """The reference harness's arguments on a ragged c3 batch -- get_pa_metadata's
    schedule, the flat page list, an explicit partition count -- plus caller-passed
    exp_sums / max_logits / temporary_output: the reference's small-block route
    ignores the metadata and fills the partials slot by slot
    (kernels/pa_decode_fp8.py:3010-3121), and so does this launcher (even at one
    slot, where its reduce reads them).  Every slot is checked against the oracle's
    token range, every sequence's output against the oracle."""
    from flydsl_amd import get_pa_metadata, pa_decode_ps_launch

    cfg = CONFIGS["c3"]
    print(f"[parity] c3 with metadata and caller partials, P={parts}", flush=True)
    w = build_workload(cfg, "cuda")
    md = get_pa_metadata(w["query"], w["key_cache"], w["context_lengths"], w["kv_indptr"], cfg.num_q_heads,
                         cfg.num_kv_heads)
    assert md["uniform_context"] is False
    eqgs = cfg.query_length * cfg.group_size
    shape = (cfg.batch, cfg.num_kv_heads, parts, eqgs)
    partials = {"exp_sums": torch.full(shape, float("nan"), device="cuda"),
                "max_logits": torch.full(shape, float("nan"), device="cuda"),
                "temporary_output": torch.full(shape + (128,), float("nan"), dtype=torch.bfloat16, device="cuda")}
    out = torch.empty_like(w["query"])
    tag = pa_decode_ps_launch(out, w["query"], w["key_cache"], w["value_cache"], w["context_lengths"],
                              w["kv_page_indices"], w["kv_indptr"], 1.0 / math.sqrt(128), w["key_scale"],
                              w["value_scale"], metadata=md, block_tables=w["block_tables"],
                              max_context_partition_num=parts, **partials)
    torch.cuda.synchronize()
    assert tag == "ps_small_block"
    compare_outputs(w, out, range(cfg.batch))
    check_partials(w, partials, parts, _spread(cfg.batch, 16))


CHAIN_CASES = {
    "bs16_pt_g4": dict(base="c2", batch=5, ctx_kind="uniform", ctx_a=1, ctx_b=3000),
    "bs16_tok_g4": dict(base="c3", batch=6, ctx_kind="uniform", ctx_a=1, ctx_b=3000),
    "sw_small": dict(base="c4", batch=4, sliding_window=300, ctx_kind="uniform", ctx_a=1, ctx_b=2000),
    "sw_mtp": dict(base="c4", batch=4, sliding_window=100, query_length=3, ctx_kind="uniform", ctx_a=3, ctx_b=900),
    "bs64_ql2_g8_tok": dict(base="c3", batch=4, num_q_heads=16, num_kv_heads=2, block_size=64, query_length=2,
                            ctx_kind="uniform", ctx_a=2, ctx_b=2500),
}


def _bits(t):
    return t.view(torch.int32) if t.dtype == torch.float32 else t.view(torch.int16)


@pytest.mark.parametrize("case", sorted(CHAIN_CASES))
@pytest.mark.parametrize("parts,spw,wg", [(3, 2, 2), (8, 3, 4), (8, 8, 1), (5, 4, 2), (17, 3, 8)])
def test_chained_slots_equal_one_slot_per_wave(case, parts, spw, wg, monkeypatch):
    """One wave running several consecutive slots (its loads running on across the
    slot boundaries) writes exactly what one wave per slot writes; and workgroups of
    wg such waves that hold every slot of their (sequence, kv head) and merge their
    own partials write the output the reduce kernel writes.  Partials and outputs
    bit-identical across the three layouts, every slot checked against the oracle's
    token range, empty slots (0, -inf, 0) included."""
    from flydsl_amd import pa_decode_fp8 as pdf

    kw = dict(CHAIN_CASES[case])
    cfg = scaled(CONFIGS[kw.pop("base")], name=case, **kw)
    print(f"[parity] chained slots {case} P={parts} spw={spw} wg={wg}", flush=True)
    w = build_workload(cfg, "cuda", seed=8)
    results = []
    for layout in ((1, 1, False), (1, spw, False), (wg, spw, True)):
        monkeypatch.setattr(pdf, "_slot_layout", lambda *a, layout=layout, **k: layout)
        pdf._PLAN_CACHE.clear()
        out, _, part = launch(w, max_parts=parts, with_partials=True)
        plan = next(reversed(pdf._PLAN_CACHE.values()))
        assert (plan.rargs is None) == layout[2]
        results.append((out, part))
    pdf._PLAN_CACHE.clear()
    out1, part1 = results[0]
    for out2, part2 in results[1:]:
        assert torch.equal(out1, out2)
        for k in part1:
            assert torch.equal(_bits(part1[k]), _bits(part2[k])), k
    compare_outputs(w, out1, range(cfg.batch))
    check_partials(w, part1, parts, range(cfg.batch))
