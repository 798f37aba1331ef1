"""GPU parity over random valid shapes, seeded: head dims 64-256, 1-4 kv heads,
GQA 1-16, query_length 1-4, every page size the launcher routes (16 / 64 small
block, 32-1024 persistent), per-tensor and per-token scales, the trans_v and 4-D
value caches where the reference reads them, sliding windows of 1-700 tokens,
contexts up to 20000 tokens, shared pages, normal and uniform inputs, bf16 / f16 /
f32 outputs, f16 queries, caller-sized partials, and get_pa_metadata's schedules
(tuned, reference) or schedules over 1 or 3 bins per kv head.  Each case checks
every output row against the CPU oracle at atol / rtol 2e-2."""

from __future__ import annotations

import random

import pytest
import torch

from flydsl_amd.workloads import CONFIGS, build_workload, scaled
from tests.pa_testlib import compare_outputs, launch, metadata_with_bins

pytestmark = pytest.mark.gpu


def _case(seed: int):
    rnd = random.Random(seed)
    d = rnd.choice([64, 128, 128, 192, 256])
    hkv = rnd.choice([1, 2, 4])
    g = rnd.choice([1, 2, 4, 5, 8, 16])
    ql = rnd.choice([1, 1, 2, 3, 4])
    path = rnd.choice(["partition", "partition", "sliding_window", "worklist", "worklist"])
    bs = rnd.choice([16, 64]) if path != "worklist" else rnd.choice([16, 32, 64, 256, 1024])
    # the small-block path takes the trans_v cache only (kernels/pa_decode_fp8.py:2082-2083)
    small_block = path == "partition" or (path == "worklist" and bs in (16, 64))
    trans_v = True if small_block else rnd.random() < 0.6
    cfg = scaled(CONFIGS["c3"], name=f"rand{seed}", batch=rnd.randint(1, 5), num_q_heads=hkv * g,
                 num_kv_heads=hkv, query_length=ql, head_dim=d, block_size=bs, per_token=rnd.random() < 0.5,
                 trans_v=trans_v, sliding_window=rnd.choice([1, 17, 100, 700]) if path == "sliding_window" else 0,
                 ctx_kind="uniform", ctx_a=ql, ctx_b=rnd.choice([40, 300, 1500, 3000, 3000, 20000]),
                 dist=rnd.choice(["normal", "uniform"]), bt_replace=rnd.random() < 0.3, num_physical_blocks=None,
                 blocks_per_seq_stride=None)
    return rnd, path, cfg


@pytest.mark.parametrize("seed", range(48))
def test_random_shape(seed):
    rnd, path, cfg = _case(5000 + seed)
    print(f"[random] seed {seed}: {path} D {cfg.head_dim} Hkv {cfg.num_kv_heads} g {cfg.group_size} "
          f"ql {cfg.query_length} bs {cfg.block_size} per_token {cfg.per_token} trans_v {cfg.trans_v} "
          f"B {cfg.batch} ctx <= {cfg.ctx_b} sw {cfg.sliding_window}", flush=True)
    w = build_workload(cfg, "cuda", seed=5000 + seed)
    out_dtype = rnd.choice([torch.bfloat16, torch.bfloat16, torch.float16, torch.float32])
    query = w["query"].to(torch.float16) if rnd.random() < 0.25 else None
    if path == "worklist":
        bins = rnd.choice([0, 1, 3])
        if bins:
            md = metadata_with_bins(w, bins * cfg.num_kv_heads)
        else:
            from flydsl_amd import get_pa_metadata

            md = get_pa_metadata(w["query"], w["key_cache"], w["context_lengths"], w["kv_indptr"], cfg.num_q_heads,
                                 cfg.num_kv_heads, tuned=rnd.random() < 0.7)
            md["uniform_context"] = False
        out, tag, _ = launch(w, metadata=md, out_dtype=out_dtype, query=query)
    else:
        parts = rnd.choice([0, 1, 2, 3, 5])
        out, tag, _ = launch(w, max_parts=parts, out_dtype=out_dtype, query=query,
                             with_partials=parts > 1 and rnd.random() < 0.5)
    if query is not None:
        w["query"] = query  # the oracle reads the f16 values
    compare_outputs(w, out, range(cfg.batch))
