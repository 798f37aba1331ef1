"""HIP-graph capture of the decode path and of the KV-cache writer.

* ``get_pa_metadata(..., graph_safe=True)`` reads nothing back to the host and
  sizes its partial buffers for the scheduler's bound; the decode over it
  equals the decode over the host-sized metadata bit for bit.
* A graph holding ``get_pa_metadata`` and ``pa_decode_ps_launch`` (persistent
  1024-token pages, and 16-token pages with the worklist) is replayed over new
  context lengths written into the captured tensors; every replay equals an
  eager launch on the same inputs, with eager work and synchronisations between
  the replays.
* A graph holding the fused RoPE + KV-cache writer is replayed over new slot
  mappings and positions; every replay equals an eager launch.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from flydsl_amd.workloads import CONFIGS, build_workload, scaled

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _decode(w, md, out, **kw):
    from flydsl_amd import pa_decode_ps_launch

    return pa_decode_ps_launch(out, w["query"], w["key_cache"], w["value_cache"], w["context_lengths"],
                               w["kv_page_indices"], w["kv_indptr"], 1.0 / math.sqrt(128), w["key_scale"],
                               w["value_scale"], metadata=md, block_tables=w["block_tables"], **kw)


def _metadata(w, cfg, graph_safe):
    from flydsl_amd import get_pa_metadata

    return get_pa_metadata(w["query"], w["key_cache"], w["context_lengths"], w["kv_indptr"], cfg.num_q_heads,
                           cfg.num_kv_heads, graph_safe=graph_safe)


CASES = {
    "bs1024_tok_ql2": dict(base="c3", batch=5, block_size=1024, query_length=2, num_q_heads=16, num_kv_heads=2,
                           ctx_kind="uniform", ctx_a=2, ctx_b=3000),
    "bs16_pt_g4": dict(base="c2", batch=9, ctx_kind="uniform", ctx_a=1, ctx_b=2600),
    # 64 query rows per kv head: the LDS-staged worklist kernel under capture
    "bs64_tok_mtp4_g16": dict(base="c5", batch=4, ctx_kind="uniform", ctx_a=4, ctx_b=3000),
}


def _case(name):
    kw = dict(CASES[name])
    base = CONFIGS[kw.pop("base")]
    return scaled(base, name=name, **kw)


@pytest.mark.parametrize("name", list(CASES))
def test_graph_safe_metadata_matches_host_sized(name):
    cfg = _case(name)
    w = build_workload(cfg, DEV, seed=11)
    md_host = _metadata(w, cfg, False)
    md_safe = _metadata(w, cfg, True)
    assert md_safe["uniform_context"] is False
    assert md_safe["partial_output"].shape[0] >= md_host["partial_output"].shape[0]
    assert md_safe["partial_output"].shape[0] == (md_safe["reduce_partial_map"].numel() + 1) * cfg.query_length
    # identical schedules (only the valid prefixes of the buffers are defined)
    for k in ("work_indptr", "reduce_indptr", "partition_indptr"):
        assert torch.equal(md_host[k], md_safe[k]), k
    nw = int(md_host["work_indptr"][-1])
    assert torch.equal(md_host["work_info_flat"][: 8 * nw], md_safe["work_info_flat"][: 8 * nw])
    ri = md_host["reduce_indptr"].cpu()
    groups = int((ri[1:] > ri[:-1]).sum())
    assert torch.equal(md_host["reduce_final_map"][:groups], md_safe["reduce_final_map"][:groups])
    assert torch.equal(md_host["reduce_partial_map"][: int(ri[-1])], md_safe["reduce_partial_map"][: int(ri[-1])])
    md_host["uniform_context"] = False
    a, b = torch.empty_like(w["query"]), torch.empty_like(w["query"])
    _decode(w, md_host, a)
    _decode(w, md_safe, b)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("partials", [False, True])
@pytest.mark.parametrize("name", list(CASES))
def test_captured_metadata_and_decode_replay_over_new_contexts(name, partials):
    cfg = _case(name)
    small = cfg.block_size in (16, 64)
    if partials and not small:
        pytest.skip("caller partials belong to the small-block route")
    w = build_workload(cfg, DEV, seed=12)
    ql = cfg.query_length
    max_ctx = list(w["context_list"])
    # Small blocks without partials: the worklist route over the captured schedule
    # (it allocates nothing).  With preallocated split-context partials (the
    # reference's capture rule for its small-block path): the partition kernel at
    # the caller's partition count, filling them.
    extra = {}
    if partials:
        P = 8
        eqgs = ql * (cfg.num_q_heads // cfg.num_kv_heads)
        extra = dict(
            exp_sums=torch.empty(cfg.batch, cfg.num_kv_heads, P, eqgs, dtype=torch.float32, device=DEV),
            max_logits=torch.empty(cfg.batch, cfg.num_kv_heads, P, eqgs, dtype=torch.float32, device=DEV),
            temporary_output=torch.empty(cfg.batch, cfg.num_kv_heads, P, eqgs, 128, dtype=torch.bfloat16, device=DEV),
        )
    out = torch.empty_like(w["query"])
    # warm the kernels and allocator outside the capture
    md = _metadata(w, cfg, True)
    _decode(w, md, out, **extra)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        md_g = _metadata(w, cfg, None)  # graph_safe is implied by the capture
        tag = _decode(w, md_g, out, **extra)
    assert tag == ("ps_small_block" if small else "ps_split_reduce")
    rng = np.random.default_rng(5)
    for rep in range(4):
        # new context lengths (within the pages each sequence owns) written into the captured tensor
        new_ctx = [int(rng.integers(ql, c + 1)) for c in max_ctx]
        w["context_lengths"].copy_(torch.tensor(new_ctx, dtype=torch.int32))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        # eager reference on the same inputs, with its own (host-sized) schedule
        eager = torch.empty_like(out)
        md_e = _metadata(w, cfg, False)
        md_e["uniform_context"] = False
        _decode(w, md_e, eager, **extra)
        torch.cuda.synchronize()
        print(f"[graph] {name} replay {rep}: ctx {new_ctx[:4]}...", flush=True)
        assert torch.equal(got, eager), f"replay {rep} differs from the eager launch"


def test_captured_rope_cache_writer_replays_over_new_slots():
    from flydsl_amd.fused_rope_cache import build_fused_rope_cache_module

    T, QH, KH, D, bs, nb = 96, 16, 4, 128, 16, 32
    g = torch.Generator().manual_seed(9)
    q, k, v = (torch.randn(T, h, D, generator=g).bfloat16().to(DEV) for h in (QH, KH, KH))
    cos, sin = (torch.randn(4096, D // 2, generator=g).bfloat16().to(DEV) for _ in range(2))
    pos = torch.zeros(T, dtype=torch.int32, device=DEV)
    slots = torch.zeros(T, dtype=torch.int32, device=DEV)
    kc = torch.zeros(nb, KH, D // 16, bs, 16, dtype=torch.float8_e4m3fn, device=DEV)
    vc = torch.zeros(nb, KH, bs // 16, D, 16, dtype=torch.float8_e4m3fn, device=DEV)
    ks = torch.zeros(nb, KH, bs, 1, device=DEV)
    vs = torch.zeros(nb, KH, bs, 1, device=DEV)
    qo = torch.empty_like(q)
    ko = torch.empty_like(k)
    launch = build_fused_rope_cache_module(head_dim=D, num_q_heads=QH, num_kv_heads=KH, block_size=bs,
                                           flash_layout=False, apply_scale=True)

    def run(kc_, vc_, ks_, vs_, qo_, ko_):
        launch(q, k, v, pos, cos, sin, slots, kc_, vc_, qo_, ko_, T, ks_, vs_)

    run(kc, vc, ks, vs, qo, ko)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(kc, vc, ks, vs, qo, ko)
    rng = np.random.default_rng(3)
    for rep in range(4):
        # alternately a prefill-like run of slots (staged V writes) and scattered slots
        if rep % 2 == 0:
            start = int(rng.integers(0, nb * bs // 16 - T // 16)) * 16
            new_slots = np.arange(start, start + T)
        else:
            new_slots = rng.permutation(nb * bs)[:T]
        slots.copy_(torch.tensor(new_slots, dtype=torch.int32))
        pos.copy_(torch.tensor(rng.integers(0, 4096, T), dtype=torch.int32))
        for t in (kc, vc, ks, vs):
            t.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in (kc, vc, ks, vs, qo, ko)]
        ref = [torch.zeros_like(t) for t in (kc, vc, ks, vs)] + [torch.empty_like(qo), torch.empty_like(ko)]
        run(*ref)
        torch.cuda.synchronize()
        print(f"[graph] rope_cache replay {rep}: slots from {int(new_slots[0])}", flush=True)
        for a, b in zip(got, ref):
            assert torch.equal(a.view(torch.uint8) if a.dtype == torch.float8_e4m3fn else a,
                               b.view(torch.uint8) if b.dtype == torch.float8_e4m3fn else b)
