"""GPU parity of the shape classes beyond the benchmark configurations, against
the CPU oracle (atol 2e-2 / rtol 2e-2, bf16):

* the 4-D value cache [nb, Hkv, D, bs] (trans_v False) on the persistent and
  sliding-window paths (kernels/pa_decode_fp8.py:283-286, :671-676;
  kernels/pa_decode_swa.py:183-186, :575), including a write -> decode round
  trip through the KV-cache writer's 4-D layout;
* head dims 64, 192 and 256 (the reference accepts multiples of 64,
  kernels/pa_decode_fp8.py:969-970, :2084-2085);
* more than 64 query rows per kv head (GQA 16 x ql 8 = 128, 80), which the
  reference loops over as MTP groups (:2101, :2642-2699);
* block tables drawn with replacement, so pages are shared within and across
  sequences (tests/kernels/test_pa.py:713-716), and uniform(-1, 1) inputs (:62).

Every partial the split paths write is checked too: the partition slots against
the oracle's token ranges, the worklist rows against its per-work restatement.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from flydsl_amd.workloads import CONFIGS, build_workload, scaled
from tests.pa_testlib import (check_partials, check_worklist_partials, compare_outputs, launch, metadata_with_bins,
                              schedule_of)

pytestmark = pytest.mark.gpu


def _metadata(w, cfg, tuned=True):
    from flydsl_amd import get_pa_metadata

    md = get_pa_metadata(w["query"], w["key_cache"], w["context_lengths"], w["kv_indptr"], cfg.num_q_heads,
                         cfg.num_kv_heads, tuned=tuned)
    md["uniform_context"] = False
    s = schedule_of(md)
    s["partial_output"].fill_(float("nan"))
    s["partial_lse"].fill_(float("nan"))
    return md


def _run_worklist(cfg, seed, bins_per_head):
    """The persistent path over get_pa_metadata's tuned schedule (0), its reference
    schedule (-1) or a schedule with few bins per head (many splits)."""
    w = build_workload(cfg, "cuda", seed=seed)
    if bins_per_head > 0:
        md = metadata_with_bins(w, bins_per_head * cfg.num_kv_heads)
    else:
        md = _metadata(w, cfg, tuned=bins_per_head == 0)
    out, tag, _ = launch(w, metadata=md)
    compare_outputs(w, out, range(cfg.batch))
    n = check_worklist_partials(w, schedule_of(md))
    return tag, n


def _run_partitions(cfg, seed, parts):
    w = build_workload(cfg, "cuda", seed=seed)
    out, tag, partials = launch(w, max_parts=parts, with_partials=parts > 1)
    compare_outputs(w, out, range(cfg.batch))
    if parts > 1:
        check_partials(w, partials, parts, range(cfg.batch))
    return tag


# ------------------------------------------------------------- 4-D value cache
@pytest.mark.parametrize("heads", [(8, 1), (16, 1)])
@pytest.mark.parametrize("quant", ["per_token", "per_tensor"])
@pytest.mark.parametrize("ql", [1, 3])
def test_4d_value_cache_persistent_path(heads, quant, ql):
    """1024-token pages with the 4-D value cache, the reference's persistent case
    set shape (tests/kernels/test_pa.py:1180-1205) with trans_v False."""
    cfg = scaled(CONFIGS["c2"], name="v4d_persistent", batch=5, num_q_heads=heads[0], num_kv_heads=heads[1],
                 block_size=1024, query_length=ql, per_token=quant == "per_token", trans_v=False,
                 ctx_kind="uniform", ctx_a=ql, ctx_b=3000)
    print(f"[shapes] 4-D V persistent {heads} {quant} ql {ql}", flush=True)
    for bins in (0, 3):
        tag, n = _run_worklist(cfg, 21, bins)
        assert tag == "ps_split_reduce"
    print(f"[shapes] {n} partial rows checked", flush=True)


@pytest.mark.parametrize("bs,window,parts", [(16, 300, 3), (16, 1000, 0), (64, 700, 4), (1024, 1500, 2)])
@pytest.mark.parametrize("quant", ["per_token", "per_tensor"])
def test_4d_value_cache_sliding_window(bs, window, parts, quant):
    """The sliding-window path reads the 4-D value cache for every block size."""
    cfg = scaled(CONFIGS["c4"], name="v4d_sw", batch=4, num_q_heads=16, num_kv_heads=2, block_size=bs,
                 query_length=2, sliding_window=window, per_token=quant == "per_token", trans_v=False,
                 ctx_kind="uniform", ctx_a=2, ctx_b=5000)
    print(f"[shapes] 4-D V sliding window bs {bs} window {window} P {parts} {quant}", flush=True)
    tag = _run_partitions(cfg, 23, parts)
    assert tag in ("ps_sw_partitioned", "ps_sw_fused_partitioned")


@pytest.mark.parametrize("per_token", [False, True])
@pytest.mark.parametrize("path", ["persistent", "sliding_window"])
def test_write_4d_layout_then_decode(per_token, path):
    """The KV-cache writer's 4-D layout (x-packed K, [nb, Hkv, D, bs] V: the
    reference writer's flash_layout=False, kernels/fused_rope_cache_kernel.py:29-35)
    decoded by pa_decode_ps_launch, against the oracle on the written cache."""
    from flydsl_amd import pa_decode_ps_launch
    from flydsl_amd.fused_rope_cache import build_fused_rope_cache_module
    from oracle import attention as oatt

    B, QH, KH, D = 4, 16, 2, 128
    bs = 256 if path == "persistent" else 16
    ctx = [37, 300, 129, 513]
    g = torch.Generator().manual_seed(17)
    blocks = [math.ceil(c / bs) for c in ctx]
    nb = sum(blocks) + 3
    perm = torch.randperm(nb, generator=g)
    tables = torch.zeros(B, max(blocks), dtype=torch.int32)
    start = 0
    for b in range(B):
        tables[b, : blocks[b]] = perm[start : start + blocks[b]]
        start += blocks[b]
    T = sum(ctx)
    slots = torch.cat([tables[b, torch.arange(ctx[b]) // bs].long() * bs + torch.arange(ctx[b]) % bs
                       for b in range(B)]).int()
    positions = torch.cat([torch.arange(c) for c in ctx]).int()
    dev = "cuda"
    k = torch.randn(T, KH, D, generator=g).bfloat16().to(dev)
    v = torch.randn(T, KH, D, generator=g).bfloat16().to(dev)
    q_tok = torch.randn(T, QH, D, generator=g).bfloat16().to(dev)
    th = torch.arange(1024)[:, None].float() * (10000.0 ** (-torch.arange(D // 2).float() / (D // 2)))
    cos, sin = th.cos().bfloat16().to(dev), th.sin().bfloat16().to(dev)
    kc = torch.zeros(nb, KH, D // 16, bs, 16, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros(nb, KH, D, bs, dtype=torch.float8_e4m3fn, device=dev)
    if per_token:
        ks = torch.zeros(nb, KH, bs, 1, device=dev)
        vs = torch.zeros(nb, KH, bs, 1, device=dev)
    else:
        ks = torch.tensor([0.02], device=dev)
        vs = torch.tensor([0.015], device=dev)
    q_out, k_out = torch.empty_like(q_tok), torch.empty_like(k)
    write = build_fused_rope_cache_module(head_dim=D, num_q_heads=QH, num_kv_heads=KH, block_size=bs,
                                          flash_layout=False, apply_scale=True)
    write(q_tok, k, v, positions.to(dev), cos, sin, slots.to(dev), kc, vc, q_out, k_out, T, ks, vs)
    last = torch.tensor(np.cumsum(ctx) - 1)
    query = q_out[last.to(dev)].contiguous()
    out = torch.empty_like(query)
    ctx_t = torch.tensor(ctx, dtype=torch.int32, device=dev)
    kv_indptr = torch.tensor(np.concatenate([[0], np.cumsum(blocks)]), dtype=torch.int32, device=dev)
    pages = torch.cat([tables[b, : blocks[b]] for b in range(B)]).to(dev)
    window = 4096 if path == "sliding_window" else 0  # wider than every context: plain attention
    tag = pa_decode_ps_launch(out, query, kc, vc, ctx_t, pages, kv_indptr, 1.0 / math.sqrt(D), ks, vs,
                              sliding_window=window, block_tables=tables.to(dev))
    torch.cuda.synchronize()
    assert tag in (("ps_split_reduce",) if path == "persistent" else ("ps_sw_partitioned", "ps_sw_fused_partitioned"))
    kx = kc.view(torch.uint8).cpu().numpy()
    v4 = vc.view(torch.uint8).cpu().numpy()
    ksn, vsn = ks.cpu().numpy(), vs.cpu().numpy()
    for b in range(B):
        kf, vf = oatt.gather_sequence(kx, v4, tables[b].numpy(), ctx[b], ksn, vsn)
        want = oatt.reference_masked_attention(query[b : b + 1].float().cpu().numpy(), kf, vf, 1.0 / math.sqrt(D),
                                               True, 0)
        np.testing.assert_allclose(out[b : b + 1].float().cpu().numpy(), want, atol=2e-2, rtol=2e-2)


# ---------------------------------------------------------------- head dims
HEAD_DIM_CASES = {
    "g4": dict(num_q_heads=8, num_kv_heads=2, query_length=1),
    "mtp2_g8": dict(num_q_heads=16, num_kv_heads=2, query_length=2),
    "mtp4_g16": dict(num_q_heads=32, num_kv_heads=2, query_length=4),
}


@pytest.mark.parametrize("d", [64, 192, 256])
@pytest.mark.parametrize("case", sorted(HEAD_DIM_CASES))
@pytest.mark.parametrize("quant", ["per_token", "per_tensor"])
def test_head_dims_partition_path(d, case, quant):
    cfg = scaled(CONFIGS["c2"], name=f"d{d}_{case}", batch=3, head_dim=d, block_size=16,
                 per_token=quant == "per_token", ctx_kind="uniform", ctx_a=4, ctx_b=2600, **HEAD_DIM_CASES[case])
    print(f"[shapes] head_dim {d} {case} {quant}: partition slots 1, 3", flush=True)
    for parts in (1, 3):
        assert _run_partitions(cfg, 31, parts) == "ps_small_block"


@pytest.mark.parametrize("d", [64, 192, 256])
@pytest.mark.parametrize("case", sorted(HEAD_DIM_CASES))
@pytest.mark.parametrize("bs", [16, 1024])
def test_head_dims_worklist_path(d, case, bs):
    cfg = scaled(CONFIGS["c3"], name=f"d{d}_{case}_wl", batch=3, head_dim=d, block_size=bs, per_token=True,
                 ctx_kind="uniform", ctx_a=4, ctx_b=2600, **HEAD_DIM_CASES[case])
    print(f"[shapes] head_dim {d} {case} bs {bs}: worklist", flush=True)
    for bins in (0, 3):
        _run_worklist(cfg, 33, bins)


@pytest.mark.parametrize("d", [64, 256])
@pytest.mark.parametrize("trans_v", [True, False])
def test_head_dims_sliding_window(d, trans_v):
    cfg = scaled(CONFIGS["c4"], name=f"d{d}_sw", batch=3, head_dim=d, num_q_heads=16, num_kv_heads=2,
                 query_length=2, sliding_window=500, trans_v=trans_v, ctx_kind="uniform", ctx_a=2, ctx_b=3000)
    print(f"[shapes] head_dim {d} sliding window trans_v {trans_v}", flush=True)
    _run_partitions(cfg, 35, 3)
    _run_partitions(cfg, 35, 0)


# --------------------------------------------------------- > 64 rows per kv head
ROW_CASES = {
    "g16_ql8": dict(num_q_heads=16, num_kv_heads=1, query_length=8),  # 128 rows: two chunks
    "g20_ql4": dict(num_q_heads=40, num_kv_heads=2, query_length=4),  # 80 rows: a 16-row second chunk
    "g48_ql3": dict(num_q_heads=48, num_kv_heads=1, query_length=3),  # 144 rows: three chunks
}


@pytest.mark.parametrize("case", sorted(ROW_CASES))
@pytest.mark.parametrize("quant", ["per_token", "per_tensor"])
def test_many_query_rows_partition_path(case, quant):
    cfg = scaled(CONFIGS["c5"], name=case, batch=3, block_size=16, per_token=quant == "per_token",
                 ctx_kind="uniform", ctx_a=8, ctx_b=2500, **ROW_CASES[case])
    print(f"[shapes] {case} {quant}: partition slots 1, 2", flush=True)
    for parts in (1, 2):
        _run_partitions(cfg, 41, parts)


@pytest.mark.parametrize("case", sorted(ROW_CASES))
@pytest.mark.parametrize("bs", [64, 1024])
def test_many_query_rows_worklist_path(case, bs):
    cfg = scaled(CONFIGS["c5"], name=f"{case}_wl", batch=3, block_size=bs, ctx_kind="uniform", ctx_a=8,
                 ctx_b=2500, **ROW_CASES[case])
    print(f"[shapes] {case} bs {bs}: worklist", flush=True)
    for bins in (0, 3):
        _run_worklist(cfg, 43, bins)


def test_many_query_rows_head_dim_256():
    cfg = scaled(CONFIGS["c5"], name="g16_ql8_d256", batch=2, head_dim=256, block_size=64, ctx_kind="uniform",
                 ctx_a=8, ctx_b=1500, num_q_heads=16, num_kv_heads=1, query_length=8)
    print("[shapes] 128 rows at head_dim 256", flush=True)
    _run_partitions(cfg, 45, 2)
    _run_worklist(cfg, 45, 3)


# ------------------------------------------------ shared pages, uniform inputs
@pytest.mark.parametrize("path", ["partition", "worklist", "sliding_window"])
@pytest.mark.parametrize("dist", ["normal", "uniform"])
def test_shared_pages(path, dist):
    """Block tables drawn with replacement from the page pool, as the reference's
    test builds them (tests/kernels/test_pa.py:713-716): the same page appears in
    several sequences and several times in one sequence."""
    base = "c4" if path == "sliding_window" else ("c3" if path == "worklist" else "c2")
    cfg = scaled(CONFIGS[base], name=f"shared_{path}", batch=6, num_q_heads=32, num_kv_heads=4, query_length=2,
                 block_size=16, bt_replace=True, num_physical_blocks=40, dist=dist, ctx_kind="uniform", ctx_a=2,
                 ctx_b=3000, sliding_window=700 if path == "sliding_window" else 0)
    w = build_workload(cfg, "cpu", seed=51)
    bt = w["block_table_np"]
    used = [int(x) for b in range(cfg.batch) for x in bt[b, : (w["context_list"][b] + 15) // 16]]
    assert len(set(used)) < len(used)  # pages are shared
    print(f"[shapes] shared pages, {path}, {dist}", flush=True)
    if path == "worklist":
        _run_worklist(cfg, 51, 0)
        _run_worklist(cfg, 51, 3)
    else:
        _run_partitions(cfg, 51, 3)
        _run_partitions(cfg, 51, 0)


# ----------------------------------------------- query magnitudes, zero K scale
@pytest.mark.parametrize("exp2", [-125, -60, 6])
@pytest.mark.parametrize("case", ["g4", "mtp4_g16"])
@pytest.mark.parametrize("quant", ["per_token", "per_tensor"])
def test_query_magnitudes(exp2, case, quant):
    """Queries scaled by 2^exp2, on the register-streaming (g4) and LDS-staged
    (mtp4_g16) layouts.  At 2^-125 the staged layout's power-of-two query scale
    saturates the E8M0 range and every row averages its visible values; at 2^6 the
    logits are 64 times the unit-scale ones, so the softmax is nearly one-hot and a
    logit error of 2^-8 relative would show: the products must be the exact q . k."""
    cfg = scaled(CONFIGS["c5"], name=f"qmag{exp2}_{case}_{quant}", batch=3, block_size=16,
                 per_token=quant == "per_token", ctx_kind="uniform", ctx_a=4, ctx_b=2000, **HEAD_DIM_CASES[case])
    w = build_workload(cfg, "cuda", seed=61)
    w["query"] = (w["query"].float() * 2.0**exp2).to(torch.bfloat16)
    print(f"[shapes] query x 2^{exp2}, {case}, {quant}", flush=True)
    out, tag, _ = launch(w)
    compare_outputs(w, out, range(cfg.batch))


@pytest.mark.parametrize("case", ["g4", "mtp4_g16"])
def test_zero_key_scale(case):
    """A per-tensor K scale of 0 (an all-zero key cache): every logit is 0 and each
    row averages its visible values."""
    cfg = scaled(CONFIGS["c2"], name=f"ks0_{case}", batch=3, block_size=16, ctx_kind="uniform", ctx_a=4,
                 ctx_b=1500, **HEAD_DIM_CASES[case])
    w = build_workload(cfg, "cuda", seed=63)
    w["key_scale"].zero_()
    print(f"[shapes] zero K scale, {case}", flush=True)
    out, tag, _ = launch(w)
    compare_outputs(w, out, range(cfg.batch))
