"""Helpers shared by the GPU parity tests: run the HIP path, compute the CPU
oracle on the same inputs, compare.  The oracle is only the checker here."""

from __future__ import annotations

import math
from typing import Dict, Iterable, List, Optional

import numpy as np
import torch

from oracle import attention as oatt
from oracle import fp8 as ofp8
from oracle import planners as oplan

ATOL = 2e-2  # bf16 output tolerance of the north-star contract (atol 2e-2 / rtol 2e-2)
RTOL = 2e-2


def sequence_inputs(w: Dict, b: int):
    """Dequantised K/V [ctx, Hkv, D] and query [ql, Hq, D] of sequence b (float32 numpy)."""
    cfg = w["config"]
    ctx = int(w["context_list"][b])
    bs = cfg.block_size
    nblk = max(1, (ctx + bs - 1) // bs)
    dev = w["key_cache"].device
    idx = torch.as_tensor(w["block_table_np"][b, :nblk], dtype=torch.long, device=dev)
    kx = w["key_cache"].index_select(0, idx).cpu().numpy()
    vt = w["value_cache"].index_select(0, idx).cpu().numpy()
    if cfg.per_token:
        ks = w["key_scale"].index_select(0, idx).cpu().numpy()
        vs = w["value_scale"].index_select(0, idx).cpu().numpy()
    else:
        ks = w["key_scale"].cpu().numpy()
        vs = w["value_scale"].cpu().numpy()
    kf, vf = oatt.gather_sequence(kx, vt, np.arange(nblk), ctx, ks, vs)
    ql = cfg.query_length
    q = w["query"][b * ql : (b + 1) * ql].float().cpu().numpy()
    return q, kf, vf


def oracle_output(w: Dict, b: int) -> np.ndarray:
    cfg = w["config"]
    q, kf, vf = sequence_inputs(w, b)
    o = oatt.reference_masked_attention(q, kf, vf, 1.0 / math.sqrt(q.shape[-1]), True, cfg.sliding_window)
    return ofp8.bf16_round(o)


def launch(w: Dict, max_parts: int = 0, out_dtype=torch.bfloat16, query=None, with_partials: bool = False,
           metadata=None):
    from flydsl_amd import pa_decode_ps_launch

    cfg = w["config"]
    q = w["query"] if query is None else query
    out = torch.empty(q.shape, dtype=out_dtype, device=q.device)
    partials = {}
    if with_partials:
        if max_parts == 0:
            raise ValueError("pass max_parts with with_partials")
        eqgs = cfg.query_length * cfg.group_size
        shape = (cfg.batch, cfg.num_kv_heads, max_parts, eqgs)
        partials = {
            "exp_sums": torch.full(shape, float("nan"), device=q.device),
            "max_logits": torch.full(shape, float("nan"), device=q.device),
            "temporary_output": torch.full(shape + (cfg.head_dim,), float("nan"), device=q.device,
                                           dtype=torch.bfloat16),
        }
    tag = pa_decode_ps_launch(
        out,
        q,
        w["key_cache"],
        w["value_cache"],
        w["context_lengths"],
        w["kv_page_indices"],
        w["kv_indptr"],
        1.0 / math.sqrt(q.shape[-1]),
        w["key_scale"],
        w["value_scale"],
        sliding_window=cfg.sliding_window,
        metadata=metadata,
        block_tables=w["block_tables"],
        max_context_partition_num=max_parts,
        **partials,
    )
    torch.cuda.synchronize()
    return out, tag, partials


def compare_outputs(w: Dict, out: torch.Tensor, batches: Iterable[int]) -> float:
    """Assert |gpu - oracle| <= atol + rtol*|oracle| on the chosen sequences; return max |diff|.

    The oracle runs per sequence on a small thread pool (numpy's products release
    the interpreter lock), so every sequence of a full-size configuration is checked
    within seconds."""
    from concurrent.futures import ThreadPoolExecutor

    cfg = w["config"]
    ql = cfg.query_length
    batches = list(batches)
    host = out.float().cpu().numpy()
    with ThreadPoolExecutor(max_workers=min(8, max(1, len(batches)))) as pool:
        expected = pool.map(lambda b: oracle_output(w, b), batches)
    worst = 0.0
    for b, exp in zip(batches, expected):
        got = host[b * ql : (b + 1) * ql]
        diff = np.abs(got - exp)
        ok = diff <= ATOL + RTOL * np.abs(exp)
        worst = max(worst, float(diff.max()))
        if not ok.all():
            bad = np.argwhere(~ok)[:5]
            raise AssertionError(
                f"seq {b}: {int((~ok).sum())} elements outside atol/rtol {ATOL}/{RTOL}; "
                f"max diff {diff.max():.4g}; first {bad.tolist()} got {got[tuple(bad[0])]:.5f} exp {exp[tuple(bad[0])]:.5f}"
            )
    return worst


def check_partials(w: Dict, partials: Dict, max_parts: int, batches: Iterable[int], heads: Optional[List[int]] = None):
    """Per-slot partials vs the oracle's partition contract.

    The slot -> token-range mapping is checked exactly: a slot the oracle calls
    empty must hold (0, -inf, 0) bit-for-bit, every other slot must match the
    oracle partial of exactly its token range (max_logit to 2e-3, exp_sum to
    1e-2 relative, output to the bf16 tolerance).
    """
    cfg = w["config"]
    g = cfg.group_size
    es = partials["exp_sums"].cpu().numpy()
    ml = partials["max_logits"].cpu().numpy()
    to = partials["temporary_output"].float().cpu().numpy()
    scale = 1.0 / math.sqrt(cfg.head_dim)
    for b in batches:
        ctx = int(w["context_list"][b])
        q, kf, vf = sequence_inputs(w, b)
        for h in heads if heads is not None else range(cfg.num_kv_heads):
            qrows = q[:, h * g : (h + 1) * g, :].reshape(cfg.query_length * g, -1)
            for z in range(max_parts):
                lo, hi = oplan.partition_token_range(ctx, z, max_parts, cfg.query_length, cfg.sliding_window)
                e_es, e_ml, e_to = oatt.partition_partial(
                    qrows, kf[:, h, :], vf[:, h, :], lo, hi, ctx, cfg.query_length, g, scale, cfg.sliding_window
                )
                g_es, g_ml, g_to = es[b, h, z], ml[b, h, z], to[b, h, z]
                empty = ~np.isfinite(e_ml)
                assert np.all(g_es[empty] == 0.0), (b, h, z, "empty exp_sum")
                assert np.all(np.isneginf(g_ml[empty])), (b, h, z, "empty max_logit")
                assert np.all(g_to[empty] == 0.0), (b, h, z, "empty output")
                live = ~empty
                if live.any():
                    np.testing.assert_allclose(g_ml[live], e_ml[live], atol=2e-3, rtol=1e-3, err_msg=f"ml {b},{h},{z}")
                    np.testing.assert_allclose(g_es[live], e_es[live], rtol=1e-2, atol=1e-3, err_msg=f"es {b},{h},{z}")
                    np.testing.assert_allclose(g_to[live], e_to[live], atol=ATOL, rtol=RTOL, err_msg=f"to {b},{h},{z}")


def metadata_with_bins(w: Dict, num_cu: int) -> Dict:
    """get_pa_metadata's dict, but scheduled over ``num_cu`` bins (few bins force many splits)."""
    from flydsl_amd import get_pa_metadata_info_v1, get_pa_metadata_v1

    cfg = w["config"]
    dev = w["query"].device
    b, ql, hq, hkv = cfg.batch, cfg.query_length, cfg.num_q_heads, cfg.num_kv_heads
    infos = get_pa_metadata_info_v1(b, hkv, num_cu=num_cu)
    ptrs, wi, winfo, ri, rfm, rpm = [torch.empty(shape, dtype=dtype, device=dev) for shape, dtype in infos]
    sq = torch.arange(b + 1, dtype=torch.int32, device=dev) * ql
    get_pa_metadata_v1(sq, w["kv_indptr"], w["context_lengths"], hq // hkv, hkv, True, ptrs, wi, winfo, ri, rfm, rpm,
                       kv_granularity=256, block_size=cfg.block_size, max_seqlen_qo=ql, uni_seqlen_qo=ql,
                       num_cu=num_cu)
    parts = (w["context_lengths"] + 255) // 256
    pind = torch.zeros(b + 1, dtype=torch.int32, device=dev)
    pind[1:] = torch.cumsum(parts, 0).to(torch.int32)
    nparts = int(ri[-1].item())
    return {
        "work_indptr": wi, "work_info_flat": winfo.reshape(-1).contiguous(), "partition_indptr": pind,
        "reduce_indptr": ri, "reduce_final_map": rfm, "reduce_partial_map": rpm, "num_sm": num_cu,
        "partial_output": torch.full(((nparts + 1) * ql, 1, hq, cfg.head_dim), float("nan"), device=dev),
        "partial_lse": torch.full(((nparts + 1) * ql, 1, hq, 1), float("nan"), device=dev),
    }


def schedule_of(md: Dict) -> Dict:
    """The schedule pa_decode_ps_launch runs for a metadata dict: get_pa_metadata's
    tuned schedule when present, else the reference's keys."""
    if md.get("tuned"):
        return dict(md["tuned"], partition_indptr=md["partition_indptr"])
    return md


def check_worklist_partials(w: Dict, md: Dict) -> int:
    """Every partial row the worklist kernel wrote vs the oracle's per-work
    restatement (oatt.worklist_decode) on the same worklist: the work -> token
    range mapping is exact, so an empty row must be (-inf, 0) bit-for-bit and a
    live row must match the oracle's lse to 2e-3 and its f32 output to the bf16
    tolerance.  Returns the number of partial rows checked."""
    cfg = w["config"]
    ql, g = cfg.query_length, cfg.group_size
    cache = {}

    def seq_kv(b):
        if b not in cache:
            _, kf, vf = sequence_inputs(w, b)
            cache[b] = (kf, vf)
        return cache[b]

    po_gpu = md["partial_output"].cpu().numpy()[:, 0]
    pl_gpu = md["partial_lse"].cpu().numpy()[:, 0, :, 0]
    _, po, pl = oatt.worklist_decode(
        w["query"].float().cpu().numpy(), seq_kv, w["context_list"], ql, g, 1.0 / math.sqrt(cfg.head_dim),
        md["work_indptr"].cpu().numpy(), md["work_info_flat"].cpu().numpy(), md["partition_indptr"].cpu().numpy(),
        po_gpu.shape[0],
    )
    written = ~np.isnan(pl)
    assert np.array_equal(written, ~np.isnan(pl_gpu)), "the kernel wrote other partial rows than the worklist names"
    empty = written & np.isneginf(pl)
    assert np.all(np.isneginf(pl_gpu[empty])), "empty partial row without -inf lse"
    assert np.all(po_gpu[empty] == 0.0), "empty partial row with non-zero output"
    live = written & ~np.isneginf(pl)
    np.testing.assert_allclose(pl_gpu[live], pl[live], atol=2e-3, rtol=1e-4, err_msg="partial lse")
    np.testing.assert_allclose(po_gpu[live], po[live], atol=ATOL, rtol=RTOL, err_msg="partial output")
    return int(written.sum())
