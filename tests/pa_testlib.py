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


def launch(w: Dict, max_parts: int = 0, out_dtype=torch.bfloat16, query=None, with_partials: bool = False):
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
            "temporary_output": torch.full(shape + (128,), float("nan"), device=q.device, dtype=torch.bfloat16),
        }
    tag = pa_decode_ps_launch(
        out,
        q,
        w["key_cache"],
        w["value_cache"],
        w["context_lengths"],
        None,
        None,
        1.0 / math.sqrt(128),
        w["key_scale"],
        w["value_scale"],
        sliding_window=cfg.sliding_window,
        block_tables=w["block_tables"],
        max_context_partition_num=max_parts,
        **partials,
    )
    torch.cuda.synchronize()
    return out, tag, partials


def compare_outputs(w: Dict, out: torch.Tensor, batches: Iterable[int]) -> float:
    """Assert |gpu - oracle| <= atol + rtol*|oracle| on the chosen sequences; return max |diff|."""
    cfg = w["config"]
    ql = cfg.query_length
    worst = 0.0
    for b in batches:
        exp = oracle_output(w, b)
        got = out[b * ql : (b + 1) * ql].float().cpu().numpy()
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
    scale = 1.0 / math.sqrt(128)
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
