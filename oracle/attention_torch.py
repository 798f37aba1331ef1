"""The reference's torch path for the paged decode, restated with torch CPU ops
(test infrastructure only: bench.py's cpu_baseline leg times it on the host
cores, and tests pin it against the numpy oracle in attention.py).

* ``reference_masked_attention`` -- tests/kernels/test_pa.py:214-274
* ``torch_mha_extend``           -- tests/kernels/test_pa.py:277-331

Same arithmetic as the numpy restatement (float32, causal bias -3.4e38,
sliding-window drop to -inf, bf16 cast of the output), on torch tensors so
that every step runs on torch's intra-op thread pool.
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch

CAUSAL_BIAS = -3.4e38  # tests/kernels/test_pa.py:236-238


def reference_masked_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, softmax_scale: float,
                               is_causal: bool = True, sliding_window: int = 0) -> torch.Tensor:
    """float32 masked attention; query [s_q, Hq, D], key / value [s_k, Hkv, D];
    q head h reads kv head h // (Hq / Hkv) (tests/kernels/test_pa.py:228-229).
    Returns float32 [s_q, Hq, D] before the cast."""
    s_q, hq, d = query.shape
    s_k, hkv, _ = key.shape
    g = hq // hkv
    qh = query.reshape(s_q, hkv, g, d).permute(1, 2, 0, 3).reshape(hkv, g * s_q, d)
    logits = torch.matmul(qh, key.permute(1, 2, 0)).reshape(hkv, g, s_q, s_k) * softmax_scale
    if is_causal:
        qi = torch.arange(s_q)[:, None]
        ki = torch.arange(s_k)[None, :]
        logits = logits + torch.where(ki > qi + (s_k - s_q), torch.tensor(CAUSAL_BIAS), torch.tensor(0.0))
    if sliding_window > 0:
        qpos = torch.arange(s_k - s_q, s_k)[:, None]
        kpos = torch.arange(s_k)[None, :]
        logits = logits.masked_fill((qpos - kpos) >= sliding_window + 1, float("-inf"))
    p = torch.softmax(logits, dim=-1)
    out = torch.matmul(p.reshape(hkv, g * s_q, s_k), value.permute(1, 0, 2)).reshape(hkv, g, s_q, d)
    return out.permute(2, 0, 1, 3).reshape(s_q, hq, d)


def gather_sequence(k_x: torch.Tensor, v_cache: torch.Tensor, block_table_row: torch.Tensor, context_length: int,
                    k_scale: torch.Tensor, v_scale: torch.Tensor):
    """Dequantised K / V [ctx, Hkv, D] float32 of one sequence: token t in block
    block_table_row[t // bs], slot t % bs (tests/kernels/test_pa.py:302-314).
    k_x [nb, Hkv, D/16, bs, 16] and v_cache (trans_v 5-D or 4-D) hold fp8 e4m3fn
    codes (uint8); per-token scales are [nb, Hkv, bs, 1]."""
    nb, hkv, dc, bs, _ = k_x.shape
    d = dc * 16
    t = torch.arange(context_length)
    phys = block_table_row.long()[t // bs]
    slot = t % bs
    kc = k_x[phys, :, :, slot, :].reshape(context_length, hkv, d)
    if v_cache.dim() == 5:  # [nb, Hkv, bs/16, D, 16]
        vc = v_cache[phys, :, slot // 16, :, slot % 16]
    else:  # [nb, Hkv, D, bs]
        vc = v_cache[phys, :, :, slot]
    kf = kc.view(torch.float8_e4m3fn).to(torch.float32)
    vf = vc.view(torch.float8_e4m3fn).to(torch.float32)
    if k_scale.numel() == 1:
        kf = kf * k_scale.reshape(())
    else:
        kf = kf * k_scale.reshape(nb, hkv, bs)[phys, :, slot][..., None]
    if v_scale.numel() == 1:
        vf = vf * v_scale.reshape(())
    else:
        vf = vf * v_scale.reshape(nb, hkv, bs)[phys, :, slot][..., None]
    return kf, vf


def torch_mha_extend(query: torch.Tensor, k_x: torch.Tensor, v_cache: torch.Tensor, block_tables: torch.Tensor,
                     context_lengths: Sequence[int], query_length: int, k_scale: torch.Tensor,
                     v_scale: torch.Tensor, sliding_window: int = 0, batches: Optional[Sequence[int]] = None,
                     round_bf16: bool = True) -> torch.Tensor:
    """Paged decode reference over the sequences in ``batches`` (all by default);
    returns float32 [B*ql, Hq, D] (bf16-rounded unless round_bf16 is False; rows of
    other sequences NaN).  softmax_scale = 1/sqrt(D) (tests/kernels/test_pa.py:289)."""
    query = query.to(torch.float32)
    d = query.shape[-1]
    out = torch.full(query.shape, float("nan"), dtype=torch.float32)
    for b in range(len(context_lengths)) if batches is None else batches:
        kf, vf = gather_sequence(k_x, v_cache, block_tables[b], int(context_lengths[b]), k_scale, v_scale)
        rows = slice(b * query_length, (b + 1) * query_length)
        o = reference_masked_attention(query[rows], kf, vf, 1.0 / d**0.5, True, sliding_window)
        out[rows] = o.to(torch.bfloat16).to(torch.float32) if round_bf16 else o
    return out
