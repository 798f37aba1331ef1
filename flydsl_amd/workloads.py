"""Synthetic decode workloads shaped like the five benchmark configurations.

Builds seeded inputs in the tensor formats ``pa_decode_ps_launch`` consumes:

* query        bf16 N(0,1)  [B*ql, Hq, D] (D = 128 unless a config says otherwise)
* key_cache    fp8 e4m3fn   [nb, Hkv, D/16, bs, 16]   (uint8 storage)
* value_cache  fp8 e4m3fn   [nb, Hkv, bs/16, D, 16]   (trans_v, uint8 storage), or
                            [nb, Hkv, D, bs]          (4-D, trans_v False)
* key/value scales: per-tensor [1] (amax/448) or per-token [nb, Hkv, bs, 1]
* block_tables int32 [B, max_blocks]: a random permutation of the physical
  blocks, handed to the sequences in order (or, with bt_replace, entries drawn
  with replacement, so pages are shared); context_lengths int32 [B]
* kv_page_indices / kv_indptr int32: the same pages as one flat list
  (tests/kernels/test_pa.py:545-559), read by the persistent path

K and V are drawn N(0,1) (or U(-1,1)) in float32 and quantised with scale = amax/448 and
``(x / scale).to(torch.float8_e4m3fn)`` -- the quantisers of
tests/kernels/test_pa.py:334-416 and tests/utils.py:29-73.  Generation runs
on any torch device (chunked, so large caches fit).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field, replace
from typing import Dict, List, Optional

import numpy as np
import torch

HEAD_DIM = 128
FP8_MAX = 448.0


@dataclass(frozen=True)
class DecodeConfig:
    name: str
    batch: int
    num_q_heads: int
    num_kv_heads: int
    block_size: int
    query_length: int = 1
    per_token: bool = False
    sliding_window: int = 0
    ctx_kind: str = "fixed"  # fixed | uniform | lognormal
    ctx_a: int = 4096
    ctx_b: int = 4096
    lognormal_sigma: float = 1.0
    num_physical_blocks: Optional[int] = None  # None: exactly the blocks the sequences use
    blocks_per_seq_stride: Optional[int] = None  # sequence b takes perm[b*stride : ...]
    head_dim: int = HEAD_DIM
    trans_v: bool = True  # value cache [nb, Hkv, bs/16, D, 16]; False: [nb, Hkv, D, bs]
    # block-table entries drawn with replacement from num_physical_blocks (default:
    # the blocks the sequences use), so pages repeat within and across sequences
    # (tests/kernels/test_pa.py:713-716)
    bt_replace: bool = False
    dist: str = "normal"  # query / K / V draws: "normal" N(0,1) or "uniform" U(-1,1) (test_pa.py:62)
    description: str = field(default="", compare=False)

    @property
    def group_size(self) -> int:
        return self.num_q_heads // self.num_kv_heads


CONFIGS: Dict[str, DecodeConfig] = {
    "c1": DecodeConfig(
        "c1", 4, 8, 2, 16, ctx_kind="uniform", ctx_a=1, ctx_b=512, num_physical_blocks=256, blocks_per_seq_stride=32,
        description="tiny CPU-runnable case: B4, 8q/2kv, bs16, ctx U[1,512], per-tensor",
    ),
    "c2": DecodeConfig(
        "c2", 64, 32, 8, 16, ctx_kind="fixed", ctx_a=4096, ctx_b=4096,
        description="Llama-3-8B-shaped: B64, 32q/8kv, bs16, ctx 4096, per-tensor",
    ),
    "c3": DecodeConfig(
        "c3", 128, 32, 8, 16, per_token=True, ctx_kind="lognormal", ctx_a=16, ctx_b=32768,
        description="ragged: B128, 32q/8kv, bs16, ctx lognormal(median 2048, sigma 1) in [16, 32768], per-token",
    ),
    "c4": DecodeConfig(
        "c4", 32, 32, 8, 16, sliding_window=4096, ctx_kind="uniform", ctx_a=8192, ctx_b=32768,
        description="sliding window 4096: B32, 32q/8kv, bs16, ctx U[8192, 32768], per-tensor",
    ),
    "c5": DecodeConfig(
        "c5", 256, 64, 4, 64, query_length=4, per_token=True, ctx_kind="uniform", ctx_a=4096, ctx_b=8192,
        description="MTP: B256, ql4 causal, 64q/4kv (GQA 16), bs64, ctx U[4096, 8192], per-token",
    ),
}


def context_lengths_for(cfg: DecodeConfig, seed: int = 123) -> List[int]:
    rng = np.random.default_rng(seed)
    if cfg.ctx_kind == "fixed":
        return [cfg.ctx_a] * cfg.batch
    if cfg.ctx_kind == "uniform":
        return [int(x) for x in rng.integers(cfg.ctx_a, cfg.ctx_b + 1, size=cfg.batch)]
    if cfg.ctx_kind == "lognormal":
        z = rng.standard_normal(cfg.batch)
        v = np.round(np.exp(math.log(2048.0) + cfg.lognormal_sigma * z))
        return [int(x) for x in np.clip(v, cfg.ctx_a, cfg.ctx_b)]
    raise ValueError(cfg.ctx_kind)


def block_tables_for(cfg: DecodeConfig, ctx: List[int], seed: int = 123):
    """(block_tables [B, max_blocks] int64 numpy, num_physical_blocks)."""
    rng = np.random.default_rng(seed + 1)
    bs = cfg.block_size
    nblk = [max(1, (c + bs - 1) // bs) for c in ctx]
    max_blocks = max(nblk)
    if cfg.blocks_per_seq_stride is not None:
        total = cfg.num_physical_blocks
        perm = rng.permutation(total)
        stride = cfg.blocks_per_seq_stride
        bt = np.zeros((cfg.batch, max(max_blocks, 1)), dtype=np.int64)
        for b in range(cfg.batch):
            bt[b, : nblk[b]] = perm[b * stride : b * stride + nblk[b]]
        return bt, total
    total = sum(nblk) if cfg.num_physical_blocks is None else cfg.num_physical_blocks
    if cfg.bt_replace:
        bt = np.zeros((cfg.batch, max_blocks), dtype=np.int64)
        for b in range(cfg.batch):
            bt[b, : nblk[b]] = rng.integers(0, total, size=nblk[b])
        return bt, total
    perm = rng.permutation(total)
    bt = np.zeros((cfg.batch, max_blocks), dtype=np.int64)
    off = 0
    for b in range(cfg.batch):
        bt[b, : nblk[b]] = perm[off : off + nblk[b]]
        off += nblk[b]
    return bt, total


def _quant_per_tensor(x: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    return (x / scale).to(torch.float8_e4m3fn).view(torch.uint8)


def _chunks(n: int, chunk: int):
    for s in range(0, n, chunk):
        yield s, min(n, s + chunk)


def _draw(shape, gen, dev, dist: str) -> torch.Tensor:
    if dist == "uniform":
        return torch.rand(shape, generator=gen, device=dev, dtype=torch.float32) * 2.0 - 1.0
    return torch.randn(shape, generator=gen, device=dev, dtype=torch.float32)


def build_kv_cache(
    num_blocks: int,
    num_kv_heads: int,
    block_size: int,
    per_token: bool,
    device,
    seed: int = 123,
    chunk_blocks: int = 4096,
    head_dim: int = HEAD_DIM,
    trans_v: bool = True,
    dist: str = "normal",
):
    """Quantised caches (key_x, value, key_scale, value_scale) on ``device``; the
    value cache is trans_v [nb, Hkv, bs/16, D, 16] or, with ``trans_v`` False,
    4-D [nb, Hkv, D, bs].

    K/V values are N(0,1) (or U(-1,1)) draws from a per-chunk seeded generator,
    token-major [blocks, Hkv, bs, D] before packing.
    """
    dev = torch.device(device)
    D = head_dim
    kx = torch.empty((num_blocks, num_kv_heads, D // 16, block_size, 16), dtype=torch.uint8, device=dev)
    if trans_v:
        vt = torch.empty((num_blocks, num_kv_heads, block_size // 16, D, 16), dtype=torch.uint8, device=dev)
    else:
        vt = torch.empty((num_blocks, num_kv_heads, D, block_size), dtype=torch.uint8, device=dev)
    if per_token:
        ks = torch.empty((num_blocks, num_kv_heads, block_size, 1), dtype=torch.float32, device=dev)
        vs = torch.empty_like(ks)
    gen = torch.Generator(device=dev)

    def draw(lo, hi, which):
        gen.manual_seed(seed * 1000003 + lo * 2 + which)
        return _draw((hi - lo, num_kv_heads, block_size, D), gen, dev, dist)

    if not per_token:
        amax = [torch.zeros((), device=dev), torch.zeros((), device=dev)]
        for lo, hi in _chunks(num_blocks, chunk_blocks):
            for w in range(2):
                amax[w] = torch.maximum(amax[w], draw(lo, hi, w).abs().max())
        scales = [(a / FP8_MAX).reshape(1).to(torch.float32) for a in amax]
        scales = [torch.where(s == 0, torch.ones_like(s), s) for s in scales]
        ks, vs = scales
    for lo, hi in _chunks(num_blocks, chunk_blocks):
        k = draw(lo, hi, 0)
        v = draw(lo, hi, 1)
        if per_token:
            ksc = k.abs().amax(dim=-1, keepdim=True) / FP8_MAX
            ksc = torch.where(ksc == 0, torch.ones_like(ksc), ksc)
            vsc = v.abs().amax(dim=-1, keepdim=True) / FP8_MAX
            vsc = torch.where(vsc == 0, torch.ones_like(vsc), vsc)
            kq = (k / ksc).to(torch.float8_e4m3fn).view(torch.uint8)
            vq = (v / vsc).to(torch.float8_e4m3fn).view(torch.uint8)
            ks[lo:hi] = ksc
            vs[lo:hi] = vsc
        else:
            kq = _quant_per_tensor(k, ks)
            vq = _quant_per_tensor(v, vs)
        n = hi - lo
        kx[lo:hi] = kq.view(n, num_kv_heads, block_size, D // 16, 16).permute(0, 1, 3, 2, 4)
        if trans_v:
            vt[lo:hi] = vq.view(n, num_kv_heads, block_size // 16, 16, D).permute(0, 1, 2, 4, 3)
        else:
            vt[lo:hi] = vq.permute(0, 1, 3, 2)
        del k, v, kq, vq
    return kx, vt, ks, vs


def build_workload(cfg: DecodeConfig, device, seed: int = 123, context_lengths: Optional[List[int]] = None):
    """Every input of one decode step for ``cfg`` on ``device`` (dict of tensors + metadata)."""
    dev = torch.device(device)
    ctx = context_lengths if context_lengths is not None else context_lengths_for(cfg, seed)
    bt, nphys = block_tables_for(cfg, ctx, seed)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    q = _draw((cfg.batch * cfg.query_length, cfg.num_q_heads, cfg.head_dim), gen, dev, cfg.dist).to(torch.bfloat16)
    kx, vt, ks, vs = build_kv_cache(nphys, cfg.num_kv_heads, cfg.block_size, cfg.per_token, dev, seed,
                                    head_dim=cfg.head_dim, trans_v=cfg.trans_v, dist=cfg.dist)
    # flat page list of the persistent path (tests/kernels/test_pa.py:545-559)
    pages = [(c + cfg.block_size - 1) // cfg.block_size for c in ctx]
    kv_indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    kv_page_indices = np.concatenate([bt[b, : pages[b]] for b in range(cfg.batch)] + [np.zeros(0, np.int64)])
    return {
        "config": cfg,
        "query": q,
        "key_cache": kx,
        "value_cache": vt,
        "key_scale": ks,
        "value_scale": vs,
        "block_tables": torch.as_tensor(bt, dtype=torch.int32).to(dev),
        "kv_page_indices": torch.as_tensor(kv_page_indices.astype(np.int32)).to(dev),
        "kv_indptr": torch.as_tensor(kv_indptr).to(dev),
        "context_lengths": torch.as_tensor(ctx, dtype=torch.int32).to(dev),
        "context_list": list(ctx),
        "block_table_np": bt,
    }


# what the copies of build_workload_copies share with the first one
SHARED_KEYS = ("context_lengths", "block_tables", "query", "context_list", "block_table_np", "kv_page_indices",
               "kv_indptr")


def build_workload_copies(cfg: DecodeConfig, device, copies: int, seed: int = 123) -> List[Dict]:
    """``copies`` workloads of ``cfg`` that differ only in their KV bytes and scales.

    Every copy is built for the first copy's context lengths, so each cache holds
    exactly the pages the shared block tables and page lists index; the copies then
    take the first copy's tables, page lists and query (``SHARED_KEYS``).  A copy
    sized for other lengths would have indices past its last page, which the
    kernels' bounds guard clamps to that page.
    """
    base = build_workload(cfg, device, seed=seed)
    works = [base]
    for i in range(1, copies):
        w = build_workload(cfg, device, seed=seed + i * 1000, context_lengths=base["context_list"])
        for k in SHARED_KEYS:
            w[k] = base[k]
        works.append(w)
    return works


def attended_tokens(ctx: List[int], query_length: int, sliding_window: int) -> List[int]:
    """Keys any query of the sequence attends: ctx, or min(ctx, sw + ql) with a window."""
    if sliding_window > 0:
        return [min(c, sliding_window + query_length) for c in ctx]
    return list(ctx)


def kv_bytes(cfg: DecodeConfig, ctx: List[int]) -> int:
    """Algorithmic fp8 K+V bytes of one decode step: sum_b sum_h attended_b * 2 * D."""
    return sum(attended_tokens(ctx, cfg.query_length, cfg.sliding_window)) * cfg.num_kv_heads * 2 * cfg.head_dim


def algorithmic_bytes(cfg: DecodeConfig, ctx: List[int]) -> int:
    """KV bytes + per-token scales + query + output + block-table entries + context lengths."""
    att = attended_tokens(ctx, cfg.query_length, cfg.sliding_window)
    total = kv_bytes(cfg, ctx)
    total += sum(att) * cfg.num_kv_heads * 8 if cfg.per_token else 8
    qo = cfg.batch * cfg.query_length * cfg.num_q_heads * cfg.head_dim * 2
    total += 2 * qo
    total += sum((a + cfg.block_size - 1) // cfg.block_size for a in att) * 4
    total += 4 * cfg.batch
    return total


def scaled(cfg: DecodeConfig, **kw) -> DecodeConfig:
    return replace(cfg, **kw)
