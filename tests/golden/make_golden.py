"""Write the committed golden fixtures of the decode path (run from the repo root:
``python tests/golden/make_golden.py``).

The reference repository holds no golden vectors for this path, so these
fixtures are produced by the CPU oracle (oracle/, a restatement of the
reference's torch path) on seeded numpy inputs, and pin the HIP path and the
oracle itself against regressions:

* ``c1.npz``          -- benchmark configuration 1 exactly: batch 4, 8 q heads,
                         2 kv heads, head_dim 128, block 16, ctx U[1, 512], block
                         table = a random permutation of 256 physical blocks
                         (sequence b takes perm[32b : 32b + ceil(ctx/16)]), Q bf16
                         N(0,1), K/V N(0,1) quantised per tensor (amax/448).
* ``mtp_tok_sw.npz``  -- batch 3, query_length 3 (causal), 8 q / 2 kv heads,
                         block 32, per-token scales, sliding window 100, ctx
                         U[3, 700], 64 physical blocks.

Each file holds the inputs in the kernel layouts (K x-layout, V trans_v), the
expected bf16 output bits, and the expected partials of a 3-slot split.
"""

from __future__ import annotations

import json
import math
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import attention as oatt  # noqa: E402
from oracle import fp8 as ofp8  # noqa: E402
from oracle import planners as oplan  # noqa: E402
from oracle import quant as oq  # noqa: E402

HERE = Path(__file__).resolve().parent
D = 128


def make_case(name, *, seed, batch, hq, hkv, bs, ql, per_token, sw, ctx_lo, ctx_hi, nblocks, stride, parts=3):
    rng = np.random.default_rng(seed)
    ctx = rng.integers(ctx_lo, ctx_hi + 1, size=batch).astype(np.int32)
    max_blocks = max(stride, int(max(math.ceil(c / bs) for c in ctx)))
    perm = rng.permutation(nblocks)
    bt = np.zeros((batch, max_blocks), dtype=np.int32)
    for b in range(batch):
        n = math.ceil(ctx[b] / bs)
        bt[b, :n] = perm[b * stride : b * stride + n]
    q = ofp8.bf16_round(rng.standard_normal((batch * ql, hq, D)).astype(np.float32))
    k_tok = rng.standard_normal((nblocks, hkv, bs, D)).astype(np.float32)
    v_tok = rng.standard_normal((nblocks, hkv, bs, D)).astype(np.float32)
    if per_token:
        kx, ks, v4, vs = oq.quantize_kv_per_token(k_tok, v_tok)
    else:
        kx, ks, v4, vs = oq.quantize_kv_per_tensor(k_tok, v_tok)
    vt = oq.v_4d_to_trans(v4)
    out = oatt.torch_mha_extend(q, kx, v4, bt, ctx, ql, ks, vs, sliding_window=sw)
    # partials of a `parts`-slot split, per (sequence, kv head, slot)
    g = hq // hkv
    es = np.zeros((batch, hkv, parts, ql * g), np.float32)
    ml = np.zeros_like(es)
    to = np.zeros((batch, hkv, parts, ql * g, D), np.float32)
    for b in range(batch):
        kf, vf = oatt.gather_sequence(kx, v4, bt[b], int(ctx[b]), ks, vs)
        qb = q[b * ql : (b + 1) * ql]
        for h in range(hkv):
            rows = qb[:, h * g : (h + 1) * g, :].reshape(ql * g, D)
            for z in range(parts):
                lo, hi = oplan.partition_token_range(int(ctx[b]), z, parts, ql, sw)
                e, m, o = oatt.partition_partial(rows, kf[:, h], vf[:, h], lo, hi, int(ctx[b]), ql, g, 1 / math.sqrt(D), sw)
                es[b, h, z], ml[b, h, z], to[b, h, z] = e, m, o
    meta = dict(name=name, seed=seed, batch=batch, num_q_heads=hq, num_kv_heads=hkv, head_dim=D, block_size=bs,
                query_length=ql, per_token=per_token, sliding_window=sw, partials_max_parts=parts,
                softmax_scale=1 / math.sqrt(D))
    np.savez_compressed(
        HERE / f"{name}.npz",
        meta=np.array(json.dumps(meta)),
        query_bf16=ofp8.f32_to_bf16_bits(q),
        key_cache=kx,
        value_cache=vt,
        key_scale=ks.astype(np.float32),
        value_scale=vs.astype(np.float32),
        block_tables=bt,
        context_lengths=ctx,
        expected_bf16=ofp8.f32_to_bf16_bits(out),
        partial_exp_sums=es,
        partial_max_logits=ml,
        partial_out_bf16=ofp8.f32_to_bf16_bits(to),
    )
    print(f"wrote {name}.npz: ctx={ctx.tolist()}")


if __name__ == "__main__":
    make_case("c1", seed=123, batch=4, hq=8, hkv=2, bs=16, ql=1, per_token=False, sw=0, ctx_lo=1, ctx_hi=512,
              nblocks=256, stride=32)
    make_case("mtp_tok_sw", seed=321, batch=3, hq=8, hkv=2, bs=32, ql=3, per_token=True, sw=100, ctx_lo=3,
              ctx_hi=700, nblocks=64, stride=22)
