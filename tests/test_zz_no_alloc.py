"""pa_fp8_decode_partitions_noalloc (the allocation-free decode, partials in the
library's static device scratch) against the existing entry points with
caller-allocated partials (pa_fp8_decode_partitions + pa_fp8_lse_reduce, as
pa_decode_ps_launch calls them): bit-identical outputs, on two calls in a row
(the second smaller, so stale scratch contents from the first would show), and
the direct one-slot case; an oversized request is refused."""

from __future__ import annotations

import ctypes
import math

import pytest
import torch

from flydsl_amd.workloads import CONFIGS, build_workload, scaled
from tests.pa_testlib import compare_outputs, launch

pytestmark = pytest.mark.gpu


def _noalloc(w, parts, out_dtype=torch.bfloat16, out=None, sync=True):
    """One call of the allocation-free entry through the C ABI (into ``out`` when given)."""
    from flydsl_amd import _lib
    from flydsl_amd import pa_decode_fp8 as pdf

    cfg = w["config"]
    q = w["query"]
    if out is None:
        out = torch.full(q.shape, float("nan"), dtype=out_dtype, device=q.device)
    a = pdf._decode_args(
        query=q, key_cache=w["key_cache"], value_cache=w["value_cache"], block_tables=w["block_tables"],
        context_lengths=w["context_lengths"], key_scale=w["key_scale"], value_scale=w["value_scale"],
        per_token_kv=cfg.per_token, exp_sums=None, max_logits=None, temporary_output=None,
        query_length=cfg.query_length, query_group_size=cfg.group_size, max_parts=parts,
        sliding_window=cfg.sliding_window, softmax_scale=1.0 / math.sqrt(q.shape[-1]),
    )
    o5 = out.view(cfg.batch, cfg.query_length, cfg.num_kv_heads, cfg.group_size, q.shape[-1])
    a.output = o5.data_ptr()
    a.stride_o_seq, a.stride_o_len, a.stride_o_head, a.stride_o_group = (o5.stride(i) for i in range(4))
    a.out_dtype = {torch.bfloat16: _lib.PA_FP8_BF16, torch.float16: _lib.PA_FP8_F16,
                   torch.float32: _lib.PA_FP8_F32}[out.dtype]
    # the launcher's layout, so both paths accumulate in the same order (a merged
    # layout's workgroups merge their own partials: direct_output with several slots)
    max_slot = pdf._max_slot_tokens(w["block_tables"].shape[1] * cfg.block_size, parts, cfg.sliding_window,
                                    cfg.query_length)
    a.waves_per_slot, a.slots_per_wave, merged = pdf._slot_layout(
        q.device, cfg.batch, cfg.num_kv_heads, parts, q.shape[-1], cfg.query_length * cfg.group_size,
        w["value_cache"].dim() != 5, max_slot)
    a.direct_output = 1 if merged else 0
    stream = torch.cuda.current_stream().cuda_stream
    status = _lib.LIB.pa_fp8_decode_partitions_noalloc(ctypes.byref(a), ctypes.c_void_p(stream))
    if sync:
        torch.cuda.synchronize()
    return status, out


def test_noalloc_matches_the_two_call_path():
    big = scaled(CONFIGS["c2"], name="noalloc_big", batch=64, ctx_kind="uniform", ctx_a=1, ctx_b=4096)
    small = scaled(CONFIGS["c3"], name="noalloc_small", batch=5, num_q_heads=16, num_kv_heads=2, query_length=2,
                   ctx_kind="uniform", ctx_a=2, ctx_b=3000)
    for cfg, parts, seed in ((big, 8, 61), (small, 3, 62)):
        print(f"[noalloc] {cfg.name} P {parts}", flush=True)
        w = build_workload(cfg, "cuda", seed=seed)
        ref, tag, _ = launch(w, max_parts=parts, with_partials=True)  # caller-allocated partials
        assert tag == "ps_small_block"
        status, got = _noalloc(w, parts)
        assert status == 0
        assert torch.equal(got, ref), f"{cfg.name}: differs from the two-call path"
        compare_outputs(w, got, range(0, cfg.batch, max(1, cfg.batch // 6)))
    # one slot: the direct-output decode, no scratch
    w = build_workload(small, "cuda", seed=63)
    ref, _, _ = launch(w, max_parts=1)
    status, got = _noalloc(w, 1)
    assert status == 0 and torch.equal(got, ref)


def test_noalloc_refuses_more_partials_than_the_scratch():
    from flydsl_amd import _lib

    cfg = scaled(CONFIGS["c2"], name="noalloc_over", batch=64, ctx_kind="fixed", ctx_a=512, ctx_b=512)
    w = build_workload(cfg, "cuda", seed=64)
    # 64 x 8 x 128 slots x 4 rows x (8 + 256) bytes = 69 MB > 32 MiB
    status, _ = _noalloc(w, 128)
    assert status == _lib.PA_FP8_ERR_SCRATCH


def test_noalloc_replays_in_a_hip_graph():
    """A call captured into a HIP graph (after one eager call on the device, which
    looks up the scratch address) replays over new context lengths written into the
    captured tensor; every replay equals an eager call on the same inputs bit for bit,
    with eager work between the replays."""
    import numpy as np

    cfg = scaled(CONFIGS["c3"], name="noalloc_graph", batch=7, ctx_kind="uniform", ctx_a=1, ctx_b=3000)
    w = build_workload(cfg, "cuda", seed=65)
    parts = 4
    max_ctx = list(w["context_list"])
    status, _ = _noalloc(w, parts)  # the first call on the device, outside the capture
    assert status == 0
    out = torch.empty_like(w["query"])
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        status, _ = _noalloc(w, parts, out=out, sync=False)
    assert status == 0
    rng = np.random.default_rng(6)
    for rep in range(4):
        new_ctx = [int(rng.integers(0, c + 1)) for c in max_ctx]
        w["context_lengths"].copy_(torch.tensor(new_ctx, dtype=torch.int32))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        status, eager = _noalloc(w, parts)
        print(f"[noalloc] graph replay {rep}: ctx {new_ctx[:4]}...", flush=True)
        assert status == 0 and torch.equal(got, eager), f"replay {rep} differs from the eager call"
