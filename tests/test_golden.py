"""Committed golden fixtures (tests/golden/*.npz, written by make_golden.py).

CPU: the oracle reproduces every stored output and partial from the stored
inputs.  GPU: the HIP path on the same inputs matches them (bf16 tolerance of
the contract; empty slots exact)."""

import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import attention as oatt
from oracle import fp8 as ofp8
from oracle import planners as oplan
from oracle import quant as oq

GOLDEN = Path(__file__).resolve().parent / "golden"
NAMES = ["c1", "mtp_tok_sw"]


def load(name):
    z = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    d = {k: z[k] for k in z.files}
    d["meta"] = json.loads(str(d["meta"]))
    return d


def bf16(x):
    return ofp8.bf16_bits_to_f32(x)


def test_fixture_c1_is_benchmark_config_1():
    d = load("c1")
    m = d["meta"]
    assert (m["batch"], m["num_q_heads"], m["num_kv_heads"], m["head_dim"], m["block_size"]) == (4, 8, 2, 128, 16)
    assert d["key_cache"].shape == (256, 2, 8, 16, 16) and d["value_cache"].shape == (256, 2, 1, 128, 16)
    assert d["key_scale"].shape == (1,) and 1 <= d["context_lengths"].min() and d["context_lengths"].max() <= 512
    used = np.concatenate([d["block_tables"][b, : math.ceil(c / 16)] for b, c in enumerate(d["context_lengths"])])
    assert len(set(used.tolist())) == len(used)  # a permutation: no block shared


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_fixture(name):
    d = load(name)
    m = d["meta"]
    v4 = oq.v_trans_to_4d(d["value_cache"])
    out = oatt.torch_mha_extend(bf16(d["query_bf16"]), d["key_cache"], v4, d["block_tables"], d["context_lengths"],
                                m["query_length"], d["key_scale"], d["value_scale"], m["sliding_window"])
    exp = bf16(d["expected_bf16"])
    # one bf16 ulp of slack for BLAS summation order on another host
    np.testing.assert_allclose(out, exp, rtol=2**-7, atol=1e-6)


@pytest.mark.parametrize("name", NAMES)
def test_oracle_partials_reproduce_fixture(name):
    d = load(name)
    m = d["meta"]
    g = m["num_q_heads"] // m["num_kv_heads"]
    ql, sw, parts = m["query_length"], m["sliding_window"], m["partials_max_parts"]
    q = bf16(d["query_bf16"])
    for b, ctx in enumerate(d["context_lengths"].tolist()):
        kf, vf = oatt.gather_sequence(d["key_cache"], d["value_cache"], d["block_tables"][b], ctx, d["key_scale"],
                                      d["value_scale"])
        for h in range(m["num_kv_heads"]):
            rows = q[b * ql : (b + 1) * ql, h * g : (h + 1) * g].reshape(ql * g, -1)
            for z in range(parts):
                lo, hi = oplan.partition_token_range(ctx, z, parts, ql, sw)
                e, mx, o = oatt.partition_partial(rows, kf[:, h], vf[:, h], lo, hi, ctx, ql, g, m["softmax_scale"], sw)
                np.testing.assert_allclose(e, d["partial_exp_sums"][b, h, z], rtol=1e-6)
                np.testing.assert_array_equal(np.isneginf(mx), np.isneginf(d["partial_max_logits"][b, h, z]))
                np.testing.assert_allclose(o, bf16(d["partial_out_bf16"][b, h, z]), rtol=2**-7, atol=1e-7)
    # the split must hold both live and empty slots to pin the empty-slot convention
    assert np.isneginf(d["partial_max_logits"]).any() and np.isfinite(d["partial_max_logits"]).any()


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("max_parts", [1, 3, 8])
def test_gpu_matches_fixture(name, max_parts):
    import torch

    from flydsl_amd import pa_decode_ps_launch

    d = load(name)
    m = d["meta"]
    dev = torch.device("cuda:0")
    q = torch.from_numpy(d["query_bf16"].view(np.int16)).view(torch.bfloat16).to(dev)
    out = torch.empty_like(q)
    g = m["num_q_heads"] // m["num_kv_heads"]
    shape = (m["batch"], m["num_kv_heads"], max_parts, m["query_length"] * g)
    kw = {}
    if max_parts > 1:
        kw = dict(exp_sums=torch.full(shape, float("nan"), device=dev),
                  max_logits=torch.full(shape, float("nan"), device=dev),
                  temporary_output=torch.zeros(shape + (128,), device=dev, dtype=torch.bfloat16))
    pa_decode_ps_launch(
        out, q, torch.from_numpy(d["key_cache"]).to(dev), torch.from_numpy(d["value_cache"]).to(dev),
        torch.from_numpy(d["context_lengths"]).to(dev), None, None, m["softmax_scale"],
        torch.from_numpy(d["key_scale"]).to(dev), torch.from_numpy(d["value_scale"]).to(dev),
        sliding_window=m["sliding_window"], block_tables=torch.from_numpy(d["block_tables"]).to(dev),
        max_context_partition_num=max_parts, **kw,
    )
    torch.cuda.synchronize()
    np.testing.assert_allclose(out.float().cpu().numpy(), bf16(d["expected_bf16"]), atol=2e-2, rtol=2e-2)
    if max_parts == m["partials_max_parts"]:
        ml = kw["max_logits"].cpu().numpy()
        empty = np.isneginf(d["partial_max_logits"])
        assert np.array_equal(np.isneginf(ml), empty)
        assert np.all(kw["exp_sums"].cpu().numpy()[empty] == 0)
        assert np.all(kw["temporary_output"].float().cpu().numpy()[empty] == 0)
        np.testing.assert_allclose(ml[~empty], d["partial_max_logits"][~empty], atol=2e-3, rtol=1e-3)
        np.testing.assert_allclose(kw["exp_sums"].cpu().numpy()[~empty], d["partial_exp_sums"][~empty], rtol=1e-2)
        np.testing.assert_allclose(kw["temporary_output"].float().cpu().numpy(), bf16(d["partial_out_bf16"]),
                                   atol=2e-2, rtol=2e-2)
