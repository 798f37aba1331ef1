"""Pins the attention oracle (restatement of tests/kernels/test_pa.py:214-331)
against an independent brute-force loop implementation, closed forms and
invariants, so a dropped term, a wrong mask bound or a transposed operand fails."""

import math

import numpy as np
import pytest

from oracle import attention as oatt
from oracle import fp8 as ofp8
from oracle import planners as oplan
from oracle import quant as oq


def brute_attention(q, k, v, scale, sliding_window=0):
    """Pure-Python loops over (query, head, key) with math.exp."""
    sq, hq, d = q.shape
    sk, hkv, _ = k.shape
    g = hq // hkv
    out = np.zeros((sq, hq, d))
    for qi in range(sq):
        pos = sk - sq + qi
        for h in range(hq):
            kh = h // g
            keys = [t for t in range(sk) if t <= pos and not (sliding_window > 0 and pos - t >= sliding_window + 1)]
            logits = [sum(float(q[qi, h, j]) * float(k[t, kh, j]) for j in range(d)) * scale for t in keys]
            m = max(logits)
            w = [math.exp(x - m) for x in logits]
            s = sum(w)
            for j in range(d):
                out[qi, h, j] = sum(wi * float(v[t, kh, j]) for wi, t in zip(w, keys)) / s
    return out


@pytest.mark.parametrize(
    "sq,sk,hq,hkv,sw",
    [(1, 7, 4, 1, 0), (3, 9, 4, 2, 0), (2, 11, 2, 2, 3), (4, 13, 8, 2, 5), (1, 20, 2, 1, 1), (3, 3, 2, 1, 0)],
)
def test_matches_brute_force(sq, sk, hq, hkv, sw):
    rng = np.random.default_rng(sq * 100 + sk)
    d = 8
    q = rng.standard_normal((sq, hq, d)).astype(np.float32)
    k = rng.standard_normal((sk, hkv, d)).astype(np.float32)
    v = rng.standard_normal((sk, hkv, d)).astype(np.float32)
    got = oatt.reference_masked_attention(q, k, v, 0.37, True, sw)
    exp = brute_attention(q, k, v, 0.37, sw)
    np.testing.assert_allclose(got, exp, rtol=2e-5, atol=2e-6)


def test_uniform_logits_give_mean_of_visible_values():
    rng = np.random.default_rng(1)
    sk, sq, d = 10, 3, 4
    q = np.zeros((sq, 2, d), np.float32)
    k = rng.standard_normal((sk, 1, d)).astype(np.float32)
    v = rng.standard_normal((sk, 1, d)).astype(np.float32)
    out = oatt.reference_masked_attention(q, k, v, 1.0, True, 0)
    for qi in range(sq):
        vis = sk - sq + qi + 1  # causal: keys 0 .. sk-sq+qi
        np.testing.assert_allclose(out[qi, 0], v[:vis, 0].mean(0), rtol=1e-6, atol=1e-6)
    out_w = oatt.reference_masked_attention(q, k, v, 1.0, True, 2)
    for qi in range(sq):
        pos = sk - sq + qi
        np.testing.assert_allclose(out_w[qi, 1], v[pos - 2 : pos + 1, 0].mean(0), rtol=1e-6, atol=1e-6)


def test_window_zero_width_keeps_diagonal_only():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((2, 1, 4)).astype(np.float32)
    k = rng.standard_normal((6, 1, 4)).astype(np.float32)
    v = rng.standard_normal((6, 1, 4)).astype(np.float32)
    # sliding_window = 1 keeps keys with pos - k <= 1: the diagonal and one behind it
    out = oatt.reference_masked_attention(q, k, v, 1.0, True, 1)
    for qi, pos in enumerate((4, 5)):
        ll = [float(q[qi, 0] @ k[t, 0]) for t in (pos - 1, pos)]
        w = np.exp(np.array(ll) - max(ll))
        exp = (w[0] * v[pos - 1, 0] + w[1] * v[pos, 0]) / w.sum()
        np.testing.assert_allclose(out[qi, 0], exp, rtol=1e-5, atol=1e-6)


def test_output_in_convex_hull_of_values():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((2, 4, 16)).astype(np.float32) * 3
    k = rng.standard_normal((50, 2, 16)).astype(np.float32)
    v = rng.standard_normal((50, 2, 16)).astype(np.float32)
    out = oatt.reference_masked_attention(q, k, v, 0.25, True, 0)
    for h in range(4):
        lo, hi = v[:, h // 2].min(0), v[:, h // 2].max(0)
        assert np.all(out[:, h] >= lo - 1e-5) and np.all(out[:, h] <= hi + 1e-5)


def test_gather_sequence_matches_elementwise_layout_walk():
    rng = np.random.default_rng(4)
    nb, h, bs, d = 6, 2, 32, 128
    k_tok = rng.standard_normal((nb, h, bs, d)).astype(np.float32)
    v_tok = rng.standard_normal((nb, h, bs, d)).astype(np.float32)
    kx, ks, v4, vs = oq.quantize_kv_per_token(k_tok, v_tok)
    vt = oq.v_4d_to_trans(v4)
    table = np.array([4, 1, 5], dtype=np.int64)
    ctx = 70
    kf, vf = oatt.gather_sequence(kx, vt, table, ctx, ks, vs)
    for t in (0, 31, 32, 45, 69):
        blk, slot = table[t // bs], t % bs
        for hh in range(h):
            for dd in (0, 15, 16, 77, 127):
                kc = kx[blk, hh, dd // 16, slot, dd % 16]
                vc = vt[blk, hh, slot // 16, dd, slot % 16]
                assert kf[t, hh, dd] == ofp8.E4M3_DECODE[kc] * ks[blk, hh, slot, 0]
                assert vf[t, hh, dd] == ofp8.E4M3_DECODE[vc] * vs[blk, hh, slot, 0]


@pytest.mark.parametrize("sw", [0, 300])
@pytest.mark.parametrize("ql", [1, 3])
def test_partials_merge_to_single_pass(sw, ql):
    """Split into arbitrary slots, LSE-merge the partials -> the one-pass result."""
    rng = np.random.default_rng(5 + sw + ql)
    ctx, g, d = 1000, 4, 128
    q = rng.standard_normal((ql * g, d)).astype(np.float32)
    k = rng.standard_normal((ctx, d)).astype(np.float32)
    v = rng.standard_normal((ctx, d)).astype(np.float32)
    scale = 1 / math.sqrt(d)
    full = oatt.reference_masked_attention(
        q.reshape(ql, g, d), k[:, None, :], v[:, None, :], scale, True, sw
    ).reshape(ql * g, d)
    for parts in (1, 2, 3, 7):
        es, ml, to = [], [], []
        for z in range(parts):
            lo, hi = oplan.partition_token_range(ctx, z, parts, ql, sw)
            e, m, o = oatt.partition_partial(q, k, v, lo, hi, ctx, ql, g, scale, sw)
            es.append(e), ml.append(m), to.append(o)
        merged = oatt.lse_reduce(np.array(es), np.array(ml), np.array(to))
        # partials are bf16-rounded, as in the kernel contract
        np.testing.assert_allclose(merged, full, atol=8e-3, rtol=1e-2)


def test_partial_of_empty_slot():
    q = np.ones((4, 128), np.float32)
    k = np.ones((10, 128), np.float32)
    e, m, o = oatt.partition_partial(q, k, k, 10, 10, 10, 1, 4, 0.1, 0)
    assert np.all(e == 0) and np.all(np.isneginf(m)) and np.all(o == 0)


def test_lse_reduce_closed_form():
    es = np.array([[2.0], [1.0], [0.0]])
    ml = np.array([[0.0], [math.log(2.0)], [-np.inf]])
    to = np.array([[[1.0, 0.0]], [[0.0, 1.0]], [[5.0, 5.0]]])
    # weights: 2*e^0 : 1*e^ln2 : 0 -> 0.5 : 0.5 : 0
    np.testing.assert_allclose(oatt.lse_reduce(es, ml, to), [[0.5, 0.5]], rtol=1e-7)
    assert np.all(oatt.lse_reduce(np.zeros((2, 1)), np.full((2, 1), -np.inf), np.ones((2, 1, 3))) == 0)


def test_torch_mha_extend_matches_direct_attention():
    rng = np.random.default_rng(6)
    nb, hkv, hq, bs, d, ql = 8, 2, 8, 16, 128, 2
    k_tok = rng.standard_normal((nb, hkv, bs, d)).astype(np.float32)
    v_tok = rng.standard_normal((nb, hkv, bs, d)).astype(np.float32)
    kx, ks, v4, vs = oq.quantize_kv_per_tensor(k_tok, v_tok)
    bt = np.array([[3, 0, 6], [1, 7, 2]], np.int32)
    ctx = np.array([40, 33], np.int32)
    q = ofp8.bf16_round(rng.standard_normal((2 * ql, hq, d)).astype(np.float32))
    out = oatt.torch_mha_extend(q, kx, v4, bt, ctx, ql, ks, vs)
    kd = oq.dequant_tok(oq.k_x_to_tok(kx), ks)
    vd = oq.dequant_tok(oq.v_4d_to_tok(v4), vs)
    for b in range(2):
        toks = [(bt[b, t // bs], t % bs) for t in range(ctx[b])]
        kk = np.stack([kd[p, :, s] for p, s in toks])
        vv = np.stack([vd[p, :, s] for p, s in toks])
        exp = oatt.reference_masked_attention(q[b * ql : (b + 1) * ql], kk, vv, 1 / math.sqrt(d), True, 0)
        np.testing.assert_array_equal(out[b * ql : (b + 1) * ql], ofp8.bf16_round(exp))


def test_torch_restatement_matches_numpy_oracle():
    """oracle/attention_torch.py (the baseline's torch CPU path) computes what the
    numpy oracle computes, on the golden fixtures (per-tensor c1; per-token, ql 3,
    window 100, bs 32) with the trans_v and the 4-D value layouts: to float32
    rounding before the bf16 cast, and the same bf16 values after it except at
    rare ties on a bf16 boundary."""
    import json
    from pathlib import Path

    import torch

    from oracle import attention_torch as oat

    golden = Path(__file__).resolve().parent / "golden"
    for name in ("c1", "mtp_tok_sw"):
        z = np.load(golden / f"{name}.npz", allow_pickle=False)
        meta = json.loads(str(z["meta"]))
        q = ofp8.bf16_bits_to_f32(z["query_bf16"])
        ql, sw = int(meta.get("query_length", 1)), int(meta.get("sliding_window", 0))
        ctx = [int(c) for c in z["context_lengths"]]
        for v in (z["value_cache"], oq.v_trans_to_4d(z["value_cache"])):
            ref = np.concatenate([
                oatt.reference_masked_attention(
                    q[b * ql:(b + 1) * ql],
                    *oatt.gather_sequence(z["key_cache"], v, z["block_tables"][b], ctx[b], z["key_scale"],
                                          z["value_scale"]),
                    1 / math.sqrt(q.shape[-1]), True, sw)
                for b in range(len(ctx))])
            got = oat.torch_mha_extend(torch.from_numpy(q), torch.from_numpy(z["key_cache"]), torch.from_numpy(v),
                                       torch.from_numpy(z["block_tables"]), ctx, ql,
                                       torch.from_numpy(z["key_scale"]), torch.from_numpy(z["value_scale"]), sw,
                                       round_bf16=False).numpy()
            np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6, err_msg=name)
            assert np.mean(ofp8.bf16_round(got) == ofp8.bf16_round(ref)) > 0.999, name
