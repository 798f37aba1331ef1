"""Host logic of the drop-in launcher, exercised on CPU tensors (no kernel runs):
routing and return tags, argument blocks handed to the C ABI, the default
partition policy, the direct-output mode and the reference's error behaviour."""

import math

import pytest
import torch

from flydsl_amd import _lib
from flydsl_amd import pa_decode_fp8 as pdf
from flydsl_amd.pa_decode_swa import get_sw_max_context_partition_num
from flydsl_amd.pa_metadata import get_pa_metadata_info_v1


@pytest.fixture(autouse=True)
def _mi355x_cus(monkeypatch):
    """Plans are built on CPU tensors here; the launcher sizes grids for 256 CUs."""
    monkeypatch.setattr(pdf, "_device_cu_count", lambda dev: 256)


def make(batch=3, hq=8, hkv=2, bs=16, ql=1, nb=20, per_token=False, max_blocks=8):
    d = 128
    t = dict(
        output=torch.empty(batch * ql, hq, d, dtype=torch.bfloat16),
        query=torch.zeros(batch * ql, hq, d, dtype=torch.bfloat16),
        key_cache=torch.zeros(nb, hkv, d // 16, bs, 16, dtype=torch.uint8),
        value_cache=torch.zeros(nb, hkv, bs // 16, d, 16, dtype=torch.uint8),
        context_lengths=torch.full((batch,), 17, dtype=torch.int32),
        block_tables=torch.zeros(batch, max_blocks, dtype=torch.int32),
    )
    if per_token:
        t["key_scale"] = torch.ones(nb, hkv, bs, 1)
        t["value_scale"] = torch.ones(nb, hkv, bs, 1)
    else:
        t["key_scale"] = torch.ones(1)
        t["value_scale"] = torch.ones(1)
    return t


def plan(t, sliding_window=0, max_parts=4, capturing=False, **over):
    t = {**t, **over}
    return pdf._build_plan(
        t["output"], t["query"], t["key_cache"], t["value_cache"], t["context_lengths"], 1 / math.sqrt(128),
        t["key_scale"], t["value_scale"], sliding_window, t["block_tables"], max_parts,
        t.get("exp_sums"), t.get("max_logits"), t.get("temporary_output"), capturing,
        kv_page_indices=t.get("kv_page_indices"), kv_indptr=t.get("kv_indptr"), metadata=t.get("metadata"),
    )


def cpu_metadata(t, num_cu):
    """get_pa_metadata's dict built on the CPU from the oracle scheduler (no device)."""
    from oracle import planners as oplan

    ctx = t["context_lengths"].tolist()
    b, ql = len(ctx), t["query"].shape[0] // len(ctx)
    hq, hkv = t["query"].shape[1], t["key_cache"].shape[1]
    md = oplan.get_pa_metadata_v1([i * ql for i in range(b + 1)], ctx, hq // hkv, hkv, num_cu, 256, ql)
    parts = [(c + 255) // 256 for c in ctx]
    nparts = int(md["reduce_indptr"][-1])
    i32 = lambda a: torch.from_numpy(a.astype("int32")).contiguous()  # noqa: E731
    return {
        "work_indptr": i32(md["work_indptr"]),
        "work_info_flat": i32(md["work_info"].reshape(-1)),
        "partition_indptr": torch.tensor([0] + list(torch.tensor(parts).cumsum(0).tolist()), dtype=torch.int32),
        "reduce_indptr": i32(md["reduce_indptr"]),
        "reduce_final_map": i32(md["reduce_final_map"]),
        "reduce_partial_map": i32(md["reduce_partial_map"]),
        "num_sm": num_cu,
        "partial_output": torch.empty(((nparts + 1) * ql, 1, hq, 128)),
        "partial_lse": torch.empty(((nparts + 1) * ql, 1, hq, 1)),
    }


def make_paged(bs=1024, batch=3, hq=16, hkv=1, ql=2, ctx=(1027, 300, 700), per_token=False, num_cu=4):
    t = make(batch=batch, hq=hq, hkv=hkv, bs=bs, ql=ql, nb=8, per_token=per_token, max_blocks=2)
    t["context_lengths"] = torch.tensor(ctx, dtype=torch.int32)
    pages = [(c + bs - 1) // bs for c in ctx]
    t["kv_indptr"] = torch.tensor([0] + list(torch.tensor(pages).cumsum(0).tolist()), dtype=torch.int32)
    t["kv_page_indices"] = torch.arange(sum(pages), dtype=torch.int32) % 8
    t["metadata"] = cpu_metadata(t, num_cu)
    return t


def test_persistent_path_routing_and_args():
    t = make_paged(per_token=True)
    p = plan(t, max_parts=0)
    assert p.tag == "ps_split_reduce" and p.dargs is None and p.rargs is None
    assert [fn.__name__ for fn, _ in p.launches] == ["decode_worklist", "reduce_v1"]
    w, v, md = p.wargs, p.vargs, t["metadata"]
    assert (w.batch_size, w.num_kv_heads, w.query_group_size, w.query_length, w.block_size) == (3, 1, 16, 2, 1024)
    assert w.num_cu == 4 and w.max_work == md["work_info_flat"].numel() // 8 and w.num_pages == 4
    assert w.work_indptr == md["work_indptr"].data_ptr() and w.kv_indptr == t["kv_indptr"].data_ptr()
    assert w.partial_rows == md["partial_output"].shape[0] and w.output_rows == 6
    assert w.stride_po_row == 16 * 128 and w.stride_pl_row == 16
    assert w.per_token_kv == 1 and w.stride_ks_block == 1024 and w.stride_ks_head == 1024
    # the reduce reads the partials from row query_length on (kernels/pa_decode_fp8.py:3190-3191)
    assert v.partial_output == md["partial_output"].data_ptr() + 2 * 16 * 128 * 4
    assert v.partial_lse == md["partial_lse"].data_ptr() + 2 * 16 * 4
    assert v.partial_rows == md["partial_output"].shape[0] - 2 and v.max_qlen == 2
    assert v.num_groups == 3 and v.num_heads == 16 and v.output == t["output"].data_ptr()
    assert int(md["reduce_indptr"][-1]) > 0  # the shape above does split


@pytest.mark.parametrize("bs", [32, 128, 256, 1024])
def test_persistent_path_for_other_block_sizes(bs):
    assert plan(make_paged(bs=bs), max_parts=0).tag == "ps_split_reduce"


def test_persistent_path_without_splits_skips_the_reduce():
    t = make_paged(num_cu=1)  # one bin holds every sequence whole
    assert int(t["metadata"]["reduce_indptr"][-1]) == 0
    p = plan(t, max_parts=0)
    assert p.vargs is None and [fn.__name__ for fn, _ in p.launches] == ["decode_worklist"]


def test_persistent_path_errors():
    t = make_paged()
    with pytest.raises(ValueError, match="kv_page_indices"):
        plan(t, kv_page_indices=None)
    with pytest.raises(ValueError, match="precomputed `metadata`"):
        plan(t, metadata=None, capturing=True)
    bad = dict(t["metadata"], work_indptr=t["metadata"]["work_indptr"][:-1].contiguous())
    with pytest.raises(ValueError, match="work_indptr"):
        plan(t, metadata=bad)
    with pytest.raises(ValueError, match="missing"):
        plan(t, metadata={"num_sm": 4})
    bad = dict(t["metadata"], partial_output=torch.empty(1, 1, 16, 128))
    with pytest.raises(ValueError, match="partial_output"):
        plan(t, metadata=bad)


def test_small_block_routing_and_args():
    t = make()
    p = plan(t, max_parts=4)
    assert p.tag == "ps_small_block" and p.max_parts == 4 and p.rargs is not None
    a = p.dargs
    assert (a.batch_size, a.num_kv_heads, a.query_group_size, a.query_length) == (3, 2, 4, 1)
    assert (a.head_dim, a.block_size, a.num_blocks, a.max_blocks_per_seq) == (128, 16, 20, 8)
    assert a.stride_k_block == 2 * 8 * 16 * 16 and a.stride_k_head == 8 * 16 * 16
    assert a.stride_v_block == 2 * 1 * 128 * 16 and a.stride_v_head == 128 * 16
    assert a.stride_q_seq == 8 * 128 and a.stride_q_head == 128 and a.stride_bt_seq == 8
    assert a.per_token_kv == 0 and a.stride_ks_block == 0 and a.direct_output == 0
    assert abs(a.softmax_scale - 1 / math.sqrt(128)) < 1e-7
    es, to = p.keepalive[0], p.keepalive[2]
    assert tuple(es.shape) == (3, 2, 4, 4) and tuple(to.shape) == (3, 2, 4, 4, 128)
    assert a.exp_sums == es.data_ptr() and a.tmp_out == to.data_ptr()
    r = p.rargs
    assert (r.batch_size, r.query_length, r.num_kv_heads, r.query_group_size, r.max_context_partition_num) == (3, 1, 2, 4, 4)
    assert r.stride_o_seq == 8 * 128 and r.stride_o_head == 4 * 128 and r.stride_o_group == 128


def test_per_token_strides_and_mtp():
    t = make(batch=2, hq=16, hkv=2, bs=64, ql=4, per_token=True)
    p = plan(t, max_parts=3)
    assert p.dargs.per_token_kv == 1
    assert p.dargs.stride_ks_block == 2 * 64 and p.dargs.stride_ks_head == 64
    assert p.dargs.query_length == 4 and p.dargs.query_group_size == 8
    r = p.rargs
    assert r.stride_o_seq == 4 * 16 * 128 and r.stride_o_len == 16 * 128


def test_direct_output_mode_for_one_slot():
    t = make()
    p = plan(t, max_parts=1)
    assert p.rargs is None and p.dargs.direct_output == 1 and p.dargs.exp_sums is None
    assert p.dargs.output == t["output"].data_ptr() and p.dargs.out_dtype == _lib.PA_FP8_BF16
    p32 = plan(t, max_parts=1, output=torch.empty(3, 8, 128))
    assert p32.dargs.out_dtype == _lib.PA_FP8_F32


def test_sliding_window_routing():
    t = make()
    assert plan(t, sliding_window=300, max_parts=3).tag == "ps_sw_partitioned"
    p = plan(t, sliding_window=300, max_parts=1)
    assert p.tag == "ps_sw_fused_partitioned" and p.dargs.sliding_window == 300
    # a window routes every block size to the split-context kernel
    assert plan(make(bs=1024, max_blocks=2), sliding_window=300, max_parts=2).tag == "ps_sw_partitioned"


def test_caller_intermediates_are_used():
    t = make()
    shape = (3, 2, 5, 4)
    es, ml = torch.empty(shape), torch.empty(shape)
    to = torch.empty(shape + (128,), dtype=torch.bfloat16)
    p = plan(t, max_parts=5, exp_sums=es, max_logits=ml, temporary_output=to)
    assert p.dargs.exp_sums == es.data_ptr() and p.dargs.max_logits == ml.data_ptr() and p.dargs.tmp_out == to.data_ptr()
    with pytest.raises(ValueError, match="exp_sums"):
        plan(t, max_parts=4, exp_sums=es, max_logits=ml, temporary_output=to)


@pytest.mark.parametrize(
    "over,exc,match",
    [
        ({"query": torch.zeros(3, 8, 128, dtype=torch.uint8)}, ValueError, "no longer accepts"),
        ({"query": torch.zeros(3, 8, 128, dtype=torch.float32)}, ValueError, "Unsupported query dtype"),
        ({"output": torch.empty(3, 8, 128, dtype=torch.int32)}, ValueError, "Unsupported output dtype"),
        ({"block_tables": None}, ValueError, "requires `block_tables`"),
        ({"value_cache": torch.zeros(20, 2, 128, 16, dtype=torch.uint8)}, NotImplementedError, "trans_v"),
        ({"value_cache": torch.zeros(20, 2, 2, 128, 16, dtype=torch.uint8)}, ValueError, "trans_v layout"),
        ({"key_cache": torch.zeros(20, 2, 8, 24, 16, dtype=torch.uint8),
          "value_cache": torch.zeros(20, 2, 1, 128, 16, dtype=torch.uint8)}, ValueError, "power of two"),
        ({"context_lengths": torch.full((3,), 17, dtype=torch.int64)}, ValueError, "int32"),
        ({"query": torch.zeros(3, 7, 128, dtype=torch.bfloat16), "output": torch.empty(3, 7, 128, dtype=torch.bfloat16)},
         ValueError, "divisible"),
        ({"key_scale": torch.ones(2)}, ValueError, "per-tensor"),
    ],
)
def test_validation_errors(over, exc, match):
    with pytest.raises(exc, match=match):
        plan(make(), max_parts=4, **over)


def test_query_rows_past_64_run_as_chunks():
    """ql * g above 64 (here 80 and GQA 16 x ql 8 = 128) is planned like any other
    shape (the kernels split the rows into chunks of 64); only the merge's grid
    limit of 65535 rows per kv head is refused."""
    p = plan(make(batch=1, hq=40, hkv=2, ql=4), max_parts=2)
    assert p.dargs.query_length * p.dargs.query_group_size == 80 and p.rargs.query_group_size == 20
    t = make_paged(bs=1024, hq=16, hkv=1, ql=8, batch=3, ctx=(1027, 300, 700))
    assert plan(t, max_parts=0).wargs.query_length == 8
    with pytest.raises(ValueError, match="65535"):
        plan(make(batch=1, hq=4096, hkv=1, ql=16, max_blocks=2), max_parts=2)


def make_4d(t):
    """The same caches with the 4-D value layout [nb, Hkv, D, bs]."""
    nb, hkv, _, bs, _ = t["key_cache"].shape
    return {**t, "value_cache": torch.zeros(nb, hkv, 128, bs, dtype=torch.uint8)}


def test_4d_value_cache_routing():
    """The 4-D value layout (trans_v False) runs on the sliding-window and
    persistent paths, as in the reference (kernels/pa_decode_swa.py:183-186,
    kernels/pa_decode_fp8.py:283-286); the small-block kernel refuses it like the
    reference's (:2082-2083), also when metadata would route it to the worklist."""
    t = make_4d(make())
    p = plan(t, sliding_window=300, max_parts=3)
    assert p.tag == "ps_sw_partitioned" and p.dargs.value_layout == _lib.PA_FP8_V_4D
    assert p.dargs.stride_v_block == 2 * 128 * 16 and p.dargs.stride_v_head == 128 * 16
    assert plan(make(), sliding_window=300, max_parts=3).dargs.value_layout == _lib.PA_FP8_V_TRANS
    tp = make_paged(bs=1024)
    tp4 = make_4d(tp)
    p = plan(tp4, max_parts=0)
    assert p.tag == "ps_split_reduce" and p.wargs.value_layout == _lib.PA_FP8_V_4D
    assert plan(tp, max_parts=0).wargs.value_layout == _lib.PA_FP8_V_TRANS
    with pytest.raises(NotImplementedError, match="trans_v=False"):
        plan(t, max_parts=4)
    with pytest.raises(NotImplementedError, match="trans_v=False"):
        plan(make_4d(make_paged(bs=16, ctx=(1027, 300, 2000), num_cu=3)), max_parts=4)
    with pytest.raises(ValueError, match="head_dim, block_size"):
        plan(t, sliding_window=300, max_parts=3, value_cache=torch.zeros(20, 2, 16, 128, dtype=torch.uint8))


@pytest.mark.parametrize("d", [64, 192, 256])
def test_other_head_dims(d):
    """Head dims 64, 192 and 256 plan like 128 (the reference accepts multiples of 64,
    kernels/pa_decode_fp8.py:2084-2085); eight-wave slots are for 128 only."""
    t = make(max_blocks=2)
    t = {**t, "query": torch.zeros(3, 8, d, dtype=torch.bfloat16), "output": torch.empty(3, 8, d, dtype=torch.bfloat16),
         "key_cache": torch.zeros(20, 2, d // 16, 16, 16, dtype=torch.uint8),
         "value_cache": torch.zeros(20, 2, 1, d, 16, dtype=torch.uint8)}
    p = plan(t, max_parts=2)
    assert p.dargs.head_dim == d and p.dargs.waves_per_slot == 4
    assert tuple(p.keepalive[2].shape) == (3, 2, 2, 4, d)
    assert pdf._auto_layout(None, 4, 8, 32768, 0, 1, d)[1] == 4


def test_unsupported_head_dims():
    t = make()
    for d in (96, 320):
        bad = {"query": torch.zeros(3, 8, d, dtype=torch.bfloat16), "output": torch.empty(3, 8, d, dtype=torch.bfloat16)}
        with pytest.raises(ValueError, match="Unsupported head_dim"):
            plan(t, max_parts=2, **bad)


def test_graph_capture_requires_preallocated_partials():
    t = make()
    with pytest.raises(ValueError, match="graph capture requires"):
        pdf._prepare_scale_tensor("key_scale", 0.5, device=torch.device("cpu"), is_graph_capturing=True)
    with pytest.raises(ValueError, match="CUDA graph capture requires preallocated"):
        pdf._build_plan(t["output"], t["query"], t["key_cache"], t["value_cache"], t["context_lengths"], 0.1,
                        t["key_scale"], t["value_scale"], 0, t["block_tables"], 4, None, None, None, True)


def test_auto_partition_policy(monkeypatch):
    monkeypatch.setattr(pdf, "_device_cu_count", lambda dev: 256)
    # c2: 64 x 8 (b, h) pairs already fill 256 CUs x 2 workgroups -> one slot, direct output
    assert pdf._auto_partitions(None, 64, 8, 4096, 0, 1) == 1
    # c3: sequences up to 32768 tokens -> slots of at most 8192 tokens
    assert pdf._auto_partitions(None, 128, 8, 32768, 0, 1) == 4
    assert pdf._auto_layout(None, 64, 8, 4096, 0, 1) == (1, 4)
    # c4: 32 x 8 pairs = one per CU -> one 8-wave slot per pair, direct output
    assert pdf._auto_layout(None, 32, 8, 32768, 4096, 1) == (1, 8)
    # between one and two pairs per CU: two 4-wave slots
    assert pdf._auto_layout(None, 48, 8, 4096, 0, 1) == (2, 4)
    # few pairs: 8-wave slots up to one workgroup per CU, never more slots than tiles
    assert pdf._auto_layout(None, 4, 8, 32768, 0, 1) == (8, 8)
    assert pdf._auto_partitions(None, 1, 1, 300, 0, 1) == 2
    assert pdf._auto_partitions(None, 1, 1, 100, 0, 1) == 1
    # explicit slot counts: eight waves only while the grid fits one workgroup per CU
    assert pdf._waves_per_slot(None, 32, 8, 1) == 8 and pdf._waves_per_slot(None, 32, 8, 2) == 4


def test_recommended_splits_reference_formula(monkeypatch):
    monkeypatch.setattr(pdf, "_cu_count", lambda idx: 256)
    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
    assert pdf.get_recommended_splits(64, 8, 16) == 8
    assert pdf.get_recommended_splits(256, 4, 4) == 4
    assert pdf.get_recommended_splits(32, 8, sliding_window=4096) == 17
    assert get_sw_max_context_partition_num(4096) == 17


def test_metadata_info_matches_oracle():
    from oracle import planners as op

    ours = get_pa_metadata_info_v1(128, 8, num_cu=768)
    ref = op.get_pa_metadata_info_v1(128, 8, 768)
    assert [s for s, _ in ours] == [s for s, _ in ref]
    assert [str(d).split(".")[-1] for _, d in ours] == [d for _, d in ref]


@pytest.mark.parametrize("bs", [16, 64])
def test_small_block_with_metadata_runs_the_worklist(bs):
    t = make_paged(bs=bs, ctx=(1027, 300, 2000), num_cu=3)
    p = plan(t, max_parts=4)
    assert p.tag == "ps_small_block" and p.wargs is not None and p.dargs is None
    assert p.wargs.block_size == bs and p.wargs.num_cu == 3
    # without the flat page list, with a window, or for a uniform batch at one slot or the
    # automatic count, the partition kernel runs; a uniform batch at several slots keeps the
    # worklist (whole sequences per bin, no slot boundaries)
    assert plan(t, max_parts=4, kv_indptr=None).dargs is not None
    uniform = dict(t["metadata"], uniform_context=True)
    assert plan(t, max_parts=1, metadata=uniform).dargs is not None
    assert plan(t, max_parts=0, metadata=uniform).dargs is not None
    assert plan(t, max_parts=4, metadata=uniform).wargs is not None
    assert plan(t, sliding_window=300, max_parts=4).dargs is not None
    # the worklist route allocates nothing, so it is capturable without partials; the
    # partition route keeps the reference's graph-capture rule
    assert plan(t, capturing=True).wargs is not None
    with pytest.raises(ValueError, match="small-block PS path"):
        plan(t, capturing=True, metadata=None)


def test_uniform_batch_at_several_slots_runs_one_slot_when_workgroups_fill_the_gpu():
    """c2's shape at the harness's 8 slots, no caller partials: workgroups of one
    (sequence, kv head) fill 256 CUs, so the partition route runs one slot per sequence
    (four waves, the output written directly), with or without a uniform batch's
    metadata; with caller partials it keeps the caller's 8 slots on the chained layout."""
    t = make(batch=64, hq=32, hkv=8, bs=16, nb=20, max_blocks=256)
    t["kv_indptr"] = torch.arange(65, dtype=torch.int32) * 256
    t["kv_page_indices"] = torch.zeros(64 * 256, dtype=torch.int32)
    for md in (None, {"uniform_context": True}):
        p = plan(t, max_parts=8, metadata=md)
        a = p.dargs
        assert p.tag == "ps_small_block" and p.wargs is None and p.rargs is None
        assert (p.max_parts, a.max_context_partition_num, a.waves_per_slot, a.slots_per_wave, a.direct_output) == (
            1, 1, 4, 0, 1)
    shape = (64, 8, 8, 4)
    p = plan(t, max_parts=8, metadata={"uniform_context": True}, exp_sums=torch.empty(shape),
             max_logits=torch.empty(shape), temporary_output=torch.empty(shape + (128,), dtype=torch.bfloat16))
    assert (p.max_parts, p.dargs.waves_per_slot, p.dargs.slots_per_wave, p.dargs.direct_output) == (8, 4, 2, 1)


@pytest.mark.parametrize("bs", [16, 64])
@pytest.mark.parametrize("parts", [1, 3, 8])
def test_caller_partials_get_the_partition_slot_format(bs, parts):
    """Caller-passed exp_sums / max_logits / temporary_output on the small-block route
    are filled in the reference's partition-slot format at the caller's count, as the
    reference's small-block route (which ignores metadata) fills them
    (kernels/pa_decode_fp8.py:3010-3121): the partition kernel runs even with the
    schedule of a ragged batch, at one slot too (then with the reduce)."""
    t = make_paged(bs=bs, ctx=(1027, 300, 2000), num_cu=3)
    hkv = t["key_cache"].shape[1]
    eqgs = (t["query"].shape[0] // 3) * (t["query"].shape[1] // hkv)  # query_length * group size
    shape = (3, hkv, parts, eqgs)
    es, ml = torch.empty(shape), torch.empty(shape)
    to = torch.empty(shape + (128,), dtype=torch.bfloat16)
    for explicit in (0, parts):
        p = plan(t, max_parts=explicit, exp_sums=es, max_logits=ml, temporary_output=to)
        assert p.tag == "ps_small_block" and p.wargs is None and p.dargs is not None
        assert p.max_parts == parts and p.dargs.max_context_partition_num == parts
        assert p.dargs.direct_output == 0 and p.rargs is not None
        assert p.dargs.exp_sums == es.data_ptr() and p.dargs.max_logits == ml.data_ptr()
        assert p.dargs.tmp_out == to.data_ptr()
    # under capture too (the reference's rule is met: the partials are preallocated)
    assert plan(t, max_parts=parts, exp_sums=es, max_logits=ml, temporary_output=to, capturing=True).dargs is not None
    # one slot without caller partials writes the output directly
    p = plan(t, max_parts=1, metadata=None)
    assert p.dargs.direct_output == 1 and p.rargs is None


def test_default_partition_count_follows_caller_partials():
    """max_context_partition_num=0 with caller-sized partials: the reference sizes them
    with get_recommended_splits and launches that many slots
    (kernels/pa_decode_fp8.py:3024-3029), so the launcher takes the count from them."""
    t = make()
    for parts in (8, 3):
        shape = (3, 2, parts, 4)
        es, ml = torch.empty(shape), torch.empty(shape)
        to = torch.empty(shape + (128,), dtype=torch.bfloat16)
        p = plan(t, max_parts=0, exp_sums=es, max_logits=ml, temporary_output=to)
        assert p.max_parts == parts and p.rargs.max_context_partition_num == parts
        assert p.dargs.exp_sums == es.data_ptr() and p.dargs.tmp_out == to.data_ptr()
        assert p.keepalive == ()  # nothing launcher-made to keep
    # sliding window: the same rule
    shape = (3, 2, 17, 4)
    es, ml = torch.empty(shape), torch.empty(shape)
    to = torch.empty(shape + (128,), dtype=torch.bfloat16)
    p = plan(t, sliding_window=4096, max_parts=0, exp_sums=es, max_logits=ml, temporary_output=to)
    assert p.max_parts == 17 and p.tag == "ps_sw_partitioned"
    # without caller partials the launcher's own count (one direct slot here)
    assert plan(t, max_parts=0).max_parts == 1


@pytest.fixture
def recorded_launches(monkeypatch):
    """pa_decode_ps_launch with the kernel launches replaced by a record of the plans."""
    seen = []

    def launch(self, stream_handle):
        seen.append(self)
        return self.tag

    monkeypatch.setattr(pdf._Plan, "launch", launch)
    pdf._PLAN_CACHE.clear()
    yield seen
    pdf._PLAN_CACHE.clear()


def _launch(t, **kw):
    args = {**t, **kw}
    return pdf.pa_decode_ps_launch(
        args["output"], args["query"], args["key_cache"], args["value_cache"], args["context_lengths"],
        args.get("kv_page_indices"), args.get("kv_indptr"), 1 / math.sqrt(128), args["key_scale"],
        args["value_scale"], block_tables=args.get("block_tables"), metadata=args.get("metadata"),
        max_context_partition_num=args.get("max_parts", 0), stream=0)


def test_cached_plans_release_caller_metadata(recorded_launches):
    """Callers rebuild the metadata every step (its contents follow the context
    lengths); plans cached on it must not keep the old dicts, and their partial
    buffers, alive."""
    import gc
    import weakref

    t = make_paged(per_token=True)
    refs = []
    for _ in range(5):
        md = cpu_metadata(t, 4)
        refs.append(weakref.ref(md["partial_output"]))
        assert _launch(t, metadata=md) == "ps_split_reduce"
        del md
    gc.collect()
    assert all(r() is None for r in refs)
    assert len(pdf._PLAN_CACHE) >= 1 and all(p.keepalive in ((), (None,)) for p in pdf._PLAN_CACHE.values())


def test_converted_scales_are_not_reused_stale(recorded_launches):
    """A scale tensor the launcher has to convert (here float64) is copied; a plan
    holding the copy must not be reused after the caller updates the original."""
    t = make()
    ks = torch.tensor([0.5], dtype=torch.float64)
    _launch(t, key_scale=ks, max_parts=4)
    ks[0] = 0.25
    _launch(t, key_scale=ks, max_parts=4)
    a0, a1 = recorded_launches[0].dargs, recorded_launches[1].dargs
    val = lambda ptr: ctypes_float(ptr)  # noqa: E731
    assert val(a0.key_scale) == 0.5 and val(a1.key_scale) == 0.25
    # a float32 tensor is used as is, so its plan is cached and reads the live value
    ks32 = torch.tensor([0.5])
    _launch(t, key_scale=ks32, max_parts=4)
    ks32[0] = 0.125
    _launch(t, key_scale=ks32, max_parts=4)
    assert recorded_launches[3] is recorded_launches[2] and val(recorded_launches[3].dargs.key_scale) == 0.125


def ctypes_float(ptr):
    import ctypes

    return ctypes.c_float.from_address(ptr).value


def test_worklist_prefers_the_tuned_schedule():
    """get_pa_metadata's dict carries the reference's schedule under the reference's
    keys and this build's own under "tuned"; the worklist kernel runs the tuned one
    when present."""
    t = make_paged(per_token=True)
    ref = cpu_metadata(t, 4)
    tuned = cpu_metadata(t, 2)
    tuned["bin_groups"] = 0
    md = dict(ref, tuned=tuned)
    p = plan(t, metadata=md, max_parts=0)
    assert p.wargs.num_cu == 2 and p.wargs.work_indptr == tuned["work_indptr"].data_ptr()
    assert p.wargs.partial_output == tuned["partial_output"].data_ptr()
    p_ref = plan(t, metadata=ref, max_parts=0)
    assert p_ref.wargs.num_cu == 4 and p_ref.wargs.work_indptr == ref["work_indptr"].data_ptr()
    with pytest.raises(ValueError, match="tuned"):
        plan(t, metadata=dict(ref, tuned={"num_sm": 2}), max_parts=0)


def test_metadata_v1_refuses_buffers_below_the_schedule_bound():
    """get_pa_metadata_v1 refuses work_info / reduce_partial_map smaller than
    get_pa_metadata_info_v1's sizes (kernels/pa_metadata.py:63-72) before launching:
    the device only marks an overflow in work_indptr[0], which a decode would read as
    a truncated worklist."""
    from flydsl_amd.pa_metadata import get_pa_metadata_v1

    b, hkv, num_cu = 5, 2, 8
    i32 = lambda *s: torch.zeros(*s, dtype=torch.int32)  # noqa: E731
    infos = get_pa_metadata_info_v1(b, hkv, num_cu=num_cu)
    ptrs, wi, winfo, ri, rfm, rpm = [torch.zeros(shape, dtype=dtype) for shape, dtype in infos]
    sq, ctx = torch.arange(b + 1, dtype=torch.int32), torch.full((b,), 700, dtype=torch.int32)
    kw = dict(kv_granularity=256, block_size=16, max_seqlen_qo=1, uni_seqlen_qo=1, num_cu=num_cu)
    with pytest.raises(ValueError, match="work_info holds"):
        get_pa_metadata_v1(sq, i32(b + 1), ctx, 4, hkv, True, ptrs, wi, winfo[:-1].contiguous(), ri, rfm, rpm, **kw)
    with pytest.raises(ValueError, match="reduce_partial_map holds"):
        get_pa_metadata_v1(sq, i32(b + 1), ctx, 4, hkv, True, ptrs, wi, winfo, ri, rfm, rpm[:-1].contiguous(), **kw)


def _shaped(batch, hq, hkv, ctx_tokens, bs=16, nb=None):
    t = make(batch=batch, hq=hq, hkv=hkv, bs=bs, nb=nb or 8, max_blocks=ctx_tokens // bs)
    return t


@pytest.mark.parametrize("batch,hkv,ctx,parts,sw,expect", [
    # c2 at the harness's 8 slots: 4 waves x 2 slots hold a (sequence, head), merged in the workgroup
    (64, 8, 4096, 8, 0, (4, 2, True)),
    (64, 8, 4096, 4, 0, (4, 1, True)),
    # c4's window at 17 slots: 8 waves x 3 slots (a slot spans at most two tiles)
    (32, 8, 32768, 17, 4096, (8, 3, True)),
    # c3-like pages (a slot of up to 64 steps): two waves per slot, then the reduce
    (128, 8, 32768, 8, 0, (2, 0, False)),
    # a small batch with many short slots: workgroups per (sequence, head) would not
    # fill the GPU, so one wave per slot
    (8, 8, 16384, 64, 0, (1, 0, False)),
    # too few slots for one wave each: waves split a slot's steps
    (64, 8, 4096, 2, 0, (2, 0, False)),
    (64, 8, 4096, 1, 0, (4, 0, False)),
    (32, 8, 32768, 1, 4096, (8, 0, False)),
])
def test_slot_layout(batch, hkv, ctx, parts, sw, expect):
    """The partition kernel's layout: the fewest waves per slot that fill 256 CUs at eight
    waves each; chained slots when one wave per slot fills them, merged in the workgroup
    when it holds every slot of its (sequence, kv head) within 32 steps per wave."""
    got = pdf._slot_layout(None, batch, hkv, parts, 128, 4, False, pdf._max_slot_tokens(ctx, parts, sw, 1))
    assert got == expect


def test_merged_layout_plan_writes_partials_and_output():
    """With the merged layout the partition kernel writes the caller's partials and the
    output; no reduce launch follows."""
    t = make(batch=64, hq=32, hkv=8, nb=20, max_blocks=256)
    shape = (64, 8, 8, 4)
    es, ml = torch.empty(shape), torch.empty(shape)
    to = torch.empty(shape + (128,), dtype=torch.bfloat16)
    p = plan(t, max_parts=8, exp_sums=es, max_logits=ml, temporary_output=to)
    a = p.dargs
    assert (a.waves_per_slot, a.slots_per_wave, a.direct_output) == (4, 2, 1)
    assert p.rargs is None and [fn.__name__ for fn, _ in p.launches] == ["decode_partitions"]
    assert a.exp_sums == es.data_ptr() and a.tmp_out == to.data_ptr() and a.output == t["output"].data_ptr()
    # without caller partials nobody reads them: one slot per sequence on the same
    # four-wave workgroups, the output written directly
    p = plan(t, max_parts=8)
    a = p.dargs
    assert (p.max_parts, a.max_context_partition_num, a.waves_per_slot, a.slots_per_wave, a.direct_output) == (
        1, 1, 4, 0, 1)
    assert p.rargs is None and len(p.keepalive) == 0


def test_get_pa_metadata_argument_blocks(monkeypatch):
    """get_pa_metadata's scheduler argument blocks (shape fields from a per-shape template,
    pointers as offsets into its one allocation) point at the tensors of the returned dict,
    on CPU tensors with the scheduler launch replaced by a recorder."""
    import ctypes

    calls = []

    def record(args, stream):
        calls.append([{f: getattr(a, f) for f, _ in _lib.MetadataArgs._fields_ if f != "bin_weight"}
                      | {"bin_weight": list(a.bin_weight)} for a in args])
        for a in args:  # the counters the host reads: no split partials, not uniform
            ctypes.memset(a.partial_count, 0, 4)
        ctypes.memset(args[0].uniform_context, 0, 4)

    class _Stream:
        cuda_stream = 0

    monkeypatch.setattr(_lib, "metadata_multi", record)
    monkeypatch.setattr(pdf, "_device_cu_count", lambda dev: 256)
    monkeypatch.setattr(torch.cuda, "current_stream", lambda *a, **k: _Stream())
    pdf._metadata_layout.cache_clear()
    B, hq, hkv = 64, 32, 8
    q = torch.zeros(B, hq, 128, dtype=torch.bfloat16)
    kc = torch.zeros(4, hkv, 8, 16, 16, dtype=torch.uint8)
    kv = torch.zeros(B + 1, dtype=torch.int32)
    for call in range(2):  # the second call reuses the cached layout with new pointers
        ctx = torch.full((B,), 4096 + call, dtype=torch.int32)
        md = pdf.get_pa_metadata(q, kc, ctx, kv, hq, hkv, graph_safe=False)
        blocks = calls[-1]
        assert len(blocks) == 2
        for k, sched in enumerate((md, md["tuned"])):
            a = blocks[k]
            assert a["context_lens"] == ctx.data_ptr() and a["seqlens_qo_indptr"] is None
            for field, key in (("work_indptr", "work_indptr"), ("work_info", "work_info_flat"),
                               ("reduce_indptr", "reduce_indptr"), ("reduce_final_map", "reduce_final_map"),
                               ("reduce_partial_map", "reduce_partial_map")):
                assert a[field] == sched[key].data_ptr(), field
            assert (a["num_batches"], a["gqa"], a["num_heads_k"], a["num_cu"], a["query_length"]) == (
                B, hq // hkv, hkv, sched["num_sm"], 1)
            assert a["max_work"] == sched["work_info_flat"].numel() // 8
            assert a["max_split_tiles"] == sched["reduce_partial_map"].numel()
            assert a["kv_granularity"] == 256
        assert blocks[0]["pack"] == 0 and blocks[1]["pack"] == 1
        assert blocks[0]["bin_groups"] == 0 and blocks[1]["bin_groups"] == md["tuned"]["bin_groups"] == 2
        assert blocks[1]["bin_weight"][:2] == list(md["tuned"]["bin_weight"])
        assert blocks[0]["partition_indptr"] == md["partition_indptr"].data_ptr()
        assert blocks[1]["partition_indptr"] is None and blocks[1]["uniform_context"] is None
        assert md["uniform_context"] is False and md["partial_output"].shape == (1, 1, hq, 128)
    assert pdf._metadata_layout.cache_info().hits >= 1
    with pytest.raises(ValueError, match="power-of-two partition_size"):
        pdf.get_pa_metadata(q, kc, ctx, kv, hq, hkv, partition_size=96)
