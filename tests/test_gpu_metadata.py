"""Device worklist scheduler (get_pa_metadata_v1 / get_pa_metadata) vs the CPU
oracle: bit-exact on every byte the reference defines (the valid prefixes)."""

import numpy as np
import pytest
import torch

from oracle import planners as op

pytestmark = pytest.mark.gpu


def weighted_quota(weights, nspk, ctx):
    """get_pa_metadata's weighted split as a per-bin quota for the oracle's state
    machine: a head's bins form len(weights) equal groups and bin i starts at
    floor(S * Wc(i) / Wt), Wc(i) the weights of the bins before it, when
    nspk % groups == 0 and S >= 4 * nspk; otherwise the reference's even quota.
    Context lengths that are all equal take the even quota too (equal sequences
    fill equal bins whole): None then."""
    if len(set(ctx)) <= 1:
        return None
    ng = len(weights)
    m = nspk // ng

    def wc(i):
        return sum(w * min(max(i - g * m, 0), m) for g, w in enumerate(weights))

    def quota(i, total):
        wt = wc(nspk)
        if nspk % ng or total < 4 * nspk or nspk > 4096 or total * min(weights) < 2 * wt:
            return total // nspk + (1 if i < total % nspk else 0)
        return total * wc(i + 1) // wt - total * wc(i) // wt

    return quota


def expected_schedule(md, sq, ctx, gqa, nhk, gran=256, ql=1):
    """The oracle's schedule for one schedule of a get_pa_metadata result: the
    reference's even one, or the tuned one (it carries bin_groups) with its
    weights -- the packing schedule where that applies, else the sequential fill."""
    qf = weighted_quota(md["bin_weight"], md["num_sm"] // nhk, ctx) if md.get("bin_groups", 0) > 1 else None
    if "bin_groups" in md:
        packed = op.get_pa_metadata_packed(sq, ctx, gqa, nhk, md["num_sm"], gran, ql, quota_of=qf)
        if packed is not None:
            return packed
    return op.get_pa_metadata_v1(sq, ctx, gqa, nhk, md["num_sm"], gran, ql, quota_of=qf)


def reference_num_sm(nhk):
    """The reference's bin count (kernels/pa_decode_fp8.py:1764-1771)."""
    cus = torch.cuda.get_device_properties(torch.device("cuda:0")).multi_processor_count
    return (cus * 3 // nhk) * nhk


def assert_schedule_equal(md, ref, label):
    """Every byte of the valid prefixes the reference defines."""
    v = op.metadata_valid_prefixes(ref)
    np.testing.assert_array_equal(md["work_indptr"].cpu().numpy(), v["work_indptr"], err_msg=label)
    nw = int(v["work_indptr"][-1])
    np.testing.assert_array_equal(md["work_info_flat"].cpu().numpy()[: nw * 8].reshape(nw, 8), v["work_info"],
                                  err_msg=label)
    np.testing.assert_array_equal(md["reduce_indptr"].cpu().numpy(), v["reduce_indptr"], err_msg=label)
    ng = len(v["reduce_final_map"])
    np.testing.assert_array_equal(md["reduce_final_map"].cpu().numpy()[:ng], v["reduce_final_map"], err_msg=label)
    npart = int(v["reduce_indptr"][-1])
    np.testing.assert_array_equal(md["reduce_partial_map"].cpu().numpy()[:npart], v["reduce_partial_map"],
                                  err_msg=label)
    return v


def run_device(ctx, ql, gqa, nhk, num_cu, gran):
    from flydsl_amd import get_pa_metadata_info_v1, get_pa_metadata_v1

    dev = torch.device("cuda:0")
    b = len(ctx)
    infos = get_pa_metadata_info_v1(b, nhk, num_cu=num_cu)
    bufs = [torch.full(shape, -7, dtype=dtype, device=dev) if dtype == torch.int32 else torch.zeros(shape, dtype=dtype, device=dev)
            for shape, dtype in infos]
    sq = torch.arange(b + 1, dtype=torch.int32, device=dev) * ql
    ctx_t = torch.tensor(ctx, dtype=torch.int32, device=dev)
    kv_indptr = torch.zeros(b + 1, dtype=torch.int32, device=dev)
    get_pa_metadata_v1(sq, kv_indptr, ctx_t, gqa, nhk, True, *bufs, kv_granularity=gran, block_size=16,
                       max_seqlen_qo=ql, uni_seqlen_qo=ql, num_cu=num_cu)
    torch.cuda.synchronize()
    ptrs, wi, winfo, ri, rfm, rpm = bufs
    assert int(ptrs[0]) == wi.data_ptr() and int(ptrs[1]) == winfo.data_ptr()
    ref = op.get_pa_metadata_v1(list(range(0, (b + 1) * ql, ql)), ctx, gqa, nhk, num_cu, gran, ql)
    return {"work_indptr": wi.cpu().numpy(), "work_info": winfo.cpu().numpy(), "reduce_indptr": ri.cpu().numpy(),
            "reduce_final_map": rfm.cpu().numpy(), "reduce_partial_map": rpm.cpu().numpy(),
            "num_reduce_groups": ref["num_reduce_groups"]}, ref


@pytest.mark.parametrize("seed", range(10))
def test_device_scheduler_matches_oracle(seed):
    rng = np.random.default_rng(seed)
    nhk = int(rng.choice([1, 2, 4, 8]))
    num_cu = nhk * int(rng.integers(1, 100))
    b = int(rng.integers(1, 140))
    ctx = [int(x) for x in rng.integers(1, int(rng.choice([300, 5000, 33000])), size=b)]
    ql = int(rng.integers(1, 5))
    gqa = int(rng.choice([1, 4, 16]))
    gran = int(rng.choice([16, 256, 1024]))
    got, ref = run_device(ctx, ql, gqa, nhk, num_cu, gran)
    for key, val in op.metadata_valid_prefixes(ref).items():
        np.testing.assert_array_equal(op.metadata_valid_prefixes(got)[key], val, err_msg=key)


@pytest.mark.parametrize("seed", range(24))
def test_device_scheduler_random_wide(seed):
    """Wider random draws: odd kv-head counts, one bin per head up to 256 per head,
    batches either side of the 4096-batch closed-form limit, and contexts that are
    all zero, all equal, partly zero or all long."""
    rng = np.random.default_rng(5000 + seed)
    nhk = int(rng.choice([1, 2, 3, 4, 8]))
    num_cu = nhk * int(rng.choice([1, 2, 3, 7, 64, 100, 192, 256]))
    b = int(rng.choice([1, 2, 7, 64, 300, 4095, 4096, 4097, 5000]))
    dist = rng.choice(["uniform", "zeros", "mixed", "long", "equal"])
    hi = int(rng.choice([2, 300, 5000, 33000]))
    if dist == "zeros":
        ctx = [0] * b
    elif dist == "equal":
        ctx = [hi] * b
    elif dist == "mixed":
        ctx = [int(x) if rng.random() > 0.3 else 0 for x in rng.integers(1, hi, size=b)]
    elif dist == "long":
        ctx = [int(x) for x in rng.integers(hi // 2, hi + 1, size=b)]
    else:
        ctx = [int(x) for x in rng.integers(1, hi, size=b)]
    ql = int(rng.integers(1, 5))
    gqa = int(rng.choice([1, 4, 16]))
    gran = int(rng.choice([16, 64, 256, 1024]))
    got, ref = run_device(ctx, ql, gqa, nhk, num_cu, gran)
    for key, val in op.metadata_valid_prefixes(ref).items():
        np.testing.assert_array_equal(op.metadata_valid_prefixes(got)[key], val, err_msg=key)


def run_device_schedule(ctx, ql, gqa, nhk, nspk, gran, weights, pack, null_sq=False):
    """One schedule from the device scheduler through the C ABI, with this build's
    options (bin_groups / bin_weight, pack) set directly; buffers pre-filled with -7.
    ``null_sq`` passes a NULL seqlens_qo_indptr (the scheduler's b * query_length)."""
    from flydsl_amd import _lib, get_pa_metadata_info_v1

    dev = torch.device("cuda:0")
    b = len(ctx)
    num_cu = nhk * nspk
    infos = get_pa_metadata_info_v1(b, nhk, num_cu=num_cu)
    bufs = [torch.full(shape, -7, dtype=torch.int32, device=dev) for shape, _ in infos[1:]]
    wi, winfo, ri, rfm, rpm = bufs
    sq = torch.arange(b + 1, dtype=torch.int32, device=dev) * ql
    ctx_t = torch.tensor(ctx, dtype=torch.int32, device=dev)
    count = torch.full((1,), -7, dtype=torch.int32, device=dev)
    a = (_lib.MetadataArgs * 1)()
    a[0].seqlens_qo_indptr, a[0].context_lens = (None if null_sq else sq.data_ptr()), ctx_t.data_ptr()
    a[0].work_indptr, a[0].work_info, a[0].reduce_indptr = wi.data_ptr(), winfo.data_ptr(), ri.data_ptr()
    a[0].reduce_final_map, a[0].reduce_partial_map = rfm.data_ptr(), rpm.data_ptr()
    a[0].partial_count = count.data_ptr()
    a[0].num_batches, a[0].gqa, a[0].num_heads_k, a[0].num_cu = b, gqa, nhk, num_cu
    a[0].kv_granularity, a[0].query_length = gran, ql
    a[0].max_work, a[0].max_split_tiles = winfo.numel() // 8, rpm.numel()
    a[0].bin_groups = len(weights) if weights else 0
    for g, w in enumerate(weights or ()):
        a[0].bin_weight[g] = w
    a[0].pack = 1 if pack else 0
    _lib.metadata_multi(a, torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize()
    got = {"work_indptr": wi.cpu().numpy(), "work_info": winfo.cpu().numpy().reshape(-1, 8),
           "reduce_indptr": ri.cpu().numpy(), "reduce_final_map": rfm.cpu().numpy(),
           "reduce_partial_map": rpm.cpu().numpy()}
    return got, int(count.item())


@pytest.mark.parametrize(
    "case",
    ["closed_form", "few_partitions", "all_empty", "serial_batches", "weighted", "packed"],
)
def test_device_scheduler_null_query_offsets(case):
    """A NULL seqlens_qo_indptr (what get_pa_metadata passes) gives the schedule of the
    offsets b * query_length on the closed-form, serial, weighted and packing paths,
    bit-exact with the oracle."""
    rng = np.random.default_rng(sum(map(ord, case)) + 11)
    ql, gqa, gran, weights, pack = 3, 4, 256, None, False
    if case == "closed_form":
        ctx, nhk, nspk = [int(x) for x in rng.integers(0, 4000, size=70)], 4, 16
    elif case == "few_partitions":
        ctx, nhk, nspk = [int(x) for x in rng.integers(1, 300, size=5)], 2, 32
    elif case == "all_empty":
        ctx, nhk, nspk = [0] * 9, 4, 8
    elif case == "serial_batches":
        ctx, nhk, nspk = [int(x) for x in rng.integers(0, 2000, size=4097)], 8, 64
    elif case == "weighted":
        ctx, nhk, nspk, weights = [int(x) for x in rng.integers(500, 9000, size=90)], 2, 24, [130, 114, 100]
    else:
        ctx, nhk, nspk, weights, pack = [int(x) for x in rng.integers(4096, 8193, size=64)], 4, 48, [115, 107, 100], True
    got, _ = run_device_schedule(ctx, ql, gqa, nhk, nspk, gran, weights, pack, null_sq=True)
    want, _ = run_device_schedule(ctx, ql, gqa, nhk, nspk, gran, weights, pack)
    for key in got:
        np.testing.assert_array_equal(got[key], want[key], err_msg=key)
    sq = [ql * i for i in range(len(ctx) + 1)]
    qf = weighted_quota(weights, nspk, ctx) if weights else None
    ref = op.get_pa_metadata_packed(sq, ctx, gqa, nhk, nhk * nspk, gran, ql, quota_of=qf) if pack else None
    assert (ref is not None) == pack  # the packed case packs
    if ref is None:
        ref = op.get_pa_metadata_v1(sq, ctx, gqa, nhk, nhk * nspk, gran, ql, quota_of=qf)
    got["num_reduce_groups"] = ref["num_reduce_groups"]
    for key, val in op.metadata_valid_prefixes(ref).items():
        np.testing.assert_array_equal(op.metadata_valid_prefixes(got)[key], val, err_msg=key)


@pytest.mark.parametrize("seed", range(60))
def test_device_packing_schedule_matches_oracle(seed):
    """The device scheduler with pack = 1 (get_pa_metadata's tuned schedule) on the
    oracle's random packing cases (weights, empty sequences, one bin per head, more
    bins than batches): bit-exact with the oracle's packing schedule where it
    applies and with its sequential fill (same quotas) where it does not."""
    from tests.test_planners import _packed_case

    rng = np.random.default_rng(7000 + seed)
    nhk, nspk, b, ctx, weights = _packed_case(rng)
    ql, gqa = int(rng.integers(1, 5)), int(rng.choice([1, 4, 16]))
    sq = [i * ql for i in range(b + 1)]
    qf = weighted_quota(weights, nspk, ctx) if weights else None
    ref = op.get_pa_metadata_packed(sq, ctx, gqa, nhk, nhk * nspk, 256, ql, quota_of=qf)
    if ref is None:
        ref = op.get_pa_metadata_v1(sq, ctx, gqa, nhk, nhk * nspk, 256, ql, quota_of=qf)
    got, count = run_device_schedule(ctx, ql, gqa, nhk, nspk, 256, weights, True)
    got["num_reduce_groups"] = ref["num_reduce_groups"]
    for key, val in op.metadata_valid_prefixes(ref).items():
        np.testing.assert_array_equal(op.metadata_valid_prefixes(got)[key], val, err_msg=key)
    assert count == int(ref["reduce_indptr"][-1])
    # pack = 0 on the same case is the sequential fill
    seq = op.get_pa_metadata_v1(sq, ctx, gqa, nhk, nhk * nspk, 256, ql, quota_of=qf)
    got0, _ = run_device_schedule(ctx, ql, gqa, nhk, nspk, 256, weights, False)
    got0["num_reduce_groups"] = seq["num_reduce_groups"]
    for key, val in op.metadata_valid_prefixes(seq).items():
        np.testing.assert_array_equal(op.metadata_valid_prefixes(got0)[key], val, err_msg=key)


@pytest.mark.parametrize("b", [1, 24, 48, 97, 700])
def test_device_packing_schedule_equal_contexts(b):
    """Equal context lengths through the packing schedule with dispatch-round weights set
    (the scheduler then knows the lengths are equal, keeps even quotas and takes both
    rank orders as the identity): bit-exact with the oracle's packing schedule, with
    fewer, as many and more sequences than bins per head."""
    nhk, nspk, weights, ql, gqa = 4, 48, [115, 107, 100], 2, 4
    ctx = [3000 + 7 * b] * b
    sq = [i * ql for i in range(b + 1)]
    ref = op.get_pa_metadata_packed(sq, ctx, gqa, nhk, nhk * nspk, 256, ql, quota_of=None)
    if ref is None:
        ref = op.get_pa_metadata_v1(sq, ctx, gqa, nhk, nhk * nspk, 256, ql, quota_of=None)
    got, count = run_device_schedule(ctx, ql, gqa, nhk, nspk, 256, weights, True)
    got["num_reduce_groups"] = ref["num_reduce_groups"]
    for key, val in op.metadata_valid_prefixes(ref).items():
        np.testing.assert_array_equal(op.metadata_valid_prefixes(got)[key], val, err_msg=key)
    assert count == int(ref["reduce_indptr"][-1])


def _metadata_for(name):
    from flydsl_amd import get_pa_metadata
    from flydsl_amd.workloads import CONFIGS, context_lengths_for

    cfg = CONFIGS[name]
    ctx = context_lengths_for(cfg)
    b, ql, hq, hk, bs = len(ctx), cfg.query_length, cfg.num_q_heads, cfg.num_kv_heads, cfg.block_size
    dev = torch.device("cuda:0")
    q = torch.zeros(b * ql, hq, 128, dtype=torch.bfloat16, device=dev)
    kc = torch.zeros(1, hk, 8, bs, 16, dtype=torch.uint8, device=dev)
    md = get_pa_metadata(q, kc, torch.tensor(ctx, dtype=torch.int32, device=dev),
                         torch.zeros(b + 1, dtype=torch.int32, device=dev), hq, hk)
    return md, ctx, b, ql, hq, hk


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
def test_get_pa_metadata_reference_keys_are_the_reference_schedule(name):
    """The keys the reference returns hold the reference's schedule byte for byte:
    (3 CUs // Hkv) * Hkv bins with even quotas (kernels/pa_decode_fp8.py:1764-1771,
    kernels/pa_metadata.py:197-206), partial buffers sized by its split count."""
    md, ctx, b, ql, hq, hk = _metadata_for(name)
    assert md["num_sm"] == reference_num_sm(hk)
    ref = op.get_pa_metadata_v1([ql * i for i in range(b + 1)], ctx, hq // hk, hk, md["num_sm"], 256, ql)
    v = assert_schedule_equal(md, ref, name)
    npart = int(v["reduce_indptr"][-1])
    assert md["partial_output"].shape == ((npart + 1) * ql, 1, hq, 128)
    assert md["partial_lse"].shape == ((npart + 1) * ql, 1, hq, 1)
    parts = (np.asarray(ctx) + 255) // 256
    np.testing.assert_array_equal(md["partition_indptr"].cpu().numpy(), np.concatenate([[0], np.cumsum(parts)]))
    assert "bin_groups" not in md  # the weights belong to the tuned schedule only


def test_get_pa_metadata_c3_tuned_schedule():
    """The tuned schedule on the ragged benchmark shape: two bins per CU (two
    register-streaming worklist workgroups fit a CU), quotas weighted by dispatch
    round, against the oracle's state machine run with the same per-bin quotas."""
    md, ctx, b, ql, hq, hk = _metadata_for("c3")
    t = md["tuned"]
    cus = torch.cuda.get_device_properties(torch.device("cuda:0")).multi_processor_count
    assert t["num_sm"] == (cus * 2 // 8) * 8
    assert t["bin_groups"] == 2 and t["bin_weight"] is not None  # c3's 1749 partitions >= 4 * 64
    v = assert_schedule_equal(t, expected_schedule(t, list(range(129)), ctx, 4, 8), "c3 tuned")
    npart = int(v["reduce_indptr"][-1])
    assert t["partial_output"].shape == ((npart + 1) * 1, 1, 32, 128)


def test_get_pa_metadata_equal_contexts_take_even_quotas():
    """Equal context lengths (c2) keep the tuned schedule's quotas even: the 64
    sequences of 16 partitions fill the 64 bins of each kv head whole, so nothing
    is split and nothing is merged, bit-exact with the oracle's packing schedule
    under even quotas."""
    md, ctx, b, ql, hq, hk = _metadata_for("c2")
    t = md["tuned"]
    assert len(set(ctx)) == 1 and t["bin_groups"] == 2  # weights requested, not applied
    sq = [ql * i for i in range(b + 1)]
    ref = op.get_pa_metadata_packed(sq, ctx, hq // hk, hk, t["num_sm"], 256, ql)
    assert ref is not None
    v = assert_schedule_equal(t, ref, "c2 tuned")
    if t["num_sm"] // hk == b:  # one bin per sequence and head
        assert int(v["reduce_indptr"][-1]) == 0
        info = v["work_info"]
        assert (info[:, 1] == -1).all() and len(info) == b * hk


def test_get_pa_metadata_c5_shape_weighted_quotas():
    """The staged kernel's schedule (three bins per CU) on the c5 shape: quotas
    weighted by dispatch round, against the oracle's state machine run with the
    same per-bin quotas; the first round's bins hold the most partitions."""
    md, ctx, b, ql, hq, hk = _metadata_for("c5")
    md = md["tuned"]
    cus = torch.cuda.get_device_properties(torch.device("cuda:0")).multi_processor_count
    assert md["num_sm"] == (cus * 3 // hk) * hk
    if md["bin_groups"] != 3:
        pytest.skip("the device's CU count does not split into whole groups of bins")
    ref = expected_schedule(md, [ql * i for i in range(b + 1)], ctx, hq // hk, hk, ql=ql)
    v = op.metadata_valid_prefixes(ref)
    np.testing.assert_array_equal(md["work_indptr"].cpu().numpy(), v["work_indptr"])
    nw = int(v["work_indptr"][-1])
    info = md["work_info_flat"].cpu().numpy()[: nw * 8].reshape(nw, 8)
    np.testing.assert_array_equal(info, v["work_info"])
    np.testing.assert_array_equal(md["reduce_indptr"].cpu().numpy(), v["reduce_indptr"])
    ng = int(v["reduce_indptr"][-1])
    np.testing.assert_array_equal(md["reduce_partial_map"].cpu().numpy()[:ng], v["reduce_partial_map"][:ng])
    # partitions per bin of head 0, by group
    nspk = md["num_sm"] // hk
    wi = md["work_indptr"].cpu().numpy()
    per_bin = [int((info[wi[c]:wi[c + 1], 5] - info[wi[c]:wi[c + 1], 4]).sum()) for c in range(nspk)]
    m = nspk // 3
    g = [np.mean(per_bin[k * m:(k + 1) * m]) for k in range(3)]
    assert g[0] > g[1] > g[2]
    assert sum(per_bin) == sum((c + 255) // 256 for c in ctx)


def test_device_scheduler_past_the_lds_staging_capacity():
    """More batches than the scheduler stages in LDS (8192): the rest are read
    from global memory, with the same result."""
    rng = np.random.default_rng(99)
    ctx = [int(x) for x in rng.integers(1, 600, size=9000)]
    got, ref = run_device(ctx, 2, 4, 2, 64, 256)
    for key, val in op.metadata_valid_prefixes(ref).items():
        np.testing.assert_array_equal(op.metadata_valid_prefixes(got)[key], val, err_msg=key)


@pytest.mark.parametrize("b,nhk,num_cu", [(3000, 1, 512), (200, 8, 4104)])
def test_device_scheduler_ring_wrap_and_large_bin_counts(b, nhk, num_cu):
    """More works than the scheduler's 1024-row LDS ring (copied out as it fills),
    and more bins than its LDS copy of work_indptr holds."""
    rng = np.random.default_rng(b)
    ctx = [int(x) for x in rng.integers(1, 3000, size=b)]
    got, ref = run_device(ctx, 1, 4, nhk, num_cu, 256)
    for key, val in op.metadata_valid_prefixes(ref).items():
        np.testing.assert_array_equal(op.metadata_valid_prefixes(got)[key], val, err_msg=key)


@pytest.mark.parametrize(
    "case",
    [
        "empty_batches",  # zero-length contexts between others (closed-form path)
        "few_partitions",  # fewer partitions than bins per head (serial path)
        "one_bin_per_head",  # nspk == 1 (closed-form path, any partition count)
        "all_empty_one_bin",  # every context 0 with one bin per head (closed-form path)
        "all_empty",  # every context 0, several bins (serial path)
        "max_parallel_batches",  # 4096 batches (closed-form path)
        "serial_batches",  # 4097 batches (serial path)
    ],
)
def test_device_scheduler_closed_form_and_serial_paths(case):
    """The parallel closed-form scheduler and the serial state machine it falls back
    to, on the shapes that select each one, bit-exact with the oracle."""
    rng = np.random.default_rng(sum(map(ord, case)))
    ql, gqa, gran = 2, 4, 256
    if case == "empty_batches":
        ctx = [int(x) if rng.random() < 0.7 else 0 for x in rng.integers(1, 4000, size=60)]
        nhk, num_cu = 4, 64
    elif case == "few_partitions":
        ctx = [int(x) for x in rng.integers(1, 300, size=5)]
        nhk, num_cu = 2, 64
    elif case == "one_bin_per_head":
        ctx = [int(x) for x in rng.integers(0, 3000, size=37)]
        nhk, num_cu = 8, 8
    elif case == "all_empty_one_bin":
        ctx = [0] * 9
        nhk, num_cu = 4, 4
    elif case == "all_empty":
        ctx = [0] * 9
        nhk, num_cu = 4, 32
    elif case == "max_parallel_batches":
        ctx = [int(x) for x in rng.integers(0, 2000, size=4096)]
        nhk, num_cu = 8, 512
    else:
        ctx = [int(x) for x in rng.integers(0, 2000, size=4097)]
        nhk, num_cu = 8, 512
    got, ref = run_device(ctx, ql, gqa, nhk, num_cu, gran)
    for key, val in op.metadata_valid_prefixes(ref).items():
        np.testing.assert_array_equal(op.metadata_valid_prefixes(got)[key], val, err_msg=key)


@pytest.mark.parametrize("b,kind", [(1, "uniform"), (37, "ragged"), (37, "uniform"), (4096, "ragged"),
                                    (9000, "ragged"), (9000, "uniform"), (9000, "last_differs")])
def test_get_pa_metadata_partition_prefix_and_uniform_flag(b, kind):
    """get_pa_metadata's partition_indptr (the exclusive prefix of ceil(ctx / 256),
    computed by the scheduler kernel in chunks of 4096 batches) and its
    uniform_context flag (every context length equal), against numpy; the
    schedule itself against the oracle."""
    from flydsl_amd import get_pa_metadata

    rng = np.random.default_rng(b + len(kind))
    if kind == "ragged":
        ctx = rng.integers(1, 5000, size=b)
    else:
        ctx = np.full(b, 1777)
        if kind == "last_differs":
            ctx[-1] = 1778
    dev = torch.device("cuda:0")
    q = torch.zeros(b, 16, 128, dtype=torch.bfloat16, device=dev)
    kc = torch.zeros(1, 2, 8, 16, 16, dtype=torch.uint8, device=dev)
    ctx_t = torch.tensor(ctx, dtype=torch.int32, device=dev)
    kv = torch.zeros(b + 1, dtype=torch.int32, device=dev)
    md = get_pa_metadata(q, kc, ctx_t, kv, 16, 2)
    parts = (ctx.astype(np.int64) + 255) // 256
    np.testing.assert_array_equal(md["partition_indptr"].cpu().numpy(), np.concatenate([[0], np.cumsum(parts)]))
    assert md["uniform_context"] is (kind != "ragged" and kind != "last_differs")
    sq, cl = list(range(b + 1)), [int(c) for c in ctx]
    for label, s in (("reference", md), ("tuned", md["tuned"])):
        v = assert_schedule_equal(s, expected_schedule(s, sq, cl, 8, 2), f"{b} {kind} {label}")
        assert s["partial_output"].shape[0] == int(v["reduce_indptr"][-1]) + 1
    assert md["num_sm"] == reference_num_sm(2)
    # graph-safe: same schedules, no host read, partial buffers at the scheduler's bound
    md_g = get_pa_metadata(q, kc, ctx_t, kv, 16, 2, graph_safe=True)
    assert md_g["uniform_context"] is False
    assert torch.equal(md_g["partition_indptr"], md["partition_indptr"])
    for s_g, s in ((md_g, md), (md_g["tuned"], md["tuned"])):
        assert torch.equal(s_g["work_indptr"], s["work_indptr"])
        assert s_g["partial_output"].shape[0] == s_g["reduce_partial_map"].numel() + 1
    # tuned=False: the reference's dict only
    md_r = get_pa_metadata(q, kc, ctx_t, kv, 16, 2, tuned=False)
    assert "tuned" not in md_r and torch.equal(md_r["work_indptr"], md["work_indptr"])


@pytest.mark.parametrize("seed", range(6))
def test_get_pa_metadata_random_shapes_both_schedules(seed):
    """Random batches, heads, query lengths and group sizes: the reference keys
    against the oracle's even schedule over the reference's bin count, the tuned
    entry against the oracle run with its weights."""
    from flydsl_amd import get_pa_metadata

    rng = np.random.default_rng(1000 + seed)
    hk = int(rng.choice([1, 2, 4, 8]))
    g = int(rng.choice([1, 4, 8, 16]))
    ql = int(rng.integers(1, 5))
    b = int(rng.integers(1, 300))
    ctx = rng.integers(0, int(rng.choice([600, 9000, 40000])), size=b)
    dev = torch.device("cuda:0")
    q = torch.zeros(b * ql, hk * g, 128, dtype=torch.bfloat16, device=dev)
    kc = torch.zeros(1, hk, 8, 16, 16, dtype=torch.uint8, device=dev)
    md = get_pa_metadata(q, kc, torch.tensor(ctx, dtype=torch.int32, device=dev),
                         torch.zeros(b + 1, dtype=torch.int32, device=dev), hk * g, hk)
    sq, cl = [ql * i for i in range(b + 1)], [int(c) for c in ctx]
    assert md["num_sm"] == reference_num_sm(hk)
    for label, s in (("reference", md), ("tuned", md["tuned"])):
        v = assert_schedule_equal(s, expected_schedule(s, sq, cl, g, hk, ql=ql), f"seed {seed} {label}")
        assert s["partial_output"].shape[0] == (int(v["reduce_indptr"][-1]) + 1) * ql
