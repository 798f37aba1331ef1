"""Device worklist scheduler (get_pa_metadata_v1 / get_pa_metadata) vs the CPU
oracle: bit-exact on every byte the reference defines (the valid prefixes)."""

import numpy as np
import pytest
import torch

from oracle import planners as op

pytestmark = pytest.mark.gpu


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


def test_get_pa_metadata_c3_shape():
    """The host entry point on the ragged benchmark shape (512 bins on 256 CUs)."""
    from flydsl_amd import get_pa_metadata
    from flydsl_amd.workloads import CONFIGS, context_lengths_for

    ctx = context_lengths_for(CONFIGS["c3"])
    dev = torch.device("cuda:0")
    q = torch.zeros(128, 32, 128, dtype=torch.bfloat16, device=dev)
    kc = torch.zeros(1, 8, 8, 16, 16, dtype=torch.uint8, device=dev)
    md = get_pa_metadata(q, kc, torch.tensor(ctx, dtype=torch.int32, device=dev),
                         torch.zeros(129, dtype=torch.int32, device=dev), 32, 8)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    num_sm = (cus * 2 // 8) * 8  # two bins per CU: two worklist workgroups fit a CU
    assert md["num_sm"] == num_sm
    ref = op.get_pa_metadata_v1(list(range(129)), ctx, 4, 8, num_sm, 256, 1)
    v = op.metadata_valid_prefixes(ref)
    np.testing.assert_array_equal(md["work_indptr"].cpu().numpy(), v["work_indptr"])
    nw = int(v["work_indptr"][-1])
    np.testing.assert_array_equal(md["work_info_flat"].cpu().numpy()[: nw * 8].reshape(nw, 8), v["work_info"])
    np.testing.assert_array_equal(md["reduce_indptr"].cpu().numpy(), v["reduce_indptr"])
    parts = (np.asarray(ctx) + 255) // 256
    np.testing.assert_array_equal(md["partition_indptr"].cpu().numpy(), np.concatenate([[0], np.cumsum(parts)]))
    npart = int(v["reduce_indptr"][-1])
    assert md["partial_output"].shape == ((npart + 1) * 1, 1, 32, 128)


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
