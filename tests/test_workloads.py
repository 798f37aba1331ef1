"""Synthetic benchmark workloads (CPU): the KV-cache copies the bench rotates
hold exactly the pages their shared block tables and page lists index, so no
index reaches past a copy's last page (where the kernels' bounds guard would
clamp it and the copy would read fewer distinct bytes than counted)."""

from __future__ import annotations

import pytest
import torch

from flydsl_amd.workloads import CONFIGS, SHARED_KEYS, build_workload_copies, scaled


@pytest.mark.parametrize("name", ["c2", "c3", "c4", "c5"])
def test_copies_index_only_their_own_pages(name):
    base_cfg = CONFIGS[name]
    # a few sequences, with contexts drawn per seed as in the benchmark (shorter)
    cfg = scaled(base_cfg, batch=5, ctx_b=min(base_cfg.ctx_b, 3000), ctx_a=min(base_cfg.ctx_a, 200))
    works = build_workload_copies(cfg, "cpu", 3)
    base = works[0]
    nblocks = base["key_cache"].shape[0]
    for w in works:
        assert w["key_cache"].shape[0] == nblocks and w["value_cache"].shape[0] == nblocks
        if cfg.per_token:
            assert w["key_scale"].shape[0] == nblocks
        for k in SHARED_KEYS:
            assert w[k] is base[k]
        pages = [(c + cfg.block_size - 1) // cfg.block_size for c in w["context_list"]]
        bt = w["block_tables"]
        used = torch.cat([bt[b, : pages[b]] for b in range(cfg.batch)])
        # every page a sequence reads is a distinct page of this copy
        assert int(used.max()) < nblocks and int(used.min()) >= 0
        assert used.unique().numel() == used.numel()
        assert int(w["kv_page_indices"].max()) < nblocks
    # the copies hold different bytes
    assert not torch.equal(works[0]["key_cache"], works[1]["key_cache"])
