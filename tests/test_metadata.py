"""Scheduler tests (CPU): the reference's metadata invariants plus exact block coverage.

Restates test_sparse_attn_sharedkv.py:721-924 against this library's
scheduler: int32 output of SAS_META_SIZE words, enabled cores chained
(each resumes where its predecessor stopped), last core ends at bn2 = B,
large prefill fans out over all cores. Adds a stricter check than the
reference's linearised (bn2, m) walk: every (item, block) pair of every item
is covered by exactly one core, and the FD merge rows list exactly the
partial pieces the kernel writes, in slot order.
"""

import math

import pytest
import torch

from oracle import gen
from oracle.golden_ref import causal_position, cmp_threshold, window_range
from sparse_attn_sharedkv_amd import metadata as M
from sparse_attn_sharedkv_amd.metadata import (AIC_CORE_NUM, AIV_CORE_NUM, FA_METADATA_SIZE,
                                               FD_METADATA_SIZE, SAS_META_SIZE, config_row,
                                               sparse_attn_sharedkv_metadata)


def _kwargs(cfg, **over):
    scen = cfg["scenario"]
    kw = dict(num_heads_q=cfg["N1"], num_heads_kv=cfg["N2"], head_dim=cfg["D"],
              cu_seqlens_q=torch.tensor(cfg["cu_seqlens_q"], dtype=torch.int32)
              if cfg["layout_q"] == "TND" else None,
              seqused_kv=torch.tensor(cfg["seqused_kv"], dtype=torch.int32),
              batch_size=cfg["B"],
              max_seqlen_q=cfg.get("T1") if cfg["layout_q"] == "TND" else cfg["S1"],
              max_seqlen_kv=max(cfg["seqused_kv"]), ori_mask_mode=cfg["ori_mask_mode"],
              ori_win_left=cfg["ori_win_left"], ori_win_right=cfg["ori_win_right"],
              layout_q=cfg["layout_q"], layout_kv="PA_ND", has_ori_kv=True,
              has_cmp_kv=scen >= 2)
    if scen >= 2:
        kw.update(cmp_ratio=cfg["cmp_ratio"], cmp_mask_mode=cfg["cmp_mask_mode"])
    if scen == 3:
        kw["cmp_topk"] = cfg["K"]
    kw.update(over)
    return kw


def _items(act_q, act_kv, n1, win_left, scen, ratio, topk, s2b):
    """Independent restatement of the item list: [(b, m, nblk)]."""
    mb = M.m_base_for(n1, batch=len(act_q))
    hb = (n1 + mb - 1) // mb
    items = []
    for b, (aq, ak) in enumerate(zip(act_q, act_kv)):
        for s in range(aq):
            lo, hi = window_range(causal_position(ak, aq, s), win_left)
            ncmp = 0
            if scen >= 2:
                thr = cmp_threshold(ak, aq, s, ratio)
                ncmp = max(0, min(topk, thr) if scen == 3 else thr)
            n = (hi - lo) + ncmp
            for h in range(hb):
                items.append((b, s * hb + h, math.ceil(n / s2b)))
    return items


def _check_schedule(md, act_q, act_kv, n1, win_left, scen, ratio, topk, ncores):
    assert md.dtype == torch.int32 and md.shape == (SAS_META_SIZE,)
    cfg = config_row(md)
    fa = md[:AIC_CORE_NUM * FA_METADATA_SIZE].view(AIC_CORE_NUM, FA_METADATA_SIZE).tolist()
    fd = md[M.FD_OFFSET:M.FD_OFFSET + AIV_CORE_NUM * FD_METADATA_SIZE].view(
        AIV_CORE_NUM, FD_METADATA_SIZE).tolist()
    used = [r for r in fa if r[0] == 1]
    assert 1 <= len(used) <= ncores and len(used) == cfg["num_fa"]
    assert all(r[0] == 0 for r in fa[len(used):]), "enabled rows must be a prefix"
    # continuity (test_sparse_attn_sharedkv.py:776-792)
    prev = (0, 0, 0)
    for r in used:
        assert tuple(r[1:4]) == prev
        prev = tuple(r[4:7])
    assert prev == (len(act_q), 0, 0)
    # exact-once block coverage and partial-slot bookkeeping
    assert cfg["m_base"] == M.m_base_for(n1, batch=len(act_q))
    items = _items(act_q, act_kv, n1, win_left, scen, ratio, topk, cfg["s2_base"])
    import bisect
    keys = [(b, m) for (b, m, _) in items]

    def locate(cur):  # first item at or after the cursor (the kernel skips empty batches)
        return bisect.bisect_left(keys, tuple(cur))
    seen = {}
    pieces = {}
    for c, r in enumerate(used):
        start, end = (r[1], r[2]), (r[4], r[5])
        i0, i1 = locate(start), locate(end)
        if i1 < len(items) and keys[i1] != end:
            assert r[6] == 0, "a cursor inside an item must name that item"
        slot = r[7]
        for i in range(i0, min(i1 + 1, len(items))):
            if i == i1 and r[6] == 0:
                break
            lo = r[3] if i == i0 else 0
            hi = r[6] if i == i1 else items[i][2]
            assert 0 <= lo <= hi <= items[i][2]
            for blk in range(lo, hi):
                assert (i, blk) not in seen, f"block {(i, blk)} covered twice"
                seen[(i, blk)] = c
            partial = (i == i0 and r[3] > 0) or i == i1
            if partial:
                pieces.setdefault(i, []).append(slot)
                slot += 1
            else:
                assert (i, -1) not in seen
                seen[(i, -1)] = c  # whole item (also items with zero blocks)
    for i, (_, _, nb) in enumerate(items):
        if i in pieces:
            assert all((i, blk) in seen for blk in range(nb))
        else:
            assert (i, -1) in seen, f"item {i} never processed"
    # FD rows: one group per split item, contiguous slots in core order
    fd_used = [r for r in fd if r[0] == 1]
    assert len(fd_used) == cfg["num_fd"]
    mb = min(n1, cfg["m_base"])
    by_item = {}
    for r in fd_used:
        by_item.setdefault((r[1], r[2]), []).append(r)
    split = {i: s for i, s in pieces.items() if len(s) > 1}
    assert len(by_item) == len(split)
    for i, slots in split.items():
        b, m, _ = items[i]
        rows = by_item[(b, m)]
        assert slots == list(range(slots[0], slots[0] + len(slots)))
        assert all(r[3] == slots[0] and r[4] == len(slots) for r in rows)
        heads = sorted((r[5], r[6]) for r in rows)
        cover = []
        for h0, hn in heads:
            cover.extend(range(h0, h0 + hn))
        assert cover == list(range(mb))
    for i, s in pieces.items():
        assert len(s) != 1, "an item with one partial piece would never be finalised"
    assert cfg["num_partial_slots"] == sum(len(s) for s in pieces.values())
    return cfg


CASES = dict(gen.REFERENCE_CASES, **gen.FAST_CASES)


@pytest.mark.parametrize("name", list(CASES))
def test_reference_cases_schedule(name):
    cfg = CASES[name]
    md = sparse_attn_sharedkv_metadata(**_kwargs(cfg))
    act_q, act_kv = M.resolve_lengths(layout_q=cfg["layout_q"], layout_kv="PA_ND",
                                      cu_seqlens_q=torch.tensor(cfg["cu_seqlens_q"]),
                                      seqused_kv=cfg["seqused_kv"], batch_size=cfg["B"],
                                      max_seqlen_q=cfg["S1"])
    _check_schedule(md, act_q, act_kv, cfg["N1"], cfg["ori_win_left"], cfg["scenario"],
                    cfg["cmp_ratio"], cfg.get("K", 0), M.DEFAULT_CORE_NUM)


@pytest.mark.parametrize("cores", [1, 7, 24, 256, 512])
def test_core_counts(cores):
    cfg = CASES["scfa_prefill_b2"]
    md = sparse_attn_sharedkv_metadata(**_kwargs(cfg, aic_core_num=cores))
    act_q, act_kv = [768, 512], [768, 512]
    c = _check_schedule(md, act_q, act_kv, 64, 127, 3, 4, 512, cores)
    assert c["num_fa"] == min(cores, c["total_items"]) or c["num_fa"] <= cores


def test_prefill_uses_all_cores():
    # test_sparse_attn_sharedkv.py:896-924: the 8K prefill spreads over every core
    cfg = CASES["scfa_prefill"]
    for cores in (24, 256):
        md = sparse_attn_sharedkv_metadata(**_kwargs(cfg, aic_core_num=cores))
        # the smallest balanced budget may pack into one core fewer
        assert cores - 1 <= config_row(md)["num_fa"] <= cores


@pytest.mark.parametrize("name", list(gen.WORKLOADS))
def test_benchmark_workload_schedules(name):
    w = gen.WORKLOADS[name]
    lens = [w["ctx"][1]] * w["B"]
    scen = 1 if w["mode"] == "swa" else 3
    md = sparse_attn_sharedkv_metadata(
        num_heads_q=w["H"], num_heads_kv=1, head_dim=w["D"],
        seqused_kv=torch.tensor(lens, dtype=torch.int32), batch_size=w["B"],
        max_seqlen_q=w["S"], max_seqlen_kv=max(lens), cmp_topk=w["K"],
        cmp_ratio=w["cmp_ratio"] or -1, ori_win_left=w["window"], layout_q="BSND",
        has_cmp_kv=scen == 3)
    cfg = _check_schedule(md, [w["S"]] * w["B"], lens, w["H"], w["window"], scen,
                          w["cmp_ratio"] or 1, w["K"], M.DEFAULT_CORE_NUM)
    if name == "mla_decode_b64_h128_k2048":
        # 64 tokens x 2 head blocks, each split in two: one workgroup per CU,
        # one merge task per 64-head item
        assert cfg["num_fa"] == 256 and cfg["num_fd"] == 128


def test_ragged_and_empty_items():
    # zero-length query batches, sequences shorter than the window and the ratio
    act_q, act_kv = [0, 3, 1, 0, 2], [5, 3, 1, 9, 700]
    md = M.build_metadata(act_q=act_q, act_kv=act_kv, num_heads=64, ori_win_left=127,
                          scenario=3, cmp_ratio=4, cmp_topk=16, core_num=256)
    _check_schedule(md, act_q, act_kv, 64, 127, 3, 4, 16, 256)
    md = M.build_metadata(act_q=[0, 0], act_kv=[0, 0], num_heads=16, ori_win_left=-1,
                          scenario=3, cmp_ratio=1, cmp_topk=8, core_num=256)
    assert config_row(md)["num_fa"] == 1


def test_invalid_arguments_raise():
    with pytest.raises(ValueError):
        M.build_metadata(act_q=[1], act_kv=[10], num_heads=64, ori_win_left=127, scenario=3,
                         cmp_ratio=0, cmp_topk=4)
    with pytest.raises(ValueError):
        M.build_metadata(act_q=[1], act_kv=[10], num_heads=64, ori_win_left=127, scenario=1,
                         cmp_ratio=4, cmp_topk=0, core_num=0)
    with pytest.raises(ValueError):
        sparse_attn_sharedkv_metadata(num_heads_q=64, num_heads_kv=2, head_dim=512,
                                      seqused_kv=torch.tensor([10]), batch_size=1,
                                      max_seqlen_q=1)


def test_item_size_rule_for_fp8_rows():
    # above 64 heads: 128-head items from 65 sequences on native rows, from 32 on
    # fp8 rows (either Q·Kᵀ form); the pipelined form and <= 64 heads keep theirs
    assert M.m_base_for(128, batch=64) == 64 and M.m_base_for(128, batch=65) == 128
    assert M.m_base_for(128, batch=31, fp8_rows=True) == 64
    assert M.m_base_for(128, batch=32, fp8_rows=True) == 128
    assert M.m_base_for(96, batch=40, fp8_rows=True) == 128
    assert M.m_base_for(64, batch=512, fp8_rows=True) == 64
    assert M.m_base_for(32, batch=512, fp8_rows=True) == 32
    assert M.m_base_for(128, item64=True, batch=512, fp8_rows=True) == 64
    # a call's own schedule counts query rows (MTP: 64 sequences x 2 rows; prefill)
    assert M.m_base_for(128, batch=64, rows=128) == 128
    assert M.m_base_for(128, batch=1, rows=4096) == 128
    assert M.m_base_for(128, batch=64, rows=64) == 64
    assert M.m_base_for(128, batch=16, rows=32, fp8_rows=True) == 128
    assert M.m_base_for(64, batch=1, rows=8192) == 64
    # the public entry point picks the size from the cache row format it is given
    lens = [3000] * 40
    common = dict(num_heads_q=128, num_heads_kv=1, head_dim=576,
                  seqused_kv=torch.tensor(lens, dtype=torch.int32), batch_size=40,
                  max_seqlen_q=1, max_seqlen_kv=3000, cmp_topk=2048, cmp_ratio=1,
                  ori_win_left=-1, layout_q="BSND", has_cmp_kv=True)
    assert config_row(sparse_attn_sharedkv_metadata(**common))["m_base"] == 64
    md8 = sparse_attn_sharedkv_metadata(**common, kv_cache_dtype="fp8_ds_mla")
    assert config_row(md8)["m_base"] == 128
    md8q = sparse_attn_sharedkv_metadata(**common, kv_cache_dtype="fp8_ds_mla", fp8_qk=True)
    assert torch.equal(md8q, md8)
