"""Pins the CPU oracle (``oracle/``) against checks that do not restate it.

* the worked example of ``docs/OnlineSoftmax 原理详解.html`` (§5.1, §6.3, §7.2):
  scores [1,3,2,5,4,0], values [10..60] -> 40.038 / LSE 5.4563, and with
  sink 2 -> 38.813 / LSE 5.4873;
* the float64 one-shot softmax over scores ∪ {sink} (golden.py:207-244), at
  the reference's own test parameters (test_sparse_attn_sharedkv.py:930-1002);
* tile-size invariance of the chunked recurrence;
* brute-force set semantics of the top-k / window index resolution;
* pack/unpack round trips of the paged pools;
* partition invariance of the split-KV merge.
Each check is chosen so a plausible slip (dropped sink, wrong max, skipped -1
break, transposed operand) fails it; ``test_checks_have_teeth`` plants such
slips in oracle outputs and asserts the checks fire.
"""

import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import gen
from oracle.checks import check_result, check_strict
from oracle.golden_ref import (attend_token, cmp_threshold, gather_paged_rows, merge_partials,
                               one_shot_reference, resolve_topk_rows, sparse_attn_oracle,
                               window_range)

KAT = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                  "online_softmax_docs_kat.json"), encoding="utf-8"))
SCORES = KAT["scores"]
VALUES = KAT["values"]


def _kat_rows():
    # Shared K = V rows [value, score]; q = [0, 1] with scale 1 gives score_i.
    return torch.tensor([[v, s] for v, s in zip(VALUES, SCORES)], dtype=torch.float32)


@pytest.mark.parametrize("tile", [3, 512])
@pytest.mark.parametrize("case", range(len(KAT["cases"])))
def test_docs_worked_example(tile, case):
    c = KAT["cases"][case]
    q = torch.tensor([[0.0, 1.0]])
    sink = float("-inf") if c["sink"] is None else c["sink"]
    out, lse = attend_token(q, [_kat_rows()], torch.tensor([sink]), 1.0, tile=tile)
    assert abs(float(out[0, 0]) - c["out"]) < KAT["tolerance"]["out"]
    assert abs(float(lse[0]) - c["lse"]) < KAT["tolerance"]["lse"]


def test_empty_row_set_gives_zero_and_sink_lse():
    q = torch.randn(4, 8)
    sinks = torch.tensor([0.5, -1.0, float("-inf"), 2.0])
    out, lse = attend_token(q, [torch.zeros(0, 8)], sinks, 0.3)
    assert torch.equal(out, torch.zeros(4, 8))
    assert torch.equal(lse, sinks)


def _reference_small_case(dtype):
    # test_sparse_attn_sharedkv.py:930-1002 parameters: B=1, S1=4, N1=64, D=512, K=8
    g = torch.Generator().manual_seed(0)
    s1, n1, d, k, kv, ratio = 4, 64, 512, 8, 128, 4
    q = (torch.rand((s1, n1, d), generator=g) * 2 - 1).to(dtype)
    ori = (torch.rand((kv, d), generator=g) * 2 - 1).to(dtype)
    cmp = (torch.rand((kv // ratio, d), generator=g) * 2 - 1).to(dtype)
    sinks = torch.rand(n1, generator=g) * 0.1
    idx = torch.full((s1, k), -1, dtype=torch.int64)
    for s in range(s1):
        thr = (kv - s1 + s + 1) // ratio
        idx[s, :min(k, thr)] = torch.arange(min(k, thr))
    return q, ori, cmp, sinks, idx, s1, kv, ratio, 1.0 / math.sqrt(d)


def test_chunked_matches_one_shot_fp32():
    q, ori, cmp, sinks, idx, s1, kv, ratio, scale = _reference_small_case(torch.float32)
    for s in range(s1):
        sg = kv - s1 + s
        lo, hi = window_range(sg, 127)
        crow = resolve_topk_rows(idx[s].tolist(), kv, s1, s, ratio)
        segs = [ori[lo:hi], cmp[crow]]
        out, lse = attend_token(q[s], segs, sinks, scale)
        ref, ref_lse = one_shot_reference(q[s].numpy(), torch.cat(segs).numpy(), sinks.numpy(),
                                          scale)
        np.testing.assert_allclose(out.numpy(), ref, rtol=2e-4, atol=2e-4)
        np.testing.assert_allclose(lse.numpy(), ref_lse, rtol=1e-4, atol=1e-4)


def test_chunked_matches_one_shot_bf16_within_port_tolerance():
    q, ori, cmp, sinks, idx, s1, kv, ratio, scale = _reference_small_case(torch.bfloat16)
    for s in range(s1):
        sg = kv - s1 + s
        lo, hi = window_range(sg, 127)
        crow = resolve_topk_rows(idx[s].tolist(), kv, s1, s, ratio)
        segs = [ori[lo:hi], cmp[crow]]
        out, lse = attend_token(q[s], segs, sinks, scale, tile=16)
        ref, ref_lse = one_shot_reference(q[s].float().numpy(), torch.cat(segs).float().numpy(),
                                          sinks.numpy(), scale)
        check_strict(out, torch.from_numpy(ref).float(), lse, torch.from_numpy(ref_lse).float())


def test_tile_size_invariance_fp32():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(16, 64, generator=g)
    rows = torch.randn(300, 64, generator=g) * 2
    sinks = torch.randn(16, generator=g)
    a, la = attend_token(q, [rows[:77], rows[77:]], sinks, 0.125, tile=512)
    b, lb = attend_token(q, [rows[:77], rows[77:]], sinks, 0.125, tile=7)
    torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(la, lb, rtol=1e-6, atol=1e-5)


def test_head_dim_v_is_a_column_slice():
    g = torch.Generator().manual_seed(5)
    q = torch.randn(8, 576, generator=g)
    rows = torch.randn(40, 576, generator=g)
    sinks = torch.randn(8, generator=g)
    full, lf = attend_token(q, [rows], sinks, 1 / 24)
    part, lp = attend_token(q, [rows], sinks, 1 / 24, d_v=512)
    torch.testing.assert_close(full[:, :512], part, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(lf, lp)


def _brute_topk(ids, act_kv, act_q, s, ratio):
    thr = (act_kv - act_q + s + 1) // ratio
    n = max(0, min(len(ids), thr))
    stop = next((i for i in range(n) if ids[i] == -1), n)
    return [v for v in ids[:stop] if 0 <= v < thr]


def test_topk_resolution_brute_force():
    rng = np.random.default_rng(11)
    for _ in range(2000):
        k = int(rng.integers(1, 12))
        act_q = int(rng.integers(1, 4))
        act_kv = int(rng.integers(act_q, 60))
        ratio = int(rng.choice([1, 2, 4]))
        s = int(rng.integers(0, act_q))
        ids = rng.integers(-1, act_kv // ratio + 3, size=k).tolist()
        got = resolve_topk_rows(ids, act_kv, act_q, s, ratio)
        assert got == _brute_topk(ids, act_kv, act_q, s, ratio), (ids, act_kv, act_q, s, ratio)


def test_topk_break_at_minus_one_is_a_stop_not_a_skip():
    # act_kv=16, act_q=1, s=0, ratio=1 -> thr=16
    assert resolve_topk_rows([3, -1, 5, 7], 16, 1, 0, 1) == [3]
    assert resolve_topk_rows([3, 20, 5, 5], 16, 1, 0, 1) == [3, 5, 5]
    assert resolve_topk_rows([15, 16], 16, 1, 0, 1) == [15]


def test_window_range():
    assert window_range(200, 127) == (73, 201)
    assert window_range(5, 127) == (0, 6)
    assert window_range(5, -1) == (6, 6)  # pure top-k: empty window
    assert cmp_threshold(8193, 1, 0, 4) == 2048


def test_paging_round_trip():
    rng = np.random.default_rng(2)
    g = torch.Generator().manual_seed(2)
    lens = [130, 64, 1, 257]
    dense = [torch.randn(n, 32, generator=g) for n in lens]
    flat = iter(torch.cat(dense).split(1))
    pool, table = gen.paged_pool(seq_lens=lens, block_size=64, block_num=12, head_dim=32,
                                 dtype=torch.float32, rng=rng,
                                 values=lambda shape: torch.zeros(shape))
    for b, n in enumerate(lens):
        for p in range(n):
            pool[table[b, p // 64], p % 64, 0] = dense[b][p]
    for b, n in enumerate(lens):
        assert torch.equal(gather_paged_rows(pool, table, b, range(n)), dense[b])
    # each sequence owns distinct physical blocks
    used = table[table >= 0].tolist()
    assert len(used) == len(set(used)) == sum(math.ceil(n / 64) for n in lens)
    del flat


def test_merge_partition_invariance():
    g = torch.Generator().manual_seed(9)
    q = torch.randn(6, 32, generator=g).numpy()
    rows = torch.randn(97, 32, generator=g).numpy()
    sinks = np.array([0.3, -2.0, float("-inf"), 1.0, 0.0, -0.5])
    full, lfull = one_shot_reference(q, rows, sinks, 0.2)
    cuts = [0, 10, 11, 50, 97]
    parts = [one_shot_reference(q, rows[a:b], np.full(6, -np.inf), 0.2)
             for a, b in zip(cuts[:-1], cuts[1:])]
    out, lse = merge_partials([p[0] for p in parts], [p[1] for p in parts], sinks)
    np.testing.assert_allclose(out, full, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse, lfull, rtol=1e-12)


def test_generated_indices_follow_golden_invariants():
    g = torch.Generator().manual_seed(1)
    idx = gen.topk_indices(thresholds=[0, 3, 10, 600], k=8, gen=g)
    assert (idx[0] == -1).all()
    assert sorted(idx[1, :3].tolist()) == [0, 1, 2] and (idx[1, 3:] == -1).all()
    assert len(set(idx[2].tolist())) == 8 and (idx[2] < 10).all()
    assert (idx[3] >= 0).all() and (idx[3] < 600).all() and len(set(idx[3].tolist())) == 8


def test_oracle_driver_matches_per_token_attend():
    cfg = gen.multibatch_case("scfa_prefill", seqs=(40, 24))
    cfg = dict(cfg, block_size1=16, block_size2=4, block_num1=8, block_num2=6)
    case = gen.build_case(cfg, torch.bfloat16)
    kw = {k: v for k, v in case.items() if k not in ("topk_cmp",)}
    out, lse = sparse_attn_oracle(**kw)
    assert out.shape == (64, 64, 512) and lse.shape == (64, 64)
    # token 45 = batch 1, s = 5: recompute directly from dense gathers
    b, s, act_q, act_kv = 1, 5, 24, 24
    sg = act_kv - act_q + s
    lo, hi = window_range(sg, 127)
    ori = gather_paged_rows(case["ori_kv"], case["ori_block_table"], b, range(lo, hi))
    crow = resolve_topk_rows(case["cmp_sparse_indices"][45, 0].tolist(), act_kv, act_q, s, 4)
    cmp = gather_paged_rows(case["cmp_kv"], case["cmp_block_table"], b, crow)
    o, l = attend_token(case["q"][45], [ori, cmp], case["sinks"], case["softmax_scale"])
    assert torch.equal(out[45], o) and torch.equal(lse[45], l)


def test_checks_have_teeth():
    g = torch.Generator().manual_seed(4)
    q = torch.randn(8, 64, generator=g).to(torch.bfloat16)
    rows = torch.randn(50, 64, generator=g).to(torch.bfloat16)
    sinks = torch.randn(8, generator=g)
    good, lse = attend_token(q, [rows], sinks, 0.125)
    check_strict(good, good, lse, lse)
    # planted slip 1: sink dropped
    no_sink, l2 = attend_token(q, [rows], torch.full((8,), float("-inf")), 0.125)
    with pytest.raises(AssertionError):
        check_strict(no_sink, good, l2, lse)
    # planted slip 2: one row missing (a skipped index)
    miss, l3 = attend_token(q, [rows[1:]], sinks, 0.125)
    with pytest.raises(AssertionError):
        check_strict(miss, good, l3, lse)
    # planted slip 3: transposed / permuted heads
    with pytest.raises(AssertionError):
        check_result(good.flip(0), good)
