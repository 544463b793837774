"""Gathered rows and masks of the HIP path, pinned exactly (integer parity).

With q = 0 every score is 0 and with sinks = -inf there is no virtual key, so
each attended row gets P = 1 exactly: the LSE is ln(n) for n attended rows and
the output is (sum of the attended V rows) / n. Every cache row holds a
one-hot V: raw row p (physical index) at column p, compressed row p at column
256 + p. So n = round(exp(lse)) and round(out * n) give, per query row and
head, the exact multiset of physical rows the kernel gathered (duplicates
counted). Both are compared word for word with the oracle's integer
resolution: ``window_range`` (golden.py:128-131), ``dense_cmp_rows``
(golden.py:146-150), ``resolve_topk_rows`` (golden.py:28-66: stop at the
first -1, skip ids >= thr, keep duplicates) and the block tables.

Block tables map only the blocks a query can reach, so long contexts and
top-k lists wider than one resolution chunk (1024 positions) fit in pools of
at most 256 rows. Covered: windows -1 / 0 / 5 / 7 / 63 / 127 / 1023, ragged TND rows,
dense compressed thresholds at ratios 4 and 16, top-k with -1 in the middle,
ids >= thr, duplicates, all -1 rows, items of more than 1024 positions, split
items (few workgroups), H = 16 / 64 / 128, d_qk 512 / 576, bf16 and fp8 rows, and
the fp8 Q·Kᵀ form (q = 0 quantizes to all-zero codes, so every score is still 0).
"""

import math
import sys

import numpy as np
import pytest
import torch

from oracle.fp8_rows import quantize_rows
from oracle.golden_ref import (causal_position, dense_cmp_rows, resolve_topk_rows,
                               token_layout, window_range)

pytestmark = pytest.mark.gpu

HAS_GPU = torch.cuda.is_available()
requires_gpu = pytest.mark.skipif(not HAS_GPU, reason="needs a ROCm GPU")

if HAS_GPU:
    from sparse_attn_sharedkv_amd import sparse_attn_sharedkv

POOL_ROWS = 256  # one-hot columns per cache


def _say(msg):
    print(f"[gpu-index] {msg}", flush=True)
    sys.stdout.flush()


def _table_for(needed, bs, rng, width):
    """Block table rows mapping the needed logical blocks to distinct physical blocks."""
    nblk = POOL_ROWS // bs
    phys = rng.permutation(nblk)
    table = np.full((len(needed), width), -1, dtype=np.int32)
    cur = 0
    for b, blocks in enumerate(needed):
        for blk in sorted(blocks):
            assert cur < nblk, "test pool too small for the attended blocks"
            table[b, blk] = phys[cur]
            cur += 1
    return table


def _one_hot_pool(bs, d, col0, dtype):
    rows = torch.zeros(POOL_ROWS, d, dtype=torch.float32)
    rows[torch.arange(POOL_ROWS), col0 + torch.arange(POOL_ROWS)] = 1.0
    return rows.to(dtype).reshape(POOL_ROWS // bs, bs, 1, d)


def _case(*, scenario, layout, qlens, kvlens, heads, d, win, ratio=1, k=0, bs1=16, bs2=16,
          seed=0, edit=None, fp8=False):
    rng = np.random.default_rng(seed)
    b = len(qlens)
    s_max = max(qlens)
    # top-k rows: ids from a small range (duplicates), then the case's edits
    idx = None
    tokens = [(bi, s) for bi in range(b) for s in range(qlens[bi])]
    if scenario == 3:
        t_all = sum(qlens) if layout == "TND" else b * s_max
        idx = np.full((t_all, k), -1, dtype=np.int32)
        for bi, s in tokens:
            thr = math.floor((kvlens[bi] - qlens[bi] + s + 1) / ratio)
            hi = max(1, min(thr + 4, 64))  # a few ids at or beyond thr are drawn too
            t = (sum(qlens[:bi]) if layout == "TND" else bi * s_max) + s
            idx[t] = rng.integers(0, hi, size=k)
        if edit is not None:
            edit(idx)
    # logical blocks each sequence can reach
    need1 = [set() for _ in range(b)]
    need2 = [set() for _ in range(b)]
    for bi, s in tokens:
        sg = causal_position(kvlens[bi], qlens[bi], s)
        lo, hi = window_range(sg, win)
        need1[bi].update(p // bs1 for p in range(lo, hi))
        if scenario == 2:
            need2[bi].update(p // bs2 for p in dense_cmp_rows(kvlens[bi], qlens[bi], s, ratio))
        elif scenario == 3:
            t = (sum(qlens[:bi]) if layout == "TND" else bi * s_max) + s
            need2[bi].update(p // bs2 for p in
                             resolve_topk_rows(idx[t].tolist(), kvlens[bi], qlens[bi], s, ratio))
    w1 = max(1, max(math.ceil(x / bs1) for x in kvlens))
    w2 = max(1, max(math.ceil(max(x // ratio, 1) / bs2) for x in kvlens))
    t1 = _table_for(need1, bs1, rng, w1)
    t2 = _table_for(need2, bs2, rng, w2)
    dt = torch.bfloat16
    ori = _one_hot_pool(bs1, d, 0, dt)
    cmp_ = _one_hot_pool(bs2, d, POOL_ROWS, dt)
    if fp8:
        ori = torch.from_numpy(quantize_rows(ori.reshape(-1, d))).reshape(POOL_ROWS // bs1, bs1, 1, 656)
        cmp_ = torch.from_numpy(quantize_rows(cmp_.reshape(-1, d))).reshape(POOL_ROWS // bs2, bs2, 1,
                                                                           656)
    t_all = sum(qlens) if layout == "TND" else b * s_max
    qshape = (t_all, heads, d) if layout == "TND" else (b, s_max, heads, d)
    cu = torch.tensor(np.cumsum([0] + list(qlens)), dtype=torch.int32)
    kw = dict(q=torch.zeros(qshape, dtype=dt), ori_kv=ori, ori_block_table=torch.from_numpy(t1),
              seqused_kv=torch.tensor(kvlens, dtype=torch.int32),
              sinks=torch.full((heads,), -math.inf), softmax_scale=1 / math.sqrt(d),
              ori_win_left=win, layout_q=layout, head_dim_v=512,
              cu_seqlens_q=cu if (layout == "TND" or qlens != [s_max] * b) else None)
    if scenario >= 2:
        kw.update(cmp_kv=cmp_, cmp_block_table=torch.from_numpy(t2), cmp_ratio=ratio)
    if scenario == 3:
        idx_t = torch.from_numpy(idx)
        kw["cmp_sparse_indices"] = (idx_t.reshape(t_all, 1, k) if layout == "TND"
                                    else idx_t.reshape(b, s_max, 1, k))
    return kw, idx, t1, t2


def _expected(kw, idx, t1, t2, scenario, ratio, bs1, bs2):
    """Per flat token: (n, counts over the 512 one-hot columns) from the oracle's resolution."""
    q = kw["q"]
    nb, s_max, prefix, act_q = token_layout(kw["layout_q"], q.shape, kw.get("cu_seqlens_q"))
    kv = kw["seqused_kv"].tolist()
    exp = {}
    for bi in range(nb):
        for s in range(act_q[bi]):
            t = prefix[bi] + s
            counts = np.zeros(512, dtype=np.int64)
            sg = causal_position(kv[bi], act_q[bi], s)
            lo, hi = window_range(sg, kw["ori_win_left"])
            for p in range(lo, hi):
                counts[t1[bi, p // bs1] * bs1 + p % bs1] += 1
            if scenario == 2:
                rows = dense_cmp_rows(kv[bi], act_q[bi], s, ratio)
            elif scenario == 3:
                rows = resolve_topk_rows(idx[t].tolist(), kv[bi], act_q[bi], s, ratio)
            else:
                rows = []
            for p in rows:
                counts[POOL_ROWS + t2[bi, p // bs2] * bs2 + p % bs2] += 1
            exp[t] = counts
    return exp


def _check(kw, idx, t1, t2, scenario, ratio, bs1, bs2, **extra):
    dev = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}
    out, lse = sparse_attn_sharedkv(**dev, return_softmax_lse=True, **extra)
    torch.cuda.synchronize()
    _verify(kw, idx, t1, t2, scenario, ratio, bs1, bs2, out, lse)


def _verify(kw, idx, t1, t2, scenario, ratio, bs1, bs2, out, lse):
    """Every token's gathered multiset (from out and lse) against the oracle's resolution."""
    heads = kw["q"].shape[-2]
    out = out.reshape(-1, heads, 512).float().cpu()
    lse = lse.reshape(-1, heads).cpu()
    exp = _expected(kw, idx, t1, t2, scenario, ratio, bs1, bs2)
    for t, counts in exp.items():
        n = int(counts.sum())
        if n == 0:  # nothing attended and no sink: golden gives out 0, lse -inf
            assert torch.isneginf(lse[t]).all(), f"token {t}: lse {lse[t][:4]}"
            assert (out[t] == 0).all(), f"token {t}: nonzero output"
            continue
        got_n = torch.round(torch.exp(lse[t].double())).long()
        assert (got_n == n).all(), f"token {t}: attended {got_n.unique().tolist()} rows, want {n}"
        got = torch.round(out[t].double() * n).long().numpy()
        want = np.broadcast_to(counts, got.shape)
        bad = np.argwhere(got != want)
        assert bad.size == 0, (f"token {t}: head {bad[0][0]} column {bad[0][1]}: "
                               f"{got[tuple(bad[0])]} gathered, want {want[tuple(bad[0])]}")


@requires_gpu
@pytest.mark.parametrize("win", [-1, 0, 127, 1023])
def test_window_rows_exact(win):
    _say(f"SWA window {win}")
    kw, idx, t1, t2 = _case(scenario=1, layout="BSND", qlens=[1, 1, 1], kvlens=[180, 30, 17],
                            heads=64, d=576, win=win, seed=1)
    _check(kw, idx, t1, t2, 1, 1, 16, 16)


@requires_gpu
def test_ragged_window_rows_exact():
    _say("SWA ragged TND rows, H=16, d=512")
    kw, idx, t1, t2 = _case(scenario=1, layout="TND", qlens=[3, 1, 17], kvlens=[40, 9, 3000],
                            heads=16, d=512, win=5, bs1=64, seed=2)
    _check(kw, idx, t1, t2, 1, 1, 64, 16)


@requires_gpu
@pytest.mark.parametrize("ratio", [4, 16])
def test_dense_compressed_rows_exact(ratio):
    _say(f"CFA ratio {ratio}")
    kw, idx, t1, t2 = _case(scenario=2, layout="TND", qlens=[2, 5], kvlens=[300, 900 if ratio == 16 else 400],
                            heads=64, d=512, win=7, ratio=ratio, bs1=16, bs2=16, seed=3)
    _check(kw, idx, t1, t2, 2, ratio, 16, 16)


def _edits(idx):
    idx[0, 17] = -1                 # stop in the middle
    idx[1, ::3] = 5000              # beyond thr -> skipped
    idx[1, 1::7] = idx[1, 0]        # duplicates
    idx[2] = -1                     # nothing from the compressed cache


@requires_gpu
@pytest.mark.parametrize("cores", [256, 7])
@pytest.mark.parametrize("win", [63, -1])
def test_topk_rows_exact(win, cores):
    # K = 1030 top-k slots (+ a 64-row window): items of more than 1024 positions,
    # so every item spans two resolution chunks; 7 workgroups split the items
    _say(f"SCFA top-k 1030 win {win} cores {cores}")
    kw, idx, t1, t2 = _case(scenario=3, layout="TND", qlens=[2, 1, 1], kvlens=[3000, 2500, 1100],
                            heads=128, d=576, win=win, ratio=1, k=1030, bs1=16, bs2=16, seed=4,
                            edit=_edits)
    _check(kw, idx, t1, t2, 3, 1, 16, 16, core_num=cores)


@requires_gpu
@pytest.mark.parametrize("fp8_qk", [False, True])
def test_topk_rows_exact_fp8_rows(fp8_qk):
    # fp8 rows through the pipelined kernel, Q·Kᵀ in bf16 or on fp8 MFMA (q = 0
    # quantizes to all-zero codes, so every score is still 0)
    _say(f"SCFA top-k, fp8 rows, fp8_qk={fp8_qk}")
    kw, idx, t1, t2 = _case(scenario=3, layout="BSND", qlens=[1, 1, 1], kvlens=[700, 2100, 90],
                            heads=64, d=576, win=3, ratio=4, k=300, bs1=16, bs2=16, seed=5,
                            edit=_edits, fp8=True)
    _check(kw, idx, t1, t2, 3, 4, 16, 16, fp8_qk=fp8_qk)


@requires_gpu
@pytest.mark.parametrize("cores", [256, 7])
def test_topk_rows_exact_fp8_qk_two_chunks(cores):
    # the fp8 Q·Kᵀ form requantizes the query for each resolution chunk: items of
    # more than 1024 positions (two chunks), split over 7 workgroups or not
    _say(f"SCFA top-k 1030, fp8 rows, fp8 Q·Kᵀ, cores {cores}")
    kw, idx, t1, t2 = _case(scenario=3, layout="TND", qlens=[2, 1, 1], kvlens=[3000, 2500, 1100],
                            heads=128, d=576, win=63, ratio=1, k=1030, bs1=16, bs2=16, seed=6,
                            edit=_edits, fp8=True)
    _check(kw, idx, t1, t2, 3, 1, 16, 16, core_num=cores, fp8_qk=True)
