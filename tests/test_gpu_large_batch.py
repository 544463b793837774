"""More than 64 sequences per call on native bf16 rows.

Up to 64 sequences the attention kernels hold every sequence's lengths and
query offset in one lane each; beyond that they load them per item
(golden.py:116-125 gives every sequence its own lengths either way). These
cases run that second path:

* the 128-head top-k decode shape (H = 128, top-k 2048 of 4096 rows) and the
  64-head sliding-window decode shape (window 128, contexts U[2048, 8192]) at
  96 and 128 sequences, every query row checked against the oracle under the
  benchmark bound (``check_strict``);
* gathered rows pinned exactly at 96 and 128 sequences (q = 0, sinks -inf,
  one-hot V rows, as in ``test_gpu_index_exact``): a window of two rows and a
  two-slot top-k list per sequence over block-size-1 caches, every sequence of
  another length, so a length or offset read for the wrong sequence shows as a
  wrong row;
* 128 sequences of 128 heads (128-head items on the wide kernel): gathered rows
  exactly at d_qk = 512, and window / top-k values at d_qk 512 and 576, bf16 and
  fp16, against the oracle under the benchmark bound.
"""

import math
import sys

import numpy as np
import pytest
import torch

from oracle import gen
from oracle.checks import check_strict
from oracle.golden_ref import sparse_attn_oracle

pytestmark = pytest.mark.gpu

HAS_GPU = torch.cuda.is_available()
requires_gpu = pytest.mark.skipif(not HAS_GPU, reason="needs a ROCm GPU")

if HAS_GPU:
    from sparse_attn_sharedkv_amd import sparse_flash_mla

from test_gpu_index_exact import _case, _check  # noqa: E402


def _say(msg):
    print(f"[gpu-large-batch] {msg}", flush=True)
    sys.stdout.flush()


@requires_gpu
@pytest.mark.parametrize("batch", [96, 128])
@pytest.mark.parametrize("name,ctx", [("mla_decode_b64_h128_k2048", 4096),
                                      ("swa_decode_b32_h64", None)])
def test_many_sequences_against_oracle(name, ctx, batch):
    _say(f"{name} with {batch} sequences")
    kw = gen.build_workload(name, device="cuda", seed=200 + batch, batch=batch,
                            ctx_override=[ctx] * batch if ctx else None)
    out, lse = sparse_flash_mla(**kw, return_softmax_lse=True)
    torch.cuda.synchronize()
    assert out.shape[0] == batch
    okw = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()
           if k != "topk_cmp"}
    ref, ref_lse = sparse_attn_oracle(**okw)
    err = check_strict(out.cpu(), ref, lse.cpu(), ref_lse)
    _say(f"{name} B={batch}: max |out - oracle| {err['out_max_abs']:.3g}")


@requires_gpu
@pytest.mark.parametrize("heads", [64, 128])
@pytest.mark.parametrize("batch", [96, 128])
def test_many_sequences_rows_exact(batch, heads):
    _say(f"rows exact, {batch} sequences, H={heads}")
    rng = np.random.default_rng(300 + batch)
    kvlens = [int(x) for x in rng.permutation(np.arange(40, 40 + 7 * batch, 7))]
    kw, idx, t1, t2 = _case(scenario=3, layout="BSND", qlens=[1] * batch, kvlens=kvlens,
                            heads=heads, d=576, win=1, ratio=1, k=2, bs1=1, bs2=1,
                            seed=300 + batch)
    _check(kw, idx, t1, t2, 3, 1, 1, 1)


# 128 sequences of a 128-head call take 128-head items (every head of a token
# against one gathered tile) on the wide kernel; d_qk 512 (no rope part in the
# ring) and fp16 rows are instances of their own. Gathered rows exactly, then values.
@requires_gpu
def test_128_head_items_d512_rows_exact():
    _say("rows exact, 128 sequences, H=128, d=512 (128-head items)")
    rng = np.random.default_rng(428)
    kvlens = [int(x) for x in rng.permutation(np.arange(40, 40 + 7 * 128, 7))]
    kw, idx, t1, t2 = _case(scenario=3, layout="BSND", qlens=[1] * 128, kvlens=kvlens,
                            heads=128, d=512, win=1, ratio=1, k=2, bs1=1, bs2=1, seed=428)
    _check(kw, idx, t1, t2, 3, 1, 1, 1)


@requires_gpu
@pytest.mark.parametrize("d", [512, 576])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scenario", [1, 3])
def test_128_head_items_against_oracle(scenario, dtype, d):
    from sparse_attn_sharedkv_amd import api, sparse_attn_sharedkv, sparse_attn_sharedkv_metadata
    from oracle.gen import build_case

    b = 128
    _say(f"128 sequences, H=128, d={d}, scenario {scenario}, {dtype}")
    rng = np.random.default_rng(500 + scenario)
    kv = [int(x) for x in rng.integers(300, 1500, size=b)]
    cu = list(np.concatenate([[0], np.cumsum([1] * b)]).astype(int))
    cfg = dict(scenario=scenario, layout_q="TND", B=b, S1=1, T1=b, N1=128, N2=1, D=d,
               K=96 if scenario == 3 else 0,
               block_num1=sum(-(-x // 64) for x in kv) + 2, block_num2=sum(max(1, -(-(x // 4) // 64)) for x in kv) + 1,
               block_size1=64, block_size2=64, cu_seqlens_q=cu, seqused_kv=kv,
               softmax_scale=1.0 / math.sqrt(d), cmp_ratio=4, ori_win_left=127,
               ori_win_right=0, ori_mask_mode=4, cmp_mask_mode=3)
    kw = build_case(cfg, dtype, seed=600 + scenario)
    kw["head_dim_v"] = 512  # (d_qk 576: the first 512 columns are V)
    # values scaled to U(-0.5, 0.5): the benchmark bound applies to every element
    for key in ("q", "ori_kv", "cmp_kv"):
        if kw.get(key) is not None:
            kw[key] = (kw[key].float() * 0.05).to(dtype)
    cuq = torch.tensor(cu, dtype=torch.int32)
    md = sparse_attn_sharedkv_metadata(
        num_heads_q=128, num_heads_kv=1, head_dim=d, cu_seqlens_q=cuq,
        seqused_kv=kw["seqused_kv"], batch_size=b, max_seqlen_q=1, max_seqlen_kv=max(kv),
        cmp_topk=cfg["K"], cmp_ratio=4, ori_win_left=127, layout_q="TND",
        has_cmp_kv=scenario >= 2)
    dev = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}
    prep = api.prepare(**dev, metadata=md.cuda())
    assert prep.args.m_base == 128, prep.args.m_base  # the 128-head kernel runs
    out, lse = sparse_attn_sharedkv(**dev, metadata=md.cuda(), return_softmax_lse=True)
    torch.cuda.synchronize()
    okw = {k: v for k, v in kw.items() if k != "topk_cmp"}
    ref, ref_lse = sparse_attn_oracle(**okw)
    err = check_strict(out.cpu(), ref, lse.cpu(), ref_lse)
    _say(f"scenario {scenario} {dtype}: max |out - oracle| {err['out_max_abs']:.3g}")


@requires_gpu
@pytest.mark.parametrize("scenario", [1, 3])
def test_multi_row_128_heads_take_128_head_items(scenario):
    # a call that builds its own schedule counts query rows (one sequence of 300
    # rows: 128-head items); the same call with a schedule from the metadata entry
    # point counts sequences (64-head items); both against the oracle
    from sparse_attn_sharedkv_amd import api, sparse_attn_sharedkv, sparse_attn_sharedkv_metadata
    from oracle.gen import build_case

    rows, d = 300, 576
    _say(f"one sequence of {rows} rows, H=128, scenario {scenario}")
    cfg = dict(scenario=scenario, layout_q="TND", B=1, S1=rows, T1=rows, N1=128, N2=1, D=d,
               K=160 if scenario == 3 else 0, block_num1=-(-(rows + 700) // 64) + 2,
               block_num2=max(1, -(-((rows + 700) // 4) // 64)) + 1, block_size1=64,
               block_size2=64, cu_seqlens_q=[0, rows], seqused_kv=[rows + 700],
               softmax_scale=1.0 / math.sqrt(d), cmp_ratio=4, ori_win_left=127,
               ori_win_right=0, ori_mask_mode=4, cmp_mask_mode=3)
    kw = build_case(cfg, torch.bfloat16, seed=900 + scenario)
    kw["head_dim_v"] = 512
    for key in ("q", "ori_kv", "cmp_kv"):
        if kw.get(key) is not None:
            kw[key] = (kw[key].float() * 0.05).to(torch.bfloat16)
    dev = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}
    assert api.prepare(**dev).args.m_base == 128
    md = sparse_attn_sharedkv_metadata(
        num_heads_q=128, num_heads_kv=1, head_dim=d, cu_seqlens_q=torch.tensor([0, rows]),
        seqused_kv=kw["seqused_kv"], batch_size=1, max_seqlen_q=rows,
        max_seqlen_kv=rows + 700, cmp_topk=cfg["K"], cmp_ratio=4, ori_win_left=127,
        layout_q="TND", has_cmp_kv=scenario >= 2)
    assert api.prepare(**dev, metadata=md).args.m_base == 64
    okw = {k: v for k, v in kw.items() if k != "topk_cmp"}
    ref, ref_lse = sparse_attn_oracle(**okw)
    for extra in ({}, {"metadata": md.cuda()}):
        out, lse = sparse_attn_sharedkv(**dev, return_softmax_lse=True, **extra)
        torch.cuda.synchronize()
        check_strict(out.cpu(), ref, lse.cpu(), ref_lse)
