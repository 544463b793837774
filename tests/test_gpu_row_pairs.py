"""Row pairs: two consecutive query rows of 64 heads per workgroup.

Launches whose sequences hold several query rows (prefill, multi-token decode)
with items of 64 heads and windows and / or dense compressed prefixes
(scenarios 1 and 2) run two consecutive query rows per workgroup on the
128-head kernel, over the union of the two rows' attended positions, each row
masking what it does not attend; pieces of split items run alone
(test_sparse_attn_sharedkv.py:105-219 runs these shapes as prefill). Checked
here:

* gathered rows pinned exactly (q = 0, sinks -inf, one-hot V rows, as in
  ``test_gpu_index_exact``): windows -1 / 0 / 5 / 127, dense compressed rows at
  ratios 4 and 16, ragged TND rows and padded BSND rows, sequences whose early
  rows attend nothing (more query rows than cached rows), odd row counts (a row
  left without a partner), 48 and 64 heads, d_qk 512 and 576, few workgroups,
  split items (merged in-kernel and by the merge kernel);
* random data against the oracle under the benchmark bound (``check_strict``),
  and against the same call with one query row per item
  (``SAS_PHASE_ROW_ITEMS``) to within rounding: bf16 and fp16, windows up to
  1023 rows (a pair's positions in two resolution chunks).
"""

import math
import sys

import numpy as np
import pytest
import torch

from oracle.checks import check_strict
from oracle.golden_ref import sparse_attn_oracle

pytestmark = pytest.mark.gpu

HAS_GPU = torch.cuda.is_available()
requires_gpu = pytest.mark.skipif(not HAS_GPU, reason="needs a ROCm GPU")

if HAS_GPU:
    from sparse_attn_sharedkv_amd import api

from test_gpu_index_exact import _case, _verify  # noqa: E402


def _say(msg):
    print(f"[gpu-row-pairs] {msg}", flush=True)
    sys.stdout.flush()


def _run(kw, row_items=False, **extra):
    dev = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}
    prep = api.prepare(**dev, _row_items=row_items, **extra)
    api.launch(prep)
    torch.cuda.synchronize()
    out, lse = api.finalize(prep, True)
    return prep, out, lse


def _pairs_on(prep):
    return api.uses_row_pairs(prep)


@requires_gpu
@pytest.mark.parametrize("scenario,win,ratio,layout,qlens,kvlens,heads,d,cores", [
    (1, 63, 1, "TND", [7, 40, 3, 61], [7, 40, 100, 61], 64, 512, 256),
    (1, 0, 1, "TND", [9, 33], [5, 40], 64, 576, 256),       # early rows attend nothing
    (1, 5, 1, "BSND", [3, 8], [20, 8], 48, 576, 256),        # padded rows, 48 heads
    (1, 127, 1, "TND", [61, 50], [100, 50], 64, 512, 7),     # few workgroups
    (2, -1, 4, "TND", [40, 17], [300, 500], 64, 512, 256),   # compressed rows only
    (2, 7, 16, "TND", [33, 20], [900, 400], 64, 576, 256),
    (2, 63, 4, "BSND", [12, 12], [100, 60], 64, 512, 256),
    (2, 127, 4, "TND", [4], [800], 64, 576, 3),      # split items (2 pieces: merged in-kernel)
    (2, 127, 4, "TND", [6], [1000], 64, 512, 256),   # every item in 3 pieces (merge kernel)
])
def test_row_pairs_rows_exact(scenario, win, ratio, layout, qlens, kvlens, heads, d, cores):
    _say(f"scenario {scenario} win {win} ratio {ratio} {layout} qlens {qlens} H={heads} d={d} "
         f"cores {cores}")
    kw, idx, t1, t2 = _case(scenario=scenario, layout=layout, qlens=qlens, kvlens=kvlens,
                            heads=heads, d=d, win=win, ratio=ratio, bs1=16, bs2=16,
                            seed=sum(qlens) + win)
    prep, out, lse = _run(kw, core_num=cores)
    assert _pairs_on(prep), "expected the row-pair path"
    _verify(kw, idx, t1, t2, scenario, ratio, 16, 16, out, lse)
    # the same call with one row per item gathers the same rows
    prep1, out1, lse1 = _run(kw, row_items=True, core_num=cores)
    assert not _pairs_on(prep1)
    _verify(kw, idx, t1, t2, scenario, ratio, 16, 16, out1, lse1)


def _prefill_case(scenario, rows, heads, win, ratio, seed, dtype=torch.bfloat16, d=512):
    g = torch.Generator().manual_seed(seed)
    bs = 128
    nblk = (rows + bs - 1) // bs
    ori = (torch.randn(nblk * 2, bs, 1, d, generator=g) * 0.5).to(dtype)
    table = torch.randperm(nblk * 2, generator=g)[:nblk].to(torch.int32).reshape(1, nblk)
    kw = dict(q=(torch.randn(rows, heads, d, generator=g) * 0.5).to(dtype),
              ori_kv=ori, ori_block_table=table,
              seqused_kv=torch.tensor([rows], dtype=torch.int32),
              cu_seqlens_q=torch.tensor([0, rows], dtype=torch.int32),
              sinks=torch.rand(heads, generator=g) * 2 - 1, softmax_scale=1 / math.sqrt(d),
              ori_win_left=win, layout_q="TND", head_dim_v=512)
    if scenario == 2:
        ncmp = max(rows // ratio, 1)
        cb = (ncmp + bs - 1) // bs
        kw.update(cmp_kv=(torch.randn(cb, bs, 1, d, generator=g) * 0.5).to(dtype),
                  cmp_block_table=torch.arange(cb, dtype=torch.int32).reshape(1, cb),
                  cmp_ratio=ratio)
    return kw


@requires_gpu
@pytest.mark.parametrize("scenario,rows,win,ratio,dtype,d", [
    (1, 1000, 127, 1, torch.bfloat16, 512), (1, 333, 31, 1, torch.float16, 512),
    (2, 1000, 127, 128, torch.bfloat16, 512), (2, 600, 63, 4, torch.bfloat16, 512),
    (1, 1100, 1023, 1, torch.bfloat16, 512),  # a pair's window union spans two 1024-row chunks
    (2, 500, 63, 4, torch.float16, 576),      # the d_qk-576 instances (rope part in the ring)
    (1, 400, 127, 1, torch.bfloat16, 576),
])
def test_row_pairs_match_oracle_and_row_items(scenario, rows, win, ratio, dtype, d):
    _say(f"prefill scenario {scenario}, {rows} rows, window {win}, ratio {ratio}, {dtype}, d {d}")
    kw = _prefill_case(scenario, rows, 64, win, ratio, seed=rows + win, dtype=dtype, d=d)
    prep, out, lse = _run(kw)
    assert _pairs_on(prep), "expected the row-pair path"
    ref, ref_lse = sparse_attn_oracle(**kw)
    err = check_strict(out.cpu(), ref, lse.cpu(), ref_lse)
    _, out1, lse1 = _run(kw, row_items=True)
    d_out = (out.float() - out1.float()).abs().max().item()
    d_lse = (lse - lse1).abs().max().item()
    _say(f"max |out - oracle| {err['out_max_abs']:.3g}; pairs vs row items: out {d_out:.3g}, "
         f"lse {d_lse:.3g}")
    assert d_out <= 2e-2 and d_lse <= 1e-3
