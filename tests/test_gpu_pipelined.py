"""SAS_PHASE_PIPELINED on native rows: the software-pipelined kernel that fp8 rows
of 64-head items use, selected for bf16 / fp16 rows by the public phase bit.

Every instance the bit reaches — bf16 and fp16 rows, d_qk 512 and 576, 32- and
64-head items — runs window and top-k cases (ragged TND rows, whole and split
items) against the oracle under the benchmark bound (values scaled to
U(-0.5, 0.5) from the reference's generators).
"""

import math
import sys

import numpy as np
import pytest
import torch

from oracle.checks import check_strict
from oracle.gen import build_case
from oracle.golden_ref import sparse_attn_oracle

pytestmark = pytest.mark.gpu

HAS_GPU = torch.cuda.is_available()
requires_gpu = pytest.mark.skipif(not HAS_GPU, reason="needs a ROCm GPU")

if HAS_GPU:
    from sparse_attn_sharedkv_amd import _lib, api


def _say(msg):
    print(f"[gpu-pipelined] {msg}", flush=True)
    sys.stdout.flush()


def _case(scenario, heads, d, dtype, seed):
    rng = np.random.default_rng(seed)
    qlens = [1, 3, 17, 2]
    kv = [int(q + rng.integers(200, 1800)) for q in qlens]
    cu = [0]
    for q in qlens:
        cu.append(cu[-1] + q)
    cfg = dict(scenario=scenario, layout_q="TND", B=len(qlens), S1=max(qlens), T1=sum(qlens),
               N1=heads, N2=1, D=d, K=200 if scenario == 3 else 0,
               block_num1=sum(-(-x // 64) for x in kv) + 2,
               block_num2=sum(max(1, -(-(x // 4) // 64)) for x in kv) + 1,
               block_size1=64, block_size2=64, cu_seqlens_q=cu, seqused_kv=kv,
               softmax_scale=1.0 / math.sqrt(d), cmp_ratio=4, ori_win_left=127,
               ori_win_right=0, ori_mask_mode=4, cmp_mask_mode=3)
    kw = build_case(cfg, dtype, seed=seed)
    kw["head_dim_v"] = 512
    for key in ("q", "ori_kv", "cmp_kv"):
        if kw.get(key) is not None:
            kw[key] = (kw[key].float() * 0.05).to(dtype)
    return kw


@requires_gpu
@pytest.mark.parametrize("cores", [256, 7])
@pytest.mark.parametrize("heads", [32, 64])
@pytest.mark.parametrize("d", [512, 576])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scenario", [1, 3])
def test_pipelined_native_rows_match_oracle(scenario, dtype, d, heads, cores):
    _say(f"scenario {scenario} {dtype} d={d} H={heads} cores={cores}")
    kw = _case(scenario, heads, d, dtype, seed=700 + 10 * scenario + d + heads)
    dev = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()
           if k != "topk_cmp"}
    prep = api.prepare(**dev, core_num=cores, _pipelined=True)
    assert prep.phase_bits & _lib.SAS_PHASE_PIPELINED
    api.launch(prep)
    torch.cuda.synchronize()
    okw = {k: v for k, v in kw.items() if k != "topk_cmp"}
    ref, ref_lse = sparse_attn_oracle(**okw)
    out = prep.out.reshape(ref.shape).cpu()
    lse = prep.lse.reshape(ref_lse.shape).cpu()
    err = check_strict(out, ref, lse, ref_lse)
    _say(f"max |out - oracle| {err['out_max_abs']:.3g}")
