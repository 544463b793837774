"""GPU parity on seeded random configurations (the HIP path against the oracle).

Each case draws a scenario (SWA / dense compressed / top-k compressed), a
layout (TND with ragged query lengths, or BSND), 1-4 sequences with 1-40 query
rows over up to ~2.5k cached rows, 16-128 heads, a window of 0, 1, 6, 128 or
1024 rows or none (``ori_win_left = -1``: empty), a compression ratio, a
top-k width from 1 to 1030 (wider than the compressed prefix, so ``-1``
padded), cache block sizes of 16 / 64 / 128 and a schedule for 1, 7, 64 or
256 workgroups (single pieces, multi-chunk items, split items). Inputs follow
the reference's generators (q, raw KV U(-10, 10); compressed KV U(-5, 10)).

Asserted for every row: the LSE within 1e-3 relative of golden, and the
output as accurate as golden against the float64 closed form (max |out -
exact| <= 2 max |golden - exact| + 2^-9 max |exact|). Reported, not asserted:
the reference's 99.5 % rule and the per-element 2e-2 bound. With these inputs
(|V| up to 10, peaked attention) rounding P to bf16 alone moves an output by
up to ~2e-2, and golden rounds P relative to the running max of 512-row tiles
while this kernel uses 32-row tiles and a lazily moved max: the two roundings
differ by up to ~3e-2 in a few elements of a long attended list, and by more
than 2^-7 relative in ~0.5-1 % of them (those near zero), while both are
equally far from the exact result. The reference's own cases, where its rule
is asserted, and the N(0, 1) * 0.5 shapes, where the 2e-2 bound is, are in
test_gpu_parity.py.
"""

import math
import os
import sys

import numpy as np
import pytest
import torch

from oracle import gen
from oracle.checks import LSE_ATOL_FLOOR, LSE_RTOL, OUT_ATOL, OUT_RTOL, check_vs_exact
from oracle.golden_ref import sparse_attn_exact, sparse_attn_oracle

pytestmark = pytest.mark.gpu

HAS_GPU = torch.cuda.is_available()
requires_gpu = pytest.mark.skipif(not HAS_GPU, reason="needs a ROCm GPU")

if HAS_GPU:
    from sparse_attn_sharedkv_amd import sparse_attn_sharedkv, sparse_attn_sharedkv_metadata

N_CASES = int(os.environ.get("SAS_SWEEP_CASES", "40"))  # more for a longer validation run
DTYPE = {"bf16": torch.bfloat16, "fp16": torch.float16}[os.environ.get("SAS_SWEEP_DTYPE", "bf16")]


def _say(msg):
    print(f"[gpu-sweep] {msg}", flush=True)
    sys.stdout.flush()


def _random_cfg(rng):
    scenario = int(rng.integers(1, 4))
    layout = "TND" if rng.random() < 0.6 else "BSND"
    b = int(rng.integers(1, 5))
    q_opts = [1, 1, 2, 3, 17, 40]
    if layout == "TND":
        qlens = [int(rng.choice(q_opts)) for _ in range(b)]
    else:
        qlens = [int(rng.choice(q_opts))] * b
    kv = [int(q + rng.integers(0, 2500)) for q in qlens]
    ratio = int(rng.choice([1, 4, 16, 128])) if scenario >= 2 else 4
    k = int(rng.choice([1, 7, 64, 512, 1030])) if scenario == 3 else 512
    bs1 = int(rng.choice([16, 64, 128]))
    bs2 = int(rng.choice([16, 64, 128]))
    cu = [0]
    for q in qlens:
        cu.append(cu[-1] + q)
    return dict(
        scenario=scenario, layout_q=layout, B=b, S1=max(qlens),
        T1=sum(qlens) if layout == "TND" else max(qlens) * b,
        N1=int(rng.choice([16, 32, 48, 64, 96, 128])), N2=1, D=512, K=k,
        block_num1=sum(math.ceil(x / bs1) for x in kv) + int(rng.integers(0, 3)),
        block_num2=sum(max(1, math.ceil((x // ratio) / bs2)) for x in kv) + 1,
        block_size1=bs1, block_size2=bs2, cu_seqlens_q=cu, seqused_kv=kv,
        softmax_scale=1.0 / math.sqrt(512), cmp_ratio=ratio,
        ori_win_left=int(rng.choice([-1, 0, 5, 127, 1023])), ori_win_right=0,
        ori_mask_mode=4, cmp_mask_mode=3,
        cores=int(rng.choice([1, 7, 64, 256])))


_CASES = [_random_cfg(np.random.default_rng(1000 + i)) for i in range(N_CASES)]


@requires_gpu
@pytest.mark.parametrize("i", range(N_CASES))
def test_random_configuration(i):
    cfg = _CASES[i]
    _say(f"case {i}: scenario {cfg['scenario']} {cfg['layout_q']} B={cfg['B']} "
         f"q={cfg['cu_seqlens_q']} kv={cfg['seqused_kv']} H={cfg['N1']} "
         f"win={cfg['ori_win_left']} ratio={cfg['cmp_ratio']} K={cfg['K']} "
         f"blocks={cfg['block_size1']}/{cfg['block_size2']} cores={cfg['cores']}")
    kw = gen.build_case(cfg, DTYPE, seed=2000 + i)
    cu = torch.tensor(cfg["cu_seqlens_q"], dtype=torch.int32)
    md = sparse_attn_sharedkv_metadata(
        num_heads_q=cfg["N1"], num_heads_kv=1, head_dim=cfg["D"],
        cu_seqlens_q=cu if cfg["layout_q"] == "TND" else None,
        seqused_kv=kw["seqused_kv"], batch_size=cfg["B"], max_seqlen_q=cfg["S1"],
        max_seqlen_kv=max(cfg["seqused_kv"]),
        cmp_topk=cfg["K"] if cfg["scenario"] == 3 else 0, cmp_ratio=cfg["cmp_ratio"],
        ori_win_left=cfg["ori_win_left"], layout_q=cfg["layout_q"],
        has_cmp_kv=cfg["scenario"] >= 2, aic_core_num=cfg["cores"])
    dev = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}
    out, lse = sparse_attn_sharedkv(**dev, metadata=md.cuda(), return_softmax_lse=True)
    torch.cuda.synchronize()
    okw = {k: v for k, v in kw.items() if k not in ("topk_cmp",)}
    ref, ref_lse = sparse_attn_oracle(**okw)
    o, r = out.cpu().float(), ref.float()
    assert torch.isfinite(o).all(), "non-finite output"
    err = (o - r).abs()
    within = (err <= 1e-4 + 0.0078125 * r.abs()).float().mean().item() * 100
    beyond = int((err > OUT_ATOL + OUT_RTOL * r.abs()).sum())
    _say(f"case {i}: {within:.3f} % within the reference's rtol 2^-7 / atol 1e-4; "
         f"{beyond} elements beyond 2e-2; max |out - golden| {err.max().item():.3g}")
    x, y = lse.cpu(), ref_lse
    fin = torch.isfinite(y)
    assert torch.equal(torch.isfinite(x), fin) and torch.equal(x[~fin], y[~fin]), "lse: non-finite"
    lse_err = (x[fin] - y[fin]).abs()
    assert (lse_err <= LSE_RTOL * y[fin].abs() + LSE_ATOL_FLOOR).all(), \
        f"lse: max abs err {lse_err.max().item()}"
    ex, _ = sparse_attn_exact(**okw)
    acc = check_vs_exact(out.cpu(), ref, ex)
    _say(f"case {i}: max |out - exact| {acc['ours']:.3g}, max |golden - exact| {acc['golden']:.3g}")
