"""GPU parity of the fp8 cache path (656-byte rows) on seeded random configurations.

The configurations are the bf16 sweep's (``gen.random_sweep_cfg``: SWA / dense
compressed / top-k compressed, TND with ragged query lengths or BSND, 1-4
sequences of 1-40 query rows over up to ~2.5k cached rows, 16-128 heads,
windows -1 / 0 / 5 / 127 / 1023, compression ratios 1-128, top-k widths 1-1030,
cache blocks of 16 / 64 / 128 rows, schedules for 1, 7, 64 or 256 workgroups)
at d_qk = 576, d_v = 512. The caches hold valid fp8 rows drawn directly in the
stored format (``fp8_rows.random_rows``: e4m3 codes uniform over the finite
values, per-128 scales in [1e-3, 1e-2], bf16 rope ~ N(0, 1) * 0.5), the query is
N(0, 1) * 0.5 in bf16 and the sinks U(-1, 1), as in the benchmark regime.

No reference code exists for fp8 caches (api.py:51-56 accepts bf16 / fp16):
the oracle dequantizes the rows (``oracle/fp8_rows.py``, pinned in
``test_fp8_oracle.py``) and runs the golden math on them. Asserted for every
case: |out - golden| <= 2e-2 + 2e-2 |golden| and |lse - golden| <= 1e-3 |golden|
(``check_strict``), and the output as accurate as golden against the float64
closed form over the same rows (``check_vs_exact``). The fp8 Q·Kᵀ form
(``fp8_qk=True``, no reference counterpart: per-head e4m3 queries) runs the same
configurations against the oracle of that form (``sparse_attn_oracle(...,
fp8_qk=True)``, whose block dot products follow the f8f6f4 MFMA's own
arithmetic, ``fp8_rows.mfma_f8_dot``, pinned on vectors the MFMA returned): the
output under ``check_strict``'s bound, the LSE within 1e-3 relative.
"""

import os
import sys

import numpy as np
import pytest
import torch

from oracle import fp8_rows as F
from oracle import gen
from oracle.checks import check_strict, check_vs_exact
from oracle.golden_ref import sparse_attn_exact, sparse_attn_oracle

pytestmark = pytest.mark.gpu

HAS_GPU = torch.cuda.is_available()
requires_gpu = pytest.mark.skipif(not HAS_GPU, reason="needs a ROCm GPU")

if HAS_GPU:
    from sparse_attn_sharedkv_amd import sparse_attn_sharedkv, sparse_attn_sharedkv_metadata

N_CASES = int(os.environ.get("SAS_FP8_SWEEP_CASES", "24"))  # more for a longer validation run
_CASES = [dict(gen.random_sweep_cfg(np.random.default_rng(5000 + i)), D=576,
               softmax_scale=1.0 / 24.0) for i in range(N_CASES)]


def _say(msg):
    print(f"[gpu-fp8-sweep] {msg}", flush=True)
    sys.stdout.flush()


def _fp8_pool(block_num, block_size, seed):
    g = torch.Generator().manual_seed(seed)
    rows = F.random_rows(block_num * block_size, g)
    return torch.from_numpy(rows).reshape(block_num, block_size, 1, F.ROW_BYTES)


def fp8_case(i):
    """Inputs of case ``i`` on the CPU: the bf16 sweep's lengths, block tables,
    top-k ids and sinks, with fp8 pools of the same geometry and an N(0, 1) * 0.5
    query."""
    cfg = _CASES[i]
    kw = gen.build_case(cfg, torch.bfloat16, seed=6000 + i)
    g = torch.Generator().manual_seed(7000 + i)
    kw["q"] = (torch.randn(kw["q"].shape, generator=g) * 0.5).to(torch.bfloat16)
    kw["ori_kv"] = _fp8_pool(cfg["block_num1"], cfg["block_size1"], 8000 + i)
    if kw.get("cmp_kv") is not None:
        kw["cmp_kv"] = _fp8_pool(cfg["block_num2"], cfg["block_size2"], 9000 + i)
    kw.update(kv_cache_dtype="fp8_ds_mla", head_dim_v=512)
    return cfg, kw


@requires_gpu
@pytest.mark.parametrize("qk", ["bf16", "fp8"])
@pytest.mark.parametrize("i", range(N_CASES))
def test_fp8_random_configuration(i, qk):
    cfg, kw = fp8_case(i)
    _say(f"case {i} (Q·Kᵀ {qk}): scenario {cfg['scenario']} {cfg['layout_q']} B={cfg['B']} "
         f"q={cfg['cu_seqlens_q']} kv={cfg['seqused_kv']} H={cfg['N1']} "
         f"win={cfg['ori_win_left']} ratio={cfg['cmp_ratio']} K={cfg['K']} "
         f"blocks={cfg['block_size1']}/{cfg['block_size2']} cores={cfg['cores']}")
    cu = torch.tensor(cfg["cu_seqlens_q"], dtype=torch.int32)
    md = sparse_attn_sharedkv_metadata(
        num_heads_q=cfg["N1"], num_heads_kv=1, head_dim=576,
        cu_seqlens_q=cu if cfg["layout_q"] == "TND" else None,
        seqused_kv=kw["seqused_kv"], batch_size=cfg["B"], max_seqlen_q=cfg["S1"],
        max_seqlen_kv=max(cfg["seqused_kv"]),
        cmp_topk=cfg["K"] if cfg["scenario"] == 3 else 0, cmp_ratio=cfg["cmp_ratio"],
        ori_win_left=cfg["ori_win_left"], layout_q=cfg["layout_q"],
        has_cmp_kv=cfg["scenario"] >= 2, aic_core_num=cfg["cores"],
        kv_cache_dtype="fp8_ds_mla")
    dev = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}
    fp8_qk = qk == "fp8"
    out, lse = sparse_attn_sharedkv(**dev, metadata=md.cuda(), return_softmax_lse=True,
                                    fp8_qk=fp8_qk)
    torch.cuda.synchronize()
    okw = {k: v for k, v in kw.items() if k != "topk_cmp"}
    ref, ref_lse = sparse_attn_oracle(**okw, fp8_qk=fp8_qk)
    o, l = out.cpu(), lse.cpu()
    assert torch.isfinite(o.float()).all(), "non-finite output"
    if fp8_qk:
        err = check_strict(o, ref)
        fin = torch.isfinite(ref_lse)
        assert torch.equal(torch.isfinite(l), fin) and torch.equal(l[~fin], ref_lse[~fin])
        lse_err = (l[fin] - ref_lse[fin]).abs()
        assert (lse_err <= 1e-3 * ref_lse[fin].abs()).all(), \
            f"lse: max abs err {lse_err.max().item()}"
        _say(f"case {i}: max |out - oracle of the form| {err['out_max_abs']:.3g}, "
             f"lse {lse_err.max().item() if lse_err.numel() else 0.0:.3g}")
        return
    err = check_strict(o, ref, l, ref_lse)
    ex, _ = sparse_attn_exact(**okw)
    acc = check_vs_exact(o, ref, ex)
    _say(f"case {i}: max |out - golden| {err['out_max_abs']:.3g}, lse {err['lse_max_abs']:.3g}; "
         f"max |out - exact| {acc['ours']:.3g} (golden {acc['golden']:.3g})")
