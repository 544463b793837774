"""GPU parity of the fp8 Q·Kᵀ form (``fp8_qk=True``, SAS_PHASE_FP8_QK) over fp8 caches.

The form has no reference counterpart: the reference forms Q·Kᵀ in bf16
(kernel.py:2036-2352). Each head's query latent is quantized to e4m3 with one
fp32 scale (``oracle.fp8_rows.quantize_q``), Q·Kᵀ runs on
``v_mfma_f32_16x16x128_f8f6f4`` with the rows' block scales applied per block,
and P·V stays on the dequantized bf16 rows. Two checks, both at
atol = rtol = 2e-2 on out and 1e-3 relative on the LSE:

* against the oracle of the same form (``sparse_attn_oracle(..., fp8_qk=True)``:
  ``fp8_rows.scores_fp8`` scores, golden's softmax and P·V) on every case;
* against golden on the dequantized cache with bf16 queries (the reference
  contract) on N(0, 1) * 0.5 data, the long-context fp8 workload's distribution.
  (On the reference tests' U(-10, 10) data the query quantization moves ~30 % of
  the outputs beyond 2e-2, which is why the form is opt-in.)
"""

import sys

import numpy as np
import pytest
import torch

from oracle import fp8_rows as F
from oracle import gen
from oracle.checks import check_strict
from oracle.golden_ref import sparse_attn_oracle

pytestmark = pytest.mark.gpu

HAS_GPU = torch.cuda.is_available()
requires_gpu = pytest.mark.skipif(not HAS_GPU, reason="needs a ROCm GPU")

if HAS_GPU:
    from sparse_attn_sharedkv_amd import api, sparse_attn_sharedkv, sparse_flash_mla


def _say(msg):
    print(f"[gpu-fp8qk] {msg}", flush=True)
    sys.stdout.flush()


def _cpu(kw):
    return {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()
            if k != "topk_cmp"}


def _run(kw, fn=None, **extra):
    fn = sparse_flash_mla if fn is None else fn
    dev = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}
    out, lse = fn(**dev, return_softmax_lse=True, fp8_qk=True, **extra)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu()


def _check(out, lse, kw, *, vs_golden, tokens=None):
    okw = _cpu(kw)
    ref, ref_lse = sparse_attn_oracle(**okw, tokens=tokens, fp8_qk=True)
    o, l = out.reshape(ref.shape), lse.reshape(ref_lse.shape)
    if tokens is not None:
        t = list(tokens)
        o, l, ref, ref_lse = o[t], l[t], ref[t], ref_lse[t]
    check_strict(o, ref, l, ref_lse)
    if vs_golden:
        g, g_lse = sparse_attn_oracle(**okw, tokens=tokens)
        if tokens is not None:
            g, g_lse = g[list(tokens)], g_lse[list(tokens)]
        check_strict(o, g, l, g_lse)


def _normal_fp8_case(*, lens, heads, k, seed, sinks=True):
    """Top-k decode over an fp8 pool of N(0, 1) * 0.5 rows quantized by the oracle writer."""
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    bs = 64
    nblk = sum((x + bs - 1) // bs for x in lens) + 2
    rows = (torch.randn((nblk * bs, 576), generator=g) * 0.5).to(torch.bfloat16)
    raw = torch.from_numpy(F.quantize_rows(rows)).reshape(nblk, bs, 1, 656)
    pool, table = gen.paged_pool(seq_lens=lens, block_size=bs, block_num=nblk,
                                 head_dim=656, dtype=torch.uint8, rng=rng,
                                 values=lambda shape: raw.clone(), zero_unused=False)
    b = len(lens)
    idx = gen.topk_indices(thresholds=lens, k=k, gen=g)
    q = (torch.randn((b, heads, 576), generator=g) * 0.5).to(torch.bfloat16)
    snk = (torch.rand(heads, generator=g) * 2 - 1) if sinks else torch.full((heads,), float("-inf"))
    return dict(q=q, ori_kv=pool, ori_block_table=table, cmp_kv=pool, cmp_block_table=table,
                cmp_sparse_indices=idx.reshape(b, 1, k),
                seqused_kv=torch.tensor(lens, dtype=torch.int32), sinks=snk,
                softmax_scale=1 / 24.0, cmp_ratio=1, ori_win_left=-1, head_dim_v=512,
                topk_cmp=k, kv_cache_dtype="fp8_ds_mla", layout_q="TND",
                cu_seqlens_q=torch.arange(b + 1, dtype=torch.int32))


@requires_gpu
@pytest.mark.parametrize("heads,k,lens,sinks,cores", [
    (128, 2048, [3000, 5000, 2100, 4097], False, 256),
    (64, 512, [700, 1500, 513], True, 256),
    (16, 256, [300, 1024], True, 256),
    (128, 2048, [1000, 2500], True, 256),        # thr < K: -1 padded rows
    (128, 2048, [4000, 2999, 3500], True, 7),    # split items, merged
    (48, 1030, [1100, 2000], True, 3),           # partial head block, split
])
def test_fp8qk_topk_decode(heads, k, lens, sinks, cores):
    _say(f"fp8 Q·Kᵀ top-k decode H={heads} K={k} lens={lens} cores={cores}")
    kw = _normal_fp8_case(lens=lens, heads=heads, k=k, seed=heads + k + cores, sinks=sinks)
    out, lse = _run(kw, core_num=cores)
    _check(out, lse, kw, vs_golden=True)


def _run_items(kw, m_base, **extra):
    """The call with items of ``m_base`` heads (128: the 128-head kernel, whose
    Q·Kᵀ reads the e4m3 blocks straight from its raw ring)."""
    dev = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}
    prep = api.prepare(**dev, fp8_qk=True, _m_base=m_base, **extra)
    assert prep.args.m_base == m_base
    api.launch(prep)
    torch.cuda.synchronize()
    out, lse = api.finalize(prep, True)
    return out.cpu(), lse.cpu()


@requires_gpu
@pytest.mark.parametrize("heads,k,lens,sinks,cores", [
    (128, 2048, [3000, 5000, 2100, 4097], False, 256),
    (128, 2048, [1000, 2500], True, 256),        # thr < K: -1 padded rows
    (128, 2048, [4000, 2999, 3500], True, 16),   # five pieces per item (merge kernel)
    (128, 2048, [4000, 2999, 3500], True, 6),    # two pieces per item (merged in-kernel)
    (96, 1030, [1100, 2000], True, 3),           # partial head block, split
])
def test_fp8qk_128_head_items(heads, k, lens, sinks, cores):
    # 128-head items: against both oracles, and against the 64-head items' kernel
    # (the same block dot products and folds, its own softmax steps)
    _say(f"fp8 Q·Kᵀ, 128-head items H={heads} K={k} lens={lens} cores={cores}")
    kw = _normal_fp8_case(lens=lens, heads=heads, k=k, seed=heads + k + cores + 1, sinks=sinks)
    out, lse = _run_items(kw, 128, core_num=cores)
    _check(out, lse, kw, vs_golden=True)
    out64, lse64 = _run_items(kw, 64, core_num=cores)
    d_out = (out.float() - out64.float()).abs().max().item()
    d_lse = (lse - lse64).abs().max().item()
    _say(f"128- vs 64-head items: out {d_out:.3g}, lse {d_lse:.3g}")
    assert d_out <= 2e-2 and d_lse <= 1e-4


@requires_gpu
def test_fp8qk_random_format_rows():
    # rows drawn directly in the stored format (codes uniform over the finite e4m3
    # values, scales 1e-3..1e-2): against the oracle of the same form
    _say("fp8 Q·Kᵀ on format-random rows")
    g = torch.Generator().manual_seed(61)
    rng = np.random.default_rng(61)
    lens, heads, k, bs = [2500, 1800], 64, 1024, 64
    nblk = sum((x + bs - 1) // bs for x in lens) + 1
    raw = torch.from_numpy(F.random_rows(nblk * bs, g)).reshape(nblk, bs, 1, 656)
    pool, table = gen.paged_pool(seq_lens=lens, block_size=bs, block_num=nblk, head_dim=656,
                                 dtype=torch.uint8, rng=rng, values=lambda shape: raw.clone(),
                                 zero_unused=False)
    idx = gen.topk_indices(thresholds=lens, k=k, gen=g)
    q = (torch.randn((2, heads, 576), generator=g) * 0.5).to(torch.bfloat16)
    q[1, 5] = 0.0                                          # an all-zero head
    kw = dict(q=q, ori_kv=pool, ori_block_table=table, cmp_kv=pool, cmp_block_table=table,
              cmp_sparse_indices=idx.reshape(2, 1, k), seqused_kv=torch.tensor(lens, dtype=torch.int32),
              sinks=torch.rand(heads, generator=g) * 2 - 1, softmax_scale=1 / 24.0, cmp_ratio=1,
              ori_win_left=-1, head_dim_v=512, topk_cmp=k, kv_cache_dtype="fp8_ds_mla",
              layout_q="TND", cu_seqlens_q=torch.arange(3, dtype=torch.int32))
    out, lse = _run(kw)
    _check(out, lse, kw, vs_golden=False)


@requires_gpu
@pytest.mark.parametrize("scenario", [1, 2, 3])
def test_fp8qk_window_and_compressed_scenarios(scenario):
    # SWA, SWA + dense compressed, SWA + top-k compressed over N(0, 1) * 0.5 fp8
    # caches; two query rows per sequence (BSND, S = 2)
    _say(f"fp8 Q·Kᵀ scenario {scenario}")
    lens = [1500, 3000, 700]
    g = torch.Generator().manual_seed(70 + scenario)
    rng = np.random.default_rng(70 + scenario)

    def pool(ls):
        bs = 64
        nblk = sum((x + bs - 1) // bs for x in ls) + 1
        rows = (torch.randn((nblk * bs, 576), generator=g) * 0.5).to(torch.bfloat16)
        raw = torch.from_numpy(F.quantize_rows(rows)).reshape(nblk, bs, 1, 656)
        return gen.paged_pool(seq_lens=ls, block_size=bs, block_num=nblk, head_dim=656,
                              dtype=torch.uint8, rng=rng, values=lambda shape: raw.clone(),
                              zero_unused=False)

    ori, ori_t = pool(lens)
    s_q, h, ratio = 2, 64, 4
    kw = dict(q=(torch.randn(len(lens), s_q, h, 576, generator=g) * 0.5).to(torch.bfloat16),
              ori_kv=ori, ori_block_table=ori_t, seqused_kv=torch.tensor(lens, dtype=torch.int32),
              sinks=torch.rand(h, generator=g) * 2 - 1, softmax_scale=1 / 24.0,
              ori_win_left=127, layout_q="BSND", head_dim_v=512, kv_cache_dtype="fp8_ds_mla")
    if scenario >= 2:
        cmp, cmp_t = pool([x // ratio for x in lens])
        kw.update(cmp_kv=cmp, cmp_block_table=cmp_t, cmp_ratio=ratio)
    if scenario == 3:
        k = 256
        thr = [(x - s_q + s + 1) // ratio for x in lens for s in range(s_q)]
        idx = gen.topk_indices(thresholds=thr, k=k, gen=g)
        kw.update(cmp_sparse_indices=idx.reshape(len(lens), s_q, 1, k), topk_cmp=k)
    out, lse = _run(kw, fn=sparse_attn_sharedkv)
    _check(out, lse, kw, vs_golden=True)


@requires_gpu
def test_fp8qk_long_context_workload_full_size():
    # the long-context fp8 workload at full size (128 sequences, ctx U[32768, 131072],
    # top-k 2048, H = 128): every 4th token against both oracles
    _say("fp8 Q·Kᵀ long-context workload, 128 sequences")
    kw = gen.build_workload("mla_fp8_decode_t128_h128_k2048", device="cuda", seed=3)
    out, lse = _run(kw)
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()
    _check(out, lse, kw, vs_golden=True, tokens=range(0, 128, 4))


@requires_gpu
def test_fp8qk_rejected_on_native_rows():
    kw = _normal_fp8_case(lens=[300], heads=16, k=64, seed=1)
    kw = {k: v for k, v in kw.items() if k not in ("kv_cache_dtype",)}
    kw["ori_kv"] = F.dequantize_rows(kw["ori_kv"]).reshape(*kw["ori_kv"].shape[:3], 576)
    kw["cmp_kv"] = kw["ori_kv"]
    with pytest.raises(ValueError, match="fp8_qk"):
        _run(kw)
