"""GPU parity of the fp8 cache path (656-byte rows) and its writer.

No reference code exists for fp8 caches (the reference is bf16/fp16 only,
api.py:51-56): parity here is against the CPU oracle of the row format
(``oracle/fp8_rows.py``, pinned in ``test_fp8_oracle.py``) followed by the
golden math on the dequantized rows, with the benchmark-regime bound
|out - golden| <= 2e-2 + 2e-2 |golden|, |lse - golden| <= 1e-3 |golden|.
Two stronger properties are checked too:

* the writer is byte-exact against the oracle's quantizer;
* the fp8 kernel gives bit-identical results to the bf16 kernel run on the
  dequantized cache (it converts each row to exactly those bf16 values in
  LDS and then runs the same code).
"""

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
    from sparse_attn_sharedkv_amd import _lib, api, sparse_flash_mla
    from sparse_attn_sharedkv_amd.kv_fp8 import append_kv_fp8, quantize_kv_fp8


def _say(msg):
    print(f"[gpu-fp8] {msg}", flush=True)
    sys.stdout.flush()


def _cpu(kw):
    return {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}


def _dev(kw):
    return {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}


def _run(kw, **extra):
    out, lse = sparse_flash_mla(**_dev(kw), return_softmax_lse=True, **extra)
    torch.cuda.synchronize()
    return out, lse


def _dequant_kw(kw):
    """The same call on the bf16 cache that the fp8 rows dequantize to."""
    d = dict(kw)
    d["ori_kv"] = F.dequantize_rows(kw["ori_kv"].cpu())
    if kw.get("cmp_kv") is not None:
        d["cmp_kv"] = (d["ori_kv"] if kw["cmp_kv"] is kw["ori_kv"]
                       else F.dequantize_rows(kw["cmp_kv"].cpu()))
    d.pop("kv_cache_dtype", None)
    return d


def _check(out, lse, kw, tokens=None):
    okw = {k: v for k, v in _cpu(kw).items() if k != "topk_cmp"}
    ref, ref_lse = sparse_attn_oracle(**okw, tokens=tokens)
    ex, _ = sparse_attn_exact(**okw, tokens=tokens)
    o, l = out.cpu(), lse.cpu()
    if tokens is not None:
        t = list(tokens)
        o, l, ref, ref_lse, ex = o[t], l[t], ref[t], ref_lse[t], ex[t]
    check_strict(o, ref, l, ref_lse)
    check_vs_exact(o, ref, ex)


# ---------------------------------------------------------------------------
# writer
# ---------------------------------------------------------------------------

@requires_gpu
def test_writer_bytes_match_oracle():
    _say("fp8 writer vs oracle")
    g = torch.Generator().manual_seed(21)
    x = (torch.randn((1000, 576), generator=g) * 0.5).to(torch.bfloat16)
    x[1, :128] = 0.0                                   # zero block -> scale 1
    x[2, 128:256] *= 3000.0                            # large block
    x[3, 256:384] *= 1e-30                             # tiny block (e4m3 subnormals / zeros)
    x[4, :] = -0.0                                     # negative zeros
    x[5, 384:512] = torch.linspace(-1, 1, 128)         # many distinct magnitudes
    got = quantize_kv_fp8(x.cuda()).cpu().numpy()
    want = F.quantize_rows(x)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} bytes differ, first at {bad[:5].tolist()}"


@requires_gpu
def test_writer_slot_mapping_skips_and_leaves_other_rows():
    _say("fp8 writer slot mapping")
    g = torch.Generator().manual_seed(22)
    x = (torch.randn((6, 576), generator=g) * 0.5).to(torch.bfloat16)
    cache = torch.full((4, 4, 1, 656), 0xAB, dtype=torch.uint8, device="cuda")
    slots = torch.tensor([5, -1, 0, 15, 16, 9], dtype=torch.int32)   # -1 and 16 are skipped
    append_kv_fp8(cache, x.cuda(), slots.cuda())
    torch.cuda.synchronize()
    flat = cache.reshape(16, 656).cpu().numpy()
    want = F.quantize_rows(x)
    for i, s in enumerate(slots.tolist()):
        if 0 <= s < 16:
            assert np.array_equal(flat[s], want[i])
    untouched = [r for r in range(16) if r not in (5, 0, 15, 9)]
    assert (flat[untouched] == 0xAB).all()


# ---------------------------------------------------------------------------
# attention over fp8 caches
# ---------------------------------------------------------------------------

def _fp8_case(*, lens, heads, k, seed, tnd=True, sinks="none"):
    """Top-k decode over an fp8 pool drawn directly in the row format."""
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    bs = 64
    nblk = sum((x + bs - 1) // bs for x in lens) + 2
    raw = torch.from_numpy(F.random_rows(nblk * bs, g)).reshape(nblk, bs, 1, 656)
    pool, table = gen.paged_pool(seq_lens=lens, block_size=bs, block_num=nblk,
                                 head_dim=656, dtype=torch.uint8, rng=rng,
                                 values=lambda shape: raw.clone(), zero_unused=False)
    b = len(lens)
    idx = gen.topk_indices(thresholds=lens, k=k, gen=g)
    q = (torch.randn((b, heads, 576), generator=g) * 0.5).to(torch.bfloat16)
    if sinks == "none":
        snk = torch.full((heads,), float("-inf"))
    else:
        snk = torch.rand(heads, generator=g) * 2 - 1
    kw = dict(q=q, ori_kv=pool, ori_block_table=table, cmp_kv=pool, cmp_block_table=table,
              cmp_sparse_indices=idx.reshape(b, 1, k),
              seqused_kv=torch.tensor(lens, dtype=torch.int32), sinks=snk,
              softmax_scale=1 / 24.0, cmp_ratio=1, ori_win_left=-1, head_dim_v=512,
              topk_cmp=k, kv_cache_dtype="fp8_ds_mla")
    if tnd:
        kw.update(layout_q="TND", cu_seqlens_q=torch.arange(b + 1, dtype=torch.int32))
    else:
        kw.update(layout_q="BSND", q=q.reshape(b, 1, heads, 576),
                  cmp_sparse_indices=idx.reshape(b, 1, 1, k))
    return kw


@requires_gpu
@pytest.mark.parametrize("heads,k,lens,sinks", [
    (128, 2048, [3000, 5000, 2100, 4097], "none"),
    (64, 512, [700, 1500, 513], "uniform"),
    (16, 256, [300, 1024], "uniform"),
    (128, 2048, [1000, 2500], "uniform"),        # thr < K: -1 padded rows
])
def test_fp8_attention_matches_oracle(heads, k, lens, sinks):
    _say(f"fp8 attention H={heads} K={k} lens={lens} sinks={sinks}")
    kw = _fp8_case(lens=lens, heads=heads, k=k, seed=heads + k, sinks=sinks)
    out, lse = _run(kw)
    _check(out, lse, kw)


@requires_gpu
@pytest.mark.parametrize("batch", [32, 40])
def test_fp8_128_head_items_from_32_sequences(batch):
    # fp8 rows take 128-head items from 32 sequences on (m_base_for): the default
    # path of such a call runs the 128-head kernel, checked against the oracle
    _say(f"fp8 rows, {batch} sequences, H=128: 128-head items by default")
    rng = np.random.default_rng(batch)
    lens = [int(x) for x in rng.integers(600, 2600, size=batch)]
    kw = _fp8_case(lens=lens, heads=128, k=512, seed=batch, sinks="uniform")
    prep = api.prepare(**{k: v for k, v in _dev(kw).items() if k != "topk_cmp"})
    assert prep.args.m_base == 128, prep.args.m_base
    out, lse = _run(kw)
    _check(out, lse, kw)


def _run_pipelined(kw, **extra):
    """Native rows through the kernel fp8 rows use (SAS_PHASE_PIPELINED)."""
    kw = {k: v for k, v in _dev(kw).items() if k != "topk_cmp"}
    prep = api.prepare(**kw, **extra, _pipelined=True)  # 64-head items, SAS_PHASE_PIPELINED
    api.launch(prep)
    torch.cuda.synchronize()
    return prep.out.clone(), prep.lse.clone()


@requires_gpu
@pytest.mark.parametrize("cores", [256, 7])
def test_fp8_equals_bf16_path_on_dequantized_cache(cores):
    # fp8 rows are dequantized into the same bf16 LDS layout the native rows are
    # gathered into, so the same kernel on the dequantized cache is bitwise equal
    _say(f"fp8 vs bf16-on-dequantized cores={cores}")
    kw = _fp8_case(lens=[4000, 2999, 3500], heads=128, k=2048, seed=5)
    out8, lse8 = _run(kw, core_num=cores)
    out16, lse16 = _run_pipelined(_dequant_kw(kw), core_num=cores)
    assert torch.equal(out8.cpu(), out16.reshape(out8.shape).cpu())
    assert torch.equal(lse8.cpu(), lse16.reshape(lse8.shape).cpu())
    # the default kernel for native rows agrees to within the accuracy contract
    out_d, lse_d = _run(_dequant_kw(kw), core_num=cores)
    _check(out_d, lse_d, _dequant_kw(kw))


def _run_items(kw, m_base, **extra):
    """The call with items of ``m_base`` heads (128: the 128-head kernel)."""
    kw = {k: v for k, v in _dev(kw).items() if k != "topk_cmp"}
    prep = api.prepare(**kw, **extra, _m_base=m_base)
    assert prep.args.m_base == m_base
    api.launch(prep)
    torch.cuda.synchronize()
    return prep.out.clone(), prep.lse.clone()


@requires_gpu
@pytest.mark.parametrize("cores", [256, 64, 7])
def test_fp8_128_head_items_equal_bf16_on_dequantized_cache(cores):
    # 128-head items: the 128-head kernel dequantizes each raw fp8 tile into the
    # bf16 stage layout it gathers native rows into, so it is bitwise the same
    # kernel on the dequantized cache; split items merged in-kernel or not
    _say(f"fp8 128-head items vs bf16 on dequantized cores={cores}")
    kw = _fp8_case(lens=[4000, 2999, 3500, 2100], heads=128, k=2048, seed=6, sinks="uniform")
    out8, lse8 = _run_items(kw, 128, core_num=cores)
    out16, lse16 = _run_items(_dequant_kw(kw), 128, core_num=cores)
    assert torch.equal(out8.cpu(), out16.reshape(out8.shape).cpu())
    assert torch.equal(lse8.cpu(), lse16.reshape(lse8.shape).cpu())
    _check(out8, lse8, kw)
    out_s, lse_s = _run_items(kw, 128, core_num=cores, _separate_merge=True)
    assert torch.equal(out8, out_s) and torch.equal(lse8, lse_s)


@requires_gpu
def test_fp8_bsnd_layout_and_uint8_inference():
    # kv_cache_dtype inferred from the uint8 cache; BSND layout
    _say("fp8 BSND, inferred format")
    kw = _fp8_case(lens=[2000, 2600], heads=64, k=1024, seed=8, tnd=False)
    kw.pop("kv_cache_dtype")
    out, lse = _run(kw)
    _check(out, lse, kw)


@requires_gpu
def test_long_context_fp8_workload_sampled():
    # the long-context fp8 workload (TND, H=128, ctx U[32768, 131072], top-k 2048)
    # at 8 sequences; every token checked
    _say("long-context fp8 workload, 8 sequences")
    kw = gen.build_workload("mla_fp8_decode_t128_h128_k2048", device="cuda", seed=3, batch=8)
    out, lse = _run(kw)
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()
    _check(out, lse, kw)


@requires_gpu
def test_unreferenced_nan_rows_do_not_leak():
    # masked slots of a tile read an all-zero row, never pool rows: NaN in
    # unreferenced rows (here every row of block 0 and of an unused block) stays out
    _say("unreferenced NaN rows (bf16 and fp8 caches)")
    kw = _fp8_case(lens=[1000, 700], heads=64, k=300, seed=9, sinks="uniform")
    tbl = kw["ori_block_table"].clone()
    used = set(tbl[tbl >= 0].tolist())
    spare = [blk for blk in range(kw["ori_kv"].shape[0]) if blk not in used]
    assert spare
    # make physical block 0 (pool row 0) the unreferenced one
    pool = kw["ori_kv"].clone()
    s = spare[0]
    if s != 0:
        pool[[0, s]] = pool[[s, 0]]
        tbl[tbl == 0] = s
    pool[0] = 0xFF                                     # e4m3 NaN codes and a NaN scale
    idx = kw["cmp_sparse_indices"]
    idx[:, :, 250:] = -1                               # tails: 250 valid rows per token
    kw.update(ori_kv=pool, cmp_kv=pool, ori_block_table=tbl, cmp_block_table=tbl,
              cmp_sparse_indices=idx)
    out, lse = _run(kw)
    assert torch.isfinite(out.float()).all()
    _check(out, lse, kw)
    # the same on a bf16 cache whose block 0 is NaN
    kb = _dequant_kw(kw)
    kb["ori_kv"][0] = float("nan")
    kb["cmp_kv"] = kb["ori_kv"]
    out, lse = _run(kb)
    assert torch.isfinite(out.float()).all()
    _check(out, lse, kb)


def _fp8_pool(lens, seed, bs=64):
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    nblk = sum((x + bs - 1) // bs for x in lens) + 1
    raw = torch.from_numpy(F.random_rows(nblk * bs, g)).reshape(nblk, bs, 1, 656)
    return gen.paged_pool(seq_lens=lens, block_size=bs, block_num=nblk, head_dim=656,
                          dtype=torch.uint8, rng=rng, values=lambda shape: raw.clone(),
                          zero_unused=False)


@requires_gpu
@pytest.mark.parametrize("scenario", [1, 2, 3])
def test_fp8_window_and_compressed_scenarios(scenario):
    # SWA (scenario 1), SWA + dense compressed (2), SWA + top-k compressed (3) over fp8
    # caches; two query rows per sequence (BSND, S = 2), sinks U(-1, 1)
    _say(f"fp8 scenario {scenario}")
    lens = [1500, 3000, 700]
    g = torch.Generator().manual_seed(30 + scenario)
    ori, ori_t = _fp8_pool(lens, 40 + scenario)
    s_q, h, ratio = 2, 64, 4
    kw = dict(q=(torch.randn(len(lens), s_q, h, 576, generator=g) * 0.5).to(torch.bfloat16),
              ori_kv=ori, ori_block_table=ori_t, seqused_kv=torch.tensor(lens, dtype=torch.int32),
              sinks=torch.rand(h, generator=g) * 2 - 1, softmax_scale=1 / 24.0,
              ori_win_left=127, layout_q="BSND", head_dim_v=512, kv_cache_dtype="fp8_ds_mla")
    if scenario >= 2:
        cmp, cmp_t = _fp8_pool([x // ratio for x in lens], 50 + scenario)
        kw.update(cmp_kv=cmp, cmp_block_table=cmp_t, cmp_ratio=ratio)
    if scenario == 3:
        k = 256
        thr = [(x - s_q + s + 1) // ratio for x in lens for s in range(s_q)]
        idx = gen.topk_indices(thresholds=thr, k=k, gen=g)
        kw.update(cmp_sparse_indices=idx.reshape(len(lens), s_q, 1, k), topk_cmp=k)
    from sparse_attn_sharedkv_amd import sparse_attn_sharedkv
    out, lse = sparse_attn_sharedkv(**{k2: (v.cuda() if isinstance(v, torch.Tensor) else v)
                                       for k2, v in kw.items()}, return_softmax_lse=True)
    torch.cuda.synchronize()
    okw = {k2: v for k2, v in kw.items() if k2 != "topk_cmp"}
    ref, ref_lse = sparse_attn_oracle(**okw)
    ex, _ = sparse_attn_exact(**okw)
    check_strict(out.cpu().reshape(ref.shape), ref, lse.cpu().reshape(ref_lse.shape), ref_lse)
    check_vs_exact(out.cpu().reshape(ref.shape), ref, ex.reshape(ref.shape))
