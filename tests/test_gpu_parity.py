"""GPU parity: the HIP path against the CPU oracle on identical seeded inputs.

Cases follow the reference's suites: decode at kv = 8193 for SWA / CFA / SCFA
in bf16 and fp16 (test_sparse_attn_sharedkv.py:81-235, :586-605), the shrunk
prefill cases including the ragged two-sequence ones
(test_sparse_attn_sharedkv_fast.py:147-179), the full 8K prefill cases on
every query row through both entry points, the return-type contract
(:608-715) and the metadata-then-kernel flow (:484-583). Beyond them: the
benchmark shapes (H = 16 / 64 / 128, d_qk = 576 with d_v = 512, pure top-k,
MTP), split-KV invariance, index edge cases, and the full-size DeepSeek-V3.2
decode checked on sampled tokens.

Acceptance:
* reference cases (q, KV ~ U(-10, 10)): the reference's own rule
  (check_result / check_lse, >= 99.5 % within bf16 rtol 2^-7, atol 1e-4);
* benchmark shapes (q, KV ~ N(0, 1) * 0.5): the stated bound
  |out - golden| <= 2e-2 + 2e-2 |golden|, |lse - golden| <= 1e-3 |golden|.
  (The 99.5 % rule is not used here: in this regime golden itself fails it
  against golden with 32-row instead of 512-row tiles, since P is rounded to
  bf16 relative to a different running max.)
* always: max |out - exact| <= 2 max |golden - exact| + 2^-9 max |exact|, with
  exact the float64 closed form over the same rows -- the kernel is as
  accurate as golden.
"""

import functools
import math
import sys

import numpy as np
import pytest
import torch

from oracle import gen
from oracle.checks import check_lse, check_result, check_strict, check_vs_exact
from oracle.golden_ref import (attend_token, one_shot_reference, sparse_attn_exact,
                               sparse_attn_oracle, token_rows)

pytestmark = pytest.mark.gpu

HAS_GPU = torch.cuda.is_available()
requires_gpu = pytest.mark.skipif(not HAS_GPU, reason="needs a ROCm GPU")

if HAS_GPU:
    from sparse_attn_sharedkv_amd import (api, sparse_attn_sharedkv, sparse_attn_sharedkv_metadata,
                                          sparse_flash_mla)
    from sparse_attn_sharedkv_amd.metadata import config_row


def _say(msg):
    print(f"[gpu-parity] {msg}", flush=True)
    sys.stdout.flush()


def _dev(kw, device="cuda"):
    return {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}


def _cpu(kw):
    return {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}


def _oracle(kw):
    okw = {k: v for k, v in _cpu(kw).items() if k not in ("topk_cmp",)}
    return sparse_attn_oracle(**okw)


def _exact(kw, max_tokens=64):
    """float64 closed form on up to ``max_tokens`` evenly spaced tokens (others NaN)."""
    okw = {k: v for k, v in _cpu(kw).items() if k not in ("topk_cmp",)}
    q = okw["q"]
    total = q.shape[0] if okw["layout_q"] == "TND" else q.shape[0] * q.shape[1]
    step = max(1, total // max_tokens)
    return sparse_attn_exact(**okw, tokens=range(0, total, step))


def _check_reference_regime(out, lse, kw, dtype):
    ref, ref_lse = _oracle(kw)
    check_result(out.cpu(), ref)
    check_lse(lse.cpu(), ref_lse, dtype)
    ex, _ = _exact(kw)
    check_vs_exact(out.cpu(), ref, ex)


def _check_benchmark_regime(out, lse, kw, dtype=torch.bfloat16):
    ref, ref_lse = _oracle(kw)
    check_strict(out.cpu(), ref, lse.cpu(), ref_lse)
    ex, _ = _exact(kw)
    check_vs_exact(out.cpu(), ref, ex)


def _run(kw, fn=None, **extra):
    fn = fn or sparse_attn_sharedkv
    out, lse = fn(**_dev(kw), return_softmax_lse=True, **extra)
    torch.cuda.synchronize()
    return out, lse


@requires_gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("name", ["scfa_decode", "swa_decode", "cfa_decode"])
def test_reference_decode(name, dtype):
    _say(f"reference decode {name} {dtype}")
    kw = gen.build_case(gen.REFERENCE_CASES[name], dtype)
    out, lse = _run(kw)
    _check_reference_regime(out, lse, kw, dtype)


@requires_gpu
@pytest.mark.parametrize("name", list(gen.FAST_CASES))
def test_reference_fast_prefill(name):
    _say(f"reference fast prefill {name}")
    kw = gen.build_case(gen.FAST_CASES[name], torch.bfloat16)
    out, lse = _run(kw)
    _check_reference_regime(out, lse, kw, torch.bfloat16)


@requires_gpu
@pytest.mark.parametrize("name", ["swa_prefill_fast", "cfa_prefill_fast", "scfa_prefill_fast"])
def test_flash_mla_fast_scenarios(name):
    # the flash-MLA twin's self-test (sparse_flash_mla_api.py:256-272) runs its
    # FAST_SCENARIOS (sparse_flash_mla_golden.py:391-461: S1 = 1024, H = 64, d 512,
    # block_num1 10, block_num2 1 / 2 / 3) through sparse_flash_mla; the shrunk
    # reference cases have exactly those parameters
    _say(f"flash-MLA fast scenario {name}")
    cfg = gen.FAST_CASES[name]
    assert (cfg["S1"], cfg["N1"], cfg["D"], cfg["block_num1"]) == (1024, 64, 512, 10)
    assert cfg["block_num2"] == {1: 1, 2: 2, 3: 3}[cfg["scenario"]]
    kw = gen.build_case(cfg, torch.bfloat16)
    out, lse = _run(kw, fn=sparse_flash_mla)
    _check_reference_regime(out, lse, kw, torch.bfloat16)


@functools.lru_cache(maxsize=1)
def _full_prefill_case(name):
    """Inputs, the oracle over every query row, and the float64 closed form on
    sampled rows (start, around the window and compressed-threshold edges,
    middle, end) for one of the reference's 8K prefill cases; kept for the
    next test, which runs the same case through the other entry point."""
    kw = gen.build_case(gen.REFERENCE_CASES[name], torch.bfloat16)
    okw = {k: v for k, v in kw.items() if k not in ("topk_cmp",)}
    ref, ref_lse = sparse_attn_oracle(**okw)
    total = kw["q"].shape[0]
    toks = sorted({0, 1, 3, 126, 127, 128, 129, 511, 512, 2047, 2048, 2049, 4095, 6143,
                   total - 2, total - 1})
    ex, _ = sparse_attn_exact(**okw, tokens=toks)
    return kw, ref, ref_lse, toks, ex[toks]


@requires_gpu
@pytest.mark.parametrize("entry", ["sparse_attn_sharedkv", "sparse_flash_mla"])
@pytest.mark.parametrize("name", ["swa_prefill", "cfa_prefill", "scfa_prefill"])
def test_reference_prefill_full_size(name, entry):
    # the reference's own 8K prefill cases (test_sparse_attn_sharedkv.py:105-220,
    # the same parameters as the flash-MLA twin's FULL_SCENARIOS,
    # sparse_flash_mla_test_full.py:5-40) at full size through either entry
    # point, every query row against the oracle by the reference's rule
    _say(f"full-size reference prefill {name} via {entry}")
    kw, ref, ref_lse, toks, ex = _full_prefill_case(name)
    out, lse = _run(kw, fn=sparse_flash_mla if entry == "sparse_flash_mla" else None)
    out, lse = out.cpu(), lse.cpu()
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()
    check_result(out, ref)
    check_lse(lse, ref_lse, torch.bfloat16)
    check_vs_exact(out[toks], ref[toks], ex)


@requires_gpu
def test_api_return_type():
    _say("api return type")
    cfg = gen.REFERENCE_CASES["swa_decode"]
    kw = _dev(gen.build_case(cfg, torch.bfloat16))
    o1 = sparse_attn_sharedkv(**kw, return_softmax_lse=False)
    o2 = sparse_attn_sharedkv(**kw, return_softmax_lse=True)
    torch.cuda.synchronize()
    assert isinstance(o1, torch.Tensor) and o1.shape == (cfg["T1"], cfg["N1"], cfg["D"])
    assert o1.dtype == torch.bfloat16
    assert isinstance(o2, tuple) and len(o2) == 2
    out, lse = o2
    assert out.shape == (cfg["T1"], cfg["N1"], cfg["D"]) and lse.shape == (cfg["T1"], cfg["N1"])
    assert lse.dtype == torch.float32
    torch.testing.assert_close(out.cpu(), o1.cpu(), rtol=0, atol=0)


@requires_gpu
@pytest.mark.parametrize("name", ["scfa_decode", "scfa_prefill_b2", "cfa_prefill_b2"])
def test_metadata_then_kernel(name):
    # test_sparse_attn_sharedkv.py:484-583: schedule on the host, pass it in on the device
    _say(f"metadata then kernel {name}")
    cfg = dict(gen.REFERENCE_CASES, **gen.FAST_CASES)[name]
    kw = gen.build_case(cfg, torch.bfloat16)
    md = sparse_attn_sharedkv_metadata(
        num_heads_q=cfg["N1"], num_heads_kv=1, head_dim=cfg["D"],
        cu_seqlens_q=kw["cu_seqlens_q"], seqused_kv=kw["seqused_kv"], batch_size=cfg["B"],
        max_seqlen_q=cfg["T1"], max_seqlen_kv=max(cfg["seqused_kv"]),
        cmp_topk=cfg["K"] if cfg["scenario"] == 3 else 0, cmp_ratio=cfg["cmp_ratio"],
        ori_win_left=127, layout_q="TND", has_cmp_kv=cfg["scenario"] >= 2)
    assert md.dtype == torch.int32 and md.numel() == 16384
    out, lse = _run(kw, metadata=md.cuda())
    _check_reference_regime(out, lse, kw, torch.bfloat16)


def _reduced_workload(name, batch, seed=0, ctx=None):
    return gen.build_workload(name, device="cuda", seed=seed, batch=batch, ctx_override=ctx)


@requires_gpu
@pytest.mark.parametrize("name,batch", [
    ("topk_decode_b2_h16_k256", None),
    ("swa_decode_b32_h64", 6),
    ("swa_topk_decode_b32_h64_k512", 3),
    ("mla_decode_b64_h128_k2048", 3),
    ("mla_mtp_decode_b64_h128_k2048", 2),
])
def test_benchmark_shapes_reduced(name, batch):
    _say(f"benchmark shape {name} batch={batch}")
    kw = _reduced_workload(name, batch)
    out, lse = _run(kw, fn=sparse_flash_mla)
    _check_benchmark_regime(out, lse, kw)


@requires_gpu
@pytest.mark.parametrize("heads,d", [(16, 576), (48, 576), (96, 576), (48, 512), (112, 512)])
@pytest.mark.parametrize("cores", [None, 5])
def test_partial_head_blocks(heads, d, cores, monkeypatch):
    # head counts that leave the last 32/64-head block partly empty (lanes without
    # a head), with and without split items (5 cores: every item in pieces)
    from sparse_attn_sharedkv_amd import workloads as wl
    _say(f"partial head blocks H={heads} d={d} cores={cores}")
    w = dict(wl.WORKLOADS["swa_topk_decode_b32_h64_k512"], H=heads, D=d, ctx=(3000, 9000))
    monkeypatch.setitem(wl.WORKLOADS, "_partial_heads", w)
    kw = gen.build_workload("_partial_heads", device="cuda", seed=heads + d, batch=4)
    extra = {"core_num": cores} if cores else {}
    out, lse = _run(kw, fn=sparse_flash_mla, **extra)
    _check_benchmark_regime(out, lse, kw)


@requires_gpu
def test_swa_topk_short_context_pads_minus_one():
    # one sequence with thr < K so the index rows carry -1 padding
    _say("swa+topk short context")
    kw = _reduced_workload("swa_topk_decode_b32_h64_k512", None, ctx=[1500, 16384, 900])
    assert (kw["cmp_sparse_indices"] == -1).any()
    out, lse = _run(kw, fn=sparse_flash_mla)
    _check_benchmark_regime(out, lse, kw)


@requires_gpu
@pytest.mark.parametrize("cores", [1, 3, 64, 256, 512])
def test_split_kv_invariance(cores):
    # the merged result must not depend on how the rows are split over workgroups
    _say(f"split invariance cores={cores}")
    kw = _reduced_workload("mla_decode_b64_h128_k2048", 2, seed=3)
    out, lse = _run(kw, fn=sparse_flash_mla, core_num=cores)
    _check_benchmark_regime(out, lse, kw)


@requires_gpu
def test_topk_index_edge_cases():
    # -1 in the middle stops the scan; ids >= thr are skipped; duplicates count twice;
    # an all -1 row attends only the sink
    _say("top-k edge cases")
    g = torch.Generator().manual_seed(7)
    lens = [300, 300, 300, 300]
    pool, table = gen.paged_pool(seq_lens=lens, block_size=64, block_num=24, head_dim=576,
                                 dtype=torch.bfloat16, rng=np.random.default_rng(7),
                                 values=lambda s: torch.randn(s, generator=g) * 0.5)
    k = 40
    idx = torch.randint(0, 300, (4, 1, 1, k), generator=g, dtype=torch.int32)
    idx[0, 0, 0, 17] = -1                  # stop in the middle
    idx[1, 0, 0, ::3] = 299 + 5            # beyond the causal bound -> skipped
    idx[2, 0, 0, 10:20] = idx[2, 0, 0, 0]  # duplicates
    idx[3] = -1                            # nothing but the sink
    kw = dict(q=(torch.randn(4, 1, 64, 576, generator=g) * 0.5).to(torch.bfloat16),
              ori_kv=pool, ori_block_table=table, cmp_kv=pool, cmp_block_table=table,
              cmp_sparse_indices=idx, seqused_kv=torch.tensor(lens, dtype=torch.int32),
              sinks=torch.rand(64, generator=g) * 2 - 1, softmax_scale=1 / 24, cmp_ratio=1,
              ori_win_left=-1, layout_q="BSND", head_dim_v=512, topk_cmp=k)
    out, lse = _run(kw)
    _check_benchmark_regime(out, lse, kw)
    torch.testing.assert_close(lse[3, 0].cpu(), kw["sinks"].float(), rtol=1e-6, atol=1e-6)


@requires_gpu
def test_full_size_mla_decode_sampled_tokens():
    # B=64, H=128, K=2048, ctx 32768: the benchmark workload itself; tokens sampled
    _say("full-size mla decode (sampled)")
    kw = gen.build_workload("mla_decode_b64_h128_k2048", device="cuda", seed=11)
    out, lse = _run(kw, fn=sparse_flash_mla)
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()
    q = kw["q"]
    b_n, s_max, n1, d = q.shape
    lens = kw["seqused_kv"].cpu().tolist()
    idx = kw["cmp_sparse_indices"]
    for b in (0, 31, 63):
        ori_rows, cmp_rows = token_rows(
            b=b, s=0, act_q=1, act_kv=lens[b], ori_kv=kw["ori_kv"],
            ori_block_table=kw["ori_block_table"], cmp_kv=kw["cmp_kv"],
            cmp_block_table=kw["cmp_block_table"], cmp_idx_row=idx[b, 0, 0].cpu().tolist(),
            cmp_ratio=1, ori_win_left=-1)
        ro, rl = attend_token(q[b, 0].cpu(), [ori_rows.cpu(), cmp_rows.cpu()],
                              kw["sinks"].cpu(), kw["softmax_scale"], d_v=512)
        check_strict(out[b, 0].cpu(), ro, lse[b, 0].cpu(), rl)
        rows = torch.cat([ori_rows, cmp_rows]).cpu().double().numpy()
        ex, _ = one_shot_reference(q[b, 0].cpu().double().numpy(), rows,
                                   kw["sinks"].cpu().double().numpy(), kw["softmax_scale"])
        check_vs_exact(out[b, 0].cpu(), ro, ex[:, :512])


def _call_phases(kw, phases, **extra):
    prep = api.prepare(**_dev(kw), **extra)
    api.launch(prep, phases=phases)
    torch.cuda.synchronize()
    return prep.out.clone(), prep.lse.clone()


@requires_gpu
def test_split_item_without_sink_and_without_keys():
    # sinks -inf (no sink) and a token whose index row is all -1: golden gives
    # m = -inf, l = 1 -> out 0, lse -inf; every split piece of that token is empty
    _say("split item with no sink and no keys")
    kw = _reduced_workload("mla_decode_b64_h128_k2048", 2, seed=9)
    kw["cmp_sparse_indices"][1] = -1
    kw["sinks"] = torch.full_like(kw["sinks"], float("-inf"))
    out, lse = _call_phases(kw, 0, core_num=256)
    out = out.reshape(kw["q"].shape[:-1] + (512,))
    lse = lse.reshape(kw["q"].shape[:-1])
    assert torch.equal(out[1].float().cpu(), torch.zeros_like(out[1].float().cpu()))
    assert torch.isneginf(lse[1]).all()
    _check_benchmark_regime(out, lse, kw)


@requires_gpu
def test_split_partials_of_large_values():
    # split-KV partials are stored as fp16 scaled by a power of two per (piece, head)
    # row; cache values of 2^24 times the usual size (q scaled down by as much, so
    # the scores are the usual ones) make the partial rows exceed fp16's range
    # unless scaled. Golden is exactly 2^24 times golden on the unscaled inputs
    # (power-of-two scalings commute with every rounding), so the result divided by
    # 2^24 is checked against golden on those, with every item split.
    _say("split partials of large values")
    kw = _reduced_workload("mla_decode_b64_h128_k2048", 2, seed=13)
    big = dict(kw)
    for key in ("ori_kv", "cmp_kv"):
        big[key] = kw[key] * 2.0 ** 24
    big["q"] = kw["q"] * 2.0 ** -24
    out, lse = _run(big, fn=sparse_flash_mla, core_num=256)
    assert torch.isfinite(out.float()).all()
    assert out.float().abs().max() > 2.0 ** 16  # beyond fp16's range
    _check_benchmark_regime((out.float() * 2.0 ** -24).to(out.dtype), lse, kw)


@requires_gpu
@pytest.mark.parametrize("separate", [False, True])
def test_split_partials_of_small_values(separate):
    # the mirror case: cache values 2^-24 times the usual size (q scaled up by as
    # much) make every partial row lie below fp16's normal range (2^-14) unless
    # scaled up; golden is exactly 2^-24 times golden on the unscaled inputs, so the
    # result times 2^24 is checked against golden on those, with every item split,
    # for the merge inside the attention kernel and for the merge kernel
    _say(f"split partials of small values (separate merge kernel: {separate})")
    kw = _reduced_workload("mla_decode_b64_h128_k2048", 2, seed=17)
    small = dict(kw)
    for key in ("ori_kv", "cmp_kv"):
        small[key] = kw[key] * 2.0 ** -24
    small["q"] = kw["q"] * 2.0 ** 24
    prep = api.prepare(**_dev(small), core_num=256, _separate_merge=separate)
    assert prep.args.num_fd > 0
    api.launch(prep)
    torch.cuda.synchronize()
    out = prep.out.reshape(kw["q"].shape[:-1] + (512,))
    lse = prep.lse.reshape(kw["q"].shape[:-1])
    assert torch.isfinite(out.float()).all()
    assert 0 < out.float().abs().max() < 2.0 ** -14  # below fp16's normal range
    _check_benchmark_regime((out.float() * 2.0 ** 24).to(out.dtype), lse, kw)
