"""The accuracy contract of the GPU random sweep, pinned on the CPU.

Golden (golden.py:156-200) rounds P to bf16 relative to the running maximum
after each 512-row tile; the HIP kernel walks the attended rows in 64-row
softmax steps (two 32-row tiles) and moves a head's running maximum at every
step whose maximum exceeds it (the same rule at 64-row granularity).
``oracle.kernel_order`` restates that order of rounding. These tests pin the
facts the contract rests on (tests/test_gpu_random_sweep.py asserts it on the
GPU):

* golden's own algorithm, run at 32- or 64-row tiles, misses the reference's
  99.5 % rule against golden at 512-row tiles on some of the sweep's
  configurations (the rule is a property of golden's tile size, not of the
  math), while staying within the contract's bound (>= 99.25 %, nothing beyond
  2e-2);
* the kernel's order (exp2 domain, eager maximum, steps across the window /
  compressed boundary) agrees with golden at the same step size as closely as
  golden does, case by case;
* a lazily moved maximum (threshold 8) agrees clearly worse;
* ``kernel_order`` at golden's tiles and rule reproduces golden.
"""

import math

import numpy as np
import pytest
import torch

from oracle import gen
from oracle.golden_ref import attend_token, sparse_attn_exact, sparse_attn_oracle
from oracle.kernel_order import attend_token_kernel_order, compare, sparse_attn_kernel_order


def _case(i):
    cfg = gen.random_sweep_cfg(np.random.default_rng(1000 + i))
    kw = gen.build_case(cfg, torch.bfloat16, seed=2000 + i)
    kw.pop("topk_cmp", None)
    return kw


def _golden_tiles(tile, **kw):
    def attend(qt, segments, sinks, scale, d_v=None):
        return attend_token(qt, segments, sinks, scale, d_v=d_v, tile=tile)
    return sparse_attn_oracle(attend=attend, **kw)[0]


@pytest.mark.parametrize("case", [16, 120])
def test_golden_at_kernel_tiles_misses_the_reference_rule(case):
    kw = _case(case)
    ref, _ = sparse_attn_oracle(**kw)
    ex, _ = sparse_attn_exact(**kw)
    g32 = compare(_golden_tiles(32, **kw), ref, ex)
    g64 = compare(_golden_tiles(64, **kw), ref, ex)
    k0 = compare(sparse_attn_kernel_order(tile=64, tau=0.0, **kw)[0], ref, ex)
    k8 = compare(sparse_attn_kernel_order(tile=64, tau=8.0, **kw)[0], ref, ex)
    # golden itself, at 32- and 64-row tiles: under the reference's 99.5 %, inside the contract
    for g in (g32, g64):
        assert 99.25 <= g["pct_ref"] < 99.5, g
        assert g["beyond_2e2"] == 0, g
    # the kernel's order tracks golden at its step size; a lazy maximum (threshold
    # 2^8) does worse
    assert abs(k0["pct_ref"] - g64["pct_ref"]) < 0.05, (k0, g64)
    assert k0["pct_ref"] >= 99.25 and k0["beyond_2e2"] <= 1, k0
    assert k8["pct_ref"] < k0["pct_ref"] - 0.1, (k8, k0)
    # all are as accurate as golden against the float64 closed form
    for r in (g32, g64, k0):
        assert r["err_exact"] <= 2 * r["golden_exact"] + 2.0 ** -9 * float(np.nanmax(np.abs(ex)))


def test_kernel_order_at_golden_tiles_reproduces_golden():
    g = torch.Generator().manual_seed(3)
    q = (torch.rand(64, 512, generator=g) * 20 - 10).to(torch.bfloat16)
    win = (torch.rand(128, 512, generator=g) * 20 - 10).to(torch.bfloat16)
    cmp_rows = (torch.rand(700, 512, generator=g) * 15 - 5).to(torch.bfloat16)
    sinks = torch.rand(64, generator=g) * 2 - 1
    scale = 1 / math.sqrt(512)
    o_ref, l_ref = attend_token(q, [win, cmp_rows], sinks, scale)
    o_k, l_k = attend_token_kernel_order(q, [win, cmp_rows], sinks, scale, tile=512, tau=0.0,
                                         segment_tiles=True)
    # exp2(x log2 e) vs exp(x) differ in the last fp32 bits: the bf16 outputs agree
    # but for rare one-ULP flips, the LSE to fp32 precision
    d = (o_k.float() - o_ref.float()).abs()
    ulp = torch.finfo(torch.bfloat16).eps * o_ref.float().abs().clamp_min(1e-3)
    assert (d <= ulp).all()
    assert (d == 0).float().mean() > 0.99
    assert torch.allclose(l_k, l_ref, rtol=1e-6, atol=1e-6)


def test_streams_and_tile_size_change_rounding_not_math():
    # two interleaved streams (each with its own maximum, merged at the end) or
    # 32- / 64-row steps give the same float64-exact answer to bf16 precision
    g = torch.Generator().manual_seed(5)
    q = (torch.randn(32, 576, generator=g) * 0.5).to(torch.bfloat16)
    rows = (torch.randn(2048, 576, generator=g) * 0.5).to(torch.bfloat16)
    sinks = torch.full((32,), -math.inf)
    scale = 1 / math.sqrt(576)
    o1, l1 = attend_token_kernel_order(q, [rows], sinks, scale, d_v=512, tile=32, tau=0.0)
    o2, l2 = attend_token_kernel_order(q, [rows], sinks, scale, d_v=512, tile=32, tau=0.0,
                                       streams=2)
    o4, l4 = attend_token_kernel_order(q, [rows], sinks, scale, d_v=512, tile=64, tau=0.0)
    o3, l3 = attend_token(q, [rows], sinks, scale, d_v=512)
    for o in (o1, o2, o4):
        assert (o.float() - o3.float()).abs().max() <= 2e-2
    for l in (l1, l2, l4):
        assert torch.allclose(l, l3, rtol=1e-5)


def test_split_pieces_merge_like_the_closed_form():
    # a token split into two pieces (each without the sink, partials in fp32) and
    # merged in fp32 equals the closed-form merge of the same pieces, and one
    # piece is the unsplit kernel order
    from oracle.golden_ref import merge_partials
    from oracle.kernel_order import attend_token_split
    g = torch.Generator().manual_seed(7)
    q = (torch.randn(32, 576, generator=g) * 2).to(torch.bfloat16)
    rows = (torch.randn(700, 576, generator=g) * 2).to(torch.bfloat16)
    sinks = torch.randn(32, generator=g)
    scale = 1 / math.sqrt(576)
    o1, l1 = attend_token_split(q, [rows], sinks, scale, d_v=512, pieces=1)
    ow, lw = attend_token_kernel_order(q, [rows], sinks, scale, d_v=512, tile=64, tau=0.0)
    assert torch.equal(o1, ow) and torch.allclose(l1, lw, rtol=1e-6, atol=1e-6)
    o2, l2 = attend_token_split(q, [rows], sinks, scale, d_v=512, pieces=2)
    no_sink = torch.full((32,), -math.inf)
    pa = attend_token_kernel_order(q, [rows[:384]], no_sink, scale, d_v=512, tile=64, tau=0.0,
                                   out_dtype=torch.float32)
    pb = attend_token_kernel_order(q, [rows[384:]], no_sink, scale, d_v=512, tile=64, tau=0.0,
                                   out_dtype=torch.float32)
    om, lm = merge_partials([pa[0].numpy(), pb[0].numpy()], [pa[1].numpy(), pb[1].numpy()],
                            sinks.numpy())
    d = (o2.float() - torch.from_numpy(om).float()).abs()
    assert (d <= torch.finfo(torch.bfloat16).eps * torch.from_numpy(np.abs(om)).float() + 1e-6).all()
    assert np.allclose(l2.numpy(), lm, rtol=1e-5, atol=1e-5)


def test_fp16_partials_keep_their_scale():
    # the kernels' split-KV partial format (fp16_partial): every row is scaled by a
    # power of two that puts its largest |value| into [2^14, 2^15), up or down, so a
    # row keeps fp16's relative precision against its largest value at any
    # magnitude a bf16 cache can produce (~1e-38 .. 3e38), and stays finite
    from oracle.kernel_order import fp16_partial
    g = torch.Generator().manual_seed(3)
    for mag in (2.0 ** -130, 2.0 ** -112, 1e-30, 2.0 ** -24, 1e-8, 1e-3, 1.0, 100.0, 2.0 ** 15,
                2.0 ** 15 * 1.999, 1e6, 3e38):
        o = torch.randn(4, 512, generator=g)
        o = o / o.abs().amax(dim=1, keepdim=True) * mag
        o = o.clamp(-3.3e38, 3.3e38)
        r = fp16_partial(o)
        assert torch.isfinite(r).all()
        m = o.abs().amax(dim=1, keepdim=True)
        # scaled into [2^14, 2^15), where fp16's half spacing is 8: every element,
        # the row max included, within 2^-11 of the row max (below 2^-112 the scale
        # stops at 2^126 and the spacing is relative to 2^-112)
        tol = torch.maximum(m, torch.full_like(m, 2.0 ** -112))
        assert ((r - o).abs() <= tol * 2.0 ** -11).all(), mag
        assert ((r.abs().amax(dim=1, keepdim=True) - m).abs() <= tol * 2.0 ** -11).all(), mag
    # the scale itself: m = 1.5 * 2^-20 is stored as fp16 of m * 2^34 (= 1.5 * 2^14, exact)
    o = torch.zeros(1, 8)
    o[0, 0] = 1.5 * 2.0 ** -20
    o[0, 1] = 2.0 ** -40  # 2^-6 after scaling: a normal fp16, kept exactly
    assert torch.equal(fp16_partial(o), o)
    # a one-sided rule (rows below 2^15 left unscaled, as fp16 subnormals) fails the
    # small rows: 2^-24 * 1.3 would be rounded to fp16's subnormal spacing 2^-24
    small = torch.full((1, 4), 1.3 * 2.0 ** -24)
    one_sided = small.to(torch.float16).to(torch.float32)
    assert (one_sided - small).abs().max() > small.abs().max() * 2.0 ** -11
    assert ((fp16_partial(small) - small).abs() <= small.abs().max() * 2.0 ** -11).all()
    # an all-zero row stays zero; NaN elements stay NaN and do not pick the scale;
    # infinities stay infinite
    assert torch.equal(fp16_partial(torch.zeros(2, 8)), torch.zeros(2, 8))
    o = torch.ones(2, 8) * 40000.0
    o[0, 3] = float("nan")
    o[1, 2] = float("inf")
    r = fp16_partial(o)
    assert torch.isnan(r[0, 3]) and torch.isinf(r[1, 2])
    assert torch.allclose(r[0, :3], o[0, :3], rtol=2 ** -11)


def test_split_with_fp16_partials_matches_fp32_partials():
    # on the reference's input distribution the fp16 partials change the merged
    # result by at most fp16's rounding of the pieces (2^-11 of the row's largest
    # value, twice for the weights summing to 1 in the worst case) plus one bf16
    # rounding step of the fp32-partial result, and only in a few elements
    from oracle.kernel_order import attend_token_split
    g = torch.Generator().manual_seed(11)
    q = ((torch.rand(64, 512, generator=g) * 20 - 10)).to(torch.bfloat16)
    rows = ((torch.rand(900, 512, generator=g) * 20 - 10)).to(torch.bfloat16)
    sinks = torch.rand(64, generator=g) * 2 - 1
    scale = 1 / math.sqrt(512)
    o32, l32 = attend_token_split(q, [rows], sinks, scale, d_v=512, pieces=3)
    o16, l16 = attend_token_split(q, [rows], sinks, scale, d_v=512, pieces=3,
                                  partial_dtype=torch.float16)
    assert torch.equal(l16, l32)
    d = (o16.float() - o32.float()).abs()
    row = o32.float().abs().amax(dim=1, keepdim=True)
    assert (d <= 2.0 ** -10 * row + torch.finfo(torch.bfloat16).eps * o32.float().abs()).all()
    assert (d > 0).float().mean() < 0.05


def test_rescale_study_reproduces_the_sweep_figures():
    # ``oracle.rescale_study`` (the 300-configuration study behind the contract)
    # on the three configurations that set its worst figures: 16 is the lowest
    # agreement for golden at 64-row tiles, the kernel's order and fp16 split
    # partials (the one configuration under 99.25 % with fp16 partials); 138 is the
    # one where the kernel's order (and fp16 split partials) put one element beyond
    # 2e-2; 48 is one where bf16 partials would put 8 elements beyond 2e-2 and fp16
    # partials none (the worst has 19) -- why the split pieces are stored in fp16.
    from oracle import rescale_study as R

    rows = {i: R.run_case(i) for i in (16, 138, 48)}
    r16, r138, r48 = rows[16], rows[138], rows[48]
    assert 99.25 <= r16["golden64"]["pct_ref"] < 99.5
    assert r16["golden64"]["beyond_2e2"] == 0
    assert r16["t64_tau0"]["pct_ref"] == pytest.approx(99.296, abs=1e-3)
    assert 99.2 <= r16["t64_split2_f16"]["pct_ref"] < 99.25
    assert r138["golden64"]["beyond_2e2"] == 0
    assert r138["t64_tau0"]["beyond_2e2"] == 1 and r138["t64_split2_f16"]["beyond_2e2"] == 1
    assert r48["t64_split2_bf16"]["beyond_2e2"] == 8
    assert r48["t64_split2_f16"]["beyond_2e2"] == 0
    s = R.summarize(list(rows.values()))
    assert s["t64_tau0"]["min_pct"] >= 99.25 and s["t64_tau0"]["max_beyond_2e2"] <= 1
    assert s["t64_split2_f16"]["max_ratio_exact"] <= 1.25
