"""The split-KV merge done inside the attention kernel (``SasAttnArgs.merge_sync``).

The last piece of a split item to finish merges the item's partials itself, so
no merge kernel runs. Its arithmetic is the merge kernel's operation for
operation, so every case here is checked bit for bit against the same call with
the merge kernel (``_separate_merge=True``), and against the oracle under the
benchmark bound (``check_strict``):

* schedules of 1 to 256 workgroups on the 128-head decode shape, in 64-head and
  in 128-head items (items split into 1 to 8 pieces, several items per
  workgroup, pieces that continue an item begun two and more workgroups
  earlier), and a partial last head block;
* calls back to back on one stream with different schedules: the arrival
  counters return to zero after every call (read back at the end), so a call
  never sees the previous call's counts;
* a device-built schedule (the kernel reads the FA rows it walks back over from
  the schedule the GPU wrote).
"""

import sys

import pytest
import torch

from oracle import gen
from oracle.checks import check_strict
from oracle.golden_ref import sparse_attn_oracle

pytestmark = pytest.mark.gpu

HAS_GPU = torch.cuda.is_available()
requires_gpu = pytest.mark.skipif(not HAS_GPU, reason="needs a ROCm GPU")

if HAS_GPU:
    from sparse_attn_sharedkv_amd import api


def _say(msg):
    print(f"[gpu-merge-in-kernel] {msg}", flush=True)
    sys.stdout.flush()


def _call(kw, separate, **extra):
    prep = api.prepare(**kw, _separate_merge=separate, **extra)
    if "_m_base" in extra:
        assert prep.args.m_base == extra["_m_base"]
    prep.out.fill_(float("nan"))
    prep.lse.fill_(float("nan"))
    api.launch(prep)
    torch.cuda.synchronize()
    return prep, prep.out.clone(), prep.lse.clone()


def _oracle_check(kw, out, lse):
    okw = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()
           if k != "topk_cmp"}
    ref, ref_lse = sparse_attn_oracle(**okw)
    check_strict(out.cpu(), ref, lse.cpu(), ref_lse)


def _sync_words_zero():
    for buf in api._MERGE_SYNC.values():
        assert int(buf.abs().sum().item()) == 0, "arrival counters left nonzero"


@requires_gpu
@pytest.mark.parametrize("m_base", [64, 128])
@pytest.mark.parametrize("cores", [1, 3, 7, 16, 64, 100, 256])
def test_merge_in_kernel_bitwise_equal_to_merge_kernel(cores, m_base):
    # 64-head items run on the one-wave-per-SIMD kernel, 128-head items on the
    # 128-head kernel: both merge in-kernel
    kw = gen.build_workload("mla_decode_b64_h128_k2048", device="cuda", seed=70 + cores, batch=8)
    if cores % 2:  # sinks U(-1, 1) (the merge folds them in); none otherwise
        g = torch.Generator(device="cuda").manual_seed(cores)
        kw["sinks"] = torch.rand(128, generator=g, device="cuda") * 2 - 1
    _say(f"H=128 K=2048 batch 8, {cores} workgroups, {m_base}-head items")
    _, o_sep, l_sep = _call(kw, True, core_num=cores, _m_base=m_base)
    _, o, l = _call(kw, False, core_num=cores, _m_base=m_base)
    assert torch.isfinite(o.float()).all()
    assert torch.equal(o, o_sep) and torch.equal(l, l_sep)
    _oracle_check(kw, o.reshape(kw["q"].shape[:-1] + (512,)), l.reshape(kw["q"].shape[:-1]))
    _sync_words_zero()


@requires_gpu
@pytest.mark.parametrize("m_base", [64, 128])
def test_merge_in_kernel_partial_head_block_and_multi_row(m_base):
    # 96 heads (a partial last head block) and 2 query rows per sequence
    kw = gen.build_workload("mla_mtp_decode_b64_h128_k2048", device="cuda", seed=81, batch=4)
    kw["q"] = kw["q"][:, :, :96].contiguous()
    kw["sinks"] = kw["sinks"][:96].contiguous()
    _say(f"H=96, 2 query rows, 4 sequences, 256 workgroups, {m_base}-head items")
    _, o_sep, l_sep = _call(kw, True, core_num=256, _m_base=m_base)
    prep, o, l = _call(kw, False, core_num=256, _m_base=m_base)
    assert prep.args.num_fd > 0
    assert torch.equal(o, o_sep) and torch.equal(l, l_sep)
    _oracle_check(kw, o.reshape(kw["q"].shape[:-1] + (512,)), l.reshape(kw["q"].shape[:-1]))


@requires_gpu
def test_merge_in_kernel_back_to_back_schedules():
    # several calls on one stream, each with another schedule; the merge
    # kernel's results are computed first, then the in-kernel merges run in a row
    cases = [(8, 256, 128), (3, 7, 64), (8, 64, 128), (1, 256, 64), (5, 100, 128)]
    expect = []
    for i, (batch, cores, mb) in enumerate(cases):
        kw = gen.build_workload("mla_decode_b64_h128_k2048", device="cuda", seed=90 + i,
                                batch=batch)
        _, o_sep, l_sep = _call(kw, True, core_num=cores, _m_base=mb)
        expect.append((kw, cores, mb, o_sep, l_sep))
    preps = [api.prepare(**kw, core_num=cores, _m_base=mb, _separate_merge=False)
             for kw, cores, mb, _, _ in expect]
    for p in preps:
        api.launch(p)  # no synchronisation between the calls
    torch.cuda.synchronize()
    for (kw, cores, _, o_sep, l_sep), p in zip(expect, preps):
        _say(f"batch {kw['q'].shape[0]} cores {cores}")
        assert torch.equal(p.out, o_sep) and torch.equal(p.lse, l_sep)
    _sync_words_zero()


@requires_gpu
def test_merge_in_kernel_device_schedule():
    kw = gen.build_workload("mla_decode_b64_h128_k2048", device="cuda", seed=99, batch=16)
    _say("device-built schedule, batch 16")
    _, o_sep, l_sep = _call(kw, True, schedule="host")
    _, o, l = _call(kw, False, schedule="device")
    assert torch.equal(o, o_sep) and torch.equal(l, l_sep)
    _sync_words_zero()


@requires_gpu
@pytest.mark.parametrize("name,batch,cores,fused", [
    ("mla_decode_b64_h128_k2048", 64, 256, True),      # 64-head items in 2 pieces
    ("swa_topk_decode_b32_h64_k512", 32, 256, False),  # items of 8 pieces
    ("mla_decode_b64_h128_k2048", 8, 256, False),
])
def test_merge_placement_default(name, batch, cores, fused):
    # by default items of at most two pieces are merged in the attention kernel,
    # items of more pieces by the merge kernel, on host- and device-built schedules
    kw = gen.build_workload(name, device="cuda", seed=5, batch=batch)
    for sched in ("host", "device"):
        prep = api.prepare(**kw, core_num=cores, schedule=sched)
        assert prep.merge_in_kernel == fused, (sched, prep.merge_in_kernel)
