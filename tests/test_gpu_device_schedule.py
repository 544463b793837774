"""The on-device scheduler (``sas_metadata_build_device``) on a GPU.

* Word-for-word equality with the host scheduler (``sas_metadata_build``) over
  seeded random decode, MTP and prefill length sets, all three scenarios,
  windows from empty to 1024 rows, top-k widths, head counts and core counts,
  including empty batches and zero-length sequences. The host scheduler's
  invariants are pinned on the CPU (tests/test_metadata.py); equality carries
  them over.
* The attention launched from a device-built schedule (no host read-back)
  gives bitwise the outputs of the host-scheduled launch.
* The whole call -- scheduler, attention, merge -- captured in one HIP graph
  and replayed with new sequence lengths written in place, every replay
  bitwise equal to the eager host-scheduled call; two calls captured into two
  graphs and replayed in alternation likewise (each capture owns its schedule
  and arrival-counter buffers).
* A schedule the kernels cannot use (wrong head count, a negative length)
  turns every output into NaN instead of leaving stale memory.
"""

import os
import sys

import numpy as np
import pytest
import torch

from oracle import gen

pytestmark = pytest.mark.gpu

HAS_GPU = torch.cuda.is_available()
requires_gpu = pytest.mark.skipif(not HAS_GPU, reason="needs a ROCm GPU")

if HAS_GPU:
    from sparse_attn_sharedkv_amd import (api, sparse_attn_sharedkv,
                                          sparse_attn_sharedkv_metadata, sparse_flash_mla)
    from sparse_attn_sharedkv_amd.metadata import build_metadata, build_metadata_device


def _say(msg):
    print(f"[gpu-devsched] {msg}", flush=True)
    sys.stdout.flush()


def _random_cases(seed=0, n=60):
    rng = np.random.default_rng(seed)
    cases = []
    for c in range(n):
        kind = ["decode", "mtp", "prefill", "ragged"][c % 4]
        scenario = int(rng.integers(1, 4))
        heads = int(rng.choice([16, 32, 48, 64, 96, 128]))
        hblocks = -(-heads // (32 if heads <= 32 else 64))
        if kind == "decode":
            b = int(rng.choice([0, 1, 2, 5, 17, 64, 128, 300]))
            act_q = [1] * b
        elif kind == "mtp":
            b = int(rng.choice([1, 8, 64]))
            act_q = [2] * b
        elif kind == "prefill":
            b = int(rng.choice([1, 2]))
            act_q = [int(rng.integers(1, 16384 // (b * hblocks) + 1)) for _ in range(b)]
        else:
            b = int(rng.integers(1, 40))
            act_q = [int(x) for x in rng.integers(0, 9, size=b)]
        act_kv = [int(q + rng.integers(0, 140000)) for q in act_q]
        if b and rng.random() < 0.3:
            act_kv[int(rng.integers(0, b))] = act_q[0] if act_q else 0  # short sequence
        win = int(rng.choice([-1, 0, 127, 1023]))
        ratio = int(rng.choice([1, 4, 128])) if scenario >= 2 else 1
        topk = int(rng.choice([1, 256, 512, 2048])) if scenario == 3 else 0
        cores = int(rng.choice([1, 3, 64, 256, 512]))
        cases.append(dict(act_q=act_q, act_kv=act_kv, num_heads=heads, ori_win_left=win,
                          scenario=scenario, cmp_ratio=ratio, cmp_topk=topk, core_num=cores))
    return cases


@requires_gpu
def test_device_schedule_equals_host_schedule_word_for_word():
    cases = _random_cases(n=int(os.environ.get("SAS_SCHED_CASES", "60")))  # more for a longer run
    for i, c in enumerate(cases):
        _say(f"case {i}: batch={len(c['act_q'])} heads={c['num_heads']} "
             f"scenario={c['scenario']} cores={c['core_num']}")
        host = build_metadata(**c)
        b = len(c["act_q"])
        aq = torch.tensor(c["act_q"], dtype=torch.int32, device="cuda")
        ak = torch.tensor(c["act_kv"], dtype=torch.int32, device="cuda")
        args = {k: v for k, v in c.items() if k not in ("act_q", "act_kv")}
        dev = build_metadata_device(batch=b, act_q=aq, act_kv=ak, **args)
        assert torch.equal(dev.cpu(), host), f"case {i} differs: {c}"
        if b and len(set(c["act_q"])) == 1:  # the uniform-rows form
            dev_u = build_metadata_device(batch=b, act_q=None, uniform_q=c["act_q"][0],
                                          act_kv=ak, **args)
            assert torch.equal(dev_u.cpu(), host), f"case {i} (uniform) differs"


@requires_gpu
def test_metadata_api_on_device_equals_host():
    _say("sparse_attn_sharedkv_metadata on the device")
    g = torch.Generator().manual_seed(3)
    cu = torch.tensor([0, 3, 3, 10, 11], dtype=torch.int32)
    skv = torch.randint(20, 9000, (4,), generator=g, dtype=torch.int32)
    common = dict(num_heads_q=64, num_heads_kv=1, head_dim=576, cmp_topk=512, cmp_ratio=4,
                  ori_win_left=127, layout_q="TND", batch_size=4)
    host = sparse_attn_sharedkv_metadata(cu_seqlens_q=cu, seqused_kv=skv, **common)
    dev = sparse_attn_sharedkv_metadata(cu_seqlens_q=cu.cuda(), seqused_kv=skv.cuda(),
                                        device="cuda", **common)
    assert dev.is_cuda and torch.equal(dev.cpu(), host)


def _run(fn, kw, **extra):
    out, lse = fn(**kw, return_softmax_lse=True, **extra)
    torch.cuda.synchronize()
    return out, lse


@requires_gpu
@pytest.mark.parametrize("name,batch", [
    ("swa_decode_b32_h64", 6),
    ("swa_topk_decode_b32_h64_k512", 3),
    ("mla_decode_b64_h128_k2048", 3),
    ("mla_mtp_decode_b64_h128_k2048", 2),
    ("mla_fp8_decode_t128_h128_k2048", 4),
])
def test_attention_from_device_schedule_is_bitwise_the_host_one(name, batch):
    _say(f"device vs host schedule {name} batch={batch}")
    kw = gen.build_workload(name, device="cuda", seed=11, batch=batch)
    o_h, l_h = _run(sparse_flash_mla, kw, schedule="host")
    o_d, l_d = _run(sparse_flash_mla, kw, schedule="device")
    assert torch.equal(o_d, o_h) and torch.equal(l_d, l_h)
    for cores in (7, 512):  # split-KV and many-piece schedules
        o_h, l_h = _run(sparse_flash_mla, kw, schedule="host", core_num=cores)
        o_d, l_d = _run(sparse_flash_mla, kw, schedule="device", core_num=cores)
        assert torch.equal(o_d, o_h) and torch.equal(l_d, l_h), f"core_num={cores}"


@requires_gpu
@pytest.mark.parametrize("name,extra,batch", [
    ("mla_decode_b64_h128_k2048", {}, 128),
    ("mla_decode_b64_h128_k2048", {}, 72),  # native rows: 128-head items from 65 on
    ("mla_fp8_decode_t128_h128_k2048", {}, 128),
    ("mla_fp8_decode_t128_h128_k2048", {"fp8_qk": True}, 128),
    ("mla_fp8_decode_t128_h128_k2048", {}, 32),  # fp8 rows: 128-head items from 32 on
    ("mla_fp8_decode_t128_h128_k2048", {"fp8_qk": True}, 48),
])
def test_128_head_items_from_device_schedule(name, extra, batch):
    # items of all 128 heads on the 128-head kernel (native rows from 65
    # sequences, fp8 rows and the fp8 Q·Kᵀ form from 32), whole, in two pieces
    # (merged in-kernel) and in many pieces (merge kernel)
    _say(f"device vs host schedule {name} {extra}, {batch} sequences")
    kw = gen.build_workload(name, device="cuda", seed=13, batch=batch,
                            ctx_override=[4096] * batch)
    prep = api.prepare(**kw, **extra)
    assert prep.args.m_base == 128, prep.args.m_base
    for cores in (256, 128, 512):
        o_h, l_h = _run(sparse_flash_mla, kw, schedule="host", core_num=cores, **extra)
        o_d, l_d = _run(sparse_flash_mla, kw, schedule="device", core_num=cores, **extra)
        assert torch.equal(o_d, o_h) and torch.equal(l_d, l_h), f"core_num={cores}"


@requires_gpu
@pytest.mark.parametrize("name", ["scfa_prefill_b2", "cfa_prefill_b2"])
def test_ragged_tnd_from_device_schedule(name):
    # TND with ragged cu_seqlens_q: lengths and prefixes derived on the GPU
    _say(f"ragged TND device schedule {name}")
    kw = {k: (v.cuda() if isinstance(v, torch.Tensor) else v)
          for k, v in gen.build_case(gen.FAST_CASES[name], torch.bfloat16).items()}
    o_h, l_h = _run(sparse_attn_sharedkv, kw, schedule="host")
    o_d, l_d = _run(sparse_attn_sharedkv, kw, schedule="device")
    assert torch.equal(o_d, o_h) and torch.equal(l_d, l_h)


@requires_gpu
def test_whole_call_in_one_graph_with_new_lengths_each_replay():
    _say("graph capture of scheduler + attention + merge")
    kw = gen.build_workload("mla_decode_b64_h128_k2048", device="cuda", seed=5, batch=4)
    base = kw["seqused_kv"].clone()
    lengths = [base,
               torch.tensor([1500, 32768, 700, 2300], dtype=torch.int32, device="cuda"),
               torch.tensor([32768, 64, 32768, 5000], dtype=torch.int32, device="cuda"),
               base]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up off the capture
        sparse_flash_mla(**kw, schedule="device", return_softmax_lse=True)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out, lse = sparse_flash_mla(**kw, schedule="device", return_softmax_lse=True)
    for r, lens in enumerate(lengths):
        kw["seqused_kv"].copy_(lens)
        graph.replay()
        torch.cuda.synchronize()
        got_o, got_l = out.clone(), lse.clone()
        ref_o, ref_l = _run(sparse_flash_mla, dict(kw, seqused_kv=lens.clone()), schedule="host")
        assert torch.equal(got_o, ref_o) and torch.equal(got_l, ref_l), f"replay {r}"
        assert torch.isfinite(got_o.float()).all()


@requires_gpu
def test_two_graphs_replayed_alternately():
    # two calls captured into two graphs (the same capture stream), each with its
    # own schedule and arrival-counter buffers, replayed in alternation with new
    # lengths; every replay bitwise the eager host-scheduled call
    _say("two captured graphs replayed alternately")
    kws = [gen.build_workload("mla_decode_b64_h128_k2048", device="cuda", seed=11, batch=64),
           gen.build_workload("swa_topk_decode_b32_h64_k512", device="cuda", seed=12, batch=5)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up off the capture
        for kw in kws:
            sparse_flash_mla(**kw, schedule="device", return_softmax_lse=True)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graphs, outs = [], []
    for kw in kws:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs.append(sparse_flash_mla(**kw, schedule="device", return_softmax_lse=True))
        graphs.append(g)
    base = [kw["seqused_kv"].clone() for kw in kws]
    rng = np.random.default_rng(3)
    for r in range(6):
        i = r % 2
        kw = kws[i]
        lens = base[i] if r < 2 else torch.tensor(
            rng.integers(2100, int(base[i].max()) + 1, size=base[i].numel()),
            dtype=torch.int32, device="cuda")
        kw["seqused_kv"].copy_(lens)
        graphs[i].replay()
        torch.cuda.synchronize()
        got_o, got_l = outs[i][0].clone(), outs[i][1].clone()
        ref_o, ref_l = _run(sparse_flash_mla, dict(kw, seqused_kv=lens.clone()), schedule="host")
        assert torch.equal(got_o, ref_o) and torch.equal(got_l, ref_l), f"replay {r} (graph {i})"
        assert torch.isfinite(got_o.float()).all()


@requires_gpu
def test_unusable_device_schedule_gives_nan():
    _say("schedule for another head count / negative length -> NaN")
    kw = gen.build_workload("swa_decode_b32_h64", device="cuda", seed=2, batch=3)
    b = kw["q"].shape[0]
    wrong = build_metadata(act_q=[1] * b, act_kv=kw["seqused_kv"].cpu().tolist(), num_heads=128,
                           ori_win_left=127, scenario=1, cmp_ratio=1, cmp_topk=0).cuda()
    out, lse = _run(sparse_attn_sharedkv, kw, metadata=wrong)
    assert torch.isnan(out.float()).all() and torch.isnan(lse).all()
    neg = dict(kw, seqused_kv=torch.tensor([100, -1, 50], dtype=torch.int32, device="cuda"))
    out, lse = _run(sparse_flash_mla, neg, schedule="device")
    assert torch.isnan(out.float()).all() and torch.isnan(lse).all()
