"""The allocation-free entry point ``sas_attention_launch_noalloc`` on a GPU.

It runs the same kernels as ``sas_attention_launch`` with the split-KV partials
in the library's fixed per-device scratch array instead of the caller's
workspace. Checked through the C-ABI: bitwise-equal outputs to
``sas_attention_launch`` on two calls in a row (the second on a smaller
input, so the scratch array holds the first call's partials when it starts),
for host-built schedules with split items and for a device-built schedule,
with the merge kernel and with the merge inside the attention kernel (whose
arrival counters sit in the scratch array too); and a schedule whose partials
do not fit is refused before any launch.
"""

import ctypes
import sys

import pytest
import torch

from oracle import gen

pytestmark = pytest.mark.gpu

HAS_GPU = torch.cuda.is_available()
requires_gpu = pytest.mark.skipif(not HAS_GPU, reason="needs a ROCm GPU")

if HAS_GPU:
    from sparse_attn_sharedkv_amd import _lib, api


def _say(msg):
    print(f"[gpu-noalloc] {msg}", flush=True)
    sys.stdout.flush()


def _launch(entry, prep):
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    prep.args.phases = 0
    prep.out.fill_(float("nan"))
    prep.lse.fill_(float("nan"))
    rc = getattr(_lib.load(), entry)(ctypes.byref(prep.args), st)
    assert rc == _lib.SAS_OK, _lib.last_error()
    torch.cuda.synchronize()
    return prep.out.clone(), prep.lse.clone()


@requires_gpu
@pytest.mark.parametrize("name,batches,extra", [
    ("mla_decode_b64_h128_k2048", (8, 2), {"core_num": 256}),      # every item split in two
    ("swa_topk_decode_b32_h64_k512", (16, 3), {"core_num": 512}),  # items in several pieces
    ("mla_decode_b64_h128_k2048", (6, 1), {"schedule": "device"}),  # device-built schedule
])
def test_noalloc_matches_launch_two_calls(name, batches, extra):
    for batch in batches:  # the second call is smaller than the first
        _say(f"{name} batch={batch} {extra}")
        kw = gen.build_workload(name, device="cuda", seed=40 + batch, batch=batch)
        prep = api.prepare(**kw, **extra)
        assert prep.args.num_fd != 0, "the case must exercise the split-KV workspace"
        o_ref, l_ref = _launch("sas_attention_launch", prep)
        o, l = _launch("sas_attention_launch_noalloc", prep)
        assert torch.isfinite(o_ref.float()).all()
        assert torch.equal(o, o_ref) and torch.equal(l, l_ref)


@requires_gpu
def test_noalloc_merge_in_kernel_two_calls():
    # a non-null merge_sync selects the merge inside the attention kernel; the
    # allocation-free entry point keeps its arrival counters in the scratch array
    # (the caller's pointer is not used), zero at load and after every call
    for batch in (8, 2):
        _say(f"merge in kernel, batch={batch}")
        kw = gen.build_workload("mla_decode_b64_h128_k2048", device="cuda", seed=60 + batch,
                                batch=batch)
        prep = api.prepare(**kw, core_num=256, _m_base=128 if batch == 8 else 64)
        assert prep.args.num_fd != 0
        prep.args.merge_sync = None
        o_ref, l_ref = _launch("sas_attention_launch", prep)  # merge kernel
        prep.args.merge_sync = 8  # any non-null 8-byte-aligned value
        o, l = _launch("sas_attention_launch_noalloc", prep)
        assert torch.isfinite(o_ref.float()).all()
        assert torch.equal(o, o_ref) and torch.equal(l, l_ref)


@requires_gpu
def test_noalloc_refuses_a_workspace_beyond_the_scratch():
    kw = gen.build_workload("mla_decode_b64_h128_k2048", device="cuda", seed=3, batch=2)
    prep = api.prepare(**kw, core_num=256)
    a = _lib.SasAttnArgs.from_buffer_copy(prep.args)
    per_slot = _lib.load().sas_workspace_bytes(1, a.m_base, a.head_dim_v)
    a.num_partial_slots = _lib.NOALLOC_SCRATCH_BYTES // per_slot + 1
    rc = _lib.load().sas_attention_launch_noalloc(ctypes.byref(a), None)
    assert rc == _lib.SAS_E_CAPACITY
    assert "scratch" in _lib.last_error()
