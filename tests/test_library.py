"""The C-ABI library loads on a CPU-only host and exports what the header declares.

No compute calls are made here (there is no GPU); host-side entry points
(the scheduler, the workspace size, the argument-struct layout) are called.
"""

import ctypes
import os
import re

import pytest
import torch

from sparse_attn_sharedkv_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sas_mi355x.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sas_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared_functions()
    assert names, "no declarations parsed"
    for n in names:
        assert hasattr(lib, n), f"{n} declared in sas_mi355x.h but not exported"
    assert set(names) == set(_lib.EXPORTS)


def test_struct_layout_matches_binding():
    lib = _lib.load()
    assert lib.sas_args_struct_size() == ctypes.sizeof(_lib.SasAttnArgs)
    assert lib.sas_version() >= 100


def test_header_constants_match_binding():
    text = open(HEADER).read()
    consts = dict(re.findall(r"#define (SAS_[A-Z0-9_]+) (\S+)", text))
    assert int(consts["SAS_AIC_CORE_NUM"]) == _lib.AIC_CORE_NUM
    assert int(consts["SAS_AIV_CORE_NUM"]) == _lib.AIV_CORE_NUM
    assert int(consts["SAS_META_SIZE"]) == _lib.SAS_META_SIZE
    assert int(consts["SAS_META_MAGIC"], 16) == _lib.META_MAGIC
    assert int(consts["SAS_KV_NATIVE"]) == _lib.KV_NATIVE
    assert int(consts["SAS_KV_FP8_DS_MLA"]) == _lib.KV_FP8_DS_MLA
    assert int(consts["SAS_FP8_ROW_BYTES"]) == _lib.FP8_ROW_BYTES == 512 + 16 + 128
    assert int(consts["SAS_PHASE_PIPELINED"]) == _lib.SAS_PHASE_PIPELINED
    assert int(consts["SAS_PHASE_FP8_QK"]) == _lib.SAS_PHASE_FP8_QK
    assert int(consts["SAS_SCHED_DEVICE"].strip("()")) == _lib.SCHED_DEVICE
    assert int(consts["SAS_DEV_SCHED_MAX_BATCH"]) == _lib.DEV_SCHED_MAX_BATCH
    assert int(consts["SAS_DEV_SCHED_MAX_ITEMS"]) == _lib.DEV_SCHED_MAX_ITEMS


def test_fp8_writer_rejects_bad_arguments_without_a_gpu():
    lib = _lib.load()
    assert lib.sas_kv_fp8_append(None, None, None, 4, 16, None) == -1
    assert lib.sas_kv_fp8_append(None, None, None, -1, 16, None) == -1
    assert lib.sas_kv_fp8_append(None, None, None, 0, 16, None) == 0   # nothing to do


def test_device_scheduler_rejects_bad_arguments_without_a_gpu():
    # host-checkable arguments are validated before any HIP call
    lib = _lib.load()
    good = dict(num_heads=64, m_base=64, win=127, scenario=1, ratio=1, topk=0, cores=256,
                s2=64, split=2, chunk=32)

    def call(meta=1, batch=1, act_q=None, uniform_q=1, act_kv=1, **kw):
        a = dict(good, **kw)
        return lib.sas_metadata_build_device(meta, batch, act_q, uniform_q, act_kv,
                                             a["num_heads"], a["m_base"], a["win"], a["scenario"],
                                             a["ratio"], a["topk"], a["cores"], a["s2"], a["split"],
                                             a["chunk"], 0, None)

    assert call(meta=None) == -1
    assert call(batch=_lib.DEV_SCHED_MAX_BATCH + 1) == -1
    assert call(act_kv=None) == -1
    assert call(uniform_q=-1) == -1
    assert call(cores=_lib.AIC_CORE_NUM + 1) == -1
    assert call(s2=48) == -1
    assert call(scenario=2, ratio=0) == -1
    assert "sas_metadata_build_device" in _lib.last_error()


def test_workspace_bytes():
    lib = _lib.load()
    # fp16 partials, fp32 lse and fp32 inverse scales per (slot, head)
    assert lib.sas_workspace_bytes(256, 64, 512) == 256 * 64 * (512 * 2 + 4 + 4)
    assert lib.sas_workspace_bytes(-1, 64, 512) == 0


def test_launch_rejects_bad_arguments_without_a_gpu():
    # argument validation runs before any HIP call
    lib = _lib.load()
    a = _lib.SasAttnArgs()
    assert lib.sas_attention_launch(None, None) == -1
    assert lib.sas_attention_launch(ctypes.byref(a), None) == -1
    assert "null" in _lib.last_error()
