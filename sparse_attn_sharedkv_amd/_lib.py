"""ctypes binding of ``libsas_mi355x.so`` (declared in ``include/sas_mi355x.h``).

The library is the only compute path: if it is missing, every entry point
raises instead of computing anything another way.
"""

from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_lib", "libsas_mi355x.so")

# metadata layout (mirrors the SAS_* macros of the C header)
AIC_CORE_NUM = 512
AIV_CORE_NUM = 1024
FA_METADATA_SIZE = 8
FD_METADATA_SIZE = 8
FD_OFFSET = AIC_CORE_NUM * FA_METADATA_SIZE
SAS_META_SIZE = 16384
CFG_OFFSET = SAS_META_SIZE - 8
META_MAGIC = 0x5A53A355

SAS_OK = 0
SAS_E_INVALID = -1
SAS_E_UNSUPPORTED = -2
SAS_E_CAPACITY = -3
SAS_E_HIP = -4
DTYPE_BF16 = 0
DTYPE_FP16 = 1
KV_NATIVE = 0
KV_FP8_DS_MLA = 1
FP8_ROW_BYTES = 656
SAS_PHASE_PIPELINED = 4        # SasAttnArgs.phases bit: native rows through the pipelined kernel
SAS_PHASE_FP8_QK = 8           # SasAttnArgs.phases bit: fp8 rows, Q·Kᵀ on fp8 MFMA (e4m3 queries)
SAS_PHASE_ROW_ITEMS = 16       # SasAttnArgs.phases bit: no row pairs (one query row per item)
SCHED_DEVICE = -1             # SasAttnArgs.num_fd: schedule summary read on the device
MERGE_SYNC_WORDS = 2 * AIC_CORE_NUM  # SasAttnArgs.merge_sync: uint64 arrival counters
DEV_SCHED_MAX_BATCH = 4096
DEV_SCHED_MAX_ITEMS = 16384


class SasAttnArgs(ctypes.Structure):
    """Field-for-field mirror of ``SasAttnArgs`` in ``include/sas_mi355x.h``."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("ori_kv", ctypes.c_void_p),
        ("ori_block_table", ctypes.c_void_p),
        ("cmp_kv", ctypes.c_void_p),
        ("cmp_block_table", ctypes.c_void_p),
        ("cmp_indices", ctypes.c_void_p),
        ("q_prefix", ctypes.c_void_p),
        ("act_q_lens", ctypes.c_void_p),
        ("seqused_kv", ctypes.c_void_p),
        ("sinks", ctypes.c_void_p),
        ("metadata", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("total_tokens", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("head_dim_v", ctypes.c_int32),
        ("ori_block_num", ctypes.c_int32),
        ("ori_block_size", ctypes.c_int32),
        ("ori_table_len", ctypes.c_int32),
        ("cmp_block_num", ctypes.c_int32),
        ("cmp_block_size", ctypes.c_int32),
        ("cmp_table_len", ctypes.c_int32),
        ("topk", ctypes.c_int32),
        ("scenario", ctypes.c_int32),
        ("cmp_ratio", ctypes.c_int32),
        ("ori_win_left", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("num_fa", ctypes.c_int32),
        ("num_fd", ctypes.c_int32),
        ("num_partial_slots", ctypes.c_int32),
        ("s2_base", ctypes.c_int32),
        ("m_base", ctypes.c_int32),
        ("phases", ctypes.c_int32),
        ("kv_format", ctypes.c_int32),
        ("merge_sync", ctypes.c_void_p),
    ]


EXPORTS = ("sas_metadata_build", "sas_metadata_build_device", "sas_workspace_bytes",
           "sas_attention_launch", "sas_attention_launch_noalloc", "sas_kv_fp8_append",
           "sas_version", "sas_args_struct_size", "sas_last_error")
NOALLOC_SCRATCH_BYTES = 72 << 20  # SAS_NOALLOC_SCRATCH_BYTES

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load the library once; raises RuntimeError when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m sparse_attn_sharedkv_amd.build` "
                "(hipcc, gfx950). There is no fallback compute path.")
        lib = ctypes.CDLL(LIB_PATH)
        i32p = ctypes.POINTER(ctypes.c_int32)
        lib.sas_metadata_build.restype = ctypes.c_int
        lib.sas_metadata_build.argtypes = [i32p, ctypes.c_int, i32p, i32p] + [ctypes.c_int] * 10
        lib.sas_metadata_build_device.restype = ctypes.c_int
        lib.sas_metadata_build_device.argtypes = ([ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                                   ctypes.c_int, ctypes.c_void_p] +
                                                  [ctypes.c_int] * 11 + [ctypes.c_void_p])
        lib.sas_workspace_bytes.restype = ctypes.c_int64
        lib.sas_workspace_bytes.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.sas_attention_launch.restype = ctypes.c_int
        lib.sas_attention_launch.argtypes = [ctypes.POINTER(SasAttnArgs), ctypes.c_void_p]
        lib.sas_attention_launch_noalloc.restype = ctypes.c_int
        lib.sas_attention_launch_noalloc.argtypes = [ctypes.POINTER(SasAttnArgs), ctypes.c_void_p]
        lib.sas_kv_fp8_append.restype = ctypes.c_int
        lib.sas_kv_fp8_append.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                          ctypes.c_int, ctypes.c_int64, ctypes.c_void_p]
        lib.sas_version.restype = ctypes.c_int
        lib.sas_args_struct_size.restype = ctypes.c_int
        lib.sas_last_error.restype = ctypes.c_char_p
        if lib.sas_args_struct_size() != ctypes.sizeof(SasAttnArgs):
            raise RuntimeError("SasAttnArgs layout mismatch between the library and its binding")
        _lib = lib
    return _lib


def last_error() -> str:
    return load().sas_last_error().decode("utf-8", "replace")
