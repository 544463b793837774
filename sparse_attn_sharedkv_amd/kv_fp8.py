"""fp8 KV cache rows (``kv_cache_dtype="fp8_ds_mla"``) and their writer.

The reference stores its caches in bf16/fp16 only (api.py:51-56). This
module adds the 656-byte row format that long-context MLA decode uses for
d_qk = 576 = 512 latent dims + 64 rope dims:

* bytes ``[0, 512)``: the latent dims as OCP fp8 e4m3 (``torch.float8_e4m3fn``)
* bytes ``[512, 528)``: four fp32 scales, scale ``t`` for dims ``128t..128t+127``
* bytes ``[528, 656)``: the rope dims as bf16

The attention kernels read latent dim ``d`` as
``bf16(fp32(e4m3[d]) * scale[d // 128])`` and then compute exactly as on a
bf16 cache. The writer quantizes each 128-dim block with
``scale = amax / 448`` (1 for an all-zero block) and
``e4m3 = rne(clamp(x / scale, -448, 448))``; both run in the HIP library
(``sas_kv_fp8_append``).
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib

ROW_BYTES = _lib.FP8_ROW_BYTES
HEAD_DIM = 576


def append_kv_fp8(cache: torch.Tensor, kv: torch.Tensor, slot_mapping: torch.Tensor,
                  stream: Optional[torch.cuda.Stream] = None) -> None:
    """Quantize ``kv`` rows into ``cache`` at ``slot_mapping`` (in place, asynchronous).

    ``cache``: ``[blocks, block_size, 1, 656]`` (or any shape whose last dim is 656)
    uint8 / float8_e4m3fn on the GPU. ``kv``: ``[n, 576]`` (or ``[n, 1, 576]``) bf16.
    ``slot_mapping``: ``[n]`` int, flat row index ``block * block_size + offset``;
    negative entries and entries past the pool are skipped.
    """
    if cache.dtype not in (torch.uint8, torch.float8_e4m3fn) or cache.shape[-1] != ROW_BYTES:
        raise ValueError(f"cache must be uint8/float8_e4m3fn with last dim {ROW_BYTES}")
    if not cache.is_contiguous():
        raise ValueError("cache must be contiguous (it is written in place)")
    if kv.dtype != torch.bfloat16 or kv.shape[-1] != HEAD_DIM:
        raise ValueError(f"kv must be bf16 with last dim {HEAD_DIM}")
    if cache.device.type != "cuda" or kv.device != cache.device:
        raise RuntimeError("append_kv_fp8 runs on a ROCm GPU; cache and kv must share it")
    rows = kv.reshape(-1, HEAD_DIM).contiguous()
    slots = slot_mapping.to(device=cache.device, dtype=torch.int32).reshape(-1).contiguous()
    if slots.numel() != rows.shape[0]:
        raise ValueError("slot_mapping must have one entry per kv row")
    lib = _lib.load()
    st = stream if stream is not None else torch.cuda.current_stream(cache.device)
    rc = lib.sas_kv_fp8_append(ctypes.c_void_p(rows.data_ptr()), ctypes.c_void_p(slots.data_ptr()),
                               ctypes.c_void_p(cache.data_ptr()), int(rows.shape[0]),
                               int(cache.numel() // ROW_BYTES), ctypes.c_void_p(st.cuda_stream))
    if rc != _lib.SAS_OK:
        raise RuntimeError(_lib.last_error())
    # the kernel reads rows / slots asynchronously: keep them alive until it has run
    rows.record_stream(st)
    slots.record_stream(st)


def quantize_kv_fp8(kv: torch.Tensor) -> torch.Tensor:
    """Quantize ``[n, 576]`` bf16 rows into a new ``[n, 656]`` uint8 tensor."""
    rows = kv.reshape(-1, HEAD_DIM)
    out = torch.zeros((rows.shape[0], ROW_BYTES), dtype=torch.uint8, device=kv.device)
    slots = torch.arange(rows.shape[0], dtype=torch.int32, device=kv.device)
    append_kv_fp8(out, rows, slots)
    return out
