"""Split-KV scheduler: ``sparse_attn_sharedkv_metadata`` (signature of metadata.py:1018-1045).

The reference ports the AICPU ``SparseAttnSharedkvMetadata`` scheduler to
Python and its kernel ignores the result (kernel.py:367, "unused, v1"). Here
the scheduler is C++ inside ``libsas_mi355x.so`` (``sas_metadata_build``) and
the attention kernel is driven by it: one FA row per workgroup, FD rows for
the split-KV merges. Row schemas keep metadata.py's field order
(:45-60); capacities are sized for MI355X (256 CUs, up to 512 workgroups).
"""

from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence

import torch

from . import _lib
from ._lib import (AIC_CORE_NUM, AIV_CORE_NUM, CFG_OFFSET, FA_METADATA_SIZE,  # noqa: F401
                   FD_METADATA_SIZE, FD_OFFSET, META_MAGIC, SAS_META_SIZE)

# Field indices (metadata.py:45-60)
FA_CORE_ENABLE_INDEX = 0
FA_BN2_START_INDEX = 1
FA_M_START_INDEX = 2
FA_S2_START_INDEX = 3
FA_BN2_END_INDEX = 4
FA_M_END_INDEX = 5
FA_S2_END_INDEX = 6
FA_FIRST_FD_DATA_WORKSPACE_IDX_INDEX = 7

FD_CORE_ENABLE_INDEX = 0
FD_BN2_IDX_INDEX = 1
FD_M_IDX_INDEX = 2
FD_WORKSPACE_IDX_INDEX = 3
FD_WORKSPACE_NUM_INDEX = 4
FD_M_START_INDEX = 5
FD_M_NUM_INDEX = 6

# MI355X: 256 compute units; one attention workgroup per CU.
DEFAULT_CORE_NUM = 256
DEFAULT_S2_BASE = 64          # positions per schedulable block
DEFAULT_MIN_SPLIT_BLOCKS = 2  # never split an item into pieces shorter than 128 positions
DEFAULT_FD_HEAD_CHUNK = 64    # heads per merge task (a whole 64-head item)


# Above 64 heads, native rows take items of every head of a token (128) from this
# many sequences on. Up to 64 sequences 64-head items fill the 256 workgroups in at
# most two pieces per item, merged inside the attention kernel; from 65 on they
# need three, and 128-head items are ahead (measured on MI355X, top-k 2048 decode,
# H = 128, us per call with 64- / 128-head items: 32 sequences 42.7 / 48.4, 64
# sequences 65.1 / 66.8, 65 sequences 88.2 / 72.2, 96 sequences 112.9 / 93.0,
# 112 sequences 104.7 / 98.2).
WIDE_ITEM_MIN_BATCH = 65
# fp8 rows take 128-head items from this many sequences on: their 64-head items
# run on the pipelined kernel, which the 128-head kernel beats from 32 sequences
# (measured on MI355X, top-k 2048 decode, H = 128, bf16 / fp8 Q·Kᵀ form: 32
# sequences 49.6 / 51.2 us per call against 50.8 / 59.7; 64 sequences 71.3 /
# 72.2 against 79.8 / 91.6; at 16 sequences 40.6 / 42.3 against 36.2 / 43.6).
WIDE_ITEM_MIN_BATCH_FP8 = 32


def m_base_for(num_heads: int, item64: bool = False, batch: Optional[int] = None,
               fp8_rows: bool = False, rows: Optional[int] = None) -> int:
    """Heads per schedulable item (the reference's mBaseSize, metadata.py:388).

    32 up to 32 heads and 64 up to 64 heads, as the reference. Above 64 heads an
    item holds all of a token's heads (128) when the call has at least
    ``WIDE_ITEM_MIN_BATCH`` sequences (``batch``), or ``WIDE_ITEM_MIN_BATCH_FP8``
    on fp8 cache rows (``fp8_rows``; either Q·Kᵀ form): the 128-head kernel then
    serves every head of the token from one gathered tile; else 64. ``item64``
    (the pipelined kernel on native rows) keeps 64.

    ``rows`` (the call's query rows) replaces the sequence count where the caller
    builds the schedule for its own launch (a call without ``metadata``): calls of
    several rows per sequence then take 128-head items too (MTP, 128-head
    prefill). Schedules handed from one entry point to another count sequences,
    the one value every entry point and both schedulers know alike (a schedule
    built on the GPU from a ragged TND call holds its row count only there)."""
    if num_heads <= 32:
        return 32
    need = WIDE_ITEM_MIN_BATCH_FP8 if fp8_rows else WIDE_ITEM_MIN_BATCH
    n = rows if rows is not None else batch
    if num_heads <= 64 or item64 or n is None or n < need:
        return 64
    return 128


def m_base_valid(num_heads: int, item64: bool, m_base: int) -> bool:
    """Item sizes the kernels accept for a head count and kernel form."""
    if num_heads <= 32:
        return m_base == 32
    if num_heads <= 64 or item64:
        return m_base == 64
    return m_base in (64, 128)


def _is_fp8(kv_cache_dtype) -> bool:
    if kv_cache_dtype in (None, "auto"):
        return False
    if kv_cache_dtype == "fp8_ds_mla":
        return True
    raise ValueError(f"unsupported kv_cache_dtype {kv_cache_dtype!r} (None, 'auto' or 'fp8_ds_mla')")


def _as_list(t) -> List[int]:
    if t is None:
        return []
    if isinstance(t, torch.Tensor):
        return [int(x) for x in t.detach().cpu().to(torch.int64).tolist()]
    return [int(x) for x in t]


def resolve_lengths(*, layout_q: str, layout_kv: str, cu_seqlens_q=None, cu_seqlens_ori_kv=None,
                    seqused_q=None, seqused_kv=None, batch_size: int = 0, max_seqlen_q: int = 0,
                    max_seqlen_kv: int = 0):
    """Per-batch (act_q, act_kv) the way metadata.py:345-407 derives them."""
    cu_q, cu_kv = _as_list(cu_seqlens_q), _as_list(cu_seqlens_ori_kv)
    sq, skv = _as_list(seqused_q), _as_list(seqused_kv)
    if sq:
        batch = len(sq)
    elif layout_q == "TND" and cu_q:
        batch = len(cu_q) - 1
    else:
        batch = int(batch_size)
    act_q, act_kv = [], []
    for b in range(batch):
        if sq:
            act_q.append(sq[b])
        elif layout_q == "TND" and cu_q:
            act_q.append(cu_q[b + 1] - cu_q[b])
        else:
            act_q.append(int(max_seqlen_q))
        if skv:
            act_kv.append(skv[b])
        elif layout_kv == "TND" and cu_kv:
            act_kv.append(cu_kv[b + 1] - cu_kv[b])
        else:
            act_kv.append(int(max_seqlen_kv))
    return act_q, act_kv


def build_metadata(*, act_q: Sequence[int], act_kv: Sequence[int], num_heads: int,
                   ori_win_left: int, scenario: int, cmp_ratio: int, cmp_topk: int,
                   core_num: int = DEFAULT_CORE_NUM, s2_base: int = DEFAULT_S2_BASE,
                   min_split_blocks: int = DEFAULT_MIN_SPLIT_BLOCKS,
                   fd_head_chunk: int = DEFAULT_FD_HEAD_CHUNK, item64: bool = False,
                   m_base: Optional[int] = None, fp8_rows: bool = False) -> torch.Tensor:
    """Run the C++ scheduler; returns an int32 CPU tensor of ``SAS_META_SIZE`` words.
    ``item64``: the schedule is for a kernel form of 64-head items at most (the
    pipelined kernel; ``m_base_for``); ``m_base``: the item size
    (default ``m_base_for``, with ``fp8_rows`` for calls on fp8 cache rows)."""
    lib = _lib.load()
    b = len(act_q)
    if m_base is None:
        m_base = m_base_for(int(num_heads), item64, b, fp8_rows)
    out = torch.zeros(SAS_META_SIZE, dtype=torch.int32)
    aq = (ctypes.c_int32 * max(b, 1))(*[int(x) for x in act_q])
    ak = (ctypes.c_int32 * max(b, 1))(*[int(x) for x in act_kv])
    i32p = ctypes.POINTER(ctypes.c_int32)
    rc = lib.sas_metadata_build(ctypes.cast(out.data_ptr(), i32p), b, aq, ak, int(num_heads),
                                int(m_base), int(ori_win_left), int(scenario),
                                int(cmp_ratio), int(cmp_topk), int(core_num), int(s2_base),
                                int(min_split_blocks), int(fd_head_chunk))
    if rc < 0:
        raise ValueError(_lib.last_error())
    return out


def device_lengths(*, layout_q: str, layout_kv: str, device, cu_seqlens_q=None,
                   cu_seqlens_ori_kv=None, seqused_q=None, seqused_kv=None, batch_size: int = 0,
                   max_seqlen_q: int = 0, max_seqlen_kv: int = 0):
    """``resolve_lengths`` on the GPU: ``(batch, act_q, uniform_q, act_kv)`` with int32
    device tensors (``act_q`` is None when every batch has ``uniform_q`` rows). Only
    tensor shapes are read on the host."""
    i32 = torch.int32

    def dev(t):
        return torch.as_tensor(t).to(device=device, dtype=i32).reshape(-1)

    def nonempty(t):
        return t is not None and torch.as_tensor(t).numel() > 0

    if nonempty(seqused_q):
        batch = torch.as_tensor(seqused_q).numel()
    elif layout_q == "TND" and nonempty(cu_seqlens_q):
        batch = torch.as_tensor(cu_seqlens_q).numel() - 1
    else:
        batch = int(batch_size)
    act_q, uniform_q = None, 0
    if nonempty(seqused_q):
        act_q = dev(seqused_q)[:batch].contiguous()
    elif layout_q == "TND" and nonempty(cu_seqlens_q):
        c = dev(cu_seqlens_q)
        act_q = (c[1:batch + 1] - c[:batch]).contiguous()
    else:
        uniform_q = int(max_seqlen_q)
    if nonempty(seqused_kv):
        act_kv = dev(seqused_kv)[:batch].contiguous()
    elif layout_kv == "TND" and nonempty(cu_seqlens_ori_kv):
        c = dev(cu_seqlens_ori_kv)
        act_kv = (c[1:batch + 1] - c[:batch]).contiguous()
    else:
        act_kv = torch.full((batch,), int(max_seqlen_kv), dtype=i32, device=device)
    return batch, act_q, uniform_q, act_kv


def build_metadata_device(*, batch: int, act_q: Optional[torch.Tensor], act_kv: torch.Tensor,
                          num_heads: int, ori_win_left: int, scenario: int, cmp_ratio: int,
                          cmp_topk: int, uniform_q: int = 0, core_num: int = DEFAULT_CORE_NUM,
                          s2_base: int = DEFAULT_S2_BASE,
                          min_split_blocks: int = DEFAULT_MIN_SPLIT_BLOCKS,
                          fd_head_chunk: int = DEFAULT_FD_HEAD_CHUNK,
                          stream: Optional[torch.cuda.Stream] = None,
                          out: Optional[torch.Tensor] = None, item64: bool = False,
                          m_base: Optional[int] = None, fp8_rows: bool = False) -> torch.Tensor:
    """Run the on-device scheduler (``sas_metadata_build_device``) on the current stream.

    ``act_q`` / ``act_kv``: int32 ``[batch]`` tensors on the GPU (``act_q`` None: every
    batch has ``uniform_q`` query rows). Returns the int32 ``SAS_META_SIZE`` schedule on
    the same GPU, word for word what ``build_metadata`` returns for the same lengths;
    nothing is read back. Lengths the host cannot check (negative, too many items) leave
    a schedule the attention launch turns into NaN outputs.

    ``out``: a persistent int32 ``[SAS_META_SIZE]`` buffer owned by the caller, which
    nothing else writes between calls. The schedule is written there, and when the
    buffer already holds the schedule of these inputs it is kept (a few microseconds
    instead of a rebuild). Without ``out`` a new buffer is allocated and always built.
    """
    lib = _lib.load()
    dev = act_kv.device
    if dev.type != "cuda":
        raise ValueError("build_metadata_device needs the lengths on a GPU")
    if batch < 0 or batch > _lib.DEV_SCHED_MAX_BATCH:
        raise ValueError(f"batch must be in [0, {_lib.DEV_SCHED_MAX_BATCH}] (got {batch})")
    for t in (act_q, act_kv):
        if t is not None and (t.dtype != torch.int32 or t.device != dev or t.numel() < batch
                              or not t.is_contiguous()):
            raise ValueError("act_q / act_kv must be contiguous int32 [batch] tensors on one GPU")
    reuse = out is not None
    if out is None:
        out = torch.empty(SAS_META_SIZE, dtype=torch.int32, device=dev)
    elif (out.dtype != torch.int32 or out.device != dev or out.numel() != SAS_META_SIZE
          or not out.is_contiguous()):
        raise ValueError(f"out must be a contiguous int32 [{SAS_META_SIZE}] tensor on {dev}")
    st = stream if stream is not None else torch.cuda.current_stream(dev)
    if m_base is None:
        m_base = m_base_for(int(num_heads), item64, int(batch), fp8_rows)
    rc = lib.sas_metadata_build_device(
        ctypes.c_void_p(out.data_ptr()), int(batch),
        ctypes.c_void_p(act_q.data_ptr() if act_q is not None else 0), int(uniform_q),
        ctypes.c_void_p(act_kv.data_ptr()), int(num_heads), int(m_base),
        int(ori_win_left), int(scenario), int(cmp_ratio), int(cmp_topk), int(core_num),
        int(s2_base), int(min_split_blocks), int(fd_head_chunk), int(reuse),
        ctypes.c_void_p(st.cuda_stream))
    if rc < 0:
        raise ValueError(_lib.last_error())
    return out


def config_row(metadata: torch.Tensor) -> dict:
    """Decode the schedule summary row (host copy; syncs if ``metadata`` is on a GPU)."""
    cfg = metadata.reshape(-1)[CFG_OFFSET:CFG_OFFSET + 8].to("cpu").tolist()
    if cfg[0] != META_MAGIC:
        raise AssertionError("metadata was not produced by sparse_attn_sharedkv_metadata")
    return dict(s2_base=cfg[1], num_fa=cfg[2], num_fd=cfg[3], num_partial_slots=cfg[4],
                num_heads=cfg[5], m_base=cfg[6], total_items=cfg[7])


def sparse_attn_sharedkv_metadata(
    *,
    num_heads_q: int,
    num_heads_kv: int,
    head_dim: int,
    cu_seqlens_q: Optional[torch.Tensor] = None,
    cu_seqlens_ori_kv: Optional[torch.Tensor] = None,
    cu_seqlens_cmp_kv: Optional[torch.Tensor] = None,
    seqused_q: Optional[torch.Tensor] = None,
    seqused_kv: Optional[torch.Tensor] = None,
    batch_size: int = 0,
    max_seqlen_q: int = 0,
    max_seqlen_kv: int = 0,
    ori_topk: int = 0,
    cmp_topk: int = 0,
    cmp_ratio: int = -1,
    ori_mask_mode: int = 4,
    cmp_mask_mode: int = 3,
    ori_win_left: int = 127,
    ori_win_right: int = 0,
    layout_q: str = "BSND",
    layout_kv: str = "PA_ND",
    has_ori_kv: bool = True,
    has_cmp_kv: bool = True,
    aic_core_num: int = DEFAULT_CORE_NUM,
    aiv_core_num: int = 2 * DEFAULT_CORE_NUM,
    device: Optional[str] = None,
    kv_cache_dtype: Optional[str] = None,
    fp8_qk: bool = False,
) -> torch.Tensor:
    """Schedule for one ``sparse_attn_sharedkv`` call: int32 ``[SAS_META_SIZE]``.

    Scenario: ``has_cmp_kv`` with ``cmp_topk > 0`` is top-k compressed (SCFA),
    ``has_cmp_kv`` alone is dense compressed (CFA), otherwise sliding window
    (SWA) -- the same rule as metadata.py:382-386. ``ori_win_left = -1`` is
    an empty raw window (golden.py:128-131 semantics, used for pure top-k
    decode). ``aic_core_num`` is the number of workgroups to balance over.
    ``aiv_core_num``, ``head_dim`` and ``ori_topk`` are accepted for signature
    parity; merge tasks are bounded by ``AIV_CORE_NUM``. With ``device`` a GPU the
    schedule is built there by the on-device scheduler from the lengths moved to
    (or already on) that GPU, without reading them back; the words are the ones
    the host scheduler produces. ``kv_cache_dtype`` (no reference counterpart):
    ``"fp8_ds_mla"`` for calls on fp8 cache rows, and ``fp8_qk`` (no reference
    counterpart) for calls of the fp8 Q·Kᵀ form (checked against the row format;
    both Q·Kᵀ forms take the same item sizes).
    Items hold 32, 64 or 128 heads (``m_base_for``: 128 only above 64 heads with at
    least ``WIDE_ITEM_MIN_BATCH`` sequences, ``WIDE_ITEM_MIN_BATCH_FP8`` on fp8
    rows), so a schedule for fp8 rows must be built with ``kv_cache_dtype``.
    """
    del cu_seqlens_cmp_kv, head_dim, ori_topk, aiv_core_num
    if num_heads_kv != 1:
        raise ValueError(f"only num_heads_kv=1 (shared KV) is supported, got {num_heads_kv}")
    if ori_mask_mode != 4 or ori_win_right != 0:
        raise ValueError("only ori_mask_mode=4 with ori_win_right=0 is supported")
    if has_cmp_kv and cmp_mask_mode != 3:
        raise ValueError("only cmp_mask_mode=3 is supported")
    if not has_ori_kv:
        raise ValueError("has_ori_kv=False is not supported")
    if has_cmp_kv:
        scenario = 3 if cmp_topk > 0 else 2
        if cmp_ratio < 1:
            raise ValueError("cmp_ratio must be >= 1 when a compressed cache is present")
    else:
        scenario = 1
    core_num = min(int(aic_core_num), AIC_CORE_NUM)
    if fp8_qk and not _is_fp8(kv_cache_dtype):
        raise ValueError("fp8_qk needs kv_cache_dtype='fp8_ds_mla'")
    item64 = False  # (either Q·Kᵀ form of fp8 rows takes the same item sizes)
    fp8_rows = _is_fp8(kv_cache_dtype)
    if device is not None and torch.device(device).type == "cuda":
        # scheduled on that GPU from device-resident lengths: nothing is read back
        batch, act_q, uniform_q, act_kv = device_lengths(
            layout_q=layout_q, layout_kv=layout_kv, device=device, cu_seqlens_q=cu_seqlens_q,
            cu_seqlens_ori_kv=cu_seqlens_ori_kv, seqused_q=seqused_q, seqused_kv=seqused_kv,
            batch_size=batch_size, max_seqlen_q=max_seqlen_q, max_seqlen_kv=max_seqlen_kv)
        return build_metadata_device(batch=batch, act_q=act_q, uniform_q=uniform_q,
                                     act_kv=act_kv, num_heads=num_heads_q,
                                     ori_win_left=ori_win_left, scenario=scenario,
                                     cmp_ratio=max(int(cmp_ratio), 1), cmp_topk=int(cmp_topk),
                                     core_num=core_num, item64=item64, fp8_rows=fp8_rows)
    act_q, act_kv = resolve_lengths(layout_q=layout_q, layout_kv=layout_kv,
                                    cu_seqlens_q=cu_seqlens_q,
                                    cu_seqlens_ori_kv=cu_seqlens_ori_kv, seqused_q=seqused_q,
                                    seqused_kv=seqused_kv, batch_size=batch_size,
                                    max_seqlen_q=max_seqlen_q, max_seqlen_kv=max_seqlen_kv)
    md = build_metadata(act_q=act_q, act_kv=act_kv, num_heads=num_heads_q,
                        ori_win_left=ori_win_left, scenario=scenario,
                        cmp_ratio=max(int(cmp_ratio), 1), cmp_topk=int(cmp_topk),
                        core_num=core_num, item64=item64, fp8_rows=fp8_rows)
    return md.to(device) if device is not None else md
