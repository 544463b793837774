"""Synthetic benchmark workloads, generated directly on the GPU.

Shapes (BSND, block_size 64, q and KV ~ N(0, 1) * 0.5, softmax_scale = 1/sqrt(d_qk)):

* ``topk_decode_b2_h16_k256``        B=2, H=16, ctx 1024, top-k 256, no sink
* ``swa_decode_b32_h64``             B=32, H=64, ctx U[2048, 8192], window 128, sinks U(-1,1)
* ``swa_topk_decode_b32_h64_k512``   B=32, H=64, ctx 16384, window 128 + compressed
                                     (ratio 4) top-k 512, sinks U(-1,1)
* ``mla_decode_b64_h128_k2048``      DeepSeek-V3.2 sparse MLA decode: B=64, H=128,
                                     ctx 32768, top-k 2048, no sink
* ``mla_mtp_decode_b64_h128_k2048``  the same with two query rows per sequence (MTP)
* ``mla_fp8_decode_t128_h128_k2048`` long-context sparse MLA over an fp8 cache: TND,
                                     128 sequences of one query row, H=128, ctx
                                     U[32768, 131072], top-k 2048, no sink; KV rows
                                     N(0, 1) * 0.5 quantized into 656-byte fp8 rows
                                     (``kv_fp8``)

Prefill (the reference's own 8K test shapes, test_sparse_attn_sharedkv.py:81-220:
TND, one sequence of 8192 query rows over 8192 cached rows, H=64, d_qk = d_v =
512, block_size 128, window 128, sinks U(-1,1)):

* ``swa_prefill_t8192_h64``          sliding window only (scenario 1)
* ``cfa_prefill_t8192_h64``          window + every compressed row below the
                                     threshold, ratio 128 (scenario 2)
* ``scfa_prefill_t8192_h64``         window + top-512 of the compressed rows, ratio 4
                                     (scenario 3)

Decode workloads: d_qk = 576 (512 latent + 64 rope), d_v = 512. Pure top-k attention
is expressed through the reference API as a compressed cache equal to the raw
pool with cmp_ratio 1 and an empty raw window (ori_win_left = -1). Block
tables hand each sequence a random permutation slice of the pool; top-k rows
are ``randperm(thr)[:K]`` per query row, ``-1`` padded (the generators of the
reference's golden.py:315-473, on the device). One generator per tensor
(q 0, kv 1, tables 2, indices 3, lengths 4, sinks 5).
"""

from __future__ import annotations

import math
from typing import Dict, Optional, Sequence

import numpy as np
import torch

WORKLOADS: Dict[str, dict] = {
    "topk_decode_b2_h16_k256": dict(B=2, S=1, H=16, D=576, DV=512, ctx=(1024, 1024), K=256,
                                    window=-1, cmp_ratio=1, mode="topk", sinks="none"),
    "swa_decode_b32_h64": dict(B=32, S=1, H=64, D=576, DV=512, ctx=(2048, 8192), K=0,
                               window=127, cmp_ratio=None, mode="swa", sinks="uniform"),
    "swa_topk_decode_b32_h64_k512": dict(B=32, S=1, H=64, D=576, DV=512, ctx=(16384, 16384),
                                         K=512, window=127, cmp_ratio=4, mode="swa+topk",
                                         sinks="uniform"),
    "mla_decode_b64_h128_k2048": dict(B=64, S=1, H=128, D=576, DV=512, ctx=(32768, 32768),
                                      K=2048, window=-1, cmp_ratio=1, mode="topk", sinks="none"),
    "mla_mtp_decode_b64_h128_k2048": dict(B=64, S=2, H=128, D=576, DV=512, ctx=(32768, 32768),
                                          K=2048, window=-1, cmp_ratio=1, mode="topk",
                                          sinks="none"),
    "mla_fp8_decode_t128_h128_k2048": dict(B=128, S=1, H=128, D=576, DV=512,
                                           ctx=(32768, 131072), K=2048, window=-1, cmp_ratio=1,
                                           mode="topk", sinks="none", kv="fp8_ds_mla",
                                           layout="TND"),
    "swa_prefill_t8192_h64": dict(B=1, S=8192, H=64, D=512, DV=512, ctx=(8192, 8192), K=0,
                                  window=127, cmp_ratio=None, mode="swa", sinks="uniform",
                                  layout="TND", block=128, prefill=True),
    "cfa_prefill_t8192_h64": dict(B=1, S=8192, H=64, D=512, DV=512, ctx=(8192, 8192), K=0,
                                  window=127, cmp_ratio=128, mode="cfa", sinks="uniform",
                                  layout="TND", block=128, prefill=True),
    "scfa_prefill_t8192_h64": dict(B=1, S=8192, H=64, D=512, DV=512, ctx=(8192, 8192), K=512,
                                   window=127, cmp_ratio=4, mode="swa+topk", sinks="uniform",
                                   layout="TND", block=128, prefill=True),
}

FP8_POOL_CHUNK_ROWS = 1 << 20  # bf16 rows generated (then quantized) at a time


def _pool(lens, block_size, d, dtype, rng, gen, device):
    per_b = [math.ceil(x / block_size) for x in lens]
    nblk = max(sum(per_b), 1)
    phys = rng.permutation(nblk).astype(np.int32)
    table = np.full((len(lens), max(max(per_b), 1)), -1, dtype=np.int32)
    cur = 0
    for b, nb in enumerate(per_b):
        table[b, :nb] = phys[cur:cur + nb]
        cur += nb
    pool = (torch.randn((nblk, block_size, 1, d), generator=gen, device=device) * 0.5).to(dtype)
    return pool, torch.as_tensor(table, dtype=torch.int32, device=device)


def _pool_fp8(lens, block_size, rng, gen, device):
    """fp8 pool: rows N(0, 1) * 0.5 in bf16, quantized chunk by chunk with the writer."""
    from .kv_fp8 import ROW_BYTES, append_kv_fp8

    per_b = [math.ceil(x / block_size) for x in lens]
    nblk = max(sum(per_b), 1)
    phys = rng.permutation(nblk).astype(np.int32)
    table = np.full((len(lens), max(max(per_b), 1)), -1, dtype=np.int32)
    cur = 0
    for b, nb in enumerate(per_b):
        table[b, :nb] = phys[cur:cur + nb]
        cur += nb
    pool = torch.empty((nblk, block_size, 1, ROW_BYTES), dtype=torch.uint8, device=device)
    rows = nblk * block_size
    for r0 in range(0, rows, FP8_POOL_CHUNK_ROWS):
        n = min(FP8_POOL_CHUNK_ROWS, rows - r0)
        src = (torch.randn((n, 576), generator=gen, device=device) * 0.5).to(torch.bfloat16)
        slots = torch.arange(r0, r0 + n, dtype=torch.int32, device=device)
        append_kv_fp8(pool, src, slots)
    return pool, torch.as_tensor(table, dtype=torch.int32, device=device)


def _topk_rows(thresholds: torch.Tensor, k: int, gen: torch.Generator) -> torch.Tensor:
    """``[n, k]`` int32: row i holds a uniformly random k-subset of ``[0, thr_i)`` in
    random order (``randperm(thr_i)[:k]`` in distribution), ``-1`` padded; one
    batched sort instead of one permutation per row."""
    n = thresholds.numel()
    m = max(int(thresholds.max().item()) if n else 0, 1)
    keys = torch.rand((n, m), generator=gen, device=thresholds.device)
    col = torch.arange(m, device=thresholds.device)
    keys = torch.where(col[None, :] < thresholds[:, None], keys, torch.full_like(keys, 2.0))
    take = min(k, m)
    idx = keys.argsort(dim=1)[:, :take].to(torch.int32)
    valid = torch.arange(take, device=thresholds.device)[None, :] < thresholds[:, None].clamp(max=k)
    out = torch.full((n, k), -1, dtype=torch.int32, device=thresholds.device)
    out[:, :take] = torch.where(valid, idx, torch.full_like(idx, -1))
    return out


def build_workload(name: str, *, device="cuda", seed: int = 0, batch: Optional[int] = None,
                   ctx_override: Optional[Sequence[int]] = None, block_size: Optional[int] = None,
                   dtype=torch.bfloat16) -> dict:
    """Keyword arguments of ``sparse_flash_mla`` for one input set (plus ``head_dim_v``)."""
    w = WORKLOADS[name]
    if block_size is None:
        block_size = w.get("block", 64)
    b = int(batch if batch is not None else w["B"])
    s_q, h, d, dv, k = w["S"], w["H"], w["D"], w["DV"], w["K"]
    dev = torch.device(device)

    def gen(i):
        return torch.Generator(device=dev).manual_seed(seed * 16 + i)

    if ctx_override is not None:
        lens = [int(x) for x in ctx_override]
        b = len(lens)
    else:
        lo, hi = w["ctx"]
        lg = torch.Generator().manual_seed(seed * 16 + 4)
        lens = [lo if lo == hi else int(x) for x in
                torch.randint(lo, hi + 1, (b,), generator=lg).tolist()]
    q = (torch.randn((b, s_q, h, d), generator=gen(0), device=dev) * 0.5).to(dtype)
    kvg = gen(1)
    rng = np.random.default_rng(seed * 16 + 2)
    fp8 = w.get("kv") == "fp8_ds_mla"
    if fp8:
        ori_kv, ori_bt = _pool_fp8(lens, block_size, rng, kvg, dev)
    else:
        ori_kv, ori_bt = _pool(lens, block_size, d, dtype, rng, kvg, dev)
    cmp_kv = cmp_bt = None
    if w["mode"] == "topk":
        cmp_kv, cmp_bt = ori_kv, ori_bt
    elif w["mode"] in ("swa+topk", "cfa"):
        cmp_kv, cmp_bt = _pool([x // w["cmp_ratio"] for x in lens], block_size, d, dtype, rng,
                               kvg, dev)
    idx = None
    if k > 0 and w.get("prefill"):
        thr = torch.cat([((lens[bi] - s_q + torch.arange(s_q, device=dev) + 1) // w["cmp_ratio"])
                         .clamp(min=0) for bi in range(b)])
        idx = _topk_rows(thr, k, gen(3)).reshape(b, s_q, 1, k)
    elif k > 0:
        ig = gen(3)
        idx = torch.full((b * s_q, k), -1, dtype=torch.int32, device=dev)
        for bi in range(b):
            for s in range(s_q):
                thr = max(0, (lens[bi] - s_q + s + 1) // w["cmp_ratio"])
                if thr:
                    perm = torch.randperm(thr, generator=ig, device=dev)[:k].to(torch.int32)
                    idx[bi * s_q + s, :perm.numel()] = perm
        idx = idx.reshape(b, s_q, 1, k)
    if w["sinks"] == "none":
        sinks = torch.full((h,), float("-inf"), dtype=torch.float32, device=dev)
    else:
        sinks = (torch.rand((h,), generator=gen(5), device=dev) * 2 - 1).to(torch.float32)
    args = dict(q=q, ori_kv=ori_kv, ori_block_table=ori_bt, cmp_kv=cmp_kv,
                cmp_block_table=cmp_bt, cmp_sparse_indices=idx,
                seqused_kv=torch.tensor(lens, dtype=torch.int32, device=dev), sinks=sinks,
                softmax_scale=1.0 / math.sqrt(d), cmp_ratio=w["cmp_ratio"],
                ori_win_left=w["window"], layout_q="BSND", head_dim_v=dv,
                topk_cmp=k if k > 0 else None)
    if fp8:
        args["kv_cache_dtype"] = "fp8_ds_mla"
    if w.get("layout") == "TND":
        # varlen tokens: sequence i owns flat tokens [i * s_q, (i + 1) * s_q)
        args["q"] = q.reshape(b * s_q, h, d)
        args["cu_seqlens_q"] = torch.arange(0, b * s_q + 1, s_q, dtype=torch.int32, device=dev)
        if idx is not None:
            args["cmp_sparse_indices"] = idx.reshape(b * s_q, 1, k)
        args["layout_q"] = "TND"
    return args


def workload_counts(args: dict) -> dict:
    """Query tokens, attended rows and top-k width of one input set."""
    q = args["q"]
    lens = [int(x) for x in args["seqused_kv"].cpu().tolist()]
    if args.get("layout_q") == "TND":
        t_n, h, d = q.shape
        b = len(lens)
        s_q = t_n // max(b, 1)
    else:
        b, s_q, h, d = q.shape
    dv = args.get("head_dim_v") or d
    win = args["ori_win_left"]
    idx = args["cmp_sparse_indices"]
    valid = None
    if idx is not None:
        valid = (idx.reshape(b * s_q, -1) >= 0).sum(dim=1).cpu().tolist()
    ratio = args.get("cmp_ratio")
    dense_cmp = args.get("cmp_kv") is not None and idx is None  # scenario 2: rows [0, thr)
    rows = 0
    for bi in range(b):
        for s in range(s_q):
            sg = lens[bi] - s_q + s
            rows += max(0, sg + 1 - max(sg - win, 0))
            if valid is not None:
                rows += int(valid[bi * s_q + s])
            elif dense_cmp:
                rows += max(0, (sg + 1) // ratio)
    fp8 = args.get("kv_cache_dtype") == "fp8_ds_mla"
    return dict(tokens=b * s_q, rows=rows, heads=h, d_qk=d, d_v=dv,
                k=idx.shape[-1] if idx is not None else 0, row_bytes=656 if fp8 else 2 * d)


def flops_and_bytes(counts: dict, kv_row_bytes: Optional[int] = None) -> tuple:
    """Algorithmic FLOPs and HBM bytes of one call.

    FLOPs = 2 * rows * H * (d_qk + d_v). Bytes = gathered rows (once per query
    token, shared by all heads) + q + out + lse + top-k indices + one block-table
    entry per gathered row.
    """
    t, rows, h = counts["tokens"], counts["rows"], counts["heads"]
    dq, dv, k = counts["d_qk"], counts["d_v"], counts["k"]
    rb = kv_row_bytes if kv_row_bytes is not None else counts.get("row_bytes", dq * 2)
    flops = 2.0 * rows * h * (dq + dv)
    nbytes = rows * rb + t * h * dq * 2 + t * h * dv * 2 + t * h * 4 + t * k * 4 + rows * 4
    return flops, float(nbytes)


def prefill_hbm_bytes(args: dict, counts: dict) -> float:
    """Algorithmic HBM bytes of one prefill call: q, out and lse once, every
    distinct cache row once (consecutive query rows re-read their neighbours'
    window and compressed rows, which stay on chip), the top-k indices and one
    block-table entry per distinct row."""
    lens = [int(x) for x in args["seqused_kv"].cpu().tolist()]
    b = len(lens)
    t, h = counts["tokens"], counts["heads"]
    dq, dv, k, rb = counts["d_qk"], counts["d_v"], counts["k"], counts["row_bytes"]
    s_q = t // max(b, 1)
    win = args["ori_win_left"]
    ratio = args.get("cmp_ratio")
    idx = args.get("cmp_sparse_indices")
    rows = 0
    for bi in range(b):
        first = lens[bi] - s_q  # global position of the first query row
        rows += lens[bi] - max(first - win, 0) if win >= 0 else 0
        if args.get("cmp_kv") is not None and idx is None:
            rows += max(0, lens[bi] // ratio)
        elif idx is not None:
            sel = idx.reshape(b, s_q, -1)[bi]
            rows += int(torch.unique(sel[sel >= 0]).numel())
    return float(rows * (rb + 4) + t * h * (dq * 2 + dv * 2 + 4) + t * k * 4)

