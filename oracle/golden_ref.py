"""CPU restatement of the reference's golden math for sparse shared-KV attention.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): never imported by the
product package.

Follows ``golden.py`` (reference) function by function:

* ``causal_position``        golden.py:125   s_global = act_kv - act_q + s
* ``window_range``           golden.py:128-131
* ``cmp_threshold``          golden.py:44, :147
* ``resolve_topk_rows``      golden.py:28-66  (sparse_block_size = 1)
* ``dense_cmp_rows``         golden.py:146-150
* ``attend_token``           golden.py:156-200 (online softmax seeded by the
                              sink, 512-row tiles that never straddle the
                              window/compressed boundary, P rounded to the
                              input dtype before P·V, fp32 state)
* ``sparse_attn_oracle``     golden.py:69-204 driver, restated over paged
                              pools (rows gathered through the block tables,
                              the way api.py:208-240 flattens tokens)
* ``sparse_attn_exact``      the same driver with the float64 closed form per
                              token (no tiling, no rounding): the exact answer
                              both golden and the HIP path approximate
* fp8 caches (656-byte rows, no reference counterpart): rows are gathered
  raw and dequantized with ``fp8_rows.dequantize_rows``; everything after
  is the bf16 math above
* ``attend_token_scores``    ``attend_token`` on precomputed scores (the same
                              tiles, sink, rounding and state); with golden's
                              scores it equals ``attend_token`` bit for bit
* ``attend_token_fp8qk``     the fp8 Q·Kᵀ form (``fp8_qk=True``, no reference
                              counterpart): scores from ``fp8_rows.scores_fp8``
                              on the raw rows, P·V on the dequantized rows
* ``merge_partials``         the closed-form split-KV merge
                              lse = log(e^sink + Σ e^lse_i),
                              o = Σ e^(lse_i - lse) · o_i

Deliberate restrictions (inputs outside the reference's contract):
``act_q <= act_kv`` per sequence (golden's Python slicing wraps for negative
ends), top-k ids are ``-1`` or non-negative (golden wraps negative ids other
than ``-1`` into Python negative indexing).
"""

from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple

import numpy as np
import torch

GOLDEN_S2_TILE = 512  # golden.py:25


# ---------------------------------------------------------------------------
# Index resolution (integer work: must match the HIP path exactly)
# ---------------------------------------------------------------------------

def causal_position(act_kv: int, act_q: int, s: int) -> int:
    """Bottom-right aligned causal position of query row ``s`` (golden.py:125)."""
    return int(act_kv) - int(act_q) + int(s)


def window_range(s_global: int, win_left: int, win_right: int = 0) -> Tuple[int, int]:
    """Half-open raw-KV window ``[left, right)`` for one query (golden.py:128-131).

    ``win_left = -1`` yields an empty window (left = right = s_global + 1),
    which is how pure top-k attention is expressed through this API.
    """
    right = s_global + win_right + 1
    left = max(s_global - win_left, 0)
    if right < left:
        right = left
    return left, right


def cmp_threshold(act_kv: int, act_q: int, s: int, cmp_ratio: int) -> int:
    """Causal bound on compressed entries: floor((s_global + 1) / ratio) (golden.py:44)."""
    return math.floor((int(act_kv) - int(act_q) + int(s) + 1) / int(cmp_ratio))


def resolve_topk_rows(idx_row: Sequence[int], act_kv: int, act_q: int, s: int,
                      cmp_ratio: int) -> List[int]:
    """Compressed rows attended by one query, in scan order (golden.py:28-66).

    Scans the first ``min(K, thr)`` entries; ``-1`` stops the scan; an entry
    at or beyond ``thr`` is skipped; the row is clipped to the sequence's
    compressed length ``floor(act_kv / ratio)``. Duplicates are kept.
    """
    ids = [int(v) for v in idx_row]
    k = len(ids)
    thr = cmp_threshold(act_kv, act_q, s, cmp_ratio)
    cmp_len = math.floor(int(act_kv) / int(cmp_ratio))
    rows: List[int] = []
    for i in range(max(0, min(k, thr))):
        v = ids[i]
        if v == -1:
            break
        if v < 0:
            continue  # outside the input contract; never attended
        begin, end = v, min(v + 1, cmp_len)
        if begin >= thr:
            continue
        end = min(end, thr)
        rows.extend(range(begin, end))
    return rows


def dense_cmp_rows(act_kv: int, act_q: int, s: int, cmp_ratio: int) -> List[int]:
    """Dense compressed rows [0, thr) of the CFA scenario (golden.py:146-150)."""
    return list(range(max(cmp_threshold(act_kv, act_q, s, cmp_ratio), 0)))


# ---------------------------------------------------------------------------
# Paged pools
# ---------------------------------------------------------------------------

def gather_paged_rows(pool: torch.Tensor, table: torch.Tensor, b: int,
                      positions: Sequence[int]) -> torch.Tensor:
    """Rows ``positions`` of sequence ``b`` from a PA_ND pool ``[blocks, bs, 1, D]``.

    Row ``p`` lives at ``pool[table[b, p // bs], p % bs, 0]`` (the DataCopyPA
    addressing of kernel.py:539-651, and the inverse of golden.py:350-358).
    """
    bs = pool.shape[1]
    if len(positions) == 0:
        return pool.new_zeros((0, pool.shape[-1]))
    pos = torch.as_tensor(list(positions), dtype=torch.long, device=pool.device)
    phys = table[b].to(torch.long)[pos // bs]
    if bool((phys < 0).any()):
        raise ValueError("block table entry -1 inside the attended range")
    return pool[phys, pos % bs, 0, :]


# ---------------------------------------------------------------------------
# Per-token online softmax (the floating-point contract)
# ---------------------------------------------------------------------------

def attend_token(q: torch.Tensor, segments: Sequence[torch.Tensor], sinks: torch.Tensor,
                 softmax_scale: float, *, d_v: Optional[int] = None,
                 tile: int = GOLDEN_S2_TILE) -> Tuple[torch.Tensor, torch.Tensor]:
    """Attention of one query token over shared K=V rows (golden.py:156-200).

    ``q``: ``[G, D]`` in the input dtype. ``segments``: row blocks ``[n_i, D]``
    walked in order (window rows, then compressed rows); each segment is cut
    into ``tile``-row tiles independently. ``sinks``: ``[G]`` fp32 logits of a
    virtual key with a zero value row. Returns ``(out [G, d_v] in q.dtype,
    lse [G] fp32)``; ``d_v`` defaults to ``D`` (output columns are
    independent, so the first ``d_v`` columns equal golden's full output
    sliced).
    """
    dtype = q.dtype
    g, d = q.shape
    dv = d if d_v is None else int(d_v)
    qf = q.to(torch.float32)
    row_max = sinks.to(torch.float32).clone()
    row_sum = torch.ones(g, dtype=torch.float32)
    acc = torch.zeros((g, dv), dtype=torch.float32)
    for seg in segments:
        if seg.shape[0] == 0:
            continue
        kf = seg.to(torch.float32)
        for t0 in range(0, kf.shape[0], tile):
            kt = kf[t0:t0 + tile]
            score = (qf @ kt.T) * softmax_scale
            new_max = torch.maximum(row_max, score.amax(dim=1))
            alpha = torch.exp(row_max - new_max)
            p = torch.exp(score - new_max[:, None])
            row_sum = alpha * row_sum + p.sum(dim=1)
            p_in = p.to(dtype).to(torch.float32)  # golden.py:193-194
            acc = acc * alpha[:, None] + p_in @ kt[:, :dv]
            row_max = new_max
    out = (acc / row_sum[:, None]).to(dtype)
    lse = row_max + torch.log(row_sum)
    return out, lse


def attend_token_scores(scores: Sequence[torch.Tensor], values: Sequence[torch.Tensor],
                        sinks: torch.Tensor, dtype: torch.dtype,
                        tile: int = GOLDEN_S2_TILE) -> Tuple[torch.Tensor, torch.Tensor]:
    """``attend_token``'s online softmax on given scores (golden.py:156-200).

    ``scores[i]``: ``[G, n_i]`` fp32 scores of segment i, already multiplied by
    the softmax scale; ``values[i]``: ``[n_i, d_v]`` value rows (input dtype
    values). Same 512-row tiles per segment, sink seeding, P rounded to
    ``dtype`` before P·V and fp32 state as ``attend_token``.
    """
    g = scores[0].shape[0] if scores else sinks.shape[0]
    dv = values[0].shape[1]
    row_max = sinks.to(torch.float32).clone()
    row_sum = torch.ones(g, dtype=torch.float32)
    acc = torch.zeros((g, dv), dtype=torch.float32)
    for sc_seg, v_seg in zip(scores, values):
        if sc_seg.shape[1] == 0:
            continue
        vf = v_seg.to(torch.float32)
        for t0 in range(0, sc_seg.shape[1], tile):
            score = sc_seg[:, t0:t0 + tile].to(torch.float32)
            new_max = torch.maximum(row_max, score.amax(dim=1))
            alpha = torch.exp(row_max - new_max)
            p = torch.exp(score - new_max[:, None])
            row_sum = alpha * row_sum + p.sum(dim=1)
            p_in = p.to(dtype).to(torch.float32)
            acc = acc * alpha[:, None] + p_in @ vf[t0:t0 + tile]
            row_max = new_max
    out = (acc / row_sum[:, None]).to(dtype)
    lse = row_max + torch.log(row_sum)
    return out, lse


def attend_token_fp8qk(q: torch.Tensor, raw_segments: Sequence[torch.Tensor], sinks: torch.Tensor,
                       softmax_scale: float, *, d_v: int = 512,
                       tile: int = GOLDEN_S2_TILE) -> Tuple[torch.Tensor, torch.Tensor]:
    """One token under the fp8 Q·Kᵀ form: scores from ``fp8_rows.scores_fp8`` on the
    raw 656-byte rows (per-head e4m3 query, per-block row scales), then golden's
    softmax and P·V on the dequantized bf16 rows (``attend_token_scores``)."""
    from .fp8_rows import dequantize_rows, scores_fp8
    scores, values = [], []
    for raw in raw_segments:
        if raw.shape[0] == 0:
            scores.append(torch.zeros((q.shape[0], 0), dtype=torch.float32))
            values.append(torch.zeros((0, d_v), dtype=q.dtype))
            continue
        scores.append(torch.from_numpy(scores_fp8(q.to(torch.float32).numpy(), raw, softmax_scale)))
        values.append(dequantize_rows(raw)[:, :d_v])
    return attend_token_scores(scores, values, sinks, q.dtype, tile=tile)


def one_shot_reference(q: np.ndarray, rows: np.ndarray, sinks: np.ndarray,
                       softmax_scale: float) -> Tuple[np.ndarray, np.ndarray]:
    """float64 closed form ``softmax(scores ∪ sink) · V`` (golden.py:207-244 semantics).

    No chunking and no rounding: the independent check the chunked
    ``attend_token`` is pinned against.
    """
    q64 = np.asarray(q, dtype=np.float64)
    k64 = np.asarray(rows, dtype=np.float64)
    s64 = np.asarray(sinks, dtype=np.float64)
    score = q64 @ k64.T * softmax_scale if k64.shape[0] else np.zeros((q64.shape[0], 0))
    allv = np.concatenate([score, s64[:, None]], axis=1)
    mx = allv.max(axis=1, keepdims=True)
    mx = np.where(np.isfinite(mx), mx, 0.0)
    e = np.exp(score - mx)
    denom = e.sum(axis=1) + np.exp(s64 - mx[:, 0])
    out = (e @ k64) / denom[:, None] if k64.shape[0] else np.zeros((q64.shape[0], 0))
    with np.errstate(divide="ignore"):
        lse = mx[:, 0] + np.log(denom)
    return out, lse


def merge_partials(o_parts: Sequence[np.ndarray], lse_parts: Sequence[np.ndarray],
                   sinks: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Closed-form split-KV merge over partials ``(o_i [G, dv], lse_i [G])``.

    Each partial is normalised over its own rows and excludes the sink; the
    sink enters the merged denominator exactly once.
    """
    lse_all = np.stack([np.asarray(x, np.float64) for x in lse_parts] +
                       [np.asarray(sinks, np.float64)], axis=0)
    mx = lse_all.max(axis=0)
    mx = np.where(np.isfinite(mx), mx, 0.0)
    w = np.exp(lse_all - mx[None, :])
    tot = w.sum(axis=0)
    with np.errstate(divide="ignore"):
        lse = mx + np.log(tot)
    out = np.zeros_like(np.asarray(o_parts[0], np.float64))
    for i, o in enumerate(o_parts):
        out += (w[i] / tot)[:, None] * np.asarray(o, np.float64)
    return out, lse


# ---------------------------------------------------------------------------
# Whole-call driver over the API's tensors
# ---------------------------------------------------------------------------

def token_layout(layout_q: str, q_shape, cu_seqlens_q: Optional[torch.Tensor]):
    """(B, S_max, q_prefix list, act_q list) exactly as api.py:208-240 derives them."""
    if layout_q == "TND":
        cu = [int(x) for x in cu_seqlens_q.tolist()]
        b = len(cu) - 1
        lens = [cu[i + 1] - cu[i] for i in range(b)]
        return b, (max(lens) if lens else 0), cu[:-1], lens
    b, s_max = int(q_shape[0]), int(q_shape[1])
    prefix = [i * s_max for i in range(b)]
    if cu_seqlens_q is not None:
        cu = [int(x) for x in cu_seqlens_q.tolist()]
        lens = [cu[i + 1] - cu[i] for i in range(b)]
    else:
        lens = [s_max] * b
    return b, s_max, prefix, lens


def _is_fp8_pool(pool, kv_cache_dtype) -> bool:
    return kv_cache_dtype == "fp8_ds_mla" or (
        kv_cache_dtype in (None, "auto") and pool.dtype in (torch.uint8, torch.float8_e4m3fn))


def token_rows(*, b: int, s: int, act_q: int, act_kv: int, ori_kv, ori_block_table,
               cmp_kv, cmp_block_table, cmp_idx_row, cmp_ratio, ori_win_left,
               ori_win_right=0, kv_cache_dtype=None,
               raw: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """The two row segments (window rows, compressed rows) one query attends.

    fp8 pools (656-byte rows) are gathered raw and returned dequantized to bf16
    (or raw, with ``raw=True``).
    """
    s_glob = causal_position(act_kv, act_q, s)
    lo, hi = window_range(s_glob, ori_win_left, ori_win_right)
    ori_rows = gather_paged_rows(ori_kv, ori_block_table, b, range(lo, hi))
    if cmp_kv is None:
        cmp_rows = ori_rows.new_zeros((0, ori_rows.shape[-1]))
    elif cmp_idx_row is None:
        cmp_rows = gather_paged_rows(cmp_kv, cmp_block_table, b,
                                     dense_cmp_rows(act_kv, act_q, s, cmp_ratio))
    else:
        cmp_rows = gather_paged_rows(cmp_kv, cmp_block_table, b,
                                     resolve_topk_rows(cmp_idx_row, act_kv, act_q, s, cmp_ratio))
    if _is_fp8_pool(ori_kv, kv_cache_dtype) and not raw:
        from .fp8_rows import dequantize_rows
        ori_rows, cmp_rows = dequantize_rows(ori_rows), dequantize_rows(cmp_rows)
    return ori_rows, cmp_rows


def sparse_attn_oracle(q: torch.Tensor, *, ori_kv: torch.Tensor, ori_block_table: torch.Tensor,
                       seqused_kv, sinks: torch.Tensor, softmax_scale: float,
                       cmp_kv: Optional[torch.Tensor] = None,
                       cmp_block_table: Optional[torch.Tensor] = None,
                       cmp_sparse_indices: Optional[torch.Tensor] = None,
                       cu_seqlens_q: Optional[torch.Tensor] = None,
                       cmp_ratio: Optional[int] = None, ori_win_left: int = 127,
                       ori_win_right: int = 0, layout_q: str = "TND",
                       head_dim_v: Optional[int] = None,
                       tokens: Optional[Sequence[int]] = None,
                       kv_cache_dtype: Optional[str] = None, attend=None,
                       fp8_qk: bool = False):
    """Golden output of ``sparse_attn_sharedkv`` for the API's own tensors.

    Returns ``(out, lse)`` in the caller's layout (``[T, N1, Dv]``/``[T, N1]``
    for TND, ``[B, S, N1, Dv]``/``[B, S, N1]`` for BSND); padded query rows
    stay zero (golden.py:106-111). ``tokens`` restricts the work to a subset
    of flat token ids (others stay zero) so large workloads can be sampled.
    ``attend`` replaces the per-token math (default ``attend_token``; the
    kernel-order restatement of ``kernel_order`` plugs in here). ``fp8_qk``
    (fp8 pools): the fp8 Q·Kᵀ form, ``attend_token_fp8qk`` on the raw rows.
    All tensors are read on the CPU.
    """
    if fp8_qk:
        if not _is_fp8_pool(ori_kv, kv_cache_dtype):
            raise ValueError("fp8_qk needs an fp8 pool")
        attend = attend_token_fp8qk
    attend = attend_token if attend is None else attend
    q = q.cpu()
    n1, d = q.shape[-2], q.shape[-1]
    dv = d if head_dim_v is None else int(head_dim_v)
    sinks = sinks.cpu().to(torch.float32)
    ori_kv, ori_block_table = ori_kv.cpu(), ori_block_table.cpu()
    if cmp_kv is not None:
        cmp_kv, cmp_block_table = cmp_kv.cpu(), cmp_block_table.cpu()
    kv_lens = [int(x) for x in torch.as_tensor(seqused_kv).cpu().tolist()]
    nb, s_max, prefix, act_q = token_layout(layout_q, q.shape, cu_seqlens_q)
    q_flat = q.reshape(-1, n1, d)
    total = q_flat.shape[0]
    idx_flat = None
    if cmp_sparse_indices is not None:
        ci = cmp_sparse_indices.cpu().to(torch.int64)
        idx_flat = ci.reshape(total, ci.shape[-2], ci.shape[-1])
    out = torch.zeros((total, n1, dv), dtype=q.dtype)
    lse = torch.zeros((total, n1), dtype=torch.float32)
    want = None if tokens is None else set(int(t) for t in tokens)
    for b in range(nb):
        for s in range(act_q[b]):
            t = prefix[b] + s
            if want is not None and t not in want:
                continue
            ori_rows, cmp_rows = token_rows(
                b=b, s=s, act_q=act_q[b], act_kv=kv_lens[b], ori_kv=ori_kv,
                ori_block_table=ori_block_table, cmp_kv=cmp_kv,
                cmp_block_table=cmp_block_table,
                cmp_idx_row=None if idx_flat is None else idx_flat[t, 0].tolist(),
                cmp_ratio=cmp_ratio, ori_win_left=ori_win_left, ori_win_right=ori_win_right,
                kv_cache_dtype=kv_cache_dtype, raw=fp8_qk)
            o, l = attend(q_flat[t], [ori_rows, cmp_rows], sinks, softmax_scale, d_v=dv)
            out[t] = o
            lse[t] = l
    if layout_q == "TND":
        return out, lse
    return out.reshape(nb, s_max, n1, dv), lse.reshape(nb, s_max, n1)


def sparse_attn_exact(q: torch.Tensor, *, ori_kv, ori_block_table, seqused_kv, sinks,
                      softmax_scale, cmp_kv=None, cmp_block_table=None, cmp_sparse_indices=None,
                      cu_seqlens_q=None, cmp_ratio=None, ori_win_left=127, ori_win_right=0,
                      layout_q="TND", head_dim_v=None, tokens=None, kv_cache_dtype=None):
    """float64 closed-form outputs ``(out, lse)`` over the same rows as ``sparse_attn_oracle``.

    Flat ``[T, N1, Dv]`` / ``[T, N1]`` numpy arrays; tokens outside ``tokens``
    (and padded rows) are NaN.
    """
    q = q.cpu()
    n1, d = q.shape[-2], q.shape[-1]
    dv = d if head_dim_v is None else int(head_dim_v)
    kv_lens = [int(x) for x in torch.as_tensor(seqused_kv).cpu().tolist()]
    nb, _, prefix, act_q = token_layout(layout_q, q.shape, cu_seqlens_q)
    q_flat = q.reshape(-1, n1, d)
    total = q_flat.shape[0]
    idx_flat = None
    if cmp_sparse_indices is not None:
        ci = cmp_sparse_indices.cpu().to(torch.int64)
        idx_flat = ci.reshape(total, ci.shape[-2], ci.shape[-1])
    out = np.full((total, n1, dv), np.nan)
    lse = np.full((total, n1), np.nan)
    want = None if tokens is None else set(int(t) for t in tokens)
    snk = sinks.cpu().to(torch.float64).numpy()
    for b in range(nb):
        for s in range(act_q[b]):
            t = prefix[b] + s
            if want is not None and t not in want:
                continue
            ori_rows, cmp_rows = token_rows(
                b=b, s=s, act_q=act_q[b], act_kv=kv_lens[b], ori_kv=ori_kv.cpu(),
                ori_block_table=ori_block_table.cpu(),
                cmp_kv=None if cmp_kv is None else cmp_kv.cpu(),
                cmp_block_table=None if cmp_block_table is None else cmp_block_table.cpu(),
                cmp_idx_row=None if idx_flat is None else idx_flat[t, 0].tolist(),
                cmp_ratio=cmp_ratio, ori_win_left=ori_win_left, ori_win_right=ori_win_right,
                kv_cache_dtype=kv_cache_dtype)
            rows = torch.cat([ori_rows, cmp_rows]).to(torch.float64).numpy()
            o, l = one_shot_reference(q_flat[t].to(torch.float64).numpy(), rows, snk,
                                      softmax_scale)
            out[t] = o[:, :dv] if o.shape[1] else 0.0
            lse[t] = l
    return out, lse
