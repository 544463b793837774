"""The online softmax in the HIP kernel's order of rounding, for the accuracy contract.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Golden (golden.py:156-200) walks each segment (window rows, then compressed
rows) in 512-row tiles and rounds P to the input dtype relative to the running
maximum *after* each tile, so the largest score of a tile gets P = 1 exactly.
The HIP kernel walks the whole attended list (window ++ compressed) in
``tile``-row tiles, in ``streams`` interleaved streams (tile t belongs to
stream t % streams, each with its own maximum, row sum and accumulator, merged
at the end), and moves a head's running maximum only when a tile's maximum
exceeds it by more than ``tau`` (log2 units): P = exp2(s·scale·log2e − m) may
then be up to 2^tau, and is rounded to the input dtype at that scale.
Everything else is the same contract: fp32 scores, fp32 row sums of the
unrounded P, fp32 accumulation of bf16(P)·V, out = RNE(acc / l), lse = m + ln l.

``attend_token_kernel_order(tile=512, tau=0, streams=1, segment_tiles=True)``
is golden's own order (up to exp vs exp2 in fp32), which the CPU tests pin
against ``golden_ref.attend_token``.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple

import numpy as np
import torch

LOG2E = 1.4426950408889634
LN2 = 0.6931471805599453


def attend_token_kernel_order(q: torch.Tensor, segments: Sequence[torch.Tensor],
                              sinks: torch.Tensor, softmax_scale: float, *,
                              d_v: Optional[int] = None, tile: int = 32, tau: float = 8.0,
                              streams: int = 1, segment_tiles: bool = False,
                              out_dtype: Optional[torch.dtype] = None
                              ) -> Tuple[torch.Tensor, torch.Tensor]:
    """One query token's ``(out [G, d_v], lse [G])`` in the kernel's rounding order.

    ``segment_tiles``: cut each segment into tiles on its own (golden's order)
    instead of tiling the concatenated list (the kernel's order). ``out_dtype``:
    the type ``acc / l`` is rounded to (default: the input type; float32 for a
    split piece's partial).
    """
    dtype = q.dtype
    g, d = q.shape
    dv = d if d_v is None else int(d_v)
    segs = [s for s in segments if s.shape[0] > 0]
    tiles = []
    if segment_tiles:
        for s in segs:
            kf = s.to(torch.float32)
            tiles += [kf[t0:t0 + tile] for t0 in range(0, kf.shape[0], tile)]
    elif segs:
        kf = torch.cat(segs).to(torch.float32)
        tiles = [kf[t0:t0 + tile] for t0 in range(0, kf.shape[0], tile)]
    qf = q.to(torch.float32)
    c = torch.tensor(softmax_scale, dtype=torch.float32) * torch.tensor(LOG2E, dtype=torch.float32)
    neg = torch.full((g,), -math.inf, dtype=torch.float32)
    m = [neg.clone() for _ in range(streams)]
    l = [torch.zeros(g, dtype=torch.float32) for _ in range(streams)]
    acc = [torch.zeros((g, dv), dtype=torch.float32) for _ in range(streams)]
    m[0] = sinks.to(torch.float32) * torch.tensor(LOG2E, dtype=torch.float32)  # sink seeds stream 0
    l[0] = torch.ones(g, dtype=torch.float32)
    for t, kt in enumerate(tiles):
        i = t % streams
        sv = (qf @ kt.T) * c
        mloc = sv.amax(dim=1)
        grow = mloc > m[i] + tau
        m_new = torch.where(grow, torch.maximum(m[i], mloc), m[i])
        alpha = torch.where(grow, torch.exp2(m[i] - m_new), torch.ones_like(m_new))
        alpha = torch.where(torch.isnan(alpha), torch.zeros_like(alpha), alpha)  # -inf - -inf
        l[i] = l[i] * alpha
        acc[i] = acc[i] * alpha[:, None]
        m[i] = m_new
        p = torch.exp2(sv - m[i][:, None])
        p = torch.where(torch.isnan(p), torch.zeros_like(p), p)
        l[i] = l[i] + p.sum(dim=1)
        acc[i] = acc[i] + p.to(dtype).to(torch.float32) @ kt[:, :dv]
    # merge the streams (exact fp32 rescale to the common maximum)
    mt = m[0]
    for i in range(1, streams):
        mt = torch.maximum(mt, m[i])
    lt = torch.zeros(g, dtype=torch.float32)
    at = torch.zeros((g, dv), dtype=torch.float32)
    for i in range(streams):
        w = torch.exp2(m[i] - mt)
        w = torch.where(torch.isnan(w), torch.zeros_like(w), w)
        lt = lt + w * l[i]
        at = at + w[:, None] * acc[i]
    out = (at / lt[:, None]).to(dtype if out_dtype is None else out_dtype)
    lse = (mt + torch.log2(lt)) * torch.tensor(LN2, dtype=torch.float32)
    return out, lse


def fp16_partial(o: torch.Tensor) -> torch.Tensor:
    """A split piece's partial rows ``o`` [heads, d_v] (fp32) as the kernels store them:
    per row, fp16 of ``o * s`` with ``s = 2^(14 - e)``, ``e = max(floor(log2 m), -112)``
    for the row's largest |value| ``m`` when it is finite and nonzero (so ``m * s``
    lies in [2^14, 2^15): rows are scaled up or down; the clamp keeps ``s`` and
    ``1 / s`` normal floats), else ``s = 1``; returned as fp32 ``fp16(o * s) / s``."""
    o = o.to(torch.float32)
    m = o.abs().nan_to_num(nan=0.0).amax(dim=1, keepdim=True)
    ok = (m > 0) & torch.isfinite(m)
    e = torch.frexp(torch.where(ok, m, torch.ones_like(m)))[1].to(torch.float32) - 1.0
    e = e.clamp(min=-112.0)
    s = torch.where(ok, torch.exp2(14.0 - e), torch.ones_like(m))
    return (o * s).to(torch.float16).to(torch.float32) / s


def attend_token_split(q: torch.Tensor, segments: Sequence[torch.Tensor], sinks: torch.Tensor,
                       softmax_scale: float, *, d_v: Optional[int] = None, tile: int = 64,
                       pieces: int = 2, partial_dtype: torch.dtype = torch.float32
                       ) -> Tuple[torch.Tensor, torch.Tensor]:
    """One token split into ``pieces`` contiguous pieces of the attended list (cut at
    multiples of ``tile``), each in the kernel's order without the sink, its
    partial ``acc / l`` rounded to ``partial_dtype`` (fp16: scaled as the kernels
    store it, ``fp16_partial``), merged in fp32 as the merge kernel does:
    lse = m + ln(e^(sink - m) + sum_i e^(lse_i - m)) over m = max(sink, lse_i),
    out = RNE(sum_i e^(lse_i - lse) o_i)."""
    dtype = q.dtype
    g = q.shape[0]
    dv = q.shape[1] if d_v is None else int(d_v)
    segs = [s for s in segments if s.shape[0] > 0]
    rows = torch.cat(segs) if segs else torch.zeros((0, q.shape[1]), dtype=dtype)
    n = rows.shape[0]
    cuts = [0] + [min(n, -(-(n * k // pieces) // tile) * tile) for k in range(1, pieces)] + [n]
    no_sink = torch.full((g,), -math.inf, dtype=torch.float32)
    parts = []
    for lo, hi in zip(cuts, cuts[1:]):
        if hi > lo:
            f16 = partial_dtype == torch.float16
            o, l = attend_token_kernel_order(q, [rows[lo:hi]], no_sink, softmax_scale, d_v=dv,
                                             tile=tile, tau=0.0,
                                             out_dtype=torch.float32 if f16 else partial_dtype)
            parts.append((fp16_partial(o) if f16 else o, l))
    sink = sinks.to(torch.float32)
    mx = sink.clone()
    for _, l in parts:
        mx = torch.maximum(mx, l)
    tot = torch.where(torch.isfinite(mx), torch.exp(sink - mx), torch.zeros_like(mx))
    tot = torch.where(torch.isnan(tot), torch.zeros_like(tot), tot)
    for _, l in parts:
        e = torch.exp(l - mx)
        tot = tot + torch.where(torch.isnan(e), torch.zeros_like(e), e)
    lse = mx + torch.log(tot)
    out = torch.zeros((g, dv), dtype=torch.float32)
    for o, l in parts:
        w = torch.exp(l - lse)
        w = torch.where(torch.isnan(w), torch.zeros_like(w), w)
        out = out + w[:, None] * o.to(torch.float32)
    return out.to(dtype), lse


def sparse_attn_kernel_order(q: torch.Tensor, *, tile: int = 32, tau: float = 8.0,
                             streams: int = 1, **kw):
    """``golden_ref.sparse_attn_oracle`` with the per-token math in the kernel's order."""
    from .golden_ref import sparse_attn_oracle

    def attend(qt, segments, sinks, softmax_scale, d_v=None):
        return attend_token_kernel_order(qt, segments, sinks, softmax_scale, d_v=d_v, tile=tile,
                                         tau=tau, streams=streams)

    return sparse_attn_oracle(q, attend=attend, **kw)


def compare(x: torch.Tensor, golden: torch.Tensor, exact: np.ndarray) -> dict:
    """Agreement of ``x`` with golden under the two acceptance rules, and accuracy.

    * ``pct_ref``: share (%) of elements within the reference's bf16 rule
      (|x - golden| <= 1e-4 + 2^-7 |golden|, test_sparse_attn_sharedkv.py:394-481);
    * ``beyond_2e2``: elements with |x - golden| > 2e-2 + 2e-2 |golden|;
    * ``max_abs``: max |x - golden|;
    * ``err_exact`` / ``golden_exact``: max |x - exact|, max |golden - exact|.
    """
    a = x.detach().to(torch.float32).reshape(-1).numpy().astype(np.float64)
    b = golden.detach().to(torch.float32).reshape(-1).numpy().astype(np.float64)
    e = np.asarray(exact, dtype=np.float64).reshape(-1)
    err = np.abs(a - b)
    keep = np.isfinite(e)
    return dict(
        pct_ref=float((err <= 1e-4 + 0.0078125 * np.abs(b)).mean() * 100) if a.size else 100.0,
        beyond_2e2=int((err > 2e-2 + 2e-2 * np.abs(b)).sum()),
        max_abs=float(err.max()) if a.size else 0.0,
        err_exact=float(np.abs(a[keep] - e[keep]).max()) if keep.any() else 0.0,
        golden_exact=float(np.abs(b[keep] - e[keep]).max()) if keep.any() else 0.0)
