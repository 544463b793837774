"""Accuracy of an fp8 Q·Kᵀ on fp8 cache rows, against golden on the dequantized cache.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): a CPU study, no GPU.

The fp8 cache rows (``fp8_rows``: 512 e4m3 latent dims with one fp32 scale per
128 dims, 64 bf16 rope dims) are attended as golden math on the dequantized
bf16 rows. An fp8-MFMA Q·Kᵀ would instead quantize each head's query latent to
e4m3 with one fp32 scale (amax / 448, round to nearest even) and form

    s = s_q * sum_blk s_k[blk] * (q8[blk] . k8[blk]) + q_rope . k_rope

in fp32 (e4m3 products are exact in fp32). Both variants then run the same
softmax and P·V (golden.py:156-200: 512-row tiles, P rounded to bf16 relative
to the running maximum, fp32 sums, V = the dequantized bf16 rows), so the
difference is the score computation alone. Reported per data set: the largest
|out - golden|, the share of elements beyond atol = rtol = 2e-2, the largest
relative LSE error.

    python -m oracle.fp8_qk_study [--tokens 8]
"""

from __future__ import annotations

import argparse
import math
import sys

import numpy as np
import torch

from .fp8_rows import LATENT, BLOCK, ROPE, decode_e4m3, quantize_rows, scores_fp8

LOG2E = 1.4426950408889634


def _bf16(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def golden_softmax_pv(s: np.ndarray, v: np.ndarray, tile: int = 512):
    """golden.py:156-200 on precomputed fp32 scores ``s`` [G, n] (already scaled),
    no sink: returns out [G, d_v] (bf16 values as float32) and lse [G]."""
    g, n = s.shape
    m = np.full(g, -np.inf, dtype=np.float32)
    l = np.zeros(g, dtype=np.float32)
    acc = np.zeros((g, v.shape[1]), dtype=np.float32)
    for t0 in range(0, n, tile):
        st = s[:, t0:t0 + tile]
        m_new = np.maximum(m, st.max(axis=1))
        alpha = np.exp(m - m_new).astype(np.float32)
        p = np.exp(st - m_new[:, None]).astype(np.float32)
        l = l * alpha + p.sum(axis=1, dtype=np.float32)
        acc = acc * alpha[:, None] + _bf16(p) @ v[t0:t0 + tile]
        m = m_new
    return _bf16(acc / l[:, None]), m + np.log(l)


def scores_bf16(q: np.ndarray, k: np.ndarray, scale: float) -> np.ndarray:
    """Golden's scores: bf16 query and dequantized bf16 rows, fp32 products."""
    return (q.astype(np.float32) @ k.T.astype(np.float32)) * np.float32(scale)


def dequant_bf16(raw: np.ndarray) -> np.ndarray:
    k8 = decode_e4m3(raw[:, :LATENT]).reshape(-1, 4, BLOCK)
    sk = np.ascontiguousarray(raw[:, 512:528]).view("<f4").reshape(-1, 4)
    lat = _bf16((k8 * sk[:, :, None]).astype(np.float32)).reshape(-1, LATENT)
    rope = torch.from_numpy(np.ascontiguousarray(raw[:, 528:]).view("<i2").astype(np.int16)) \
        .view(torch.bfloat16).float().numpy()
    return np.concatenate([lat, rope], axis=1)


def run(dist: str, tokens: int, heads: int = 128, rows: int = 2048, seed: int = 0) -> dict:
    gen = torch.Generator().manual_seed(seed)
    scale = 1.0 / math.sqrt(LATENT + ROPE)
    worst, beyond, total, lse_rel = 0.0, 0, 0, 0.0
    for _ in range(tokens):
        if dist == "normal":   # the benchmark's data: N(0, 1) * 0.5
            q = (torch.randn(heads, LATENT + ROPE, generator=gen) * 0.5).to(torch.bfloat16)
            kv = (torch.randn(rows, LATENT + ROPE, generator=gen) * 0.5).to(torch.bfloat16)
        else:                  # the reference's test data: U(-10, 10)
            q = (torch.rand(heads, LATENT + ROPE, generator=gen) * 20 - 10).to(torch.bfloat16)
            kv = (torch.rand(rows, LATENT + ROPE, generator=gen) * 20 - 10).to(torch.bfloat16)
        raw = quantize_rows(kv)
        k = dequant_bf16(raw)
        qn = q.float().numpy()
        o_ref, l_ref = golden_softmax_pv(scores_bf16(qn, k, scale), k[:, :LATENT])
        o_f8, l_f8 = golden_softmax_pv(scores_fp8(qn, raw, scale), k[:, :LATENT])
        d = np.abs(o_f8 - o_ref)
        worst = max(worst, float(d.max()))
        beyond += int((d > 2e-2 + 2e-2 * np.abs(o_ref)).sum())
        total += d.size
        lse_rel = max(lse_rel, float((np.abs(l_f8 - l_ref) / np.maximum(np.abs(l_ref), 1e-6)).max()))
    return dict(dist=dist, tokens=tokens, max_abs=worst, beyond_2e2=beyond, elements=total,
                beyond_frac=beyond / total, lse_max_rel=lse_rel)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--tokens", type=int, default=8)
    args = ap.parse_args(argv)
    for dist in ("normal", "uniform"):
        r = run(dist, args.tokens)
        print(f"{r['dist']:8s} tokens {r['tokens']}: max |out - golden| {r['max_abs']:.4g}, "
              f"beyond 2e-2: {r['beyond_2e2']} of {r['elements']} ({100 * r['beyond_frac']:.3f} %), "
              f"max LSE rel err {r['lse_max_rel']:.3g}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
