"""Every benchmark configuration at full size, every query row checked against the oracle.

SWA decode B = 32 (H = 64, ctx U[2048, 8192], window 128), SWA + top-k compressed
decode B = 32 (ctx 16384, ratio 4, K = 512), the DeepSeek-V3.2-shape top-k decode B =
64 at S = 1 and S = 2 (H = 128, ctx 32768, K = 2048) and the long-context fp8 decode
(128 sequences, ctx U[32768, 131072], fp8 rows): the same schedules the benchmark
runs. Rows are resolved with the oracle's integer functions (``causal_position``,
``window_range``, ``resolve_topk_rows``, golden.py:28-66, :125-131) and the block
tables, their bytes gathered by index from the pools where they lie (the pools are
too large to copy whole), and each query row's output computed by ``attend_token``
(golden.py:156-200) on the CPU. Asserted: every output element within atol = rtol =
2e-2 of golden and every LSE within 1e-3 relative (``check_strict``), and on a
sample of rows the float64 closed form (``check_vs_exact``).
"""

import sys

import numpy as np
import pytest
import torch

from oracle import gen
from oracle.checks import check_strict, check_vs_exact
from oracle.fp8_rows import dequantize_rows
from oracle.golden_ref import (attend_token, causal_position, dense_cmp_rows, one_shot_reference,
                               resolve_topk_rows, token_layout, window_range)

pytestmark = pytest.mark.gpu

HAS_GPU = torch.cuda.is_available()
requires_gpu = pytest.mark.skipif(not HAS_GPU, reason="needs a ROCm GPU")

if HAS_GPU:
    from sparse_attn_sharedkv_amd import sparse_flash_mla


def _say(msg):
    print(f"[gpu-full] {msg}", flush=True)
    sys.stdout.flush()


def _phys(table_row, positions, bs):
    pos = np.asarray(positions, dtype=np.int64)
    if pos.size == 0:
        return pos
    blk = table_row[pos // bs]
    assert (blk >= 0).all(), "block table entry -1 inside the attended range"
    return blk.astype(np.int64) * bs + pos % bs


def _check_all_rows(kw, out, lse, exact_every=8):
    q = kw["q"]
    n1, d = q.shape[-2], q.shape[-1]
    dv = kw.get("head_dim_v") or d
    nb, s_max, prefix, act_q = token_layout(kw.get("layout_q", "TND"), q.shape,
                                            kw.get("cu_seqlens_q"))
    kv = kw["seqused_kv"].cpu().tolist()
    ratio = kw.get("cmp_ratio") or 1
    win = kw["ori_win_left"]
    q_flat = q.reshape(-1, n1, d)
    fp8 = kw["ori_kv"].shape[-1] == 656
    ori = kw["ori_kv"].reshape(-1, kw["ori_kv"].shape[-1])
    bs1 = kw["ori_kv"].shape[1]
    t1 = kw["ori_block_table"].cpu().numpy()
    cmp_ = kw.get("cmp_kv")
    if cmp_ is not None:
        bs2 = cmp_.shape[1]
        t2 = kw["cmp_block_table"].cpu().numpy()
        cmp_ = cmp_.reshape(-1, cmp_.shape[-1])
    idx = kw.get("cmp_sparse_indices")
    idx = None if idx is None else idx.reshape(q_flat.shape[0], -1).cpu().numpy()
    sinks = kw["sinks"].cpu().float()
    out = out.reshape(-1, n1, dv).cpu()
    lse = lse.reshape(-1, n1).cpu()
    refs, ref_l, outs, lses, ex, ex_ref, ex_out = [], [], [], [], [], [], []
    n_checked = 0
    for b in range(nb):
        for s in range(act_q[b]):
            t = prefix[b] + s
            lo, hi = window_range(causal_position(kv[b], act_q[b], s), win)
            rows_o = ori[torch.as_tensor(_phys(t1[b], range(lo, hi), bs1), device=ori.device)]
            if cmp_ is None:
                rows_c = rows_o[:0]
            else:
                pos = (resolve_topk_rows(idx[t].tolist(), kv[b], act_q[b], s, ratio) if idx is not None
                       else dense_cmp_rows(kv[b], act_q[b], s, ratio))
                rows_c = cmp_[torch.as_tensor(_phys(t2[b], pos, bs2), device=cmp_.device)]
            rows_o, rows_c = rows_o.cpu(), rows_c.cpu()
            if fp8:
                rows_o, rows_c = dequantize_rows(rows_o), dequantize_rows(rows_c)
            o, l = attend_token(q_flat[t].cpu(), [rows_o, rows_c], sinks, kw["softmax_scale"],
                                d_v=dv)
            refs.append(o)
            ref_l.append(l)
            outs.append(out[t])
            lses.append(lse[t])
            if n_checked % exact_every == 0:
                rows = torch.cat([rows_o, rows_c]).double().numpy()
                e, _ = one_shot_reference(q_flat[t].cpu().double().numpy(), rows,
                                          sinks.double().numpy(), kw["softmax_scale"])
                ex.append(e[:, :dv])
                ex_ref.append(o)
                ex_out.append(out[t])
            n_checked += 1
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()
    err = check_strict(torch.stack(outs), torch.stack(refs), torch.stack(lses), torch.stack(ref_l))
    acc = check_vs_exact(torch.stack(ex_out), torch.stack(ex_ref), np.stack(ex))
    return n_checked, err, acc


@requires_gpu
@pytest.mark.parametrize("name", [
    "swa_decode_b32_h64",
    "swa_topk_decode_b32_h64_k512",
    "mla_decode_b64_h128_k2048",
    "mla_mtp_decode_b64_h128_k2048",
    "mla_fp8_decode_t128_h128_k2048",
])
def test_benchmark_configuration_full_size(name):
    _say(f"{name} at full size")
    kw = gen.build_workload(name, device="cuda", seed=21)
    out, lse = sparse_flash_mla(**kw, return_softmax_lse=True)
    torch.cuda.synchronize()
    n, err, acc = _check_all_rows(kw, out, lse)
    _say(f"{name}: {n} query rows; max |out - golden| {err['out_max_abs']:.3g}, "
         f"max |lse - golden| {err['lse_max_abs']:.3g}; max |out - exact| {acc['ours']:.3g} "
         f"(golden {acc['golden']:.3g})")
