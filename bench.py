#!/usr/bin/env python
"""Benchmark: DeepSeek-V3.2-shape sparse MLA decode on one MI355X.

Workload (default ``mla_decode_b64_h128_k2048``): B=64 sequences, one query
row each, H=128 heads, d_qk=576 (512 latent + 64 rope), d_v=512, bf16 q and
paged KV (block 64) ~ N(0,1)*0.5, ctx 32768, top-k 2048 rows per query, no
sink; split-KV schedule + LSE merge kernel. A "step" is one call (attention
kernel + merge kernel) over one input set. Four independent input sets (own pool,
block tables, top-k sets, q) rotate so the 256 MB Infinity Cache cannot hold
the gathered rows between calls. Inputs are resident in HBM and the schedule
is precomputed before the timed region.

Other workloads (``--workload``): the MTP and fp8 long-context decode shapes
(the fp8 one with its Q·Kᵀ on fp8 MFMA with e4m3 queries and bf16 P·V by
default, as the configuration names it; ``--qk bf16`` runs bf16 queries on the
dequantized rows instead),
and the reference's own 8K prefill test shapes (``swa_prefill_t8192_h64``,
``cfa_prefill_t8192_h64``, ``scfa_prefill_t8192_h64``: H=64, d=512, block 128),
whose ``roofline`` counts q, out and the distinct cache rows once (the rows are
re-read by up to 128 consecutive query rows and stay on chip) and is rated
against HBM or the bf16 MFMA peak, whichever bounds the shape.

Prints one JSON line. ``value`` is TFLOP/s of the whole call; the
``roofline`` object rates the attention kernel alone: algorithmic bytes per
launch / its mean duration (HIP events around each launch in the timed loop)
against 8 TB/s HBM. ``profiled_counters`` repeats the MFMA / VALU / LDS activity
of the same kernel and workload from the committed rocprofv3 SQ counter summary
(``profiles/attn_kernel_<workload>_sq.txt``). ``cpu_baseline`` times the CPU
restatement of the reference's golden math on this host over query rows of one
input set.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = ("sparse-attn decode TFLOP/s + gathered-KV HBM GB/s (% roofline), µs/call")
HBM_PEAK_GBPS = 8000.0        # MI355X HBM3E
BF16_PEAK_TFLOPS = 2516.6     # MI355X dense bf16 MFMA
# The reference's own published timings for a workload of the same shape (other
# hardware; context, not a ratio: the metric differs)
REFERENCE_PUBLISHED = {
    "swa_prefill_t8192_h64": {
        "ascend_c_kernel_us": 1838, "tilelang_kernel_us": 5330, "hardware": "Ascend 910B",
        "source": "compiler_changes/003-ascend-copy-pa-paged-kv-load.md:20-33"},
}


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=2000,
                    help="untimed calls first (the GPU reaches its sustained clocks after ~100 ms of load)")
    ap.add_argument("--workload", default="mla_decode_b64_h128_k2048")
    ap.add_argument("--sets", type=int, default=4)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--qk", choices=("auto", "bf16", "fp8"), default="auto",
                    help="Q·Kᵀ form over fp8 cache rows: fp8 MFMA with e4m3 queries (fp8) or "
                         "bf16 MFMA on the dequantized rows (bf16); auto = fp8, the form the "
                         "long-context fp8 configuration names (level with bf16 or up to 2 %% faster on MI355X "
                         "at 128 sequences, H=128, top-k 2048)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="after the benchmark, run 5 plain device copies of MIB MiB (the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    return ap.parse_args()


def summary_kernel(path):
    """The kernel a committed rocprofv3 summary measured: its ``# kernel:`` header line, else
    the ``sas::...`` name in its first line."""
    with open(path, encoding="utf-8") as f:
        lines = f.readlines()
    for line in lines:
        if line.startswith("# kernel:"):
            return line.split(":", 1)[1].strip()
    for tok in (lines[0].split() if lines else []):
        if tok.startswith("sas::"):
            return tok.rstrip(",")
    return None


def measured_traffic(workload, kernel):
    """HBM bytes per attention launch from the committed rocprofv3 PMC summary of ``kernel``,
    or None (no summary, or one of another kernel)."""
    path = os.path.join(ROOT, "profiles", f"attn_kernel_{workload}_pmc.txt")
    if not os.path.exists(path) or summary_kernel(path) != kernel:
        return None
    for line in open(path, encoding="utf-8"):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def kernel_source_sha16():
    """First 16 hex digits of the SHA-256 over the kernel sources (csrc/*.hip, *.h, *.cpp in
    name order): the fingerprint a counter summary records for the code it measured."""
    import hashlib

    d = os.path.join(ROOT, "sparse_attn_sharedkv_amd", "csrc")
    h = hashlib.sha256()
    for name in sorted(os.listdir(d)):
        if name.endswith((".hip", ".h", ".cpp")):
            h.update(name.encode())
            h.update(open(os.path.join(d, name), "rb").read())
    return h.hexdigest()[:16]


def profiled_counters(workload, kernel):
    """MFMA / VALU / LDS activity of the attention kernel from the committed rocprofv3 SQ
    counter summary (``profiles/attn_kernel_<workload>_sq.txt``), or None.

    The summary's header names the kernel it measured (``# kernel: ...``) and the
    fingerprint of the sources it was built from (``# source_sha16: ...``). A summary of
    another kernel is not used; one whose fingerprint differs from the current sources
    is reported with ``"stale": true``."""
    path = os.path.join(ROOT, "profiles", f"attn_kernel_{workload}_sq.txt")
    if not os.path.exists(path):
        return None
    out = {}
    meta = {"kernel": summary_kernel(path)}
    for line in open(path, encoding="utf-8"):
        if line.startswith("# source_sha16:") or line.startswith("# measured_commit:"):
            key, val = line[1:].split(":", 1)
            meta[key.strip()] = val.strip()
            continue
        if ":" in line and not line.startswith("#"):
            key, val = line.split(":", 1)
            key = key.strip()
            if key in ("mfma_busy_frac", "valu_active_frac", "lds_active_frac",
                       "valu_insts_per_wave_per_tile", "lds_bank_conflict_frac"):
                try:
                    out[key] = float(val.split()[0])
                except ValueError:
                    pass
    if not out or meta.get("kernel") != kernel:
        return None
    out["source"] = os.path.relpath(path, ROOT)
    out["measured_commit"] = meta.get("measured_commit")
    out["source_sha16"] = meta.get("source_sha16")
    out["stale"] = meta.get("source_sha16") != kernel_source_sha16()
    return out


def cpu_baseline(inputs, counts, max_tokens=64, fp8_qk=False, budget_s=20.0):
    """Golden-faithful CPU restatement (oracle/) over the query rows of one input set.

    Times up to ``max_tokens`` rows (all of them for the benchmark workloads up to
    64 tokens; fewer when one row takes long enough that three passes would
    exceed about ``budget_s`` seconds) and scales the rate to the whole call
    (FLOPs of the rows timed).
    """
    import torch

    from oracle.golden_ref import attend_token, attend_token_fp8qk, token_layout, token_rows
    from sparse_attn_sharedkv_amd.workloads import flops_and_bytes

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    kw = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in inputs.items()}
    q = kw["q"]
    n1, d = q.shape[-2], q.shape[-1]
    nb, _, prefix, act_q = token_layout(kw["layout_q"], q.shape, kw.get("cu_seqlens_q"))
    q_flat = q.reshape(-1, n1, d)
    lens = kw["seqused_kv"].tolist()
    idx = kw["cmp_sparse_indices"]
    idx_flat = None if idx is None else idx.reshape(q_flat.shape[0], -1)
    every = [(b, s) for b in range(nb) for s in range(act_q[b])]

    def one_row(b, s):
        t = prefix[b] + s
        ori, cmp = token_rows(
            b=b, s=s, act_q=act_q[b], act_kv=lens[b], ori_kv=kw["ori_kv"],
            ori_block_table=kw["ori_block_table"], cmp_kv=kw["cmp_kv"],
            cmp_block_table=kw["cmp_block_table"],
            cmp_idx_row=None if idx_flat is None else idx_flat[t].tolist(),
            cmp_ratio=kw["cmp_ratio"], ori_win_left=kw["ori_win_left"],
            kv_cache_dtype=kw.get("kv_cache_dtype"), raw=fp8_qk)
        (attend_token_fp8qk if fp8_qk else attend_token)(
            q_flat[t], [ori, cmp], kw["sinks"], kw["softmax_scale"], d_v=kw["head_dim_v"])
        return ori.shape[0] + cmp.shape[0]

    # bound the sample: one untimed row sizes it to about budget_s for three passes
    t0 = time.perf_counter()
    one_row(*every[len(every) // 2])
    per_row = time.perf_counter() - t0
    n = max(2, min(max_tokens, int(budget_s / (3 * max(per_row, 1e-6)))))
    step = max(1, len(every) // n)  # evenly spaced sample (prefill rows differ in length)
    rows = every[::step][:n]
    times = []
    attended = 0
    for rep in range(3):
        t0 = time.perf_counter()
        for b, s in rows:
            got = one_row(b, s)
            if rep == 0:
                attended += got
        times.append(time.perf_counter() - t0)
        print(f"[bench] cpu baseline pass {rep + 1}/3: {len(rows)} rows, {times[-1]:.1f} s",
              file=sys.stderr, flush=True)
    sec = sorted(times)[1]
    flops, _ = flops_and_bytes(counts)
    share = attended / max(counts["rows"], 1)  # FLOP share of the sampled rows
    fp8 = (" (fp8 rows: e4m3 Q·Kᵀ scores in float64, dequantized values)" if fp8_qk else
           " (fp8 rows dequantized on the CPU)" if kw.get("kv_cache_dtype") else "")
    return {"value": round(flops * share / sec / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port", "us_per_call": round(sec / share * 1e6, 1),
            "sample": f"{len(rows)} of {counts['tokens']} query rows of one input set, evenly "
                      f"spaced ({attended} attended rows; paged gather{fp8} + 512-row online "
                      f"softmax, torch fp32), median of 3, scaled to the call by FLOPs"}


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: this library has no multi-GPU path "
              f"(asked for --gpus {args.gpus}, WORLD_SIZE={world})", file=sys.stderr)
        sys.exit(2)

    import torch

    from sparse_attn_sharedkv_amd import api
    from sparse_attn_sharedkv_amd.workloads import (WORKLOADS, build_workload, flops_and_bytes,
                                                    workload_counts)

    assert torch.cuda.is_available(), "bench.py needs a ROCm GPU"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    w = WORKLOADS[args.workload]
    sets = [build_workload(args.workload, device=dev, seed=100 + i) for i in range(args.sets)]
    counts = workload_counts(sets[0])
    flops, nbytes = flops_and_bytes(counts)
    fp8_rows = sets[0].get("kv_cache_dtype") is not None
    fp8_qk = fp8_rows and args.qk in ("auto", "fp8")
    if args.qk == "fp8" and not fp8_rows:
        print("--qk fp8 needs a workload with fp8 cache rows", file=sys.stderr)
        sys.exit(2)
    # committed profile summaries are named for the workload (and the Q·Kᵀ form)
    prof_key = args.workload + ("_fp8qk" if fp8_qk else "")
    preps = []
    for kw in sets:
        call = {k: v for k, v in kw.items()}
        preps.append(api.prepare(**call, fp8_qk=fp8_qk))
    torch.cuda.synchronize()

    k, wu = args.steps, args.warmup
    for i in range(wu):
        api.launch(preps[i % len(preps)])
    torch.cuda.synchronize()

    # timed region 1: K whole calls (one C-ABI launch each: attention + merge kernels)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for i in range(k):
        api.launch(preps[i % len(preps)])
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = e0.elapsed_time(e1) / k

    # timed region 2: the attention kernel alone, then the merge kernel alone, HIP
    # events around every launch (on torch's current stream, which the events record on)
    def per_launch(phases):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * k)]
        torch.cuda.synchronize()
        for i in range(k):
            ev[2 * i].record()
            api.launch(preps[i % len(preps)], phases=phases)
            ev[2 * i + 1].record()
        torch.cuda.synchronize()
        return sorted(ev[2 * i].elapsed_time(ev[2 * i + 1]) for i in range(k))

    attn_ms = per_launch(1)
    # split items are merged by the merge kernel, or inside the attention kernel
    # (native rows): then the attention launch includes the merge
    # (the 128-head kernel on either row format, the native-row kernel)
    merge_in_attn = preps[0].merge_in_kernel and (
        preps[0].args.m_base == 128 or not sets[0].get("kv_cache_dtype"))
    has_merge = preps[0].args.num_fd > 0 and not merge_in_attn
    merge_ms = per_launch(2) if has_merge else [0.0] * k  # no merge kernel
    attn_avg = sum(attn_ms) / k
    merge_avg = sum(merge_ms) / k
    srt = attn_ms

    achieved = nbytes / (attn_avg * 1e-3) / 1e9
    # items of 128 heads run on the 128-head kernel (either row format); smaller
    # items on the pipelined kernel for fp8 rows, else the one-wave-per-SIMD kernel
    kernel = ("sas::wide_kernel" if preps[0].args.m_base == 128 or api.uses_row_pairs(preps[0])
              else "sas::attn3_kernel" if sets[0].get("kv_cache_dtype") else "sas::attn2_kernel")
    if w.get("prefill"):
        # prefill: consecutive query rows re-read each other's cache rows, which
        # stay on chip; the algorithmic HBM bytes are q, out and lse once plus the
        # distinct rows. The bound is whichever of HBM and MFMA time is larger.
        from sparse_attn_sharedkv_amd.workloads import prefill_hbm_bytes
        pbytes = prefill_hbm_bytes(sets[0], counts)
        t_hbm, t_mfma = pbytes / (HBM_PEAK_GBPS * 1e9), flops / (BF16_PEAK_TFLOPS * 1e12)
        if t_hbm >= t_mfma:
            ach = pbytes / (attn_avg * 1e-3) / 1e9
            roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS,
                    "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBPS, 4),
                    "traffic": measured_traffic(prof_key, kernel), "algorithmic_bytes": int(pbytes),
                    "kernel": kernel}
        else:
            ach = flops / (attn_avg * 1e-3) / 1e12
            roof = {"bound": "mfma", "achieved": round(ach, 1), "peak": BF16_PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(ach / BF16_PEAK_TFLOPS, 4),
                    "traffic": measured_traffic(prof_key, kernel), "algorithmic_bytes": int(pbytes),
                    "kernel": kernel}
        roof["hbm_time_us"] = round(t_hbm * 1e6, 1)
        roof["mfma_time_us"] = round(t_mfma * 1e6, 1)
    else:
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                "traffic": measured_traffic(prof_key, kernel), "algorithmic_bytes": int(nbytes),
                "kernel": kernel}
    res = {
        "metric": METRIC,
        "value": round(flops / (ms_step * 1e-3) / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": k,
        "warmup": wu,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("bf16" if not fp8_rows else
                  "fp8 e4m3 Q·Kᵀ, bf16 P·V (fp8 e4m3 KV rows)" if fp8_qk else
                  "bf16 (fp8 e4m3 KV rows)"),
        "data": "synthetic",
        "config": {"workload": args.workload, "batch": w["B"], "s_q": w["S"], "heads": w["H"],
                   "d_qk": w["D"], "d_v": w["DV"], "topk": w["K"], "ctx": list(w["ctx"]),
                   "block_size": w.get("block", 64), "input_sets": len(preps),
                   "tokens": counts["tokens"],
                   "attended_rows": counts["rows"], "layout_q": sets[0]["layout_q"],
                   "kv_row_bytes": counts["row_bytes"],
                   "qk": "fp8" if fp8_qk else "bf16"},
        "us_per_call": round(ms_step * 1e3, 2),
        "gathered_kv_GBps_call": round(counts["rows"] * counts["row_bytes"] / (ms_step * 1e-3)
                                       / 1e9, 1),
        "hbm_roofline_frac_call": round(nbytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
        "mfma_frac_call": round(flops / (ms_step * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
        "attn_kernel_us": {"mean": round(attn_avg * 1e3, 2), "p10": round(srt[k // 10] * 1e3, 2),
                           "p50": round(srt[k // 2] * 1e3, 2),
                           "p90": round(srt[(9 * k) // 10] * 1e3, 2)},
        "merge_kernel_us": round(merge_avg * 1e3, 2),
        "split_items_merged": ("in the attention kernel" if merge_in_attn and
                               preps[0].args.num_fd > 0 else
                               "by the merge kernel" if has_merge else "no split items"),
        "host_wall_us_per_step": round(wall / k * 1e6, 2),
        "timing": "value/ms_per_step: K whole calls between two events; attn_kernel_us and "
                  "merge_kernel_us: events around each of K separate launches",
        "roofline": roof,
        "peaks": {"hbm_GBps": HBM_PEAK_GBPS, "bf16_mfma_TFLOPs": BF16_PEAK_TFLOPS},
    }
    prof = profiled_counters(prof_key, kernel)
    if prof is not None:
        res["profiled_counters"] = prof
    if args.workload in REFERENCE_PUBLISHED:
        res["reference_published"] = REFERENCE_PUBLISHED[args.workload]
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(sets[0], counts, fp8_qk=fp8_qk)
    print(json.dumps(res), flush=True)
    if args.calibrate_copy > 0:
        n = args.calibrate_copy << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"calibration: 5 device copies of {n} bytes", file=sys.stderr, flush=True)


if __name__ == "__main__":
    main()
