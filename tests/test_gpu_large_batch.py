"""More than 64 sequences per call on native bf16 rows.

Up to 64 sequences the attention kernels hold every sequence's lengths and
query offset in one lane each; beyond that they load them per item
(golden.py:116-125 gives every sequence its own lengths either way). These
cases run that second path:

* the 128-head top-k decode shape (H = 128, top-k 2048 of 4096 rows) and the
  64-head sliding-window decode shape (window 128, contexts U[2048, 8192]) at
  96 and 128 sequences, every query row checked against the oracle under the
  benchmark bound (``check_strict``);
* gathered rows pinned exactly at 96 and 128 sequences (q = 0, sinks -inf,
  one-hot V rows, as in ``test_gpu_index_exact``): a window of two rows and a
  two-slot top-k list per sequence over block-size-1 caches, every sequence of
  another length, so a length or offset read for the wrong sequence shows as a
  wrong row.
"""

import sys

import numpy as np
import pytest
import torch

from oracle import gen
from oracle.checks import check_strict
from oracle.golden_ref import sparse_attn_oracle

pytestmark = pytest.mark.gpu

HAS_GPU = torch.cuda.is_available()
requires_gpu = pytest.mark.skipif(not HAS_GPU, reason="needs a ROCm GPU")

if HAS_GPU:
    from sparse_attn_sharedkv_amd import sparse_flash_mla

from test_gpu_index_exact import _case, _check  # noqa: E402


def _say(msg):
    print(f"[gpu-large-batch] {msg}", flush=True)
    sys.stdout.flush()


@requires_gpu
@pytest.mark.parametrize("batch", [96, 128])
@pytest.mark.parametrize("name,ctx", [("mla_decode_b64_h128_k2048", 4096),
                                      ("swa_decode_b32_h64", None)])
def test_many_sequences_against_oracle(name, ctx, batch):
    _say(f"{name} with {batch} sequences")
    kw = gen.build_workload(name, device="cuda", seed=200 + batch, batch=batch,
                            ctx_override=[ctx] * batch if ctx else None)
    out, lse = sparse_flash_mla(**kw, return_softmax_lse=True)
    torch.cuda.synchronize()
    assert out.shape[0] == batch
    okw = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()
           if k != "topk_cmp"}
    ref, ref_lse = sparse_attn_oracle(**okw)
    err = check_strict(out.cpu(), ref, lse.cpu(), ref_lse)
    _say(f"{name} B={batch}: max |out - oracle| {err['out_max_abs']:.3g}")


@requires_gpu
@pytest.mark.parametrize("heads", [64, 128])
@pytest.mark.parametrize("batch", [96, 128])
def test_many_sequences_rows_exact(batch, heads):
    _say(f"rows exact, {batch} sequences, H={heads}")
    rng = np.random.default_rng(300 + batch)
    kvlens = [int(x) for x in rng.permutation(np.arange(40, 40 + 7 * batch, 7))]
    kw, idx, t1, t2 = _case(scenario=3, layout="BSND", qlens=[1] * batch, kvlens=kvlens,
                            heads=heads, d=576, win=1, ratio=1, k=2, bs1=1, bs2=1,
                            seed=300 + batch)
    _check(kw, idx, t1, t2, 3, 1, 1, 1)
