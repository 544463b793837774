"""Host-side behaviour of the drop-in API on CPU tensors (no launch happens).

The reference raises before any launch: AssertionError for unsupported masks /
layouts / missing TND cu_seqlens / top-k mismatch / metadata size, ValueError
for dtypes and shapes (api.py:186-191, :209, :248-250, :279-282, :362-364,
:51-56). The same conditions raise the same types here; a well-formed call on
CPU tensors raises RuntimeError because there is no CPU compute path.
"""

import pytest
import torch

from oracle import gen
from sparse_attn_sharedkv_amd import sparse_attn_sharedkv, sparse_flash_mla


@pytest.fixture(scope="module")
def swa_case():
    return gen.build_case(gen.REFERENCE_CASES["swa_decode"], torch.bfloat16)


@pytest.fixture(scope="module")
def scfa_case():
    return gen.build_case(gen.REFERENCE_CASES["scfa_decode"], torch.bfloat16)


@pytest.mark.parametrize("bad", [dict(ori_mask_mode=3), dict(ori_win_right=1),
                                 dict(layout_kv="BSND"), dict(layout_q="BNSD")])
def test_assertions(swa_case, bad):
    with pytest.raises(AssertionError):
        sparse_attn_sharedkv(**dict(swa_case, **bad))


def test_tnd_needs_cu_seqlens(swa_case):
    with pytest.raises(AssertionError):
        sparse_attn_sharedkv(**dict(swa_case, cu_seqlens_q=None))


def test_topk_mismatch(scfa_case):
    with pytest.raises(AssertionError):
        sparse_attn_sharedkv(**dict(scfa_case, topk_cmp=7))


def test_metadata_size(swa_case):
    with pytest.raises(AssertionError):
        sparse_attn_sharedkv(**dict(swa_case), metadata=torch.zeros(1024, dtype=torch.int32))


def test_dtype(swa_case):
    with pytest.raises(ValueError):
        sparse_attn_sharedkv(**dict(swa_case, q=swa_case["q"].float()))


@pytest.mark.parametrize("bad_heads", [48 + 8, 256])
def test_head_count_gate(swa_case, bad_heads):
    q = torch.zeros(1, bad_heads, 512, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        sparse_attn_sharedkv(**dict(swa_case, q=q, sinks=torch.zeros(bad_heads)))


def test_head_dim_gate(swa_case):
    q = torch.zeros(1, 64, 256, dtype=torch.bfloat16)
    kv = torch.zeros(4, 128, 1, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        sparse_attn_sharedkv(**dict(swa_case, q=q, ori_kv=kv))
    with pytest.raises(ValueError):
        sparse_attn_sharedkv(**dict(swa_case), head_dim_v=576)


def test_no_cpu_path(swa_case, scfa_case):
    with pytest.raises(RuntimeError):
        sparse_attn_sharedkv(**swa_case)
    with pytest.raises(RuntimeError):
        sparse_flash_mla(**{k: v for k, v in scfa_case.items()})
