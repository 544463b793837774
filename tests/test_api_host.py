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


def _fp8_call(**over):
    q = torch.zeros(1, 64, 576, dtype=torch.bfloat16)
    kv = torch.zeros(4, 64, 1, 656, dtype=torch.uint8)
    tbl = torch.zeros(1, 4, dtype=torch.int32)
    kw = dict(q=q, ori_kv=kv, ori_block_table=tbl, cmp_kv=kv, cmp_block_table=tbl,
              cmp_sparse_indices=torch.zeros(1, 1, 8, dtype=torch.int32),
              cu_seqlens_q=torch.tensor([0, 1], dtype=torch.int32),
              seqused_kv=torch.tensor([100], dtype=torch.int32),
              sinks=torch.zeros(64), softmax_scale=1 / 24, cmp_ratio=1, ori_win_left=-1)
    kw.update(over)
    return kw


def test_fp8_cache_gates():
    # well-formed fp8 call: passes validation, then has no CPU path
    with pytest.raises(RuntimeError):
        sparse_flash_mla(**_fp8_call())
    with pytest.raises(RuntimeError):
        sparse_flash_mla(**_fp8_call(), kv_cache_dtype="fp8_ds_mla")
    with pytest.raises(ValueError):                      # unknown format name
        sparse_flash_mla(**_fp8_call(), kv_cache_dtype="fp8_e5m2")
    with pytest.raises(ValueError):                      # fp16 queries
        sparse_flash_mla(**_fp8_call(q=torch.zeros(1, 64, 576, dtype=torch.float16)))
    with pytest.raises(ValueError):                      # D = 512 queries
        sparse_flash_mla(**_fp8_call(q=torch.zeros(1, 64, 512, dtype=torch.bfloat16)))
    kv = torch.zeros(4, 64, 1, 576, dtype=torch.uint8)   # not 656-byte rows
    with pytest.raises(ValueError):
        sparse_flash_mla(**_fp8_call(ori_kv=kv, cmp_kv=kv))
    kv = torch.zeros(4, 64, 1, 656, dtype=torch.bfloat16)  # bf16 tensor named fp8
    with pytest.raises(ValueError):
        sparse_flash_mla(**_fp8_call(ori_kv=kv, cmp_kv=kv), kv_cache_dtype="fp8_ds_mla")


def test_short_length_and_table_tensors(swa_case, scfa_case):
    # the kernels read seqused_kv[b] and table row b for every sequence b: a shorter
    # tensor is rejected on the host before anything reaches the device
    nb = swa_case["cu_seqlens_q"].numel() - 1
    with pytest.raises(ValueError):
        sparse_attn_sharedkv(**dict(swa_case, seqused_kv=swa_case["seqused_kv"][: nb - 1]))
    with pytest.raises(ValueError):
        sparse_attn_sharedkv(**dict(swa_case, ori_block_table=swa_case["ori_block_table"][: nb - 1]))
    with pytest.raises(ValueError):
        sparse_attn_sharedkv(**dict(scfa_case,
                                    cmp_block_table=scfa_case["cmp_block_table"][: nb - 1]))


def test_fp8_qk_needs_fp8_rows(swa_case):
    # the fp8 Q·Kᵀ form reads e4m3 cache rows: on native rows it is a ValueError
    with pytest.raises(ValueError, match="fp8_qk"):
        sparse_attn_sharedkv(**dict(swa_case), fp8_qk=True)
