"""``sparse_flash_mla`` (signature of sparse_flash_mla/sparse_flash_mla_api.py:94-117).

Same computation as ``sparse_attn_sharedkv`` without the ``metadata``
argument: the schedule is always built on the host from the inputs. The
reference twin only runs D = 512; for MLA rows (d_qk = 576 = 512 latent +
64 rope) the value part is the 512-wide latent, so ``head_dim_v`` defaults
to 512 here (identical to the reference's behaviour at D = 512).
"""

from __future__ import annotations

from typing import Optional, Tuple, Union

import torch

from .api import DEFAULT_BLOCK_I, finalize, launch, prepare  # noqa: F401
from .metadata import DEFAULT_CORE_NUM


def sparse_flash_mla(
    q: torch.Tensor,
    *,
    ori_kv: torch.Tensor,
    cmp_kv: Optional[torch.Tensor] = None,
    cmp_sparse_indices: Optional[torch.Tensor] = None,
    ori_block_table: torch.Tensor,
    cmp_block_table: Optional[torch.Tensor] = None,
    cu_seqlens_q: Optional[torch.Tensor] = None,
    seqused_q: Optional[torch.Tensor] = None,
    seqused_kv: torch.Tensor,
    sinks: torch.Tensor,
    softmax_scale: float,
    cmp_ratio: Optional[int] = None,
    ori_mask_mode: int = 4,
    cmp_mask_mode: int = 3,
    ori_win_left: int = 127,
    ori_win_right: int = 0,
    layout_q: str = "TND",
    layout_kv: str = "PA_ND",
    return_softmax_lse: bool = False,
    core_num: int = DEFAULT_CORE_NUM,
    topk_cmp: Optional[int] = None,
    head_dim_v: Optional[int] = 512,
    kv_cache_dtype: Optional[str] = None,
    schedule: Optional[str] = None,
    fp8_qk: bool = False,
) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """Sparse flash-MLA forward: ``attention_out`` (and lse) in q's layout.

    ``fp8_qk``: as in ``sparse_attn_sharedkv`` (fp8 caches: Q·Kᵀ on fp8 MFMA).
    """
    prep = prepare(q, ori_kv=ori_kv, cmp_kv=cmp_kv, cmp_sparse_indices=cmp_sparse_indices,
                   ori_block_table=ori_block_table, cmp_block_table=cmp_block_table,
                   cu_seqlens_q=cu_seqlens_q, seqused_q=seqused_q, seqused_kv=seqused_kv,
                   sinks=sinks, metadata=None, softmax_scale=softmax_scale,
                   cmp_ratio=cmp_ratio, ori_mask_mode=ori_mask_mode,
                   cmp_mask_mode=cmp_mask_mode, ori_win_left=ori_win_left,
                   ori_win_right=ori_win_right, layout_q=layout_q, layout_kv=layout_kv,
                   core_num=core_num, topk_cmp=topk_cmp, head_dim_v=head_dim_v,
                   kv_cache_dtype=kv_cache_dtype, schedule=schedule, fp8_qk=fp8_qk,
                   _stream_schedule=True)
    launch(prep)
    return finalize(prep, return_softmax_lse)
