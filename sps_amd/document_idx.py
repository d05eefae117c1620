"""Document ids and left-padding helpers feeding the attention kernels' document mask.

Restates model.py:35-99 of lil-lab/sps (src/modeling/models/model.py): ``infer_is_real_tokens``,
``validate_left_padded_tokens``, ``compute_left_padded_position_ids`` and
``generate_left_padded_document_idx`` (an EOS ends the current document; left-pad tokens form
isolated fake documents 0..P-1 ahead of the real suffix). The SPS families repeat each token's id
for its input and <predict> positions (reverse_sps/core.py:226): ``interleave_document_idx``.
"""

from __future__ import annotations

import torch
from torch import Tensor


def infer_is_real_tokens(idx_BxT: Tensor, pad_token_id: int) -> Tensor:
    """Marks positions whose token is not the pad token."""
    return idx_BxT != pad_token_id


def validate_left_padded_tokens(is_real_BxT: Tensor, *, allow_all_pad: bool, context: str) -> None:
    """Raises ValueError unless every row is pad* real* (and, optionally, has a real token)."""
    is_real_BxT = is_real_BxT.to(dtype=torch.bool)
    ever_real = is_real_BxT.cumsum(dim=1) > 0
    has_pad_after_real = ((~is_real_BxT) & ever_real).any(dim=1)
    if bool(has_pad_after_real.any()):
        bad_rows = has_pad_after_real.nonzero(as_tuple=False).flatten().tolist()
        raise ValueError(
            f"{context} must be left padded only; found pad tokens after real tokens in rows {bad_rows}"
        )
    if not allow_all_pad:
        empty_rows = is_real_BxT.sum(dim=1) == 0
        if bool(empty_rows.any()):
            bad_rows = empty_rows.nonzero(as_tuple=False).flatten().tolist()
            raise ValueError(f"{context} must contain at least one real token per row; empty rows: {bad_rows}")


def compute_left_padded_position_ids(is_real_BxT: Tensor) -> Tensor:
    """Consecutive positions for real tokens, 0 at pad positions."""
    is_real_BxT = is_real_BxT.to(dtype=torch.bool)
    cumsum = is_real_BxT.long().cumsum(dim=1) - 1
    return torch.where(is_real_BxT, cumsum, torch.zeros_like(cumsum))


def generate_left_padded_document_idx(idx_BxT: Tensor, *, eos_token_id: int, pad_token_id: int) -> Tensor:
    """Document ids: real token t gets pad_count + (number of real EOS strictly before t); the
    i-th pad token gets id i, so pads never share a document with real tokens."""
    is_real_BxT = infer_is_real_tokens(idx_BxT, pad_token_id)
    validate_left_padded_tokens(is_real_BxT, allow_all_pad=True, context="document index inputs")
    b, t = idx_BxT.shape
    pad_count_Bx1 = (~is_real_BxT).sum(dim=1, keepdim=True)
    is_real_eos_BxT = is_real_BxT & (idx_BxT == eos_token_id)
    eos_before = torch.zeros((b, t), dtype=idx_BxT.dtype, device=idx_BxT.device)
    if t > 1:
        eos_before[:, 1:] = torch.cumsum(is_real_eos_BxT[:, :-1], dim=1, dtype=idx_BxT.dtype)
    real_ids = eos_before + pad_count_Bx1.to(dtype=idx_BxT.dtype)
    pad_ids = torch.clamp(torch.cumsum((~is_real_BxT).long(), dim=1) - 1, min=0).to(dtype=idx_BxT.dtype)
    return torch.where(is_real_BxT, real_ids, pad_ids)


def interleave_document_idx(documents_idx_BxT: Tensor) -> Tensor:
    """[B, T] token document ids -> [B, 2T] ids of the interleaved input/<predict> sequence."""
    return documents_idx_BxT.repeat_interleave(2, dim=1)
