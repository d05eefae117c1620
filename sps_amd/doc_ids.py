"""Document ids for the attention path, computed on the GPU (``sps_document_ids``).

The modeling code derives its document-mask ids from token ids (model.py:70-99 of lil-lab/sps, under
src/modeling/models/) and the SPS callers repeat each id for the token's input and <predict>
positions (reverse_sps/core.py:218-227). ``document_ids`` does both in one launch and returns the ids
the attention entry points take as ``documents_idx_BxT``; ``left_padded_document_ids`` keeps the
modeling function's keyword signature for the drop-in (integration.py), with the same ValueError on
rows that are not left padded.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _native as N

_INT_CODES = {torch.int32: N.DTYPE_I32, torch.int64: N.DTYPE_I64}


def document_ids(idx_BxT: Tensor, *, eos_token_id: int, pad_token_id: int, repeat: int = 2,
                 dtype: torch.dtype | None = None, validate: bool = True) -> Tensor:
    """Ids of the documents the tokens of ``idx_BxT`` ([B, T] int32/int64, on the GPU) belong to.

    A real token (not ``pad_token_id``) belongs to document pad_count + (real EOS tokens before it);
    the i-th left pad is its own document i. ``repeat=2`` returns [B, 2T] ids for the interleaved
    input/<predict> sequence, ``repeat=1`` [B, T]. ``validate`` raises ValueError when a row has a pad
    token after a real one (this reads one flag per row back to the host)."""
    if idx_BxT.dim() != 2:
        raise ValueError(f"token ids must be [B, T], got shape {tuple(idx_BxT.shape)}")
    if not idx_BxT.is_cuda:
        raise RuntimeError("sps_amd document_ids runs on the GPU only (got a CPU tensor)")
    if idx_BxT.dtype not in _INT_CODES:
        raise TypeError(f"token ids must be int32 or int64, got {idx_BxT.dtype}")
    tok = idx_BxT if idx_BxT.stride(1) == 1 else idx_BxT.contiguous()
    b, t = tok.shape
    out_dtype = dtype or tok.dtype
    if out_dtype not in _INT_CODES:
        raise TypeError(f"document ids must be int32 or int64, got {out_dtype}")
    out = torch.empty((b, t * repeat), dtype=out_dtype, device=tok.device)
    bad = torch.zeros((b,), dtype=torch.int32, device=tok.device) if validate else None
    status = N.lib().sps_document_ids(
        b, t, tok.data_ptr(), _INT_CODES[tok.dtype], tok.stride(0) if b > 1 else t, int(eos_token_id),
        int(pad_token_id), int(repeat), out.data_ptr(), _INT_CODES[out_dtype], out.stride(0) if b > 1 else t * repeat,
        bad.data_ptr() if bad is not None else None, torch.cuda.current_stream(tok.device).cuda_stream)
    N.check("sps_document_ids", status)
    if bad is not None:
        rows = bad.nonzero().flatten().tolist()
        if rows:
            raise ValueError(f"token rows {rows} are not left padded: a pad token follows a real token")
    return out


def left_padded_document_ids(idx_BxT: Tensor, *, eos_token_id: int, pad_token_id: int) -> Tensor:
    """[B, T] document ids in the token dtype, keyword signature of the modeling code's id function."""
    return document_ids(idx_BxT, eos_token_id=eos_token_id, pad_token_id=pad_token_id, repeat=1)
