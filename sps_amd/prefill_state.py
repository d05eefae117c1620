"""Prefill -> decode state materialisation in one launch per layer.

The reference copies each batch row's current document into the decode caches with a host loop
(``_materialize_prefill_layer_state``, reverse_sps/inference.py:568-613): the retained buffer gets
every token of the document from the retained slot's rows, the ring the last ``window_tokens``
tokens from the window slot's rows, and the lengths are set (ring position 0). Here the whole batch
is one kernel (``sps_prefill_to_decode``), and ``materialize_prefill_layer_state`` keeps the
method's signature so it can replace it on the reference's inference classes.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _native as N

_FLOAT_DTYPES = {torch.bfloat16: N.DTYPE_BF16, torch.float16: N.DTYPE_F16, torch.float32: N.DTYPE_F32}
_LEN_DTYPES = {torch.int32: N.DTYPE_I32, torch.int64: N.DTYPE_I64}


def _aligned(t: Tensor) -> bool:
    el = t.element_size()
    return t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all((s * el) % 16 == 0 for s in t.stride()[:-1])


def prefill_to_decode(k_Bx2TxHxD: Tensor, v_Bx2TxHxD: Tensor, current_doc_mask_BxT: Tensor, *, window_slot: int,
                      retained_slot: int, nw_k: Tensor, nw_v: Tensor, nw_len: Tensor, nw_pos: Tensor,
                      br_k: Tensor, br_v: Tensor, br_len: Tensor, window_tokens: int) -> None:
    """Writes one layer's decode caches from the prefill K/V (in place). Shapes: K/V [B, 2T, H, D];
    mask [B, T] bool; ring caches [B, H, Sw, D] with lengths/positions [B]; retained caches
    [B, H, Sr, D] with lengths [B, H]. The ring tensors are ignored when window_tokens <= 0."""
    b, two_t, h, d = k_Bx2TxHxD.shape
    t = two_t // 2
    assert two_t == 2 * t and v_Bx2TxHxD.shape == k_Bx2TxHxD.shape
    assert current_doc_mask_BxT.shape == (b, t), f"mask {tuple(current_doc_mask_BxT.shape)} vs ({b}, {t})"
    assert br_k.shape[:2] == (b, h) and br_k.shape[3] == d and br_v.shape == br_k.shape
    assert br_len.shape == (b, h)
    window_tokens = int(window_tokens)
    use_ring = window_tokens > 0
    if use_ring:
        assert nw_k.shape[:2] == (b, h) and nw_k.shape[3] == d and nw_v.shape == nw_k.shape
        assert nw_len.shape == (b,) and nw_pos.shape == (b,)
        assert window_tokens <= nw_k.size(2), "window_tokens exceeds the ring storage"
    assert k_Bx2TxHxD.dtype in _FLOAT_DTYPES and v_Bx2TxHxD.dtype == k_Bx2TxHxD.dtype
    assert br_k.dtype in _FLOAT_DTYPES and (not use_ring or nw_k.dtype == br_k.dtype)
    assert br_len.dtype in _LEN_DTYPES and (not use_ring or (nw_len.dtype == br_len.dtype and nw_pos.dtype == br_len.dtype))
    assert d % 8 == 0, f"head_dim {d} must be a multiple of 8"
    assert k_Bx2TxHxD.is_cuda and br_k.is_cuda, "prefill_to_decode: tensors must be on the GPU"
    # The reference's slice assignment fails when a document does not fit the retained buffer. A
    # document has at most T tokens, so with a buffer of T rows or more this is a shape check; only a
    # shorter buffer needs the lengths read back (a host sync).
    if b and br_k.size(2) < t:
        longest = int(current_doc_mask_BxT.sum(dim=1).max())
        if longest > br_k.size(2):
            raise RuntimeError(f"a prompt document of {longest} tokens does not fit the retained buffer "
                               f"({br_k.size(2)} rows)")
    k = k_Bx2TxHxD if _aligned(k_Bx2TxHxD) else k_Bx2TxHxD.contiguous()
    v = v_Bx2TxHxD if _aligned(v_Bx2TxHxD) else v_Bx2TxHxD.contiguous()
    for c in (br_k, br_v) + ((nw_k, nw_v) if use_ring else ()):
        assert _aligned(c), "KV caches must have 16-byte aligned rows"
    # A bool mask with unit column stride is read in place (one byte per flag, 0 or 1).
    if current_doc_mask_BxT.dtype == torch.bool and current_doc_mask_BxT.stride(1) == 1:
        mask = current_doc_mask_BxT.view(torch.uint8)
    else:
        mask = current_doc_mask_BxT.to(torch.uint8).contiguous()
    cs = lambda x, y: N.i64_array((x.stride(0), x.stride(1), x.stride(2), y.stride(0), y.stride(1), y.stride(2)))  # noqa: E731
    if use_ring:
        ring = (nw_k.data_ptr(), nw_v.data_ptr(), cs(nw_k, nw_v), nw_k.size(2), window_tokens, nw_len.data_ptr(),
                nw_pos.data_ptr(), N.i64_array((nw_len.stride(0), nw_pos.stride(0))))
    else:
        ring = (None, None, N.i64_array((0,) * 6), 0, 0, None, None, N.i64_array((0, 0)))
    status = N.lib().sps_prefill_to_decode(
        b, t, h, d, _FLOAT_DTYPES[k.dtype], k.data_ptr(), N.i64_array((k.stride(0), k.stride(1), k.stride(2))),
        v.data_ptr(), N.i64_array((v.stride(0), v.stride(1), v.stride(2))), int(window_slot), int(retained_slot),
        mask.data_ptr(), mask.stride(0), _FLOAT_DTYPES[br_k.dtype], *ring,
        br_k.data_ptr(), br_v.data_ptr(), cs(br_k, br_v), br_k.size(2), br_len.data_ptr(),
        N.i64_array((br_len.stride(0), br_len.stride(1))), _LEN_DTYPES[br_len.dtype],
        torch.cuda.current_stream(k.device).cuda_stream)
    N.check("sps_prefill_to_decode", status)


def materialize_prefill_layer_state(self, state, layer_idx: int, k_Bx2TxHxD: Tensor, v_Bx2TxHxD: Tensor,
                                    current_doc_mask_BxT: Tensor) -> None:
    """Drop-in for the reference method (reverse_sps/inference.py:568-613): `self` supplies
    ``_window_slot_index`` / ``_retained_slot_index``, `state` the layer's ring (``normal_window``)
    and retained (``predict_retained``) caches and ``normal_window_tokens``."""
    nw, br = state.normal_window, state.predict_retained
    window = int(state.normal_window_tokens)
    prefill_to_decode(
        k_Bx2TxHxD, v_Bx2TxHxD, current_doc_mask_BxT, window_slot=self._window_slot_index,
        retained_slot=self._retained_slot_index,
        nw_k=nw.k[layer_idx] if window > 0 else None, nw_v=nw.v[layer_idx] if window > 0 else None,
        nw_len=nw.len[layer_idx] if window > 0 else None, nw_pos=nw.pos[layer_idx] if window > 0 else None,
        br_k=br.k[layer_idx], br_v=br.v[layer_idx], br_len=br.len[layer_idx], window_tokens=window)
