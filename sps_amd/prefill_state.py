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


def _rows16(ptr: int, strides: tuple, el: int) -> bool:
    """For a 4-D tensor: unit last stride, and every row start 16-byte aligned (base and the three
    outer strides; with a power-of-two element size, one test of the strides' OR covers all three)."""
    s0, s1, s2, s3 = strides
    return s3 == 1 and ptr % 16 == 0 and ((s0 | s1 | s2) * el) % 16 == 0


def prefill_to_decode(k_Bx2TxHxD: Tensor, v_Bx2TxHxD: Tensor, current_doc_mask_BxT: Tensor, *, window_slot: int,
                      retained_slot: int, nw_k: Tensor, nw_v: Tensor, nw_len: Tensor, nw_pos: Tensor,
                      br_k: Tensor, br_v: Tensor, br_len: Tensor, window_tokens: int) -> None:
    """Writes one layer's decode caches from the prefill K/V (in place). Shapes: K/V [B, 2T, H, D];
    mask [B, T] bool; ring caches [B, H, Sw, D] with lengths/positions [B]; retained caches
    [B, H, Sr, D] with lengths [B, H]. The ring tensors are ignored when window_tokens <= 0.

    One call per layer at the prefill -> decode switch, so the host work is kept short: every shape
    and stride is read once, and the stride arrays handed to the library are cached by value."""
    kshape = tuple(k_Bx2TxHxD.shape)
    b, two_t, h, d = kshape
    t = two_t // 2
    assert two_t == 2 * t and tuple(v_Bx2TxHxD.shape) == kshape
    mshape = tuple(current_doc_mask_BxT.shape)
    assert mshape == (b, t), f"mask {mshape} vs ({b}, {t})"
    rshape = tuple(br_k.shape)
    assert rshape[:2] == (b, h) and rshape[3] == d and tuple(br_v.shape) == rshape
    assert tuple(br_len.shape) == (b, h)
    window_tokens = int(window_tokens)
    use_ring = window_tokens > 0
    if use_ring:
        wshape = tuple(nw_k.shape)
        assert wshape[:2] == (b, h) and wshape[3] == d and tuple(nw_v.shape) == wshape
        assert tuple(nw_len.shape) == (b,) and tuple(nw_pos.shape) == (b,)
        assert window_tokens <= wshape[2], "window_tokens exceeds the ring storage"
    kdt, cdt, ldt = k_Bx2TxHxD.dtype, br_k.dtype, br_len.dtype
    assert kdt in _FLOAT_DTYPES and v_Bx2TxHxD.dtype == kdt
    assert cdt in _FLOAT_DTYPES and (not use_ring or nw_k.dtype == cdt)
    assert ldt in _LEN_DTYPES and (not use_ring or (nw_len.dtype == ldt and nw_pos.dtype == ldt))
    assert d % 8 == 0, f"head_dim {d} must be a multiple of 8"
    assert k_Bx2TxHxD.is_cuda and br_k.is_cuda, "prefill_to_decode: tensors must be on the GPU"
    # The reference's slice assignment fails when a document does not fit the retained buffer. A
    # document has at most T tokens, so with a buffer of T rows or more this is a shape check; only a
    # shorter buffer needs the lengths read back (a host sync).
    if b and rshape[2] < t:
        longest = int(current_doc_mask_BxT.sum(dim=1).max())
        if longest > rshape[2]:
            raise RuntimeError(f"a prompt document of {longest} tokens does not fit the retained buffer "
                               f"({rshape[2]} rows)")
    el_in, el_c = k_Bx2TxHxD.element_size(), br_k.element_size()
    k, v = k_Bx2TxHxD, v_Bx2TxHxD
    ks, vs = k.stride(), v.stride()
    if not _rows16(k.data_ptr(), ks, el_in):
        k = k.contiguous()
        ks = k.stride()
    if not _rows16(v.data_ptr(), vs, el_in):
        v = v.contiguous()
        vs = v.stride()
    rk, rv = br_k.stride(), br_v.stride()
    caches = [(br_k.data_ptr(), rk), (br_v.data_ptr(), rv)]
    if use_ring:
        wk, wv = nw_k.stride(), nw_v.stride()
        caches += [(nw_k.data_ptr(), wk), (nw_v.data_ptr(), wv)]
    for ptr, st in caches:
        assert _rows16(ptr, st, el_c), "KV caches must have 16-byte aligned rows"
    # A bool mask with unit column stride is read in place (one byte per flag, 0 or 1).
    mask = current_doc_mask_BxT
    if mask.dtype == torch.bool and mask.stride(1) == 1:
        mask = mask.view(torch.uint8)
    else:
        mask = mask.to(torch.uint8).contiguous()
    if use_ring:
        ring = (caches[2][0], caches[3][0], N.i64_const(wk[:3] + wv[:3]), wshape[2], window_tokens,
                nw_len.data_ptr(), nw_pos.data_ptr(), N.i64_const((nw_len.stride(0), nw_pos.stride(0))))
    else:
        ring = (None, None, N.i64_const((0,) * 6), 0, 0, None, None, N.i64_const((0, 0)))
    status = N.lib().sps_prefill_to_decode(
        b, t, h, d, _FLOAT_DTYPES[kdt], k.data_ptr(), N.i64_const(ks[:3]), v.data_ptr(), N.i64_const(vs[:3]),
        int(window_slot), int(retained_slot), mask.data_ptr(), mask.stride(0), _FLOAT_DTYPES[cdt], *ring,
        caches[0][0], caches[1][0], N.i64_const(rk[:3] + rv[:3]), rshape[2], br_len.data_ptr(),
        N.i64_const(tuple(br_len.stride())), _LEN_DTYPES[ldt], torch.cuda.current_stream(k.device).cuda_stream)
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
