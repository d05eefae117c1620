"""Decode KV-cache update of one layer in one launch (ring insert + retained append).

Drop-in for the reference's ``fused_sps_kv_update`` (utils/decode_attention_fast.py:139-221): same
keyword-only signature and shape asserts. Semantics follow the un-fused path it replaces,
``_update_normal_memory_unfused`` / ``_update_predict_memory_unfused``
(reverse_sps/inference.py:137-168, 240-268), with the fused kernel's retained bound check
(decode_attention_fast.py:95-104): a retained buffer that is already full is left as it is.

For every active sequence b:
  ring (``window_tokens > 0``): slot = len[b] if the ring is not full, else pos[b]; every head's
  K/V row at that slot is replaced; then len[b] += 1 while the ring fills, else
  pos[b] = (pos[b] + 1) % window_tokens.
  retained: if 0 <= len[b, h] < storage, K/V[b, h, len[b, h]] = new and len[b, h] += 1.
The caches and lengths are updated in place; the new K/V may be any of bf16 / f16 / fp32 and are
rounded to the cache dtype (round to nearest even, as ``Tensor.to``).

``segmented_q2_attention_with_kv_update`` / ``segmented_q1_attention_with_kv_update`` run a decode
step's attention over the caches and this update together (``sps_decode_kv_update``): the update
then costs no launch of its own.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _native as N

_FLOAT_DTYPES = {torch.bfloat16: N.DTYPE_BF16, torch.float16: N.DTYPE_F16, torch.float32: N.DTYPE_F32}
_LEN_DTYPES = {torch.int32: N.DTYPE_I32, torch.int64: N.DTYPE_I64}
_FLAG_DTYPES = {torch.bool: N.DTYPE_U8, torch.uint8: N.DTYPE_U8, torch.int8: N.DTYPE_U8,
                torch.int32: N.DTYPE_I32, torch.int64: N.DTYPE_I64}


def _cache_strides(t: Tensor):
    st = t.stride()
    assert len(st) == 4 and st[3] == 1, "KV caches must be [B, H, storage, D] with a contiguous D axis"
    return st[:3]


def _new_strides(t: Tensor):
    st = t.stride()
    assert len(st) == 3 and st[2] == 1, "new K/V must be [B, H, D] with a contiguous D axis"
    return st[:2]


def kv_update_args(
    *,
    nw_k: Tensor,
    nw_v: Tensor,
    nw_len: Tensor,
    nw_pos: Tensor,
    br_k: Tensor,
    br_v: Tensor,
    br_len: Tensor,
    k_window_BxHxD: Tensor,
    v_window_BxHxD: Tensor,
    k_retained_BxHxD: Tensor,
    v_retained_BxHxD: Tensor,
    active_mask_B: Tensor,
    window_tokens: int,
) -> tuple:
    """Validates the arguments of fused_sps_kv_update and returns the argument tuple of its C-ABI call
    (``sps_kv_update``) on the current stream; the tuple's last element keeps the tensors it points
    into alive. A caller that repeats one update on the same buffers may build it once."""
    batch_size, n_head, head_dim = k_retained_BxHxD.shape
    window_tokens = int(window_tokens)
    use_ring = window_tokens > 0
    assert br_k.shape == br_v.shape, "br.k/v shape mismatch"
    assert br_k.size(0) == batch_size and br_k.size(1) == n_head and br_k.size(3) == head_dim
    assert br_len.shape == (batch_size, n_head)
    assert v_retained_BxHxD.shape == k_retained_BxHxD.shape
    if use_ring:
        assert nw_k.shape == nw_v.shape, "nw.k/v shape mismatch"
        assert nw_k.size(0) == batch_size and nw_k.size(1) == n_head and nw_k.size(3) == head_dim
        assert nw_len.shape == (batch_size,)
        assert nw_pos.shape == (batch_size,)
        assert k_window_BxHxD.shape == k_retained_BxHxD.shape and v_window_BxHxD.shape == k_retained_BxHxD.shape
        assert nw_k.dtype == br_k.dtype, "ring and retained caches must share a dtype"
        assert nw_len.dtype == br_len.dtype and nw_pos.dtype == br_len.dtype, "lengths must share a dtype"
        assert window_tokens <= nw_k.size(2), "window_tokens exceeds the ring storage"
    tensors = [br_k, br_v, br_len, k_retained_BxHxD, v_retained_BxHxD, active_mask_B]
    if use_ring:
        tensors += [nw_k, nw_v, nw_len, nw_pos, k_window_BxHxD, v_window_BxHxD]
    assert all(t.is_cuda for t in tensors), "fused_sps_kv_update: every tensor must be on the GPU"
    assert br_k.dtype in _FLOAT_DTYPES, f"unsupported cache dtype {br_k.dtype}"
    assert br_len.dtype in _LEN_DTYPES, f"lengths must be int32 or int64, got {br_len.dtype}"
    assert active_mask_B.dim() == 1 and active_mask_B.numel() == batch_size
    assert active_mask_B.dtype in _FLAG_DTYPES, f"unsupported active-mask dtype {active_mask_B.dtype}"

    new_dtype = k_retained_BxHxD.dtype
    assert new_dtype in _FLOAT_DTYPES, f"unsupported K/V dtype {new_dtype}"
    new = [k_retained_BxHxD, v_retained_BxHxD] + ([k_window_BxHxD, v_window_BxHxD] if use_ring else [])
    new = [t if t.dtype == new_dtype else t.to(new_dtype) for t in new]
    kr, vr = new[0], new[1]
    kw, vw = (new[2], new[3]) if use_ring else (kr, vr)
    ns = _new_strides(kw) + _new_strides(vw) + _new_strides(kr) + _new_strides(vr)
    ret_st = _cache_strides(br_k) + _cache_strides(br_v)
    if use_ring:
        ring_st = _cache_strides(nw_k) + _cache_strides(nw_v)
        ring = (nw_k.data_ptr(), nw_v.data_ptr(), N.i64_const(ring_st), nw_k.size(2), window_tokens,
                nw_len.data_ptr(), nw_pos.data_ptr(), N.i64_const((nw_len.stride(0), nw_pos.stride(0))))
    else:
        ring = (None, None, N.i64_const((0,) * 6), 0, 0, None, None, N.i64_const((0, 0)))
    args = (
        batch_size, n_head, head_dim, _FLOAT_DTYPES[br_k.dtype],
        *ring,
        br_k.data_ptr(), br_v.data_ptr(), N.i64_const(ret_st), br_k.size(2),
        br_len.data_ptr(), N.i64_const(tuple(br_len.stride())), _LEN_DTYPES[br_len.dtype],
        _FLOAT_DTYPES[new_dtype], kw.data_ptr(), vw.data_ptr(), kr.data_ptr(), vr.data_ptr(), N.i64_const(ns),
        active_mask_B.data_ptr(), _FLAG_DTYPES[active_mask_B.dtype], active_mask_B.stride(0),
        torch.cuda.current_stream(br_k.device).cuda_stream,
    )
    return args, tuple(new)


def run_kv_update(args: tuple) -> None:
    """Launches a KV update from kv_update_args' tuple."""
    N.check("sps_kv_update", N.lib().sps_kv_update(*args[0]))


def fused_sps_kv_update(
    *,
    nw_k: Tensor,
    nw_v: Tensor,
    nw_len: Tensor,
    nw_pos: Tensor,
    br_k: Tensor,
    br_v: Tensor,
    br_len: Tensor,
    k_window_BxHxD: Tensor,
    v_window_BxHxD: Tensor,
    k_retained_BxHxD: Tensor,
    v_retained_BxHxD: Tensor,
    active_mask_B: Tensor,
    window_tokens: int,
) -> None:
    """One-launch KV update of one decode layer (see the module docstring)."""
    run_kv_update(kv_update_args(
        nw_k=nw_k, nw_v=nw_v, nw_len=nw_len, nw_pos=nw_pos, br_k=br_k, br_v=br_v, br_len=br_len,
        k_window_BxHxD=k_window_BxHxD, v_window_BxHxD=v_window_BxHxD, k_retained_BxHxD=k_retained_BxHxD,
        v_retained_BxHxD=v_retained_BxHxD, active_mask_B=active_mask_B, window_tokens=window_tokens))


def segmented_q2_attention_with_kv_update(
    q_Bx2xHxD: Tensor,
    segments,
    *,
    current_normal_k_BxHxD: Tensor,
    current_normal_v_BxHxD: Tensor,
    current_predict_k_BxHxD: Tensor,
    current_predict_v_BxHxD: Tensor,
    attn_dtype: torch.dtype,
    nw_k: Tensor,
    nw_v: Tensor,
    nw_len: Tensor,
    nw_pos: Tensor,
    br_k: Tensor,
    br_v: Tensor,
    br_len: Tensor,
    k_window_BxHxD: Tensor,
    v_window_BxHxD: Tensor,
    k_retained_BxHxD: Tensor,
    v_retained_BxHxD: Tensor,
    active_mask_B: Tensor,
    window_tokens: int,
) -> Tensor:
    """One decode step of one layer in the attention's launches: ``triton_segmented_q2_attention``
    over the caches (as they are before the update), then ``fused_sps_kv_update`` of the same caches
    (the keyword arguments from ``nw_k`` on are that function's). This is the pair the reference's
    generation step runs back to back (reverse_sps/inference.py:322-362, then the update of :169-238
    via ``_update_normal_memory`` / ``_update_predict_memory``). Returns fp32 [B, 2, H, D]; the caches
    and lengths are updated in place. The caches must have the segments' dtype."""
    from .decode_attention import triton_segmented_q2_attention

    upd = kv_update_args(
        nw_k=nw_k, nw_v=nw_v, nw_len=nw_len, nw_pos=nw_pos, br_k=br_k, br_v=br_v, br_len=br_len,
        k_window_BxHxD=k_window_BxHxD, v_window_BxHxD=v_window_BxHxD, k_retained_BxHxD=k_retained_BxHxD,
        v_retained_BxHxD=v_retained_BxHxD, active_mask_B=active_mask_B, window_tokens=window_tokens)
    return triton_segmented_q2_attention(
        q_Bx2xHxD, segments, current_normal_k_BxHxD=current_normal_k_BxHxD,
        current_normal_v_BxHxD=current_normal_v_BxHxD, current_predict_k_BxHxD=current_predict_k_BxHxD,
        current_predict_v_BxHxD=current_predict_v_BxHxD, attn_dtype=attn_dtype, _kv_update=upd)


def segmented_q1_attention_with_kv_update(
    q_BxHxD: Tensor,
    segments,
    *,
    extra_kv=None,
    attn_dtype: torch.dtype,
    nw_k: Tensor,
    nw_v: Tensor,
    nw_len: Tensor,
    nw_pos: Tensor,
    br_k: Tensor,
    br_v: Tensor,
    br_len: Tensor,
    k_window_BxHxD: Tensor,
    v_window_BxHxD: Tensor,
    k_retained_BxHxD: Tensor,
    v_retained_BxHxD: Tensor,
    active_mask_B: Tensor,
    window_tokens: int,
) -> Tensor:
    """As segmented_q2_attention_with_kv_update for one query per (batch, head): the attention of
    ``triton_segmented_q1_attention`` (the reference's decode of one slot through
    ``masked_kv_attention``, reverse_sps/inference.py:270-320), then ``fused_sps_kv_update``. Returns
    fp32 [B, H, D]; raises RuntimeError where the q1 kernel does not apply (there is no other path)."""
    from .decode_attention import triton_segmented_q1_attention

    upd = kv_update_args(
        nw_k=nw_k, nw_v=nw_v, nw_len=nw_len, nw_pos=nw_pos, br_k=br_k, br_v=br_v, br_len=br_len,
        k_window_BxHxD=k_window_BxHxD, v_window_BxHxD=v_window_BxHxD, k_retained_BxHxD=k_retained_BxHxD,
        v_retained_BxHxD=v_retained_BxHxD, active_mask_B=active_mask_B, window_tokens=window_tokens)
    out = triton_segmented_q1_attention(q_BxHxD, segments, extra_kv=extra_kv, attn_dtype=attn_dtype, _kv_update=upd)
    if out is None:
        raise RuntimeError("segmented_q1_attention_with_kv_update: inputs outside what the decode kernel supports")
    return out
