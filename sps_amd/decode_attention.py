"""Drop-in segmented decode attention for SPS-family (and Standard-model) generation.

Keeps the reference names, signatures and error conventions of utils/decode_attention.py
(src/modeling/models/ of lil-lab/sps):

* ``KVSegment``                     <- decode_attention.py:21-32
* ``triton_segmented_q1_attention`` <- decode_attention.py:393-480 (returns None when unsupported)
* ``triton_segmented_q2_attention`` <- decode_attention.py:483-594 (raises RuntimeError)
* ``masked_kv_attention``           <- decode_attention.py:597-704

The names still say "triton" because callers import them by those names; every path here runs the
HIP kernels of libsps_attn.so. There is no CPU path: ``masked_kv_attention`` on CPU tensors raises.
"""

from __future__ import annotations

import functools
import math
from dataclasses import dataclass
from typing import Optional

import torch
from torch import Tensor

from . import _native as N

_KV_DTYPES = {torch.bfloat16: N.DTYPE_BF16, torch.float16: N.DTYPE_F16, torch.float32: N.DTYPE_F32}
_DECODE_HEAD_DIMS = (16, 32, 64, 128, 256)


@dataclass
class KVSegment:
    """A contiguous block of keys/values with per-element validity lengths.

    k, v: [B, H, max_T, D]; lengths: [B, H] (per head) or [B] (shared across heads);
    max_len_cap: optional host-side cap on the scanned length.
    """

    k: Tensor
    v: Tensor
    lengths: Tensor
    max_len_cap: int | None = None


def _segment_scan_len(seg: KVSegment) -> int:
    """Number of leading storage rows a segment may contribute (reference decode_attention.py:381-390)."""
    max_t = int(seg.k.size(2))
    if max_t == 0:
        return 0
    if seg.max_len_cap is None:
        return max_t
    cap = int(seg.max_len_cap)
    if cap < 0:
        raise ValueError(f"KVSegment.max_len_cap must be non-negative, got {cap}")
    return max(1, min(max_t, cap))


def _len_dtype(lengths: Tensor) -> int:
    if lengths.dtype == torch.int64:
        return N.DTYPE_I64
    if lengths.dtype == torch.int32:
        return N.DTYPE_I32
    raise TypeError(f"segment lengths must be int32 or int64, got {lengths.dtype}")


def _as_attn(t: Tensor, attn_dtype: torch.dtype) -> Tensor:
    """The tensor in the attention dtype (no copy when it already is, and its last dim is contiguous)."""
    if t.dtype != attn_dtype:
        t = t.to(attn_dtype)
    return t if t.stride(-1) == 1 else t.contiguous()


@functools.lru_cache(maxsize=256)
def _decode_ws_bytes(fused_update: bool, b: int, h: int, d: int, nq: int, kv_dtype: int, scans: tuple) -> int:
    lib = N.lib()
    fn = lib.sps_decode_kv_update_workspace_bytes if fused_update else lib.sps_decode_workspace_bytes
    return int(fn(b, h, d, nq, kv_dtype, len(scans), N.i64_const(scans)))


def _run_decode(q: Tensor, nq: int, segments, extras, extra_masks, out: Tensor, static_scratch: bool = False,
                kv_update: Optional[tuple] = None) -> Tensor:
    """Calls sps_decode. q: [B, nq, H, D] (bf16/f16/f32); extras: list of (k, v) [B, H, D] sharing one
    dtype and one (b, h) stride pair. ``static_scratch`` calls sps_decode_static instead, which keeps
    its partial records in the library's own scratch array (no workspace is allocated). ``kv_update``
    (the argument tuple of decode_attention_fast.kv_update_args) calls sps_decode_kv_update instead:
    the same attention, then that KV update of the caches, in the attention's launches.

    One call per layer and generated token, so the host work is kept short: the workspace sizes are
    memoized per shape, and the array arguments, which repeat from step to step (the caches and their
    strides stay put), are cached by value."""
    b, _, h, d = q.shape
    kv_dtype = _KV_DTYPES[segments[0].k.dtype] if segments else N.DTYPE_BF16
    scans = tuple(_segment_scan_len(sg) for sg in segments)
    lens = [sg.lengths.contiguous() for sg in segments]
    lib = N.lib()
    ws = None
    if kv_update is not None:
        upd = kv_update[0]
        if segments and upd[3] != kv_dtype:
            raise RuntimeError("decode with KV update: the caches must have the segments' dtype")
        ws = torch.empty(max(_decode_ws_bytes(True, b, h, d, nq, kv_dtype, scans), 1), dtype=torch.uint8,
                         device=q.device)
    elif not static_scratch:
        ws = torch.empty(max(_decode_ws_bytes(False, b, h, d, nq, kv_dtype, scans), 1), dtype=torch.uint8,
                         device=q.device)
    k_strides = tuple(x for sg in segments for x in sg.k.stride()[:3])
    v_strides = tuple(x for sg in segments for x in sg.v.stride()[:3])
    if extras:
        ek = tuple(e[0].data_ptr() for e in extras)
        ev = tuple(e[1].data_ptr() for e in extras)
        e_strides = extras[0][0].stride()[:2]
        e_dtype = _KV_DTYPES[extras[0][0].dtype]
    else:
        ek = ev = ()
        e_strides, e_dtype = (0, 0), N.DTYPE_F32
    if kv_update is not None:
        name, entry, tail = "sps_decode_kv_update", lib.sps_decode_kv_update, (*kv_update[0][4:-1], ws.data_ptr(),
                                                                                ws.numel())
    elif static_scratch:
        name, entry, tail = "sps_decode_static", lib.sps_decode_static, ()
    else:
        name, entry, tail = "sps_decode", lib.sps_decode, (ws.data_ptr(), ws.numel())
    status = entry(
        b, h, d, nq,
        q.data_ptr(), _KV_DTYPES[q.dtype], N.i64_const(q.stride()[:3]),
        kv_dtype, len(segments),
        N.ptr_const(tuple(sg.k.data_ptr() for sg in segments)), N.i64_const(k_strides),
        N.ptr_const(tuple(sg.v.data_ptr() for sg in segments)), N.i64_const(v_strides),
        N.ptr_const(tuple(ln.data_ptr() for ln in lens)), N.i32_const(tuple(_len_dtype(ln) for ln in lens)),
        N.i32_const(tuple(int(ln.dim() == 2) for ln in lens)), N.i64_const(scans),
        len(extras), N.ptr_const(ek), N.ptr_const(ev), e_dtype,
        N.i64_const(tuple(e_strides)), N.i32_const(tuple(extra_masks)),
        1.0 / math.sqrt(d), out.data_ptr(), N.i64_const(out.stride()[:3]),
        *tail, torch.cuda.current_stream(q.device).cuda_stream,
    )
    N.check(name, status)
    return out


def _extras_in(extra_kv, attn_dtype, b, h, d):
    """Extra (k, v) pairs in the attention dtype with one shared (b, h) stride pair."""
    shape = (b, h, d)

    def conv(t):
        t = _as_attn(t, attn_dtype)
        return t if t.shape == shape else t.expand(b, h, d)

    out = [(conv(ek), conv(ev)) for ek, ev in extra_kv]
    if len({k.stride()[:2] for pair in out for k in pair}) > 1:
        out = [(k.contiguous(), v.contiguous()) for k, v in out]
    return out


def _segments_compatible(segments, batch_size, n_head, head_dim, device) -> bool:
    dtype = None
    for seg in segments:
        k, v, ln = seg.k, seg.v, seg.lengths
        if dtype is None:
            dtype = k.dtype
        if k.dtype != dtype or v.dtype != dtype:
            return False
        kshape = k.shape
        if len(kshape) != 4 or v.shape != kshape:
            return False
        if kshape[0] != batch_size or kshape[1] != n_head or kshape[3] != head_dim:
            return False
        if ln.device != device or ln.dtype not in (torch.int32, torch.int64):
            return False
        ldim = ln.dim()
        if ldim == 2:
            if tuple(ln.shape) != (batch_size, n_head):
                return False
        elif ldim != 1 or ln.shape[0] != batch_size:
            return False
        # Unit d stride and 16-byte aligned rows (power-of-two element sizes: one test of the three
        # outer strides' OR covers all three).
        esize = k.element_size()
        for t in (k, v):
            s0, s1, s2, s3 = t.stride()
            if s3 != 1 or t.data_ptr() % 16 != 0 or ((s0 | s1 | s2) * esize) % 16 != 0:
                return False
    return dtype is None or dtype in _KV_DTYPES


def triton_segmented_q1_attention(
    q_BxHxD: Tensor,
    segments: list[KVSegment],
    *,
    extra_kv: list[tuple[Tensor, Tensor]] | None = None,
    attn_dtype: torch.dtype,
    _kv_update: Optional[tuple] = None,
) -> Optional[Tensor]:
    """One query per (batch, head) over <= 3 segments plus <= 2 always-visible extra keys.

    Returns fp32 [B, H, D], or None when the inputs are outside what the kernel supports (the
    reference's contract: the caller then falls back). ``_kv_update`` is internal
    (decode_attention_fast.segmented_q1_attention_with_kv_update).
    """
    if not q_BxHxD.is_cuda:
        return None
    if len(segments) > 3:
        return None
    if extra_kv is not None and len(extra_kv) > 2:
        return None
    batch_size, n_head, head_dim = q_BxHxD.shape
    if head_dim not in _DECODE_HEAD_DIMS:
        return None
    for seg in segments:
        if not (seg.k.is_cuda and seg.v.is_cuda and seg.k.is_contiguous() and seg.v.is_contiguous()):
            return None
    if not _segments_compatible(segments, batch_size, n_head, head_dim, q_BxHxD.device):
        return None
    if attn_dtype not in _KV_DTYPES:
        return None
    extras = _extras_in(extra_kv or [], attn_dtype, batch_size, n_head, head_dim)
    q4 = _as_attn(q_BxHxD, attn_dtype).unsqueeze(1)
    out = torch.empty((batch_size, n_head, head_dim), device=q_BxHxD.device, dtype=torch.float32)
    out4 = out.view(batch_size, 1, n_head, head_dim)
    _run_decode(q4, 1, list(segments), extras, [1] * len(extras), out4, kv_update=_kv_update)
    return out


def triton_segmented_q2_attention(
    q_Bx2xHxD: Tensor,
    segments: list[KVSegment],
    *,
    current_normal_k_BxHxD: Tensor,
    current_normal_v_BxHxD: Tensor,
    current_predict_k_BxHxD: Tensor,
    current_predict_v_BxHxD: Tensor,
    attn_dtype: torch.dtype,
    _kv_update: Optional[tuple] = None,
) -> Tensor:
    """Two queries per (batch, head): slot 0 (input) sees the segments + current input key; slot 1
    (<predict>) additionally sees the current <predict> key. Fail-fast: raises RuntimeError on any
    unsupported input, as the reference does. Returns fp32 [B, 2, H, D]. ``_kv_update`` is internal
    (decode_attention_fast.segmented_q2_attention_with_kv_update)."""
    if not q_Bx2xHxD.is_cuda:
        raise RuntimeError("CUDA tensors are required for SPS-family cached generation attention")
    if len(segments) > 2:
        raise RuntimeError(f"SPS-family q2 attention supports at most 2 segments, got {len(segments)}")
    batch_size, n_slots, n_head, head_dim = q_Bx2xHxD.shape
    if n_slots != 2:
        raise RuntimeError(f"Expected q_Bx2xHxD slot dimension to be 2, got {n_slots}")
    if head_dim <= 0 or head_dim > 256:
        raise RuntimeError(f"Unsupported SPS-family q2 attention head_dim={head_dim}")
    if head_dim not in _DECODE_HEAD_DIMS:
        raise RuntimeError(f"sps_amd q2 attention is built for head_dim in {_DECODE_HEAD_DIMS}, got {head_dim}")
    current = [current_normal_k_BxHxD, current_normal_v_BxHxD, current_predict_k_BxHxD, current_predict_v_BxHxD]
    for tensor in current:
        if not tensor.is_cuda:
            raise RuntimeError("Current-token K/V tensors must be CUDA tensors")
        if tensor.shape != (batch_size, n_head, head_dim):
            raise RuntimeError(
                "Current-token K/V tensors must have shape "
                f"{(batch_size, n_head, head_dim)}, got {tuple(tensor.shape)}"
            )
    for seg in segments:
        if seg.k.dim() != 4 or seg.v.dim() != 4:
            raise RuntimeError("Segment K/V tensors must be rank-4 [B,H,T,D]")
        if seg.k.shape != seg.v.shape:
            raise RuntimeError(f"Segment K/V shapes differ: {tuple(seg.k.shape)} vs {tuple(seg.v.shape)}")
        if seg.k.size(0) != batch_size or seg.k.size(1) != n_head or seg.k.size(3) != head_dim:
            raise RuntimeError(
                "Segment K/V tensors must match query batch/head/head_dim, got "
                f"{tuple(seg.k.shape)} for query {(batch_size, n_head, head_dim)}"
            )
        if (not seg.k.is_cuda) or (not seg.v.is_cuda):
            raise RuntimeError("Segment K/V tensors must be CUDA tensors")
        if (not seg.k.is_contiguous()) or (not seg.v.is_contiguous()):
            raise RuntimeError("Segment K/V tensors must be contiguous")
        if seg.lengths.device != q_Bx2xHxD.device:
            raise RuntimeError("Segment lengths must live on the same device as query")
        _segment_scan_len(seg)
    if not _segments_compatible(segments, batch_size, n_head, head_dim, q_Bx2xHxD.device):
        raise RuntimeError("sps_amd q2 attention: segments must share a bf16/f16/f32 dtype, int lengths "
                           "of shape [B] or [B, H] and 16-byte aligned rows")
    if attn_dtype not in _KV_DTYPES:
        raise RuntimeError(f"sps_amd q2 attention supports attn_dtype bf16, f16 or f32, got {attn_dtype}")
    extras = _extras_in([(current_normal_k_BxHxD, current_normal_v_BxHxD),
                         (current_predict_k_BxHxD, current_predict_v_BxHxD)], attn_dtype, batch_size, n_head, head_dim)
    q = _as_attn(q_Bx2xHxD, attn_dtype)
    out = torch.empty((batch_size, 2, n_head, head_dim), device=q_Bx2xHxD.device, dtype=torch.float32)
    return _run_decode(q, 2, list(segments), extras, [0b11, 0b10], out, kv_update=_kv_update)


def masked_kv_attention(
    q_BxHxD: Tensor,
    segments: list[KVSegment],
    *,
    extra_kv: list[tuple[Tensor, Tensor]] | None = None,
    attn_dtype: torch.dtype,
    check_finite: bool = False,
    error_context: str = "",
    prefer_triton: bool = False,
    require_triton: bool = False,
) -> Tensor:
    """Attention of one query per (batch, head) over variable-length KV segments plus extra keys.

    Same contract as the reference (decode_attention.py:597-704): fp32 [B, H, D] output, zeros when
    there is no key at all, RuntimeError on an empty row / non-finite input when ``check_finite``.
    ``prefer_triton`` / ``require_triton`` are accepted for compatibility; every call runs the HIP
    kernel. A row with no attended key yields 0 (the reference's padded-SDPA path yields NaN there).
    """
    del prefer_triton
    if not q_BxHxD.is_cuda:
        raise RuntimeError(f"sps_amd masked_kv_attention runs on the GPU only{error_context}")
    b, n_head, head_dim = q_BxHxD.shape
    n_extra = len(extra_kv) if extra_kv else 0
    if check_finite:
        seg_maxlens = [
            0 if seg.lengths.numel() == 0 else min(int(seg.lengths.max().item()), _segment_scan_len(seg))
            for seg in segments
        ]
        total_len = sum(seg_maxlens) + n_extra
        if total_len == 0:
            return q_BxHxD.new_zeros((b, n_head, head_dim), dtype=torch.float32)
        counts = torch.full((b, n_head), n_extra, device=q_BxHxD.device, dtype=torch.long)
        for seg, max_len in zip(segments, seg_maxlens):
            if max_len == 0:
                continue
            ln = seg.lengths.clamp(min=0, max=max_len).long()
            counts = counts + (ln.view(b, 1).expand(b, n_head) if ln.dim() == 1 else ln)
        if bool((counts <= 0).any()):
            raise RuntimeError(f"Invalid mask with no valid keys{error_context}")
        finite = bool(torch.isfinite(q_BxHxD).all())
        for seg, max_len in zip(segments, seg_maxlens):
            if max_len:
                finite = finite and bool(torch.isfinite(seg.k[:, :, :max_len]).all())
                finite = finite and bool(torch.isfinite(seg.v[:, :, :max_len]).all())
        for ek, ev in extra_kv or []:
            finite = finite and bool(torch.isfinite(ek).all()) and bool(torch.isfinite(ev).all())
        if not finite:
            raise RuntimeError(f"Non-finite QKV{error_context}")
    out = triton_segmented_q1_attention(q_BxHxD, segments, extra_kv=extra_kv, attn_dtype=attn_dtype)
    if out is None:
        if require_triton:
            raise RuntimeError(f"Triton segmented q1 attention is required but unavailable{error_context}")
        raise RuntimeError(f"sps_amd masked_kv_attention: unsupported inputs (no fallback path){error_context}")
    if check_finite and not bool(torch.isfinite(out).all()):
        raise RuntimeError(f"Non-finite attention output{error_context}")
    return out
