"""Drop-in prefill/training attention for the SPS model families, backed by libsps_attn.so.

Public functions keep the reference names, signatures, argument meaning and assertion behaviour:

* ``sps_sliding_attention``          <- attention/triton_sps_flash_attention.py:725-753
* ``reverse_sps_sliding_attention``  <- attention/triton_reverse_sps_flash_attention.py:827-853
* ``full_attention``                 <- attention/triton_full_flash_attention.py:679-709

(paths relative to src/modeling/models/ of lil-lab/sps). Differences that do not change results:
no padding of N to a multiple of 128 (the kernels bounds-check), no ``.contiguous()`` copies of
[B, N, H, D]-strided views (the kernels take element strides), and the output is allocated in
[B, N, H, D] memory order so the caller's ``y.transpose(1, 2).contiguous()`` is free.
``warp_specialize`` is accepted and ignored (it selects a Triton code path in the reference).
"""

from __future__ import annotations

import functools
from typing import Optional, Tuple

import torch

from . import _native as N

_SUPPORTED_HEAD_DIMS = (16, 32, 64, 128, 256)
_REFERENCE_HEAD_DIMS = {16, 32, 64, 128, 256}


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return N.DTYPE_BF16
    if t.dtype == torch.float16:
        return N.DTYPE_F16
    raise TypeError(f"sps_amd attention supports bfloat16 and float16 inputs, got {t.dtype}")


def _kernel_view(t: torch.Tensor) -> torch.Tensor:
    """Returns t if the kernels can read it in place (unit d stride, 16-byte aligned rows: base and the
    three outer strides, in 16-bit elements multiples of 8, tested at once on their OR)."""
    s0, s1, s2, s3 = t.stride()
    return t if (s3 == 1 and t.data_ptr() % 16 == 0 and (s0 | s1 | s2) % 8 == 0) else t.contiguous()


def _strides(t: torch.Tensor):
    return N.i64_const(t.stride()[:3])


def _docs_args(docs: Optional[torch.Tensor]):
    if docs is None:
        return None, 0, 0
    if docs.dtype == torch.int64:
        code = N.DTYPE_I64
    elif docs.dtype == torch.int32:
        code = N.DTYPE_I32
    else:
        raise TypeError(f"documents_idx_BxT must be int32 or int64, got {docs.dtype}")
    return docs.data_ptr(), code, docs.stride(0)


def _alloc_like_bnhd(q: torch.Tensor) -> torch.Tensor:
    b, h, n, d = q.shape
    return torch.empty((b, n, h, d), dtype=q.dtype, device=q.device).transpose(1, 2)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


@functools.lru_cache(maxsize=256)
def _workspace_bytes(family: int, b: int, h: int, n: int, has_docs: bool, backward: bool) -> int:
    return int(N.lib().sps_attn_workspace_bytes(family, b, h, n, int(has_docs), int(backward)))


def _workspace(family: int, b: int, h: int, n: int, has_docs: bool, backward: bool, device) -> Optional[torch.Tensor]:
    """The call's workspace, or None when it needs none (the entry points take a null pointer then:
    the forward without documents)."""
    nbytes = _workspace_bytes(family, b, h, n, bool(has_docs), bool(backward))
    return torch.empty(nbytes, dtype=torch.uint8, device=device) if nbytes else None


def _ws_args(ws: Optional[torch.Tensor]):
    return (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)


def _validate(q, k, v, family, documents_idx_BxT):
    head_dim_q, head_dim_k = q.shape[-1], k.shape[-1]
    head_dim_v = v.shape[-1]
    assert head_dim_q == head_dim_k and head_dim_k == head_dim_v
    assert head_dim_k in _REFERENCE_HEAD_DIMS
    if family != N.FAMILY_FULL:
        assert q.shape[2] % 2 == 0, "Expected doubled sequence length (2T)."
    if documents_idx_BxT is not None:
        assert documents_idx_BxT.shape[0] == q.shape[0]
        assert documents_idx_BxT.shape[1] == q.shape[2]
        assert documents_idx_BxT.is_cuda and documents_idx_BxT.is_contiguous()
    if head_dim_k not in _SUPPORTED_HEAD_DIMS:
        raise NotImplementedError(f"sps_amd: head_dim {head_dim_k} is not built (supported: {_SUPPORTED_HEAD_DIMS})")
    if not q.is_cuda:
        raise RuntimeError("sps_amd attention runs on the GPU only (got a CPU tensor)")
    if not (k.shape == q.shape and v.shape == q.shape):
        raise ValueError(f"q, k, v must share one shape, got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("q, k and v must share one dtype")


def attention_forward(q, k, v, sm_scale, family, window=0, documents_idx_BxT=None, persistent_key_window=None,
                      keep_layout=False):
    """Runs the forward kernel; returns (o, lse, q, k, v, workspace) with q/k/v as the kernels read them.

    With ``keep_layout`` (and documents) the workspace is sized for the backward and keeps the document
    row layout the forward computed; pass it to ``attention_backward(layout_workspace=...)`` so the
    backward skips recomputing it."""
    q, k, v = _kernel_view(q), _kernel_view(k), _kernel_view(v)
    b, h, n, d = q.shape
    o = _alloc_like_bnhd(q)
    lse = torch.empty((b, h, n), dtype=torch.float32, device=q.device)
    docs_ptr, docs_code, docs_sb = _docs_args(documents_idx_BxT)
    keep = bool(keep_layout) and documents_idx_BxT is not None
    ws = _workspace(family, b, h, n, documents_idx_BxT is not None, keep, q.device)
    has_pkw = persistent_key_window is not None
    status = N.lib().sps_attn_fwd(
        family, b, h, n, d, _dtype_code(q),
        q.data_ptr(), _strides(q), k.data_ptr(), _strides(k), v.data_ptr(), _strides(v),
        o.data_ptr(), _strides(o), lse.data_ptr(),
        docs_ptr, docs_code, docs_sb,
        float(sm_scale), int(window), int(has_pkw), int(persistent_key_window) if has_pkw else -1,
        *_ws_args(ws), _stream(q),
    )
    N.check("sps_attn_fwd", status)
    return o, lse, q, k, v, (ws if keep else None)


def backward_pass_args(do, q, k, v, o, lse, dq, dk, dv, sm_scale, family, window=0, documents_idx_BxT=None,
                       persistent_key_window=None, workspace=None):
    """The argument tuple of sps_attn_bwd_pass after its `pass` argument, for callers that launch the
    passes themselves (q, k, v, do as the kernels read them; dq, dk, dv allocated like q, k, v)."""
    b, h, n, d = q.shape
    docs_ptr, docs_code, docs_sb = _docs_args(documents_idx_BxT)
    ws = workspace if workspace is not None else _workspace(family, b, h, n, documents_idx_BxT is not None, True,
                                                            q.device)
    has_pkw = persistent_key_window is not None
    return (
        family, b, h, n, d, _dtype_code(q),
        q.data_ptr(), _strides(q), k.data_ptr(), _strides(k), v.data_ptr(), _strides(v),
        o.data_ptr(), _strides(o), do.data_ptr(), _strides(do), lse.data_ptr(),
        dq.data_ptr(), _strides(dq), dk.data_ptr(), _strides(dk), dv.data_ptr(), _strides(dv),
        docs_ptr, docs_code, docs_sb,
        float(sm_scale), int(window), int(has_pkw), int(persistent_key_window) if has_pkw else -1,
        *_ws_args(ws), _stream(q),
    ), ws


def attention_backward(do, q, k, v, o, lse, sm_scale, family, window=0, documents_idx_BxT=None,
                       persistent_key_window=None, between_passes=None, layout_workspace=None):
    """Runs the backward kernels; returns (dq, dk, dv) laid out like q, k, v.

    ``between_passes``: optional callable run on the host after the dQ pass is enqueued and before the
    dK/dV pass (e.g. to record a torch.cuda.Event on the current stream for per-kernel timing); the two
    passes are then launched separately. ``layout_workspace``: the workspace returned by
    ``attention_forward(keep_layout=True)`` for the same arguments; the backward then reuses its
    document layout instead of recomputing it."""
    do = _kernel_view(do)
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    reuse = layout_workspace is not None and documents_idx_BxT is not None
    args, ws = backward_pass_args(do, q, k, v, o, lse, dq, dk, dv, sm_scale, family, window, documents_idx_BxT,
                                  persistent_key_window, layout_workspace if reuse else None)
    lib = N.lib()
    reuse_bit = N.BWD_REUSE_LAYOUT if reuse else 0
    if between_passes is None:
        N.check("sps_attn_bwd_pass", lib.sps_attn_bwd_pass(N.BWD_DQ | N.BWD_DKDV | reuse_bit, *args))
    else:
        N.check("sps_attn_bwd_pass", lib.sps_attn_bwd_pass(N.BWD_DQ | reuse_bit, *args))
        between_passes()
        N.check("sps_attn_bwd_pass", lib.sps_attn_bwd_pass(N.BWD_DKDV, *args))
    return dq, dk, dv


# The attention as torch.library custom ops, so a torch.compile'd model (the reference trains with
# torch.compile, scripts/train.py:420-422) traces it as two opaque calls without a graph break. The
# forward returns its outputs and, when a backward will follow and documents are given, the
# workspace holding the document row layout; the backward reads that layout. It also writes its
# -LSE / -Delta seeds into the workspace's seed region, which is scratch: the backward writes it
# before reading it, and nothing else reads it, so the op's results depend on its inputs only and
# the op is declared pure. (Declaring the workspace mutated would bump the version of the tensor
# the forward saved, and a second backward over a retained graph would then be refused.)
@torch.library.custom_op("sps_amd::attention_fwd", mutates_args=())
def _attention_fwd_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, docs: Optional[torch.Tensor],
                      sm_scale: float, family: int, window: int, pkw: Optional[int],
                      keep_layout: bool) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    o, lse, _, _, _, ws = attention_forward(q, k, v, sm_scale, family, window, docs, pkw, keep_layout=keep_layout)
    if ws is None:
        ws = torch.empty((0,), dtype=torch.uint8, device=q.device)
    return o, lse, ws


@_attention_fwd_op.register_fake
def _(q, k, v, docs, sm_scale, family, window, pkw, keep_layout):
    b, h, n, d = q.shape
    o = q.new_empty((b, n, h, d)).transpose(1, 2)
    lse = q.new_empty((b, h, n), dtype=torch.float32)
    nbytes = 0
    if keep_layout and docs is not None:
        nbytes = int(N.lib().sps_attn_workspace_bytes(family, int(b), int(h), int(n), 1, 1))
    return o, lse, q.new_empty((nbytes,), dtype=torch.uint8)


@torch.library.custom_op("sps_amd::attention_bwd", mutates_args=())
def _attention_bwd_op(do: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
                      lse: torch.Tensor, docs: Optional[torch.Tensor], ws: torch.Tensor, sm_scale: float, family: int,
                      window: int, pkw: Optional[int]) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    q, k, v = _kernel_view(q), _kernel_view(k), _kernel_view(v)
    return attention_backward(do, q, k, v, o, lse, sm_scale, family, window, docs, pkw,
                              layout_workspace=ws if ws.numel() > 0 else None)


@_attention_bwd_op.register_fake
def _(do, q, k, v, o, lse, docs, ws, sm_scale, family, window, pkw):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


def _attention_setup_context(ctx, inputs, output):
    q, k, v, docs, sm_scale, family, window, pkw, _ = inputs
    o, lse, ws = output
    ctx.save_for_backward(q, k, v, o, lse, docs, ws)
    ctx.params = (float(sm_scale), int(family), int(window), pkw)


def _attention_backward(ctx, do, _dlse, _dws):
    q, k, v, o, lse, docs, ws = ctx.saved_tensors
    sm_scale, family, window, pkw = ctx.params
    dq, dk, dv = torch.ops.sps_amd.attention_bwd(do, q, k, v, o, lse, docs, ws, sm_scale, family, window, pkw)
    return dq, dk, dv, None, None, None, None, None, None


_attention_fwd_op.register_autograd(_attention_backward, setup_context=_attention_setup_context)


def _attention(q, k, v, sm_scale, family, window, documents_idx_BxT, persistent_key_window):
    _validate(q, k, v, family, documents_idx_BxT)
    keep = torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v))
    o, _, _ = torch.ops.sps_amd.attention_fwd(
        q, k, v, documents_idx_BxT, float(sm_scale), int(family), int(window),
        None if persistent_key_window is None else int(persistent_key_window), keep)
    return o


def sps_sliding_attention(
    q,
    k,
    v,
    sm_scale,
    temporary_key_window,
    warp_specialize=True,
    documents_idx_BxT=None,
    persistent_key_window=None,
):
    """Attention over the interleaved input/<predict> (2T) sequence, SPS variant.

    The persistent (window-exempt) key is the EVEN/input position; the <predict> position (odd) is
    the temporary key, visible only within ``temporary_key_window`` tokens of the query. The
    persistent key always self-attends and, when ``persistent_key_window`` is given, is otherwise
    visible only within that many tokens. ``documents_idx_BxT`` ([B, 2T] ids) confines attention to
    equal ids. q, k, v: [B, H, 2T, D] bf16/f16. Reference: triton_sps_flash_attention.py:725-753.
    """
    del warp_specialize
    return _attention(q, k, v, sm_scale, N.FAMILY_SPS, temporary_key_window, documents_idx_BxT, persistent_key_window)


def reverse_sps_sliding_attention(
    q,
    k,
    v,
    sm_scale,
    temporary_key_window,
    warp_specialize=True,
    documents_idx_BxT=None,
    persistent_key_window=None,
):
    """As ``sps_sliding_attention`` with the persistent key at the ODD/<predict> position.

    Used by the Reverse-SPS and Delayed-State models. Reference:
    triton_reverse_sps_flash_attention.py:827-853.
    """
    del warp_specialize
    return _attention(q, k, v, sm_scale, N.FAMILY_REVERSE_SPS, temporary_key_window, documents_idx_BxT,
                      persistent_key_window)


def full_attention(
    q,
    k,
    v,
    sm_scale,
    warp_specialize=True,
    documents_idx_BxT=None,
):
    """Document-masked causal attention (Standard model). q, k, v: [B, H, T, D].

    A query attends causally to keys with its document id (or to all causal keys when
    ``documents_idx_BxT`` is None). Reference: triton_full_flash_attention.py:679-709.
    """
    del warp_specialize
    return _attention(q, k, v, sm_scale, N.FAMILY_FULL, 0, documents_idx_BxT, None)


def attention_mask(family: int, n: int, documents_idx_BxT: Optional[torch.Tensor] = None, *, batch: int = 1,
                   window: int = 0, persistent_key_window: Optional[int] = None, schedule: int = 0,
                   device=None) -> torch.Tensor:
    """Materialises the [B, N, N] uint8 mask the kernels evaluate (schedule 0: forward/dQ block
    schedule, 1: dK/dV block schedule). A verification entry point; see include/sps_attn.h."""
    if documents_idx_BxT is not None:
        batch = documents_idx_BxT.shape[0]
        device = documents_idx_BxT.device
    device = torch.device(device if device is not None else "cuda")
    mask = torch.zeros((batch, n, n), dtype=torch.uint8, device=device)
    docs_ptr, docs_code, docs_sb = _docs_args(documents_idx_BxT)
    ws = _workspace(family, batch, 1, n, documents_idx_BxT is not None, False, device)
    has_pkw = persistent_key_window is not None
    status = N.lib().sps_attn_mask(
        family, batch, n, docs_ptr, docs_code, docs_sb, int(window), int(has_pkw),
        int(persistent_key_window) if has_pkw else -1, int(schedule), mask.data_ptr(),
        *_ws_args(ws), torch.cuda.current_stream(device).cuda_stream,
    )
    N.check("sps_attn_mask", status)
    return mask
