"""Rotary position embedding for the attention path, fused with the casts and layout the attention
kernels take.

``apply_rotary_emb(xq, xk, freqs_cis)`` keeps the reference's signature and result
(model.py:201-230: each (x[2i], x[2i+1]) pair times the complex frequency of its position, in fp32,
returned in the inputs' dtype and shape; ``freqs_cis`` is (T, D/2) or per-sequence (B, T, D/2),
model.py:160-199). ``rope_qkv_for_attention(q, k, v, freqs_cis)`` is the whole pre-attention step of
the attention modules (sps/core.py:45-55, reverse_sps/core.py:60-75): RoPE on Q and K, every tensor
cast to bf16 and handed over as the [B, H, N, D] transposed views of [B, N, H, D] buffers, in one
launch. Both run in libsps_attn.so (``sps_rope_qkv``); there is no CPU path.

Both are differentiable. The rotation by a unit complex frequency f is a real-linear map whose
adjoint is the rotation by conj(f), and the casts pass gradients through in the input's dtype (the
autograd of model.py:201-230's ``.float()`` / ``view_as_complex`` / ``* freqs_cis`` / ``type_as``), so
the backward is the same kernel on the incoming gradients with the conjugate frequencies (V's
gradient is cast back to V's dtype in the same launch).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from . import _native as N

_FLOAT_DTYPES = {torch.bfloat16: N.DTYPE_BF16, torch.float16: N.DTYPE_F16, torch.float32: N.DTYPE_F32}


def _freqs_view(freqs_cis: Tensor, b: int, n: int, d: int) -> Tuple[Tensor, Tuple[int, int]]:
    """Float (re, im) view of the complex frequencies and its {b, n} float strides."""
    if freqs_cis.ndim == 3:
        assert freqs_cis.shape == (b, n, d // 2), f"freqs_cis {tuple(freqs_cis.shape)} vs ({b}, {n}, {d // 2})"
    else:
        assert freqs_cis.shape == (n, d // 2), f"freqs_cis {tuple(freqs_cis.shape)} vs ({n}, {d // 2})"
    f = freqs_cis if freqs_cis.dtype == torch.complex64 else freqs_cis.to(torch.complex64)
    fr = torch.view_as_real(f)
    if fr.stride(-1) != 1 or fr.stride(-2) != 2 or (fr.stride(-3) * 4) % 16 or fr.data_ptr() % 16:
        fr = fr.contiguous()
    if fr.ndim == 4:
        return fr, (fr.stride(0), fr.stride(1))
    return fr, (0, fr.stride(0))


def _aligned(t: Tensor) -> bool:
    el = t.element_size()
    return t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all((s * el) % 16 == 0 for s in t.stride()[:-1])


def _launch(q: Tensor, k: Tensor, v: Optional[Tensor], freqs_cis: Tensor, q_out: Tensor, k_out: Tensor,
            v_out: Optional[Tensor]) -> None:
    b, n, h, d = q.shape
    assert k.shape == q.shape and (v is None or v.shape == q.shape), "q/k/v shapes differ"
    assert q.dtype in _FLOAT_DTYPES and k.dtype == q.dtype and (v is None or v.dtype == q.dtype)
    assert d % 8 == 0, f"head_dim {d} must be a multiple of 8"
    assert q.is_cuda and k.is_cuda and freqs_cis.is_cuda, "rope: tensors must be on the GPU"
    q, k = (t if _aligned(t) else t.contiguous() for t in (q, k))
    if v is not None and not _aligned(v):
        v = v.contiguous()
    fr, fst = _freqs_view(freqs_cis, b, n, d)
    st = lambda t: N.i64_array((t.stride(0), t.stride(1), t.stride(2)))  # noqa: E731
    status = N.lib().sps_rope_qkv(
        b, n, h, d, _FLOAT_DTYPES[q.dtype], q.data_ptr(), st(q), k.data_ptr(), st(k),
        v.data_ptr() if v is not None else None, st(v) if v is not None else None,
        fr.data_ptr(), N.i64_array(fst), _FLOAT_DTYPES[q_out.dtype], q_out.data_ptr(), st(q_out),
        k_out.data_ptr(), st(k_out), v_out.data_ptr() if v_out is not None else None,
        st(v_out) if v_out is not None else None, torch.cuda.current_stream(q.device).cuda_stream)
    N.check("sps_rope_qkv", status)


# Both functions as torch.library custom ops with fake implementations and registered autograd, so a
# torch.compile'd model (the reference trains compiled, scripts/train.py:420-422; sps/core.py:50-52
# calls apply_rotary_emb inside the compiled forward) traces them without a graph break. The
# backward of each is the same op on the incoming gradients with the conjugate frequencies, cast
# back to the input dtype.
@torch.library.custom_op("sps_amd::rope_pair", mutates_args=())
def _rope_pair_op(xq: Tensor, xk: Tensor, freqs_cis: Tensor) -> Tuple[Tensor, Tensor]:
    q_out = torch.empty(xq.shape, device=xq.device, dtype=xq.dtype)
    k_out = torch.empty(xk.shape, device=xk.device, dtype=xk.dtype)
    _launch(xq, xk, None, freqs_cis, q_out, k_out, None)
    return q_out, k_out


@_rope_pair_op.register_fake
def _(xq, xk, freqs_cis):
    return torch.empty_like(xq, memory_format=torch.contiguous_format), torch.empty_like(
        xk, memory_format=torch.contiguous_format)


def _rope_pair_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[2])


def _rope_pair_backward(ctx, gq, gk):
    (freqs_cis,) = ctx.saved_tensors
    ref = gq if gq is not None else gk
    gq = gq if gq is not None else torch.zeros_like(ref)
    gk = gk if gk is not None else torch.zeros_like(ref)
    dq, dk = torch.ops.sps_amd.rope_pair(gq, gk, _conj(freqs_cis))
    return dq, dk, None


_rope_pair_op.register_autograd(_rope_pair_backward, setup_context=_rope_pair_setup)


@torch.library.custom_op("sps_amd::rope_qkv", mutates_args=())
def _rope_qkv_op(q: Tensor, k: Tensor, v: Tensor, freqs_cis: Tensor,
                 out_dtype: torch.dtype) -> Tuple[Tensor, Tensor, Tensor]:
    outs = [torch.empty(q.shape, device=q.device, dtype=out_dtype) for _ in range(3)]
    _launch(q, k, v, freqs_cis, *outs)
    return tuple(outs)


@_rope_qkv_op.register_fake
def _(q, k, v, freqs_cis, out_dtype):
    return tuple(torch.empty(q.shape, device=q.device, dtype=out_dtype) for _ in range(3))


def _rope_qkv_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[3])
    ctx.in_dtype = inputs[0].dtype


def _rope_qkv_backward(ctx, gq, gk, gv):
    (freqs_cis,) = ctx.saved_tensors
    ref = next(g for g in (gq, gk, gv) if g is not None)
    gq, gk, gv = (g if g is not None else torch.zeros_like(ref) for g in (gq, gk, gv))
    dq, dk, dv = torch.ops.sps_amd.rope_qkv(gq, gk.to(gq.dtype), gv.to(gq.dtype), _conj(freqs_cis), ctx.in_dtype)
    return dq, dk, dv, None, None


_rope_qkv_op.register_autograd(_rope_qkv_backward, setup_context=_rope_qkv_setup)


def _conj(freqs_cis: Tensor) -> Tensor:
    return freqs_cis.conj().resolve_conj()


def apply_rotary_emb(xq: Tensor, xk: Tensor, freqs_cis: Tensor) -> Tuple[Tensor, Tensor]:
    """RoPE on [B, T, H, D] queries and keys; returns new tensors of the inputs' dtype and shape."""
    assert xq.ndim == 4 and xk.shape == xq.shape
    return torch.ops.sps_amd.rope_pair(xq, xk, freqs_cis)


def rope_qkv_for_attention(q: Tensor, k: Tensor, v: Tensor, freqs_cis: Tensor,
                           out_dtype: torch.dtype = torch.bfloat16) -> Tuple[Tensor, Tensor, Tensor]:
    """The attention modules' pre-attention step in one launch: q, k, v [B, T, H, D] (views of the
    QKV projection are fine) -> RoPE(q), RoPE(k), v in ``out_dtype`` as [B, H, T, D] views of
    [B, T, H, D] buffers, ready for sps_sliding_attention / reverse_sps_sliding_attention /
    full_attention."""
    assert q.ndim == 4 and k.shape == q.shape and v.shape == q.shape
    assert out_dtype in _FLOAT_DTYPES
    outs = torch.ops.sps_amd.rope_qkv(q, k, v, freqs_cis, out_dtype)
    return tuple(t.transpose(1, 2) for t in outs)
