"""Rotary position embedding reference in float64 numpy (test infrastructure only).

Restates apply_rotary_emb of lil-lab/sps (src/modeling/models/model.py:201-230, with the
broadcast rules of reshape_for_broadcast, model.py:160-199): the last axis of a [B, T, H, D] query
or key is read as D/2 complex numbers (x[2i] + 1j * x[2i+1]) and multiplied by freqs_cis[t, i]
((T, D/2), shared by the batch) or freqs_cis[b, t, i] ((B, T, D/2), per sequence). The reference
computes in fp32 and then casts (type_as, .to(bfloat16)); this oracle computes in float64, so a
kernel result rounded once to bf16 is within one bf16 rounding of it.
"""

from __future__ import annotations

import numpy as np


def rope(x: np.ndarray, freqs: np.ndarray) -> np.ndarray:
    """x: [B, T, H, D] real; freqs: complex [T, D/2] or [B, T, D/2]. Returns float64 [B, T, H, D]."""
    x = np.asarray(x, dtype=np.float64)
    B, T, H, D = x.shape
    z = x[..., 0::2] + 1j * x[..., 1::2]
    f = np.asarray(freqs, dtype=np.complex128)
    f = f[None, :, None, :] if f.ndim == 2 else f[:, :, None, :]
    w = z * f
    out = np.empty_like(x)
    out[..., 0::2] = w.real
    out[..., 1::2] = w.imag
    return out


def freqs_cis(dim: int, end: int, theta: float = 10000.0) -> np.ndarray:
    """The reference's frequency table (model.py:134-158): exp(1j * t * theta^(-2i/dim))."""
    inv = 1.0 / (theta ** (np.arange(0, dim, 2)[: dim // 2] / dim))
    t = np.arange(end)
    return np.exp(1j * np.outer(t, inv))
