"""The reference kernels' own arithmetic, emulated on the CPU in float32 (test infrastructure only).

oracle.attention gives the exact (float64) attention. The reference's Triton kernels do not compute
that: they round some intermediates to the 16-bit input type. This module restates their
arithmetic step by step, so that tests can tell the error the algorithm itself carries from an
error of the HIP kernels:

  forward   (triton_sps_flash_attention.py:26-139, 142-269)
            S = Q K^T accumulated in fp32 from the 16-bit inputs; qk = S * (sm_scale * 1.44269504)
            in fp32 (:78-79, :195-197); masked pairs get an additive -1e6 (:81-111); online softmax
            over key blocks of BLOCK_N with m_0 = -1e9 and l_0 = 1 (:195-196):
              m_ij = max(m_i, rowmax(qk)), p = exp2(qk - m_ij), alpha = exp2(m_i - m_ij),
              l_i = l_i * alpha + rowsum(p) (of the fp32 p), acc = acc * alpha + p.to(16 bit) @ V;
            O = (acc / l_i).to(16 bit) (:266-269); M = m_i + log2(l_i) (:266).
  backward  Delta = rowsum(O * dO) in fp32 from the stored 16-bit O
            (triton_reverse_sps_flash_attention.py:334-348);
            p = exp2(S * (sm_scale * 1.44269504) - M), zero where masked (:332-369, :456-479);
            dV = p.to(16 bit)^T dO; dP = dO V^T in fp32; dS = p * (dP - Delta) in fp32;
            dK = (dS.to(16 bit)^T Q) * sm_scale; dQ = (dS.to(16 bit) K) * sm_scale (:361-381, :471-488);
            the gradients are stored in the 16-bit input type (:712-714).

With rounding=False every step runs in float64 with no 16-bit casts; the result must then equal
oracle.attention to float64 precision, which pins the structure (online softmax, Delta, scale
placement, mask) independently of the rounding (tests/test_oracle_emulate.py).

Masked pairs are excluded as -inf here. The reference adds -1e6 instead; exp2 of that is 0 in fp32,
and a block with no visible key for a row is wiped by alpha = 0 once a visible key arrives, so the
two agree for every row that sees at least one key. A row that sees none (a temporary-stream query
at its stream's first position under window -1) gets O = 0 and M = -1e9 here, as in the exact
oracle; the reference's additive mask would instead average the masked keys of its first block.
"""

from __future__ import annotations

import numpy as np
import torch

LOG2E_REF = 1.44269504  # the reference's literal (triton_sps_flash_attention.py:197)


def _prep(x, dt):
    return torch.as_tensor(np.asarray(x) if not isinstance(x, torch.Tensor) else x).to(dt)


def forward(q, k, v, mask, sm_scale, *, dtype=torch.bfloat16, block_n=64, rounding=True):
    """q, k, v: [B, H, N, D] (values representable in `dtype`); mask: [B, N, N] bool.

    Returns (O, M): O [B, H, N, D] (in `dtype` when rounding, else float64) and M = m + log2(l)
    [B, H, N] (float32 when rounding, else float64)."""
    ft = torch.float32 if rounding else torch.float64
    q, k, v = (_prep(x, ft) for x in (q, k, v))
    mask_t = torch.as_tensor(np.asarray(mask, dtype=bool))[:, None]  # [B, 1, N, N]
    b, h, n, d = q.shape
    qk_scale = torch.tensor(sm_scale, dtype=ft) * torch.tensor(LOG2E_REF, dtype=ft)
    m_i = torch.full((b, h, n), -1e9, dtype=ft)
    l_i = torch.ones((b, h, n), dtype=ft)
    acc = torch.zeros((b, h, n, d), dtype=ft)
    for s in range(0, n, block_n):
        e = min(s + block_n, n)
        qk = (q @ k[:, :, s:e].transpose(-1, -2)) * qk_scale
        qk = qk.masked_fill(~mask_t[..., s:e], float("-inf"))
        m_ij = torch.maximum(m_i, qk.amax(dim=-1))
        p = torch.exp2(qk - m_ij[..., None])
        alpha = torch.exp2(m_i - m_ij)
        l_ij = p.sum(dim=-1)
        p_mm = p.to(dtype).to(ft) if rounding else p
        acc = acc * alpha[..., None] + p_mm @ v[:, :, s:e]
        l_i = l_i * alpha + l_ij
        m_i = m_ij
    lse = m_i + torch.log2(l_i)
    o = acc / l_i[..., None]
    return (o.to(dtype) if rounding else o), lse


def backward(q, k, v, o, lse, do, mask, sm_scale, *, dtype=torch.bfloat16, rounding=True):
    """Gradients of sum(O * dO) as the reference's dK/dV and dQ kernels form them.

    o and lse are the forward's outputs (forward(...) above). Returns (dq, dk, dv) in `dtype` when
    rounding, else float64."""
    ft = torch.float32 if rounding else torch.float64
    q, k, v, o, do = (_prep(x, ft) for x in (q, k, v, o, do))
    lse = _prep(lse, ft)
    mask_t = torch.as_tensor(np.asarray(mask, dtype=bool))[:, None]
    scale = torch.tensor(sm_scale, dtype=ft)
    qk_scale = scale * torch.tensor(LOG2E_REF, dtype=ft)
    delta = (o * do).sum(dim=-1)
    qk = (q @ k.transpose(-1, -2)) * qk_scale
    p = torch.exp2(qk - lse[..., None]).masked_fill(~mask_t, 0.0)
    p_mm = p.to(dtype).to(ft) if rounding else p
    dv = p_mm.transpose(-1, -2) @ do
    dp = do @ v.transpose(-1, -2)
    ds = p * (dp - delta[..., None])
    ds_mm = ds.to(dtype).to(ft) if rounding else ds
    dk = (ds_mm.transpose(-1, -2) @ q) * scale
    dq = (ds_mm @ k) * scale
    if rounding:
        return dq.to(dtype), dk.to(dtype), dv.to(dtype)
    return dq, dk, dv
