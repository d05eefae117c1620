"""Dense masked attention forward/backward in float64 numpy (test infrastructure only).

Restates the math of the reference kernels (lil-lab/sps, src/modeling/models/attention/):
  forward  O = softmax(S) V with S = (Q K^T) * sm_scale over visible pairs only,
           LSE2 = log2(sum exp2(S * log2 e))        triton_sps_flash_attention.py:142-269
  backward Delta = rowsum(O * dO)                     triton_reverse_sps_flash_attention.py:334-348
           P = exp2(S log2e - LSE2) on visible pairs, dV = P^T dO, dS = P (dO V^T - Delta),
           dK = sm_scale dS^T Q, dQ = sm_scale dS K   triton_sps_flash_attention.py:272-488
The mask comes from oracle.mask (the boolean form of the reference's additive biases).
"""

from __future__ import annotations

import numpy as np

LOG2E = 1.4426950408889634


def forward(q, k, v, mask, sm_scale):
    """q, k, v: [B, H, N, D]; mask: [B, N, N] bool. Returns (O float64, LSE2 float64 [B, H, N])."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    b, h, n, d = q.shape
    o = np.zeros((b, h, n, d))
    lse2 = np.full((b, h, n), -np.inf)
    for bi in range(b):
        m = mask[bi]
        for hi in range(h):
            s = (q[bi, hi] @ k[bi, hi].T) * sm_scale
            s = np.where(m, s, -np.inf)
            mx = s.max(axis=1, keepdims=True)
            mx = np.where(np.isfinite(mx), mx, 0.0)
            e = np.exp(s - mx)
            l = e.sum(axis=1, keepdims=True)
            p = np.divide(e, l, out=np.zeros_like(e), where=l > 0)
            o[bi, hi] = p @ v[bi, hi]
            with np.errstate(divide="ignore"):
                lse2[bi, hi] = ((np.log(l[:, 0]) + mx[:, 0]) * LOG2E)
    return o, lse2


def backward(q, k, v, do, mask, sm_scale):
    """Returns (dq, dk, dv) float64 for the loss sum(O * dO)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    do = np.asarray(do, dtype=np.float64)
    b, h, n, d = q.shape
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    for bi in range(b):
        m = mask[bi]
        for hi in range(h):
            s = (q[bi, hi] @ k[bi, hi].T) * sm_scale
            s = np.where(m, s, -np.inf)
            mx = s.max(axis=1, keepdims=True)
            mx = np.where(np.isfinite(mx), mx, 0.0)
            e = np.exp(s - mx)
            l = e.sum(axis=1, keepdims=True)
            p = np.divide(e, l, out=np.zeros_like(e), where=l > 0)
            o = p @ v[bi, hi]
            delta = (o * do[bi, hi]).sum(axis=1, keepdims=True)
            dp = do[bi, hi] @ v[bi, hi].T
            ds = p * (dp - delta)
            dv[bi, hi] = p.T @ do[bi, hi]
            dq[bi, hi] = sm_scale * (ds @ k[bi, hi])
            dk[bi, hi] = sm_scale * (ds.T @ q[bi, hi])
    return dq, dk, dv
