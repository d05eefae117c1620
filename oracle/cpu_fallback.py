"""CPU restatement of the reference's own CPU attention paths — TEST INFRASTRUCTURE ONLY.

Used only by bench.py's ``cpu_baseline`` leg (timed on the GPU box's host cores) and by tests that
check it against the numpy oracle. Never imported by the product (``sps_amd``).

* ``dense_sdpa_fwd_bwd``: the reference's correctness reference for the prefill kernels, an additive
  mask (0 on visible pairs, -inf elsewhere) fed to ``torch.nn.functional.scaled_dot_product_attention``
  in fp32, with the backward from autograd (src/modeling/tests/attention/triton/
  test_sps_attention.py:25-73, test_full_flash_attention.py:29-59). The dense SPS forward of the
  reference has no CPU path of its own (src/modeling/models/sps/core.py:63-67), so this is the CPU
  form of that computation the reference ships.
* ``stepwise_sps_forward``: the reference's CPU inference path for an SPS-family layer
  (``forward_efficient`` on CPU, src/modeling/models/reverse_sps/inference.py:437-457,766-830, slot
  roles sps/inference.py:8-12): token by token, each of the two slots' queries attends through
  ``masked_kv_attention``'s CPU fallback to the window ring, the retained segment and the current
  token's keys, and then the ring takes the window slot's K/V and the retained segment the other's.
* ``padded_masked_kv_attention``: the CPU fallback of ``masked_kv_attention``
  (src/modeling/models/utils/decode_attention.py:637-698): every segment is cut to its largest live
  length, segments and the always-visible extra keys are concatenated into one zero-padded K/V
  tensor with a boolean validity mask, and one SDPA call runs over it in ``attn_dtype``.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F


def dense_sdpa_fwd_bwd(q, k, v, do, mask_bool, sm_scale):
    """q, k, v, do: [B, H, N, D] fp32 CPU tensors; mask_bool: [B, N, N] (True = visible).

    Returns (o, dq, dk, dv) in fp32."""
    qr, kr, vr = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    bias = torch.zeros(mask_bool.shape, dtype=q.dtype)
    bias.masked_fill_(~mask_bool, float("-inf"))
    o = F.scaled_dot_product_attention(qr, kr, vr, attn_mask=bias.unsqueeze(1), scale=sm_scale)
    o.backward(do)
    return o.detach(), qr.grad, kr.grad, vr.grad


def _scan_len(storage: int, max_len_cap) -> int:
    if storage == 0:
        return 0
    if max_len_cap is None:
        return storage
    return max(1, min(storage, int(max_len_cap)))


def padded_masked_kv_attention(q, segments, extra_kv, attn_dtype=torch.float32):
    """q: [B, H, D]; segments: list of (k [B,H,S,D], v, lengths [B] or [B,H], max_len_cap);
    extra_kv: list of (k [B,H,D], v [B,H,D]). Returns fp32 [B, H, D]."""
    b, h, d = q.shape
    maxlens = []
    for (k, _, lengths, cap) in segments:
        maxlens.append(0 if lengths.numel() == 0 else min(int(lengths.max()), _scan_len(k.shape[2], cap)))
    total = sum(maxlens) + len(extra_kv)
    if total == 0:
        return torch.zeros((b, h, d), dtype=torch.float32)
    keys = torch.zeros((b, h, total, d), dtype=attn_dtype)
    vals = torch.zeros_like(keys)
    valid = torch.zeros((b, h, total), dtype=torch.bool)
    col = 0
    for (k, v, lengths, _), n in zip(segments, maxlens):
        if n == 0:
            continue
        keys[:, :, col:col + n] = k[:, :, :n]
        vals[:, :, col:col + n] = v[:, :, :n]
        pos = torch.arange(n)
        lens = lengths.view(b, 1, 1) if lengths.dim() == 1 else lengths.view(b, h, 1)
        valid[:, :, col:col + n] = pos.view(1, 1, n) < lens
        col += n
    for ek, ev in extra_kv:
        keys[:, :, col] = ek
        vals[:, :, col] = ev
        valid[:, :, col] = True
        col += 1
    out = F.scaled_dot_product_attention(
        q.to(attn_dtype).reshape(b * h, 1, d), keys.reshape(b * h, total, d), vals.reshape(b * h, total, d),
        attn_mask=valid.reshape(b * h, 1, total), scale=1.0 / math.sqrt(d))
    return out.reshape(b, h, d).float()


def mask_from_docs(family: int, docs_row: np.ndarray, window: int) -> torch.Tensor:
    """[N, N] bool visibility of one batch row, built with torch on the CPU from the predicate of
    sps_oracle.c (causal, same document, temporary keys within `window` tokens)."""
    n = docs_row.shape[0]
    q = torch.arange(n).view(n, 1)
    k = torch.arange(n).view(1, n)
    d = torch.as_tensor(docs_row)
    vis = (k <= q) & (d.view(n, 1) == d.view(1, n))
    if family != 0:
        persistent = (k % 2) == (1 if family == 2 else 0)
        vis &= persistent | ((q // 2 - k // 2) <= window)
    return vis


def stepwise_sps_forward(q, k, v, family: int, window: int, attn_dtype=torch.float32):
    """q, k, v: [B, H, 2T, D] CPU tensors of one document per row (positions 2t input, 2t+1
    <predict>). Returns the [B, H, 2T, D] fp32 outputs of the token-by-token decode path.

    SPS (family 1): the ring holds the last `window` <predict> K/V (window slot 1) and the retained
    segment every earlier input K/V (slot 0); reverse-SPS (family 2) swaps the slots. The input
    query sees ring + retained + the current input key; the <predict> query also the current
    <predict> key."""
    b, h, n, d = q.shape
    t_max = n // 2
    window_slot, retained_slot = (1, 0) if family == 1 else (0, 1)
    ring_k = torch.zeros((b, h, max(window, 1), d), dtype=attn_dtype)
    ring_v = torch.zeros_like(ring_k)
    ret_k = torch.zeros((b, h, t_max, d), dtype=attn_dtype)
    ret_v = torch.zeros_like(ret_k)
    out = torch.zeros((b, h, n, d), dtype=torch.float32)
    qa, ka, va = (x.to(attn_dtype) for x in (q, k, v))
    for t in range(t_max):
        segs = []
        if window > 0:
            segs.append((ring_k, ring_v, torch.full((b,), min(t, window), dtype=torch.int64), window))
        segs.append((ret_k, ret_v, torch.full((b, h), t, dtype=torch.int64), t_max))
        cur = [(ka[:, :, 2 * t + s], va[:, :, 2 * t + s]) for s in (0, 1)]
        out[:, :, 2 * t] = padded_masked_kv_attention(qa[:, :, 2 * t], segs, cur[:1], attn_dtype)
        out[:, :, 2 * t + 1] = padded_masked_kv_attention(qa[:, :, 2 * t + 1], segs, cur, attn_dtype)
        if window > 0:
            ring_k[:, :, t % window] = cur[window_slot][0]
            ring_v[:, :, t % window] = cur[window_slot][1]
        ret_k[:, :, t] = cur[retained_slot][0]
        ret_v[:, :, t] = cur[retained_slot][1]
    return out
