"""Decode KV-cache update reference in numpy (test infrastructure only).

Restates the reference's un-fused update path (lil-lab/sps, src/modeling/models/):
  * ring (normal window), per sequence b, when window_tokens > 0   reverse_sps/inference.py:137-168
      full = len[b] >= window_tokens; slot = pos[b] if full else len[b]
      active rows: K/V[b, :, slot, :] = new (every head)
      len[b] += 1 if active and not full; pos[b] = (pos[b] + 1) % window_tokens if active and full
  * retained, per (b, h)                                            reverse_sps/inference.py:240-268
      active rows: K/V[b, h, len[b, h], :] = new; len[b, h] += 1
    with the fused kernel's bound check: nothing happens when len[b, h] >= storage
                                                                    utils/decode_attention_fast.py:95-104
    (a negative length is treated the same way: the reference never produces one).
  * the new K/V are first cast to the cache dtype (Tensor.to)       reverse_sps/inference.py:197-202
The arrays are updated in place; new K/V must already be in the cache dtype (tests cast with torch).
"""

from __future__ import annotations

import numpy as np


def kv_update(ring_k, ring_v, ring_len, ring_pos, ret_k, ret_v, ret_len, k_window, v_window, k_retained,
              v_retained, active, window_tokens: int) -> None:
    """In-place update of numpy caches: ring_k/v [B, H, Sw, D], ring_len/pos [B], ret_k/v
    [B, H, Sr, D], ret_len [B, H], new K/V [B, H, D], active [B] (bool)."""
    B, H = ret_len.shape
    storage = ret_k.shape[2]
    for b in range(B):
        if not bool(active[b]):
            continue
        if window_tokens > 0:
            full = int(ring_len[b]) >= window_tokens
            slot = int(ring_pos[b]) if full else int(ring_len[b])
            ring_k[b, :, slot, :] = k_window[b]
            ring_v[b, :, slot, :] = v_window[b]
            if full:
                ring_pos[b] = (int(ring_pos[b]) + 1) % window_tokens
            else:
                ring_len[b] = int(ring_len[b]) + 1
        for h in range(H):
            n = int(ret_len[b, h])
            if 0 <= n < storage:
                ret_k[b, h, n, :] = k_retained[b, h]
                ret_v[b, h, n, :] = v_retained[b, h]
                ret_len[b, h] = n + 1
