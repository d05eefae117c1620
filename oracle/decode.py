"""Segmented decode attention reference in float64 numpy (test infrastructure only).

Restates utils/decode_attention.py of lil-lab/sps (src/modeling/models/):
  * a segment contributes its keys t < min(max(len, 0), scan_len)        decode_attention.py:218-223, 381-390
    (scan_len = 0 for empty storage, storage if max_len_cap is None, else max(1, min(storage, cap)))
  * lengths are [B] (shared by heads) or [B, H]                            decode_attention.py:21-32
  * extras are always visible; in the q=2 form slot 0 sees the current input key and slot 1 sees
    the current input and <predict> keys                                  decode_attention.py:354-361
  * softmax with scale 1/sqrt(D), fp32 result, 0 where nothing is visible  decode_attention.py:363-368
and the per-(b,h) loop of the reference test models/attention/test_segmented_q2_attention.py:25-62.
"""

from __future__ import annotations

import math

import numpy as np


def scan_len(storage: int, max_len_cap) -> int:
    if storage == 0:
        return 0
    if max_len_cap is None:
        return storage
    if max_len_cap < 0:
        raise ValueError("max_len_cap must be non-negative")
    return max(1, min(storage, int(max_len_cap)))


def live_len(lengths: np.ndarray, b: int, h: int, scan: int) -> int:
    ln = int(lengths[b]) if lengths.ndim == 1 else int(lengths[b, h])
    return max(0, min(ln, scan))


def attend(q: np.ndarray, segments, extras, extra_masks, nq: int) -> np.ndarray:
    """q: [B, nq, H, D]; segments: list of (k [B,H,S,D], v, lengths, max_len_cap);
    extras: list of (k [B,H,D], v [B,H,D]); extra_masks[e]: bitmask of query slots seeing extra e.
    Returns float64 [B, nq, H, D]."""
    q = np.asarray(q, dtype=np.float64)
    b, _, h, d = q.shape
    scale = 1.0 / math.sqrt(d)
    out = np.zeros((b, nq, h, d))
    for bi in range(b):
        for hi in range(h):
            keys, vals = [], []
            for (k, v, lengths, cap) in segments:
                s = scan_len(k.shape[2], cap)
                n = live_len(np.asarray(lengths), bi, hi, s)
                if n:
                    keys.append(np.asarray(k[bi, hi, :n], dtype=np.float64))
                    vals.append(np.asarray(v[bi, hi, :n], dtype=np.float64))
            for qi in range(nq):
                kk, vv = list(keys), list(vals)
                for e, (ek, ev) in enumerate(extras):
                    if (extra_masks[e] >> qi) & 1:
                        kk.append(np.asarray(ek[bi, hi], dtype=np.float64).reshape(1, d))
                        vv.append(np.asarray(ev[bi, hi], dtype=np.float64).reshape(1, d))
                if not kk:
                    continue
                K = np.concatenate(kk, axis=0)
                V = np.concatenate(vv, axis=0)
                s = K @ q[bi, qi, hi] * scale
                p = np.exp(s - s.max())
                out[bi, qi, hi] = (p / p.sum()) @ V
    return out

