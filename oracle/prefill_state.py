"""Prefill -> decode state materialisation reference in numpy (test infrastructure only).

Restates _materialize_prefill_layer_state of lil-lab/sps (src/modeling/models/reverse_sps/
inference.py:568-613) for one layer, updating numpy caches in place:
  rows of the window slot: K/V[:, window_slot::2], of the retained slot: K/V[:, retained_slot::2]
                                                                   inference.py:576-587
  per row b: doc = nonzero(mask[b]) (increasing); n = len(doc); skip the row when n == 0
                                                                   inference.py:589-593
  retained K/V[b, :, :n] = retained rows at doc (transposed to [H, n, D]); retained len[b, :] = n
                                                                   inference.py:595-601
  if window_tokens > 0: w = doc[-window_tokens:]; ring K/V[b, :, :len(w)] = window rows at w;
    ring len[b] = len(w); ring pos[b] = 0                          inference.py:603-613
The caller casts to the cache dtype as the reference's .to(dtype=...) does.
"""

from __future__ import annotations

import numpy as np


def materialize(k, v, mask, window_slot, retained_slot, ring_k, ring_v, ring_len, ring_pos, ret_k, ret_v, ret_len,
                window_tokens):
    k_w, v_w = k[:, window_slot::2], v[:, window_slot::2]
    k_r, v_r = k[:, retained_slot::2], v[:, retained_slot::2]
    for b in range(mask.shape[0]):
        doc = np.flatnonzero(mask[b])
        n = doc.size
        if n == 0:
            continue
        ret_k[b, :, :n, :] = np.transpose(k_r[b, doc], (1, 0, 2))
        ret_v[b, :, :n, :] = np.transpose(v_r[b, doc], (1, 0, 2))
        ret_len[b, :] = n
        if window_tokens > 0:
            w = doc[-window_tokens:]
            ring_k[b, :, : w.size, :] = np.transpose(k_w[b, w], (1, 0, 2))
            ring_v[b, :, : w.size, :] = np.transpose(v_w[b, w], (1, 0, 2))
            ring_len[b] = w.size
            ring_pos[b] = 0
