"""Document-id generation in numpy (test infrastructure only).

Restates generate_left_padded_document_idx (src/modeling/models/model.py:70-99 of lil-lab/sps) with
explicit loops: a real token's id is pad_count + the number of real EOS tokens strictly before it;
the i-th left-pad token gets id i. SPS rows repeat each token's id for its two positions
(reverse_sps/core.py:226).
"""

from __future__ import annotations

import numpy as np


def document_idx(idx_bt, eos_token_id: int, pad_token_id: int) -> np.ndarray:
    idx_bt = np.asarray(idx_bt)
    out = np.zeros(idx_bt.shape, dtype=np.int64)
    for b, row in enumerate(idx_bt):
        real = row != pad_token_id
        seen_real = False
        for t, r in enumerate(real):
            if r:
                seen_real = True
            elif seen_real:
                raise ValueError("pad after real token")
        pads = int((~real).sum())
        eos_seen = 0
        pad_seen = 0
        for t, tok in enumerate(row):
            if real[t]:
                out[b, t] = pads + eos_seen
                if tok == eos_token_id:
                    eos_seen += 1
            else:
                out[b, t] = pad_seen
                pad_seen += 1
    return out


def interleave(docs_bt) -> np.ndarray:
    return np.repeat(np.asarray(docs_bt), 2, axis=1)
