"""Visibility mask oracle (test infrastructure only).

Two independent restatements of the reference predicate:
  * ``mask_c`` / ``count_c``: the C loop in sps_oracle.c (boolean predicate, pair by pair);
  * ``mask_np``: a numpy construction that follows the reference kernel's additive-bias steps
    (triton_sps_flash_attention.py:81-111; triton_reverse_sps_flash_attention.py:106-137;
    triton_full_flash_attention.py:95-104): bias = where(k_is_persistent, persistent_bias,
    normal_bias), self-persistent exemption, + causal and document biases; visible = bias == 0.
"""

from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "libsps_oracle.so"

FAMILY_FULL, FAMILY_SPS, FAMILY_REVERSE_SPS = 0, 1, 2

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def _load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = C.CDLL(str(LIB))
        lib.sps_oracle_visible.restype = C.c_int
        lib.sps_oracle_visible.argtypes = [C.c_int, C.c_int64, C.c_int64, C.c_int, C.c_int64, C.c_int64,
                                           C.c_int64, C.c_int, C.c_int64]
        lib.sps_oracle_mask.restype = None
        lib.sps_oracle_mask.argtypes = [C.c_int, C.c_int64, C.c_void_p, C.c_int64, C.c_int, C.c_int64, C.c_void_p]
        lib.sps_oracle_count.restype = C.c_int64
        lib.sps_oracle_count.argtypes = [C.c_int, C.c_int64, C.c_void_p, C.c_int64, C.c_int, C.c_int64]
        _lib = lib
    return _lib


def visible_c(family, q, k, window=0, docs=None, pkw=None) -> bool:
    hd = docs is not None
    return bool(_load().sps_oracle_visible(family, q, k, int(hd), int(docs[q]) if hd else 0,
                                           int(docs[k]) if hd else 0, window, int(pkw is not None),
                                           -1 if pkw is None else pkw))


def mask_c(family: int, n: int, docs=None, window: int = 0, pkw=None) -> np.ndarray:
    """[n, n] uint8 mask of one batch row (rows = queries)."""
    out = np.zeros((n, n), dtype=np.uint8)
    d = None if docs is None else np.ascontiguousarray(np.asarray(docs, dtype=np.int64))
    _load().sps_oracle_mask(family, n, None if d is None else d.ctypes.data, window, int(pkw is not None),
                            -1 if pkw is None else pkw, out.ctypes.data)
    return out


def count_c(family: int, n: int, docs=None, window: int = 0, pkw=None) -> int:
    d = None if docs is None else np.ascontiguousarray(np.asarray(docs, dtype=np.int64))
    return int(_load().sps_oracle_count(family, n, None if d is None else d.ctypes.data, window,
                                        int(pkw is not None), -1 if pkw is None else pkw))


def mask_np(family: int, n: int, docs=None, window: int = 0, pkw=None) -> np.ndarray:
    """Vectorised restatement following the reference's bias construction; bool [n, n]."""
    q = np.arange(n).reshape(n, 1)
    k = np.arange(n).reshape(1, n)
    bias = np.zeros((n, n), dtype=np.float64)
    if family != FAMILY_FULL:
        q_tok, k_tok = q // 2, k // 2
        rel = q_tok - k_tok
        normal_bias = np.where(rel > window, -1.0e6, 0.0)
        persistent_remainder = 1 if family == FAMILY_REVERSE_SPS else 0
        k_is_persistent = (k % 2) == persistent_remainder
        persistent_bias = np.zeros((n, n)) if pkw is None else np.where(rel <= pkw, 0.0, -1.0e6)
        bias = np.where(k_is_persistent, persistent_bias, normal_bias)
        is_self_persistent = (q == k) & k_is_persistent
        bias = np.where(is_self_persistent, 0.0, bias)
    bias = bias + np.where(q >= k, 0.0, -1.0e6)
    if docs is not None:
        d = np.asarray(docs).reshape(-1)
        bias = bias + np.where(d.reshape(n, 1) == d.reshape(1, n), 0.0, -1.0e6)
    return bias == 0.0


def batch_mask(family: int, docs_bn=None, n: int | None = None, window: int = 0, pkw=None, batch: int = 1):
    """[B, n, n] bool mask (docs_bn: [B, n] ids or None)."""
    if docs_bn is None:
        m = mask_c(family, n, None, window, pkw).astype(bool)
        return np.broadcast_to(m, (batch, n, n)).copy()
    docs_bn = np.asarray(docs_bn)
    return np.stack([mask_c(family, docs_bn.shape[1], row, window, pkw).astype(bool) for row in docs_bn])


def sps_pairs_closed_form(doc_lengths, window: int) -> int:
    """Visible pairs of one SPS row made of whole documents (lengths in tokens), no pkw:
    per document of L tokens, L(L+1) persistent pairs + L diagonal temporaries + 2*sum_t min(t, w)."""
    total = 0
    for L in doc_lengths:
        t = np.arange(L)
        total += L * (L + 1) + L + 2 * int(np.minimum(t, window).sum())
    return total


def full_pairs_closed_form(doc_lengths) -> int:
    return int(sum(L * (L + 1) // 2 for L in doc_lengths))
