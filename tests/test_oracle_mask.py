"""Pins the mask oracle (CPU): reference KATs, two independent restatements agree, closed forms."""

import numpy as np
import pytest

from oracle import mask as M


def _tok_lists(mask, q_idx, parity):
    """Tokens of keys with the given parity visible to query position q_idx."""
    return [k // 2 for k in range(mask.shape[1]) if k % 2 == parity and mask[q_idx, k]]


@pytest.mark.parametrize("window_size", [0, 1, 2])
def test_reverse_sps_visibility_lists_kat(window_size):
    # Reference KAT: models/reverse_sps/test_forward_efficient.py:130-156 — with T=5, a normal
    # (input, even) or predict (odd) query at token t sees normal tokens max(0, t-w) .. t.
    t = 5
    m = M.mask_c(M.FAMILY_REVERSE_SPS, 2 * t, window=window_size)
    for token_idx in range(t):
        expected = list(range(max(0, token_idx - window_size), token_idx + 1))
        for q_idx in (2 * token_idx, 2 * token_idx + 1):
            assert _tok_lists(m, q_idx, 0) == expected
        # predict keys (persistent for reverse SPS) are visible causally
        assert _tok_lists(m, 2 * token_idx, 1) == list(range(token_idx))
        assert _tok_lists(m, 2 * token_idx + 1, 1) == list(range(token_idx + 1))


def test_sps_window_semantics_kat():
    # Reference kernel semantics (triton_sps_flash_attention.py:88-108): an input query at token t
    # sees predict tokens t-w .. t-1, a predict query sees t-w .. t; both see every input token <= t.
    t, w = 9, 3
    m = M.mask_c(M.FAMILY_SPS, 2 * t, window=w)
    for tok in range(t):
        assert _tok_lists(m, 2 * tok, 1) == list(range(max(0, tok - w), tok))
        assert _tok_lists(m, 2 * tok + 1, 1) == list(range(max(0, tok - w), tok + 1))
        assert _tok_lists(m, 2 * tok, 0) == list(range(tok + 1))
        assert _tok_lists(m, 2 * tok + 1, 0) == list(range(tok + 1))


def test_sps_document_layout_kat():
    # Reference test layout (attention/triton/test_sps_attention.py:82-104): T=16, w=3,
    # docs [0]*6 + [1]*8 + [2]*2 repeated for both slots. No cross-document key is visible.
    docs_t = np.array([0] * 6 + [1] * 8 + [2] * 2)
    docs = np.repeat(docs_t, 2)
    m = M.mask_c(M.FAMILY_SPS, 32, docs, window=3)
    assert not m[np.not_equal.outer(docs, docs)].any()
    # first predict of document 1 (token 6, position 13) sees only input token 6 and itself
    assert np.flatnonzero(m[13]).tolist() == [12, 13]
    assert m.sum() == M.sps_pairs_closed_form([6, 8, 2], 3)


def test_causal_matrix_kat():
    # core/test_masking.py: the full family without documents is the lower-triangular matrix.
    n = 7
    assert (M.mask_c(M.FAMILY_FULL, n).astype(bool) == np.tril(np.ones((n, n), dtype=bool))).all()


def test_persistent_key_window_kat():
    # models/attention/test_persistent_key_window.py:14-51: n_ctx 8, temporary window 8, pkw 1.
    n = 8
    for fam, rem in ((M.FAMILY_SPS, 0), (M.FAMILY_REVERSE_SPS, 1)):
        m = M.mask_c(fam, n, window=n, pkw=1)
        for q in range(n):
            for k in range(q + 1):
                if k % 2 == rem:
                    expect = (q // 2 - k // 2 <= 1) or q == k
                else:
                    expect = True
                assert bool(m[q, k]) == expect, (fam, q, k)


@pytest.mark.parametrize("seed", range(12))
def test_c_and_numpy_restatements_agree(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 40)) * 2
    fam = int(rng.integers(0, 3))
    w = int(rng.integers(-1, 12))
    pkw = None if rng.random() < 0.5 else int(rng.integers(-2, 6))
    docs = None
    if rng.random() < 0.7:
        docs = np.sort(rng.integers(0, 5, size=n)) if rng.random() < 0.7 else rng.integers(0, 3, size=n)
    mc = M.mask_c(fam, n, docs, w, pkw).astype(bool)
    mn = M.mask_np(fam, n, docs, w, pkw)
    assert (mc == mn).all()
    assert M.count_c(fam, n, docs, w, pkw) == int(mc.sum())


@pytest.mark.parametrize("w", [0, 1, 5, 64])
def test_closed_form_pair_counts(w):
    rng = np.random.default_rng(w)
    lengths = [int(x) for x in rng.integers(1, 40, size=5)]
    docs = np.repeat(np.repeat(np.arange(len(lengths)), lengths), 2)
    n = docs.size
    assert M.count_c(M.FAMILY_SPS, n, docs, w) == M.sps_pairs_closed_form(lengths, w)
    assert M.count_c(M.FAMILY_REVERSE_SPS, n, docs, w) == M.sps_pairs_closed_form(lengths, w)
    docs_t = np.repeat(np.arange(len(lengths)), lengths)
    assert M.count_c(M.FAMILY_FULL, docs_t.size, docs_t) == M.full_pairs_closed_form(lengths)


def test_large_window_is_dense_causal():
    # w >= T: every temporary key is in the window, the SPS mask is dense causal over 2T.
    n = 40
    for fam in (M.FAMILY_SPS, M.FAMILY_REVERSE_SPS):
        assert (M.mask_c(fam, n, window=n) == M.mask_c(M.FAMILY_FULL, n)).all()


def test_zero_window_predict_sees_only_itself():
    n = 30
    m = M.mask_c(M.FAMILY_SPS, n, window=0)
    for q in range(1, n, 2):
        assert [k for k in range(1, n, 2) if m[q, k]] == [q]
