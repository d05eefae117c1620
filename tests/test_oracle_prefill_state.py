"""The prefill -> decode materialisation oracle against worked examples and the decode-side ring
semantics (CPU only)."""

import numpy as np

from oracle import kv_update as KU
from oracle import prefill_state as PS


def _caches(B, H, D, Sw, Sr):
    z = lambda *s: np.zeros(s, np.float64)  # noqa: E731
    return dict(ring_k=z(B, H, Sw, D), ring_v=z(B, H, Sw, D), ring_len=np.zeros(B, np.int64),
                ring_pos=np.full(B, 7, np.int64), ret_k=z(B, H, Sr, D), ret_v=z(B, H, Sr, D),
                ret_len=np.zeros((B, H), np.int64))


def _kv(B, T, H, D):
    # K[b, n, h, :] = 1000 b + 10 n + h, V = -K: every row says where it came from.
    n = np.arange(2 * T)[None, :, None, None]
    k = 1000.0 * np.arange(B)[:, None, None, None] + 10.0 * n + np.arange(H)[None, None, :, None] + np.zeros(D)
    return k, -k


def test_worked_example():
    B, T, H, D = 2, 5, 2, 4
    k, v = _kv(B, T, H, D)
    mask = np.array([[0, 1, 1, 1, 0], [0, 0, 0, 0, 0]], bool)
    c = _caches(B, H, D, 4, 6)
    PS.materialize(k, v, mask, 1, 0, c["ring_k"], c["ring_v"], c["ring_len"], c["ring_pos"], c["ret_k"], c["ret_v"],
                   c["ret_len"], 2)
    # retained slot 0: positions 2t for t = 1, 2, 3 -> rows 2, 4, 6; ring slot 1, last two tokens -> rows 5, 7
    np.testing.assert_array_equal(c["ret_k"][0, 1, :3, 0], [10 * 2 + 1, 10 * 4 + 1, 10 * 6 + 1])
    np.testing.assert_array_equal(c["ret_v"][0, 0, :3, 0], [-20, -40, -60])
    np.testing.assert_array_equal(c["ring_k"][0, 0, :2, 0], [50, 70])
    assert c["ret_len"][0].tolist() == [3, 3] and c["ring_len"][0] == 2 and c["ring_pos"][0] == 0
    # the empty row is untouched
    assert c["ring_pos"][1] == 7 and (c["ret_k"][1] == 0).all() and c["ret_len"][1].tolist() == [0, 0]


def test_same_key_sets_as_stepwise_decode_updates():
    # Materialising a document == inserting its tokens one by one with the decode update (ring as a
    # set of keys, retained in order), the consistency the dense-vs-stepwise reference tests rely on.
    B, T, H, D, W = 1, 9, 2, 3, 4
    k, v = _kv(B, T, H, D)
    mask = np.zeros((B, T), bool)
    mask[0, 2:] = True
    c = _caches(B, H, D, W, T)
    PS.materialize(k, v, mask, 0, 1, c["ring_k"], c["ring_v"], c["ring_len"], c["ring_pos"], c["ret_k"], c["ret_v"],
                   c["ret_len"], W)
    s = _caches(B, H, D, W, T)
    s["ring_pos"][:] = 0
    for t in np.flatnonzero(mask[0]):
        KU.kv_update(s["ring_k"], s["ring_v"], s["ring_len"], s["ring_pos"], s["ret_k"], s["ret_v"], s["ret_len"],
                     k[:, 2 * t], v[:, 2 * t], k[:, 2 * t + 1], v[:, 2 * t + 1], np.array([True]), W)
    np.testing.assert_array_equal(c["ret_k"], s["ret_k"])
    assert c["ret_len"].tolist() == s["ret_len"].tolist() and c["ring_len"][0] == s["ring_len"][0] == W
    assert sorted(c["ring_k"][0, 1, :, 0]) == sorted(s["ring_k"][0, 1, :, 0])
