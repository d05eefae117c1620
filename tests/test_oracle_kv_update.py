"""The decode KV-update oracle against the reference's known answers and the closed form of a ring
buffer (CPU only)."""

import numpy as np
import pytest

from oracle import kv_update as KU


def _state(B, H, D, window_storage, ret_storage):
    return dict(
        ring_k=np.zeros((B, H, window_storage, D), np.float32), ring_v=np.zeros((B, H, window_storage, D), np.float32),
        ring_len=np.zeros(B, np.int64), ring_pos=np.zeros(B, np.int64),
        ret_k=np.zeros((B, H, ret_storage, D), np.float32), ret_v=np.zeros((B, H, ret_storage, D), np.float32),
        ret_len=np.zeros((B, H), np.int64))


def _step(st, kw, vw, kr, vr, active, window):
    KU.kv_update(st["ring_k"], st["ring_v"], st["ring_len"], st["ring_pos"], st["ret_k"], st["ret_v"], st["ret_len"],
                 kw, vw, kr, vr, active, window)


def test_ring_wraps_without_shifting_reference_kat():
    # delayed_state/test_forward_efficient.py:280-312: window 2, inserts 1, 2, 3 -> ring [3, 2],
    # len 2, pos 1 (values broadcast over heads and D; V = K + 10).
    B, H, D = 1, 2, 4
    st = _state(B, H, D, 2, 5)
    for value in (1.0, 2.0, 3.0):
        k = np.full((B, H, D), value, np.float32)
        _step(st, k, k + 10.0, k, k + 10.0, np.array([True]), 2)
    assert st["ring_len"][0] == 2 and st["ring_pos"][0] == 1
    np.testing.assert_array_equal(st["ring_k"][0, 0, :, 0], [3.0, 2.0])
    np.testing.assert_array_equal(st["ring_v"][0, 1, :, 0], [13.0, 12.0])


@pytest.mark.parametrize("window,n", [(1, 5), (3, 2), (4, 4), (4, 11), (7, 30)])
def test_ring_closed_form(window, n):
    # Insert i lands in slot i mod W; len = min(n, W); pos = n mod W once the ring is full.
    B, H, D = 2, 3, 2
    st = _state(B, H, D, window, n + 1)
    for i in range(n):
        k = np.full((B, H, D), float(i), np.float32)
        _step(st, k, -k, k, -k, np.array([True, True]), window)
    assert (st["ring_len"] == min(n, window)).all()
    assert (st["ring_pos"] == ((n % window) if n >= window else 0)).all()
    for s in range(min(n, window)):
        last = max(i for i in range(n) if i % window == s)
        assert (st["ring_k"][:, :, s, :] == last).all() and (st["ring_v"][:, :, s, :] == -last).all()
    # Retained append: every insert in order.
    assert (st["ret_len"] == n).all()
    np.testing.assert_array_equal(st["ret_k"][1, 2, :n, 0], np.arange(n, dtype=np.float32))


def test_retained_stops_at_storage_and_inactive_rows_are_untouched():
    B, H, D = 2, 2, 3
    st = _state(B, H, D, 2, 3)
    st["ret_len"][0] = [2, 3]
    for i in range(3):
        k = np.full((B, H, D), float(i + 1), np.float32)
        _step(st, k, k, k, k, np.array([True, False]), 2)
    assert st["ret_len"][0].tolist() == [3, 3]
    assert st["ret_k"][0, 0, 2, 0] == 1.0  # only the first insert fitted
    assert (st["ret_k"][0, 1] == 0).all()  # already full
    assert (st["ret_len"][1] == 0).all() and (st["ring_len"][1] == 0) and (st["ret_k"][1] == 0).all()


def test_no_window_updates_only_the_retained_buffer():
    B, H, D = 1, 1, 2
    st = _state(B, H, D, 2, 4)
    k = np.ones((B, H, D), np.float32)
    _step(st, k, k, k, k, np.array([True]), 0)
    assert st["ring_len"][0] == 0 and (st["ring_k"] == 0).all()
    assert st["ret_len"][0, 0] == 1
