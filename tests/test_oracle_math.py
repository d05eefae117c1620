"""Pins the attention, decode and document-id oracles (CPU)."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import decode as Dc
from oracle import docidx
from oracle import mask as M


def _inputs(b, h, n, d, seed):
    g = np.random.default_rng(seed)
    return [g.standard_normal((b, h, n, d)) for _ in range(4)]


@pytest.mark.parametrize("family", [M.FAMILY_FULL, M.FAMILY_SPS, M.FAMILY_REVERSE_SPS])
def test_attention_oracle_matches_torch_autograd(family):
    # The hand-written forward/backward formulas against float64 torch autograd of masked softmax
    # attention on the same inputs (independent derivation of the gradients).
    b, h, n, d = 2, 2, 24, 16
    q, k, v, do = _inputs(b, h, n, d, 3)
    docs = np.repeat(np.array([[0] * 5 + [1] * 7, [3] * 12]), 2, axis=1)
    mask = M.batch_mask(family, docs, window=2)
    scale = 1.0 / math.sqrt(d)
    o, lse2 = A.forward(q, k, v, mask, scale)
    dq, dk, dv = A.backward(q, k, v, do, mask, scale)

    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    s = torch.einsum("bhqd,bhkd->bhqk", tq, tk) * scale
    s = s.masked_fill(~torch.tensor(mask)[:, None], float("-inf"))
    to = torch.softmax(s, dim=-1) @ tv
    (to * torch.tensor(do)).sum().backward()
    np.testing.assert_allclose(o, to.detach().numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(lse2, torch.logsumexp(s, dim=-1).detach().numpy() / math.log(2), rtol=1e-10)
    np.testing.assert_allclose(dq, tq.grad.numpy(), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dk, tk.grad.numpy(), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dv, tv.grad.numpy(), rtol=1e-9, atol=1e-11)


def test_attention_oracle_finite_difference():
    b, h, n, d = 1, 1, 10, 4
    q, k, v, do = _inputs(b, h, n, d, 5)
    mask = M.batch_mask(M.FAMILY_SPS, None, n=n, window=1)
    scale = 0.7
    dq, dk, dv = A.backward(q, k, v, do, mask, scale)
    eps = 1e-6
    for arr, grad in ((q, dq), (k, dk), (v, dv)):
        for idx in [(0, 0, 3, 1), (0, 0, 7, 2), (0, 0, 0, 0)]:
            old = arr[idx]
            arr[idx] = old + eps
            fp = (A.forward(q, k, v, mask, scale)[0] * do).sum()
            arr[idx] = old - eps
            fm = (A.forward(q, k, v, mask, scale)[0] * do).sum()
            arr[idx] = old
            assert abs((fp - fm) / (2 * eps) - grad[idx]) < 1e-6


def test_attention_oracle_uniform_scores_give_mean_and_count():
    # Zero queries: every visible key has the same score, so O is the mean of the visible V rows and
    # 2**LSE2 is the number of visible keys (the property the GPU count test relies on).
    n, d = 20, 8
    rng = np.random.default_rng(0)
    v = rng.standard_normal((1, 1, n, d))
    z = np.zeros((1, 1, n, d))
    mask = M.batch_mask(M.FAMILY_SPS, None, n=n, window=2)
    o, lse2 = A.forward(z, z, v, mask, 0.125)
    for qi in range(n):
        vis = mask[0, qi]
        np.testing.assert_allclose(o[0, 0, qi], v[0, 0, vis].mean(axis=0), rtol=1e-12)
        assert round(2 ** lse2[0, 0, qi]) == vis.sum()


def _q2_reference_loop(q, segments, cnk, cnv, cpk, cpv):
    # Restatement of models/attention/test_segmented_q2_attention.py:25-62 (explicit loops).
    bsz, _, n_head, head_dim = q.shape
    out = np.zeros(q.shape)
    scale = 1.0 / math.sqrt(head_dim)
    for bi in range(bsz):
        for hi in range(n_head):
            keys, vals = [], []
            for (k, v, lengths, cap) in segments:
                length = int(lengths[bi]) if lengths.ndim == 1 else int(lengths[bi, hi])
                if cap is not None:
                    length = min(length, cap)
                length = max(length, 0)
                if length:
                    keys.append(k[bi, hi, :length])
                    vals.append(v[bi, hi, :length])
            s0k = np.concatenate(keys + [cnk[bi, hi][None]])
            s0v = np.concatenate(vals + [cnv[bi, hi][None]])
            s1k = np.concatenate(keys + [cnk[bi, hi][None], cpk[bi, hi][None]])
            s1v = np.concatenate(vals + [cnv[bi, hi][None], cpv[bi, hi][None]])
            for slot, (kk, vv) in enumerate(((s0k, s0v), (s1k, s1v))):
                s = kk @ q[bi, slot, hi] * scale
                p = np.exp(s - s.max())
                out[bi, slot, hi] = (p / p.sum()) @ vv
    return out


@pytest.mark.parametrize("first_lengths", ["shared", "empty"])
def test_decode_oracle_matches_reference_test_semantics(first_lengths):
    rng = np.random.default_rng(123)
    bsz, n_head, head_dim = 2, 3, 16
    q = rng.standard_normal((bsz, 2, n_head, head_dim))
    k0 = rng.standard_normal((bsz, n_head, 7, head_dim))
    v0 = rng.standard_normal(k0.shape)
    k1 = rng.standard_normal((bsz, n_head, 11, head_dim))
    v1 = rng.standard_normal(k1.shape)
    if first_lengths == "empty":
        len0, cap0 = np.zeros(bsz, dtype=np.int64), 0
    else:
        len0, cap0 = np.array([2, 5]), 5
    len1 = np.array([[1, 3, 6], [2, 4, 7]])
    segs = [(k0, v0, len0, cap0), (k1, v1, len1, 8)]
    cur = [rng.standard_normal((bsz, n_head, head_dim)) for _ in range(4)]
    got = Dc.attend(q, segs, [(cur[0], cur[1]), (cur[2], cur[3])], [0b11, 0b10], 2)
    want = _q2_reference_loop(q, segs, *cur)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_decode_scan_len_semantics():
    # decode_attention.py:381-390
    assert Dc.scan_len(0, None) == 0
    assert Dc.scan_len(9, None) == 9
    assert Dc.scan_len(9, 0) == 1
    assert Dc.scan_len(9, 4) == 4
    assert Dc.scan_len(9, 20) == 9
    with pytest.raises(ValueError):
        Dc.scan_len(9, -1)


def test_dense_sps_equals_stepwise_decode():
    # Dense SPS attention (one document) == stepwise decode over ring (predict K/V of the last w
    # tokens) + retained (input K/V of earlier tokens) + current keys: the decode path's slot
    # semantics (sps/inference.py:8-12, reverse_sps/inference.py:437-457) reproduce the dense mask.
    t, w, d = 9, 3, 8
    rng = np.random.default_rng(7)
    q, k, v = (rng.standard_normal((1, 1, 2 * t, d)) for _ in range(3))
    mask = M.batch_mask(M.FAMILY_SPS, None, n=2 * t, window=w)
    dense, _ = A.forward(q, k, v, mask, 1.0 / math.sqrt(d))
    for tok in range(t):
        ring_toks = list(range(max(0, tok - w), tok))
        ring_k = np.zeros((1, 1, w, d))
        ring_v = np.zeros((1, 1, w, d))
        for i, s in enumerate(ring_toks):
            ring_k[0, 0, i] = k[0, 0, 2 * s + 1]
            ring_v[0, 0, i] = v[0, 0, 2 * s + 1]
        ret_k = np.zeros((1, 1, t, d))
        ret_v = np.zeros((1, 1, t, d))
        for s in range(tok):
            ret_k[0, 0, s] = k[0, 0, 2 * s]
            ret_v[0, 0, s] = v[0, 0, 2 * s]
        segs = [(ring_k, ring_v, np.array([len(ring_toks)]), w), (ret_k, ret_v, np.array([[tok]]), t)]
        qq = np.stack([q[0, 0, 2 * tok], q[0, 0, 2 * tok + 1]]).reshape(1, 2, 1, d)
        extras = [(k[:, :, 2 * tok], v[:, :, 2 * tok]), (k[:, :, 2 * tok + 1], v[:, :, 2 * tok + 1])]
        out = Dc.attend(qq, segs, extras, [0b11, 0b10], 2)
        np.testing.assert_allclose(out[0, 0, 0], dense[0, 0, 2 * tok], rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(out[0, 1, 0], dense[0, 0, 2 * tok + 1], rtol=1e-10, atol=1e-12)


EOS, PAD = 50256, 50255


@pytest.mark.parametrize(
    "idx,expected",
    [
        ([[1, 2, 3, 4, 5, 6, 7, 8, 9, 10]], [[0] * 10]),
        ([[1, 2, 3, EOS, 4, 5, 6, 7, 8, 9]], [[0, 0, 0, 0, 1, 1, 1, 1, 1, 1]]),
        ([[1, 2, EOS, 3, 4, EOS, 5, 6, 7, 8]], [[0, 0, 0, 1, 1, 1, 2, 2, 2, 2]]),
        ([[EOS, 1, 2, 3, 4]], [[0, 1, 1, 1, 1]]),
        ([[1, 2, 3, 4, EOS]], [[0, 0, 0, 0, 0]]),
        ([[1, EOS, EOS, EOS, 2, 3]], [[0, 0, 1, 2, 3, 3]]),
        ([[PAD, PAD, 1, 2, EOS, 3, 4]], [[0, 1, 2, 2, 2, 3, 3]]),
        (
            [[1, 2, EOS, 3, 4, 5, 6, 7, 8, 9], [1, EOS, 2, 3, EOS, 4, 5, 6, 7, 8], [1, 2, 3, 4, 5, 6, 7, 8, 9, 10]],
            [[0, 0, 0, 1, 1, 1, 1, 1, 1, 1], [0, 0, 1, 1, 1, 2, 2, 2, 2, 2], [0] * 10],
        ),
    ],
)
def test_document_idx_kats(idx, expected):
    # KATs of core/test_document_idx.py:22-115.
    assert docidx.document_idx(idx, EOS, PAD).tolist() == expected
