"""Document ids on the GPU (sps_document_ids) against the known answers of the reference's id tests
and the pinned oracle (oracle/docidx.py). Bit-exact (integer work)."""

import numpy as np
import pytest
import torch

from oracle import docidx
from sps_amd import document_ids, left_padded_document_ids

pytestmark = pytest.mark.gpu

EOS, PAD = 50256, 50255

# core/test_document_idx.py:22-115 (token rows -> ids), restated.
KATS = [
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
]


@pytest.mark.parametrize("idx,expected", KATS)
@pytest.mark.parametrize("tok_dtype", [torch.int64, torch.int32])
def test_known_answers(idx, expected, tok_dtype):
    tok = torch.tensor(idx, dtype=tok_dtype, device="cuda")
    got = left_padded_document_ids(tok, eos_token_id=EOS, pad_token_id=PAD)
    assert got.dtype == tok_dtype
    assert got.cpu().tolist() == expected
    inter = document_ids(tok, eos_token_id=EOS, pad_token_id=PAD)
    assert inter.cpu().tolist() == np.repeat(np.array(expected), 2, axis=1).tolist()


def _random_rows(rng, b, t, max_pads):
    rows = rng.integers(0, 50, size=(b, t))
    rows[rng.random((b, t)) < 0.05] = EOS
    for i in range(b):
        p = int(rng.integers(0, max_pads + 1))
        rows[i, :p] = PAD
    return rows


@pytest.mark.parametrize("t", [1, 7, 1023, 1024, 1025, 4096, 10000])
def test_against_oracle(t):
    # Rows longer than one 1024-token tile carry their counts across tiles.
    rng = np.random.default_rng(t)
    rows = _random_rows(rng, 3, t, max_pads=min(t, 1500))
    rows[1, :] = PAD  # an all-pad row is allowed (ids 0 .. T-1)
    want = docidx.document_idx(rows, EOS, PAD)
    tok = torch.tensor(rows, device="cuda")
    got = document_ids(tok, eos_token_id=EOS, pad_token_id=PAD, repeat=1)
    assert np.array_equal(got.cpu().numpy(), want)
    got32 = document_ids(tok.to(torch.int32), eos_token_id=EOS, pad_token_id=PAD, repeat=2, dtype=torch.int32)
    assert got32.dtype == torch.int32
    assert np.array_equal(got32.cpu().numpy(), docidx.interleave(want))


@pytest.mark.parametrize("seed", range(4))
def test_random_sweep(seed):
    # Random batch sizes, lengths (across the 1024-token tile boundaries), pad counts, EOS densities,
    # token and id dtypes and repeat factors: bit-exact against the oracle.
    rng = np.random.default_rng(7000 + seed)
    for _ in range(4):
        b, t = int(rng.integers(1, 6)), int(rng.integers(1, 5000))
        rows = _random_rows(rng, b, t, max_pads=int(rng.integers(0, t + 1)))
        if rng.random() < 0.3:  # EOS runs of random density
            rows[rng.random(rows.shape) < float(rng.uniform(0.0, 0.5))] = EOS
            for r in range(b):  # keep the rows left padded: no pad after a real token
                first_real = int(np.argmax(rows[r] != PAD)) if (rows[r] != PAD).any() else t
                rows[r, first_real:][rows[r, first_real:] == PAD] = 1
        want = docidx.document_idx(rows, EOS, PAD)
        tok_dtype = torch.int64 if rng.random() < 0.5 else torch.int32
        out_dtype = torch.int64 if rng.random() < 0.5 else torch.int32
        repeat = int(rng.integers(1, 3))
        got = document_ids(torch.tensor(rows, device="cuda").to(tok_dtype), eos_token_id=EOS, pad_token_id=PAD,
                           repeat=repeat, dtype=out_dtype)
        assert got.dtype == out_dtype
        assert np.array_equal(got.cpu().numpy(), want if repeat == 1 else docidx.interleave(want))


def test_strided_rows():
    rng = np.random.default_rng(2)
    rows = _random_rows(rng, 4, 300, max_pads=20)
    big = torch.zeros((4, 512), dtype=torch.int64, device="cuda")
    big[:, 100:400] = torch.tensor(rows, device="cuda")
    got = document_ids(big[:, 100:400], eos_token_id=EOS, pad_token_id=PAD)
    assert np.array_equal(got.cpu().numpy(), docidx.interleave(docidx.document_idx(rows, EOS, PAD)))


def test_pad_after_real_raises():
    # model.py:50-57: rows must be left padded.
    tok = torch.tensor([[PAD, 1, 2, 3], [1, PAD, 2, 3], [PAD, PAD, PAD, PAD]], device="cuda")
    with pytest.raises(ValueError, match=r"\[1\]"):
        document_ids(tok, eos_token_id=EOS, pad_token_id=PAD)
    # without validation the ids still follow the formula
    ids = document_ids(tok, eos_token_id=EOS, pad_token_id=PAD, repeat=1, validate=False)
    assert ids[0].tolist() == [0, 1, 1, 1] and ids[2].tolist() == [0, 1, 2, 3]


def test_ids_feed_the_attention_kernel():
    # The ids drive the document mask exactly as the repeat_interleave(2) of the torch ids does.
    from oracle import mask as M
    from sps_amd import attention as SA
    from sps_amd import _native as N

    rng = np.random.default_rng(9)
    rows = _random_rows(rng, 2, 400, max_pads=30)
    tok = torch.tensor(rows, device="cuda")
    ids = document_ids(tok, eos_token_id=EOS, pad_token_id=PAD)
    got = SA.attention_mask(N.FAMILY_SPS, 800, ids, window=16).cpu().numpy().astype(bool)
    want = M.batch_mask(N.FAMILY_SPS, docidx.interleave(docidx.document_idx(rows, EOS, PAD)), window=16)
    assert (got == want).all()
