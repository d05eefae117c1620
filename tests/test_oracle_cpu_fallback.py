"""The CPU restatement of the reference's CPU paths (bench.py's cpu_baseline leg) agrees with the
float64 numpy oracle, so the baseline times the same computation the GPU kernels perform."""

import math

import numpy as np
import torch

from oracle import attention as A
from oracle import cpu_fallback as CF
from oracle import decode as Dc
from oracle import mask as M


def test_mask_from_docs_matches_c_predicate():
    rng = np.random.default_rng(0)
    for family, n, w in ((1, 64, 3), (2, 50, 0), (0, 40, 0), (1, 96, 100)):
        docs = np.sort(rng.integers(0, 4, size=n))
        got = CF.mask_from_docs(family, docs, w).numpy()
        want = M.mask_c(family, n, docs, w).astype(bool)
        assert (got == want).all()


def test_dense_sdpa_matches_oracle():
    g = torch.Generator().manual_seed(1)
    b, h, n, d = 1, 2, 48, 16
    q, k, v, do = (torch.randn((b, h, n, d), generator=g) for _ in range(4))
    docs = np.repeat(np.array([0] * 10 + [1] * 14), 2)
    mask = CF.mask_from_docs(1, docs, 3).unsqueeze(0)
    o, dq, dk, dv = CF.dense_sdpa_fwd_bwd(q, k, v, do, mask, 0.25)
    m = mask.numpy()
    o_ref, _ = A.forward(q.numpy(), k.numpy(), v.numpy(), m, 0.25)
    grads = A.backward(q.numpy(), k.numpy(), v.numpy(), do.numpy(), m, 0.25)
    np.testing.assert_allclose(o.numpy(), o_ref, atol=1e-5)
    for got, want in zip((dq, dk, dv), grads):
        np.testing.assert_allclose(got.numpy(), want, atol=1e-4)


def test_padded_masked_kv_attention_matches_oracle():
    g = torch.Generator().manual_seed(2)
    b, h, d = 3, 2, 32
    k0, v0 = torch.randn((b, h, 9, d), generator=g), torch.randn((b, h, 9, d), generator=g)
    k1, v1 = torch.randn((b, h, 20, d), generator=g), torch.randn((b, h, 20, d), generator=g)
    l0 = torch.tensor([9, 4, 0])
    l1 = torch.tensor([[3, 20], [0, 7], [11, 1]])
    q = torch.randn((b, h, d), generator=g)
    ex = [(torch.randn((b, h, d), generator=g), torch.randn((b, h, d), generator=g))]
    got = CF.padded_masked_kv_attention(q, [(k0, v0, l0, None), (k1, v1, l1, 15)], ex)
    want = Dc.attend(q.numpy().reshape(b, 1, h, d),
                     [(k0.numpy(), v0.numpy(), l0.numpy(), None), (k1.numpy(), v1.numpy(), l1.numpy(), 15)],
                     [(ex[0][0].numpy(), ex[0][1].numpy())], [1], 1)[:, 0]
    np.testing.assert_allclose(got.numpy(), want, atol=1e-5)
    assert math.isfinite(float(got.abs().max()))


import pytest


@pytest.mark.parametrize("family,window", [(1, 3), (1, 0), (2, 4), (1, 64)])
def test_stepwise_decode_path_matches_dense_oracle(family, window):
    # The token-by-token CPU path (ring + retained + current keys per slot) computes the same
    # attention as the dense masked forward over the interleaved sequence of one document.
    g = torch.Generator().manual_seed(family * 10 + window)
    b, h, t, d = 2, 2, 20, 16
    q, k, v = (torch.randn((b, h, 2 * t, d), generator=g) for _ in range(3))
    got = CF.stepwise_sps_forward(q, k, v, family, window)
    mask = M.batch_mask(family, None, n=2 * t, window=window, batch=b)
    want, _ = A.forward(q.numpy(), k.numpy(), v.numpy(), mask, 1 / math.sqrt(d))
    np.testing.assert_allclose(got.numpy(), want, atol=1e-5)
