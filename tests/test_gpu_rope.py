"""Parity of the fused RoPE / cast kernel with the float64 oracle (GPU)."""

import math

import numpy as np
import pytest
import torch

from oracle import rope as R
from sps_amd import rope as SR
from sps_amd.attention import sps_sliding_attention

pytestmark = pytest.mark.gpu


def _freqs(d, t, theta=10000.0):
    inv = 1.0 / (theta ** (torch.arange(0, d, 2)[: d // 2].float() / d))
    return torch.polar(torch.ones(t, d // 2), torch.outer(torch.arange(t).float(), inv))  # complex64, as the reference


def _check(got, ref64, dtype):
    # The kernel's fp32 products and sum (error ~2^-23 of the unit-magnitude terms, so absolute:
    # 1e-6 here, where the inputs are ~N(0, 1)) rounded once to `dtype`: within one unit in the
    # last place of the output type plus that absolute term, and almost always identical to the
    # float64 result rounded to `dtype`.
    expect = torch.from_numpy(ref64).to(dtype)
    g = got.float().cpu()
    e = expect.float()
    ulp = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10, torch.float32: 2.0 ** -22}[dtype]
    bad = (g - e).abs() > ulp * e.abs() + 1e-6
    assert not bad.any(), f"{int(bad.sum())} elements beyond one ulp"
    assert (g == e).float().mean() > (0.97 if dtype != torch.float32 else 0.5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("per_sequence", [False, True])
def test_apply_rotary_emb_matches_oracle(dtype, per_sequence):
    g = torch.Generator().manual_seed(7)
    B, T, H, D = 2, 33, 3, 64
    xq = torch.randn(B, T, H, D, generator=g).to(dtype)
    xk = torch.randn(B, T, H, D, generator=g).to(dtype)
    table = _freqs(D, 64)
    if per_sequence:
        pos = torch.randint(0, 64, (B, T), generator=g)
        f = table[pos]
    else:
        f = table[:T]
    q_out, k_out = SR.apply_rotary_emb(xq.cuda(), xk.cuda(), f.cuda())
    torch.cuda.synchronize()
    assert q_out.dtype == dtype and q_out.shape == xq.shape
    _check(q_out, R.rope(xq.float().numpy(), f.numpy()), dtype)
    _check(k_out, R.rope(xk.float().numpy(), f.numpy()), dtype)


@pytest.mark.parametrize("D", [16, 32, 128, 256])
def test_rope_qkv_from_packed_projection(D):
    # q, k, v as the attention modules split them: views of one [B, T, 3C] projection (fp32).
    g = torch.Generator().manual_seed(D)
    B, T, H = 2, 40, 4
    qkv = torch.randn(B, T, 3 * H * D, generator=g).cuda()
    q, k, v = (t.view(B, T, H, D) for t in qkv.split(H * D, dim=2))
    f = _freqs(D, T)
    qo, ko, vo = SR.rope_qkv_for_attention(q, k, v, f.cuda())
    torch.cuda.synchronize()
    assert qo.shape == (B, H, T, D) and qo.dtype == torch.bfloat16
    _check(qo.transpose(1, 2), R.rope(q.cpu().numpy(), f.numpy()), torch.bfloat16)
    _check(ko.transpose(1, 2), R.rope(k.cpu().numpy(), f.numpy()), torch.bfloat16)
    assert torch.equal(vo.transpose(1, 2).cpu(), v.cpu().to(torch.bfloat16))


def test_fused_pre_attention_feeds_the_attention_kernel():
    # sps/core.py:45-77: RoPE, transpose, cast, then sps_sliding_attention. The fused step gives the
    # same attention output as the unfused op sequence (torch RoPE on the GPU, transpose, cast).
    g = torch.Generator().manual_seed(3)
    B, T2, H, D = 2, 256, 4, 64
    qkv = torch.randn(B, T2, 3 * H * D, generator=g).cuda()
    q, k, v = (t.view(B, T2, H, D) for t in qkv.split(H * D, dim=2))
    f = _freqs(D, T2).cuda()
    docs = torch.zeros(B, T2, dtype=torch.long, device="cuda")
    qo, ko, vo = SR.rope_qkv_for_attention(q, k, v, f)
    y = sps_sliding_attention(qo, ko, vo, 1 / math.sqrt(D), 16, documents_idx_BxT=docs)

    def ref_rope(x):
        z = torch.view_as_complex(x.float().reshape(*x.shape[:-1], -1, 2))
        return torch.view_as_real(z * f.view(1, T2, 1, D // 2)).flatten(3)

    qr = ref_rope(q).transpose(1, 2).to(torch.bfloat16)
    kr = ref_rope(k).transpose(1, 2).to(torch.bfloat16)
    vr = v.transpose(1, 2).to(torch.bfloat16)
    y_ref = sps_sliding_attention(qr, kr, vr, 1 / math.sqrt(D), 16, documents_idx_BxT=docs)
    torch.testing.assert_close(y.float(), y_ref.float(), atol=2e-2, rtol=1e-2)
