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


@pytest.mark.parametrize("seed", range(4))
def test_apply_rotary_emb_random_sweep(seed):
    # Random shapes, head dims (multiples of 8), dtypes and shared or per-sequence frequency tables:
    # within one output rounding of the float64 oracle.
    rng = np.random.default_rng(8000 + seed)
    g = torch.Generator().manual_seed(seed)
    for _ in range(4):
        B, T, H = int(rng.integers(1, 4)), int(rng.integers(1, 200)), int(rng.integers(1, 6))
        D = 8 * int(rng.integers(1, 33))
        dtype = (torch.bfloat16, torch.float16, torch.float32)[int(rng.integers(3))]
        xq = torch.randn(B, T, H, D, generator=g).to(dtype)
        xk = torch.randn(B, T, H, D, generator=g).to(dtype)
        table = _freqs(D, T + 17)
        f = table[torch.randint(0, T + 17, (B, T), generator=g)] if rng.random() < 0.5 else table[:T]
        q_out, k_out = SR.apply_rotary_emb(xq.cuda(), xk.cuda(), f.cuda())
        torch.cuda.synchronize()
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


def _reference_rope_autograd(x64, f):
    # The reference's op sequence (model.py:201-230: view_as_complex of the fp32 input, times the
    # complex frequencies, view_as_real), in float64 on the CPU, differentiated by torch autograd.
    z = torch.view_as_complex(x64.reshape(*x64.shape[:-1], -1, 2))
    ff = f.to(torch.complex128)
    ff = ff.view(1, ff.shape[0], 1, ff.shape[1]) if ff.ndim == 2 else ff.view(ff.shape[0], ff.shape[1], 1, ff.shape[2])
    return torch.view_as_real(z * ff).flatten(3)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("per_sequence", [False, True])
def test_apply_rotary_emb_gradients(dtype, per_sequence):
    # The rotation is linear, so the gradient of sum(out * g) is the inverse rotation of g: the
    # backward runs the kernel with the conjugate frequencies. Checked against autograd of the
    # reference formula (one rounding of the result to `dtype`).
    g = torch.Generator().manual_seed(11)
    B, T, H, D = 2, 17, 3, 32
    xq, xk, gq, gk = (torch.randn(B, T, H, D, generator=g).to(dtype) for _ in range(4))
    table = _freqs(D, 32)
    f = table[torch.randint(0, 32, (B, T), generator=g)] if per_sequence else table[:T]
    q = xq.cuda().requires_grad_(True)
    k = xk.cuda().requires_grad_(True)
    qo, ko = SR.apply_rotary_emb(q, k, f.cuda())
    (qo.float() * gq.cuda().float()).sum().add((ko.float() * gk.cuda().float()).sum()).backward()
    for x, grad_out, got in ((xq, gq, q.grad), (xk, gk, k.grad)):
        x64 = x.double().requires_grad_(True)
        (_reference_rope_autograd(x64, f) * grad_out.double()).sum().backward()
        assert got.dtype == dtype
        _check(got, x64.grad.numpy(), dtype)


def test_rope_qkv_for_attention_gradients_reach_the_projection():
    # Training path: projection (fp32, requires grad) -> fused RoPE + bf16 casts -> attention. The
    # gradient reaching the projection equals the one through the reference's op sequence, with the
    # same attention backward feeding both.
    g = torch.Generator().manual_seed(5)
    B, T, H, D = 1, 64, 2, 64
    qkv = torch.randn(B, 2 * T, 3 * H * D, generator=g)
    f = _freqs(D, 2 * T)
    do = torch.randn(B, H, 2 * T, D, generator=g).to(torch.bfloat16).cuda()

    def run(fused):
        x = qkv.cuda().requires_grad_(True)
        q, k, v = (t.view(B, 2 * T, H, D) for t in x.split(H * D, dim=2))
        if fused:
            qa, ka, va = SR.rope_qkv_for_attention(q, k, v, f.cuda())
        else:
            zq = torch.view_as_complex(q.float().reshape(B, 2 * T, H, -1, 2))
            zk = torch.view_as_complex(k.float().reshape(B, 2 * T, H, -1, 2))
            ff = f.cuda().view(1, 2 * T, 1, D // 2)
            qa = torch.view_as_real(zq * ff).flatten(3).transpose(1, 2).to(torch.bfloat16)
            ka = torch.view_as_real(zk * ff).flatten(3).transpose(1, 2).to(torch.bfloat16)
            va = v.transpose(1, 2).to(torch.bfloat16)
        out = sps_sliding_attention(qa, ka, va, 1 / math.sqrt(D), 8)
        out.backward(do)
        return x.grad

    got, want = run(True), run(False)
    assert got is not None and torch.isfinite(got).all()
    torch.testing.assert_close(got, want, atol=2e-2, rtol=1e-2)
