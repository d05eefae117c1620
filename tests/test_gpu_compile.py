"""The attention under torch.compile (GPU): the reference trains torch.compile'd models
(scripts/train.py:420-422, conf/system/default.yaml:6), so the custom ops must trace without a graph
break and give what eager gives. The aot_eager backend runs dynamo and AOTAutograd (the tracing,
fake tensors and registered autograd formula) and executes the captured graph with eager kernels."""

import math

import numpy as np
import pytest
import torch

import sps_amd

pytestmark = pytest.mark.gpu


def _block(q, k, v, docs_2t, docs_t, w):
    a = sps_amd.sps_sliding_attention(q, k, v, 1 / math.sqrt(q.shape[-1]), w, documents_idx_BxT=docs_2t)
    # A Standard-family layer over the input positions of the same rows.
    qi, ki, vi = (t[:, :, 0::2].contiguous() for t in (a, k, v))
    b = sps_amd.full_attention(qi, ki, vi, 1 / math.sqrt(q.shape[-1]), documents_idx_BxT=docs_t)
    r = sps_amd.reverse_sps_sliding_attention(q, k, v, 1 / math.sqrt(q.shape[-1]), w, documents_idx_BxT=docs_2t)
    return a.float().sum() + (b.float() * 0.5).sum() + (r.float() ** 2).mean()


def test_compiled_fullgraph_matches_eager():
    torch._dynamo.reset()
    g = torch.Generator().manual_seed(1)
    b, h, n, d, w = 2, 2, 320, 64, 16
    base = [torch.randn((b, n, h, d), generator=g).to(torch.bfloat16).cuda().transpose(1, 2) for _ in range(3)]
    tok = np.repeat(np.array([[0] * 70 + [1] * 90] * b), 1, axis=1)
    docs_t = torch.tensor(tok, device="cuda")
    docs_2t = docs_t.repeat_interleave(2, dim=1)
    results = []
    for fn in (_block, torch.compile(_block, fullgraph=True, backend="aot_eager")):
        q, k, v = (t.detach().clone().requires_grad_(True) for t in base)
        loss = fn(q, k, v, docs_2t, docs_t, w)
        loss.backward()
        torch.cuda.synchronize()
        results.append((loss.detach(), q.grad, k.grad, v.grad))
    for x, y in zip(*results):
        assert torch.equal(x, y)


def test_compiled_inference_without_grad():
    torch._dynamo.reset()
    q = torch.randn(1, 2, 128, 64, device="cuda").to(torch.bfloat16)
    eager = sps_amd.full_attention(q, q, q, 0.125)
    compiled = torch.compile(lambda x: sps_amd.full_attention(x, x, x, 0.125), fullgraph=True, backend="aot_eager")
    with torch.no_grad():
        assert torch.equal(compiled(q), eager)


def _reference_apply_rotary_emb(xq, xk, freqs_cis):
    # The reference's own formula (model.py:201-230), as the CPU original the installed dispatcher
    # wraps: fp32 complex product, results in the inputs' dtype.
    xq_ = torch.view_as_complex(xq.float().reshape(*xq.shape[:-1], -1, 2))
    xk_ = torch.view_as_complex(xk.float().reshape(*xk.shape[:-1], -1, 2))
    f = freqs_cis.view(1, xq_.shape[1], 1, xq_.shape[-1])
    return torch.view_as_real(xq_ * f).flatten(3).type_as(xq), torch.view_as_real(xk_ * f).flatten(3).type_as(xk)


def test_compiled_block_through_the_installed_rope_matches_eager(monkeypatch):
    # The SPS attention module's forward (sps/core.py:45-80) under torch.compile(fullgraph=True): QKV
    # projection, apply_rotary_emb looked up in modeling.models.model at call time (:50-52) after
    # install_into_modeling() made it the device dispatcher (CUDA tensors -> the HIP RoPE custom op),
    # bf16 casts, sps_sliding_attention, output projection. Output and the projections' gradients
    # equal eager.
    import sys
    import types

    model_mod = types.ModuleType("modeling.models.model")
    model_mod.apply_rotary_emb = _reference_apply_rotary_emb
    monkeypatch.setitem(sys.modules, "modeling.models.model", model_mod)
    sps_amd.install_into_modeling()
    assert model_mod.apply_rotary_emb.__sps_amd_original__ is _reference_apply_rotary_emb
    torch._dynamo.reset()

    b, two_t, h, d, w = 2, 256, 4, 64, 16
    c = h * d
    g = torch.Generator().manual_seed(9)
    x = torch.randn((b, two_t, c), generator=g).cuda()
    inv = 1.0 / (10000.0 ** (torch.arange(0, d, 2).float() / d))
    freqs = torch.polar(torch.ones(two_t, d // 2), torch.outer(torch.arange(two_t).float(), inv)).cuda()
    docs = torch.tensor(np.repeat(np.array([[0] * 50 + [1] * 78] * b), 2, axis=1), device="cuda")
    torch.manual_seed(0)
    c_attn, c_proj = torch.nn.Linear(c, 3 * c).cuda(), torch.nn.Linear(c, c).cuda()

    def block(x):
        from modeling.models.model import apply_rotary_emb

        q, k, v = c_attn(x).split(c, dim=2)
        q, k = q.view(b, two_t, h, d), k.view(b, two_t, h, d)
        v = v.view(b, two_t, h, d).transpose(1, 2)
        q, k = apply_rotary_emb(q, k, freqs_cis=freqs)
        q, k, v = q.transpose(1, 2).to(torch.bfloat16), k.transpose(1, 2).to(torch.bfloat16), v.to(torch.bfloat16)
        y = sps_amd.sps_sliding_attention(q, k, v, 1 / math.sqrt(d), w, documents_idx_BxT=docs)
        y = y.transpose(1, 2).contiguous().view(b, two_t, c).to(c_proj.weight.dtype)
        return c_proj(y).square().mean()

    results = []
    for fn in (block, torch.compile(block, fullgraph=True, backend="aot_eager")):
        for p in (*c_attn.parameters(), *c_proj.parameters()):
            p.grad = None
        loss = fn(x)
        loss.backward()
        torch.cuda.synchronize()
        results.append([loss.detach()] + [p.grad.clone() for p in (*c_attn.parameters(), *c_proj.parameters())])
    for got, want in zip(results[1], results[0]):
        torch.testing.assert_close(got, want, atol=0, rtol=0)


def test_inductor_compiled_block_matches_eager(monkeypatch):
    # The same attention-module forward under the default torch.compile backend (inductor), as the
    # reference trains: the surrounding projection, casts and loss are compiled by inductor, the RoPE
    # and attention stay the library's custom ops (extern calls in the compiled graph). Fused
    # elementwise work and reductions may round differently from eager, so the comparison has a
    # tolerance; the attention itself sees the same inputs either way.
    import sys
    import types

    model_mod = types.ModuleType("modeling.models.model")
    model_mod.apply_rotary_emb = _reference_apply_rotary_emb
    monkeypatch.setitem(sys.modules, "modeling.models.model", model_mod)
    sps_amd.install_into_modeling()
    torch._dynamo.reset()

    b, two_t, h, d, w = 2, 256, 4, 64, 16
    c = h * d
    g = torch.Generator().manual_seed(11)
    x = torch.randn((b, two_t, c), generator=g).cuda()
    inv = 1.0 / (10000.0 ** (torch.arange(0, d, 2).float() / d))
    freqs = torch.polar(torch.ones(two_t, d // 2), torch.outer(torch.arange(two_t).float(), inv)).cuda()
    docs = torch.tensor(np.repeat(np.array([[0] * 60 + [1] * 68] * b), 2, axis=1), device="cuda")
    torch.manual_seed(0)
    c_attn, c_proj = torch.nn.Linear(c, 3 * c).cuda(), torch.nn.Linear(c, c).cuda()

    def block(x):
        from modeling.models.model import apply_rotary_emb

        q, k, v = c_attn(x).split(c, dim=2)
        q, k = q.view(b, two_t, h, d), k.view(b, two_t, h, d)
        v = v.view(b, two_t, h, d).transpose(1, 2)
        q, k = apply_rotary_emb(q, k, freqs_cis=freqs)
        q, k, v = q.transpose(1, 2).to(torch.bfloat16), k.transpose(1, 2).to(torch.bfloat16), v.to(torch.bfloat16)
        y = sps_amd.sps_sliding_attention(q, k, v, 1 / math.sqrt(d), w, documents_idx_BxT=docs)
        y = y.transpose(1, 2).contiguous().view(b, two_t, c).to(c_proj.weight.dtype)
        return c_proj(y).square().mean()

    results = []
    for fn in (block, torch.compile(block, fullgraph=True)):
        for p in (*c_attn.parameters(), *c_proj.parameters()):
            p.grad = None
        loss = fn(x)
        loss.backward()
        torch.cuda.synchronize()
        results.append([loss.detach()] + [p.grad.clone() for p in (*c_attn.parameters(), *c_proj.parameters())])
    for got, want in zip(results[1], results[0]):
        torch.testing.assert_close(got, want, atol=1e-4, rtol=2e-2)
