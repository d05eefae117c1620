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
