"""The attention's torch.library registration (CPU: fake tensors, no kernel runs)."""

import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import sps_amd  # noqa: F401  (registers the ops)
from sps_amd import _native as N


def test_fake_impls_give_the_kernels_layouts():
    # The forward's output is [B, H, N, D] over [B, N, H, D] memory (the caller's transpose back is
    # free), LSE [B, H, N] fp32, and the layout workspace is the backward-sized one when kept.
    with FakeTensorMode():
        q = torch.empty(2, 64, 3, 32, dtype=torch.bfloat16, device="cuda").transpose(1, 2)
        docs = torch.zeros(2, 64, dtype=torch.int64, device="cuda")
        o, lse, ws = torch.ops.sps_amd.attention_fwd(q, q, q, docs, 0.125, N.FAMILY_SPS, 8, None, True)
        assert o.shape == (2, 3, 64, 32) and o.transpose(1, 2).is_contiguous()
        assert lse.shape == (2, 3, 64) and lse.dtype == torch.float32
        assert ws.numel() == N.lib().sps_attn_workspace_bytes(N.FAMILY_SPS, 2, 3, 64, 1, 1)
        _, _, ws0 = torch.ops.sps_amd.attention_fwd(q, q, q, None, 0.125, N.FAMILY_SPS, 8, None, True)
        assert ws0.numel() == 0
        dq, dk, dv = torch.ops.sps_amd.attention_bwd(o, q, q, q, o, lse, docs, ws, 0.125, N.FAMILY_SPS, 8, None)
        assert dq.shape == q.shape and dq.stride() == q.stride()


def test_backward_op_is_pure():
    # The backward writes only the workspace's seed region, scratch it writes before reading; it is
    # declared pure so the workspace the forward saved keeps its version and a second backward over
    # a retained graph is allowed (as with the reference's autograd.Function).
    schema = torch.ops.sps_amd.attention_bwd.default._schema
    assert all(a.alias_info is None or not a.alias_info.is_write for a in schema.arguments)


def test_rope_ops_fake_impls():
    # RoPE as custom ops: the fakes give the real kernels' outputs (contiguous, input dtype for the
    # pair; the requested dtype for the attention-ready triple), so a compiled model traces them.
    with FakeTensorMode():
        x = torch.empty(2, 16, 3, 64, dtype=torch.float32, device="cuda")
        f = torch.empty(16, 32, dtype=torch.complex64, device="cuda")
        q, k = torch.ops.sps_amd.rope_pair(x, x, f)
        assert q.shape == x.shape and q.dtype == torch.float32 and q.is_contiguous()
        outs = torch.ops.sps_amd.rope_qkv(x, x, x, f, torch.bfloat16)
        assert all(o.shape == x.shape and o.dtype == torch.bfloat16 and o.is_contiguous() for o in outs)
