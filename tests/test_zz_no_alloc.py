"""sps_decode_static (decode without a workspace argument: the partial records live in the library's
scratch array) against sps_decode on the same inputs (GPU). Two calls in a row, the second smaller,
so the second reads only what it wrote over the first call's records."""

import ctypes as C

import pytest
import torch

from sps_amd import _native as N
from sps_amd import decode_attention as DA

pytestmark = pytest.mark.gpu


def _inputs(seed, b, h, d, storage, ring, nq, kv_dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    dev = "cuda"
    q = torch.randn((b, nq, h, d), generator=g).to(kv_dtype).to(dev)
    rk, rv = (torch.randn((b, h, storage, d), generator=g).to(kv_dtype).to(dev) for _ in range(2))
    wk, wv = (torch.randn((b, h, ring, d), generator=g).to(kv_dtype).to(dev) for _ in range(2))
    ret_len = torch.randint(0, storage + 1, (b, h), generator=g).to(dev)
    ring_len = torch.randint(0, ring + 1, (b,), generator=g).to(dev)
    extras = [tuple(torch.randn((b, h, d), generator=g).to(kv_dtype).to(dev) for _ in range(2)) for _ in range(2)]
    segs = [DA.KVSegment(wk, wv, ring_len, max_len_cap=ring), DA.KVSegment(rk, rv, ret_len, max_len_cap=storage)]
    return q, segs, extras


def _both(q, segs, extras, nq):
    b, _, h, d = q.shape
    masks = [0b11, 0b10] if nq == 2 else [1, 1]
    ref = torch.empty((b, nq, h, d), device="cuda", dtype=torch.float32)
    got = torch.full((b, nq, h, d), float("nan"), device="cuda", dtype=torch.float32)
    DA._run_decode(q, nq, segs, extras, masks, ref)
    DA._run_decode(q, nq, segs, extras, masks, got, static_scratch=True)
    torch.cuda.synchronize()
    return ref, got


@pytest.mark.parametrize("nq", [1, 2])
def test_static_scratch_matches_workspace_path_twice(nq):
    # First call: C5-like shape (64 sequences, 16 heads, retained up to 4096 keys).
    ref, got = _both(*_inputs(0, 64, 16, 64, 4096, 64, nq), nq)
    assert torch.equal(ref, got)
    # Second call, smaller (fewer sequences, shorter segments): the scratch still holds the first
    # call's records beyond what this call writes; none of them may reach the output.
    ref, got = _both(*_inputs(1, 5, 3, 64, 700, 16, nq), nq)
    assert torch.equal(ref, got)


def test_static_scratch_rejects_oversized_records():
    # 64 sequences x 16 heads x 64 chunks of 512 keys x 68 floats = 17.8 MB > 16 MiB: rejected before
    # any launch (the segment tensors are only shape carriers here).
    b, h, d = 64, 16, 64
    q = torch.zeros((b, 1, h, d), device="cuda", dtype=torch.bfloat16)
    k = torch.zeros((1, 1, 1, d), device="cuda", dtype=torch.bfloat16).expand(b, h, 32768, d)
    seg = DA.KVSegment(k, k, torch.zeros((b,), dtype=torch.int64, device="cuda"))
    out = torch.empty((b, 1, h, d), device="cuda", dtype=torch.float32)
    with pytest.raises(N.NativeError, match="scratch"):
        DA._run_decode(q, 1, [seg], [], [], out, static_scratch=True)
