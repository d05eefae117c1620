"""Parity of the HIP segmented decode kernels with the CPU oracle (GPU)."""

import math

import numpy as np
import pytest
import torch

from oracle import decode as Dc
from sps_amd import decode_attention as DA

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def _np_segs(segments):
    return [(s.k.float().cpu().numpy(), s.v.float().cpu().numpy(), s.lengths.cpu().numpy(), s.max_len_cap)
            for s in segments]


def _round(t, dtype):
    return t.to(dtype).float().cpu().numpy()


@pytest.mark.parametrize("first_lengths", ["shared", "empty"])
def test_q2_reference_test_config(first_lengths):
    # models/attention/test_segmented_q2_attention.py:67-117 (B2 H3 D16, seed 123).
    torch.manual_seed(123)
    bsz, n_head, head_dim = 2, 3, 16
    dev = "cuda"
    q = torch.randn(bsz, 2, n_head, head_dim, device=dev, dtype=torch.bfloat16)
    k0 = torch.randn(bsz, n_head, 7, head_dim, device=dev, dtype=torch.bfloat16)
    v0 = torch.randn_like(k0)
    k1 = torch.randn(bsz, n_head, 11, head_dim, device=dev, dtype=torch.bfloat16)
    v1 = torch.randn_like(k1)
    if first_lengths == "empty":
        len0 = torch.zeros((bsz,), device=dev, dtype=torch.long)
        cap0 = 0
    else:
        len0 = torch.tensor([2, 5], device=dev, dtype=torch.long)
        cap0 = 5
    len1 = torch.tensor([[1, 3, 6], [2, 4, 7]], device=dev, dtype=torch.long)
    segments = [DA.KVSegment(k0, v0, len0, max_len_cap=cap0), DA.KVSegment(k1, v1, len1, max_len_cap=8)]
    cur = [torch.randn(bsz, n_head, head_dim, device=dev, dtype=torch.bfloat16) for _ in range(4)]
    got = DA.triton_segmented_q2_attention(
        q, segments, current_normal_k_BxHxD=cur[0], current_normal_v_BxHxD=cur[1],
        current_predict_k_BxHxD=cur[2], current_predict_v_BxHxD=cur[3], attn_dtype=torch.bfloat16)
    want = Dc.attend(q.float().cpu().numpy(), _np_segs(segments),
                     [(cur[0].float().cpu().numpy(), cur[1].float().cpu().numpy()),
                      (cur[2].float().cpu().numpy(), cur[3].float().cpu().numpy())], [0b11, 0b10], 2)
    assert got.dtype == torch.float32 and got.shape == (bsz, 2, n_head, head_dim)
    torch.testing.assert_close(got.cpu(), torch.from_numpy(want).float(), atol=2e-2, rtol=2e-2)


Q1_CASES = [
    # head_dim, kv dtype, storages, caps, per_head flags, len dtype, n_extra
    (64, torch.bfloat16, [64, 4096], [64, 4096], [False, True], torch.int64, 2),
    (64, torch.bfloat16, [7, 300, 33], [None, 250, 0], [True, False, True], torch.int32, 1),
    (128, torch.float16, [64, 1000], [64, None], [False, True], torch.int64, 2),
    (32, torch.bfloat16, [5, 70], [5, None], [True, True], torch.int64, 0),
    (16, torch.float32, [3, 129], [None, 100], [False, True], torch.int64, 2),
    (256, torch.bfloat16, [64, 520], [64, 520], [False, True], torch.int64, 2),
    (64, torch.bfloat16, [0, 100], [None, None], [True, True], torch.int64, 1),
]


@pytest.mark.parametrize("case", Q1_CASES, ids=[f"d{c[0]}-{str(c[1])[6:]}-s{len(c[2])}-e{c[6]}" for c in Q1_CASES])
def test_q1_matches_oracle(case):
    head_dim, kv_dtype, storages, caps, per_head, len_dtype, n_extra = case
    rng = np.random.default_rng(head_dim + len(storages))
    g = torch.Generator().manual_seed(head_dim)
    b, h = 5, 3
    dev = "cuda"
    segments = []
    for storage, cap, ph in zip(storages, caps, per_head):
        k = torch.randn((b, h, storage, head_dim), generator=g).to(kv_dtype).to(dev)
        v = torch.randn((b, h, storage, head_dim), generator=g).to(kv_dtype).to(dev)
        shape = (b, h) if ph else (b,)
        lens = rng.integers(-2, storage + 3, size=shape) if storage else np.zeros(shape, dtype=np.int64)
        segments.append(DA.KVSegment(k, v, torch.tensor(lens, dtype=len_dtype, device=dev), max_len_cap=cap))
    q = torch.randn((b, h, head_dim), generator=g).to(dev)
    extras = [(torch.randn((b, h, head_dim), generator=g).to(dev), torch.randn((b, h, head_dim), generator=g).to(dev))
              for _ in range(n_extra)]
    got = DA.triton_segmented_q1_attention(q, segments, extra_kv=extras or None, attn_dtype=torch.bfloat16)
    assert got is not None
    want = Dc.attend(_round(q, torch.bfloat16).reshape(b, 1, h, head_dim), _np_segs(segments),
                     [(_round(ek, torch.bfloat16), _round(ev, torch.bfloat16)) for ek, ev in extras],
                     [1] * n_extra, 1)[:, 0]
    torch.testing.assert_close(got.cpu(), torch.from_numpy(want).float(), atol=ATOL, rtol=RTOL)


def _random_segments(rng, g, b, h, d, n_seg, dev):
    kv_dtype = (torch.bfloat16, torch.float16, torch.float32)[int(rng.integers(3))]
    len_dtype = torch.int64 if rng.random() < 0.7 else torch.int32
    segments = []
    for _ in range(n_seg):
        storage = int(rng.choice([0, 1, 5, 64, int(rng.integers(1, 1200))]))
        cap = (None, 0, 1, storage, storage + 9, int(rng.integers(0, max(storage, 1) + 1)))[int(rng.integers(6))]
        shape = (b, h) if rng.random() < 0.5 else (b,)
        lens = rng.integers(-3, storage + 4, size=shape) if storage else np.zeros(shape, dtype=np.int64)
        k = torch.randn((b, h, storage, d), generator=g).to(kv_dtype).to(dev)
        v = torch.randn((b, h, storage, d), generator=g).to(kv_dtype).to(dev)
        segments.append(DA.KVSegment(k, v, torch.tensor(lens, dtype=len_dtype, device=dev), max_len_cap=cap))
    return segments


@pytest.mark.parametrize("seed", range(6))
def test_decode_random_sweep(seed):
    # q=1 and q=2 decode at random configurations against the oracle: batch, heads, head dim, 0-3
    # segments (q=2: up to 2) of random storage, caps (none, 0, 1, the storage, past it, random),
    # lengths from -3 to past the storage, per-head or shared, int32/int64, bf16/f16/fp32 K/V, bf16 or
    # fp32 queries, 0-2 extra keys.
    rng = np.random.default_rng(3000 + seed)
    g = torch.Generator().manual_seed(seed)
    dev = "cuda"
    for _ in range(3):
        b, h = int(rng.integers(1, 7)), int(rng.integers(1, 5))
        d = int(rng.choice([16, 32, 64, 64, 128, 256]))
        segments = _random_segments(rng, g, b, h, d, int(rng.integers(0, 4)), dev)
        q_dtype = torch.bfloat16 if rng.random() < 0.5 else torch.float32
        q = torch.randn((b, h, d), generator=g).to(q_dtype).to(dev)
        n_extra = int(rng.integers(0, 3))
        extras = [(torch.randn((b, h, d), generator=g).to(dev), torch.randn((b, h, d), generator=g).to(dev))
                  for _ in range(n_extra)]
        got = DA.triton_segmented_q1_attention(q, segments, extra_kv=extras or None, attn_dtype=torch.bfloat16)
        assert got is not None
        want = Dc.attend(_round(q, torch.bfloat16).reshape(b, 1, h, d), _np_segs(segments),
                         [(_round(ek, torch.bfloat16), _round(ev, torch.bfloat16)) for ek, ev in extras],
                         [1] * n_extra, 1)[:, 0]
        torch.testing.assert_close(got.cpu(), torch.from_numpy(want).float(), atol=ATOL, rtol=RTOL)
    for _ in range(2):
        b, h = int(rng.integers(1, 7)), int(rng.integers(1, 5))
        d = int(rng.choice([16, 32, 64, 64, 128, 256]))
        segments = _random_segments(rng, g, b, h, d, int(rng.integers(0, 3)), dev)
        q = torch.randn((b, 2, h, d), generator=g).to(torch.bfloat16).to(dev)
        cur = [torch.randn((b, h, d), generator=g).to(torch.bfloat16).to(dev) for _ in range(4)]
        got = DA.triton_segmented_q2_attention(
            q, segments, current_normal_k_BxHxD=cur[0], current_normal_v_BxHxD=cur[1],
            current_predict_k_BxHxD=cur[2], current_predict_v_BxHxD=cur[3], attn_dtype=torch.bfloat16)
        want = Dc.attend(q.float().cpu().numpy(), _np_segs(segments),
                         [(cur[0].float().cpu().numpy(), cur[1].float().cpu().numpy()),
                          (cur[2].float().cpu().numpy(), cur[3].float().cpu().numpy())], [0b11, 0b10], 2)
        torch.testing.assert_close(got.cpu(), torch.from_numpy(want).float(), atol=ATOL, rtol=RTOL)


def test_c5_full_size_against_oracle():
    # C5: 64 sequences, 16 heads, D 64, retained lengths U[512, 4096] (seed 0), ring of 64 full,
    # one <predict> query (ring + retained + current input + current <predict>).
    from sps_amd.workloads import C5, decode_lengths

    dev = "cuda"
    lengths = decode_lengths(C5, seed=0)
    g = torch.Generator().manual_seed(0)
    B, H, D = C5.seqs, C5.heads, C5.head_dim
    q = torch.randn((B, H, D), generator=g).to(torch.bfloat16)
    rk = torch.randn((B, H, C5.storage, D), generator=g).to(torch.bfloat16)
    rv = torch.randn((B, H, C5.storage, D), generator=g).to(torch.bfloat16)
    wk = torch.randn((B, H, C5.ring, D), generator=g).to(torch.bfloat16)
    wv = torch.randn((B, H, C5.ring, D), generator=g).to(torch.bfloat16)
    ck, cv, pk, pv = (torch.randn((B, H, D), generator=g).to(torch.bfloat16) for _ in range(4))
    ring_len = torch.full((B,), C5.ring, dtype=torch.int64)
    ret_len = lengths.view(B, 1).expand(B, H).contiguous()
    segs = [DA.KVSegment(wk.to(dev), wv.to(dev), ring_len.to(dev), max_len_cap=C5.ring),
            DA.KVSegment(rk.to(dev), rv.to(dev), ret_len.to(dev), max_len_cap=C5.storage)]
    got = DA.masked_kv_attention(q.to(dev), segs, extra_kv=[(ck.to(dev), cv.to(dev)), (pk.to(dev), pv.to(dev))],
                                 attn_dtype=torch.bfloat16, prefer_triton=True)
    want = Dc.attend(q.float().numpy().reshape(B, 1, H, D),
                     [(wk.float().numpy(), wv.float().numpy(), ring_len.numpy(), C5.ring),
                      (rk.float().numpy(), rv.float().numpy(), ret_len.numpy(), C5.storage)],
                     [(ck.float().numpy(), cv.float().numpy()), (pk.float().numpy(), pv.float().numpy())],
                     [1, 1], 1)[:, 0]
    torch.testing.assert_close(got.cpu(), torch.from_numpy(want).float(), atol=ATOL, rtol=RTOL)
    # The q=2 form on the same state: slot 1 equals the q=1 predict query above.
    q2 = torch.stack([torch.randn((B, H, D), generator=g).to(torch.bfloat16), q], dim=1).to(dev)
    got2 = DA.triton_segmented_q2_attention(q2, segs, current_normal_k_BxHxD=ck.to(dev), current_normal_v_BxHxD=cv.to(dev),
                                            current_predict_k_BxHxD=pk.to(dev), current_predict_v_BxHxD=pv.to(dev),
                                            attn_dtype=torch.bfloat16)
    torch.testing.assert_close(got2[:, 1], got, atol=1e-6, rtol=1e-6)


def test_masked_kv_attention_contract():
    dev = "cuda"
    b, h, d = 2, 2, 64
    k = torch.randn((b, h, 10, d), device=dev, dtype=torch.bfloat16)
    q = torch.randn((b, h, d), device=dev, dtype=torch.bfloat16)
    # No key anywhere -> zeros.
    empty = DA.KVSegment(k, k, torch.zeros((b,), dtype=torch.long, device=dev))
    out = DA.masked_kv_attention(q, [empty], attn_dtype=torch.bfloat16)
    assert torch.equal(out, torch.zeros((b, h, d), device=dev))
    # check_finite: a row with no valid key raises, like the reference.
    partial = DA.KVSegment(k, k, torch.tensor([3, 0], device=dev))
    with pytest.raises(RuntimeError, match="no valid keys"):
        DA.masked_kv_attention(q, [partial], attn_dtype=torch.bfloat16, check_finite=True)
    bad = k.clone()
    bad[0, 0, 1] = float("nan")
    with pytest.raises(RuntimeError, match="Non-finite"):
        DA.masked_kv_attention(q, [DA.KVSegment(bad, k, torch.tensor([3, 3], device=dev))],
                               attn_dtype=torch.bfloat16, check_finite=True)
    ok = DA.masked_kv_attention(q, [DA.KVSegment(k, k, torch.tensor([3, 4], device=dev))], attn_dtype=torch.bfloat16,
                                check_finite=True)
    assert torch.isfinite(ok).all()


def test_q2_error_conventions():
    dev = "cuda"
    q = torch.randn((1, 3, 2, 64), device=dev)
    cur = torch.randn((1, 2, 64), device=dev)
    with pytest.raises(RuntimeError, match="slot dimension"):
        DA.triton_segmented_q2_attention(q, [], current_normal_k_BxHxD=cur, current_normal_v_BxHxD=cur,
                                         current_predict_k_BxHxD=cur, current_predict_v_BxHxD=cur,
                                         attn_dtype=torch.bfloat16)
    q = torch.randn((1, 2, 2, 64), device=dev)
    seg = DA.KVSegment(torch.randn((1, 2, 4, 64), device=dev), torch.randn((1, 2, 5, 64), device=dev),
                       torch.ones((1,), dtype=torch.long, device=dev))
    with pytest.raises(RuntimeError, match="shapes differ"):
        DA.triton_segmented_q2_attention(q, [seg], current_normal_k_BxHxD=cur, current_normal_v_BxHxD=cur,
                                         current_predict_k_BxHxD=cur, current_predict_v_BxHxD=cur,
                                         attn_dtype=torch.bfloat16)


def test_installed_shim_sends_cuda_calls_to_the_kernel(monkeypatch):
    # After install_into_modeling, the reference module's masked_kv_attention name reaches the HIP
    # kernel for CUDA tensors (bit-identical to calling sps_amd directly) and the module's original
    # function for CPU tensors (reference: decode_attention.py:597-704).
    import sys
    import types

    import sps_amd

    mod = types.ModuleType("modeling.models.utils.decode_attention")
    seen = []

    def original(q_BxHxD, segments, **kwargs):
        seen.append(q_BxHxD.device.type)
        return torch.zeros(q_BxHxD.shape, dtype=torch.float32)

    mod.masked_kv_attention = original
    monkeypatch.setitem(sys.modules, mod.__name__, mod)
    sps_amd.install_into_modeling()
    g = torch.Generator().manual_seed(4)
    b, h, d, storage = 3, 2, 64, 50
    k, v = (torch.randn((b, h, storage, d), generator=g).to(torch.bfloat16).cuda() for _ in range(2))
    lens = torch.tensor([5, 50, 17], device="cuda")
    q = torch.randn((b, h, d), generator=g).to(torch.bfloat16).cuda()
    seg = [DA.KVSegment(k, v, lens)]
    got = mod.masked_kv_attention(q, seg, attn_dtype=torch.bfloat16)
    want = DA.masked_kv_attention(q, seg, attn_dtype=torch.bfloat16)
    assert got.is_cuda and torch.equal(got, want)
    assert seen == []
    mod.masked_kv_attention(q.cpu(), [DA.KVSegment(k.cpu(), v.cpu(), lens.cpu())], attn_dtype=torch.float32)
    assert seen == ["cpu"]
