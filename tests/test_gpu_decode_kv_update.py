"""A decode step's attention and KV-cache update in one entry point (sps_decode_kv_update), GPU.

Every case runs the same step twice on copies of one state: through the fused entry point and as
the reference's decode step runs it, the segmented attention over the caches and then the KV update
(reverse_sps/inference.py:322-362, then fused_sps_kv_update via :169-238). Outputs and every cache
and length tensor must be identical bit for bit, and the caches must equal the CPU oracle's update.
The segments are the caches themselves: the ring (the SPS <predict>-slot keys) and the retained
buffer (input-slot keys), as sps/inference.py:8-12 assigns them.
"""

import math

import numpy as np
import pytest
import torch

from oracle import kv_update as KU
from sps_amd import decode_attention as DA
from sps_amd import decode_attention_fast as DF

pytestmark = pytest.mark.gpu


def _state(B, H, D, ring_storage, window, ret_storage, cache_dtype, len_dtype, gen, strided=False):
    def cache(S):
        if strided:  # a [B, H, S, D] view inside a padded buffer
            return torch.randn(B, H, S + 3, D + 8, generator=gen).to(cache_dtype)[:, :, :S, :D]
        return torch.randn(B, H, S, D, generator=gen).to(cache_dtype)

    ring_len = torch.randint(0, max(window, 0) + 1, (B,), generator=gen)
    ring_pos = torch.where(ring_len >= max(window, 1), torch.randint(0, max(window, 1), (B,), generator=gen),
                           torch.zeros_like(ring_len))
    ret_len = torch.randint(0, ret_storage + 1, (B, H), generator=gen)  # ret_storage itself: a full buffer
    return dict(nw_k=cache(ring_storage), nw_v=cache(ring_storage), nw_len=ring_len.to(len_dtype),
                nw_pos=ring_pos.to(len_dtype), br_k=cache(ret_storage), br_v=cache(ret_storage),
                br_len=ret_len.to(len_dtype))


def _to_gpu(st):
    out = {}
    for k, v in st.items():
        out[k] = torch.empty_strided(v.shape, v.stride(), dtype=v.dtype, device="cuda")
        out[k].copy_(v)
    return out


def _clone(st):
    out = {}
    for k, v in st.items():
        out[k] = torch.empty_strided(v.shape, v.stride(), dtype=v.dtype, device=v.device)
        out[k].copy_(v)
    return out


def _segments(st, window):
    segs = []
    if window > 0:
        segs.append(DA.KVSegment(st["nw_k"], st["nw_v"], st["nw_len"], max_len_cap=min(window, st["br_k"].size(2))))
    segs.append(DA.KVSegment(st["br_k"], st["br_v"], st["br_len"], max_len_cap=st["br_k"].size(2)))
    return segs


def _update_kwargs(st, cur, active, window):
    # SPS slot roles: the ring takes the current <predict> K/V, the retained buffer the input K/V.
    return dict(nw_k=st["nw_k"], nw_v=st["nw_v"], nw_len=st["nw_len"], nw_pos=st["nw_pos"], br_k=st["br_k"],
                br_v=st["br_v"], br_len=st["br_len"], k_window_BxHxD=cur[2], v_window_BxHxD=cur[3],
                k_retained_BxHxD=cur[0], v_retained_BxHxD=cur[1], active_mask_B=active, window_tokens=window)


def _step(st, q, cur, active, window, nq, fused, attn_dtype):
    segs = _segments(st, window)
    upd = _update_kwargs(st, cur, active, window)
    if nq == 2:
        kw = dict(current_normal_k_BxHxD=cur[0], current_normal_v_BxHxD=cur[1], current_predict_k_BxHxD=cur[2],
                  current_predict_v_BxHxD=cur[3], attn_dtype=attn_dtype)
        if fused:
            return DF.segmented_q2_attention_with_kv_update(q, segs, **kw, **upd)
        out = DA.triton_segmented_q2_attention(q, segs, **kw)
    else:
        extra = [(cur[0], cur[1]), (cur[2], cur[3])]
        if fused:
            return DF.segmented_q1_attention_with_kv_update(q, segs, extra_kv=extra, attn_dtype=attn_dtype, **upd)
        out = DA.triton_segmented_q1_attention(q, segs, extra_kv=extra, attn_dtype=attn_dtype)
    DF.fused_sps_kv_update(**upd)
    return out


def _oracle_update(st_cpu, cur, active, window, cache_dtype):
    f = lambda t: t.cpu().to(cache_dtype).float().numpy()  # noqa: E731
    arr = {k: (v.float().numpy().copy() if v.is_floating_point() else v.numpy().copy()) for k, v in st_cpu.items()}
    KU.kv_update(arr["nw_k"], arr["nw_v"], arr["nw_len"], arr["nw_pos"], arr["br_k"], arr["br_v"], arr["br_len"],
                 f(cur[2]), f(cur[3]), f(cur[0]), f(cur[1]), active.cpu().numpy().astype(bool), window)
    return arr


def _same(a, b, label):
    for k in a:
        assert torch.equal(a[k], b[k]), f"{label}: {k} differs between the fused and the two-call step"


def _matches_oracle(st, ref, label):
    for k, v in st.items():
        got = v.cpu()
        got = got.float().numpy() if got.is_floating_point() else got.numpy()
        np.testing.assert_array_equal(got, ref[k], err_msg=f"{label}: {k}")


def _run_case(B, H, D, ring_storage, window, ret_storage, cache_dtype, new_dtype, nq, steps, seed, len_dtype=torch.long,
              active_p=0.8):
    gen = torch.Generator().manual_seed(seed)
    st_a = _to_gpu(_state(B, H, D, ring_storage, window, ret_storage, cache_dtype, len_dtype, gen))
    st_b = _clone(st_a)
    for step in range(steps):
        q = torch.randn((B, nq, H, D) if nq == 2 else (B, H, D), generator=gen).to(cache_dtype).cuda()
        cur = [torch.randn(B, H, D, generator=gen).to(new_dtype).cuda() for _ in range(4)]
        active = (torch.rand(B, generator=gen) < active_p).cuda()
        before = {k: v.cpu() for k, v in st_a.items()}
        out_a = _step(st_a, q, cur, active, window, nq, True, cache_dtype)
        out_b = _step(st_b, q, cur, active, window, nq, False, cache_dtype)
        torch.cuda.synchronize()
        label = f"step {step}"
        assert torch.equal(out_a, out_b), f"{label}: attention output differs"
        _same(st_a, st_b, label)
        _matches_oracle(st_a, _oracle_update(before, cur, active, window, cache_dtype), label)


@pytest.mark.parametrize("nq", [1, 2])
@pytest.mark.parametrize("cache_dtype,new_dtype", [
    (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16), (torch.float32, torch.float32),
    # a conversion of the new rows: the update runs as its own launch after the attention
    (torch.bfloat16, torch.float32),
])
def test_fused_step_equals_attention_then_update(nq, cache_dtype, new_dtype):
    _run_case(9, 5, 64, 8, 6, 700, cache_dtype, new_dtype, nq, steps=4, seed=11)


@pytest.mark.parametrize("seed", range(6))
def test_random_sweep(seed):
    # Random shapes, head dims, windows (0 = no ring), storages (including buffers that fill during the
    # run), cache and new-K/V dtypes, length dtypes, q=1 / q=2 and active rates: the fused step equals
    # the attention followed by the update, and the oracle's caches, every step.
    rng = np.random.default_rng(5000 + seed)
    dtypes = (torch.bfloat16, torch.float16, torch.float32)
    for case in range(2):
        window = int(rng.integers(0, 9))
        cache_dtype = dtypes[int(rng.integers(3))]
        new_dtype = cache_dtype if rng.random() < 0.7 else dtypes[int(rng.integers(3))]
        _run_case(int(rng.integers(1, 10)), int(rng.integers(1, 6)), int(rng.choice([16, 32, 64, 128, 256])),
                  window + int(rng.integers(0, 4)) if window else int(rng.integers(1, 4)), window,
                  int(rng.integers(1, 400)), cache_dtype, new_dtype, int(rng.integers(1, 3)),
                  steps=int(rng.integers(2, 6)), seed=int(rng.integers(1 << 30)),
                  len_dtype=torch.long if rng.random() < 0.6 else torch.int32, active_p=float(rng.uniform(0.3, 1.0)))


@pytest.mark.parametrize("D", [16, 32, 128, 256])
def test_head_dims_and_int32_lengths(D):
    _run_case(5, 3, D, 4, 4, 300, torch.bfloat16, torch.bfloat16, 2, steps=3, seed=D, len_dtype=torch.int32)


def test_no_window_only_retained():
    # window_tokens = 0: one (retained) segment, no ring update.
    _run_case(4, 2, 64, 2, 0, 40, torch.float16, torch.float16, 1, steps=3, seed=5)


def test_ring_wrap_reference_kat_through_the_fused_step():
    # delayed_state/test_forward_efficient.py:280-312 (window 2, inserts 1, 2, 3) through the fused entry.
    B, H, D = 1, 2, 16
    st = dict(nw_k=torch.zeros(B, H, 2, D, device="cuda", dtype=torch.bfloat16),
              nw_v=torch.zeros(B, H, 2, D, device="cuda", dtype=torch.bfloat16),
              nw_len=torch.zeros(B, device="cuda", dtype=torch.long), nw_pos=torch.zeros(B, device="cuda", dtype=torch.long),
              br_k=torch.zeros(B, H, 5, D, device="cuda", dtype=torch.bfloat16),
              br_v=torch.zeros(B, H, 5, D, device="cuda", dtype=torch.bfloat16),
              br_len=torch.zeros(B, H, device="cuda", dtype=torch.long))
    q = torch.zeros(B, 2, H, D, device="cuda", dtype=torch.bfloat16)
    for value in (1.0, 2.0, 3.0):
        k = torch.full((B, H, D), value, device="cuda", dtype=torch.bfloat16)
        _step(st, q, (k, k + 10.0, k, k + 10.0), torch.tensor([True], device="cuda"), 2, 2, True, torch.bfloat16)
    torch.cuda.synchronize()
    assert int(st["nw_len"][0]) == 2 and int(st["nw_pos"][0]) == 1
    assert st["nw_k"][0, 0, :, 0].float().cpu().tolist() == [3.0, 2.0]
    assert st["nw_v"][0, 1, :, 3].float().cpu().tolist() == [13.0, 12.0]
    assert st["br_len"].cpu().tolist() == [[3, 3]]
    assert st["br_k"][0, 1, :3, 5].float().cpu().tolist() == [1.0, 2.0, 3.0]


def test_strided_caches_through_the_c_abi():
    # Caches that are views inside padded buffers (the C-ABI takes strides; the Python wrappers, like
    # the reference's, ask for contiguous segments).
    gen = torch.Generator().manual_seed(21)
    B, H, D, window, ret_storage = 6, 4, 64, 8, 90
    st_a = _to_gpu(_state(B, H, D, window, window, ret_storage, torch.bfloat16, torch.long, gen, strided=True))
    assert not st_a["br_k"].is_contiguous()
    st_b = _clone(st_a)
    for step in range(3):
        q = torch.randn(B, 1, H, D, generator=gen).to(torch.bfloat16).cuda()
        cur = [torch.randn(B, H, D, generator=gen).to(torch.bfloat16).cuda() for _ in range(4)]
        active = (torch.rand(B, generator=gen) < 0.8).cuda()
        before = {k: v.cpu() for k, v in st_a.items()}
        outs = []
        for st, fused in ((st_a, True), (st_b, False)):
            out = torch.empty(B, 1, H, D, device="cuda")
            upd = DF.kv_update_args(**_update_kwargs(st, cur, active, window))
            DA._run_decode(q, 1, _segments(st, window), [(cur[0], cur[1]), (cur[2], cur[3])], [1, 1], out,
                           kv_update=upd if fused else None)
            if not fused:
                DF.run_kv_update(upd)
            outs.append(out)
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1])
        _same(st_a, st_b, f"strided step {step}")
        _matches_oracle(st_a, _oracle_update(before, cur, active, window, torch.bfloat16), f"strided step {step}")


def test_c5_shape_70_steps():
    # The C5 decode shape (64 sequences, 16 heads, D 64, ring 64, retained lengths U[512, 4096]) over
    # 70 steps through the fused entry and through the two calls: the ring wraps, the retained
    # buffers grow, outputs and caches stay identical, and the caches equal the oracle's.
    from sps_amd.workloads import C5, decode_lengths

    gen = torch.Generator().manual_seed(3)
    B, H, D, window, storage = C5.seqs, C5.heads, C5.head_dim, C5.ring, C5.storage + 80
    lengths = decode_lengths(C5, seed=0)
    st_a = dict(nw_k=torch.randn(B, H, window, D, generator=gen).to(torch.bfloat16).cuda(),
                nw_v=torch.randn(B, H, window, D, generator=gen).to(torch.bfloat16).cuda(),
                nw_len=torch.full((B,), window, dtype=torch.long).cuda(),
                nw_pos=torch.randint(0, window, (B,), generator=gen).cuda(),
                br_k=torch.randn(B, H, storage, D, generator=gen).to(torch.bfloat16).cuda(),
                br_v=torch.randn(B, H, storage, D, generator=gen).to(torch.bfloat16).cuda(),
                br_len=lengths.view(B, 1).expand(B, H).contiguous().cuda())
    st_b = _clone(st_a)
    arr = {k: (v.cpu().float().numpy() if v.is_floating_point() else v.cpu().numpy()) for k, v in st_a.items()}
    for step in range(70):
        q = torch.randn(B, H, D, generator=gen).to(torch.bfloat16).cuda()
        cur = [torch.randn(B, H, D, generator=gen).to(torch.bfloat16).cuda() for _ in range(4)]
        active = (torch.rand(B, generator=gen) < 0.9).cuda()
        out_a = _step(st_a, q, cur, active, window, 1, True, torch.bfloat16)
        out_b = _step(st_b, q, cur, active, window, 1, False, torch.bfloat16)
        KU.kv_update(arr["nw_k"], arr["nw_v"], arr["nw_len"], arr["nw_pos"], arr["br_k"], arr["br_v"], arr["br_len"],
                     *(t.cpu().float().numpy() for t in (cur[2], cur[3], cur[0], cur[1])),
                     active.cpu().numpy(), window)
        assert torch.equal(out_a, out_b), f"step {step}: attention output differs"
    torch.cuda.synchronize()
    _same(st_a, st_b, "C5 70 steps")
    _matches_oracle(st_a, arr, "C5 70 steps")
    assert math.isfinite(float(out_a.abs().max()))
