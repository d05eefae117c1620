"""Bit-exact parity of the HIP decode KV-cache update with the CPU oracle (GPU)."""

import numpy as np
import pytest
import torch

from oracle import kv_update as KU
from sps_amd.decode_attention_fast import fused_sps_kv_update

pytestmark = pytest.mark.gpu


def _make_state(B, H, D, ring_storage, window, ret_storage, cache_dtype, len_dtype, gen, strided=False):
    def cache(S):
        if strided:  # a [B, H, S, D] view inside a padded buffer (D contiguous, other strides not)
            return torch.randn(B, H, S + 3, D + 8, generator=gen).to(cache_dtype)[:, :, :S, :D]
        return torch.randn(B, H, S, D, generator=gen).to(cache_dtype)

    ring_len = torch.randint(0, window + 1, (B,), generator=gen)
    ring_pos = torch.where(ring_len >= window, torch.randint(0, window, (B,), generator=gen), torch.zeros_like(ring_len))
    ret_len = torch.randint(0, ret_storage + 1, (B, H), generator=gen)
    return dict(nw_k=cache(ring_storage), nw_v=cache(ring_storage), nw_len=ring_len.to(len_dtype),
                nw_pos=ring_pos.to(len_dtype), br_k=cache(ret_storage), br_v=cache(ret_storage),
                br_len=ret_len.to(len_dtype))


def _oracle_step(st, new, active, window, cache_dtype):
    # The reference casts the new K/V to the cache dtype before updating (reverse_sps/inference.py:197-202).
    f = lambda t: t.to(cache_dtype).float().numpy()  # noqa: E731
    arr = {k: (v.float().numpy().copy() if v.is_floating_point() else v.numpy().copy()) for k, v in st.items()}
    KU.kv_update(arr["nw_k"], arr["nw_v"], arr["nw_len"], arr["nw_pos"], arr["br_k"], arr["br_v"], arr["br_len"],
                 f(new[0]), f(new[1]), f(new[2]), f(new[3]), active.numpy().astype(bool), window)
    return arr


def _gpu_step(st_gpu, new, active, window):
    fused_sps_kv_update(nw_k=st_gpu["nw_k"], nw_v=st_gpu["nw_v"], nw_len=st_gpu["nw_len"], nw_pos=st_gpu["nw_pos"],
                        br_k=st_gpu["br_k"], br_v=st_gpu["br_v"], br_len=st_gpu["br_len"],
                        k_window_BxHxD=new[0].cuda(), v_window_BxHxD=new[1].cuda(), k_retained_BxHxD=new[2].cuda(),
                        v_retained_BxHxD=new[3].cuda(), active_mask_B=active.cuda(), window_tokens=window)


def _to_gpu(st):
    # Keep the strided layout of the views: move the underlying buffer, then take the same view.
    out = {}
    for k, v in st.items():
        if v.is_contiguous():
            out[k] = v.cuda()
        else:
            out[k] = torch.empty_strided(v.shape, v.stride(), dtype=v.dtype, device="cuda")
            out[k].copy_(v)
    return out


def _check(st_gpu, ref, label):
    for k, v in st_gpu.items():
        got = v.cpu()
        got = got.float().numpy() if got.is_floating_point() else got.numpy()
        np.testing.assert_array_equal(got, ref[k], err_msg=f"{label}: {k}")


def test_ring_wrap_reference_kat():
    # delayed_state/test_forward_efficient.py:280-312 on the GPU: window 2, inserts 1, 2, 3.
    B, H, D = 1, 2, 16
    st = dict(nw_k=torch.zeros(B, H, 2, D, device="cuda", dtype=torch.bfloat16),
              nw_v=torch.zeros(B, H, 2, D, device="cuda", dtype=torch.bfloat16),
              nw_len=torch.zeros(B, device="cuda", dtype=torch.long), nw_pos=torch.zeros(B, device="cuda", dtype=torch.long),
              br_k=torch.zeros(B, H, 5, D, device="cuda", dtype=torch.bfloat16),
              br_v=torch.zeros(B, H, 5, D, device="cuda", dtype=torch.bfloat16),
              br_len=torch.zeros(B, H, device="cuda", dtype=torch.long))
    for value in (1.0, 2.0, 3.0):
        k = torch.full((B, H, D), value)
        _gpu_step(st, (k, k + 10.0, k, k + 10.0), torch.tensor([True]), 2)
    torch.cuda.synchronize()
    assert int(st["nw_len"][0]) == 2 and int(st["nw_pos"][0]) == 1
    assert st["nw_k"][0, 0, :, 0].float().cpu().tolist() == [3.0, 2.0]
    assert st["nw_v"][0, 1, :, 3].float().cpu().tolist() == [13.0, 12.0]
    assert st["br_len"].cpu().tolist() == [[3, 3]]
    assert st["br_k"][0, 1, :3, 5].float().cpu().tolist() == [1.0, 2.0, 3.0]


@pytest.mark.parametrize("cache_dtype,new_dtype", [
    (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16), (torch.float32, torch.float32),
    (torch.bfloat16, torch.float32), (torch.float16, torch.float32), (torch.float32, torch.bfloat16),
    (torch.bfloat16, torch.float16),
])
def test_random_states_match_oracle(cache_dtype, new_dtype):
    gen = torch.Generator().manual_seed(11)
    B, H, D, window = 9, 5, 64, 6
    st = _make_state(B, H, D, 8, window, 12, cache_dtype, torch.long, gen)
    st_gpu = _to_gpu(st)
    for step in range(4):
        new = [torch.randn(B, H, D, generator=gen).to(new_dtype) for _ in range(4)]
        active = torch.rand(B, generator=gen) < 0.7
        ref = _oracle_step(st, new, active, window, cache_dtype)
        _gpu_step(st_gpu, new, active, window)
        torch.cuda.synchronize()
        _check(st_gpu, ref, f"step {step}")
        st = {k: v.cpu() for k, v in st_gpu.items()}


@pytest.mark.parametrize("seed", range(6))
def test_random_sweep(seed):
    # Random shapes, windows (0 = no ring), storages, cache and new-K/V dtypes, length dtypes, strided
    # or contiguous caches and active flags, over several consecutive steps: bit-exact every step.
    rng = np.random.default_rng(4000 + seed)
    gen = torch.Generator().manual_seed(seed)
    dtypes = (torch.bfloat16, torch.float16, torch.float32)
    for case in range(3):
        B, H = int(rng.integers(1, 10)), int(rng.integers(1, 6))
        D = int(rng.choice([16, 64, 100, 128, 256]))
        window = int(rng.integers(0, 8))
        ring_storage = window + int(rng.integers(0, 4)) if window else int(rng.integers(1, 4))
        ret_storage = int(rng.integers(1, 21))
        cache_dtype, new_dtype = dtypes[int(rng.integers(3))], dtypes[int(rng.integers(3))]
        len_dtype = torch.long if rng.random() < 0.6 else torch.int32
        st = _make_state(B, H, D, ring_storage, max(window, 1), ret_storage, cache_dtype, len_dtype, gen,
                         strided=bool(rng.random() < 0.4))
        st_gpu = _to_gpu(st)
        for step in range(int(rng.integers(3, 6))):
            new = [torch.randn(B, H, D, generator=gen).to(new_dtype) for _ in range(4)]
            active = torch.rand(B, generator=gen) < 0.75
            ref = _oracle_step(st, new, active, window, cache_dtype)
            _gpu_step(st_gpu, new, active, window)
            torch.cuda.synchronize()
            _check(st_gpu, ref, f"case {case} (B{B} H{H} D{D} w{window} {cache_dtype}<-{new_dtype}) step {step}")
            st = {k: v.cpu() for k, v in st_gpu.items()}


@pytest.mark.parametrize("D", [16, 100, 128, 256])
def test_strided_caches_int32_lengths_int64_flags(D):
    gen = torch.Generator().manual_seed(D)
    B, H, window = 5, 3, 4
    st = _make_state(B, H, D, 4, window, 7, torch.bfloat16, torch.int32, gen, strided=True)
    st_gpu = _to_gpu(st)
    assert not st_gpu["br_k"].is_contiguous()
    for step in range(3):
        new = [torch.randn(B, H, D, generator=gen).to(torch.bfloat16) for _ in range(4)]
        active = (torch.rand(B, generator=gen) < 0.8).to(torch.int64)
        ref = _oracle_step(st, new, active, window, torch.bfloat16)
        _gpu_step(st_gpu, new, active, window)
        torch.cuda.synchronize()
        _check(st_gpu, ref, f"D {D} step {step}")
        st = {k: v.cpu() for k, v in st_gpu.items()}


def test_no_window_updates_only_retained():
    gen = torch.Generator().manual_seed(5)
    B, H, D = 4, 2, 32
    st = _make_state(B, H, D, 2, 2, 6, torch.float16, torch.long, gen)
    st_gpu = _to_gpu(st)
    new = [torch.randn(B, H, D, generator=gen).to(torch.float16) for _ in range(4)]
    active = torch.tensor([True, False, True, True])
    ref = _oracle_step(st, new, active, 0, torch.float16)
    _gpu_step(st_gpu, new, active, 0)
    torch.cuda.synchronize()
    _check(st_gpu, ref, "no window")
    np.testing.assert_array_equal(st_gpu["nw_k"].cpu().float().numpy(), st["nw_k"].float().numpy())


def test_long_decode_sequence_c5_shape():
    # The C5 decode shape (64 sequences, 16 heads, D 64, ring 64) over 70 steps: the ring wraps.
    gen = torch.Generator().manual_seed(3)
    B, H, D, window = 64, 16, 64, 64
    st = dict(nw_k=torch.zeros(B, H, window, D, dtype=torch.bfloat16), nw_v=torch.zeros(B, H, window, D, dtype=torch.bfloat16),
              nw_len=torch.zeros(B, dtype=torch.long), nw_pos=torch.zeros(B, dtype=torch.long),
              br_k=torch.zeros(B, H, 80, D, dtype=torch.bfloat16), br_v=torch.zeros(B, H, 80, D, dtype=torch.bfloat16),
              br_len=torch.zeros(B, H, dtype=torch.long))
    st_gpu = _to_gpu(st)
    arr = {k: (v.float().numpy().copy() if v.is_floating_point() else v.numpy().copy()) for k, v in st.items()}
    for step in range(70):
        new = [torch.randn(B, H, D, generator=gen).to(torch.bfloat16) for _ in range(4)]
        active = torch.rand(B, generator=gen) < 0.9
        KU.kv_update(arr["nw_k"], arr["nw_v"], arr["nw_len"], arr["nw_pos"], arr["br_k"], arr["br_v"], arr["br_len"],
                     *(t.float().numpy() for t in new), active.numpy(), window)
        _gpu_step(st_gpu, new, active, window)
    torch.cuda.synchronize()
    _check(st_gpu, arr, "C5 70 steps")
    assert int(st_gpu["nw_len"].max()) == window and int(st_gpu["nw_pos"].max()) > 0
