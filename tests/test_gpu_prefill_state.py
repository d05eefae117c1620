"""Bit-exact parity of the prefill -> decode materialisation kernel with the CPU oracle (GPU)."""

import numpy as np
import pytest
import torch

from oracle import prefill_state as PS
from sps_amd.prefill_state import materialize_prefill_layer_state, prefill_to_decode

pytestmark = pytest.mark.gpu


def _run(B, T, H, D, W, in_dtype, cache_dtype, mask, window_slot, retained_slot, seed, len_dtype=torch.long,
         strided=False):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(B, 2 * T, H, D, generator=g).to(in_dtype)
    v = torch.randn(B, 2 * T, H, D, generator=g).to(in_dtype)
    Sw, Sr = max(W, 1) + 2, T + 3

    def cache(S):
        x = torch.randn(B, H, S + (2 if strided else 0), D, generator=g).to(cache_dtype)
        return x[:, :, :S] if strided else x

    st = dict(ring_k=cache(Sw), ring_v=cache(Sw), ring_len=torch.randint(0, 5, (B,), generator=g).to(len_dtype),
              ring_pos=torch.randint(0, 5, (B,), generator=g).to(len_dtype), ret_k=cache(Sr), ret_v=cache(Sr),
              ret_len=torch.randint(0, 5, (B, H), generator=g).to(len_dtype))
    arr = {n: (x.float().numpy().copy() if x.is_floating_point() else x.numpy().copy()) for n, x in st.items()}
    # The reference casts the rows to the cache dtype (inference.py:576-587) before copying them.
    PS.materialize(k.to(cache_dtype).float().numpy(), v.to(cache_dtype).float().numpy(), mask.numpy(), window_slot,
                   retained_slot, arr["ring_k"], arr["ring_v"], arr["ring_len"], arr["ring_pos"], arr["ret_k"],
                   arr["ret_v"], arr["ret_len"], W)
    gst = {}
    for n, x in st.items():
        y = torch.empty_strided(x.shape, x.stride(), dtype=x.dtype, device="cuda")
        y.copy_(x)
        gst[n] = y
    prefill_to_decode(k.cuda(), v.cuda(), mask.cuda(), window_slot=window_slot, retained_slot=retained_slot,
                      nw_k=gst["ring_k"], nw_v=gst["ring_v"], nw_len=gst["ring_len"], nw_pos=gst["ring_pos"],
                      br_k=gst["ret_k"], br_v=gst["ret_v"], br_len=gst["ret_len"], window_tokens=W)
    torch.cuda.synchronize()
    for n, x in gst.items():
        got = x.cpu()
        got = got.float().numpy() if got.is_floating_point() else got.numpy()
        np.testing.assert_array_equal(got, arr[n], err_msg=n)


def _trailing_docs(B, T, g):
    # Left-padded prompts whose last document starts somewhere: the reference's current-doc masks.
    start = torch.randint(0, T, (B,), generator=g)
    m = torch.arange(T)[None, :] >= start[:, None]
    m[0] = False  # one row with an empty document
    return m


@pytest.mark.parametrize("in_dtype,cache_dtype", [(torch.float32, torch.bfloat16), (torch.bfloat16, torch.bfloat16),
                                                  (torch.float16, torch.float32), (torch.float32, torch.float16)])
def test_trailing_documents(in_dtype, cache_dtype):
    g = torch.Generator().manual_seed(1)
    B, T, H, D = 5, 70, 3, 64
    _run(B, T, H, D, 8, in_dtype, cache_dtype, _trailing_docs(B, T, g), 1, 0, seed=2)


@pytest.mark.parametrize("seed", range(6))
def test_random_sweep(seed):
    # Random shapes, head dims, windows, dtypes, slot roles, length dtypes, strided or contiguous caches,
    # and masks (trailing documents, arbitrary bits, all, none): bit-exact against the oracle.
    rng = np.random.default_rng(6000 + seed)
    dtypes = (torch.bfloat16, torch.float16, torch.float32)
    for case in range(3):
        B, T, H = int(rng.integers(1, 7)), int(rng.integers(1, 300)), int(rng.integers(1, 5))
        D = int(rng.choice([16, 64, 128, 256]))
        g = torch.Generator().manual_seed(int(rng.integers(1 << 30)))
        kind = int(rng.integers(4))
        if kind == 0:
            mask = _trailing_docs(B, T, g)
        elif kind == 1:
            mask = torch.rand(B, T, generator=g) < float(rng.uniform(0.1, 0.9))
        else:
            mask = torch.full((B, T), kind == 2)
        slot = int(rng.integers(2))
        _run(B, T, H, D, int(rng.choice([0, 1, 5, 64, T + 3])), dtypes[int(rng.integers(3))],
             dtypes[int(rng.integers(3))], mask, slot, 1 - slot, seed=int(rng.integers(1 << 30)),
             len_dtype=torch.long if rng.random() < 0.6 else torch.int32, strided=bool(rng.random() < 0.4))


@pytest.mark.parametrize("W", [0, 1, 64, 100])
def test_window_sizes_and_reverse_slots(W):
    g = torch.Generator().manual_seed(W)
    B, T, H, D = 4, 90, 2, 32
    _run(B, T, H, D, W, torch.float32, torch.bfloat16, _trailing_docs(B, T, g), 0, 1, seed=W, len_dtype=torch.int32)


def test_arbitrary_masks_long_rows_strided_caches():
    # Non-contiguous member sets and rows longer than one compaction chunk (2048 tokens).
    g = torch.Generator().manual_seed(9)
    B, T, H, D = 3, 2600, 2, 16
    mask = torch.rand(B, T, generator=g) < torch.tensor([[0.5], [0.02], [1.0]])
    _run(B, T, H, D, 16, torch.bfloat16, torch.bfloat16, mask, 1, 0, seed=4, strided=True)


def test_method_drop_in_on_a_state_object():
    class _Mem:
        pass

    class _State:
        pass

    class _Model:
        _window_slot_index, _retained_slot_index = 0, 1

    g = torch.Generator().manual_seed(5)
    B, T, H, D, W = 2, 12, 2, 16, 4
    st = _State()
    st.normal_window_tokens = W
    st.normal_window, st.predict_retained = _Mem(), _Mem()
    for mem, S in ((st.normal_window, W), (st.predict_retained, T)):
        mem.k = [torch.zeros(B, H, S, D, device="cuda", dtype=torch.bfloat16)]
        mem.v = [torch.zeros(B, H, S, D, device="cuda", dtype=torch.bfloat16)]
    st.normal_window.len = [torch.zeros(B, device="cuda", dtype=torch.long)]
    st.normal_window.pos = [torch.full((B,), 3, device="cuda", dtype=torch.long)]
    st.predict_retained.len = [torch.zeros(B, H, device="cuda", dtype=torch.long)]
    k = torch.randn(B, 2 * T, H, D, generator=g).cuda()
    v = torch.randn(B, 2 * T, H, D, generator=g).cuda()
    mask = torch.zeros(B, T, dtype=torch.bool)
    mask[0, 5:] = True
    mask[1, 10:] = True
    materialize_prefill_layer_state(_Model(), st, 0, k, v, mask.cuda())
    torch.cuda.synchronize()
    assert st.predict_retained.len[0].tolist() == [[7, 7], [2, 2]]
    assert st.normal_window.len[0].tolist() == [4, 2] and st.normal_window.pos[0].tolist() == [0, 0]
    torch.testing.assert_close(st.predict_retained.k[0][1, :, :2].float().cpu(),
                               k[1, 21::2][:2].transpose(0, 1).to(torch.bfloat16).float().cpu(), rtol=0, atol=0)
    torch.testing.assert_close(st.normal_window.v[0][0, :, :4].float().cpu(),
                               v[0, 0::2][8:12].transpose(0, 1).to(torch.bfloat16).float().cpu(), rtol=0, atol=0)
