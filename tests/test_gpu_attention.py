"""Parity of the HIP attention kernels with the CPU oracle (GPU).

Bar: masks bit-exact; bf16/f16 outputs and gradients within
max-abs 2e-2 / rel 1e-2 of the float64 oracle evaluated on the same (16-bit) inputs. The one
exception is the gradients at sharp-softmax inputs (activations x4 / x8, sm_scale = 1), where the
reference's own 16-bit arithmetic misses that bound: there the kernels are held to the error of an
emulation of that arithmetic (_scaled_check).
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import mask as M
from sps_amd import attention as SA
from sps_amd import _native as N

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2
FAMILY = {"full": N.FAMILY_FULL, "sps": N.FAMILY_SPS, "reverse_sps": N.FAMILY_REVERSE_SPS}
API = {
    "full": lambda q, k, v, s, w, d, p: SA.full_attention(q, k, v, s, documents_idx_BxT=d),
    "sps": lambda q, k, v, s, w, d, p: SA.sps_sliding_attention(q, k, v, s, w, documents_idx_BxT=d,
                                                                  persistent_key_window=p),
    "reverse_sps": lambda q, k, v, s, w, d, p: SA.reverse_sps_sliding_attention(
        q, k, v, s, w, documents_idx_BxT=d, persistent_key_window=p),
}


def _packed_docs(rng, b, tokens, family, max_len=None):
    rows = []
    for _ in range(b):
        row, fill, i = [], 0, 0
        while fill < tokens:
            ln = int(rng.integers(1, max_len or max(2, tokens // 2)))
            ln = min(ln, tokens - fill)
            row += [i] * ln
            fill += ln
            i += 1
        rows.append(row)
    ids = np.array(rows, dtype=np.int64)
    return ids if family == "full" else np.repeat(ids, 2, axis=1)


def _check(family, b, h, n, d, window=0, docs=None, pkw=None, dtype=torch.bfloat16, seed=0, layout="bhnd",
           grads=True, docs_dtype=torch.int64):
    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(seed)
    shape = (b, n, h, d) if layout == "bnhd" else (b, h, n, d)
    q, k, v, do = (torch.randn(shape, generator=g).to(dtype) for _ in range(4))
    if layout == "bnhd":
        q, k, v, do = (t.transpose(1, 2) for t in (q, k, v, do))
    scale = 1.0 / math.sqrt(d)
    docs_t = None if docs is None else torch.tensor(docs, dtype=docs_dtype, device=dev)
    qg, kg, vg = (t.to(dev).requires_grad_(grads) for t in (q, k, v))
    out = API[family](qg, kg, vg, scale, window, docs_t, pkw)
    mask = M.batch_mask(FAMILY[family], docs, n=n, window=window, pkw=pkw, batch=b)
    qn, kn, vn, don = (t.float().numpy() for t in (q, k, v, do))
    o_ref, _ = A.forward(qn, kn, vn, mask, scale)
    torch.testing.assert_close(out.float().cpu(), torch.from_numpy(o_ref).float(), atol=ATOL, rtol=RTOL)
    if grads:
        out.backward(do.to(dev))
        dq, dk, dv = A.backward(qn, kn, vn, don, mask, scale)
        for name, got, want in (("dq", qg.grad, dq), ("dk", kg.grad, dk), ("dv", vg.grad, dv)):
            torch.testing.assert_close(got.float().cpu(), torch.from_numpy(want).float(), atol=ATOL, rtol=RTOL,
                                       msg=lambda m, name=name: f"{name}: {m}")


@pytest.mark.parametrize("seed", range(6))
def test_parity_random_sweep(seed):
    # Outputs and gradients at random small configurations against the float64 oracle, to the same
    # bound as the fixed matrix: each family with a random length, head dim, window, persistent-key
    # window, document layout (none, packed runs, non-monotone random ids), dtype and memory layout.
    rng = np.random.default_rng(2000 + seed)
    for family in ("full", "sps", "reverse_sps"):
        n = int(rng.integers(1, 401)) if family == "full" else 2 * int(rng.integers(1, 201))
        d = int(rng.choice([16, 32, 64, 64, 128, 256]))
        b, h = int(rng.integers(1, 3)), int(rng.integers(1, 3))
        window = int(rng.choice([-1, 0, 3, 64, n, int(rng.integers(0, n + 1))])) if family != "full" else 0
        pkw = int(rng.choice([0, 1, int(rng.integers(0, n + 1))])) if family != "full" and rng.random() < 0.5 else None
        tokens = n if family == "full" else n // 2
        kind = int(rng.integers(3))
        docs = (None if kind == 0 else _packed_docs(rng, b, tokens, family, max_len=int(rng.integers(2, max(3, tokens + 1))))
                if kind == 1 else rng.integers(0, 3, size=(b, n)).astype(np.int64))
        dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float16
        layout = "bhnd" if rng.random() < 0.5 else "bnhd"
        _check(family, b, h, n, d, window=window, docs=docs, pkw=pkw, dtype=dtype, seed=int(rng.integers(1 << 30)),
               layout=layout)


@pytest.mark.parametrize("family", ["sps", "reverse_sps"])
@pytest.mark.parametrize("has_docs", [False, True])
def test_reference_kernel_test_shape(family, has_docs):
    # attention/triton/test_sps_attention.py:79-131: B1 H2 T16 D64, w=3, seed 17, docs [0*6,1*8,2*2].
    docs = None
    if has_docs:
        docs = np.repeat(np.array([[0] * 6 + [1] * 8 + [2] * 2]), 2, axis=1)
    _check(family, 1, 2, 32, 64, window=3, docs=docs, seed=17)


@pytest.mark.parametrize("family", ["sps", "reverse_sps"])
def test_persistent_key_window_reference_config(family):
    # models/attention/test_persistent_key_window.py:62-98: n_ctx 8, D 64, fp16, window 8, pkw 1.
    _check(family, 1, 1, 8, 64, window=8, pkw=1, dtype=torch.float16, grads=True)


CASES = [
    # family, b, h, n, d, window, docs, pkw, dtype, layout
    ("full", 2, 3, 200, 64, 0, "packed", None, torch.bfloat16, "bhnd"),
    ("full", 1, 2, 512, 128, 0, None, None, torch.bfloat16, "bnhd"),
    ("full", 1, 2, 300, 32, 0, "random", None, torch.float16, "bhnd"),
    ("sps", 2, 2, 512, 64, 64, "packed", None, torch.bfloat16, "bnhd"),
    ("sps", 1, 2, 1030, 64, 64, "packed", None, torch.bfloat16, "bhnd"),
    ("sps", 1, 1, 768, 64, 0, None, None, torch.bfloat16, "bhnd"),
    ("sps", 1, 2, 400, 128, 5000, "packed", None, torch.bfloat16, "bhnd"),
    ("sps", 2, 1, 260, 16, 7, "random", 3, torch.float16, "bhnd"),
    ("sps", 1, 2, 512, 32, 33, "packed", 0, torch.bfloat16, "bnhd"),
    ("reverse_sps", 2, 2, 512, 64, 64, "packed", None, torch.bfloat16, "bhnd"),
    ("reverse_sps", 1, 2, 340, 128, 17, None, 40, torch.float16, "bnhd"),
    ("reverse_sps", 1, 1, 200, 64, -1, "packed", None, torch.bfloat16, "bhnd"),
    # D = 64 temporary-stream key tiles of at most 16 chunks take the skewed dK/dV schedule: with
    # arbitrary (non-monotone) ids; at 16 chunks (window 128: a 128-key tile's queries span
    # 2 (127 + 128) + 2 positions); at 17 chunks (window 130, the grouped schedule)
    ("sps", 1, 2, 384, 64, 24, "random", None, torch.bfloat16, "bhnd"),
    ("reverse_sps", 1, 2, 1024, 64, 128, "packed", None, torch.bfloat16, "bnhd"),
    ("sps", 1, 1, 1024, 64, 130, None, None, torch.float16, "bhnd"),
    ("sps", 2, 1, 512, 64, 40, "packed", None, torch.float16, "bnhd"),
    # head dim 256 (accepted by the reference's prefill asserts, triton_sps_flash_attention.py:510)
    ("full", 1, 2, 300, 256, 0, "packed", None, torch.bfloat16, "bhnd"),
    ("sps", 1, 2, 320, 256, 17, "packed", None, torch.float16, "bnhd"),
    ("reverse_sps", 2, 1, 260, 256, 64, None, 5, torch.bfloat16, "bhnd"),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-n{c[3]}-d{c[4]}-w{c[5]}-{c[6]}-pkw{c[7]}" for c in CASES])
def test_parity_matrix(case):
    family, b, h, n, d, w, docs_kind, pkw, dtype, layout = case
    rng = np.random.default_rng(n + d)
    tokens = n if family == "full" else n // 2
    docs = None
    if docs_kind == "packed":
        docs = _packed_docs(rng, b, tokens, family)
    elif docs_kind == "random":
        docs = rng.integers(0, 3, size=(b, n)).astype(np.int64)
    _check(family, b, h, n, d, window=w, docs=docs, pkw=pkw, dtype=dtype, layout=layout, seed=n)


TINY_CASES = [
    # family, n, d, window, docs: the smallest sequences each family accepts (one partial block)
    ("full", 1, 64, 0, None),
    ("full", 3, 16, 0, [[0, 1, 1]]),
    ("sps", 2, 64, 0, None),
    ("sps", 4, 32, 1, [[0, 0, 1, 1]]),
    ("sps", 6, 128, 64, [[0, 0, 0, 0, 0, 0]]),
    ("reverse_sps", 2, 64, -1, None),
    ("reverse_sps", 4, 64, 3, [[5, 5, 7, 7]]),
]


@pytest.mark.parametrize("case", TINY_CASES, ids=[f"{c[0]}-n{c[1]}-d{c[2]}-w{c[3]}" for c in TINY_CASES])
def test_tiny_sequences(case):
    family, n, d, w, docs = case
    _check(family, 1, 2, n, d, window=w, docs=None if docs is None else np.array(docs, dtype=np.int64),
           seed=n + d)


def test_empty_batch():
    # No (batch, head) slice: empty outputs and gradients, no launch.
    q, k, v = (torch.randn(0, 2, 64, 64, device="cuda", dtype=torch.bfloat16).requires_grad_() for _ in range(3))
    out = SA.sps_sliding_attention(q, k, v, 0.125, 64)
    assert out.shape == (0, 2, 64, 64)
    out.sum().backward()
    assert q.grad.shape == q.shape and k.grad.shape == k.shape and v.grad.shape == v.shape


def test_int32_documents():
    rng = np.random.default_rng(1)
    docs = _packed_docs(rng, 2, 160, "sps")
    _check("sps", 2, 2, 320, 64, window=9, docs=docs, docs_dtype=torch.int32)


MASK_CASES = [
    ("sps", 512, 64, "packed", None),
    ("sps", 300, 5, "random", None),
    ("sps", 256, 0, None, 2),
    ("reverse_sps", 512, 64, "packed", 7),
    ("reverse_sps", 130, 3, "random", -1),
    ("full", 333, 0, "packed", None),
    ("full", 256, 0, "random", None),
    ("sps", 1024, 4096, "packed", None),
    # closed-form tile plans where every other position sees nothing of a stream (window 0 or -1,
    # a persistent-key window of 0 or the diagonal only), over documents in runs
    ("sps", 514, 0, "packed", -1),
    ("reverse_sps", 386, -1, "packed", 0),
    # rows longer than 8192 positions take the prepass's looped (not register-resident) path
    ("sps", 8320, 64, "packed", None),
    ("full", 8200, 0, "random", None),
]


@pytest.mark.parametrize("schedule", [0, 1])
@pytest.mark.parametrize("case", MASK_CASES, ids=[f"{c[0]}-n{c[1]}-w{c[2]}-{c[3]}-pkw{c[4]}" for c in MASK_CASES])
def test_mask_bit_exact(case, schedule):
    # The block schedule + tile classification + per-element predicate of the kernels, materialised
    # by sps_attn_mask, equals the oracle predicate on every (query, key) pair.
    family, n, w, docs_kind, pkw = case
    rng = np.random.default_rng(n + w)
    b = 2
    tokens = n if family == "full" else n // 2
    docs = None
    if docs_kind == "packed":
        docs = _packed_docs(rng, b, tokens, family, max_len=90)
    elif docs_kind == "random":
        docs = rng.integers(0, 4, size=(b, n)).astype(np.int64)
    docs_t = None if docs is None else torch.tensor(docs, device="cuda")
    got = SA.attention_mask(FAMILY[family], n, docs_t, batch=b, window=w, persistent_key_window=pkw,
                            schedule=schedule).cpu().numpy().astype(bool)
    want = M.batch_mask(FAMILY[family], docs, n=n, window=w, pkw=pkw, batch=b)
    assert (got == want).all(), f"{int((got != want).sum())} mismatching pairs"


def _random_mask_case(rng):
    family = ("full", "sps", "reverse_sps")[int(rng.integers(3))]
    n = int(rng.integers(1, 701)) if family == "full" else 2 * int(rng.integers(1, 351))
    b = int(rng.integers(1, 4))
    window = int(rng.choice([-1, 0, 1, 2, n, n + 5, int(rng.integers(0, n + 1))]))
    pkw = None
    if family != "full" and rng.random() < 0.4:
        pkw = int(rng.choice([-1, 0, 1, int(rng.integers(0, n + 1))]))
    tokens = n if family == "full" else n // 2
    kind = int(rng.integers(4))
    if kind == 0:
        docs = None
    elif kind == 1:
        docs = _packed_docs(rng, b, tokens, family, max_len=int(rng.integers(2, max(3, tokens + 1))))
    elif kind == 2:
        docs = rng.integers(0, int(rng.integers(1, 5)), size=(b, n)).astype(np.int64)
    else:
        docs = np.zeros((b, n), dtype=np.int64)
    return family, n, b, window, pkw, docs


@pytest.mark.parametrize("seed", range(8))
def test_mask_random_sweep(seed):
    # Random families, lengths (odd ones for full attention), batch sizes, windows (-1, 0, 1, 2, past
    # the row, random), persistent-key windows and document layouts (none, packed runs down to length
    # 1, non-monotone random ids, one document): the kernels' masks under both block schedules equal
    # the oracle predicate on every pair.
    rng = np.random.default_rng(1000 + seed)
    for _ in range(8):
        family, n, b, window, pkw, docs = _random_mask_case(rng)
        docs_t = None if docs is None else torch.tensor(docs, device="cuda")
        want = M.batch_mask(FAMILY[family], docs, n=n, window=window, pkw=pkw, batch=b)
        for schedule in (0, 1):
            got = SA.attention_mask(FAMILY[family], n, docs_t, batch=b, window=window, persistent_key_window=pkw,
                                    schedule=schedule).cpu().numpy().astype(bool)
            case = f"{family} n={n} b={b} w={window} pkw={pkw} docs={'none' if docs is None else docs[0, :12]}"
            assert (got == want).all(), f"schedule {schedule}, {case}: {int((got != want).sum())} mismatching pairs"


@pytest.mark.parametrize("family,n", [("sps", 4096), ("full", 4096), ("reverse_sps", 8320)])
def test_visible_count_through_forward_kernel(family, n):
    # Q = K = 0 makes every visible score equal, so the forward kernel's LSE is log2(#visible keys):
    # an end-to-end check of the mask the real kernel applies, row by row, at C3-like lengths.
    b, h, d = 2, 2, 64
    rng = np.random.default_rng(5)
    tokens = n if family == "full" else n // 2
    docs = _packed_docs(rng, b, tokens, family, max_len=900)
    z = torch.zeros((b, h, n, d), dtype=torch.bfloat16, device="cuda")
    v = torch.randn((b, h, n, d), device="cuda").to(torch.bfloat16)
    _, lse, *_ = SA.attention_forward(z, z, v, 0.125, FAMILY[family], 64, torch.tensor(docs, device="cuda"))
    counts = torch.round(torch.exp2(lse.double())).long().cpu().numpy()
    for bi in range(b):
        want = M.mask_c(FAMILY[family], n, docs[bi], 64).sum(axis=1)
        for hi in range(h):
            assert (counts[bi, hi] == want).all()


def test_full_size_c3_heads_against_oracle():
    # C3 shape (N = 4096, w = 64, packed log-normal documents) checked head by head against the
    # oracle for a subset of (batch, head) pairs, forward and backward.
    from sps_amd.workloads import C3, make_qkv, position_doc_ids

    ids, _ = position_doc_ids(C3, seed=0)
    q, k, v, do = make_qkv(C3, seed=0)
    sel_b, sel_h = [0, 3], [0, 15]
    dev = torch.device("cuda")
    qg, kg, vg = (t.to(dev).requires_grad_(True) for t in (q, k, v))
    docs = torch.tensor(ids, device=dev)
    out = SA.sps_sliding_attention(qg, kg, vg, 0.125, 64, documents_idx_BxT=docs)
    out.backward(do.to(dev))
    for bi in sel_b:
        mask = M.batch_mask(N.FAMILY_SPS, ids[bi:bi + 1], window=64)
        for hi in sel_h:
            sl = (slice(bi, bi + 1), slice(hi, hi + 1))
            qn, kn, vn, don = (t[sl].float().numpy() for t in (q, k, v, do))
            o_ref, _ = A.forward(qn, kn, vn, mask, 0.125)
            dq, dk, dv = A.backward(qn, kn, vn, don, mask, 0.125)
            torch.testing.assert_close(out[sl].float().cpu(), torch.from_numpy(o_ref).float(), atol=ATOL, rtol=RTOL)
            for got, want in ((qg.grad, dq), (kg.grad, dk), (vg.grad, dv)):
                torch.testing.assert_close(got[sl].float().cpu(), torch.from_numpy(want).float(), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("cfg_name,sel", [("C2", [(0, 0), (7, 11)]), ("C4", [(0, 0), (1, 15)])])
def test_full_size_c2_c4_heads_against_oracle(cfg_name, sel):
    # The other benchmark configurations at full size: C2 (standard family, B8 H12 T2048, packed
    # documents) and C4 (SPS w = 4096, D = 128, B2 H16, 4096 positions): the whole batch runs through
    # the kernels, and selected (batch, head) slices are checked against the oracle, fwd and bwd.
    from sps_amd import workloads as W

    cfg = getattr(W, cfg_name)
    ids, _ = W.position_doc_ids(cfg, seed=0)
    q, k, v, do = W.make_qkv(cfg, seed=0)
    fam = {"full": N.FAMILY_FULL, "sps": N.FAMILY_SPS, "reverse_sps": N.FAMILY_REVERSE_SPS}[cfg.family]
    scale = 1.0 / math.sqrt(cfg.head_dim)
    dev = torch.device("cuda")
    qg, kg, vg = (t.to(dev).requires_grad_(True) for t in (q, k, v))
    docs = torch.tensor(ids, device=dev)
    out = API[cfg.family](qg, kg, vg, scale, cfg.window, docs, None)
    out.backward(do.to(dev))
    for bi, hi in sel:
        mask = M.batch_mask(fam, ids[bi:bi + 1], window=cfg.window)
        sl = (slice(bi, bi + 1), slice(hi, hi + 1))
        qn, kn, vn, don = (t[sl].float().numpy() for t in (q, k, v, do))
        o_ref, _ = A.forward(qn, kn, vn, mask, scale)
        dq, dk, dv = A.backward(qn, kn, vn, don, mask, scale)
        torch.testing.assert_close(out[sl].float().cpu(), torch.from_numpy(o_ref).float(), atol=ATOL, rtol=RTOL)
        for got, want in ((qg.grad, dq), (kg.grad, dk), (vg.grad, dv)):
            torch.testing.assert_close(got[sl].float().cpu(), torch.from_numpy(want).float(), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("family", ["sps", "reverse_sps"])
def test_rows_beyond_the_sorted_tile_limit(family):
    # 262272 positions: 2049 query tiles and 2050 key tiles, past the 2048 tiles the prepass sorts,
    # so the plans are written in the closed-form order. Documents of at most 48 tokens make the
    # attention block-diagonal per document: the whole row runs through the kernels, and a few
    # documents (first, middle, last) are checked against the oracle on their own slices.
    n, d, w = 262272, 64, 16
    rng = np.random.default_rng(11)
    docs = _packed_docs(rng, 1, n // 2, family, max_len=48)[0]
    g = torch.Generator().manual_seed(11)
    q, k, v, do = (torch.randn((1, 1, n, d), generator=g).to(torch.bfloat16) for _ in range(4))
    dev = torch.device("cuda")
    qg, kg, vg = (t.to(dev).requires_grad_(True) for t in (q, k, v))
    out = API[family](qg, kg, vg, 0.125, w, torch.from_numpy(docs[None]).to(dev), None)
    out.backward(do.to(dev))
    starts = [0] + [i for i in range(1, n) if docs[i] != docs[i - 1]]
    ends = starts[1:] + [n]
    for j in (0, 1, len(starts) // 2, len(starts) - 2, len(starts) - 1):
        s, e = starts[j], ends[j]
        mask = M.batch_mask(FAMILY[family], [list(docs[s:e])], window=w)  # positions s.. keep their parity (s even)
        sl = (slice(0, 1), slice(0, 1), slice(s, e))
        qn, kn, vn, don = (t[sl].float().numpy() for t in (q, k, v, do))
        o_ref, _ = A.forward(qn, kn, vn, mask, 0.125)
        dq, dk, dv = A.backward(qn, kn, vn, don, mask, 0.125)
        torch.testing.assert_close(out[sl].float().cpu(), torch.from_numpy(o_ref).float(), atol=ATOL, rtol=RTOL)
        for got, want in ((qg.grad, dq), (kg.grad, dk), (vg.grad, dv)):
            torch.testing.assert_close(got[sl].float().cpu(), torch.from_numpy(want).float(), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("family", ["full", "reverse_sps"])
def test_no_cross_document_leakage(family):
    # attention/triton/test_document_leakage.py: poison document 2's K/V with NaN; document 1's
    # outputs stay finite and equal a solo run on document 1.
    torch.manual_seed(2024)
    dev = "cuda"
    b, h, n, d = 1, 2, 256, 64
    half = n // 2
    q, k, v = (torch.randn(b, h, n, d, device=dev, dtype=torch.bfloat16) for _ in range(3))
    fn = API[family]
    solo = fn(q[:, :, :half], k[:, :, :half], v[:, :, :half], 1 / 8, 4, None, None)
    kp, vp = k.clone(), v.clone()
    kp[:, :, half:] = float("nan")
    vp[:, :, half:] = float("nan")
    docs = torch.zeros((b, n), dtype=torch.int64, device=dev)
    docs[:, half:] = 1
    out = fn(q, kp, vp, 1 / 8, 4, docs, None)
    assert torch.isfinite(out[:, :, :half]).all()
    torch.testing.assert_close(out[:, :, :half].float(), solo.float(), atol=2e-2, rtol=1e-2)


def test_strided_and_contiguous_inputs_agree():
    g = torch.Generator().manual_seed(3)
    b, h, n, d = 2, 4, 384, 64
    base = torch.randn((b, n, 3 * h * d), generator=g).to(torch.bfloat16).cuda()
    q, k, v = base.split(h * d, dim=2)
    q, k, v = (t.view(b, n, h, d).transpose(1, 2) for t in (q, k, v))  # the model's views
    docs = torch.tensor(np.repeat(np.array([[0] * 100 + [1] * 92] * b), 2, axis=1), device="cuda")
    o1 = SA.sps_sliding_attention(q, k, v, 0.125, 16, documents_idx_BxT=docs)
    o2 = SA.sps_sliding_attention(q.contiguous(), k.contiguous(), v.contiguous(), 0.125, 16, documents_idx_BxT=docs)
    torch.testing.assert_close(o1, o2, atol=0, rtol=0)
    assert o1.transpose(1, 2).is_contiguous()


def test_reference_assertions_preserved():
    q = torch.randn(1, 1, 30, 64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(AssertionError):
        SA.sps_sliding_attention(q[:, :, :29], q[:, :, :29], q[:, :, :29], 0.125, 3)
    with pytest.raises(AssertionError):
        SA.sps_sliding_attention(q, q, q, 0.125, 3, documents_idx_BxT=torch.zeros(1, 28, dtype=torch.long, device="cuda"))
    with pytest.raises(AssertionError):
        SA.full_attention(q[..., :48], q[..., :48], q[..., :48], 0.125)


@pytest.mark.parametrize("family", ["sps", "full"])
def test_backward_reusing_forward_layout_is_identical(family):
    # attention_forward(keep_layout=True) leaves the document layout in a backward-sized workspace;
    # the backward that reuses it (SPS_BWD_REUSE_LAYOUT) matches the one that recomputes it bit for bit.
    rng = np.random.default_rng(11)
    b, h, n, d = 2, 3, 1000, 64
    tokens = n if family == "full" else n // 2
    docs = torch.tensor(_packed_docs(rng, b, tokens, family, max_len=300), device="cuda")
    g = torch.Generator().manual_seed(4)
    q, k, v, do = (torch.randn((b, h, n, d), generator=g).to(torch.bfloat16).cuda() for _ in range(4))
    fam = FAMILY[family]
    o, lse, _, _, _, ws = SA.attention_forward(q, k, v, 0.125, fam, 17, docs, keep_layout=True)
    assert ws is not None
    ref = SA.attention_backward(do, q, k, v, o, lse, 0.125, fam, 17, docs)
    got = SA.attention_backward(do, q, k, v, o, lse, 0.125, fam, 17, docs, layout_workspace=ws)
    split = SA.attention_backward(do, q, k, v, o, lse, 0.125, fam, 17, docs, layout_workspace=ws,
                                  between_passes=lambda: None)
    for r, x, y in zip(ref, got, split):
        assert torch.equal(r, x) and torch.equal(r, y)


# Activation scales seen in trained models: Q and K drawn with standard deviation 4 and 8, or
# sm_scale = 1 at D = 64, so the scaled scores reach tens of units and the softmax is sharp. The
# kernels scale the fp32 scores (S * sm_scale * log2 e, as triton_sps_flash_attention.py:78-79 does),
# so the forward meets the plain bound against the exact (float64) oracle. The gradients go through
# 16-bit P and dS, as the reference's own kernels do (:361-377, :471-488), and at these inputs that
# arithmetic itself misses the plain bound on dQ and dK against the exact gradients (by 3-7x), and
# two block sizes of the reference's autotuner disagree with each other beyond it
# (tests/test_oracle_emulate.py, on oracle.emulate, the CPU emulation of the reference's
# arithmetic). So each gradient is held to what the reference's arithmetic achieves on the same
# inputs: with errors measured against the plain bound, the HIP gradient's worst element may not
# exceed 1.5x the emulated reference's worst (the largest over its block sizes 32, 64, 128), nor its
# root-mean-square error 1.25x the reference's.
EMU_BLOCKS = (32, 64, 128)
WORST_FACTOR, RMS_FACTOR = 1.5, 1.25


def _bound_ratio(got, want):
    err = (got.double() - want.double()).abs()
    return float((err / (ATOL + RTOL * want.double().abs())).max())


def _rms(got, want):
    return float(((got.double() - want.double()) ** 2).mean().sqrt())


def _scaled_check(family, n, d, s, dtype, window=64, sm_scale=None, seed=0):
    from oracle import emulate as X

    dev = torch.device("cuda")
    b, h = 1, 2
    g = torch.Generator().manual_seed(seed)
    q, k = ((torch.randn((b, h, n, d), generator=g) * s).to(dtype) for _ in range(2))
    v, do = (torch.randn((b, h, n, d), generator=g).to(dtype) for _ in range(2))
    rng = np.random.default_rng(seed)
    tokens = n if family == "full" else n // 2
    docs = _packed_docs(rng, b, tokens, family, max_len=tokens)
    scale = 1.0 / math.sqrt(d) if sm_scale is None else sm_scale
    qg, kg, vg = (t.to(dev).requires_grad_(True) for t in (q, k, v))
    out = API[family](qg, kg, vg, scale, window, torch.tensor(docs, device=dev), None)
    out.backward(do.to(dev))
    mask = M.batch_mask(FAMILY[family], docs, n=n, window=window, batch=b)
    qn, kn, vn, don = (t.float().numpy() for t in (q, k, v, do))
    o_ref, _ = A.forward(qn, kn, vn, mask, scale)
    torch.testing.assert_close(out.float().cpu(), torch.from_numpy(o_ref).float(), atol=ATOL, rtol=RTOL)
    exact = [torch.from_numpy(x) for x in A.backward(qn, kn, vn, don, mask, scale)]
    emulated = []
    for bn in EMU_BLOCKS:
        o_e, lse_e = X.forward(q, k, v, mask, scale, dtype=dtype, block_n=bn)
        emulated.append(X.backward(q, k, v, o_e, lse_e, do, mask, scale, dtype=dtype))
    for i, (name, got) in enumerate((("dq", qg.grad), ("dk", kg.grad), ("dv", vg.grad))):
        got = got.cpu()
        worst = _bound_ratio(got, exact[i])
        worst_ref = max(_bound_ratio(e[i], exact[i]) for e in emulated)
        rms, rms_ref = _rms(got, exact[i]), sum(_rms(e[i], exact[i]) for e in emulated) / len(emulated)
        assert worst <= max(1.0, WORST_FACTOR * worst_ref), (
            f"{name}: worst error / plain bound {worst:.2f}, the reference's arithmetic {worst_ref:.2f}")
        assert rms <= RMS_FACTOR * rms_ref + 1e-7, f"{name}: rms error {rms:.3g}, the reference's arithmetic {rms_ref:.3g}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("s", [4.0, 8.0])
@pytest.mark.parametrize("family", ["sps", "full"])
def test_scaled_activations(family, s, dtype):
    _scaled_check(family, 512, 64, s, dtype)


@pytest.mark.parametrize("sm_scale", [-0.125, 0.0, 1.0])
@pytest.mark.parametrize("family", ["sps", "reverse_sps", "full"])
def test_any_sm_scale(family, sm_scale):
    # The reference takes any sm_scale (it multiplies the fp32 scores by it and adds its masks to
    # the scaled scores): a zero scale gives the mean of the visible values, a negative one flips
    # the scores.
    _scaled_check(family, 256, 64, 1.0, torch.bfloat16, window=5, sm_scale=sm_scale, seed=3)


def test_c1_shape_forward_against_oracle():
    # C1 (SPS forward, B2 H8 D64, 512 tokens -> 1024 positions, w=64, one document per row; fp32 on
    # the reference's CPU path): the same seeded inputs cast to bf16 through the HIP forward, every
    # (batch, head) against the oracle on the rounded inputs.
    from sps_amd.workloads import C1, make_qkv

    q, k, v = (t.to(torch.bfloat16) for t in make_qkv(C1, seed=0, with_grad=False))
    out = SA.sps_sliding_attention(q.cuda(), k.cuda(), v.cuda(), 1 / math.sqrt(C1.head_dim), C1.window)
    mask = M.batch_mask(N.FAMILY_SPS, None, n=C1.n, window=C1.window, batch=C1.batch)
    o_ref, _ = A.forward(q.float().numpy(), k.float().numpy(), v.float().numpy(), mask, 1 / math.sqrt(C1.head_dim))
    torch.testing.assert_close(out.float().cpu(), torch.from_numpy(o_ref).float(), atol=ATOL, rtol=RTOL)


def test_second_backward_over_a_retained_graph():
    # The reference's autograd.Function allows backward(retain_graph=True) twice; the saved layout
    # workspace is not declared mutated by the backward, so the second pass is accepted and gives the
    # same gradients.
    rng = np.random.default_rng(2)
    b, h, n, d = 1, 2, 512, 64
    docs = torch.tensor(_packed_docs(rng, b, n // 2, "sps", max_len=100), device="cuda")
    g = torch.Generator().manual_seed(2)
    q, k, v, do = (torch.randn((b, h, n, d), generator=g).to(torch.bfloat16).cuda() for _ in range(4))
    qg, kg, vg = (t.requires_grad_(True) for t in (q, k, v))
    out = SA.sps_sliding_attention(qg, kg, vg, 0.125, 16, documents_idx_BxT=docs)
    first = torch.autograd.grad(out, (qg, kg, vg), do, retain_graph=True)
    second = torch.autograd.grad(out, (qg, kg, vg), do)
    for x, y in zip(first, second):
        assert torch.equal(x, y)
