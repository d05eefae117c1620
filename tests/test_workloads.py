"""The benchmark workloads: the seeded packed-document lengths reproduce the committed fixture
(tests/golden/doc_lengths_c2_c4.json, written by tests/golden/make_doc_lengths.py), and the closed-form
visible-pair counts behind the headline FLOP figures equal the C oracle's brute-force counts on the
same rows."""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import mask as M
from sps_amd import workloads as W

FIXTURE = json.loads((Path(__file__).resolve().parent / "golden" / "doc_lengths_c2_c4.json").read_text())
FAMILY = {"full": M.FAMILY_FULL, "sps": M.FAMILY_SPS, "reverse_sps": M.FAMILY_REVERSE_SPS}


@pytest.mark.parametrize("name", ["C2", "C3", "C4"])
def test_doc_lengths_reproduce_fixture(name):
    cfg = getattr(W, name)
    fx = FIXTURE[name]
    assert (fx["batch"], fx["tokens"]) == (cfg.batch, cfg.tokens)
    lengths = W.packed_doc_lengths(cfg.batch, cfg.tokens, seed=fx["seed"])
    assert lengths == fx["lengths"]
    lo, hi = W.DOC_CLIP
    for row in lengths:
        assert sum(row) == cfg.tokens
        assert all(lo <= x <= hi for x in row[:-1]) and 1 <= row[-1] <= hi


@pytest.mark.parametrize("name", ["C2", "C3", "C4"])
def test_visible_pairs_match_oracle_counts(name):
    cfg = getattr(W, name)
    ids, lengths = W.position_doc_ids(cfg, seed=0)
    ids = np.asarray(ids)
    brute = sum(M.count_c(FAMILY[cfg.family], cfg.n, ids[b], cfg.window) for b in range(cfg.batch))
    assert W.visible_pairs(cfg, lengths) == brute


def test_headline_flops():
    # C3 fwd+bwd useful work, 14 * D per visible pair over 16 heads (the bench's metric denominator).
    assert round(W.useful_flops(W.C3, FIXTURE["C3"]["lengths"]) / 1e9, 3) == 89.232


def test_recorded_traffic_covers_every_attention_config():
    # The bench line's roofline.traffic for C2, C3 and C4 comes from the committed counter summaries;
    # each must give fetch + write bytes for every attention kernel, at least the kernel's compulsory
    # traffic (K and V read, dK and dV written once: 4 B*H*N*D*2 bytes).
    import bench

    for name in ("C2", "C3", "C4"):
        cfg = getattr(W, name)
        t = bench.recorded_traffic(bench.TRAFFIC_FILES[name])
        for kernel in ("row_layout_kernel", "attn_fwd_kernel", "attn_bwd_dq_kernel", "attn_bwd_dkdv_kernel"):
            assert t.get(kernel, 0) > 0, (name, kernel)
        compulsory = 4 * cfg.batch * cfg.heads * cfg.n * cfg.head_dim * 2
        assert t["attn_bwd_dkdv_kernel"] >= compulsory, name
