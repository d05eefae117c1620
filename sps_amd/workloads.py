"""Synthetic workloads of the benchmark configurations and their algorithmic work.

Configurations: C1 SPS forward fp32 on the CPU path; C2 Standard fwd+bwd; C3 SPS
w=64 fwd+bwd (the headline); C4 SPS w=4096 D=128 fwd+bwd; C5 segmented decode.

Packed documents: each row is filled with documents whose token lengths are
round(exp(ln(400) + 0.8 * z)), z ~ N(0, 1), clipped to [16, 2048], the last one truncated to fit.
The log-normal sigma is not specified by the configuration; 0.8 is fixed here once. Lengths come
from torch.Generator().manual_seed(seed) (CPU), so they are identical on every machine.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

DOC_MEDIAN = 400
DOC_SIGMA = 0.8
DOC_CLIP = (16, 2048)


@dataclass(frozen=True)
class AttnConfig:
    name: str
    family: str  # "full" | "sps" | "reverse_sps"
    batch: int
    heads: int
    head_dim: int
    tokens: int  # tokens per row; N = 2 * tokens for the SPS families
    window: int
    packed_docs: bool
    dtype: torch.dtype

    @property
    def n(self) -> int:
        return self.tokens if self.family == "full" else 2 * self.tokens


C1 = AttnConfig("C1", "sps", 2, 8, 64, 512, 64, False, torch.float32)
C2 = AttnConfig("C2", "full", 8, 12, 64, 2048, 0, True, torch.bfloat16)
C3 = AttnConfig("C3", "sps", 4, 16, 64, 2048, 64, True, torch.bfloat16)
C4 = AttnConfig("C4", "sps", 2, 16, 128, 2048, 4096, True, torch.bfloat16)


@dataclass(frozen=True)
class DecodeConfig:
    name: str
    seqs: int
    heads: int
    head_dim: int
    len_lo: int
    len_hi: int
    ring: int
    storage: int


C5 = DecodeConfig("C5", 64, 16, 64, 512, 4096, 64, 4096)


def packed_doc_lengths(rows: int, tokens: int, seed: int = 0, median: int = DOC_MEDIAN, sigma: float = DOC_SIGMA,
                       clip=DOC_CLIP) -> list[list[int]]:
    """Per-row document lengths (tokens) that exactly fill each row."""
    g = torch.Generator().manual_seed(seed)
    mu = math.log(median)
    out = []
    for _ in range(rows):
        row, filled = [], 0
        while filled < tokens:
            z = float(torch.randn((), generator=g))
            length = int(round(math.exp(mu + sigma * z)))
            length = max(clip[0], min(clip[1], length))
            length = min(length, tokens - filled)
            row.append(length)
            filled += length
        out.append(row)
    return out


def doc_ids_from_lengths(lengths_rows, tokens: int) -> np.ndarray:
    """[B, tokens] int64 ids 0, 1, ... per row following the lengths."""
    out = np.zeros((len(lengths_rows), tokens), dtype=np.int64)
    for b, row in enumerate(lengths_rows):
        pos = 0
        for i, length in enumerate(row):
            out[b, pos:pos + length] = i
            pos += length
    return out


def position_doc_ids(cfg: AttnConfig, seed: int = 0):
    """Document ids per attention position ([B, N] int64) and the per-row token lengths."""
    if not cfg.packed_docs:
        lengths = [[cfg.tokens] for _ in range(cfg.batch)]
    else:
        lengths = packed_doc_lengths(cfg.batch, cfg.tokens, seed)
    ids = doc_ids_from_lengths(lengths, cfg.tokens)
    if cfg.family != "full":
        ids = np.repeat(ids, 2, axis=1)
    return ids, lengths


def visible_pairs(cfg: AttnConfig, lengths_rows) -> int:
    """Exact number of visible (query, key) pairs per head summed over the batch rows, for rows
    made of whole contiguous documents and no persistent-key window. SPS families, per document of
    L tokens: L(L+1) + L + 2 * sum_{t<L} min(t, w); full family: L(L+1)/2."""
    total = 0
    for row in lengths_rows:
        for length in row:
            if cfg.family == "full":
                total += length * (length + 1) // 2
            else:
                t = np.arange(length)
                total += length * (length + 1) + length + 2 * int(np.minimum(t, cfg.window).sum())
    return total


def useful_flops(cfg: AttnConfig, lengths_rows, fwd: bool = True, bwd: bool = True) -> float:
    """Useful FLOPs: 4*D per visible pair forward, 10*D backward (the reference's 2.5x convention,
    original_flash_attn.py:749-755), times the number of heads."""
    pairs = visible_pairs(cfg, lengths_rows) * cfg.heads
    per = (4.0 if fwd else 0.0) + (10.0 if bwd else 0.0)
    return per * cfg.head_dim * pairs


def make_qkv(cfg: AttnConfig, seed: int = 0, with_grad: bool = True):
    """Q, K, V (and dO) ~ N(0, 1) drawn in that order on the CPU from one seeded generator."""
    g = torch.Generator().manual_seed(seed)
    shape = (cfg.batch, cfg.heads, cfg.n, cfg.head_dim)
    tensors = [torch.randn(shape, generator=g, dtype=torch.float32) for _ in range(4 if with_grad else 3)]
    return [t.to(cfg.dtype) for t in tensors]


def decode_lengths(cfg: DecodeConfig, seed: int = 0) -> torch.Tensor:
    """Per-sequence retained lengths, uniform in [len_lo, len_hi] (int64, CPU)."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(cfg.len_lo, cfg.len_hi + 1, (cfg.seqs,), generator=g, dtype=torch.int64)


def decode_bytes(cfg: DecodeConfig, lengths: torch.Tensor, nq: int = 1, n_extra: int = 2, kv_bytes: int = 2) -> int:
    """Algorithmic HBM bytes of one decode step: K and V of every live key (retained + full ring +
    extras) for every head, plus the query (kv dtype) and the fp32 output."""
    keys = int(lengths.sum()) * cfg.heads + cfg.seqs * cfg.heads * (cfg.ring + n_extra)
    return keys * cfg.head_dim * kv_bytes * 2 + cfg.seqs * cfg.heads * nq * cfg.head_dim * (kv_bytes + 4)
