"""Writes doc_lengths_c2_c4.json: the per-row document lengths (tokens) of the packed benchmark
workloads C2, C3 and C4 (seed 0), as sps_amd.workloads.packed_doc_lengths draws them. The fixture
fixes the synthetic workload across machines and torch versions; tests/test_workloads.py checks that
the generator still reproduces it.

Run from the repository root: python tests/golden/make_doc_lengths.py
"""
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from sps_amd.workloads import C2, C3, C4, packed_doc_lengths  # noqa: E402

out = {}
for cfg in (C2, C3, C4):
    out[cfg.name] = {"batch": cfg.batch, "tokens": cfg.tokens, "seed": 0,
                     "lengths": packed_doc_lengths(cfg.batch, cfg.tokens, seed=0)}
(Path(__file__).resolve().parent / "doc_lengths_c2_c4.json").write_text(json.dumps(out, indent=1) + "\n")
print({k: [len(r) for r in v["lengths"]] for k, v in out.items()})
