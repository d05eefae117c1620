"""HIP-graph capture of the attention training step (GPU).

The step's launches (row-layout prepass, forward, dQ, dK/dV) are captured once with torch's graph
capture and replayed; every replay, with eager work and synchronizations between the replays, must
reproduce the eager step bit for bit (the kernels are deterministic and record no memset nodes).
"""

import math

import pytest
import torch

from sps_amd import _native as N
from sps_amd import attention as SA
from sps_amd.workloads import AttnConfig, make_qkv, position_doc_ids

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("family,docs", [("sps", True), ("reverse_sps", True), ("full", False)])
def test_graph_replays_match_eager(family, docs):
    cfg = AttnConfig("G", family, 2, 4, 64, 512, 16, docs, torch.bfloat16)
    fam = {"full": N.FAMILY_FULL, "sps": N.FAMILY_SPS, "reverse_sps": N.FAMILY_REVERSE_SPS}[family]
    q, k, v, do = (t.cuda() for t in make_qkv(cfg, seed=3))
    d = torch.tensor(position_doc_ids(cfg, seed=3)[0], device="cuda") if docs else None
    scale = 1.0 / math.sqrt(cfg.head_dim)

    def step():
        o, lse, _, _, _, ws = SA.attention_forward(q, k, v, scale, fam, cfg.window, d, keep_layout=True)
        dq, dk, dv = SA.attention_backward(do, q, k, v, o, lse, scale, fam, cfg.window, d, layout_workspace=ws)
        return o, dq, dk, dv

    eager = step()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()
    for rep in range(4):
        graph.replay()
        torch.cuda.synchronize()
        for name, x, y in zip(("o", "dq", "dk", "dv"), captured, eager):
            assert torch.equal(x, y), f"replay {rep}: {name} differs from the eager step"
        step()  # eager work between the replays
        torch.cuda.synchronize()
