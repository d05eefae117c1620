"""CPU oracle of the SPS attention hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithms of the reference (lil-lab/sps) for the attention
path: the visibility predicate (C, ``sps_oracle.c``, and an independent numpy form), dense masked
attention forward/backward (numpy, float64), an emulation of the reference kernels' own 16-bit
arithmetic (torch CPU, float32: ``emulate.py``), segmented decode attention (numpy, float64), document
ids (numpy), and a torch-CPU port of the reference's CPU fallback path used as the timed CPU
baseline. Each function cites the reference file:line it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import it,
and only as the checker (or the timed CPU baseline) — never as the thing measured or shipped.
The product (``sps_amd``) never imports it.

Pinning (what makes each function trustworthy; see tests/test_oracle_*.py):
  mask (C and numpy)     — reference KATs (test_sps_attention.py doc layout, reverse-SPS visibility
                           lists, persistent-key-window config, causal matrix), C == numpy on random
                           configs, brute-force closed-form pair counts, w >= T == dense causal.
  dense attention        — float64 torch autograd on the same inputs (independent of the hand-written
                           backward formulas), finite differences, softmax invariants.
  decode                 — the reference test's explicit per-(b,h) softmax semantics, dense SPS
                           attention == stepwise decode over ring + retained + current keys.
  kv update              — the reference's ring-wrap KAT (delayed_state/test_forward_efficient.py),
                           the closed form of a ring after n inserts (insert i in slot i mod W,
                           len = min(n, W), pos = n mod W once full), retained append up to storage.
  document ids           — reference KATs (core/test_document_idx.py).
  emulate (the reference — with rounding off it equals the float64 dense attention for every family,
   kernels' 16-bit         block size and mask; with float32 as the "16-bit" type it is fp32-accurate;
   arithmetic)             uniform scores give the closed form (mean of V, M = log2 count).
"""
