"""CPU oracle for the speculative-decoding hot path -- TEST INFRASTRUCTURE ONLY.

This package is a plain PyTorch-CPU restatement of the reference's decode path
(the model forward with a shared KV cache and tree masks, the level-by-level
tree drafter, greedy / sampling verification, KV compaction and the round
loop). It exists to check the HIP path; it is never the thing measured or
shipped. Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may import it, and only as the checker / CPU baseline.

How each part is pinned (so that a plausible mistake fails a check):

* ``model``: layer math against the transformers ``LlamaForCausalLM`` in the
  image (a library routine) in fp32 to 1e-5 (tests/test_oracle_model.py),
  zero-init bridges against plain layer skipping, incremental cache against
  the full forward, and tree masks against decoding each root->node path
  alone (the reference's own invariants, tests/test_forward_pass.py:109-180).
* ``engine``: greedy SD == autoregressive == HF ``generate`` for chain, tree,
  pruned and deep-chain drafts; draft-vocab subsets and EOS; tree-shape
  limits; the V=8 brute-force joint for sampling (tests/test_engine.py).
  Tree pruning order and ``warp_probs`` boundaries are also pinned by small
  hand-derived known-answer cases (tests/test_oracle_engine.py). The per-level
  expansion ``expand_level`` (stable sort on -score, width cut) is pinned by a
  hand-derived case with ties across parents and ranks, a brute-force ranking by
  the explicit key (-score, frontier index, rank), and mutation guards (sign flip,
  other tie orders, dropped or shifted width cut) that must fail
  (tests/test_oracle_expand.py).
* ``sampling``: the sampling path with the kernels' Philox4x32-10 streams: the
  generator against its published known-answer vectors, the nucleus warp against
  hand-derived cases (ties included) and the fp32 rule, the verify.py:60-95 loop
  against the precomputed-state formulation decision for decision, and the
  speculative-sampling theorem (first committed token ~ warped target, chi-square,
  with a planted-mistake negative control) (tests/test_oracle_sampling.py).
* ``kernels``: per-kernel reference functions (tree attention with ancestor
  lists, KV compaction, the bf16 rounding chains). Each is pinned against
  the ``model`` forward (itself pinned to HF) or a closed form.

Parity unpinned: none of the functions above is left without an independent
check. Sampled trajectories of the HIP path are compared draw for draw with
``sampling`` (same Philox streams); against the reference's own torch-generator
streams they can only be compared distributionally (the reference was not run
here to record them).
"""
