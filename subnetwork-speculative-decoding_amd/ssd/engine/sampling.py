"""Device state of a sampled decode (temperature > 0).

The reference samples on the host (ssd/engine/tree_drafter.py:134-144 for draft proposals,
ssd/engine/verify.py:60-95 for acceptance, ssd/engine/speculative.py:81-84 for single draws)
with torch's CPU generator. Here the same algorithms run as kernels
(``ssd_warp_probs_bf16``, ``ssd_gumbel_topk``, ``ssd_accept_sample``, ``ssd_sample_rows``)
drawing from Philox4x32-10: a generation is reproducible from its seed, and a round needs
no host round trip.

Counters: draw ``c`` of a generation uses Philox counter ``c`` (0 = the token after the
prompt, then one per speculative round or autoregressive step); the kernels separate the
draws inside one counter (proposals per level and row, acceptance tests, bonus) by tag.
"""

from __future__ import annotations

import os
from typing import Optional

import torch

from ssd import ops


def new_seed() -> int:
    return int.from_bytes(os.urandom(8), "little") & ((1 << 63) - 1)


def seed_from_generator(generator: Optional[torch.Generator]) -> int:
    """A Philox seed drawn from a torch generator (reference API calls pass one), so a seeded
    generator gives a reproducible draw."""
    if generator is None:
        return new_seed()
    return int(torch.randint(0, 2**62, (1,), generator=generator))


class Sampler:
    """Buffers of one sampled decode stream on ``device``.

    ``Q`` [q_rows, V] fp32: warped draft distributions, row 0 for the root and 1 + i for tree
    node i (written while drafting, read by acceptance); ``P`` [p_rows, V] fp32: warped target
    rows of the current verify pass; ``ws``: the kernels' workspace (chunk partials, histograms).
    """

    def __init__(self, temperature: float, top_p: float, vocab: int, device, q_rows: int, p_rows: int,
                 seed: Optional[int] = None):
        if not temperature > 0:
            raise ValueError("sampling needs temperature > 0")
        self.temperature, self.top_p, self.vocab = float(temperature), float(top_p), int(vocab)
        self.seed = new_seed() if seed is None else int(seed) & ((1 << 64) - 1)
        self.counter = 0
        ld = (self.vocab + 3) // 4 * 4
        f32 = dict(dtype=torch.float32, device=device)
        self.Q = torch.zeros(max(q_rows, 1), ld, **f32)
        self.P = torch.zeros(max(p_rows, 1), ld, **f32)
        self.ws = torch.empty(ops.sample_ws_bytes(max(p_rows, q_rows, 1), self.vocab), dtype=torch.uint8,
                              device=device)
        self.max_kids = 1

    # ------------------------------------------------------------------ drafting
    def propose(self, draft, logits: torch.Tensor, rows: int, level: int, k: int, tree_meta: torch.Tensor,
                cand_tok: torch.Tensor, cand_lp: torch.Tensor) -> None:
        """Sampling branch of _propose for the frontier proposing ``level``: warp the draft
        logits into Q (full vocabulary, zero outside a draft-vocab subset), then draw the
        children by Gumbel top-k."""
        n = logits.shape[1]
        ops.warp_probs(logits, rows, n, self.temperature, self.top_p, self.Q, V=self.vocab,
                       vocab_ids=draft._vocab_ids_i32, vocab_inv=draft._vocab_inv, tree_meta=tree_meta, level=level,
                       ws=self.ws)
        ops.gumbel_topk(self.Q, rows, self.vocab, k, self.seed, self.counter, cand_tok, cand_lp,
                        tree_meta=tree_meta, level=level, ws=self.ws)

    # --------------------------------------------------------------- verification
    def accept(self, tree, logits: torch.Tensor, m: int, committed: int, result: torch.Tensor,
               keep_src: torch.Tensor, n_keep: torch.Tensor, root_token: torch.Tensor) -> None:
        """sample_verify on the device: warp the m target rows into P, then the acceptance walk
        (writes the round record like ssd_accept_greedy)."""
        ops.warp_probs(logits, m, self.vocab, self.temperature, self.top_p, self.P, ws=self.ws)
        ops.accept_sample(tree.struct, self.P, self.Q, self.vocab, m, self.max_kids, self.seed, self.counter,
                          committed, result, keep_src, n_keep, root_token, ws=self.ws)

    # ------------------------------------------------------------------ one draw
    def draw(self, logits: torch.Tensor, out_tok: torch.Tensor, counter: Optional[int] = None) -> None:
        """torch.multinomial(warp_probs(logits)) for one row of logits into out_tok[0]."""
        ops.warp_probs(logits, 1, self.vocab, self.temperature, self.top_p, self.P, ws=self.ws)
        ops.sample_rows(self.P, 1, self.vocab, self.seed, self.counter if counter is None else counter, out_tok,
                        ws=self.ws)
