"""Draft-vocabulary selection (reference ssd/data/token_freq.py).

``top_vocab`` picks the N most frequent token ids (forced ids included), sorted ascending;
the draft's lm_head then scores only those rows. Counting frequencies over a text dataset
is training-side and stays out of this package; ``zipf_counts`` gives the seeded synthetic
frequencies used by the benchmarks (Zipf(s) expected counts over a seeded permutation).
"""

from __future__ import annotations

from pathlib import Path

import torch


def token_freq_path(cfg) -> Path:
    return Path(cfg.training.output_dir) / "token_freq.pt"


def top_vocab(counts: torch.Tensor, size: int, always=frozenset()) -> torch.Tensor:
    """The ``size`` most frequent ids (stable on ties), always including ``always``, sorted
    ascending (reference token_freq.py:49-55)."""
    order = counts.argsort(descending=True, stable=True)
    forced = [t for t in always if 0 <= t < counts.numel()]
    keep = torch.tensor(forced, dtype=torch.long)
    rest = order[~torch.isin(order, keep)][: max(0, size - len(forced))]
    return torch.cat([keep, rest]).sort().values


def zipf_counts(vocab: int, s: float = 1.1, seed: int = 0, total: float = 1e9) -> torch.Tensor:
    """Expected counts of a Zipf(s) law over a seeded permutation of the vocabulary."""
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(vocab, generator=g)
    rank = torch.arange(1, vocab + 1, dtype=torch.float64)
    w = rank.pow(-s)
    counts = torch.empty(vocab, dtype=torch.float64)
    counts[perm] = w / w.sum() * total
    return counts.round().long()
