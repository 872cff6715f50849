"""CPU restatement of the reference's decode engine (test infrastructure only).

Follows:

* ``ssd/engine/tree_drafter.py:34-45`` ``warp_probs`` (temperature + nucleus);
* ``ssd/engine/tree_drafter.py:48-95`` ``DraftTree`` (children in rank order,
  ancestors root->i inclusive, ``subset`` renumbering in original order);
* ``ssd/engine/tree_drafter.py:107-122`` capacity helpers;
* ``ssd/engine/tree_drafter.py:124-145`` ``_propose``; greedy top-k is taken as
  a stable descending sort, which pins the order of exactly equal log-probs to
  "lower column first" (``torch.topk`` leaves that order unspecified; the HIP
  draft head uses the same rule);
* ``ssd/engine/tree_drafter.py:147-208`` ``TreeDrafter.build``;
* ``ssd/engine/verify.py:32-95`` ``verify_inputs``, ``greedy_verify``,
  ``sample_verify``;
* ``ssd/engine/speculative.py:81-174`` ``_first_token``, ``_finish``,
  ``autoregressive_generate``, ``SpeculativeGenerator.generate``;
* ``ssd/data/token_freq.py:49-55`` ``top_vocab``.

Scores are Python floats (doubles), as in the reference, where ``.tolist()``
turns the fp32 log-probs into floats before they are summed.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Optional

import torch
import torch.nn.functional as F

ROOT = -1


def per_depth(value, depth: int, name: str) -> list:
    if value is None or isinstance(value, int):
        return [value] * depth
    if len(value) != depth:
        raise ValueError(f"drafting.{name} has {len(value)} entries but depth={depth}")
    return list(value)


@dataclass
class Drafting:
    depth: int = 4
    branch: object = 1
    width: object = None
    max_nodes: Optional[int] = None
    temperature: float = 0.0
    top_p: float = 1.0
    draft_vocab: Optional[int] = None


def warp_probs(logits: torch.Tensor, temperature: float, top_p: float) -> torch.Tensor:
    """softmax(logits/T); with top_p < 1 keep the smallest descending prefix whose mass
    reaches top_p (an entry is dropped when the mass *before* it already exceeds top_p),
    then renormalise."""
    probs = torch.softmax(logits.float() / temperature, dim=-1)
    if top_p >= 1.0:
        return probs
    sp, idx = probs.sort(dim=-1, descending=True)
    before = sp.cumsum(-1) - sp
    sp = sp.masked_fill(before > top_p, 0.0)
    out = torch.zeros_like(probs).scatter(-1, idx, sp)
    return out / out.sum(-1, keepdim=True)


@dataclass
class DraftTree:
    tokens: list = field(default_factory=list)
    parents: list = field(default_factory=list)
    depths: list = field(default_factory=list)
    scores: list = field(default_factory=list)
    ranks: list = field(default_factory=list)
    draft_pos: list = field(default_factory=list)
    child_q: dict = field(default_factory=dict)
    cache_start: int = 0

    def __len__(self) -> int:
        return len(self.tokens)

    def children(self) -> dict:
        out: dict = {}
        for i, p in enumerate(self.parents):
            out.setdefault(p, []).append(i)
        for kids in out.values():
            kids.sort(key=lambda i: self.ranks[i])
        return out

    def ancestors(self, i: int) -> list:
        path = []
        while i != ROOT:
            path.append(i)
            i = self.parents[i]
        return path[::-1]

    def subset(self, keep) -> "DraftTree":
        keep = sorted(keep)
        remap = {old: new for new, old in enumerate(keep)}
        remap[ROOT] = ROOT
        t = DraftTree(cache_start=self.cache_start)
        for old in keep:
            t.tokens.append(self.tokens[old])
            t.parents.append(remap[self.parents[old]])
            t.depths.append(self.depths[old])
            t.scores.append(self.scores[old])
            t.ranks.append(self.ranks[old])
            t.draft_pos.append(self.draft_pos[old])
        for p, q in self.child_q.items():
            if p in remap:
                t.child_q[remap[p]] = q
        return t


def level_sizes(cfg: Drafting) -> list:
    branch = per_depth(cfg.branch, cfg.depth, "branch")
    width = per_depth(cfg.width, cfg.depth, "width")
    n, out = 1, []
    for d in range(cfg.depth):
        n *= branch[d]
        if width[d] is not None:
            n = min(n, width[d])
        out.append(n)
    return out


def max_tree_cache(cfg: Drafting) -> int:
    return sum(level_sizes(cfg)[:-1])


def max_verify_nodes(cfg: Drafting) -> int:
    total = sum(level_sizes(cfg))
    return min(total, cfg.max_nodes) if cfg.max_nodes else total


def greedy_topk(logits: torch.Tensor, k: int):
    """Row-wise top-k of log_softmax(fp32 logits); equal values keep lower column first."""
    lp = F.log_softmax(logits.float(), -1)
    vals, idx = torch.sort(lp, dim=-1, descending=True, stable=True)
    return vals[:, :k], idx[:, :k]


def gumbel_topk(q: torch.Tensor, k: int, gumbel: torch.Tensor) -> list:
    """Draw min(k, support) tokens without replacement from q via keys log q + G, in draw
    order (tree_drafter.py:139-143). ``gumbel`` holds the standard-Gumbel noise."""
    support = int((q > 0).sum())
    keys = q.log() + gumbel
    return torch.topk(keys, min(k, support)).indices.tolist()


class TreeDrafter:
    def __init__(self, draft, cfg: Drafting, vocab_size: int):
        self.draft, self.cfg, self.vocab_size = draft, cfg, vocab_size
        self.branch = per_depth(cfg.branch, cfg.depth, "branch")
        self.width = per_depth(cfg.width, cfg.depth, "width")
        self.greedy = cfg.temperature == 0

    def propose(self, logits: torch.Tensor, k: int, gen: Optional[torch.Generator]):
        vocab_ids = self.draft.vocab_ids
        if self.greedy:
            lp, tok = greedy_topk(logits, k)
            if vocab_ids is not None:
                tok = vocab_ids[tok]
            return [(t, l, None) for t, l in zip(tok.tolist(), lp.tolist())]
        probs = warp_probs(logits, self.cfg.temperature, self.cfg.top_p)
        if vocab_ids is not None:
            full = torch.zeros(probs.shape[0], self.vocab_size)
            probs = full.index_copy_(1, vocab_ids, probs)
        out = []
        for q in probs:
            g = -torch.empty_like(q).exponential_(generator=gen).log()
            tok = gumbel_topk(q, k, g)
            out.append((tok, q[tok].log().tolist(), q))
        return out

    def build(self, cache, pending: list, root_pos: int, gen: Optional[torch.Generator] = None) -> DraftTree:
        n_pend = len(pending)
        pos = torch.arange(root_pos - n_pend + 1, root_pos + 1)
        logits, _ = self.draft(torch.tensor(pending), pos, cache, logits_to_keep=1)
        tree_start = cache.get_seq_length()
        tree = DraftTree(cache_start=tree_start)
        frontier, f_logits = [ROOT], logits[-1:]
        for d in range(self.cfg.depth):
            proposals = self.propose(f_logits, self.branch[d], gen)
            for parent, (_, _, q) in zip(frontier, proposals):
                if q is not None:
                    tree.child_q[parent] = q
            level = expand_level(tree, frontier, [(t, l) for t, l, _ in proposals], d, self.width[d])
            if d == self.cfg.depth - 1 or not level:
                break
            past = cache.get_seq_length()
            for j, i in enumerate(level):
                tree.draft_pos[i] = past + j
            mask = torch.zeros(len(level), past + len(level), dtype=torch.bool)
            mask[:, :tree_start] = True
            for j, i in enumerate(level):
                for a in tree.ancestors(i):
                    mask[j, tree.draft_pos[a]] = True
            ids = torch.tensor([tree.tokens[i] for i in level])
            frontier = level
            f_logits, _ = self.draft(ids, torch.full((len(level),), root_pos + d + 1), cache, mask)
        return prune_tree(tree, self.cfg.max_nodes)


def expand_level(tree: DraftTree, frontier: list, proposals: list, d: int, width: Optional[int]) -> list:
    """One level of TreeDrafter.build (tree_drafter.py:166-183): every frontier node's
    proposals (tokens, log-probs) become candidates scored parent score + lp (doubles); a
    stable sort on -score keeps (frontier order, proposal rank) among ties; the first
    ``width`` are appended. Returns the new node indices."""
    cands = []
    for parent, (toks, lps) in zip(frontier, proposals):
        base = tree.scores[parent] if parent != ROOT else 0.0
        cands += [(base + lp, parent, t, r) for r, (t, lp) in enumerate(zip(toks, lps))]
    cands.sort(key=lambda c: -c[0])
    if width is not None:
        cands = cands[:width]
    level = []
    for score, parent, tok, rank in cands:
        level.append(len(tree))
        tree.tokens.append(tok)
        tree.parents.append(parent)
        tree.depths.append(d + 1)
        tree.scores.append(score)
        tree.ranks.append(rank)
        tree.draft_pos.append(-1)
    return level


def prune_tree(tree: DraftTree, max_nodes: Optional[int]) -> DraftTree:
    """Final cut (tree_drafter.py:202-207): best ``max_nodes`` by (-score, depth), closed
    under ancestors, renumbered in original order."""
    if max_nodes is None or len(tree) <= max_nodes:
        return tree
    keep = set(prune_order(tree.scores, tree.depths, max_nodes))
    for i in list(keep):
        keep.update(tree.ancestors(i))
    return tree.subset(sorted(keep))


def prune_order(scores: list, depths: list, max_nodes: int) -> list:
    """Indices kept by the final max_nodes cut (tree_drafter.py:202-207), before ancestor closure."""
    order = sorted(range(len(scores)), key=lambda i: (-scores[i], depths[i]))
    return sorted(order[:max_nodes])


def verify_inputs(tree: DraftTree, root_token: int, root_pos: int, past_len: int):
    n = len(tree)
    ids = torch.tensor([root_token] + tree.tokens)
    pos = torch.tensor([root_pos] + [root_pos + d for d in tree.depths])
    mask = torch.zeros(n + 1, past_len + n + 1, dtype=torch.bool)
    mask[:, : past_len + 1] = True
    for i in range(n):
        for a in tree.ancestors(i):
            mask[i + 1, past_len + 1 + a] = True
    return ids, pos, mask


def greedy_verify(tree: DraftTree, logits: torch.Tensor):
    argmax = logits.argmax(-1).tolist()
    kids = tree.children()
    accepted, cur = [], ROOT
    while True:
        want = argmax[cur + 1]
        nxt = next((c for c in kids.get(cur, []) if tree.tokens[c] == want), None)
        if nxt is None:
            return accepted, want
        accepted.append(nxt)
        cur = nxt


def sample_verify(tree: DraftTree, logits: torch.Tensor, temperature: float, top_p: float, gen=None):
    kids = tree.children()
    accepted, cur = [], ROOT
    while True:
        p = warp_probs(logits[cur + 1], temperature, top_p)
        children = kids.get(cur, [])
        if children:
            q = tree.child_q[cur].clone()
            chosen = None
            for c in children:
                x = tree.tokens[c]
                if q[x] <= 0:
                    continue
                if torch.rand((), generator=gen).item() < min(1.0, (p[x] / q[x]).item()):
                    chosen = c
                    break
                residual = (p - q).clamp_min(0)
                if residual.sum() > 0:
                    p = residual / residual.sum()
                q[x] = 0
                if q.sum() <= 0:
                    break
                q = q / q.sum()
            if chosen is not None:
                accepted.append(chosen)
                cur = chosen
                continue
        return accepted, torch.multinomial(p, 1, generator=gen).item()


def first_token(logits: torch.Tensor, temperature: float, top_p: float, gen) -> int:
    if temperature == 0:
        return int(logits.argmax())
    return int(torch.multinomial(warp_probs(logits, temperature, top_p), 1, generator=gen))


def finish(tokens: list, eos_ids: set, max_new: int):
    for i, t in enumerate(tokens[:max_new]):
        if t in eos_ids:
            return tokens[: i + 1], True
    return tokens[:max_new], len(tokens) >= max_new


@dataclass
class Result:
    tokens: list
    accepted_per_round: list = field(default_factory=list)
    tree_sizes: list = field(default_factory=list)
    decode_seconds: float = 0.0  # wall time of the rounds (prefill excluded)

    @property
    def mean_accepted(self) -> float:
        return sum(self.accepted_per_round) / max(1, len(self.accepted_per_round))


@torch.no_grad()
def autoregressive_generate(target, input_ids: list, max_new: int, eos_ids: set, temperature=0.0, top_p=1.0,
                            seed=None) -> Result:
    gen = torch.Generator().manual_seed(seed) if seed is not None else None
    cache = target.new_cache(len(input_ids) + max_new + 1)
    logits, _ = target(torch.tensor(input_ids), None, cache, logits_to_keep=1)
    out = [first_token(logits[-1], temperature, top_p, gen)]
    while not finish(out, eos_ids, max_new)[1]:
        logits, _ = target(torch.tensor([out[-1]]), None, cache)
        out.append(first_token(logits[-1], temperature, top_p, gen))
    return Result(tokens=finish(out, eos_ids, max_new)[0])


class SpeculativeGenerator:
    def __init__(self, target, draft, cfg: Drafting, vocab_size: int):
        self.target, self.draft, self.cfg = target, draft, cfg
        self.drafter = TreeDrafter(draft, cfg, vocab_size)

    @torch.no_grad()
    def generate(self, input_ids: list, max_new: int, eos_ids: set, seed=None, max_rounds=None) -> Result:
        cfg = self.cfg
        gen = torch.Generator().manual_seed(seed) if seed is not None else None
        extra = max(max_verify_nodes(cfg), max_tree_cache(cfg)) + 1
        cache = self.target.new_cache(len(input_ids) + max_new + cfg.depth + extra + 1)
        logits, _ = self.target(torch.tensor(input_ids), None, cache, logits_to_keep=1)
        out = [first_token(logits[-1], cfg.temperature, cfg.top_p, gen)]
        res = Result(tokens=[])
        t0 = time.perf_counter()
        while not finish(out, eos_ids, max_new)[1]:
            if max_rounds is not None and len(res.accepted_per_round) >= max_rounds:
                break
            committed = cache.get_seq_length()
            tree = self.drafter.build(cache, [out[-1]], committed, gen)
            cache.crop(committed)
            ids, pos, mask = verify_inputs(tree, out[-1], committed, committed)
            logits, _ = self.target(ids, pos, cache, mask)
            if cfg.temperature == 0:
                accepted, bonus = greedy_verify(tree, logits)
            else:
                accepted, bonus = sample_verify(tree, logits, cfg.temperature, cfg.top_p, gen)
            cache.keep_positions(committed, [committed] + [committed + 1 + i for i in accepted])
            new = [tree.tokens[i] for i in accepted] + [bonus]
            out.extend(new)
            res.accepted_per_round.append(len(new))
            res.tree_sizes.append(len(tree))
        res.decode_seconds = time.perf_counter() - t0
        res.tokens = finish(out, eos_ids, max_new)[0]
        return res


def top_vocab(counts: torch.Tensor, size: int, always=frozenset()) -> torch.Tensor:
    """The ``size`` most frequent ids (always including ``always``), sorted ascending."""
    order = counts.argsort(descending=True, stable=True)
    forced = [t for t in always if 0 <= t < counts.numel()]
    keep = torch.tensor(forced, dtype=torch.long)
    rest = order[~torch.isin(order, keep)][: max(0, size - len(forced))]
    return torch.cat([keep, rest]).sort().values
