"""Pins ``oracle.engine.expand_level`` -- one level of ``TreeDrafter.build``
(reference ``ssd/engine/tree_drafter.py:165-183``): candidates scored parent score + log-prob,
a stable sort on -score (ties keep frontier order, then proposal rank), the ``width`` cut.

Three independent checks, chosen so that a plausible slip fails at least one:
* a hand-derived known answer with exact ties across parents and ranks and a width cut;
* a brute-force restatement on random tiny inputs that ranks every candidate by counting how
  many others precede it under the explicit key (-score, frontier index, rank) -- no sort,
  no reliance on stability;
* mutation guards: the sign of the sort flipped, ties broken by token, by rank before
  frontier order, or in reverse, and a dropped width cut must each fail the checks above.
All scores are dyadic fractions, so every sum is exact in doubles and ties are real ties.
"""

import inspect
import random

import pytest

from oracle import engine as oe


def _tree_with_frontier(scores):
    """A tree whose level-1 nodes 0..n-1 carry the given scores (root children)."""
    t = oe.DraftTree()
    for i, s in enumerate(scores):
        t.tokens.append(100 + i)
        t.parents.append(oe.ROOT)
        t.depths.append(1)
        t.scores.append(s)
        t.ranks.append(i)
        t.draft_pos.append(i)
    return t


# frontier nodes 0, 1, 2 with scores -1.0, -0.5, -1.0; proposals in (tokens, log-probs) per parent
KA_FRONTIER_SCORES = [-1.0, -0.5, -1.0]
KA_PROPOSALS = [
    ([50, 11], [-0.5, -1.0]),          # -> -1.5 (r0), -2.0 (r1)
    ([20, 21, 22], [-1.0, -1.0, -1.5]),  # -> -1.5 (r0), -1.5 (r1), -2.0 (r2)
    ([30, 5], [-0.5, -0.25]),          # -> -1.5 (r0), -1.25 (r1)
]
# Sorted by -score, ties in (frontier, rank) order:
#   -1.25: (p2, 5, r1); -1.5: (p0, 50, r0), (p1, 20, r0), (p1, 21, r1), (p2, 30, r0);
#   -2.0: (p0, 11, r1), (p1, 22, r2)
KA_ALL = {
    "tokens": [5, 50, 20, 21, 30, 11, 22],
    "parents": [2, 0, 1, 1, 2, 0, 1],
    "ranks": [1, 0, 0, 1, 0, 1, 2],
    "scores": [-1.25, -1.5, -1.5, -1.5, -1.5, -2.0, -2.0],
}


def _run(fn, frontier_scores, proposals, width, d=1):
    tree = _tree_with_frontier(frontier_scores)
    frontier = list(range(len(frontier_scores)))
    n0 = len(tree)
    level = fn(tree, frontier, proposals, d, width)
    return tree, level, n0


def _known_answer_ok(fn) -> bool:
    for width in (None, 4, 1):
        tree, level, n0 = _run(fn, KA_FRONTIER_SCORES, KA_PROPOSALS, width)
        n = 7 if width is None else width
        if level != list(range(n0, n0 + n)) or len(tree) != n0 + n:
            return False
        got = {k: getattr(tree, k)[n0:] for k in KA_ALL}
        want = {k: v[:n] for k, v in KA_ALL.items()}
        if got != want or tree.depths[n0:] != [2] * n or tree.draft_pos[n0:] != [-1] * n:
            return False
    # the root as the only parent: base score 0.0
    t = oe.DraftTree()
    lv = fn(t, [oe.ROOT], [([7, 3, 9], [-0.75, -0.25, -0.75])], 0, 2)
    return lv == [0, 1] and t.tokens == [3, 7] and t.scores == [-0.25, -0.75] and t.parents == [oe.ROOT] * 2 \
        and t.ranks == [1, 0] and t.depths == [1, 1]


def _brute(frontier_scores, proposals, width):
    """Expected level by counting: candidate c goes to position #{c' : key(c') < key(c)} with
    key = (-score, frontier index, rank); kept when the position is below the width."""
    cands = []
    for f, (toks, lps) in enumerate(proposals):
        for r, (t, lp) in enumerate(zip(toks, lps)):
            cands.append((frontier_scores[f] + lp, f, r, t))
    out = [None] * len(cands)
    for c in cands:
        key = (-c[0], c[1], c[2])
        pos = sum(1 for o in cands if (-o[0], o[1], o[2]) < key)
        out[pos] = c
    if width is not None:
        out = out[:width]
    return out


def _brute_ok(fn, trials=300, seed=0) -> bool:
    rng = random.Random(seed)
    for _ in range(trials):
        F = rng.randint(1, 4)
        fs = [-0.5 * rng.randint(0, 3) for _ in range(F)]
        props = []
        for _ in range(F):
            k = rng.randint(0, 4)  # 0: a parent with an empty support
            toks = rng.sample(range(64), k)
            props.append((toks, [-0.25 * rng.randint(0, 4) for _ in range(k)]))
        total = sum(len(t) for t, _ in props)
        width = rng.choice([None, 1, 2, 3, max(1, total // 2), total + 1])
        tree, level, n0 = _run(fn, fs, props, width)
        want = _brute(fs, props, width)
        if level != list(range(n0, n0 + len(want))):
            return False
        got = list(zip(tree.scores[n0:], tree.parents[n0:], tree.ranks[n0:], tree.tokens[n0:]))
        if got != [(s, f, r, t) for s, f, r, t in want]:
            return False
    return True


def test_expand_level_known_answer():
    assert _known_answer_ok(oe.expand_level)


def test_expand_level_brute_force():
    assert _brute_ok(oe.expand_level)


def _mutant(old: str, new: str):
    src = inspect.getsource(oe.expand_level)
    assert old in src, f"mutation site {old!r} not found"
    ns = dict(vars(oe))
    exec(compile(src.replace(old, new), "<mutant>", "exec"), ns)
    return ns["expand_level"]


MUTANTS = {
    "sign flipped": ("key=lambda c: -c[0]", "key=lambda c: c[0]"),
    "ties by token": ("key=lambda c: -c[0]", "key=lambda c: (-c[0], c[2])"),
    "ties by rank first": ("key=lambda c: -c[0]", "key=lambda c: (-c[0], c[3])"),
    "ties reversed": ("key=lambda c: -c[0]", "key=lambda c: -c[0], reverse=False) or cands.reverse() or cands.sort(key=lambda c: c[0], reverse=True"),
    "no width cut": ("cands = cands[:width]", "pass"),
    "width off by one": ("cands = cands[:width]", "cands = cands[:width + 1]"),
    "parent score dropped": ("base + lp", "lp"),
}


@pytest.mark.parametrize("name", list(MUTANTS))
def test_expand_level_mutants_fail(name):
    fn = _mutant(*MUTANTS[name])
    assert not (_known_answer_ok(fn) and _brute_ok(fn, trials=100)), f"mutant '{name}' passed every check"
