"""Pins of the sampling restatement (oracle/sampling.py) on the CPU.

* Philox4x32-10 against the generator's published known-answer vectors.
* The Exp(1) transform against its closed-form extremes and a Kolmogorov-Smirnov test.
* The nucleus warp against hand-derived cases (including exact ties, which the reference leaves
  to torch's sort order) and against oracle.engine.warp_probs where nothing ties.
* The loop restatement of verify.py:60-95 (Philox randomness) against the precomputed-state
  formulation the kernels use, decision for decision.
* The speculative-sampling theorem: the first committed token of a round is distributed as the
  warped target, whatever the draft (chi-square over many counters).
"""

import numpy as np
import pytest
import torch
from scipy import stats

from oracle import engine as oe
from oracle import sampling as osm


def test_philox_known_answers():
    """Random123 kat_vectors for philox4x32_10."""
    kat = [
        ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
        ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
        ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
         (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
    ]
    for ctr, key, want in kat:
        got = osm.philox4x32_10(*[np.uint32(c) for c in ctr], *key)
        assert tuple(int(g) for g in got) == want


def test_philox_vectorised_matches_scalar():
    idx = np.arange(8, dtype=np.uint32)
    s = osm.Stream(seed=0x1234_5678_9ABC_DEF0, counter=(5 << 32) | 77)
    batch = s.bits(idx, 3, osm.TAG_BONUS)
    for i in range(8):
        one = osm.philox4x32_10(np.uint32(i), np.uint32(3), np.uint32(77), np.uint32((5 << 8) | osm.TAG_BONUS),
                                0x9ABCDEF0, 0x12345678)
        assert tuple(int(x) for x in one) == tuple(int(x) for x in batch[i])


def test_exp1_transform():
    e = osm.exp1_from_bits(np.array([0, 0xFFFFFFFF, 0x7FFFFFFF, 0x80000000], dtype=np.uint32))
    assert e[0] == pytest.approx(-np.log(0.5 * 2.0 ** -32), rel=1e-6)  # largest value, 22.87
    assert e[1] == pytest.approx(0.5 * 2.0 ** -32, rel=1e-3)  # smallest, through 1 - U
    assert e[2] == pytest.approx(np.log(2.0), rel=1e-6) and e[3] == pytest.approx(np.log(2.0), rel=1e-6)
    x = osm.exp1_from_bits(osm.Stream(7, 0).element_bits(200_000, 0, osm.TAG_DRAW))
    assert stats.kstest(x, "expon").pvalue > 1e-3
    assert abs(x.mean() - 1.0) < 0.01


def test_warp_known_answers():
    lg = torch.log(torch.tensor([0.5, 0.3, 0.2]))
    p, _ = osm.warp_probs(lg, 1.0, 0.6)  # before = [0, .5, .8] -> keep 2
    torch.testing.assert_close(p, torch.tensor([0.625, 0.375, 0.0]), atol=1e-6, rtol=0)
    p, _ = osm.warp_probs(lg, 1.0, 0.4)  # before .5 > .4 -> keep 1
    torch.testing.assert_close(p, torch.tensor([1.0, 0.0, 0.0]), atol=1e-6, rtol=0)
    p, _ = osm.warp_probs(lg, 1.0, 1.0)  # no cut, no renormalisation
    torch.testing.assert_close(p, torch.tensor([0.5, 0.3, 0.2]), atol=1e-6, rtol=0)
    # temperature: softmax(logits / T)
    p, _ = osm.warp_probs(torch.tensor([0.0, 1.0]), 0.5, 1.0)
    torch.testing.assert_close(p, torch.softmax(torch.tensor([0.0, 2.0]), -1))
    # exact ties: four equal entries at 0.25, top_p 0.3 keeps two (before = 0, .25), lowest columns
    p, _ = osm.warp_probs(torch.zeros(4), 1.0, 0.3)
    torch.testing.assert_close(p, torch.tensor([0.5, 0.5, 0.0, 0.0]), atol=1e-6, rtol=0)
    # ties mixed with a larger entry: [.4, .2, .2, .2], top_p .5 -> before = 0, .4, .6 -> keep 2
    lg = torch.log(torch.tensor([0.2, 0.4, 0.2, 0.2]))
    p, _ = osm.warp_probs(lg, 1.0, 0.5)
    torch.testing.assert_close(p, torch.tensor([1 / 3, 2 / 3, 0.0, 0.0]), atol=1e-6, rtol=0)


@pytest.mark.parametrize("V", [8, 128256])
def test_warp_exact_equality_at_the_cut(V):
    """Four tied leaders (logit 0, p = 0.25 exactly; every other logit -1000, p = 0): the mass
    before them is 0, .25, .5, .75 and an entry survives while that mass is <= top_p. top_p 0.5
    keeps three, 0.25 two, 0.75 all four; ties keep the lowest columns. Both the fp32 rule and
    the float64 checker must agree exactly, without a band."""
    x = torch.full((V,), -1000.0)
    leaders = [2, 3, 6, 7] if V == 8 else [5, 4100, 70000, 128255]
    x[leaders] = 0.0
    for T in (1.0, 0.7):
        for top_p, n in ((0.5, 3), (0.25, 2), (0.75, 4)):
            p, _ = osm.warp_probs(x, T, top_p)
            assert (p > 0).nonzero().flatten().tolist() == leaders[:n], (T, top_p)
            torch.testing.assert_close(p[leaders[:n]], torch.full((n,), 1.0 / n))
            p64, kept, _ = osm.warp_probs64(x, T, top_p)
            assert kept.nonzero().flatten().tolist() == leaders[:n], (T, top_p)
            assert float(p64[leaders[0]]) == 0.25


def test_warp_matches_engine_without_ties():
    g = torch.Generator().manual_seed(0)
    for top_p in (1.0, 0.9, 0.5, 0.05):
        lg = torch.randn(5, 1000, generator=g) * 3
        for row in lg:
            a, _ = osm.warp_probs(row, 0.7, top_p)
            torch.testing.assert_close(a, oe.warp_probs(row, 0.7, top_p), atol=1e-7, rtol=1e-6)


def random_tree(rng, V, depth, branch, q_rows, p_rows, subset=None):
    """A tree whose children are real Gumbel top-k draws from q (so they are distinct and in
    q's support), with random target rows. Returns tokens, parents, ranks, P, child_q."""
    tokens, parents, ranks, child_q = [], [], [], {}
    frontier = [osm.ROOT]
    stream = osm.Stream(int(rng.integers(1 << 62)), int(rng.integers(1 << 20)))
    for d in range(depth):
        nxt = []
        for f, par in enumerate(frontier):
            q = q_rows(rng)
            child_q[par] = q
            toks, _, _ = osm.gumbel_topk(q, branch[d], stream, f, d)
            for r, t in enumerate(toks):
                tokens.append(t)
                parents.append(par)
                ranks.append(r)
                nxt.append(len(tokens) - 1)
        frontier = nxt
    P = torch.stack([p_rows(rng) for _ in range(len(tokens) + 1)])
    return tokens, parents, ranks, P, child_q


def dist(rng, V, sharp=2.0, zero_frac=0.0):
    w = torch.from_numpy(rng.standard_normal(V).astype(np.float32)) * sharp
    p = torch.softmax(w, -1)
    if zero_frac:
        p[torch.from_numpy(rng.random(V) < zero_frac)] = 0
        p = p / p.sum()
    return p


@pytest.mark.parametrize("V,branch,zero", [(16, [3, 2], 0.0), (64, [4, 2, 1], 0.3), (9, [5, 3], 0.5)])
def test_state_formulation_matches_loop(V, branch, zero):
    rng = np.random.default_rng(V)
    agree = fragile = 0
    for trial in range(150):
        tokens, parents, ranks, P, child_q = random_tree(
            rng, V, len(branch), branch, lambda r: dist(r, V, 2.0, zero), lambda r: dist(r, V, 1.0, zero))
        s = osm.Stream(trial, trial + 1)
        acc, bonus, frag = osm.sample_verify(tokens, parents, ranks, P, child_q, s)
        acc2, bonus2 = osm.sample_verify_states(tokens, parents, ranks, P, child_q, s)
        if frag:
            fragile += 1
            continue
        assert (acc, bonus) == (acc2, bonus2), f"trial {trial}"
        agree += 1
    assert agree >= 140


@pytest.mark.parametrize("top_p,residual", [(1.0, True), (0.8, True), (1.0, False)])
def test_first_token_is_target_distributed(top_p, residual):
    """Speculative sampling is exact: the first committed token ~ warp(target row 0), for any
    draft. Chi-square over 6000 rounds with fresh Philox counters. Negative control: without the
    residual update (a plausible slip) the test must reject."""
    V, T = 12, 0.9
    rng = np.random.default_rng(3)
    tl = torch.from_numpy(rng.permutation(np.linspace(0.0, 1.5, V)).astype(np.float32))
    dl = tl + torch.from_numpy(rng.standard_normal(V).astype(np.float32))
    p_root, _ = osm.warp_probs(tl, T, top_p)
    q_root, _ = osm.warp_probs(dl, T, top_p)
    other = torch.stack([osm.warp_probs(torch.from_numpy(rng.standard_normal(V).astype(np.float32)), T, top_p)[0]
                         for _ in range(8)])
    counts = np.zeros(V)
    N = 6000
    for n in range(N):
        s = osm.Stream(99, n)
        toks, _, _ = osm.gumbel_topk(q_root, 3, s, 0, 0)
        k = len(toks)
        tokens, parents, ranks = toks, [osm.ROOT] * k, list(range(k))
        P = torch.cat([p_root[None], other[:k]])
        acc, bonus, _ = osm.sample_verify(tokens, parents, ranks, P, {osm.ROOT: q_root}, s, _residual=residual)
        first = tokens[acc[0]] if acc else bonus
        counts[first] += 1
    exp = p_root.double().numpy()
    exp = exp / exp.sum() * N
    keep = exp >= 5
    obs = np.append(counts[keep], counts[~keep].sum())
    ex = np.append(exp[keep], exp[~keep].sum())
    if ex[-1] == 0:
        obs, ex = obs[:-1], ex[:-1]
    assert len(ex) >= 4  # several tokens survive the warp, so the test has power
    pv = stats.chisquare(obs, ex).pvalue
    assert pv > 1e-3 if residual else pv < 1e-6


def test_warp64_checker_agrees_with_fp32_rule():
    """The float64 statement used to check the kernel: same kept set as the fp32 restatement away
    from the boundary band, same values to fp32 precision, and the hand-derived tie case."""
    g = torch.Generator().manual_seed(1)
    for top_p in (1.0, 0.9, 0.3):
        lg = (torch.randn(6, 3000, generator=g) * 2).to(torch.bfloat16).float()
        for row in lg:
            p32, _ = osm.warp_probs(row, 0.8, top_p)
            p64, kept, band = osm.warp_probs64(row, 0.8, top_p)
            assert not ((p32 > 0) != kept)[~band].any()
            if not band.any():
                torch.testing.assert_close(p64[kept] / (p64[kept].sum() if top_p < 1 else 1.0),
                                           p32[kept].double(), rtol=1e-5, atol=0)
    p64, kept, band = osm.warp_probs64(torch.zeros(4), 1.0, 0.3)
    assert kept.tolist() == [True, True, False, False] and not band.any()


def test_sample_next_top64_known_answers():
    """generate_selfdistill.py:50-60: topk(64) of the logits, then warp_probs over those 64.
    100 equal logits: the candidates are columns 0..63 (equal logits rank lower column first),
    uniform at top_p 1; at top_p 0.5 the mass before rank j is j/64, kept while <= 0.5: ranks
    0..32 (33 entries); at top_p 0.25, 17."""
    x = torch.zeros(100)
    for top_p, n in ((1.0, 64), (0.5, 33), (0.25, 17)):
        p = osm.top64_probs(x, 0.7, top_p)
        assert torch.equal((p > 0).nonzero().flatten(), torch.arange(n)), top_p
        torch.testing.assert_close(p[:n], torch.full((n,), 1.0 / n, dtype=torch.float64))
    # against torch.topk and the engine's warp where no two logits tie
    g = torch.Generator().manual_seed(3)
    x = torch.randn(5000, generator=g) * 3
    val, idx = torch.topk(x, 64)
    ref = torch.zeros(5000).index_copy_(0, idx, oe.warp_probs(val, 0.7, 0.9))
    torch.testing.assert_close(osm.top64_probs(x, 0.7, 0.9).float(), ref)
    # a draw never leaves the candidates
    for s in range(50):
        tok, _ = osm.sample_next_top64(torch.zeros(100), 1.0, 0.5, osm.Stream(s, 0), 0)
        assert 0 <= tok <= 32


def test_sample_next_top64_draws_follow_the_top64_warp():
    """20000 seeded draws from one row whose 0.9-nucleus over the full row holds ~390 tokens: the
    counts fit warp(top-64(logits)) by chi-square and reject the full-row warp (which puts a third
    of its mass outside the 64 candidates)."""
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(4000, generator=g) * 3.0).to(torch.bfloat16).float()
    N = 20000
    counts = np.bincount([osm.sample_next_top64(x, 0.7, 0.9, osm.Stream(s, 5), 2)[0] for s in range(N)],
                         minlength=4000)
    p = osm.top64_probs(x, 0.7, 0.9).numpy()
    p = p / p.sum()
    support = p > 0
    assert counts[~support].sum() == 0
    assert stats.chisquare(counts[support], p[support] * N).pvalue > 0.01
    full, _, _ = osm.warp_probs64(x, 0.7, 0.9)
    full = full.numpy() / full.numpy().sum()
    bins = full * N >= 5
    obs = np.append(counts[bins], counts[~bins].sum())
    exp = np.append(full[bins] * N, full[~bins].sum() * N)
    assert stats.chisquare(obs, exp).pvalue < 1e-6
