"""Pins the oracle's decode engine (CPU, fp32) with the reference's own invariants
(tests/test_engine.py in the reference) plus small hand-derived known-answer cases for
the parts no invariant fixes (pruning order, nucleus boundary, draft-vocab selection)."""

import itertools

import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM

from oracle import engine as oe
from oracle import model as om


def tiny_hf(vocab=128, seed=0, scale=1.0):
    torch.manual_seed(seed)
    m = LlamaForCausalLM(LlamaConfig(vocab_size=vocab, hidden_size=64, intermediate_size=128,
                                     num_hidden_layers=6, num_attention_heads=4, num_key_value_heads=2)).eval()
    with torch.no_grad():
        m.lm_head.weight.mul_(scale)
    return m


TREES = {
    "chain": oe.Drafting(depth=4, branch=1),
    "tree": oe.Drafting(depth=3, branch=[3, 2, 2]),
    "pruned": oe.Drafting(depth=5, branch=[4, 3, 2, 2, 1], width=[4, 6, 6, 4, 4], max_nodes=12),
    "deep_chain": oe.Drafting(depth=8, branch=1),
}


@pytest.fixture(scope="module")
def hf():
    return tiny_hf()


@pytest.fixture(scope="module")
def base(hf):
    return om.Llama.from_hf(hf)


def make_draft(base, kind):
    if kind == "perfect":
        return om.Subnetwork(base, list(range(6)))
    specs = om.plan_bridges([0, 3, 5], 6)
    return om.Subnetwork(base, [0, 3, 5], om.random_bridges(specs, 64, seed=11, init_std=0.02))


@pytest.mark.parametrize("tree_name", list(TREES))
@pytest.mark.parametrize("kind", ["untrained", "perfect"])
def test_greedy_sd_matches_autoregressive_and_hf(hf, base, tree_name, kind):
    target, draft = om.Target(base), make_draft(base, kind)
    for prompt_seed in range(3):
        g = torch.Generator().manual_seed(prompt_seed)
        ids = torch.randint(0, 128, (5 + 4 * prompt_seed,), generator=g).tolist()
        ref = oe.autoregressive_generate(target, ids, 40, {-1}).tokens
        with torch.no_grad():
            gen = hf.generate(torch.tensor([ids]), max_new_tokens=40, do_sample=False, pad_token_id=0)
        assert ref == gen[0, len(ids):].tolist()
        res = oe.SpeculativeGenerator(target, draft, TREES[tree_name], 128).generate(ids, 40, {-1})
        assert res.tokens == ref, f"{tree_name}/{kind} diverged"
        assert sum(res.accepted_per_round) >= 39
        if kind == "perfect" and TREES[tree_name].max_nodes is None:
            assert res.mean_accepted > TREES[tree_name].depth


def test_greedy_sd_with_draft_vocab_subset(base):
    target, draft = om.Target(base), om.Subnetwork(base, list(range(6)))
    draft.set_vocab_subset(oe.top_vocab(torch.arange(128).flip(0), 40, always={127}))
    assert draft.vocab_ids.numel() == 40 and 127 in draft.vocab_ids.tolist()
    ids = torch.randint(0, 128, (7,), generator=torch.Generator().manual_seed(5)).tolist()
    ref = oe.autoregressive_generate(target, ids, 40, {-1}).tokens
    res = oe.SpeculativeGenerator(target, draft, TREES["tree"], 128).generate(ids, 40, {-1})
    assert res.tokens == ref
    assert draft(torch.tensor(ids))[0].shape[-1] == 40


def test_greedy_sd_stops_at_eos(base):
    target, draft = om.Target(base), om.Subnetwork(base, list(range(6)))
    ids = torch.randint(0, 128, (6,), generator=torch.Generator().manual_seed(0)).tolist()
    free = oe.autoregressive_generate(target, ids, 30, {-1}).tokens
    eos = {free[10]}
    ref = oe.autoregressive_generate(target, ids, 30, eos).tokens
    res = oe.SpeculativeGenerator(target, draft, TREES["chain"], 128).generate(ids, 30, eos)
    assert res.tokens == ref and res.tokens[-1] in eos


def test_tree_shape_limits(base):
    draft = make_draft(base, "untrained")
    cfg = TREES["pruned"]
    drafter = oe.TreeDrafter(draft, cfg, 128)
    cache = draft.new_cache(64)
    draft(torch.tensor([1, 2]), None, cache)
    tree = drafter.build(cache, [3], root_pos=2)
    assert len(tree) <= cfg.max_nodes
    for i in range(len(tree)):
        p = tree.parents[i]
        assert p == -1 or (p < i and tree.depths[p] == tree.depths[i] - 1)
    assert cache.get_seq_length() == 3 + oe.max_tree_cache(cfg)


def test_level_sizes_closed_form():
    """Level sizes of the tree configurations (n_d = min(n_{d-1} * branch_d, width_d))."""
    assert oe.level_sizes(oe.Drafting(depth=4, branch=[3, 2, 2, 1], width=8)) == [3, 6, 8, 8]
    assert oe.level_sizes(oe.Drafting(depth=6, branch=[4, 2, 2, 1, 1, 1])) == [4, 8, 16, 16, 16, 16]
    assert oe.level_sizes(oe.Drafting(depth=4, branch=[3, 2, 2, 1])) == [3, 6, 12, 12]
    assert oe.max_verify_nodes(oe.Drafting(depth=4, branch=[3, 2, 2, 1], max_nodes=24)) == 24
    assert oe.max_tree_cache(oe.Drafting(depth=4, branch=[3, 2, 2, 1], width=8)) == 17


def test_prune_order_known_answer():
    """(-score, depth) order with Python's stable sort: equal (score, depth) keeps index order."""
    scores = [-0.1, -0.5, -0.5, -0.2, -0.5, -0.9]
    depths = [1, 1, 2, 2, 1, 3]
    # sorted: 0(-0.1), 3(-0.2), 1(-0.5,d1), 4(-0.5,d1), 2(-0.5,d2), 5
    assert oe.prune_order(scores, depths, 3) == [0, 1, 3]
    assert oe.prune_order(scores, depths, 4) == [0, 1, 3, 4]
    assert oe.prune_order(scores, depths, 5) == [0, 1, 2, 3, 4]


def test_prune_tree_cross_depth_ties_prefer_smaller_depth():
    """A log-prob of exactly 0 gives a child its parent's score, so (score) ties across depths
    are real. Nodes: 0 (d1, 0.0), 1 (d1, -1.0), 2 (d2 under 0, 0.0), 3 (d2 under 1, -1.0).
    (-score, depth) order is 0, 2, 1, 3: max_nodes 3 keeps {0, 1, 2}, max_nodes 1 keeps {0}.
    The reversed depth order (2, 0, 3, 1) would keep {2, 0, 3} and close it to all four nodes,
    or keep {2} and close it to {0, 2}."""
    def tree():
        return oe.DraftTree(tokens=[10, 11, 12, 13], parents=[-1, -1, 0, 1], depths=[1, 1, 2, 2],
                            scores=[0.0, -1.0, 0.0, -1.0], ranks=[0, 1, 0, 0], draft_pos=[-1] * 4)
    t = oe.prune_tree(tree(), 3)
    assert t.tokens == [10, 11, 12] and t.parents == [-1, -1, 0]
    t = oe.prune_tree(tree(), 1)
    assert t.tokens == [10] and t.parents == [-1]
    t = oe.prune_tree(tree(), 2)
    assert t.tokens == [10, 12] and t.parents == [-1, 0]
    # equal (score, depth): index order decides
    t = oe.DraftTree(tokens=[1, 2, 3], parents=[-1, -1, -1], depths=[1, 1, 1], scores=[-0.5, -0.5, -0.5],
                     ranks=[0, 1, 2], draft_pos=[-1] * 3)
    assert oe.prune_tree(t, 2).tokens == [1, 2]


def test_greedy_topk_ties_lower_column_first():
    logits = torch.tensor([[1.0, 3.0, 3.0, 2.0, 3.0]])
    lp, idx = oe.greedy_topk(logits, 4)
    assert idx[0].tolist() == [1, 2, 4, 3]
    lse = torch.logsumexp(logits[0], 0)
    torch.testing.assert_close(lp[0], (logits[0, [1, 2, 4, 3]] - lse))


def test_warp_probs_nucleus_boundary_known_answer():
    """p = [0.5, 0.3, 0.15, 0.05]. An entry is dropped when the mass strictly before it exceeds
    top_p: 0.75 keeps {0.5, 0.3} (a cumulative-mass rule would keep only 0.5); 0.85 keeps three;
    0.45 keeps one."""
    logits = torch.tensor([0.5, 0.3, 0.15, 0.05]).log()
    p = oe.warp_probs(logits, 1.0, 0.75)
    torch.testing.assert_close(p, torch.tensor([0.625, 0.375, 0.0, 0.0]))
    p = oe.warp_probs(logits, 1.0, 0.85)
    torch.testing.assert_close(p, torch.tensor([0.5, 0.3, 0.15, 0.0]) / 0.95)
    p = oe.warp_probs(logits, 1.0, 0.45)
    torch.testing.assert_close(p, torch.tensor([1.0, 0.0, 0.0, 0.0]))
    p = oe.warp_probs(logits * 2, 2.0, 1.0)
    torch.testing.assert_close(p, torch.tensor([0.5, 0.3, 0.15, 0.05]))


@pytest.mark.parametrize("V", [8, 128256])
def test_warp_probs_exact_equality_at_the_cut(V):
    """Masses that are exact in fp32: four tied leaders at logit 0 (p = 0.25 each), every other
    logit -1000 (its probability underflows to 0). The mass before the leaders is 0, .25, .5, .75;
    an entry is dropped only when that mass is strictly greater than top_p, so top_p 0.5 keeps
    three (a >= rule would keep two) and top_p 0.25 keeps two."""
    x = torch.full((V,), -1000.0)
    x[[1, 3, 5, 7]] = 0.0
    for T in (1.0, 0.7):
        for top_p, n in ((0.5, 3), (0.25, 2), (0.75, 4), (0.0, 1)):
            p = oe.warp_probs(x, T, top_p)
            assert int((p > 0).sum()) == n, (T, top_p)
            torch.testing.assert_close(p[p > 0], torch.full((n,), 1.0 / n))


def test_top_vocab_known_answer():
    counts = torch.tensor([5, 9, 9, 1, 7, 0])
    assert oe.top_vocab(counts, 3).tolist() == [1, 2, 4]
    assert oe.top_vocab(counts, 3, always={5}).tolist() == [1, 2, 5]
    assert oe.top_vocab(counts, 2, always={3, 99}).tolist() == [1, 3]


def test_greedy_verify_walk_known_answer():
    """root -> {0:'7', 1:'4'}; 0 -> {2:'5'}. Target argmax rows: root 7, node0 5, node2 9."""
    t = oe.DraftTree(tokens=[7, 4, 5], parents=[-1, -1, 0], depths=[1, 1, 2], scores=[0, 0, 0],
                     ranks=[0, 1, 0], draft_pos=[-1] * 3)
    logits = torch.full((4, 10), -1.0)
    logits[0, 7] = logits[1, 5] = logits[3, 9] = 1.0
    logits[2, 2] = 1.0
    assert oe.greedy_verify(t, logits) == ([0, 2], 9)
    logits[0, 7], logits[0, 4] = -1.0, 1.0
    assert oe.greedy_verify(t, logits) == ([1], 2)


@pytest.mark.parametrize("tree_cfg,subset", [
    (oe.Drafting(depth=2, branch=[2, 2], temperature=1.0), None),
    (oe.Drafting(depth=2, branch=1, temperature=0.8, top_p=0.9), None),
    (oe.Drafting(depth=2, branch=[2, 2], temperature=1.0), [0, 2, 3, 5, 6]),
])
def test_sampling_sd_matches_target_distribution(tree_cfg, subset):
    """Tokens 2 and 3 come from one speculative round; their empirical joint must match the
    target's exact joint by brute force (reference tests/test_engine.py:173-207)."""
    V = 8
    hfm = tiny_hf(vocab=V, seed=1, scale=8.0)
    base = om.Llama.from_hf(hfm)
    draft = om.Subnetwork(base, [0, 5], om.random_bridges(om.plan_bridges([0, 5], 6), 64, seed=7, init_std=0.05))
    if subset is not None:
        draft.set_vocab_subset(torch.tensor(subset))
    target = om.Target(base)
    prompt = [1, 5, 2]
    T, P = tree_cfg.temperature, tree_cfg.top_p
    with torch.no_grad():
        p1 = oe.warp_probs(target(torch.tensor(prompt))[0][-1], T, P)
        exact = torch.zeros(V, V, V)
        for a, b in itertools.product(range(V), range(V)):
            lg = target(torch.tensor(prompt + [a, b]))[0]
            exact[a, b] = p1[a] * oe.warp_probs(lg[-2], T, P)[b] * oe.warp_probs(lg[-1], T, P)
    exact23 = exact.sum(0)
    sd = oe.SpeculativeGenerator(target, draft, tree_cfg, V)
    N = 3000
    counts = torch.zeros(V, V)
    for s in range(N):
        toks = sd.generate(prompt, 3, set(), seed=s).tokens
        counts[toks[1], toks[2]] += 1
    tv = 0.5 * (counts / N - exact23).abs().sum().item()
    assert tv < 0.06, f"TV distance {tv:.3f}"
