"""Parity of the sampling kernels (ssd_warp_probs_bf16, ssd_gumbel_topk, ssd_sample_rows,
ssd_accept_sample) and of the sampled engine.

* Draw for draw against oracle/sampling.py, which restates the reference algorithms
  (tree_drafter.py:34-45, :124-145, verify.py:60-95) with the kernels' Philox streams. A result
  may differ only where the oracle flags the decision as fragile (a margin below 1e-4, where
  fp32 rounding on either side can flip it); every other case must match exactly (tokens,
  accepted paths) or to fp32 precision (probabilities: rel 1e-5).
* Distributionally: the first committed token of a speculative round is distributed as the
  warped target (chi-square at the 8B vocabulary, target logits N(0, 4^2), draft = target +
  N(0, 1)); the sampled engine reproduces the brute-force V=8 joint of the reference's own test
  (tests/test_engine.py:173-207, TV < 0.06).
"""

import itertools

import numpy as np
import pytest
import torch
from scipy import stats

from oracle import sampling as osm

pytestmark = pytest.mark.gpu
DEV = "cuda"


def ops():
    from ssd import ops as o
    return o


def bf16_logits(rows, V, scale, seed, levels=None):
    g = torch.Generator().manual_seed(seed)
    if levels is not None:
        x = torch.randint(0, levels, (rows, V), generator=g).float() * scale
    else:
        x = torch.randn(rows, V, generator=g) * scale
    ld = (V + 7) // 8 * 8
    buf = torch.zeros(rows, ld, dtype=torch.bfloat16)
    buf[:, :V] = x.to(torch.bfloat16)
    return buf


def run_warp(lg, V, T, top_p, vocab=None, Vfull=None):
    o = ops()
    rows = lg.shape[0]
    Vo = Vfull or V
    out = torch.full((rows, (Vo + 3) // 4 * 4), float("nan"), dtype=torch.float32, device=DEV)
    dl = lg.to(DEV)
    if vocab is not None:
        inv = torch.full((Vo,), -1, dtype=torch.int32)
        inv[vocab] = torch.arange(len(vocab), dtype=torch.int32)
        o.warp_probs(dl, rows, V, T, top_p, out, V=Vo, vocab_ids=vocab.to(torch.int32).to(DEV), vocab_inv=inv.to(DEV))
    else:
        o.warp_probs(dl, rows, V, T, top_p, out)
    return out[:, :Vo].cpu()


def check_warp_rows(got, lg, V, T, top_p, vocab=None, Vfull=None):
    """Kept set equal to the float64 rule except inside the boundary band; values equal to p
    renormalised over the kernel's own kept set (rel 1e-5); no renormalisation at top_p = 1."""
    for r in range(lg.shape[0]):
        p, kept, band = osm.warp_probs64(lg[r, :V].float(), T, top_p)
        g = got[r] if vocab is None else got[r, vocab]
        gk = g > 0
        diff = gk != kept
        assert not (diff & ~band).any(), f"row {r}: {int((diff & ~band).sum())} entries disagree outside the band"
        ref = p if top_p >= 1.0 else torch.where(gk, p / p[gk].sum(), torch.zeros_like(p))
        torch.testing.assert_close(g.double(), ref, rtol=1e-5, atol=1e-12)


@pytest.mark.parametrize("V", [128256, 1000])
@pytest.mark.parametrize("T", [0.7, 1.0])
@pytest.mark.parametrize("top_p", [1.0, 0.9, 0.5, 1e-4])
def test_warp_matches_oracle(V, T, top_p):
    lg = bf16_logits(4, V, 3.0, seed=V + int(T * 10))
    got = run_warp(lg, V, T, top_p)
    assert not torch.isnan(got).any()
    check_warp_rows(got, lg, V, T, top_p)


def test_warp_ties_at_the_cut_keep_lower_columns():
    """bf16 logits tie constantly; the nucleus boundary then splits a group of equal
    probabilities. Uniform row: top_p .5004 keeps exactly columns 0..500; three levels:
    the cut lands inside a tie group."""
    V = 1000
    lg = torch.zeros(1, 1000, dtype=torch.bfloat16)
    got = run_warp(lg, V, 1.0, 0.5004)
    assert torch.equal((got[0] > 0).nonzero().flatten(), torch.arange(501))
    lg = bf16_logits(6, 4000, 0.75, seed=3, levels=3)
    got = run_warp(lg, 4000, 1.0, 0.6)
    check_warp_rows(got, lg, 4000, 1.0, 0.6)


@pytest.mark.parametrize("T", [1.0, 0.7])
def test_warp_exact_equality_at_the_cut(T):
    """Four tied leaders in four different 4096-column chunks of a 128256 row (bf16 logit 0,
    p = 0.25 exactly; every other logit -1000, p = 0). The reference keeps an entry while the mass
    before it is <= top_p (tree_drafter.py:41): top_p 0.5 keeps three, 0.25 two, 0.75 four, each
    tie at the cut by lowest column; probabilities 1/n exactly. No boundary band."""
    V = 128256
    leaders = [5, 4100, 70000, 128255]
    ld = (V + 7) // 8 * 8
    lg = torch.full((3, ld), -1000.0).to(torch.bfloat16)
    lg[:, leaders] = 0.0
    got = torch.stack([run_warp(lg[i:i + 1], V, T, tp)[0] for i, tp in enumerate((0.5, 0.25, 0.75))])
    for r, n in enumerate((3, 2, 4)):
        assert (got[r] > 0).nonzero().flatten().tolist() == leaders[:n], (T, r)
        assert torch.equal(got[r, leaders[:n]], torch.full((n,), 1.0 / n))


def test_warp_tie_ranks_cross_chunks():
    """A tie group spread over every 4096-column chunk of a 128256 row: the kept ties are the
    lowest columns across chunks (per-chunk tie counts give the prefix)."""
    V = 128256
    g = torch.Generator().manual_seed(6)
    x = torch.full((1, V), -3.0)
    x[0, torch.randperm(V, generator=g)[:20]] = 2.0  # 20 leaders
    ld = (V + 7) // 8 * 8
    lg = torch.zeros(1, ld, dtype=torch.bfloat16)
    lg[:, :V] = x.to(torch.bfloat16)
    # leaders hold 20 e^5 / (20 e^5 + 128236) ~ 0.0225 of the mass; top_p 0.5 cuts deep into the
    # -3 tie group, which spans all chunks
    got = run_warp(lg, V, 1.0, 0.5)
    check_warp_rows(got, lg, V, 1.0, 0.5)
    kept_low = (got[0] > 0) & (x[0] < 0)
    idx = kept_low.nonzero().flatten()
    assert len(idx) > 4096 and torch.equal(idx, (x[0] < 0).nonzero().flatten()[:len(idx)])


@pytest.mark.parametrize("top_p", [1.0, 0.9])
def test_warp_vocab_subset_scatters_to_full_vocabulary(top_p):
    V, n = 5000, 1200
    vocab = torch.randperm(V, generator=torch.Generator().manual_seed(4))[:n].sort().values
    lg = bf16_logits(3, n, 2.0, seed=5)
    got = run_warp(lg, n, 0.8, top_p, vocab=vocab, Vfull=V)
    outside = torch.ones(V, dtype=torch.bool)
    outside[vocab] = False
    assert (got[:, outside] == 0).all()
    check_warp_rows(got, lg, n, 0.8, top_p, vocab=vocab, Vfull=V)


def probs_rows(rows, V, seed, zero_frac=0.0, scale=2.0):
    rng = np.random.default_rng(seed)
    w = torch.from_numpy(rng.standard_normal((rows, V)).astype(np.float32)) * scale
    p = torch.softmax(w, -1)
    if zero_frac:
        p[torch.from_numpy(rng.random((rows, V)) < zero_frac)] = 0
        p = p / p.sum(-1, keepdim=True)
    return p


@pytest.mark.parametrize("V,k,zero", [(128256, 3, 0.0), (128256, 16, 0.0), (500, 8, 0.5), (64, 5, 0.97)])
def test_gumbel_topk_matches_oracle(V, k, zero):
    o = ops()
    rows = 6
    q = probs_rows(rows, V, seed=V + k, zero_frac=zero)
    ld = (V + 3) // 4 * 4
    qd = torch.zeros(rows, ld, device=DEV)
    qd[:, :V] = q.to(DEV)
    tok = torch.zeros(rows * k, dtype=torch.int32, device=DEV)
    lp = torch.zeros(rows * k, dtype=torch.float32, device=DEV)
    seed, ctr = 1234567 + V, 42
    o.gumbel_topk(qd, rows, V, k, seed, ctr, tok, lp)
    tok, lp = tok.view(rows, k).cpu(), lp.view(rows, k).cpu()
    s = osm.Stream(seed, ctr)
    checked = 0
    for r in range(rows):
        want, wlp, fragile = osm.gumbel_topk(q[r], k, s, r, 0)
        got = [t for t in tok[r].tolist() if t >= 0]
        assert len(got) == len(want) == min(k, int((q[r] > 0).sum()))
        assert all(t == -1 for t in tok[r, len(want):].tolist())
        if fragile:
            continue
        assert got == want, f"row {r}"
        torch.testing.assert_close(lp[r, :len(want)], torch.tensor(wlp, dtype=torch.float32), rtol=1e-6, atol=1e-6)
        checked += 1
    assert checked >= rows - 1


def test_tree_meta_rows_addressing():
    """With tree meta, the frontier of level d (size from meta) reads logits rows 0..F-1 and
    writes q rows 1 + start(level d-1) + f; rows past F are untouched; Gumbel top-k reads the
    same rows."""
    o = ops()
    V, k = 3000, 2
    meta = torch.zeros(65, dtype=torch.int32)
    meta[1 + 1], meta[33 + 1] = 4, 3  # level 1: nodes 4..6
    lg = bf16_logits(5, V, 2.0, seed=8)
    Q = torch.full((12, V), -7.0, device=DEV)
    o.warp_probs(lg.to(DEV), 5, V, 1.0, 1.0, Q, tree_meta=meta.to(DEV), level=2)
    Qc = Q.cpu()
    for f in range(3):
        ref, _, _ = osm.warp_probs64(lg[f, :V].float(), 1.0, 1.0)
        torch.testing.assert_close(Qc[5 + f].double(), ref, rtol=1e-5, atol=1e-12)
    assert (Qc[:5] == -7).all() and (Qc[8:] == -7).all()
    tok = torch.full((5 * k,), -5, dtype=torch.int32, device=DEV)
    lp = torch.zeros(5 * k, device=DEV)
    o.gumbel_topk(Q, 5, V, k, 9, 3, tok, lp, tree_meta=meta.to(DEV), level=2)
    tok = tok.view(5, k).cpu()
    s = osm.Stream(9, 3)
    for f in range(3):
        want, _, fragile = osm.gumbel_topk(Qc[5 + f], k, s, f, 2)
        if not fragile:
            assert tok[f].tolist() == want
    assert (tok[3:] == -5).all()


@pytest.mark.parametrize("V", [128256, 37])
def test_sample_rows_matches_oracle(V):
    o = ops()
    rows = 8
    p = probs_rows(rows, V, seed=V, zero_frac=0.3)
    ld = (V + 3) // 4 * 4
    pd = torch.zeros(rows, ld, device=DEV)
    pd[:, :V] = p.to(DEV)
    out = torch.zeros(rows, dtype=torch.int32, device=DEV)
    o.sample_rows(pd, rows, V, 77, 5, out)
    s = osm.Stream(77, 5)
    for r in range(rows):
        want, fragile = osm.categorical(p[r], s, r)
        if not fragile:
            assert int(out[r]) == want


def device_tree(tokens, parents, ranks):
    from ssd.engine.tree_drafter import DeviceTree

    n = len(tokens)
    t = DeviceTree(DEV)
    i32 = dict(dtype=torch.int32, device=DEV)
    if n:
        t.vtokens[:n] = torch.tensor(tokens, **i32)
        t.vparents[:n] = torch.tensor(parents, **i32)
        t.vranks[:n] = torch.tensor(ranks, **i32)
        t.vorig[:n] = torch.arange(n, **i32)
    t.vmeta[0] = n
    return t


def accept_on_gpu(tree, P, child_q, V, seed, ctr, rows_pad=0, max_kids=16):
    """ssd_accept_sample with Q rows at 1 + node (row 0 the root)."""
    from ssd import ops as o

    ld = (V + 3) // 4 * 4
    m = P.shape[0] + rows_pad
    Pd = torch.zeros(m, ld, device=DEV)
    Pd[:P.shape[0], :V] = P.to(DEV)
    Qd = torch.zeros(m, ld, device=DEV)
    for p, q in child_q.items():
        Qd[0 if p == -1 else 1 + p, :V] = q.to(DEV)
    i32 = dict(dtype=torch.int32, device=DEV)
    result, keep = torch.zeros(40, **i32), torch.zeros(40, **i32)
    nk, root = torch.zeros(1, **i32), torch.zeros(1, **i32)
    o.accept_sample(tree.struct, Pd, Qd, V, m, max_kids, seed, ctr, 0, result, keep, nk, root)
    r = result.tolist()
    n_new = r[0]
    accepted = [x - 1 for x in keep[1:n_new].tolist()]
    assert int(nk) == n_new and int(root) == r[n_new] and int(keep[0]) == 0
    assert r[1:n_new] == [int(tree.vtokens[a]) for a in accepted]
    return accepted, r[n_new]


def random_tree(rng, V, branch, zero):
    tokens, parents, ranks, child_q = [], [], [], {}
    frontier = [-1]
    stream = osm.Stream(int(rng.integers(1 << 62)), int(rng.integers(1 << 20)))
    for d, k in enumerate(branch):
        nxt = []
        for f, par in enumerate(frontier):
            q = probs_rows(1, V, int(rng.integers(1 << 30)), zero_frac=zero, scale=2.0)[0]
            child_q[par] = q
            toks, _, _ = osm.gumbel_topk(q, k, stream, f, d)
            for r, t in enumerate(toks):
                tokens.append(t)
                parents.append(par)
                ranks.append(r)
                nxt.append(len(tokens) - 1)
        frontier = nxt
    P = probs_rows(len(tokens) + 1, V, int(rng.integers(1 << 30)), zero_frac=zero, scale=1.0)
    return tokens, parents, ranks, P, child_q


@pytest.mark.parametrize("V,branch,zero", [(64, [3, 2, 2], 0.0), (9, [4, 2], 0.4), (5000, [3, 2, 2, 1], 0.0)])
def test_accept_sample_matches_oracle(V, branch, zero):
    rng = np.random.default_rng(V)
    checked = accepted_any = 0
    for trial in range(60):
        tokens, parents, ranks, P, child_q = random_tree(rng, V, branch, zero)
        t = device_tree(tokens, parents, ranks)
        seed, ctr = int(rng.integers(1 << 62)), trial
        got = accept_on_gpu(t, P, child_q, V, seed, ctr, rows_pad=3)
        want_acc, want_bonus, fragile = osm.sample_verify(tokens, parents, ranks, P, child_q, osm.Stream(seed, ctr))
        if fragile:
            continue
        assert got == (want_acc, want_bonus), f"trial {trial}"
        checked += 1
        accepted_any += bool(want_acc)
    assert checked >= 50 and accepted_any >= 5


def test_accept_sample_leaf_root_and_empty_tree():
    """No children: the bonus is a draw from p_root (the state pass 0)."""
    V = 100
    P = probs_rows(1, V, 3)
    t = device_tree([], [], [])
    acc, bonus = accept_on_gpu(t, P, {}, V, 5, 6)
    want, frag = osm.categorical(P[0], osm.Stream(5, 6), 0, tag=osm.TAG_BONUS, c1=0)
    assert acc == [] and (frag or bonus == want)


@pytest.mark.parametrize("top_p", [1.0, 0.9])
def test_first_committed_token_is_target_distributed(top_p):
    """The isolated-acceptance check at the 8B vocabulary: target logits N(0, 4^2), draft =
    target + N(0, 1), T = 0.7; the root proposes 4 children by ssd_gumbel_topk, then
    ssd_accept_sample. Over 4000 rounds (fresh counters) the first committed token must follow
    warp(target) (chi-square, bins with expected count >= 5, the rest pooled)."""
    from ssd import ops as o

    V, T, k, N = 128256, 0.7, 4, 4000
    g = torch.Generator().manual_seed(11)
    tl = torch.randn(V, generator=g) * 4
    dl = tl + torch.randn(V, generator=g)
    ld = (V + 7) // 8 * 8
    lgb = torch.zeros(k + 1, ld, dtype=torch.bfloat16)
    lgb[0, :V] = tl.to(torch.bfloat16)
    for r in range(1, k + 1):
        lgb[r, :V] = (torch.randn(V, generator=g) * 4).to(torch.bfloat16)
    dgb = torch.zeros(1, ld, dtype=torch.bfloat16)
    dgb[0, :V] = dl.to(torch.bfloat16)
    lgb, dgb = lgb.to(DEV), dgb.to(DEV)
    ldp = (V + 3) // 4 * 4
    P = torch.zeros(k + 1, ldp, device=DEV)
    Q = torch.zeros(k + 1, ldp, device=DEV)
    o.warp_probs(lgb, k + 1, V, T, top_p, P)
    o.warp_probs(dgb, 1, V, T, top_p, Q)
    t = device_tree([0] * k, [-1] * k, list(range(k)))
    tok = torch.zeros(k, dtype=torch.int32, device=DEV)
    lp = torch.zeros(k, device=DEV)
    i32 = dict(dtype=torch.int32, device=DEV)
    result, keep = torch.zeros(8, **i32), torch.zeros(8, **i32)
    nk, root = torch.zeros(1, **i32), torch.zeros(1, **i32)
    first = torch.zeros(N, dtype=torch.int32, device=DEV)
    for n in range(N):
        o.gumbel_topk(Q, 1, V, k, 2024, n, tok, lp)
        t.vtokens[:k].copy_(tok)
        o.accept_sample(t.struct, P, Q, V, k + 1, k, 2024, n, 0, result, keep, nk, root)
        first[n:n + 1].copy_(result[1:2])
    first = first.cpu().numpy()
    p = P[0, :V].double().cpu().numpy()
    exp = p / p.sum() * N
    counts = np.bincount(first, minlength=V).astype(np.float64)
    keep_b = exp >= 5
    obs = np.append(counts[keep_b], counts[~keep_b].sum())
    ex = np.append(exp[keep_b], exp[~keep_b].sum())
    if ex[-1] < 5:
        obs[-2] += obs[-1]
        ex[-2] += ex[-1]
        obs, ex = obs[:-1], ex[:-1]
    assert len(ex) >= 4
    assert stats.chisquare(obs, ex).pvalue > 1e-3


# -------------------------------------------------------------------------- engine
def tiny_hf(vocab, seed, scale):
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(seed)
    m = LlamaForCausalLM(LlamaConfig(vocab_size=vocab, hidden_size=128, intermediate_size=256, num_hidden_layers=6,
                                     num_attention_heads=4, num_key_value_heads=2, rope_theta=500000.0,
                                     max_position_embeddings=256)).eval()
    with torch.no_grad():
        m.lm_head.weight.mul_(scale)
    return m.to(torch.bfloat16)


@pytest.mark.parametrize("tree_cfg,subset", [
    (dict(depth=2, branch=[2, 2], temperature=1.0), None),
    (dict(depth=2, branch=1, temperature=0.8, top_p=0.9), None),
    (dict(depth=2, branch=[2, 2], temperature=1.0), [0, 2, 3, 5, 6]),
])
def test_sampled_engine_matches_target_joint(tree_cfg, subset):
    """Tokens 2 and 3 come from one speculative round (token 1 from prefill); their empirical
    joint over 3000 seeds must match the target's exact joint (brute force over V=8, computed
    from this engine's own target logits)."""
    import ssd.engine.speculative as sp
    from ssd.config import BridgeConfig, DraftingConfig
    from ssd.engine.tree_drafter import warp_probs
    from ssd.models.subnetwork_draft import SubnetworkDraftModel

    V = 8
    hf = tiny_hf(V, 1, 8.0)
    torch.manual_seed(3)
    draft = SubnetworkDraftModel(hf, [0, 5], BridgeConfig(init_std=0.05))
    if subset is not None:
        draft.set_vocab_subset(torch.tensor(subset))
    target = sp.TargetRunner(hf)
    cfg = DraftingConfig(**tree_cfg)
    T, P = cfg.temperature, cfg.top_p
    prompt = torch.tensor([[1, 5, 2]])
    with torch.no_grad():
        p1 = warp_probs(target(prompt).logits[0, -1], T, P).cpu()
        exact = torch.zeros(V, V, V)
        for a, b in itertools.product(range(V), range(V)):
            lg = target(torch.cat([prompt, torch.tensor([[a, b]])], 1)).logits[0]
            exact[a, b] = p1[a] * warp_probs(lg[-2], T, P).cpu()[b] * warp_probs(lg[-1], T, P).cpu()
    exact23 = exact.sum(0)
    gen = sp.SpeculativeGenerator(hf, draft, cfg, target)
    N = 3000
    counts = torch.zeros(V, V)
    for s in range(N):
        toks = gen.generate(prompt, 3, set(), seed=s).tokens
        counts[toks[1], toks[2]] += 1
    tv = 0.5 * (counts / N - exact23).abs().sum().item()
    assert tv < 0.06, f"TV distance {tv:.3f}"


def test_sampled_generation_is_reproducible_and_ar_matches_warp():
    import ssd.engine.speculative as sp
    from ssd.config import BridgeConfig, DraftingConfig
    from ssd.engine.tree_drafter import warp_probs
    from ssd.models.subnetwork_draft import SubnetworkDraftModel

    V = 8
    hf = tiny_hf(V, 2, 6.0)
    torch.manual_seed(4)
    draft = SubnetworkDraftModel(hf, [0, 3, 5], BridgeConfig(init_std=0.02))
    target = sp.TargetRunner(hf)
    cfg = DraftingConfig(depth=3, branch=[3, 2, 1], temperature=0.7, top_p=0.9)
    gen = sp.SpeculativeGenerator(hf, draft, cfg, target)
    prompt = torch.tensor([[3, 1, 4, 1, 5]])
    a = gen.generate(prompt, 20, set(), seed=9).tokens
    b = gen.generate(prompt, 20, set(), seed=9).tokens
    assert a == b and len(a) == 20
    # AR sampling: first token ~ warp(logits of the prompt's last row)
    p = warp_probs(target(prompt).logits[0, -1], 0.7, 0.9).cpu().double().numpy()
    N = 1500
    counts = np.zeros(V)
    for s in range(N):
        counts[sp.autoregressive_generate(target, prompt, 1, set(), temperature=0.7, top_p=0.9, seed=s).tokens[0]] += 1
    assert counts[p == 0].sum() == 0
    keep = p * N >= 5
    assert stats.chisquare(counts[keep], p[keep] / p[keep].sum() * counts[keep].sum()).pvalue > 1e-3
