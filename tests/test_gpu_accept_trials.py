"""The acceptance rule at scale: a 24-node unpruned tree (depth 2, branch [4, 5]) over the 8B
vocabulary, target logits N(0, 4^2) per node, draft logits = target + N(0, 1), warped with
T 0.7 / top_p 0.9 (and T 1.0 / top_p 0.9), 1e6 seeded trials in one launch
(ssd_accept_sample_trials).

* Draw for draw: trial t equals the engine's own kernels run as one round with counter t --
  ssd_gumbel_topk for the root's children and for each level-0 node's children, then
  ssd_accept_sample over that tree -- so the batched kernel is the engine's acceptance.
* The speculative-sampling theorem (reference ssd/engine/verify.py:60-95; RESEARCH_LOG.md:162-165
  ran the same check): the first committed token is distributed as the warped target of the
  root. Chi-square over 1e6 trials, bins with expected count >= 5 (the rest pooled), p > 0.01;
  the same counts against the draft's distribution must be rejected (the test has power).
"""

import numpy as np
import pytest
import torch
from scipy import stats

pytestmark = pytest.mark.gpu
DEV = "cuda"
V = 128256
BRANCH = [4, 5]
NODES = 4 + 4 * 5


def warped_rows(T, top_p, seed):
    """P (target) and Q (draft) rows [25, V]: row 0 the root, row 1 + v node v."""
    from ssd import ops as o
    g = torch.Generator().manual_seed(seed)
    rows = 1 + NODES
    tl = torch.randn(rows, V, generator=g) * 4
    dl = tl + torch.randn(rows, V, generator=g)
    ld = (V + 7) // 8 * 8
    ldp = (V + 3) // 4 * 4
    out = []
    for logits in (tl, dl):
        lg = torch.zeros(rows, ld, dtype=torch.bfloat16)
        lg[:, :V] = logits.to(torch.bfloat16)
        pr = torch.zeros(rows, ldp, device=DEV)
        o.warp_probs(lg.to(DEV), rows, V, T, top_p, pr)
        out.append(pr)
    return out


def run_trials(P, Q, trials, seed, counter0=0):
    from ssd import ops as o
    toks = torch.zeros(trials * 3, dtype=torch.int32, device=DEV)
    n = torch.zeros(trials, dtype=torch.int32, device=DEV)
    o.accept_sample_trials(P, Q, 1 + NODES, BRANCH, seed, counter0, trials, toks, n)
    return toks.view(trials, 3).cpu(), n.cpu()


def engine_round(P, Q, seed, counter):
    """One round of the engine's kernels: proposals level by level, then the acceptance walk."""
    from ssd import ops as o
    from ssd.engine.tree_drafter import DeviceTree
    i32 = dict(dtype=torch.int32, device=DEV)
    t0, lp0 = torch.zeros(4, **i32), torch.zeros(4, device=DEV)
    o.gumbel_topk(Q, 1, V, 4, seed, counter, t0, lp0)
    t1, lp1 = torch.zeros(4 * 5, **i32), torch.zeros(4 * 5, device=DEV)
    o.gumbel_topk(Q[1:5], 4, V, 5, seed, counter, t1, lp1, level=1)
    tokens = t0.tolist() + t1.tolist()
    parents = [-1] * 4 + [f for f in range(4) for _ in range(5)]
    ranks = list(range(4)) + [i for _ in range(4) for i in range(5)]
    tree = DeviceTree(DEV)
    tree.vtokens[:NODES] = torch.tensor(tokens, **i32)
    tree.vparents[:NODES] = torch.tensor(parents, **i32)
    tree.vranks[:NODES] = torch.tensor(ranks, **i32)
    tree.vorig[:NODES] = torch.arange(NODES, **i32)
    tree.vmeta[0] = NODES
    result, keep = torch.zeros(40, **i32), torch.zeros(40, **i32)
    nk, root = torch.zeros(1, **i32), torch.zeros(1, **i32)
    o.accept_sample(tree.struct, P, Q, V, 1 + NODES, 5, seed, counter, 0, result, keep, nk, root)
    r = result.tolist()
    return r[1:1 + r[0]]


@pytest.mark.parametrize("T,top_p", [(0.7, 0.9), (1.0, 0.9)])
def test_trials_equal_engine_rounds_draw_for_draw(T, top_p):
    P, Q = warped_rows(T, top_p, seed=31)
    toks, n = run_trials(P, Q, 96, seed=2024)
    depths = []
    for t in range(96):
        want = engine_round(P, Q, 2024, t)
        got = toks[t, :int(n[t])].tolist()
        assert got == want, f"trial {t}: {got} != {want}"
        depths.append(len(want))
    assert set(depths) >= {1, 2, 3}  # rejections at the root, at level 1, and whole paths accepted


@pytest.mark.parametrize("T,top_p", [(0.7, 0.9), (1.0, 0.9)])
def test_first_committed_token_chi_square_1e6_trials(T, top_p):
    P, Q = warped_rows(T, top_p, seed=32)
    N = 1_000_000
    toks, n = run_trials(P, Q, N, seed=7, counter0=10_000)
    assert int(n.min()) >= 1 and int(n.max()) <= 3
    first = toks[:, 0].numpy()
    counts = np.bincount(first, minlength=V).astype(np.float64)

    def chi2_pvalue(p_row):
        p = p_row[:V].double().cpu().numpy()
        exp = p / p.sum() * N
        keep = exp >= 5
        obs = np.append(counts[keep], counts[~keep].sum())
        ex = np.append(exp[keep], exp[~keep].sum())
        if ex[-1] < 5:  # pool a tiny tail into the last kept bin
            obs[-2] += obs[-1]
            ex[-2] += ex[-1]
            obs, ex = obs[:-1], ex[:-1]
        assert len(ex) >= 4
        return stats.chisquare(obs, ex).pvalue

    assert chi2_pvalue(P[0]) > 0.01
    assert chi2_pvalue(Q[0]) < 1e-6  # the draft's own distribution is rejected at this sample size
    # the mixture of accepted drafts and residual bonuses reaches every deeper level too
    assert (n == 3).float().mean() > 0.05 and (n == 1).float().mean() > 0.01
