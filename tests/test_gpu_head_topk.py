"""The vocabulary head fused with its top-k chunk pass (ssd_gemm_topk_bf16: the draft head of
ssd/models/subnetwork_draft.py:345-349 and the proposal top-k of ssd/engine/tree_drafter.py:129-133 in
one launch) against the two-launch path (head logits, then ssd_row_topk_bf16) on the same logits and
against the oracle's log_softmax top-k.

Tolerances: keys are exact (tokens, raw values, the order of equal values by lower column); the
log-softmax values and logsumexp differ from the chunk pass only in the order in which the sums of
exp are taken (slab by slab instead of 4096-column chunks): atol 2e-5 / rtol 1e-5, the oracle
check's tolerance. The logits the fused launch can also store are bit-identical to ssd_gemm_bf16's
for N >= 65536 (the same kernel and summation order) and within one bf16 step otherwise.
"""

import pytest
import torch

from oracle import kernels as ok

pytestmark = pytest.mark.gpu
DEV = "cuda"


def bf(t):
    return t.to(torch.bfloat16)


def rand(*shape, std=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * std


def _head(seed, m, n, kd, norm, tie_cols=()):
    """x [m, kd], packed head [n, kd] (folded RMSNorm weight when norm), with the rows of tie_cols all
    equal to one vector aligned with x's first row (exactly tied logits at the top of row 0)."""
    from ssd import ops

    x = bf(rand(m, kd, seed=seed))
    w = rand(n, kd, std=0.05, seed=seed + 1)
    if tie_cols:
        v = torch.sign(x[0].float()) * 0.25
        for c in tie_cols:
            w[c] = v
    w = bf(w)
    if norm:
        scale = bf(rand(kd, seed=seed + 2).abs() + 0.5)
        wp = ops.pack_weight(w.to(DEV), col_scale=scale.to(DEV))
    else:
        wp = ops.pack_weight(w.to(DEV))
    return x.to(DEV), wp, (1e-5 if norm else 0.0)


CASES = [
    # seed, rows, N, K, k, folded norm, tied columns
    (0, 1, 128256, 512, 3, False, (7, 600, 70000, 128255)),   # 251 slabs of 4 groups
    (1, 12, 128256, 256, 4, True, (3, 513, 514)),              # draft-level rows, norm folded
    (2, 25, 70001, 256, 1, False, (70000, 9)),                 # ragged N, argmax rows
    (3, 16, 32768, 512, 4, False, (0, 128, 32767)),            # one group per slab (256 slabs)
    (4, 40, 1000, 128, 3, True, (999, 0)),                     # small head, three column tiles
    (5, 70, 65560, 128, 2, False, (65559, 1)),                 # rows beyond 64: two launches
]


@pytest.mark.parametrize("seed,m,n,kd,k,norm,ties", CASES)
def test_gemm_topk_records_merge_like_the_chunk_pass(seed, m, n, kd, k, norm, ties):
    from ssd import ops

    x, wp, eps = _head(seed, m, n, kd, norm, ties)
    S = ops.gemm_topk_parts(n)
    assert S <= 256 and S * k <= 1024
    ld = (n + 7) // 8 * 8  # 16-byte rows for the chunk pass
    y = torch.zeros(m, ld, dtype=torch.bfloat16, device=DEV)[:, :n]
    ops.gemm(x, m, wp, n, kd, y, norm_eps=eps)
    for mode in (1, 0):
        parts = torch.zeros(ops.gemm_topk_bytes(m, n), dtype=torch.uint8, device=DEV)
        yt = torch.zeros(m, ld, dtype=torch.bfloat16, device=DEV)[:, :n]
        assert ops.gemm_topk(x, m, wp, n, kd, k, mode, parts, norm_eps=eps, out=yt) == S
        if n >= 65536:
            assert torch.equal(yt, y)  # same kernel, same summation order
        else:
            diff = (yt.float() - y.float()).abs()
            assert (diff <= 2e-2 * y.float().abs() + 1e-3).all()
        # the records do not depend on whether the logits are stored (the records are packed for k:
        # m * S records of 8 + 8 k bytes, every byte written; the rest of the buffer is untouched)
        used = m * S * (8 + 8 * k)
        bare = torch.full_like(parts, 7)
        ops.gemm_topk(x, m, wp, n, kd, k, mode, bare, norm_eps=eps)
        assert torch.equal(bare[:used], parts[:used])
        assert (bare[used:] == 7).all()
        # merged records == the chunk pass over the logits the fused launch computed
        tok = torch.zeros(m * k, dtype=torch.int32, device=DEV)
        val = torch.zeros(m * k, dtype=torch.float32, device=DEV)
        lse = torch.zeros(m, dtype=torch.float32, device=DEV)
        ops.row_topk_merge(parts, m, S, k, mode, None, tok, val, lse if mode == 1 else None)
        rt = torch.zeros(m * k, dtype=torch.int32, device=DEV)
        rv = torch.zeros(m * k, dtype=torch.float32, device=DEV)
        rl = torch.zeros(m, dtype=torch.float32, device=DEV)
        ops.row_topk(yt, m, n, k, mode, None, rt, rv, rl if mode == 1 else None)
        assert tok.tolist() == rt.tolist()
        if mode == 0:
            assert torch.equal(val, rv)
            ref = torch.sort(yt.float().cpu(), dim=1, descending=True, stable=True)
            assert tok.view(m, k).cpu().tolist() == ref.indices[:, :k].tolist()
        else:
            torch.testing.assert_close(val, rv, atol=2e-5, rtol=1e-5)
            torch.testing.assert_close(lse, rl, atol=2e-5, rtol=1e-5)
            ov, oi, olse = ok.log_softmax_topk(yt.cpu(), k)
            assert tok.view(m, k).cpu().tolist() == oi.tolist()
            torch.testing.assert_close(val.view(m, k).cpu(), ov, atol=2e-5, rtol=1e-5)
            torch.testing.assert_close(lse.cpu(), olse, atol=2e-5, rtol=1e-5)
        if ties:
            # row 0's best logits are the tied columns: they come out in column order
            want = sorted(ties)[:k]
            assert tok.view(m, k)[0, :len(want)].tolist() == want
        # a row's records are the same computed alone (batch invariance of the head)
        row_bytes = S * (8 + 8 * k)  # records are packed for the call's k (max, sum of exp, k keys)
        for r in sorted({0, m - 1}):
            one = torch.zeros(ops.gemm_topk_bytes(1, n), dtype=torch.uint8, device=DEV)
            ops.gemm_topk(x[r:r + 1].contiguous(), 1, wp, n, kd, k, mode, one, norm_eps=eps)
            assert torch.equal(one[:row_bytes], parts[r * row_bytes:(r + 1) * row_bytes]), f"row {r}"


def test_gemm_topk_argument_errors():
    from ssd import ops

    x, wp, _ = _head(9, 2, 4096, 64, False)
    parts = torch.zeros(ops.gemm_topk_bytes(2, 4096), dtype=torch.uint8, device=DEV)
    with pytest.raises(ValueError):
        ops.gemm_topk(x, 2, wp, 4096, 64, 17, 1, parts)  # k above 16
    with pytest.raises(ValueError):
        ops.gemm_topk(x, 2, wp, 4096, 64, 2, 2, parts)  # mode
    with pytest.raises(ValueError):
        ops.gemm_topk(x, 2, wp, 4096, 64, 2, 1, parts[:100])  # records do not fit
    tok = torch.zeros(2 * 16, dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError):  # 256 records x 16 keys exceed the merge's 1024 candidates
        ops.row_topk_merge(torch.zeros(2 * 256 * ops.TOPK_PART_BYTES, dtype=torch.uint8, device=DEV), 2, 256, 16, 1, None, tok)


@pytest.mark.parametrize("seed,V,mapped", [(0, 128256, False), (1, 32768, True)])
def test_tree_level_topk_from_fused_head_records(seed, V, mapped):
    """The level launch merging the fused head's records builds the same tree and draft rows as
    ssd_row_topk_bf16 over the stored logits followed by ssd_tree_level (tokens, parents, depths,
    ranks and rows exact; scores to the log-softmax tolerance). Logits are a coarse grid (one-hot
    rows of X pick columns of a quarter-step W), so ties within and across slabs are everywhere."""
    from ssd import _lib, ops
    from ssd.models.subnetwork_draft import Rows
    from test_gpu_kernels import _device_tree

    g = torch.Generator().manual_seed(seed)
    kd = 64
    w = torch.randint(-40, 8, (V, kd), generator=g).float() * 0.25
    w[[5, 700, V - 1]] = 2.0  # top value only in a few columns, across slabs
    wp = ops.pack_weight(bf(w).to(DEV))
    vocab_ids = torch.randperm(128256, generator=g)[:V].to(torch.int32).to(DEV) if mapped else None
    depth, branch, width = 4, [3, 2, 2, 1], [None, None, 8, 6]
    committed, tree_start = 40, 41
    trees = [_device_tree(), _device_tree()]
    rows = [Rows(64, DEV), Rows(64, DEV)]
    ct = torch.zeros(1024, dtype=torch.int32, device=DEV)
    cl = torch.zeros(1024, dtype=torch.float32, device=DEV)
    F, past = 1, tree_start
    S = ops.gemm_topk_parts(V)
    for d in range(depth):
        k = branch[d]
        x = torch.zeros(F, kd)
        x[torch.arange(F), torch.randint(0, kd, (F,), generator=g)] = 1.0
        x = bf(x).to(DEV)
        feed = d < depth - 1
        m = min(F * k, width[d] or F * k)
        logits = torch.zeros(F, V, dtype=torch.bfloat16, device=DEV)
        parts = torch.zeros(ops.gemm_topk_bytes(F, V), dtype=torch.uint8, device=DEV)
        ops.gemm_topk(x, F, wp, V, kd, k, 1, parts, out=logits)
        ops.row_topk(logits, F, V, k, 1, vocab_ids, ct, cl)
        _lib.call("ssd_tree_level", trees[0].struct, d, ct.data_ptr(), cl.data_ptr(), F, k, width[d] or 0, int(feed),
                  committed, tree_start, past, rows[0].struct, m if feed else 0, None, ops.stream())
        _lib.call("ssd_tree_level_topk", trees[1].struct, d, parts.data_ptr(), parts.numel(), V, S,
                  None if vocab_ids is None else vocab_ids.data_ptr(), F, k, width[d] or 0, int(feed), committed,
                  tree_start, past, rows[1].struct, m if feed else 0, None, ops.stream())
        torch.cuda.synchronize()
        if feed:
            for name in ("ids", "pos", "slot", "prefix", "depth"):
                assert getattr(rows[0], name)[:m].tolist() == getattr(rows[1], name)[:m].tolist(), (d, name)
            assert rows[0].anc[:m, :d + 1].tolist() == rows[1].anc[:m, :d + 1].tolist()
            past += m
        F = m
    n = int(trees[0].meta[0])
    assert n == int(trees[1].meta[0]) and n > 0
    for name in ("tokens", "parents", "depths", "ranks", "draft_pos"):
        assert getattr(trees[0], name)[:n].tolist() == getattr(trees[1], name)[:n].tolist(), name
    torch.testing.assert_close(trees[1].scores[:n], trees[0].scores[:n], atol=1e-4, rtol=1e-5)
    assert trees[0].meta.tolist() == trees[1].meta.tolist()
