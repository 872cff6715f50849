"""Batched generation (reference tests/test_selfdistill.py): continuing a batch of prompts of
different lengths must equal continuing each prompt alone. Here the equality is bit for bit in bf16
(every row's arithmetic is independent of the other rows), with prompts on both sides of the
prefill threshold and of 64- and 256-key block boundaries, batches larger than one 64-row chunk,
and the real per-layer shapes of Llama-3.2-1B."""

import numpy as np
import pytest
import torch
from scipy import stats

pytestmark = pytest.mark.gpu


def _small_hf(vocab=512, layers=4):
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(0)
    m = LlamaForCausalLM(LlamaConfig(vocab_size=vocab, hidden_size=256, intermediate_size=512,
                                     num_hidden_layers=layers, num_attention_heads=4, num_key_value_heads=2,
                                     rope_theta=500000.0, max_position_embeddings=4096)).eval()
    return m.to(torch.bfloat16)


def _prompts(lengths, vocab, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, vocab - 8, (n,), generator=g).tolist() for n in lengths]


def _check_equal_to_single(target, prompts, n_new, eos):
    from ssd.data.generate_selfdistill import generate_batch
    from ssd.engine.speculative import autoregressive_generate
    rows = generate_batch(target, prompts, n_new, eos, temperature=0.0, top_p=1.0, pad_id=0)
    assert len(rows) == len(prompts)
    for i, (p, row) in enumerate(zip(prompts, rows)):
        ref = autoregressive_generate(target, torch.tensor([p]), n_new, eos).tokens
        assert row == ref, f"prompt {i} (length {len(p)})"
    return rows


def test_batched_greedy_matches_single_prompts():
    from ssd.engine.speculative import TargetRunner
    target = TargetRunner(_small_hf())
    prompts = _prompts([3, 9, 6, 1, 70, 300, 257], 512, seed=1)
    rows = _check_equal_to_single(target, prompts, 20, {-1})
    assert all(len(r) == 20 for r in rows)
    # an EOS that one of the rows produces: that row stops after it, the others continue
    eos = {rows[2][5]}
    cut = _check_equal_to_single(target, prompts, 20, eos)
    assert len(cut[2]) <= 6 and cut[2][-1] in eos


def test_batched_greedy_more_rows_than_a_chunk():
    from ssd.engine.speculative import TargetRunner
    target = TargetRunner(_small_hf(layers=2))
    g = torch.Generator().manual_seed(5)
    lengths = torch.randint(1, 140, (70,), generator=g).tolist()
    _check_equal_to_single(target, _prompts(lengths, 512, seed=2), 8, {-1})


def test_batched_greedy_llama32_1b_layer_shapes():
    from ssd.engine.speculative import TargetRunner
    from ssd.models.llama import LlamaShape, MI355XLlama
    s = LlamaShape(hidden=2048, layers=2, heads=32, kv_heads=8, head_dim=64, inter=8192, vocab=128256, eps=1e-5)
    target = TargetRunner(MI355XLlama.synthetic(s, seed=3))
    _check_equal_to_single(target, _prompts([5, 64, 65, 255, 256, 257, 600, 31], 128256, seed=4), 24, {-1})


def test_sample_next_and_sampled_batches():
    """Greedy rows are the first-index argmax; a seeded generator reproduces sampled rows, and one
    generator advances: consecutive calls (and consecutive generate_batch calls) draw anew, as
    torch.multinomial's generator would."""
    from ssd.data.generate_selfdistill import generate_batch, sample_next
    from ssd.engine.speculative import TargetRunner
    g = torch.Generator().manual_seed(9)
    logits = (torch.randn(6, 1000, generator=g) * 0.5).to(torch.bfloat16).cuda()
    assert sample_next(logits, 0.0, 1.0).cpu()[:, 0].tolist() == logits.float().argmax(1).cpu().tolist()
    a = sample_next(logits, 0.7, 0.9, torch.Generator().manual_seed(1))
    b = sample_next(logits, 0.7, 0.9, torch.Generator().manual_seed(1))
    assert a.shape == (6, 1) and torch.equal(a, b)
    one = torch.Generator().manual_seed(1)
    first, second = sample_next(logits, 0.7, 0.9, one), sample_next(logits, 0.7, 0.9, one)
    assert torch.equal(first, a) and not torch.equal(first, second)
    again = torch.Generator().manual_seed(1)
    sample_next(logits, 0.7, 0.9, again)
    assert torch.equal(sample_next(logits, 0.7, 0.9, again), second)
    target = TargetRunner(_small_hf())
    prompts = _prompts([4, 40, 300], 512, seed=6)
    r1 = generate_batch(target, prompts, 16, {-1}, 0.8, 0.95, 0, torch.Generator().manual_seed(3))
    r2 = generate_batch(target, prompts, 16, {-1}, 0.8, 0.95, 0, torch.Generator().manual_seed(3))
    r3 = generate_batch(target, prompts, 16, {-1}, 0.8, 0.95, 0, torch.Generator().manual_seed(4))
    assert r1 == r2 and r1 != r3
    assert all(len(r) == 16 and all(0 <= t < 512 for t in r) for r in r1)
    shared = torch.Generator().manual_seed(3)
    s1 = generate_batch(target, prompts, 16, {-1}, 0.8, 0.95, 0, shared)
    s2 = generate_batch(target, prompts, 16, {-1}, 0.8, 0.95, 0, shared)
    assert s1 == r1 and s2 != s1


def _top64(lg, V, T, top_p, seed, counter):
    from ssd import ops
    out = torch.full((lg.shape[0],), -1, dtype=torch.int32, device="cuda")
    ops.sample_top64(lg, lg.shape[0], V, T, top_p, seed, counter, out)
    return out.cpu()


def _bf16_rows(rows, V, scale, seed):
    g = torch.Generator().manual_seed(seed)
    ld = (V + 7) // 8 * 8
    lg = torch.zeros(rows, ld, dtype=torch.bfloat16)
    lg[:, :V] = (torch.randn(rows, V, generator=g) * scale).to(torch.bfloat16)
    return lg


@pytest.mark.parametrize("V", [128256, 4096 + 7, 1000, 64])
@pytest.mark.parametrize("T,top_p", [(0.7, 0.9), (1.0, 1.0), (0.5, 0.3)])
def test_sample_top64_draw_for_draw(V, T, top_p):
    """ssd_sample_top64_bf16 against oracle.sampling.sample_next_top64 (generate_selfdistill.py:50-60
    with the kernels' Philox stream): same column for every row and counter, except draws the
    oracle flags as within 1e-4 of a tie of two Gumbel keys or of the nucleus cut."""
    from oracle import sampling as osm
    lg = _bf16_rows(12, V, 3.0, seed=V)
    dev = lg.cuda()
    fragile = 0
    for counter in (0, 1, 1 << 33):
        got = _top64(dev, V, T, top_p, 0x5EED, counter)
        for r in range(lg.shape[0]):
            want, fr = osm.sample_next_top64(lg[r, :V].float(), T, top_p, osm.Stream(0x5EED, counter), r)
            if fr:
                fragile += 1
                continue
            assert int(got[r]) == want, (counter, r)
    assert fragile <= 3


def test_sample_top64_ties_and_equality():
    """100 equal leaders spread over every chunk of a 128256 row (logit 0; every other logit -1000):
    the 64 candidates are the 64 lowest-column leaders; at top_p 0.5 the mass before rank j is
    exactly j/64, so ranks 0..32 are kept (an entry is dropped only when that mass exceeds top_p)
    and they are drawn uniformly; nothing else is ever drawn."""
    V = 128256
    cols = torch.randperm(V, generator=torch.Generator().manual_seed(2))[:100].sort().values
    ld = (V + 7) // 8 * 8
    row = torch.full((ld,), -1000.0)
    row[cols] = 0.0
    rows = 4000
    dev = row.to(torch.bfloat16).cuda().expand(rows, ld).contiguous()
    draws = torch.cat([_top64(dev, V, 1.0, 0.5, 77, c) for c in range(5)])
    kept = set(cols[:33].tolist())
    assert set(draws.tolist()) == kept
    counts = np.array([(draws == c).sum().item() for c in cols[:33].tolist()])
    assert stats.chisquare(counts).pvalue > 0.01


def test_sample_next_top64_chi_square_1e5():
    """1e5 seeded draws at V = 128256 from one row whose 0.9-nucleus over the full row holds ~390
    tokens (bf16 logits N(0, 3^2), T 0.7): the counts fit warp(top-64(logits)) by chi-square
    (p > 0.01) and reject the full-row warp (p < 1e-6), the distribution sampled before."""
    from oracle import sampling as osm
    V = 128256
    x = _bf16_rows(1, V, 3.0, seed=11)
    rows = 2000
    dev = x.cuda().expand(rows, x.shape[1]).contiguous()
    draws = torch.cat([_top64(dev, V, 0.7, 0.9, 1234, c) for c in range(50)]).numpy()
    counts = np.bincount(draws, minlength=V)
    N = counts.sum()
    assert N == 100000
    p = osm.top64_probs(x[0, :V].float(), 0.7, 0.9).numpy()
    p = p / p.sum()
    support = p > 0
    assert counts[~support].sum() == 0
    assert stats.chisquare(counts[support], p[support] * N).pvalue > 0.01
    full, _, _ = osm.warp_probs64(x[0, :V].float(), 0.7, 0.9)
    full = full.numpy() / full.numpy().sum()
    bins = full * N >= 5
    obs = np.append(counts[bins], counts[~bins].sum())
    exp = np.append(full[bins] * N, full[~bins].sum() * N)
    assert stats.chisquare(obs, exp).pvalue < 1e-6


def test_sample_top64_argument_errors():
    from ssd import ops
    out = torch.zeros(2, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError):
        ops.sample_top64(torch.zeros(2, 32, dtype=torch.bfloat16, device="cuda"), 2, 32, 1.0, 0.9, 1, 0, out)


def test_rows_view_keeps_per_sequence_offsets():
    """A view of rows that carry per-sequence KV arena offsets addresses the same offsets from its
    first row on (a view without them would read and write sequence 0's region)."""
    from ssd.models.subnetwork_draft import Rows
    rows = Rows(8, "cuda")
    off = torch.arange(8, dtype=torch.int64, device="cuda") * 1000
    rows.set_kv_offsets(off)
    v = rows.view(3)
    assert v.struct.kv_off == off[3:].data_ptr() and torch.equal(v.kv_off.cpu(), off[3:].cpu())
    assert Rows(8, "cuda").view(2).struct.kv_off is None
