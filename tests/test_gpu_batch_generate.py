"""Batched generation (reference tests/test_selfdistill.py): continuing a batch of prompts of
different lengths must equal continuing each prompt alone. Here the equality is bit for bit in bf16
(every row's arithmetic is independent of the other rows), with prompts on both sides of the
prefill threshold and of 64- and 256-key block boundaries, batches larger than one 64-row chunk,
and the real per-layer shapes of Llama-3.2-1B."""

import pytest
import torch

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
    from ssd.data.generate_selfdistill import generate_batch, sample_next
    from ssd.engine.speculative import TargetRunner
    g = torch.Generator().manual_seed(9)
    logits = (torch.randn(6, 1000, generator=g) * 3).to(torch.bfloat16).cuda()
    assert sample_next(logits, 0.0, 1.0).cpu()[:, 0].tolist() == logits.float().argmax(1).cpu().tolist()
    a = sample_next(logits, 0.7, 0.9, torch.Generator().manual_seed(1))
    b = sample_next(logits, 0.7, 0.9, torch.Generator().manual_seed(1))
    assert a.shape == (6, 1) and torch.equal(a, b)
    target = TargetRunner(_small_hf())
    prompts = _prompts([4, 40, 300], 512, seed=6)
    r1 = generate_batch(target, prompts, 16, {-1}, 0.8, 0.95, 0, torch.Generator().manual_seed(3))
    r2 = generate_batch(target, prompts, 16, {-1}, 0.8, 0.95, 0, torch.Generator().manual_seed(3))
    r3 = generate_batch(target, prompts, 16, {-1}, 0.8, 0.95, 0, torch.Generator().manual_seed(4))
    assert r1 == r2 and r1 != r3
    assert all(len(r) == 16 and all(0 <= t < 512 for t in r) for r in r1)
