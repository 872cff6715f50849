"""Pins the oracle's model forward (CPU, fp32) against the transformers Llama in the image
and against the reference's own forward-path invariants (tests/test_forward_pass.py:109-180
in the reference)."""

import copy

import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM

from oracle import model as om


def tiny_hf(vocab=128, seed=0, layers=6):
    torch.manual_seed(seed)
    cfg = LlamaConfig(vocab_size=vocab, hidden_size=64, intermediate_size=128, num_hidden_layers=layers,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256,
                      rope_theta=500000.0, attn_implementation="eager")
    return LlamaForCausalLM(cfg).eval()


@pytest.fixture(scope="module")
def hf():
    return tiny_hf()


@pytest.fixture(scope="module")
def base(hf):
    return om.Llama.from_hf(hf)


def test_full_selection_matches_hf(hf, base):
    tgt = om.Target(base)
    ids = torch.randint(0, 128, (13,), generator=torch.Generator().manual_seed(0))
    logits, _ = tgt(ids)
    with torch.no_grad():
        ref = hf(ids[None]).logits[0]
    torch.testing.assert_close(logits, ref, atol=1e-5, rtol=1e-4)


def test_identity_bridges_equal_layer_skipping(hf, base):
    layers = [0, 3, 5]
    specs = om.plan_bridges(layers, 6)
    draft = om.Subnetwork(base, layers, om.identity_bridges(specs, 64))
    skip = LlamaForCausalLM(copy.deepcopy(hf.config)).eval()
    skip.load_state_dict(hf.state_dict())
    skip.model.layers = torch.nn.ModuleList([skip.model.layers[i] for i in layers])
    for j, layer in enumerate(skip.model.layers):
        layer.self_attn.layer_idx = j
    skip.config.num_hidden_layers = 3
    ids = torch.randint(0, 128, (9,), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        ref = skip(ids[None]).logits[0]
    torch.testing.assert_close(draft(ids)[0], ref, atol=1e-5, rtol=1e-4)


def test_bridge_plan_matches_reference_cases():
    assert [(s.name, s.src_boundary, s.tgt_boundary) for s in om.plan_bridges([0, 2, 5], 6)] == [
        ("into_2", 1, 2), ("into_5", 3, 5)]
    assert [s.name for s in om.plan_bridges([1, 2, 4], 6)] == ["into_1", "into_4", "into_norm"]
    assert [s.name for s in om.plan_bridges([0, 7, 15], 16)] == ["into_7", "into_15"]
    assert [(s.src_boundary, s.tgt_boundary) for s in om.plan_bridges([0, 15, 31], 32)] == [(1, 15), (16, 31)]


def test_incremental_cache_matches_full(base):
    draft = om.Subnetwork(base, [0, 2, 5], om.random_bridges(om.plan_bridges([0, 2, 5], 6), 64, seed=3,
                                                                init_std=0.05))
    ids = torch.randint(0, 128, (12,), generator=torch.Generator().manual_seed(2))
    full, _ = draft(ids)
    cache = draft.new_cache(32)
    chunks = [draft(ids[:7], None, cache)[0]]
    for t in range(7, 12):
        chunks.append(draft(ids[t:t + 1], None, cache)[0])
    assert cache.get_seq_length() == 12
    torch.testing.assert_close(torch.cat(chunks), full, atol=1e-5, rtol=1e-4)


def test_tree_mask_matches_per_branch_decoding_and_compaction(base):
    """prefix -> a -> {b, c}; b -> d: each node's logits == decoding its path alone; after
    keep_positions on a->b->d, the next step == re-decoding prefix+path."""
    draft = om.Subnetwork(base, [0, 2, 5], om.random_bridges(om.plan_bridges([0, 2, 5], 6), 64, seed=4,
                                                                init_std=0.05))
    prefix = torch.randint(0, 128, (6,), generator=torch.Generator().manual_seed(1))
    a, b, c, d = 10, 20, 30, 40
    parents, depth = [-1, 0, 0, 1], [0, 1, 1, 2]
    mask = torch.zeros(4, 4, dtype=torch.bool)
    for i in range(4):
        j = i
        while j != -1:
            mask[i, j] = True
            j = parents[j]
    cache = draft.new_cache(32)
    draft(prefix, None, cache)
    tree_logits, _ = draft(torch.tensor([a, b, c, d]), torch.tensor([6 + x for x in depth]), cache, mask)
    for node, path in {0: [a], 1: [a, b], 2: [a, c], 3: [a, b, d]}.items():
        ref, _ = draft(torch.cat([prefix, torch.tensor(path)]))
        torch.testing.assert_close(tree_logits[node], ref[-1], atol=1e-5, rtol=1e-4)
    cache.keep_positions(6, [6, 7, 9])
    nxt, _ = draft(torch.tensor([50]), None, cache)
    ref, _ = draft(torch.tensor(prefix.tolist() + [a, b, d, 50]))
    torch.testing.assert_close(nxt[-1], ref[-1], atol=1e-5, rtol=1e-4)


def test_keep_positions_overlapping_ranges_is_a_gather():
    """start=10, positions [10,12,13]: dst slot 12 is the src of the 3rd entry; the move must
    read every source before writing (kv_cache.py:68-69 materialises with index_select)."""
    cache = om.KVCache(1, 16)
    k = torch.arange(16, dtype=torch.float)[None, :, None].repeat(2, 1, 3)
    cache.update(0, k, k.clone())
    cache.advance(16)
    cache.keep_positions(10, [10, 12, 13])
    assert cache.k[0][0, 10:13, 0].tolist() == [10.0, 12.0, 13.0]
    assert cache.seq_len == 13


def test_kv_overflow_raises(base):
    tgt = om.Target(base)
    cache = tgt.new_cache(4)
    with pytest.raises(RuntimeError):
        tgt(torch.arange(5), None, cache)


def test_bridge_zero_init_is_identity():
    br = om.identity_bridges(om.plan_bridges([0, 3], 6), 64)["into_3"]
    x = torch.randn(5, 64)
    torch.testing.assert_close(br(x), x)


def test_rope_table_matches_hf(hf):
    pos = torch.tensor([0, 1, 7, 100, 255])
    cos, sin = om.rope_cos_sin(pos, 16, 500000.0, torch.float32)
    rc, rs = hf.model.rotary_emb(torch.zeros(1, dtype=torch.float32), pos[None])
    torch.testing.assert_close(cos, rc[0], atol=0, rtol=0)
    torch.testing.assert_close(sin, rs[0], atol=0, rtol=0)


def test_bf16_forward_close_to_hf_bf16(hf):
    """The bf16 restatement (the cast points of the reference's bf16 path) stays within the
    per-node logit tolerance of the HF bf16 model."""
    hfb = copy.deepcopy(hf).to(torch.bfloat16)
    base = om.Llama.from_hf(hfb)
    ids = torch.randint(0, 128, (10,), generator=torch.Generator().manual_seed(5))
    with torch.no_grad():
        ref = hfb(ids[None]).logits[0].float()
    got = om.Target(base)(ids)[0].float()
    torch.testing.assert_close(got, ref, atol=1e-2, rtol=2e-2)


LLAMA3_ROPE = {"rope_type": "llama3", "rope_theta": 500000.0, "factor": 8.0, "low_freq_factor": 1.0,
               "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}


def test_llama3_rope_tables_match_hf():
    """Llama 3.1 frequency scaling (rope_type "llama3", the Llama-3.1/3.2 checkpoints' setting): the
    oracle's and the package's cos/sin tables equal transformers' LlamaRotaryEmbedding exactly, at
    head_dim 128 and 64 where all three wavelength bands (kept, blended, scaled) occur."""
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

    from ssd.models.llama import LlamaShape, rope_tables

    for hd in (128, 64):
        cfg = LlamaConfig(hidden_size=hd * 4, num_attention_heads=4, head_dim=hd, max_position_embeddings=131072,
                          rope_parameters=dict(LLAMA3_ROPE))
        rot = LlamaRotaryEmbedding(cfg)
        pos = torch.arange(0, 5000, 7)
        cos_hf, sin_hf = rot(torch.zeros(1, dtype=torch.float32), pos[None])
        cos_o, sin_o = om.rope_cos_sin(pos, hd, 500000.0, torch.float32, om.LlamaShape.from_hf_config(cfg).rope_scaling)
        assert torch.equal(cos_o, cos_hf[0]) and torch.equal(sin_o, sin_hf[0])
        shape = LlamaShape.from_hf_config(cfg)
        assert shape.rope_scaling == (8.0, 1.0, 4.0, 8192)
        cos_p, sin_p = rope_tables(5000, hd, shape.theta, "cpu", shape.rope_scaling)
        half = hd // 2
        assert torch.equal(cos_p[pos], cos_hf[0, :, :half].to(torch.bfloat16))
        assert torch.equal(sin_p[pos], sin_hf[0, :, :half].to(torch.bfloat16))
        # the scaling matters: plain tables differ
        cos_plain, _ = om.rope_cos_sin(pos, hd, 500000.0, torch.float32)
        assert (cos_plain - cos_hf[0]).abs().max() > 1e-2


def test_llama3_rope_forward_matches_hf():
    torch.manual_seed(4)
    cfg = LlamaConfig(vocab_size=128, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=131072,
                      rope_parameters=dict(LLAMA3_ROPE, original_max_position_embeddings=64),
                      attn_implementation="eager")
    hf = LlamaForCausalLM(cfg).eval()
    base = om.Llama.from_hf(hf)
    assert base.shape.rope_scaling == (8.0, 1.0, 4.0, 64)
    ids = torch.randint(0, 128, (40,), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        ref = hf(ids[None]).logits[0]
    torch.testing.assert_close(om.Target(base)(ids)[0], ref, atol=1e-5, rtol=1e-4)
    plain = om.Llama(base.sd, om.LlamaShape(**{**vars(base.shape), "rope_scaling": None}), torch.float32)
    assert (om.Target(plain)(ids)[0] - ref).abs().max() > 1e-3


def test_unsupported_rope_type_is_rejected():
    from ssd.models.llama import LlamaShape

    cfg = LlamaConfig(hidden_size=64, num_attention_heads=4,
                      rope_parameters={"rope_type": "linear", "rope_theta": 10000.0, "factor": 2.0})
    with pytest.raises(ValueError, match="rope_type"):
        LlamaShape.from_hf_config(cfg)
