"""The CPU plumbing configuration at its full size, on the oracle (no GPU).

Random-init Llama-3.2-1B-shaped target in fp32 (hidden 2048, 16 layers, 32 q / 8 kv heads,
head_dim 64, SwiGLU 8192, vocabulary 128256, RoPE theta 500000), built the reference's way:
``torch.manual_seed(0); LlamaForCausalLM(cfg)`` (reference tests/test_engine.py:20-28), so the
weights are N(0, 0.02). Draft layers [0, 7, 15] with the two bridges this plan needs
(into_7 from boundary 1, into_15 from boundary 8: RMSNorm + MLP 2048 -> 2048 -> 2048 with a
random first layer and a zero-initialised output projection, reference bridges.py:118-129).
Greedy chain of depth 4, a 128-token uniform prompt from seed 1, 64 new tokens: speculative
output must equal plain greedy decoding of the target (reference tests/test_engine.py:44-63).
"""

import torch
from transformers import LlamaConfig, LlamaForCausalLM

from oracle import engine as oe
from oracle import model as om


def test_config_a_llama32_1b_fp32_chain_sd_equals_ar():
    cfg = LlamaConfig(vocab_size=128256, hidden_size=2048, intermediate_size=8192, num_hidden_layers=16,
                      num_attention_heads=32, num_key_value_heads=8, head_dim=64, rope_theta=500000.0,
                      tie_word_embeddings=False, max_position_embeddings=4096)
    torch.manual_seed(0)
    hf = LlamaForCausalLM(cfg).eval()
    base = om.Llama.from_hf(hf, torch.float32)
    del hf
    specs = om.plan_bridges([0, 7, 15], 16)
    assert [(s.name, s.src_boundary, s.tgt_boundary) for s in specs] == [("into_7", 1, 7), ("into_15", 8, 15)]
    g = torch.Generator().manual_seed(2)
    bridges = {s.name: om.Bridge({
        "norm.weight": torch.ones(2048),
        "mlp.body.0.weight": torch.randn(2048, 2048, generator=g) * 0.02,
        "mlp.body.0.bias": torch.zeros(2048),
        "mlp.out_proj.weight": torch.zeros(2048, 2048),
        "mlp.out_proj.bias": torch.zeros(2048),
    }) for s in specs}
    draft = om.Subnetwork(base, [0, 7, 15], bridges)
    target = om.Target(base)
    ids = torch.randint(0, 128256, (128,), generator=torch.Generator().manual_seed(1)).tolist()
    ar = oe.autoregressive_generate(target, ids, 64, {-1})
    sd = oe.SpeculativeGenerator(target, draft, oe.Drafting(depth=4, branch=1), 128256).generate(ids, 64, {-1})
    assert len(ar.tokens) == 64
    assert sd.tokens == ar.tokens
    assert len(sd.accepted_per_round) <= 64
