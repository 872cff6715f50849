"""Pins the per-kernel oracle references (oracle/kernels.py) against the oracle model
forward (pinned to transformers) and closed forms. CPU only."""

import math

import torch
from transformers import LlamaConfig, LlamaForCausalLM

from oracle import kernels as ok
from oracle import model as om


def test_composed_layer_equals_model_layer():
    torch.manual_seed(0)
    hf = LlamaForCausalLM(LlamaConfig(vocab_size=64, hidden_size=128, intermediate_size=256, num_hidden_layers=1,
                                      num_attention_heads=4, num_key_value_heads=2, rope_theta=500000.0)).eval()
    base = om.Llama.from_hf(hf.to(torch.bfloat16))
    s, w = base.shape, base.w
    ids = torch.randint(0, 64, (7,), generator=torch.Generator().manual_seed(1))
    _, ref_h = om.Target(base)(ids)  # final-norm output
    # compose the same layer from the kernel references
    h = w("model.embed_tokens.weight")[ids].float()
    p = "model.layers.0."
    x = ok.rmsnorm(h, w(p + "input_layernorm.weight"), s.eps)
    q, k, v = ok.qkv_rope(x, w(p + "self_attn.q_proj.weight"), w(p + "self_attn.k_proj.weight"),
                          w(p + "self_attn.v_proj.weight"), s.heads, s.kv_heads, s.head_dim, torch.arange(7), s.theta)
    att = ok.rbf(ok.tree_attention(q, k.transpose(0, 1), v.transpose(0, 1), [t + 1 for t in range(7)], [[]] * 7))
    h = ok.linear(att.reshape(7, -1), w(p + "self_attn.o_proj.weight"), residual=h)
    x = ok.rmsnorm(h, w(p + "post_attention_layernorm.weight"), s.eps)
    a = ok.swiglu(x, w(p + "mlp.gate_proj.weight"), w(p + "mlp.up_proj.weight"))
    h = ok.linear(a, w(p + "mlp.down_proj.weight"), residual=h)
    got = ok.rmsnorm(h, w("model.norm.weight"), s.eps)
    torch.testing.assert_close(got, ref_h.float(), atol=2e-2, rtol=2e-2)
    assert (got - ref_h.float()).abs().mean() < 2e-3


def test_tree_attention_ref_matches_masked_attention():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(5, 4, 16, generator=g)
    k = torch.randn(2, 20, 16, generator=g)
    v = torch.randn(2, 20, 16, generator=g)
    prefix = [12, 12, 12, 13, 10]
    anc = [[], [14], [14, 17], [15, 18, 19], []]
    mask = torch.zeros(5, 20, dtype=torch.bool)
    for t in range(5):
        mask[t, :prefix[t]] = True
        mask[t, anc[t]] = True
    ref = om.attention(q.transpose(0, 1), k, v, mask).transpose(0, 1)
    torch.testing.assert_close(ok.tree_attention(q, k, v, prefix, anc), ref, atol=1e-5, rtol=1e-5)


def test_argmax_first_and_topk_known_answers():
    x = torch.tensor([[1.0, 3.0, 3.0, 2.0], [0.0, -1.0, 0.0, 0.0]])
    assert ok.argmax_first(x).tolist() == [1, 0]
    vals, idx, lse = ok.log_softmax_topk(x, 3)
    assert idx.tolist() == [[1, 2, 3], [0, 2, 3]]
    torch.testing.assert_close(lse[0], torch.tensor(math.log(math.e + 2 * math.e ** 3 + math.e ** 2)))


def test_kv_compact_ref_overlap():
    k = torch.arange(16.0)[:, None].repeat(1, 2)
    out = ok.kv_compact(k, 10, [10, 12, 13])
    assert out[10:13, 0].tolist() == [10.0, 12.0, 13.0]
    assert out[13:, 0].tolist() == [13.0, 14.0, 15.0]


def test_rope_rounding_chain_matches_model():
    x = torch.randn(3, 2, 16).to(torch.bfloat16)
    pos = torch.tensor([0, 5, 300])
    cos, sin = om.rope_cos_sin(pos, 16, 500000.0, torch.bfloat16)
    ref = om.apply_rope(x.transpose(0, 1), cos, sin).transpose(0, 1)
    torch.testing.assert_close(ok.rope(x.float(), pos, 500000.0), ref.float(), atol=0, rtol=0)
