"""End-to-end parity of the HIP decode path (the reference's own invariants, on the GPU).

* Greedy speculative output is bit-identical to greedy autoregressive decoding with the
  same kernels, for chain / tree / pruned / deep-chain / d4 [3,2,2,1] max 24 (with and without
  width 8) / d6 [4,2,2,1,1,1] max 32 trees, untrained and perfect drafts, draft-vocab subsets and
  EOS (reference tests/test_engine.py:44-92).
* Tree rows are bit-identical to decoding each root->node path alone, before and after KV
  compaction (reference tests/test_forward_pass.py:146-180) -- stronger than the reference,
  which checks them to 1e-5 in fp32.
* Logits match the CPU oracle's bf16 forward within rel 2e-2 / abs 1e-2; greedy tokens match
  the oracle's greedy decoding up to the first near-tie (a flip is allowed only where the
  oracle's two candidates are within that tolerance).
"""

import random

import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM

from oracle import engine as oe
from oracle import model as om

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = dict(atol=1e-2, rtol=2e-2)


def assert_logits_close(got, ref_bf16, ref_exact):
    """Per-node logit tolerance (abs 1e-2, rel 2e-2): every element against the exact fp32
    evaluation of the same bf16 weights; against the oracle's own bf16 rounding chain (a second,
    independent set of roundings) for >= 99.9% of elements, none beyond twice the tolerance."""
    torch.testing.assert_close(got, ref_exact, **TOL)
    err = (got - ref_bf16).abs()
    lim = TOL["atol"] + TOL["rtol"] * ref_bf16.abs()
    assert (err <= lim).float().mean() >= 0.999, f"{(err > lim).sum()} elements outside the tolerance"
    assert (err <= 2 * lim).all(), f"max deviation {err.max():.4f}"


def fp32_view(base):
    """The oracle evaluating the same bf16-valued weights in fp32 (no intermediate rounding)."""
    return om.Llama({k: v.float() for k, v in base.sd.items()}, base.shape, torch.float32)


def hf_model(seed=0, layers=6, hidden=256, heads=4, kv=2, inter=512, vocab=512, scale=1.0):
    torch.manual_seed(seed)
    m = LlamaForCausalLM(LlamaConfig(vocab_size=vocab, hidden_size=hidden, intermediate_size=inter,
                                     num_hidden_layers=layers, num_attention_heads=heads, num_key_value_heads=kv,
                                     rope_theta=500000.0, max_position_embeddings=4096)).eval()
    with torch.no_grad():
        m.lm_head.weight.mul_(scale)
    return m.to(torch.bfloat16)


@pytest.fixture(scope="module")
def hf():
    return hf_model()


@pytest.fixture(scope="module")
def oracle_base(hf):
    return om.Llama.from_hf(hf)


def ssd():
    import ssd.engine.speculative as sp
    from ssd.config import BridgeConfig, DraftingConfig
    from ssd.models.subnetwork_draft import SubnetworkDraftModel
    return sp, BridgeConfig, DraftingConfig, SubnetworkDraftModel


def make_draft(hf, kind, layers=(0, 3, 5), seed=11):
    _, BridgeConfig, _, SDM = ssd()
    if kind == "perfect":
        return SDM(hf, list(range(hf.config.num_hidden_layers)))
    torch.manual_seed(seed)
    return SDM(hf, list(layers), BridgeConfig(init_std=0.02))


def oracle_draft(base, draft):
    bridges = {name: om.Bridge({k: v.detach().to(torch.bfloat16).cpu() for k, v in br.state_dict().items()})
               for name, br in draft.bridges.items()}
    return om.Subnetwork(base, draft.layer_indices, bridges)


def prompt(n, seed, vocab=512):
    return torch.randint(0, vocab, (1, n), generator=torch.Generator().manual_seed(seed))


TREES = {
    "chain": dict(depth=4, branch=1),
    "tree": dict(depth=3, branch=[3, 2, 2]),
    "pruned": dict(depth=5, branch=[4, 3, 2, 2, 1], width=[4, 6, 6, 4, 4], max_nodes=12),
    "deep_chain": dict(depth=8, branch=1),
    "d4_3221_max24": dict(depth=4, branch=[3, 2, 2, 1], max_nodes=24),
    "d4_3221_w8_max24": dict(depth=4, branch=[3, 2, 2, 1], width=8, max_nodes=24),
    "d6_422111_max32": dict(depth=6, branch=[4, 2, 2, 1, 1, 1], max_nodes=32),  # 76 drafted, 33 verify rows
}


# ------------------------------------------------------------------------ forward
def test_target_logits_match_oracle(hf, oracle_base):
    sp, *_ = ssd()
    target = sp.TargetRunner(hf)
    ids = prompt(40, 1)
    got = target(ids).logits[0].float().cpu()
    ref = om.Target(oracle_base)(ids[0])[0].float()
    exact = om.Target(fp32_view(oracle_base))(ids[0])[0]
    assert_logits_close(got, ref, exact)


def test_llama3_rope_target_logits_match_oracle():
    """A model with Llama 3.1 frequency scaling (rope_type "llama3", original context 64 so that the
    scaled and blended bands reach the positions used): logits vs the oracle, and greedy SD == AR."""
    sp, _, DraftingConfig, _ = ssd()
    torch.manual_seed(5)
    cfg = LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=4,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=4096,
                      rope_parameters={"rope_type": "llama3", "rope_theta": 500000.0, "factor": 8.0,
                                       "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                                       "original_max_position_embeddings": 64})
    hf3 = LlamaForCausalLM(cfg).eval().to(torch.bfloat16)
    base = om.Llama.from_hf(hf3)
    assert base.shape.rope_scaling is not None
    target = sp.TargetRunner(hf3)
    assert target.model.shape.rope_scaling == (8.0, 1.0, 4.0, 64)
    ids = prompt(48, 7)
    got = target(ids).logits[0].float().cpu()
    assert_logits_close(got, om.Target(base)(ids[0])[0].float(), om.Target(fp32_view(base))(ids[0])[0])
    draft = make_draft(hf3, "untrained", layers=(0, 3))
    ar = sp.autoregressive_generate(target, ids, 24, {-1}).tokens
    sd = sp.SpeculativeGenerator(hf3, draft, DraftingConfig(depth=3, branch=[2, 2, 1]), target).generate(ids, 24, {-1})
    assert sd.tokens == ar


def test_draft_logits_match_oracle(hf, oracle_base):
    draft = make_draft(hf, "untrained")
    ids = prompt(30, 2)
    got = draft(ids).logits[0].float().cpu()
    ref = oracle_draft(oracle_base, draft)(ids[0])[0].float()
    od = oracle_draft(oracle_base, draft)
    exact_bridges = {k: om.Bridge({n: t.float() for n, t in b.sd.items()}) for k, b in od.bridges.items()}
    exact = om.Subnetwork(fp32_view(oracle_base), draft.layer_indices, exact_bridges)(ids[0])[0]
    assert_logits_close(got, ref, exact)


@pytest.mark.parametrize("bridge", [dict(), dict(num_layers=3, activation="gelu", hidden_dim=384),
                                    dict(mlp_type="swiglu", hidden_dim=320, bias=False)])
def test_forward_sequencer_bitwise_equals_per_kernel_calls(hf, bridge):
    """ssd_forward (one C call per forward) == the same kernels called one by one from Python
    (the path taken when bridge states are requested), with bridges of every kind, a skipped
    final layer (pre-norm bridge) and a vocabulary-subset head."""
    _, BridgeConfig, _, SDM = ssd()
    torch.manual_seed(5)
    draft = SDM(hf, [1, 2, 4], BridgeConfig(init_std=0.02, **bridge))
    ids = prompt(70, 9)
    for subset in (None, torch.arange(0, 512, 3)):
        draft.set_vocab_subset(subset)
        seq = draft(ids)
        per = draft(ids, output_bridge_states=True)
        assert set(per.bridge_states) == {"into_1", "into_4", "into_norm"}
        assert torch.equal(seq.hidden_states, per.hidden_states)
        assert torch.equal(seq.logits, per.logits)


def test_incremental_cache_bitwise_equals_full(hf):
    draft = make_draft(hf, "untrained")
    ids = prompt(100, 3)
    full = draft(ids).logits[0]
    cache = draft.new_cache(128)
    parts = [draft(ids[:, :70], past_key_values=cache).logits[0]]
    for t in range(70, 100):
        parts.append(draft(ids[:, t:t + 1], past_key_values=cache).logits[0])
    assert cache.get_seq_length() == 100
    assert torch.equal(torch.cat(parts), full)


def test_tree_rows_bitwise_equal_path_decoding_and_compaction(hf):
    """prefix -> a -> {b, c}; b -> d, at a prefix crossing a 64-key block boundary."""
    draft = make_draft(hf, "untrained")
    pre = prompt(66, 4)
    a, b, c, d = 10, 20, 30, 40
    parents, depth = [-1, 0, 0, 1], [0, 1, 1, 2]
    mask = torch.zeros(4, 4, dtype=torch.bool)
    for i in range(4):
        j = i
        while j != -1:
            mask[i, j] = True
            j = parents[j]
    cache = draft.new_cache(128)
    draft(pre, past_key_values=cache)
    P = pre.shape[1]
    tree = draft(torch.tensor([[a, b, c, d]]), position_ids=torch.tensor([[P + x for x in depth]]),
                 past_key_values=cache, tree_attention_mask=mask).logits[0]
    for node, path in {0: [a], 1: [a, b], 2: [a, c], 3: [a, b, d]}.items():
        ref = draft(torch.cat([pre, torch.tensor([path])], 1)).logits[0, -1]
        assert torch.equal(tree[node], ref), f"node {node}"
    cache.keep_positions(P, torch.tensor([P, P + 1, P + 3]))
    nxt = draft(torch.tensor([[50]]), past_key_values=cache).logits[0, -1]
    ref = draft(torch.cat([pre, torch.tensor([[a, b, d, 50]])], 1)).logits[0, -1]
    assert torch.equal(nxt, ref)


# -------------------------------------------------------------------------- engine
@pytest.mark.parametrize("tree_name", list(TREES))
@pytest.mark.parametrize("kind", ["untrained", "perfect"])
def test_greedy_sd_bitwise_equals_autoregressive(hf, tree_name, kind):
    sp, _, DraftingConfig, _ = ssd()
    target = sp.TargetRunner(hf)
    draft = make_draft(hf, kind)
    cfg = DraftingConfig(**TREES[tree_name])
    for n_prompt, seed in ((5, 0), (70, 1), (300, 2)):
        ids = prompt(n_prompt, seed)
        ref = sp.autoregressive_generate(target, ids, 48, {-1}).tokens
        res = sp.SpeculativeGenerator(hf, draft, cfg, target).generate(ids, 48, {-1})
        assert res.tokens == ref, f"{tree_name}/{kind}/prompt{n_prompt} diverged"
        assert sum(res.accepted_per_round) >= 47
        if kind == "perfect" and cfg.max_nodes is None:
            assert res.mean_accepted > cfg.depth


@pytest.mark.parametrize("kind,n_new", [("untrained", 330), ("perfect", 600)])
def test_graph_rounds_across_segments_bitwise(hf, kind, n_new):
    """Captured rounds (one HIP graph per 256-position segment of root positions, replayed with one
    round queued behind the one being read) give exactly the tokens of plain launches and of
    autoregressive decoding, across segment boundaries (prompt 250: roots cross 256 and 512) and up
    to the end of the cache."""
    sp, _, DraftingConfig, _ = ssd()
    target = sp.TargetRunner(hf)
    draft = make_draft(hf, kind)
    cfg = DraftingConfig(depth=4, branch=[3, 2, 2, 1], max_nodes=24)
    ids = prompt(250, 4)
    ref = sp.autoregressive_generate(target, ids, n_new, {-1}).tokens
    gen = sp.SpeculativeGenerator(hf, draft, cfg, target)
    sess = gen.session(gen.capacity(ids.shape[1], n_new), graphs=True)
    assert sess.graphs
    out = [sess.prefill(ids[0].tolist())]
    while len(out) < n_new:
        out.extend(sess.step())
    sess.drain()
    assert out[:n_new] == ref
    rounds = len(sess.accepted_per_round)
    assert sess.captures >= 2 and sess.graph_rounds >= rounds - 3, (sess.captures, sess.graph_rounds, rounds)
    assert sess.graph_launches > 20
    plain = gen.generate(ids, n_new, {-1})
    assert plain.tokens == ref
    assert gen.generate(ids, 40, {-1}, graphs=True).tokens == ref[:40]


def test_greedy_sd_with_draft_vocab_subset(hf):
    sp, _, DraftingConfig, _ = ssd()
    from ssd.data.token_freq import top_vocab

    target = sp.TargetRunner(hf)
    draft = make_draft(hf, "perfect")
    draft.set_vocab_subset(top_vocab(torch.arange(512).flip(0), 200, always={511}))
    assert draft.vocab_ids.numel() == 200 and 511 in draft.vocab_ids.tolist()
    ids = prompt(7, 5)
    ref = sp.autoregressive_generate(target, ids, 40, {-1}).tokens
    res = sp.SpeculativeGenerator(hf, draft, DraftingConfig(depth=3, branch=[3, 2, 2]), target).generate(ids, 40, {-1})
    assert res.tokens == ref
    assert draft(ids).logits.shape[-1] == 200


def test_greedy_sd_stops_at_eos(hf):
    sp, _, DraftingConfig, _ = ssd()
    target = sp.TargetRunner(hf)
    ids = prompt(6, 0)
    free = sp.autoregressive_generate(target, ids, 30, {-1}).tokens
    eos = {free[10]}
    ref = sp.autoregressive_generate(target, ids, 30, eos).tokens
    res = sp.SpeculativeGenerator(hf, make_draft(hf, "perfect"), DraftingConfig(depth=4, branch=1),
                                  target).generate(ids, 30, eos)
    assert res.tokens == ref and res.tokens[-1] in eos


@pytest.mark.parametrize("tree", ["pruned", "d4_3221_max24"])
def test_fused_head_proposals_equal_two_launch_proposals(hf, tree):
    """Greedy drafting with the proposals' top-k chunk pass in the head launch (ssd_gemm_topk_bf16)
    and with stored logits + ssd_row_topk_partial_bf16: both decode exactly like AR, with the same
    accepted counts and tree sizes round by round."""
    sp, _, DraftingConfig, _ = ssd()
    target = sp.TargetRunner(hf)
    ids = prompt(40, 5)
    ref = sp.autoregressive_generate(target, ids, 40, {-1}).tokens
    out = []
    for fused in (True, False):
        gen = sp.SpeculativeGenerator(hf, make_draft(hf, "untrained"), DraftingConfig(**TREES[tree]), target)
        gen.drafter.fused_head = fused
        res = gen.generate(ids, 40, {-1})
        assert res.tokens == ref, f"fused_head={fused}"
        out.append((res.accepted_per_round, res.tree_sizes))
    assert out[0] == out[1]


def test_tree_shape_limits(hf):
    _, _, DraftingConfig, _ = ssd()
    from ssd.engine.tree_drafter import TreeDrafter

    draft = make_draft(hf, "untrained")
    cfg = DraftingConfig(**TREES["pruned"])
    drafter = TreeDrafter(draft, cfg)
    cache = draft.new_cache(64)
    tree = drafter.build(cache, torch.tensor([[1, 2, 3]]), root_pos=2)
    assert len(tree) <= cfg.max_nodes
    for i in range(len(tree)):
        p = tree.parents[i]
        assert p == -1 or (p < i and tree.depths[p] == tree.depths[i] - 1)
    assert cache.get_seq_length() == 3 + drafter.max_tree_cache()


def test_greedy_tokens_match_oracle_up_to_near_ties(hf, oracle_base):
    """Our bf16 greedy decoding vs the oracle's bf16 greedy decoding: identical until a step
    where the oracle's logits of the two tokens are within the logit tolerance."""
    sp, *_ = ssd()
    target = sp.TargetRunner(hf)
    otarget = om.Target(oracle_base)
    for seed in range(3):
        ids = prompt(20, 10 + seed)
        got = sp.autoregressive_generate(target, ids, 32, {-1}).tokens
        ref = oe.autoregressive_generate(otarget, ids[0].tolist(), 32, {-1}).tokens
        if got == ref:
            continue
        i = next(j for j in range(len(ref)) if got[j] != ref[j])
        logits = otarget(torch.tensor(ids[0].tolist() + ref[:i]))[0][-1].float()
        gap = (logits[ref[i]] - logits[got[i]]).abs().item()
        assert gap <= TOL["atol"] + TOL["rtol"] * logits[ref[i]].abs().item(), \
            f"seed {seed}: diverged at {i} with oracle logit gap {gap:.4f}"


@pytest.mark.parametrize("shape", ["llama32_1b", "llama3_8b"])
def test_realistic_shapes_sd_equals_ar(shape):
    """Two layers at the real per-layer shapes (1B: hd 64, 32/8 heads; 8B: hd 128, 32/8 heads;
    vocab 128256), synthetic weights, ~600-token context crossing superblock boundaries. Both
    shapes run their MLPs as the fused one-launch kernel (ssd_mlp_bf16) in draft, verify and the
    autoregressive baseline."""
    sp, BridgeConfig, DraftingConfig, SDM = ssd()
    from ssd.models.llama import LlamaShape, MI355XLlama

    dims = {"llama32_1b": (2048, 32, 8, 64, 8192), "llama3_8b": (4096, 32, 8, 128, 14336)}[shape]
    s = LlamaShape(hidden=dims[0], layers=2, heads=dims[1], kv_heads=dims[2], head_dim=dims[3], inter=dims[4],
                   vocab=128256, eps=1e-5)
    model = MI355XLlama.synthetic(s, seed=1)
    assert model.mlp_fused
    target = sp.TargetRunner(model)
    torch.manual_seed(0)
    draft = SDM(model, [1], BridgeConfig(init_std=0.02))
    ids = prompt(600, 7, vocab=128256)
    cfg = DraftingConfig(depth=4, branch=[3, 2, 2, 1], max_nodes=24)
    ref = sp.autoregressive_generate(target, ids, 40, {-1}).tokens
    res = sp.SpeculativeGenerator(model, draft, cfg, target).generate(ids, 40, {-1})
    assert res.tokens == ref
    perfect = SDM(model, [0, 1])
    res = sp.SpeculativeGenerator(model, perfect, cfg, target).generate(ids, 40, {-1})
    assert res.tokens == ref and res.mean_accepted > 3.0


def test_mlp_timeout_count_fails_the_round(hf):
    """A nonzero fused-MLP timeout count (preset from the host: no kernel is made to stall) makes
    the round, greedy decoding and the generic forward raise instead of returning tokens."""
    from ssd import _lib
    sp, _, DraftingConfig, _ = ssd()
    target = sp.TargetRunner(hf)
    draft = make_draft(hf, "untrained")
    gen = sp.SpeculativeGenerator(hf, draft, DraftingConfig(depth=3, branch=[2, 2, 1]), target)
    ids = torch.randint(0, 512, (1, 12), generator=torch.Generator().manual_seed(3))
    sess = gen.session(gen.capacity(12, 16))
    sess.prefill(ids[0].tolist())
    sess.step()
    sess.ws.status[sess.ws.timeout_word] = 1
    try:
        with pytest.raises(_lib.SsdError, match="flag waits gave up"):
            sess.step()
        ws = target.workspace()
        ws.status[ws.timeout_word] = 1
        with pytest.raises(_lib.SsdError, match="flag waits gave up"):
            sp.autoregressive_generate(target, ids, 4, {-1})
        with pytest.raises(_lib.SsdError, match="flag waits gave up"):
            target(ids)
    finally:
        for w in (sess.ws, target.workspace()):
            w.clear_faults()
    torch.cuda.synchronize()
    assert sp.autoregressive_generate(target, ids, 4, {-1}).tokens
