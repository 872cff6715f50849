"""The reference's Python surface that the drop-in keeps, on the CPU (no GPU, no kernels):

* ``SSDConfig.from_yaml`` on every YAML the reference ships (read in place from the reference
  checkout where it is present, skipped elsewhere), with the reference's own expectations
  (tests/test_training.py:49-73 there): draft layers, stage-2 temperature, per-depth lists;
  bad configs and unknown keys rejected with ``ValueError``;
* the checkpoint layout: ``{output_dir}/{L-profile}/stage{1,2}.pt | online.pt`` and
  ``latest_checkpoint``'s order online > stage2 > stage1 (reference ssd/runtime.py:87-98);
* the bridge checkpoint format ``{layer_indices, bridge_config, state_dict, meta}`` (reference
  ssd/models/subnetwork_draft.py:455-472): a file written with the reference's module tree
  loads into ``TransitionBridge`` with ``weights_only=True``, every tensor in place;
* ``top_vocab`` against its closed form and the draft-vocabulary files' paths;
* ``ssd-run``'s flag set (reference ssd/cli/run.py:46-67).
"""

import glob
import json
import os

import pytest
import torch
import torch.nn as nn

from ssd.config import BridgeConfig, DraftingConfig, SSDConfig, profile_name

REF_CONFIGS = "/root/reference/configs"
SHIPPED = sorted(glob.glob(os.path.join(REF_CONFIGS, "*.yaml")) + glob.glob(os.path.join(REF_CONFIGS, "*", "*.yaml")))
need_ref = pytest.mark.skipif(not SHIPPED, reason="the reference's config files are not present here")


@need_ref
@pytest.mark.parametrize("name,layers", [("llama32_1b", [0, 7, 15]), ("llama3_8b", [0, 15, 31]),
                                         ("llama3_70b", [0, 39, 79])])
def test_shipped_subnetwork_configs_load(name, layers):
    cfg = SSDConfig.from_yaml(os.path.join(REF_CONFIGS, f"{name}_subnetwork.yaml"))
    assert cfg.draft_layers == layers
    assert cfg.training.stage2.temperature == 2.0
    assert len(cfg.drafting.per_depth(cfg.drafting.branch, "branch")) == cfg.drafting.depth
    assert cfg.model.torch_dtype == "bfloat16"


@need_ref
def test_every_shipped_config_loads():
    assert len(SHIPPED) >= 14, SHIPPED
    for path in SHIPPED:
        cfg = SSDConfig.from_yaml(path)
        assert cfg.draft_layers == sorted(set(cfg.draft_layers)), path
        cfg.drafting.validate()
        assert profile_name(cfg.draft_layers).startswith("L")


@pytest.mark.parametrize("yaml_text", [
    "draft_layers: {1: [0, 1]}\n",  # the old per-K map is no longer accepted
    "draft_layers: [0, 1]\ndrafting: {depth: 3, branch: [2, 2]}\n",  # branch list length != depth
    "draft_layers: [0, 1]\ndrafting: {depth: 0}\n",
    "draft_layers: [0, 1]\ndrafting: {depth: 2, width: [4]}\n",
])
def test_bad_configs_rejected(tmp_path, yaml_text):
    p = tmp_path / "c.yaml"
    p.write_text(yaml_text)
    with pytest.raises(ValueError):
        SSDConfig.from_yaml(p)


@pytest.mark.parametrize("yaml_text,key", [
    ("draft_layers: [0, 1]\ntraining: {stage1: {lrr: 1.0}}\n", "lrr"),
    ("draft_layers: [0, 1]\ndrafting: {depht: 3}\n", "depht"),
    ("draft_layers: [0, 1]\nbridges: {}\n", "bridges"),
])
def test_unknown_config_keys_rejected(tmp_path, yaml_text, key):
    p = tmp_path / "c.yaml"
    p.write_text(yaml_text)
    with pytest.raises(ValueError, match=key):
        SSDConfig.from_yaml(p)


def test_layer_indices_validated_against_the_model():
    cfg = SSDConfig(draft_layers=[0, 15, 31])
    cfg.validate_against(32)
    for bad, n in (([0, 15, 32], 32), ([3, 3], 8), ([], 8), ([-1, 2], 8)):
        with pytest.raises(ValueError):
            SSDConfig(draft_layers=bad).validate_against(n)


def test_drafting_level_sizes():
    assert DraftingConfig(depth=4, branch=[3, 2, 2, 1], width=8, max_nodes=24).level_sizes() == [3, 6, 8, 8]
    assert DraftingConfig(depth=6, branch=[4, 2, 2, 1, 1, 1]).level_sizes() == [4, 8, 16, 16, 16, 16]
    assert DraftingConfig(depth=4, branch=[3, 2, 2, 1], max_nodes=24).level_sizes() == [3, 6, 12, 12]


def test_checkpoint_paths_and_latest_order(tmp_path):
    from ssd.runtime import checkpoint_path, latest_checkpoint

    cfg = SSDConfig(draft_layers=[0, 7, 15])
    cfg.training.output_dir = str(tmp_path)
    assert checkpoint_path(cfg, 1) == tmp_path / "L0-7-15" / "stage1.pt"
    assert checkpoint_path(cfg, 2) == tmp_path / "L0-7-15" / "stage2.pt"
    assert checkpoint_path(cfg, "online") == tmp_path / "L0-7-15" / "online.pt"
    assert latest_checkpoint(cfg) is None
    (tmp_path / "L0-7-15").mkdir()
    for stage, expect in ((1, "stage1.pt"), (2, "stage2.pt"), ("online", "online.pt")):
        checkpoint_path(cfg, stage).write_bytes(b"")
        assert latest_checkpoint(cfg).name == expect
    checkpoint_path(cfg, "online").unlink()
    assert latest_checkpoint(cfg).name == "stage2.pt"


def _reference_layout_bridge(d, hidden, bias=True, mlp_type="mlp", num_layers=2):
    """A bridge built with plain torch modules in the reference's module tree
    (norm.weight; mlp.body.{0,2}.*, mlp.out_proj.*; or mlp.{gate,up,out}_proj.*)."""
    br = nn.Module()
    br.norm = nn.Module()
    br.norm.weight = nn.Parameter(torch.randn(d))
    br.mlp = nn.Module()
    if mlp_type == "mlp":
        dims = [d] + [hidden] * (num_layers - 1)
        mods = []
        for a, b in zip(dims[:-1], dims[1:]):
            mods += [nn.Linear(a, b, bias=bias), nn.SiLU()]
        br.mlp.body = nn.Sequential(*mods)
        br.mlp.out_proj = nn.Linear(hidden, d, bias=bias)
    else:
        br.mlp.gate_proj = nn.Linear(d, hidden, bias=bias)
        br.mlp.up_proj = nn.Linear(d, hidden, bias=bias)
        br.mlp.out_proj = nn.Linear(hidden, d, bias=bias)
    return br


@pytest.mark.parametrize("bcfg", [dict(), dict(num_layers=3, hidden_dim=96), dict(mlp_type="swiglu", bias=False)])
def test_bridge_checkpoint_format_loads(tmp_path, bcfg):
    from ssd.models.bridges import TransitionBridge

    d = 64
    cfg = BridgeConfig(**bcfg)
    hidden = cfg.hidden_dim or d
    torch.manual_seed(0)
    written = nn.ModuleDict({"into_7": _reference_layout_bridge(d, hidden, cfg.bias, cfg.mlp_type, cfg.num_layers),
                             "into_15": _reference_layout_bridge(d, hidden, cfg.bias, cfg.mlp_type, cfg.num_layers)})
    path = tmp_path / "L0-7-15" / "stage2.pt"
    path.parent.mkdir()
    torch.save({"layer_indices": [0, 7, 15], "bridge_config": vars(cfg), "state_dict": written.state_dict(),
                "meta": {"stage": 2, "step": 1000}}, path)
    ckpt = torch.load(path, map_location="cpu", weights_only=True)
    assert set(ckpt) == {"layer_indices", "bridge_config", "state_dict", "meta"}
    ours = nn.ModuleDict({k: TransitionBridge.from_config(d, BridgeConfig(**ckpt["bridge_config"]))
                          for k in ("into_7", "into_15")})
    ours.load_state_dict(ckpt["state_dict"], strict=True)
    for k, v in written.state_dict().items():
        assert torch.equal(ours.state_dict()[k], v), k
    # and the bridge computes x + MLP(RMSNorm(x)) with those weights
    x = torch.randn(3, d)
    b, w = ours["into_7"], written["into_7"]
    xf = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + cfg.norm_eps) * w.norm.weight
    if cfg.mlp_type == "mlp":
        ref = x + w.mlp.out_proj(w.mlp.body(xf))
    else:
        ref = x + w.mlp.out_proj(torch.nn.functional.silu(w.mlp.gate_proj(xf)) * w.mlp.up_proj(xf))
    torch.testing.assert_close(b(x), ref, atol=1e-5, rtol=1e-5)


def test_top_vocab_closed_form():
    from ssd.data.token_freq import top_vocab, token_freq_path, zipf_counts

    counts = torch.tensor([5, 9, 9, 1, 7, 0, 3])
    assert top_vocab(counts, 3).tolist() == [1, 2, 4]  # 9, 9 (stable: 1 before 2), 7
    assert top_vocab(counts, 3, always={5}).tolist() == [1, 2, 5]  # forced id replaces the last pick
    assert top_vocab(counts, 10).tolist() == list(range(7))
    z = zipf_counts(128256, 1.1, seed=0)
    ids = top_vocab(z, 32768)
    assert ids.numel() == 32768 and bool((ids[1:] > ids[:-1]).all())
    assert int(z[ids].min()) >= int(z[~torch.isin(torch.arange(128256), ids)].max())
    cfg = SSDConfig(draft_layers=[0, 1])
    cfg.training.output_dir = "outputs/x"
    assert str(token_freq_path(cfg)) == os.path.join("outputs", "x", "token_freq.pt")


def test_ssd_run_flags():
    from ssd.cli.run import parse

    a = parse(["--config", "c.yaml", "--prompt", "hi", "--mode", "target", "--max-new-tokens", "12", "--seed", "3",
               "--no-warmup", "--depth", "4", "--branch", "3,2,2,1", "--width", "8", "--max-nodes", "24",
               "--temperature", "0.7", "--top-p", "0.9", "--draft-vocab", "32768", "--untrained"])
    assert (a.mode, a.max_new_tokens, a.seed, a.no_warmup, a.depth, a.branch, a.width, a.max_nodes) == (
        "target", 12, 3, True, 4, [3, 2, 2, 1], 8, 24)
    assert (a.temperature, a.top_p, a.draft_vocab, a.untrained) == (0.7, 0.9, 32768, True)
    assert parse(["--config", "c.yaml", "--prompt-file", "p.txt", "--bridges", "b.pt"]).bridges == "b.pt"
    with pytest.raises(SystemExit):
        parse(["--config", "c.yaml", "--prompt", "a", "--bridges", "b.pt", "--untrained"])
    with pytest.raises(SystemExit):
        parse(["--config", "c.yaml"])


def test_selfdistill_resume_keeps_dataset_order(tmp_path):
    """The self-distillation loop (reference generate_selfdistill.py:134-178) with a stub generator:
    batches are formed from length-sorted chunks but rows land in dataset order; a run stopped by
    --tokens and resumed writes exactly the file of one uninterrupted run, skipping the written
    prompts and seeding with seed + rows done."""
    from ssd.data import generate_selfdistill as gs

    prompts = [(f"q{i}", [i] + [0] * ((i * 7) % 5)) for i in range(40)]
    seeds = []

    def fake_generate(target, batch, n, eos, T, top_p, pad, generator):
        seeds.append(generator.initial_seed())
        return [[p[0], len(p), 9] for p in batch]  # a reply depends on its prompt only

    kw = dict(batch_size=3, max_new_tokens=8, eos_ids=set(), temperature=0.7, top_p=0.9, pad_id=0, seed=5,
              decode=lambda toks: " ".join(map(str, toks)), generate=fake_generate)
    full = tmp_path / "full.jsonl"
    assert gs.write_selfdistill(None, iter(prompts), full, 10 ** 9, **kw) == (40, 120)
    assert seeds and set(seeds) == {5}
    rows = [json.loads(x) for x in full.read_text().splitlines()]
    assert [r["messages"][0]["content"] for r in rows] == [t for t, _ in prompts]
    assert [r["messages"][1]["content"] for r in rows] == [f"{i} {1 + (i * 7) % 5} 9" for i in range(40)]
    part = tmp_path / "part.jsonl"
    seeds.clear()
    done = gs.write_selfdistill(None, iter(prompts), part, 30, **kw)  # stops after the first chunk of 24
    assert done == (24, 72) and set(seeds) == {5}
    seeds.clear()
    assert gs.write_selfdistill(None, iter(prompts), part, 10 ** 9, **kw) == (40, 120)
    assert set(seeds) == {5 + 24}
    assert part.read_text() == full.read_text()


def test_selfdistill_iter_prompts_local_jsonl(tmp_path):
    """iter_prompts takes each example's first user turn, chat-formatted, and skips examples that
    start with another role or exceed max_prompt_tokens."""
    from ssd.config import SSDConfig
    from ssd.data.generate_selfdistill import iter_prompts

    data = tmp_path / "chat.jsonl"
    exs = [{"messages": [{"role": "user", "content": "hi there"}, {"role": "assistant", "content": "x"}]},
           {"messages": [{"role": "system", "content": "s"}, {"role": "user", "content": "no"}]},
           {"messages": []},
           {"messages": [{"role": "user", "content": "one two three four five six"}]},
           {"messages": [{"role": "user", "content": "ok"}]}]
    data.write_text("\n".join(json.dumps(e) for e in exs) + "\n")

    class Tok:
        def apply_chat_template(self, msgs, add_generation_prompt, return_dict):
            assert add_generation_prompt and return_dict and len(msgs) == 1
            return {"input_ids": [1] + [len(w) for w in msgs[0]["content"].split()] + [2]}

    cfg = SSDConfig()
    cfg.data.local_path = str(data)
    got = list(iter_prompts(cfg, Tok(), 5))
    assert got == [("hi there", [1, 2, 5, 2]), ("ok", [1, 2, 2])]
