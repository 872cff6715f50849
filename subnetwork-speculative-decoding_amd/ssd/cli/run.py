"""ssd-run: speculative decoding (``--mode sd``) or the target alone (``--mode target``).

Same flags and stats as the reference (ssd/cli/run.py:45-135). Prompts come from a local
tokenizer when ``model.base_model`` is a local checkpoint directory; for ``synthetic:<shape>``
models give token ids (``--prompt-ids 1,2,3``) or ``--random-prompt N`` (uniform ids,
seeded by ``--seed``).

    python -m ssd.cli.run --config configs/llama3_8b_subnetwork.yaml --synthetic llama3_8b \
        --random-prompt 4096 --depth 4 --branch 3,2,2,1 --max-nodes 24 --untrained
"""

from __future__ import annotations

import argparse
import logging
from dataclasses import replace

import torch

from ssd.config import SSDConfig, profile_name
from ssd.engine.speculative import SpeculativeGenerator, TargetRunner, autoregressive_generate
from ssd.runtime import build_draft, eos_ids_of, load_base_model, setup_env

log = logging.getLogger("ssd")


def _int_or_list(s: str):
    parts = [int(x) for x in s.split(",")]
    return parts[0] if len(parts) == 1 else parts


def parse(argv=None):
    p = argparse.ArgumentParser(prog="ssd-run", description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--config", required=True)
    g = p.add_mutually_exclusive_group(required=True)
    g.add_argument("--prompt")
    g.add_argument("--prompt-file")
    g.add_argument("--prompt-ids", help="comma-separated token ids")
    g.add_argument("--random-prompt", type=int, help="N uniform random token ids (seeded by --seed)")
    p.add_argument("--synthetic", help="random-init model of a named shape instead of model.base_model")
    p.add_argument("--mode", choices=["sd", "target"], default="sd")
    p.add_argument("--max-new-tokens", type=int, default=256)
    p.add_argument("--raw", action="store_true", help="don't wrap the prompt in the chat template")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--no-warmup", action="store_true")
    t = p.add_argument_group("tree overrides (default: config `drafting:`)")
    t.add_argument("--depth", type=int)
    t.add_argument("--branch", type=_int_or_list)
    t.add_argument("--width", type=_int_or_list)
    t.add_argument("--max-nodes", type=int)
    t.add_argument("--temperature", type=float)
    t.add_argument("--top-p", type=float)
    t.add_argument("--draft-vocab", type=int, help="0 = full vocab")
    b = p.add_mutually_exclusive_group()
    b.add_argument("--bridges")
    b.add_argument("--untrained", action="store_true")
    return p.parse_args(argv)


def main(argv=None):
    args = parse(argv)
    setup_env()
    cfg = SSDConfig.from_yaml(args.config)
    if args.synthetic:
        cfg.model.base_model = f"synthetic:{args.synthetic}"
    over = {k: getattr(args, k) for k in ("depth", "branch", "width", "max_nodes", "temperature", "top_p",
                                          "draft_vocab") if getattr(args, k) is not None}
    if over.get("draft_vocab") == 0:
        over["draft_vocab"] = None
    dcfg = replace(cfg.drafting, **over)
    dcfg.validate()
    cfg.drafting = dcfg
    base = load_base_model(cfg, seed=args.seed)
    tokenizer = None
    if args.prompt_ids:
        ids = torch.tensor([[int(x) for x in args.prompt_ids.split(",")]])
    elif args.random_prompt:
        ids = torch.randint(0, base.shape.vocab, (1, args.random_prompt),
                            generator=torch.Generator().manual_seed(args.seed + 1))
    else:
        from transformers import AutoTokenizer

        tokenizer = AutoTokenizer.from_pretrained(cfg.model.base_model, local_files_only=True)
        text = args.prompt if args.prompt is not None else open(args.prompt_file).read()
        if not args.raw and tokenizer.chat_template:
            ids = tokenizer.apply_chat_template([{"role": "user", "content": text}], add_generation_prompt=True,
                                                return_tensors="pt", return_dict=True)["input_ids"]
        else:
            ids = tokenizer(text, return_tensors="pt")["input_ids"]
    eos = eos_ids_of(base)
    target = TargetRunner(base)
    draft = None
    if args.mode == "sd":
        draft = build_draft(cfg, base, None if args.untrained else (args.bridges or "latest"), inference=True)
    L = base.shape.layers
    print(f"\nprompt: {ids.shape[1]} tokens | device: {base.device} | draft layers "
          f"{profile_name(cfg.draft_layers)} ({len(cfg.draft_layers)}/{L})")
    print(f"tree: depth={dcfg.depth} branch={dcfg.branch} width={dcfg.width} max_nodes={dcfg.max_nodes} "
          f"temperature={dcfg.temperature} top_p={dcfg.top_p} draft_vocab={dcfg.draft_vocab or 'full'}")

    def run_ar(n):
        return autoregressive_generate(target, ids, n, eos, dcfg.temperature, dcfg.top_p, args.seed)

    if not args.no_warmup:
        run_ar(8)
        if args.mode == "sd":
            SpeculativeGenerator(base, draft, dcfg, target).generate(ids, 8, eos, seed=args.seed)
    ar = run_ar(args.max_new_tokens)
    ar_tps = len(ar.tokens) / ar.decode_time
    decode = (lambda toks: tokenizer.decode(toks, skip_special_tokens=True)) if tokenizer else str
    if args.mode == "target":
        print(f"\n=== target: {len(ar.tokens)} tokens, {ar_tps:.1f} tok/s ===")
        print(decode(ar.tokens))
        return
    sd = SpeculativeGenerator(base, draft, dcfg, target).generate(ids, args.max_new_tokens, eos, seed=args.seed)
    sd_tps = len(sd.tokens) / sd.decode_time
    rounds = len(sd.accepted_per_round)
    print(f"\n=== speculative: {len(sd.tokens)} tokens ===")
    print(decode(sd.tokens))
    print("\n--- stats (decode phase; prefill excluded) ---")
    print(f"rounds:                {rounds}")
    print(f"accepted tokens/round: {sd.mean_accepted:.2f}   (incl. bonus; max {dcfg.depth + 1})")
    print(f"mean tree size:        {sum(sd.tree_sizes) / max(1, rounds):.1f} nodes")
    acc = [n - 1 for n in sd.accepted_per_round]
    parts = []
    for d in range(1, dcfg.depth + 1):
        reached = sum(a >= d - 1 for a in acc)
        if reached:
            parts.append(f"d{d}={sum(a >= d for a in acc) / reached:.0%}")
    print("accept rate by depth:  " + "  ".join(parts) + "   (given all shallower depths accepted)")
    per = {k: 1000 * v / max(1, rounds) for k, v in sd.times.items() if k != "prefill"}
    print("per round:             " + "  ".join(f"{k}={v:.2f}ms" for k, v in per.items()))
    print(f"target step (AR):      {1000 * ar.decode_time / max(1, len(ar.tokens) - 1):.2f}ms/token")
    print(f"throughput:            AR {ar_tps:.1f} tok/s  |  SD {sd_tps:.1f} tok/s  |  speedup {sd_tps / ar_tps:.2f}x")
    if dcfg.temperature == 0:
        n = min(len(ar.tokens), len(sd.tokens))
        print(f"greedy output identical to AR: {ar.tokens[:n] == sd.tokens[:n]}")


if __name__ == "__main__":
    main()
