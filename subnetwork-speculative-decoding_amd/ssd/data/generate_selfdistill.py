"""Batched generation: many prompts continued by the target together (reference
ssd/data/generate_selfdistill.py:50-108, ``sample_next`` and ``generate_batch``).

The reference left-pads the prompts into one [B, T] batch with one shared cache, gives every row
its own positions and a 3-D mask hiding the padding, then decodes all rows in lock step. Here each
sequence owns a region of one KV arena ([B][layers][kv_heads][capacity * head_dim], the cache
block layout), so no padding exists: every prompt is prefilled into its own region (MFMA prefill
kernels for long prompts), and each decode step is one forward over the B rows (one per sequence,
chunks of 64) whose q/k/v GEMM writes and whose attention reads each row's own region (per-row
arena offsets, ``SsdRows.kv_off``). The weight-streaming GEMMs are shared by all rows; every row's
arithmetic is independent of the others, so a greedy batch reproduces greedy decoding of each
prompt alone bit for bit.

Sampling (temperature > 0) follows the reference's ``sample_next``: the 64 largest logits of each
row, the temperature + nucleus warp of those 64 alone, one categorical draw among them
(ssd_sample_top64_bf16: one launch finds each 4096-column chunk's 64 best, a second merges them and
draws; Philox keyed by (step, row)). The Philox seed is drawn from ``generator``, which advances it
as torch.multinomial would: successive calls with one generator draw independently, and a
generator seeded alike reproduces them.

The module also keeps the reference's command-line entry point (``python -m
ssd.data.generate_selfdistill --config ... --out data/x.jsonl --tokens N``, reference :110-178): prompts
are the first user turns of a chat dataset (``iter_prompts``; a local ``data.local_path`` .jsonl or the
``data.dataset`` split), generated in length-sorted batches and written in dataset order as
``{"messages": [user, assistant], "n_tokens": n}`` lines; a rerun resumes after the rows already in
the file, seeding with ``--seed`` + rows done.
"""
from __future__ import annotations

import argparse
import json
import logging
import time
from pathlib import Path
from typing import Callable, Iterable, Iterator, Optional

import torch

from ssd import ops
from ssd.engine.kv_cache import KVCache
from ssd.engine.sampling import seed_from_generator
from ssd.engine.speculative import TargetRunner, _prefill_logits
from ssd.models.subnetwork_draft import CHUNK, Rows


def sample_next(logits: torch.Tensor, temperature: float, top_p: float,
                generator: Optional[torch.Generator] = None) -> torch.Tensor:
    """[B, V] logits -> [B, 1] token ids (reference generate_selfdistill.py:50-60): the first-index
    argmax at temperature 0; otherwise, per row, the 64 largest logits (equal logits: lower column
    first), warp_probs over those 64 and one draw among them. Needs V >= 64 when sampling."""
    if logits.dim() != 2:
        raise ValueError("sample_next: logits must be [B, V]")
    B, V = logits.shape
    lg = logits if logits.dtype == torch.bfloat16 and logits.is_contiguous() and V % 8 == 0 else None
    if lg is None:
        lg = torch.zeros(B, (V + 7) // 8 * 8, dtype=torch.bfloat16, device=logits.device)
        lg[:, :V] = logits
    out = torch.zeros(B, dtype=torch.int32, device=logits.device)
    if temperature == 0:
        ops.row_topk(lg, B, V, 1, 0, None, out)
    else:
        if not temperature > 0:
            raise ValueError("sample_next: temperature must be >= 0")
        ops.sample_top64(lg, B, V, temperature, top_p, seed_from_generator(generator), 0, out)
    return out.long()[:, None]


@torch.no_grad()
def generate_batch(target: TargetRunner, prompts: list, max_new_tokens: int, eos_ids: set, temperature: float,
                   top_p: float, pad_id: int, generator: Optional[torch.Generator] = None,
                   check_every: int = 16) -> list:
    """Continue every prompt by up to ``max_new_tokens`` tokens; returns the new tokens of each,
    cut after the first EOS (inclusive). ``pad_id`` is accepted for the reference's signature; no
    padding is needed since each sequence has its own cache region."""
    model = target.model
    s, dev = model.shape, model.device
    B = len(prompts)
    if B == 0 or max_new_tokens <= 0:
        return [[] for _ in range(B)]
    lens = [len(p) for p in prompts]
    if min(lens) < 1:
        raise ValueError("generate_batch: empty prompt")
    cap = (max(lens) + max_new_tokens + 1 + 63) // 64 * 64
    shape = (B, s.layers, s.kv_heads, cap * s.head_dim)
    k_all = torch.zeros(shape, dtype=torch.bfloat16, device=dev)
    vt_all = torch.zeros(shape, dtype=torch.bfloat16, device=dev)
    per_seq = s.layers * s.kv_heads * cap * s.head_dim
    caches = []
    for b in range(B):
        c = KVCache(s.layers, cap)
        c.kv_heads, c.head_dim, c.device = s.kv_heads, s.head_dim, dev
        c.k, c.vt = k_all[b], vt_all[b]
        caches.append(c)
    ws = target.workspace(CHUNK)
    V = s.vocab
    ld = (V + 7) // 8 * 8
    sampled = temperature != 0
    if sampled and not temperature > 0:
        raise ValueError("generate_batch: temperature must be >= 0")
    seed = seed_from_generator(generator) if sampled else 0
    out = torch.zeros(max_new_tokens, B, dtype=torch.int32, device=dev)
    batch_logits = torch.zeros(B, ld, dtype=torch.bfloat16, device=dev) if sampled else None

    def choose(step: int, logits: torch.Tensor, c0: int, m: int) -> None:
        if not sampled:
            ops.row_topk(logits, m, V, 1, 0, None, out[step, c0:c0 + m])
        else:
            batch_logits[c0:c0 + m, :V].copy_(logits[:m, :V])

    def draw_all(step: int) -> None:
        if sampled:
            ops.sample_top64(batch_logits, B, V, temperature, top_p, seed, step, out[step])

    for b in range(B):  # each prompt into its own region; first token from its last row
        choose(0, _prefill_logits(target, list(prompts[b]), caches[b], ws), b, 1)
    draw_all(0)

    chunks = []
    for c0 in range(0, B, CHUNK):
        c1 = min(B, c0 + CHUNK)
        rows = Rows(CHUNK, dev)
        pos = lens[c0:c1]
        rows.upload(None, pos, pos, [p + 1 for p in pos], [0] * (c1 - c0))
        rows.set_kv_offsets(torch.arange(c0, c1, dtype=torch.int64, device=dev) * per_seq)
        chunks.append((c0, c1, rows))
    torch.cuda.current_stream().synchronize()  # the pinned staging buffers are reused by nothing else
    l_max = max(lens) + 1
    step = 0
    while step < max_new_tokens - 1:
        stop = min(max_new_tokens - 1, step + check_every)
        while step < stop:  # step s feeds token s, writes token s + 1
            for c0, c1, rows in chunks:
                m = c1 - c0
                rows.ids[:m].copy_(out[step, c0:c1])
                logits = target.forward_rows(rows, m, 0, l_max, caches[0], ws)
                choose(step + 1, logits, c0, m)
                rows._flat[rows.cap:4 * rows.cap].view(3, rows.cap)[:, :m] += 1  # pos, slot, prefix
            draw_all(step + 1)
            step += 1
            l_max += 1
        ws.check_faults()
        if eos_ids:
            eos = torch.tensor(sorted(eos_ids), device=dev)
            if bool(torch.isin(out[:step + 1], eos).any(0).all()):
                break
    rows_out = []
    for r in out[:step + 1].t().tolist():
        cut = next((i + 1 for i, t in enumerate(r) if t in eos_ids), len(r))
        rows_out.append(r[:cut])
    return rows_out


log = logging.getLogger("ssd")


def _examples(cfg) -> Iterator[dict]:
    if cfg.data.local_path:
        with open(cfg.data.local_path) as f:
            for line in f:
                if line.strip():
                    yield json.loads(line)
    else:
        from datasets import load_dataset  # streams from the hub: needs network access

        yield from load_dataset(cfg.data.dataset, split=cfg.data.split, streaming=True)


def iter_prompts(cfg, tokenizer, max_prompt_tokens: int) -> Iterator[tuple]:
    """(user text, chat-formatted prompt ids) for each example's first user turn (reference
    generate_selfdistill.py:38-47); examples whose first message is not the user's, or whose prompt
    is longer than ``max_prompt_tokens``, are skipped. Examples come from ``data.local_path`` (a .jsonl
    with a ``data.messages_field`` column) when set, else from the ``data.dataset`` split."""
    for ex in _examples(cfg):
        msgs = ex.get(cfg.data.messages_field) or []
        if not msgs or msgs[0].get("role") != "user":
            continue
        ids = tokenizer.apply_chat_template([msgs[0]], add_generation_prompt=True, return_dict=True)["input_ids"]
        if len(ids) <= max_prompt_tokens:
            yield msgs[0]["content"], list(ids)


def write_selfdistill(target, prompts: Iterable, out_path, tokens: int, batch_size: int, max_new_tokens: int,
                      eos_ids: set, temperature: float, top_p: float, pad_id: int, seed: int,
                      decode: Callable[[list], str], generate: Callable = generate_batch) -> tuple:
    """The generation loop of the reference's main (generate_selfdistill.py:134-178). Rows already in
    ``out_path`` are counted (rows and their ``n_tokens``) and that many prompts skipped, so a rerun
    resumes where the file ends; sampling is seeded with ``seed`` + rows done (a torch.Generator; the
    reference seeds the global generator the same way). Prompts are pulled batch_size * 8 at a time,
    generated in batches of similar length, and written in dataset order until ``tokens`` generated
    tokens are in the file. Returns (rows, tokens) in the file."""
    out_path = Path(out_path)
    out_path.parent.mkdir(parents=True, exist_ok=True)
    done_rows, done_tokens = 0, 0
    if out_path.exists():
        with open(out_path) as f:
            for line in f:
                done_rows += 1
                done_tokens += json.loads(line)["n_tokens"]
        log.info("resuming: %d rows / %d tokens already in %s", done_rows, done_tokens, out_path)
    generator = torch.Generator().manual_seed(seed + done_rows)
    it = iter(prompts)
    for _ in zip(range(done_rows), it):
        pass
    t0, new_tokens = time.perf_counter(), 0
    with open(out_path, "a") as f:
        while done_tokens < tokens:
            chunk = [x for _, x in zip(range(batch_size * 8), it)]
            if not chunk:
                break
            order = sorted(range(len(chunk)), key=lambda i: len(chunk[i][1]))  # similar lengths together
            results: dict = {}
            for s0 in range(0, len(order), batch_size):
                idx = order[s0:s0 + batch_size]
                rows = generate(target, [chunk[i][1] for i in idx], max_new_tokens, eos_ids, temperature, top_p,
                                pad_id, generator)
                results.update(zip(idx, rows))
            for i, (text, _) in enumerate(chunk):  # dataset order keeps a resume exact
                toks = results[i]
                f.write(json.dumps({"messages": [{"role": "user", "content": text},
                                                 {"role": "assistant", "content": decode(toks)}],
                                    "n_tokens": len(toks)}) + "\n")
                done_rows += 1
                done_tokens += len(toks)
                new_tokens += len(toks)
            f.flush()
            log.info("%d / %d tokens (%.0f tok/s)", done_tokens, tokens, new_tokens / (time.perf_counter() - t0))
    return done_rows, done_tokens


def main(argv: Optional[list] = None) -> None:
    """``python -m ssd.data.generate_selfdistill`` (reference generate_selfdistill.py:110-178)."""
    from ssd.config import SSDConfig
    from ssd.runtime import eos_ids_of, load_base_model, setup_env

    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--config", required=True)
    p.add_argument("--out", required=True)
    p.add_argument("--tokens", type=int, default=3_000_000,
                   help="stop after this many generated tokens (total, incl. resumed)")
    p.add_argument("--batch-size", type=int, default=32)
    p.add_argument("--max-new-tokens", type=int, default=384)
    p.add_argument("--max-prompt-tokens", type=int, default=384)
    p.add_argument("--temperature", type=float, default=0.7)
    p.add_argument("--top-p", type=float, default=0.9, help="applied within the top 64 tokens")
    p.add_argument("--seed", type=int, default=0)
    args = p.parse_args(argv)

    setup_env()
    cfg = SSDConfig.from_yaml(args.config)
    if not Path(cfg.model.base_model).is_dir():
        raise FileNotFoundError("self-distillation needs a local checkpoint directory with its tokenizer "
                                f"(model.base_model = {cfg.model.base_model!r})")
    from transformers import AutoTokenizer

    tokenizer = AutoTokenizer.from_pretrained(cfg.model.base_model, local_files_only=True)
    base = load_base_model(cfg)
    target = TargetRunner(base)
    pad_id = tokenizer.convert_tokens_to_ids("<|finetune_right_pad_id|>")
    write_selfdistill(target, iter_prompts(cfg, tokenizer, args.max_prompt_tokens), args.out, args.tokens,
                      args.batch_size, args.max_new_tokens, eos_ids_of(base), args.temperature, args.top_p, pad_id,
                      args.seed, lambda toks: tokenizer.decode(toks, skip_special_tokens=True))


if __name__ == "__main__":
    main()
