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
"""

from __future__ import annotations

from typing import Optional

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
