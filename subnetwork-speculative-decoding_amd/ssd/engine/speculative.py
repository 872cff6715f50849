"""Speculative decoding loop and the autoregressive baseline (reference ssd/engine/speculative.py).

The target runs through ``SubnetworkDraftModel`` with every layer selected, the same kernels
as the draft; the baseline uses them too with one row per step, so the comparison is like
for like and greedy speculative output is bit-identical to greedy decoding (every kernel's
per-row arithmetic is independent of how many rows share a launch).

One round, all enqueued on the current HIP stream with no host round trip inside:
  draft   root forward -> draft head + log-softmax top-k -> level expansion (x depth)
  verify  max_nodes cut + verify rows -> target forward -> argmax -> greedy acceptance
  commit  KV compaction of the root + accepted path (one launch, all layers)
then a single device->host copy of the round record (committed tokens, tree size).
Phase times come from HIP events (no extra synchronisation); the reference's metric
definitions are kept: tokens/s = committed tokens / non-prefill time, ms/round per phase,
mean tokens committed per round.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Optional

import torch
import torch.nn as nn

from ssd import _lib, ops
from ssd.config import DraftingConfig
from ssd.engine.kv_cache import KVCache
from ssd.engine.tree_drafter import TREE_CAP, DeviceTree, TreeDrafter
from ssd.models.subnetwork_draft import CHUNK, Rows, SubnetworkDraftModel


@dataclass
class GenerationResult:
    tokens: list
    times: dict  # seconds per phase
    accepted_per_round: list = field(default_factory=list)
    tree_sizes: list = field(default_factory=list)

    @property
    def decode_time(self) -> float:
        return sum(v for k, v in self.times.items() if k != "prefill")

    @property
    def mean_accepted(self) -> float:
        return sum(self.accepted_per_round) / max(1, len(self.accepted_per_round))


def _finish(tokens: list, eos_ids: set, max_new: int):
    for i, t in enumerate(tokens[:max_new]):
        if t in eos_ids:
            return tokens[: i + 1], True
    return tokens[:max_new], len(tokens) >= max_new


class TargetRunner(SubnetworkDraftModel):
    """The full target through the draft's layer implementation (reference speculative.py:94-99)."""

    def __init__(self, base: nn.Module):
        from ssd.models.subnetwork_draft import as_device_model

        super().__init__(base, list(range(as_device_model(base).shape.layers)))


class _Phases:
    """HIP-event phase timer: events are recorded on the stream between phases and resolved
    after the round's one synchronisation (no extra host syncs inside a round)."""

    def __init__(self):
        self.totals: dict = {}
        self._pending: list = []

    def mark(self, name: Optional[str]) -> None:
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        self._pending.append((name, ev))

    def resolve(self) -> None:
        for (name, a), (_, b) in zip(self._pending, self._pending[1:]):
            if name is not None:
                self.totals[name] = self.totals.get(name, 0.0) + a.elapsed_time(b) / 1000.0
        self._pending = []


def _prefill(target: SubnetworkDraftModel, ids: list, cache: KVCache, ws, out_dev: torch.Tensor) -> None:
    """Target forward over the prompt (chunks of 64 causal rows) and the first-index argmax of
    the last row into out_dev[0] (reference speculative.py:149-151, :81-84)."""
    dev = target.model.device
    rows = Rows(CHUNK, dev)
    past = cache.get_seq_length()
    q = len(ids)
    cache.check_room(past + q)
    hn = ws.x
    for c0 in range(0, q, CHUNK):
        c1 = min(q, c0 + CHUNK)
        m = c1 - c0
        slots = list(range(past + c0, past + c1))
        rows.upload(ids[c0:c1], slots, slots, [s + 1 for s in slots], [0] * m)
        h = target.run_rows(rows, m, past + c0 + 1, past + c1, cache, ws)
        if c1 == q:
            target.final_norm(h[m - 1:], 1, hn)
        torch.cuda.current_stream().synchronize()
    cache.advance(q)
    logits = target.head(hn, 1, ws)
    ops.row_topk(logits, 1, logits.shape[1], 1, 0, None, out_dev)


@torch.no_grad()
def autoregressive_generate(target: TargetRunner, input_ids: torch.Tensor, max_new_tokens: int, eos_ids: set,
                            temperature: float = 0.0, top_p: float = 1.0, seed: Optional[int] = None,
                            check_every: int = 16) -> GenerationResult:
    """Greedy decoding with the target, one row per step (reference speculative.py:101-122).
    Steps are enqueued back to back (the next step's input id is the previous step's argmax,
    written on the device); the host checks EOS / length every ``check_every`` steps."""
    if temperature != 0:
        raise NotImplementedError("sampled autoregressive decoding is not part of this build yet")
    ids = torch.as_tensor(input_ids).reshape(-1).tolist()
    dev = target.model.device
    n_prompt = len(ids)
    cache = target.new_cache(n_prompt + max_new_tokens + 1)
    ws = target.workspace(CHUNK)
    steps = max(max_new_tokens, 1)
    rows = Rows(steps, dev)
    times: dict = {}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    _prefill(target, ids, cache, ws, rows.ids[0:1])
    torch.cuda.synchronize()
    times["prefill"] = time.perf_counter() - t0
    # Step s feeds generated token s at position n_prompt + s.
    slots = [n_prompt + s for s in range(steps)]
    rows.upload(None, slots, slots, [s + 1 for s in slots], [0] * steps)
    t0 = time.perf_counter()
    s = 0
    out = rows.ids[:1].tolist()
    while not _finish(out, eos_ids, max_new_tokens)[1] and s < steps - 1:
        stop = min(steps - 1, s + check_every)
        while s < stop:  # step s feeds token s, writes token s + 1
            h = target.run_rows(rows.view(s), 1, n_prompt + s + 1, n_prompt + s + 1, cache, ws)
            logits = target.head(target.final_norm(h, 1, ws.x), 1, ws)
            ops.row_topk(logits, 1, logits.shape[1], 1, 0, None, rows.ids[s + 1:s + 2])
            s += 1
        cache.seq_len = n_prompt + s
        out = rows.ids[: s + 1].tolist()
    times["decode"] = time.perf_counter() - t0
    return GenerationResult(tokens=_finish(out, eos_ids, max_new_tokens)[0], times=times)


class SpeculativeGenerator:
    def __init__(self, base: nn.Module, draft: SubnetworkDraftModel, cfg: DraftingConfig,
                 target: Optional[TargetRunner] = None):
        self.target = target or TargetRunner(base)
        self.draft = draft
        self.cfg = cfg
        self.drafter = TreeDrafter(draft, cfg)

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int, eos_ids: set, seed: Optional[int] = None,
                 max_rounds: Optional[int] = None) -> GenerationResult:
        cfg, drafter, target, draft = self.cfg, self.drafter, self.target, self.draft
        if cfg.temperature != 0:
            raise NotImplementedError("sampling speculative decoding is not part of this build yet")
        dev = target.model.device
        ids = torch.as_tensor(input_ids).reshape(-1).tolist()
        n_prompt = len(ids)
        extra = max(drafter.max_verify_nodes(), drafter.max_tree_cache()) + 1
        cache = target.new_cache(n_prompt + max_new_tokens + cfg.depth + extra + 1)
        ws = draft.workspace(CHUNK)
        root_rows, level_rows, verify_rows = Rows(CHUNK, dev), Rows(CHUNK, dev), Rows(CHUNK, dev)
        record = torch.zeros(4 + cfg.depth + 2, dtype=torch.int32, device=dev)  # [_, vn, n_new, tokens...]
        record_host = torch.zeros_like(record, device="cpu").pin_memory()
        tree = DeviceTree(dev, vmeta=record[1:2])
        cand_tok = torch.zeros(TREE_CAP, dtype=torch.int32, device=dev)
        cand_lp = torch.zeros(TREE_CAP, dtype=torch.float32, device=dev)
        argmax = torch.zeros(ROW_CAP_VERIFY, dtype=torch.int32, device=dev)
        keep_src = torch.zeros(cfg.depth + 2, dtype=torch.int32, device=dev)
        n_keep = torch.zeros(1, dtype=torch.int32, device=dev)

        times: dict = {}
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        _prefill(target, ids, cache, ws, root_rows.ids[0:1])
        first = int(root_rows.ids[0])
        times["prefill"] = time.perf_counter() - t0
        out = [first]
        result = GenerationResult(tokens=[], times=times)
        phases = _Phases()
        t_dec = time.perf_counter()
        while not _finish(out, eos_ids, max_new_tokens)[1]:
            if max_rounds is not None and len(result.accepted_per_round) >= max_rounds:
                break
            committed = cache.get_seq_length()
            phases.mark("draft")
            drafter.build_device(cache, root_rows, committed, tree, level_rows, cand_tok, cand_lp, ws)
            cache.crop(committed)
            phases.mark("verify")
            m = drafter.finalize_device(tree, committed, root_rows, verify_rows)
            cache.check_room(committed + m)
            h = target.run_rows(verify_rows, m, committed + 1, committed + 1 + cfg.depth, cache, ws)
            logits = target.head(target.final_norm(h, m, ws.x), m, ws)
            ops.row_topk(logits, m, logits.shape[1], 1, 0, None, argmax)
            _lib.call("ssd_accept_greedy", tree.struct, argmax.data_ptr(), committed, record[2:].data_ptr(),
                      keep_src.data_ptr(), n_keep.data_ptr(), root_rows.ids.data_ptr(), ops.stream())
            phases.mark("bookkeeping")
            cache.compact_device(committed, keep_src, n_keep, cfg.depth + 1)
            record_host.copy_(record, non_blocking=True)
            phases.mark(None)
            torch.cuda.current_stream().synchronize()
            phases.resolve()
            n_new = int(record_host[2])
            new = record_host[3:3 + n_new].tolist()
            cache.seq_len = committed + n_new
            out.extend(new)
            result.accepted_per_round.append(n_new)
            result.tree_sizes.append(int(record_host[1]))
        wall = time.perf_counter() - t_dec
        times.update(phases.totals)
        # Host time between rounds (read-back, Python) is part of decode time, as in the reference.
        times["host"] = max(0.0, wall - sum(phases.totals.values()))
        result.tokens = _finish(out, eos_ids, max_new_tokens)[0]
        return result


ROW_CAP_VERIFY = 64
