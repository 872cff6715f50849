"""Speculative decoding loop and the autoregressive baseline (reference ssd/engine/speculative.py).

The target runs through ``SubnetworkDraftModel`` with every layer selected, the same kernels
as the draft; the baseline uses them too with one row per step, so the comparison is like
for like and greedy speculative output is bit-identical to greedy decoding (every kernel's
per-row arithmetic is independent of how many rows share a launch).

One round, all enqueued on the current HIP stream with no host round trip inside:
  draft   root forward -> draft head + log-softmax top-k (sampled: warp + Gumbel top-k)
          -> level expansion (x depth)
  verify  max_nodes cut + verify rows -> target forward -> argmax -> greedy acceptance
          (sampled: warp -> speculative-sampling walk)
  commit  KV compaction of the root + accepted path (one launch, all layers)
then a single device->host copy of the round record (committed tokens, tree size).
Phase times come from HIP events (no extra synchronisation); the reference's metric
definitions are kept: tokens/s = committed tokens / non-prefill time, ms/round per phase,
mean tokens committed per round.

Greedy rounds can be captured as a HIP graph and replayed (``graphs=True``). A round then has no
host-side position:
the root position lives in a device word that the round's first kernel advances by the previous
round's committed count, and every other position is read relative to it. One graph serves every
root position of a 256-position segment (attention bounds are fixed per segment, so its split into
shared and per-token superblocks is exact); the next segment is captured when the root reaches it.
The host keeps one round queued behind the one it reads, so the GPU never waits for the host.
Measured on the Llama-3-8B tree workload, a replayed round runs 5.65 ms on the GPU against 5.52 ms for
the same kernels launched one by one (an empty dependent launch does cost 1.7 us replayed against
2.5 us launched, but real kernels do not get that back), so plain launches stay the default.
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
from ssd.engine.sampling import Sampler
from ssd.engine.tree_drafter import TREE_CAP, DeviceTree, TreeDrafter
from ssd.models.subnetwork_draft import CHUNK, PREFILL_CHUNK, PREFILL_MIN, Rows, SubnetworkDraftModel


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
        """Adds up every closed phase; a phase still open (the last mark, when named) stays pending."""
        for (name, a), (_, b) in zip(self._pending, self._pending[1:]):
            if name is not None:
                self.totals[name] = self.totals.get(name, 0.0) + a.elapsed_time(b) / 1000.0
        self._pending = self._pending[-1:] if self._pending and self._pending[-1][0] is not None else []


def _prefill_logits(target: SubnetworkDraftModel, ids: list, cache: KVCache, ws) -> torch.Tensor:
    """Target forward over the prompt into ``cache`` (reference speculative.py:149-151); returns the
    last row's logits (a [1, V] view of a buffer the next forward reuses). Prompts of at least
    PREFILL_MIN tokens run on the MFMA prefill kernels (chunks of PREFILL_CHUNK rows), shorter
    ones as causal rows through the decode forward (chunks of 64)."""
    dev = target.model.device
    past = cache.get_seq_length()
    q = len(ids)
    cache.check_room(past + q)
    cache.ensure(target.num_kv_heads, target.head_dim, dev)
    logits = None
    if q >= PREFILL_MIN and target.prefill_capable():
        for c0 in range(0, q, PREFILL_CHUNK):
            c1 = min(q, c0 + PREFILL_CHUNK)
            logits = target.prefill_chunk(ids[c0:c1], past + c0, cache, c1 == q)
    else:
        rows = Rows(CHUNK, dev)
        for c0 in range(0, q, CHUNK):
            c1 = min(q, c0 + CHUNK)
            m = c1 - c0
            slots = list(range(past + c0, past + c1))
            rows.upload(ids[c0:c1], slots, slots, [s + 1 for s in slots], [0] * m)
            last = c1 == q
            logits = target.forward_rows(rows, m, past + c0 + 1, past + c1, cache, ws, m - 1 if last else 0,
                                         int(last))
            torch.cuda.current_stream().synchronize()  # the pinned staging buffer is reused next chunk
    ws.check_faults()
    cache.advance(q)
    return logits


def _prefill(target: SubnetworkDraftModel, ids: list, cache: KVCache, ws, out_dev: torch.Tensor,
             sampler: Optional[Sampler] = None) -> None:
    """Prefill and the first token into out_dev[0]: the first-index argmax of the last row, or with
    ``sampler`` a draw from its warped distribution with counter 0 (reference speculative.py:81-84)."""
    logits = _prefill_logits(target, ids, cache, ws)
    if sampler is not None:
        sampler.draw(logits, out_dev, counter=0)
    else:
        ops.row_topk(logits, 1, logits.shape[1], 1, 0, None, out_dev)


@torch.no_grad()
def autoregressive_generate(target: TargetRunner, input_ids: torch.Tensor, max_new_tokens: int, eos_ids: set,
                            temperature: float = 0.0, top_p: float = 1.0, seed: Optional[int] = None,
                            check_every: int = 16) -> GenerationResult:
    """Decoding with the target, one row per step (reference speculative.py:101-122): argmax, or
    with temperature > 0 a draw from the warped distribution (Philox counter = step, from
    ``seed``). Steps are enqueued back to back (the next step's input id is written on the
    device); the host checks EOS / length every ``check_every`` steps."""
    ids = torch.as_tensor(input_ids).reshape(-1).tolist()
    dev = target.model.device
    sampler = None
    if temperature != 0:
        sampler = Sampler(temperature, top_p, target.model.shape.vocab, dev, 0, 1, seed)
    n_prompt = len(ids)
    cache = target.new_cache(n_prompt + max_new_tokens + 1)
    ws = target.workspace(CHUNK)
    steps = max(max_new_tokens, 1)
    rows = Rows(steps, dev)
    times: dict = {}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    _prefill(target, ids, cache, ws, rows.ids[0:1], sampler)
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
            logits = target.forward_rows(rows.view(s), 1, n_prompt + s + 1, n_prompt + s + 1, cache, ws)
            if sampler is not None:
                sampler.draw(logits, rows.ids[s + 1:s + 2], counter=s + 1)
            else:
                ops.row_topk(logits, 1, logits.shape[1], 1, 0, None, rows.ids[s + 1:s + 2])
            s += 1
        cache.seq_len = n_prompt + s
        out = rows.ids[: s + 1].tolist()
        ws.check_faults()
    times["decode"] = time.perf_counter() - t0
    return GenerationResult(tokens=_finish(out, eos_ids, max_new_tokens)[0], times=times)


GRAPH_SEG = 256  # root positions one captured round serves (one attention superblock)


class DecodeSession:
    """One speculative decode stream on the device: buffers, cache and the round step.

    ``prefill(ids)`` runs the target over the prompt and returns the first token;
    ``step()`` runs one round (draft -> verify -> commit) with a single host synchronisation
    and returns the committed tokens. ``SpeculativeGenerator.generate`` is a loop over it.
    ``graphs`` (greedy decoding only, off by default) replays captured rounds instead of enqueuing
    every launch (the first round and rounds near the end of the cache run as plain launches).
    """

    def __init__(self, gen: "SpeculativeGenerator", capacity: int, seed: Optional[int] = None,
                 graphs: Optional[bool] = None):
        cfg, drafter, target, draft = gen.cfg, gen.drafter, gen.target, gen.draft
        self.cfg, self.drafter, self.target, self.draft = cfg, drafter, target, draft
        dev = target.model.device
        self.sampler = None
        if cfg.temperature != 0:
            self.sampler = Sampler(cfg.temperature, cfg.top_p, target.model.shape.vocab, dev,
                                   1 + drafter.max_tree_cache(), ROW_CAP_VERIFY, seed)
            self.sampler.max_kids = max(drafter.branch)
        self.cache = target.new_cache(capacity)
        self.ws = draft.workspace(CHUNK)
        self.root_rows, self.level_rows, self.verify_rows = Rows(CHUNK, dev), Rows(CHUNK, dev), Rows(CHUNK, dev)
        # [_, vn, n_new, tokens...], placed after the workspace's fused-MLP sync words so that the one
        # read-back per round also returns the MLP's timeout count (status_host[0])
        n_rec = 4 + cfg.depth + 2
        self.record = self.ws.record(n_rec)
        self.status = self.ws.status_span(n_rec)
        self.status_host = torch.zeros(self.status.numel(), dtype=torch.int32).pin_memory()
        self.record_host = self.status_host[self.status.numel() - n_rec:]
        self.tree = DeviceTree(dev, vmeta=self.record[1:2])
        self.cand_tok = torch.zeros(TREE_CAP, dtype=torch.int32, device=dev)
        self.cand_lp = torch.zeros(TREE_CAP, dtype=torch.float32, device=dev)
        self.argmax = torch.zeros(ROW_CAP_VERIFY, dtype=torch.int32, device=dev)
        # greedy verify: the head's per-slab argmax records (the head fused with its chunk pass)
        self.verify_parts = None if self.sampler is not None else torch.empty(
            ops.gemm_topk_bytes(ROW_CAP_VERIFY, self.target._head_n()), dtype=torch.uint8, device=dev)
        self.keep_src = torch.zeros(cfg.depth + 2, dtype=torch.int32, device=dev)
        self.n_keep = torch.zeros(1, dtype=torch.int32, device=dev)
        self.phases = _Phases()
        self.accepted_per_round: list = []
        self.tree_sizes: list = []
        self._begun = False  # the next round's first draft forward is already enqueued
        greedy = cfg.temperature == 0
        self.graphs = bool(graphs) and greedy
        self.pos_base = torch.zeros(1, dtype=torch.int32, device=dev)  # device root position (graph rounds)
        self._graph = None
        self._graph_seg, self._graph_hi = -1, -1
        self._queue: list = []  # graph rounds replayed but not read yet: (start, end event, pinned status)
        self._pinned = [torch.zeros_like(self.status_host).pin_memory() for _ in range(2)]
        self._slot = 0
        self.graph_rounds = 0
        self.captures = 0
        self.graph_launches = 0

    def prefill(self, ids: list) -> int:
        _prefill(self.target, ids, self.cache, self.ws, self.root_rows.ids[0:1], self.sampler)
        return int(self.root_rows.ids[0])

    def _begin(self, base: int, n_new_dev: Optional[torch.Tensor], counter: int) -> None:
        if self.sampler is not None:
            self.sampler.counter = counter
        self.phases.mark("draft")
        self.drafter.begin_device(self.cache, self.root_rows, base, self.tree, self.cand_tok, self.cand_lp, self.ws,
                                  self.sampler, n_new_dev)

    def step(self, lookahead: bool = True) -> list:
        """One round: a replayed graph round when possible (see the module docstring), otherwise the
        round's launches enqueued one by one. ``lookahead`` False: enqueue nothing of the next round
        before returning (a caller timing an exact number of rounds)."""
        if self.graphs and not self._begun and self.accepted_per_round:  # the first round warms up
            out = self._step_graph(lookahead)
            if out is not None:
                return out
        return self._step_eager(lookahead=lookahead and not self.graphs)

    # ------------------------------------------------------------------ graph rounds
    def _window(self, seg: int) -> tuple:
        """Root positions [lo, hi] a graph of segment ``seg`` serves: (root + 1) // GRAPH_SEG == seg, and
        every cache slot the round touches within capacity."""
        d = self.drafter
        room = max(d.max_verify_nodes() + 1, d.max_tree_cache() + 1, self.cfg.depth + 2)
        lo = seg * GRAPH_SEG - 1
        hi = min(lo + GRAPH_SEG - 1, self.cache.max_length - room)
        return lo, hi

    def _round_body(self, window: tuple) -> None:
        """One greedy round with positions relative to the device root position (captured)."""
        cfg, drafter, target, cache, ws = self.cfg, self.drafter, self.target, self.cache, self.ws
        lo, hi = window
        drafter.begin_device(cache, self.root_rows, 0, self.tree, self.cand_tok, self.cand_lp, ws, None,
                             self.record[2:3], pos_base=self.pos_base, window=window)
        drafter.levels_device(cache, 0, self.tree, self.level_rows, self.cand_tok, self.cand_lp, ws, None,
                              pos_base=self.pos_base, window=window)
        m = drafter.finalize_device(self.tree, 0, self.root_rows, self.verify_rows, pos_base=self.pos_base)
        cache.check_room(hi + m)
        self._verify_argmax(m, lo + 1, hi + 1 + cfg.depth)
        _lib.call("ssd_accept_greedy", self.tree.struct, self.argmax.data_ptr(), 0, self.record[2:].data_ptr(),
                  self.keep_src.data_ptr(), self.n_keep.data_ptr(), self.root_rows.ids.data_ptr(),
                  self.pos_base.data_ptr(), ops.stream())
        cache.compact_device(0, self.keep_src, self.n_keep, cfg.depth + 1, pos_base=self.pos_base)

    def _verify_argmax(self, m: int, p_min: int, l_max: int) -> None:
        """Target forward over the verify rows and each row's first-index argmax into self.argmax
        (greedy_verify, reference verify.py:45-57): the head runs fused with its top-k chunk pass
        (k = 1 over the bf16-rounded logits, ties to the lower column, as ssd_row_topk_bf16 on
        stored logits) and the records are merged, so the [m, V] logits are never written."""
        target, ws = self.target, self.ws
        target.forward_rows(self.verify_rows, m, p_min, l_max, self.cache, ws, head_rows=0)
        s = target.head_topk(ws.h, m, 1, self.verify_parts, mode=0)
        ops.row_topk_merge(self.verify_parts, m, s, 1, 0, None, self.argmax)

    def _capture(self, committed: int) -> bool:
        """Capture the round of the segment holding root position ``committed`` (nothing in flight).
        The device root position is set to ``committed`` with a zero committed count before it."""
        seg = (committed + 1) // GRAPH_SEG
        window = self._window(seg)
        if committed > window[1]:
            return False
        torch.cuda.synchronize()
        self.pos_base.fill_(committed)
        self.record[2:3].zero_()
        g = torch.cuda.CUDAGraph()
        n0 = int(_lib.load().ssd_launch_count())
        with torch.cuda.graph(g):
            self._round_body(window)
        self.graph_launches = int(_lib.load().ssd_launch_count()) - n0  # kernels in one replayed round
        self._graph, self._graph_seg, self._graph_hi = g, seg, window[1]
        self.captures += 1
        return True

    def _covers(self, root_hi: int) -> bool:
        return self._graph is not None and (root_hi + 1) // GRAPH_SEG == self._graph_seg and root_hi <= self._graph_hi

    def _replay(self) -> None:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        self._graph.replay()
        b.record()
        buf = self._pinned[self._slot]
        self._slot ^= 1
        buf.copy_(self.status, non_blocking=True)
        done = torch.cuda.Event()
        done.record()
        self._queue.append((a, b, done, buf))

    def _step_graph(self, lookahead: bool = True) -> Optional[list]:
        cache = self.cache
        committed = cache.get_seq_length()
        if not self._queue:
            if not self._covers(committed) and not self._capture(committed):
                return None
            self._replay()
        # one round queued behind this one when its root (at most depth + 1 further) stays covered
        if lookahead and len(self._queue) == 1 and self._covers(committed + self.cfg.depth + 1):
            self._replay()
        a, b, done, buf = self._queue.pop(0)
        done.synchronize()
        self.phases.totals["round"] = self.phases.totals.get("round", 0.0) + a.elapsed_time(b) / 1000.0
        ops.check_mlp_timeouts(int(buf[0]))
        rec = buf[buf.numel() - self.record_host.numel():]
        n_new = int(rec[2])
        new = rec[3:3 + n_new].tolist()
        cache.seq_len = committed + n_new
        self.accepted_per_round.append(n_new)
        self.tree_sizes.append(int(rec[1]))
        self.graph_rounds += 1
        return new

    def drain(self) -> None:
        """Wait for a graph round still queued (the lookahead past the last round read)."""
        if self._queue:
            self._queue[-1][2].synchronize()
            self._queue.clear()

    # ------------------------------------------------------------------ plain rounds
    def _step_eager(self, lookahead: bool = True) -> list:
        """One round. The round's first draft forward (root at the new committed length, read on
        the device) is enqueued for the next round before this one's result is read, so the GPU
        keeps working while the host reads the result and enqueues the rest."""
        cfg, drafter, target, cache, ws = self.cfg, self.drafter, self.target, self.cache, self.ws
        committed = cache.get_seq_length()
        ph = self.phases
        counter = len(self.accepted_per_round) + 1
        if not self._begun:
            self._begin(committed, None, counter)
        self._begun = False
        if self.sampler is not None:
            self.sampler.counter = counter
        drafter.levels_device(cache, committed, self.tree, self.level_rows, self.cand_tok, self.cand_lp, ws,
                              self.sampler)
        cache.crop(committed)
        ph.mark("verify")
        m = drafter.finalize_device(self.tree, committed, self.root_rows, self.verify_rows)
        cache.check_room(committed + m)
        if self.sampler is not None:
            logits = target.forward_rows(self.verify_rows, m, committed + 1, committed + 1 + cfg.depth, cache, ws)
            self.sampler.accept(self.tree, logits, m, committed, self.record[2:], self.keep_src, self.n_keep,
                                self.root_rows.ids)
        else:
            self._verify_argmax(m, committed + 1, committed + 1 + cfg.depth)
            _lib.call("ssd_accept_greedy", self.tree.struct, self.argmax.data_ptr(), committed,
                      self.record[2:].data_ptr(), self.keep_src.data_ptr(), self.n_keep.data_ptr(),
                      self.root_rows.ids.data_ptr(), None, ops.stream())
        ph.mark("bookkeeping")
        cache.compact_device(committed, self.keep_src, self.n_keep, cfg.depth + 1)
        self.status_host.copy_(self.status, non_blocking=True)
        ph.mark(None)
        done = torch.cuda.Event()
        done.record()
        hi = committed + cfg.depth + 1  # the next root position is at most this
        if lookahead and hi + 1 + drafter.max_tree_cache() <= cache.max_length:
            self._begin(committed, self.record[2:3], counter + 1)
            self._begun = True
        done.synchronize()
        ph.resolve()
        ops.check_mlp_timeouts(int(self.status_host[0]))
        n_new = int(self.record_host[2])
        new = self.record_host[3:3 + n_new].tolist()
        cache.seq_len = committed + n_new
        self.accepted_per_round.append(n_new)
        self.tree_sizes.append(int(self.record_host[1]))
        return new


class SpeculativeGenerator:
    def __init__(self, base: nn.Module, draft: SubnetworkDraftModel, cfg: DraftingConfig,
                 target: Optional[TargetRunner] = None):
        self.target = target or TargetRunner(base)
        self.draft = draft
        self.cfg = cfg
        self.drafter = TreeDrafter(draft, cfg)

    def capacity(self, n_prompt: int, max_new_tokens: int) -> int:
        """Cache slots for a generation; one round can overshoot max_new by depth+1 tokens and
        the draft/verify of the last round need their own room (reference speculative.py:145-147)."""
        extra = max(self.drafter.max_verify_nodes(), self.drafter.max_tree_cache()) + 1
        return n_prompt + max_new_tokens + self.cfg.depth + extra + 1

    def session(self, capacity: int, seed: Optional[int] = None, graphs: Optional[bool] = None) -> DecodeSession:
        return DecodeSession(self, capacity, seed, graphs)

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int, eos_ids: set, seed: Optional[int] = None,
                 max_rounds: Optional[int] = None, graphs: Optional[bool] = None) -> GenerationResult:
        ids = torch.as_tensor(input_ids).reshape(-1).tolist()
        sess = self.session(self.capacity(len(ids), max_new_tokens), seed, graphs)
        times: dict = {}
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        out = [sess.prefill(ids)]
        times["prefill"] = time.perf_counter() - t0
        t_dec = time.perf_counter()
        while not _finish(out, eos_ids, max_new_tokens)[1]:
            if max_rounds is not None and len(sess.accepted_per_round) >= max_rounds:
                break
            out.extend(sess.step())
        sess.drain()
        wall = time.perf_counter() - t_dec
        times.update(sess.phases.totals)
        # Host time between rounds (read-back, Python) is part of decode time, as in the reference.
        times["host"] = max(0.0, wall - sum(sess.phases.totals.values()))
        return GenerationResult(tokens=_finish(out, eos_ids, max_new_tokens)[0], times=times,
                                accepted_per_round=sess.accepted_per_round, tree_sizes=sess.tree_sizes)


ROW_CAP_VERIFY = 64
