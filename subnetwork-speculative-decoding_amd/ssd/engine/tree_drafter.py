"""Dynamic tree drafting with the sub-network draft, built on the device.

Same algorithm and API as the reference's ssd/engine/tree_drafter.py: feed the root; at
depth d every kept node proposes ``branch[d]`` children (top log-probs for greedy); the
``width[d]`` best by cumulative draft log-prob are kept and, unless d is the last depth,
fed through the draft in one batched forward where each attends to the committed prefix
and its own ancestors; finally the best ``max_nodes`` nodes go to verification.

Here every step of that loop is a kernel: the draft forward, the draft head, the proposals
(greedy: the log-softmax top-k's chunk pass ``ssd_row_topk_partial_bf16``, whose merge runs inside
the level launch ``ssd_tree_level_topk``; sampled drafts: the warp ``ssd_warp_probs_bf16`` and the
Gumbel top-k draw ``ssd_gumbel_topk``, then ``ssd_tree_level``), the level expansion / width cut /
next-level attention rows, then the max_nodes cut and the verify rows (``ssd_tree_finalize``). No
host round trip happens inside a round.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch

from ssd import _lib, ops
from ssd.config import DraftingConfig
from ssd.engine.kv_cache import KVCache

ROOT = -1
TREE_CAP = 1024
ROW_CAP = 64
TOPK_MAX = 16


def warp_probs(logits: torch.Tensor, temperature: float, top_p: float) -> torch.Tensor:
    """Temperature + nucleus warp (reference tree_drafter.py:34-45) of device logits [..., V]
    through ``ssd_warp_probs_bf16`` (logits are taken in bf16, the dtype the decode path
    produces); returns fp32 probabilities of the same shape. Equal probabilities at the nucleus
    boundary keep lower columns first."""
    V = logits.shape[-1]
    lg = logits.reshape(-1, V)
    rows = lg.shape[0]
    ld = (V + 7) // 8 * 8
    buf = torch.zeros(rows, ld, dtype=torch.bfloat16, device=logits.device)
    buf[:, :V] = lg
    out = torch.empty(rows, (V + 3) // 4 * 4, dtype=torch.float32, device=logits.device)
    ops.warp_probs(buf, rows, V, temperature, top_p, out)
    return out[:, :V].reshape(logits.shape)


@dataclass
class DraftTree:
    """Host view of a tree (reference tree_drafter.py:48-95)."""
    tokens: list = field(default_factory=list)
    parents: list = field(default_factory=list)
    depths: list = field(default_factory=list)
    scores: list = field(default_factory=list)
    ranks: list = field(default_factory=list)
    draft_pos: list = field(default_factory=list)
    child_q: dict = field(default_factory=dict)
    cache_start: int = 0

    def __len__(self) -> int:
        return len(self.tokens)

    def children(self) -> dict:
        out: dict = {}
        for i, p in enumerate(self.parents):
            out.setdefault(p, []).append(i)
        for kids in out.values():
            kids.sort(key=lambda i: self.ranks[i])
        return out

    def ancestors(self, i: int) -> list:
        path = []
        while i != ROOT:
            path.append(i)
            i = self.parents[i]
        return path[::-1]

    def subset(self, keep) -> "DraftTree":
        keep = sorted(keep)
        remap = {old: new for new, old in enumerate(keep)}
        remap[ROOT] = ROOT
        t = DraftTree(cache_start=self.cache_start)
        for old in keep:
            t.tokens.append(self.tokens[old])
            t.parents.append(remap[self.parents[old]])
            t.depths.append(self.depths[old])
            t.scores.append(self.scores[old])
            t.ranks.append(self.ranks[old])
            t.draft_pos.append(self.draft_pos[old])
        t.child_q = {remap[p]: q for p, q in self.child_q.items() if p in remap}
        return t


class DeviceTree:
    """Device buffers of one tree (include/ssd_mi355x.h SsdTree)."""

    def __init__(self, device, vmeta: Optional[torch.Tensor] = None, cap: int = TREE_CAP):
        i32 = dict(dtype=torch.int32, device=device)
        self.cap = cap
        self.buf = torch.zeros(11, cap, **i32)
        (self.tokens, self.parents, self.depths, self.ranks, self.draft_pos, self.vtokens, self.vparents,
         self.vdepths, self.vranks, self.vorig, _) = self.buf.unbind(0)
        self.scores = torch.zeros(cap, dtype=torch.float64, device=device)
        self.meta = torch.zeros(1 + 2 * 32, **i32)
        self.vmeta = vmeta if vmeta is not None else torch.zeros(1, **i32)
        p = lambda t: t.data_ptr()
        self.struct = _lib.SsdTree(p(self.tokens), p(self.parents), p(self.depths), p(self.ranks), p(self.draft_pos),
                                   p(self.scores), p(self.meta), p(self.vtokens), p(self.vparents), p(self.vdepths),
                                   p(self.vranks), p(self.vorig), p(self.vmeta), cap)

    def reset(self) -> None:
        self.meta.zero_()

    def to_host(self, sampler=None) -> DraftTree:
        """The finalized (verify) tree as a DraftTree (synchronises). With the sampler of a
        sampled draft, ``child_q`` maps every node with children (and the root) to the warped
        draft distribution they were drawn from (device rows over the full vocabulary)."""
        vn = int(self.vmeta[0])
        orig = self.vorig[:vn].long()
        t = DraftTree(tokens=self.vtokens[:vn].tolist(), parents=self.vparents[:vn].tolist(),
                      depths=self.vdepths[:vn].tolist(), scores=self.scores[orig].tolist(),
                      ranks=self.vranks[:vn].tolist(), draft_pos=self.draft_pos[orig].tolist())
        if sampler is not None:
            V = sampler.vocab
            for p in set(t.parents):
                t.child_q[p] = sampler.Q[0 if p == ROOT else 1 + int(orig[p]), :V]
        return t


class TreeDrafter:
    def __init__(self, draft, cfg: DraftingConfig):
        cfg.validate()
        self.draft, self.cfg = draft, cfg
        self.branch = cfg.per_depth(cfg.branch, "branch")
        self.width = cfg.per_depth(cfg.width, "width")
        self.greedy = cfg.temperature == 0
        self.levels = self.max_nodes_per_level()
        if max(self.branch) > TOPK_MAX:
            raise ValueError(f"drafting.branch entries must be <= {TOPK_MAX} (per-node top-k kernel limit)")
        if cfg.depth > 32:
            raise ValueError("drafting.depth must be <= 32 (ancestor lists hold 32 slots)")
        fed = self.levels[:-1]
        if fed and max(fed) > ROW_CAP:
            raise ValueError(f"a fed level has {max(fed)} nodes > {ROW_CAP}; set drafting.width")
        if sum(self.levels) > TREE_CAP or max([1] + fed) * max(self.branch) > TREE_CAP:
            raise ValueError(f"tree of {sum(self.levels)} nodes exceeds {TREE_CAP}")
        if self.max_verify_nodes() + 1 > ROW_CAP:
            raise ValueError(f"{self.max_verify_nodes()} verify nodes > {ROW_CAP - 1}; set drafting.max_nodes")
        # greedy proposals: the chunk records of the last proposal, merged by the next level's launch
        self._parts: Optional[torch.Tensor] = None
        self._parts_n = 0
        self._parts_s = 0
        # greedy proposals from the head launch itself (ssd_gemm_topk_bf16) where its records fit
        # the merge (records * k <= 1024); False: head logits, then ssd_row_topk_partial_bf16
        self.fused_head = True

    def max_nodes_per_level(self) -> list:
        return self.cfg.level_sizes()

    def max_tree_cache(self) -> int:
        """Draft-cache slots one round uses after the root (the last level is never fed)."""
        return sum(self.max_nodes_per_level()[:-1])

    def max_verify_nodes(self) -> int:
        total = sum(self.max_nodes_per_level())
        return min(total, self.cfg.max_nodes) if self.cfg.max_nodes else total

    # ------------------------------------------------------------------ device
    def _parts_buf(self, need: int, device) -> torch.Tensor:
        if self._parts is None or self._parts.numel() < need or self._parts.device != device:
            self._parts = torch.empty(need, dtype=torch.uint8, device=device)
        return self._parts

    def _uses_fused_head(self, d: int) -> bool:
        if not (self.greedy and self.fused_head and hasattr(self.draft, "head_topk")):
            return False
        return ops.gemm_topk_parts(self.draft._head_n()) * self.branch[d] <= 64 * TOPK_MAX

    def _forward_propose(self, rows, m: int, d: int, p_min: int, l_max: int, cache: KVCache, ws, tree: DeviceTree,
                         cand_tok, cand_lp, sampler) -> None:
        """Draft forward over ``m`` rows and the proposals of depth ``d`` from its head."""
        if self._uses_fused_head(d):
            # log-softmax top-k (tree_drafter.py:129-133 of the reference) in two halves: the chunk
            # pass in the head launch's epilogue, the merge inside the next level's expansion
            self.draft.forward_rows(rows, m, p_min, l_max, cache, ws, head_rows=0)
            n = self.draft._head_n()
            parts = self._parts_buf(ops.gemm_topk_bytes(max([1] + self.levels), n), ws.h.device)
            self._parts_s = self.draft.head_topk(ws.h, m, self.branch[d], parts)
            self._parts_n = n
            return
        logits = self.draft.forward_rows(rows, m, p_min, l_max, cache, ws)
        self._propose(logits, m, d, tree, cand_tok, cand_lp, sampler)

    def _propose(self, logits, rows: int, d: int, tree: DeviceTree, cand_tok, cand_lp, sampler) -> None:
        if self.greedy:
            # the same two halves from stored logits: the chunk pass here (4096-column chunks)
            n = logits.shape[1]
            parts = self._parts_buf(ops.row_topk_ws_bytes(max([1] + self.levels), n), logits.device)
            ops.row_topk_partial(logits, rows, n, self.branch[d], 1, parts)
            self._parts_n = n
            self._parts_s = (n + 4095) // 4096
        else:
            sampler.propose(self.draft, logits, rows, d, self.branch[d], tree.meta, cand_tok, cand_lp)

    def begin_device(self, cache: KVCache, root_rows, base_pos: int, tree: DeviceTree, cand_tok, cand_lp, ws,
                     sampler=None, n_new_dev: Optional[torch.Tensor] = None,
                     pos_base: Optional[torch.Tensor] = None, window: Optional[tuple] = None) -> None:
        """First part of the draft phase: empty tree, the root (token in ``root_rows.ids[0]``) fed
        at root_pos = base_pos + n_new_dev[0] (``n_new_dev`` None: base_pos), and the root's
        proposals. With ``n_new_dev`` the position is only read on the device, so this can be
        enqueued before the host has read the previous round; the root forward then gets bounds
        (root_pos is at most depth + 1 past base_pos) instead of the exact position.

        ``pos_base`` (a device int32 word holding the previous round's root position; base_pos is
        then 0) makes the round position-free on the host: the root position is pos_base +
        n_new_dev[0], stored back into pos_base for the round's other calls, and ``window`` =
        (lo, hi) bounds the root positions the call may see (attention bounds, room check)."""
        if not self.greedy and sampler is None:
            raise ValueError("sampled drafting needs a Sampler")
        if window is not None:
            lo, hi = window
        else:
            lo, hi = base_pos, base_pos + (self.cfg.depth + 1 if n_new_dev is not None else 0)
        cache.check_room(hi + 1 + self.max_tree_cache())
        _lib.call("ssd_round_begin", tree.struct, root_rows.struct, base_pos,
                  None if n_new_dev is None else n_new_dev.data_ptr(),
                  None if pos_base is None else pos_base.data_ptr(), ops.stream())
        self._forward_propose(root_rows, 1, 0, lo + 1, hi + 1, cache, ws, tree, cand_tok, cand_lp, sampler)

    def levels_device(self, cache: KVCache, root_pos: int, tree: DeviceTree, level_rows, cand_tok, cand_lp, ws,
                      sampler=None, pos_base: Optional[torch.Tensor] = None, window: Optional[tuple] = None) -> None:
        """Rest of the draft phase once root_pos is known on the host: every level's expansion /
        width cut and the forwards of the fed levels; leaves the unpruned tree in ``tree``. With
        ``pos_base`` root_pos is relative to that device word (0) and ``window`` bounds the root
        positions, as in begin_device."""
        lo, hi = window if window is not None else (root_pos, root_pos)
        tree_start = root_pos + 1
        cache.check_room(hi + 1 + self.max_tree_cache())
        past = tree_start
        pb = None if pos_base is None else pos_base.data_ptr()
        for d in range(self.cfg.depth):
            feed = d < self.cfg.depth - 1
            f_max = 1 if d == 0 else self.levels[d - 1]
            m = self.levels[d]
            if self.greedy:
                vocab_ids = self.draft._vocab_ids_i32
                _lib.call("ssd_tree_level_topk", tree.struct, d, self._parts.data_ptr(), self._parts.numel(),
                          self._parts_n, self._parts_s, None if vocab_ids is None else vocab_ids.data_ptr(), f_max,
                          self.branch[d],
                          self.width[d] or 0, int(feed), root_pos, tree_start, past, level_rows.struct,
                          m if feed else 0, pb, ops.stream())
            else:
                _lib.call("ssd_tree_level", tree.struct, d, cand_tok.data_ptr(), cand_lp.data_ptr(), f_max,
                          self.branch[d], self.width[d] or 0, int(feed), root_pos, tree_start, past,
                          level_rows.struct, m if feed else 0, pb, ops.stream())
            if not feed:
                break
            self._forward_propose(level_rows, m, d + 1, lo + 1, hi + 1 + d + 1, cache, ws, tree, cand_tok, cand_lp,
                                  sampler)
            past += m
        if pos_base is None:
            cache.seq_len = past

    def build_device(self, cache: KVCache, root_rows, root_pos: int, tree: DeviceTree, level_rows, cand_tok,
                     cand_lp, ws, sampler=None) -> None:
        """Enqueue the whole draft phase for the root held in ``root_rows.ids[0]``; leaves the
        unpruned tree in ``tree`` (no host synchronisation). Sampled drafting (temperature > 0)
        needs ``sampler`` (ssd.engine.sampling.Sampler): proposals are Gumbel top-k draws from
        the warped draft distribution, which is kept per node in ``sampler.Q``."""
        self.begin_device(cache, root_rows, root_pos, tree, cand_tok, cand_lp, ws, sampler)
        self.levels_device(cache, root_pos, tree, level_rows, cand_tok, cand_lp, ws, sampler)

    def finalize_device(self, tree: DeviceTree, committed: int, root_rows, verify_rows,
                        pos_base: Optional[torch.Tensor] = None) -> int:
        """max_nodes cut + verify rows; returns the verify row count used for the launch. With
        ``pos_base`` committed is relative to that device word."""
        rows = self.max_verify_nodes() + 1
        _lib.call("ssd_tree_finalize", tree.struct, self.cfg.max_nodes or 0, committed, root_rows.ids.data_ptr(),
                  verify_rows.struct, rows, None if pos_base is None else pos_base.data_ptr(), ops.stream())
        return rows

    # -------------------------------------------------------------- reference API
    @torch.no_grad()
    def build(self, cache: KVCache, pending: torch.Tensor, root_pos: int, generator=None) -> DraftTree:
        """Reference signature (tree_drafter.py:147-208): ``pending`` [1, n] committed tokens not
        yet in the cache (the last is the root at ``root_pos``). Returns the pruned tree."""
        from ssd.models.subnetwork_draft import Rows

        pend = torch.as_tensor(pending).reshape(-1).tolist()
        dev = self.draft.model.device
        if len(pend) > 1:  # earlier pending tokens go in first, as an ordinary causal chunk
            self.draft(torch.tensor([pend[:-1]]), torch.arange(root_pos - len(pend) + 1, root_pos)[None], cache,
                       compute_logits=False)
        ws = self.draft.workspace()
        root_rows, level_rows = Rows(ROW_CAP, dev), Rows(ROW_CAP, dev)
        root_rows.ids[:1].fill_(pend[-1])
        tree = DeviceTree(dev)
        cand_tok = torch.zeros(TREE_CAP, dtype=torch.int32, device=dev)
        cand_lp = torch.zeros(TREE_CAP, dtype=torch.float32, device=dev)
        sampler = None
        if not self.greedy:
            from ssd.engine.sampling import Sampler, seed_from_generator

            sampler = Sampler(self.cfg.temperature, self.cfg.top_p, self.draft.model.shape.vocab, dev,
                              1 + self.max_tree_cache(), 1, seed_from_generator(generator))
        self.build_device(cache, root_rows, root_pos, tree, level_rows, cand_tok, cand_lp, ws, sampler)
        verify_rows = Rows(ROW_CAP, dev)
        self.finalize_device(tree, root_pos, root_rows, verify_rows)
        out = tree.to_host(sampler)
        out.cache_start = root_pos + 1
        return out
