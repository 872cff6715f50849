"""Draft model = a frozen subset of the target's layers joined by bridges, on gfx950 kernels.

API of the reference's ``SubnetworkDraftModel`` (ssd/models/subnetwork_draft.py:101-357):
``forward(input_ids, position_ids, past_key_values, tree_attention_mask, logits_to_keep,
compute_logits, ...) -> DraftOutput``, ``new_cache``, ``set_vocab_subset``, bridge
planning/placement, ``save_bridges``/``load_bridges``. With every layer selected it is the
target (``TargetRunner``), exactly as in the reference.

Each forward runs, per selected layer: [bridge] -> RMSNorm -> fused q/k/v GEMM with RoPE
and the KV-cache write in its epilogue -> tree attention (+ split combine) -> o GEMM with
the residual add in its epilogue -> RMSNorm -> gate/up GEMM with SwiGLU in its epilogue ->
down GEMM with the residual add. Then [pre-norm bridge] -> RMSNorm -> lm_head GEMM (full
vocabulary, or the draft-vocab subset). Every step is a hand-written HIP kernel; torch
only owns the buffers.

Attention rows: a dense boolean mask (True = attend) is turned into per-row
(prefix length, ancestor slots) -- the reference's masks always have that shape: an
all-true committed prefix plus each node's own ancestors (subnetwork_draft.py:165-191).
"""

from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field
from typing import Optional

import torch
import torch.nn as nn

from ssd import _lib, ops
from ssd.config import BridgeConfig, validate_layer_indices
from ssd.engine.kv_cache import KVCache
from ssd.models.bridges import TransitionBridge
from ssd.models.llama import MI355XLlama

MAXD = 32        # ancestors per row (ssd_attn_max_depth)
CHUNK = 64       # rows per kernel launch chain (GEMM column tiles of 16 x 4)
PREFILL_MIN = 256     # causal prompt chunks at least this long run on the MFMA prefill kernels
PREFILL_CHUNK = 4096  # prompt rows per ssd_prefill call


@dataclass
class BridgeSpec:
    name: str
    src_boundary: int
    tgt_boundary: int


@dataclass
class DraftOutput:
    logits: Optional[torch.Tensor]
    hidden_states: torch.Tensor
    past_key_values: Optional[KVCache]
    bridge_states: dict = field(default_factory=dict)
    vocab_ids: Optional[torch.Tensor] = None
    layer_inputs: dict = field(default_factory=dict)


def plan_bridges(layer_indices: list, num_base_layers: int) -> list:
    """Boundary i = residual stream entering base layer i (L = the final norm). A bridge maps
    the boundary the draft has to the one the next selected module expects, wherever layers
    are skipped (reference subnetwork_draft.py:61-73)."""
    specs, have = [], 0
    for idx in layer_indices:
        if idx != have:
            specs.append(BridgeSpec(f"into_{idx}", have, idx))
        have = idx + 1
    if have != num_base_layers:
        specs.append(BridgeSpec("into_norm", have, num_base_layers))
    return specs


def required_boundaries(layer_indices: list, num_base_layers: int) -> set:
    return {b for s in plan_bridges(layer_indices, num_base_layers) for b in (s.src_boundary, s.tgt_boundary)}


def as_device_model(base) -> MI355XLlama:
    """Accept our device model or an HF LlamaForCausalLM (packed once, cached on the object)."""
    if isinstance(base, MI355XLlama):
        return base
    cached = getattr(base, "_ssd_mi355x", None)
    if cached is None:
        dev = torch.device("cuda", torch.cuda.current_device())
        cached = MI355XLlama.from_hf(base, dev)
        base._ssd_mi355x = cached
    return cached


class Rows:
    """Device buffers describing the rows of one forward (include/ssd_mi355x.h SsdRows)."""

    def __init__(self, cap: int, device):
        self.cap = cap
        self._pinned = torch.zeros(5 * cap + cap * MAXD, dtype=torch.int32, pin_memory=True)
        self._flat = torch.zeros(5 * cap + cap * MAXD, dtype=torch.int32, device=device)
        self.ids = self._flat[0:cap]
        self.pos = self._flat[cap:2 * cap]
        self.slot = self._flat[2 * cap:3 * cap]
        self.prefix = self._flat[3 * cap:4 * cap]
        self.depth = self._flat[4 * cap:5 * cap]
        self.anc = self._flat[5 * cap:].view(cap, MAXD)
        self.struct = _lib.SsdRows(self.ids.data_ptr(), self.pos.data_ptr(), self.slot.data_ptr(),
                                   self.prefix.data_ptr(), self.depth.data_ptr(), self.anc.data_ptr(), cap)

    def set_kv_offsets(self, offsets: Optional[torch.Tensor]) -> None:
        """Per-row element offsets of each row's sequence in the KV arenas (int64 device tensor of
        length >= rows, kept alive here), or None: rows of several sequences in one forward."""
        self.kv_off = offsets
        self.struct.kv_off = offsets.data_ptr() if offsets is not None else None

    def view(self, off: int) -> "_RowsView":
        """Rows [off, cap) as a forward's rows (pointer offsets, no copy)."""
        v = _RowsView(self.ids[off:], self.pos[off:], self.slot[off:], self.prefix[off:], self.depth[off:],
                      self.anc[off:])
        v.struct = _lib.SsdRows(v.ids.data_ptr(), v.pos.data_ptr(), v.slot.data_ptr(), v.prefix.data_ptr(),
                                v.depth.data_ptr(), v.anc.data_ptr(), self.cap - off)
        kv_off = getattr(self, "kv_off", None)
        if kv_off is not None:  # rows of several sequences: the view keeps each row's arena offset
            v.kv_off = kv_off[off:]
            v.struct.kv_off = v.kv_off.data_ptr()
        return v

    def upload(self, ids, pos, slot, prefix, depth, anc=None) -> None:
        """Fill rows [0, n) from host lists with one pinned async copy (the pinned staging buffer
        is reused, so callers synchronise between uploads; the engine does, once per round)."""
        n = len(pos)
        if n > self.cap:
            raise ValueError(f"{n} rows > capacity {self.cap}")
        c = self.cap
        p = self._pinned
        if ids is not None:
            p[0:n] = torch.as_tensor(ids, dtype=torch.int32)
        p[c:c + n] = torch.as_tensor(pos, dtype=torch.int32)
        p[2 * c:2 * c + n] = torch.as_tensor(slot, dtype=torch.int32)
        p[3 * c:3 * c + n] = torch.as_tensor(prefix, dtype=torch.int32)
        p[4 * c:4 * c + n] = torch.as_tensor(depth, dtype=torch.int32)
        if anc is not None:
            a = p[5 * c:].view(c, MAXD)
            for r, lst in enumerate(anc):
                if lst:
                    a[r, :len(lst)] = torch.as_tensor(lst, dtype=torch.int32)
        if ids is None:  # keep device ids (e.g. produced by a kernel)
            self._flat[c:].copy_(p[c:], non_blocking=True)
        else:
            self._flat.copy_(p, non_blocking=True)


@dataclass
class _RowsView:
    ids: torch.Tensor
    pos: torch.Tensor
    slot: torch.Tensor
    prefix: torch.Tensor
    depth: torch.Tensor
    anc: torch.Tensor
    struct: Optional[_lib.SsdRows] = None
    kv_off: Optional[torch.Tensor] = None


class Workspace:
    """Activation buffers for forwards of up to ``m_cap`` rows."""

    def __init__(self, model: MI355XLlama, m_cap: int, bridge_hidden: int = 0):
        s, dev = model.shape, model.device
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.m_cap = m_cap
        self.h = torch.zeros(m_cap, s.hidden, **bf)
        self.x = torch.zeros(m_cap, s.hidden, **bf)
        self.q = torch.zeros(m_cap, s.heads * s.head_dim, **bf)
        self.attn = torch.zeros(m_cap, s.heads * s.head_dim, **bf)
        self.mlp = torch.zeros(m_cap, s.inter, **bf)
        bh = max(bridge_hidden, 32)
        self.mids = [torch.zeros(m_cap, bh, **bf), torch.zeros(m_cap, bh, **bf)]
        # split-K partials of the largest GEMM that writes them (q/k/v, o, down, bridge out_proj)
        n_qkv = (s.heads + 2 * s.kv_heads) * s.head_dim
        shapes = [(n_qkv, s.hidden), (s.hidden, s.heads * s.head_dim), (s.hidden, s.inter), (s.hidden, bh)]
        self.part = torch.zeros(max([ops.partial_floats(m_cap, n, k) for n, k in shapes]
                                    + [ops.residual_floats(m_cap, n, k) for n, k in shapes]), dtype=torch.float32,
                                device=dev)
        self.ws = torch.zeros(0, dtype=torch.float32, device=dev)
        self.logits = torch.zeros(0, **bf)
        # The fused MLP's flag words, followed by RECORD_WORDS words for the decode loop's per-round
        # record, so that one device->host copy returns the record and the MLP's timeout count.
        n_sync = ops.mlp_sync_words()
        self.status = torch.zeros(n_sync + self.RECORD_WORDS, dtype=torch.int32, device=dev)
        self.sync = self.status[:n_sync]
        self.timeout_word = ops.mlp_timeout_word()
        self._native: dict = {}

    RECORD_WORDS = 64

    def record(self, n: int) -> torch.Tensor:
        """The n-word round record (n <= RECORD_WORDS) that follows the sync words, zeroed."""
        if n > self.RECORD_WORDS:
            raise ValueError(f"record of {n} words > {self.RECORD_WORDS}")
        r = self.status[self.sync.numel():self.sync.numel() + n]
        r.zero_()
        return r

    def status_span(self, n: int) -> torch.Tensor:
        """Words [timeout word, end of an n-word record): what the decode loop copies back."""
        return self.status[self.timeout_word:self.sync.numel() + n]

    def check_faults(self) -> None:
        """Raises SsdError when a fused-MLP flag wait gave up on this workspace (synchronises)."""
        ops.check_mlp_timeouts(int(self.status[self.timeout_word]))

    def clear_faults(self) -> None:
        self.status[self.timeout_word] = 0

    def attn_ws(self, model: MI355XLlama, max_len: int) -> torch.Tensor:
        s = model.shape
        n = ops.attn_workspace_floats(self.m_cap, s.heads, s.head_dim, max_len)
        if self.ws.numel() < n:
            self.ws = torch.zeros(n, dtype=torch.float32, device=model.device)
        return self.ws

    def logits_buf(self, m: int, n: int) -> torch.Tensor:
        ld = (n + 7) // 8 * 8
        if self.logits.numel() < m * ld:
            self.logits = torch.zeros(max(m, self.m_cap) * ld, dtype=torch.bfloat16, device=self.h.device)
        return self.logits[: m * ld].view(m, ld)

    def native(self, model: MI355XLlama, cache: KVCache, n: int):
        """(SsdBuffers, logits [m_cap, ld]) for ssd_forward over these buffers, ``cache``'s arena and
        a head of ``n`` columns. Descriptors are cached per (arena, logits, workspace) pointers."""
        ld = (n + 7) // 8 * 8
        if self.logits.numel() < self.m_cap * ld:
            self.logits = torch.zeros(self.m_cap * ld, dtype=torch.bfloat16, device=self.h.device)
        aws = self.attn_ws(model, cache.capacity)
        key = (cache.k.data_ptr(), cache.vt.data_ptr(), cache.capacity, ld, self.logits.data_ptr(), aws.data_ptr())
        st = self._native.get(key)
        if st is None:
            if len(self._native) >= 8:
                self._native.pop(next(iter(self._native)))
            st = _lib.SsdBuffers(self.h.data_ptr(), self.x.data_ptr(), self.q.data_ptr(), self.attn.data_ptr(),
                                 self.mlp.data_ptr(), self.mids[0].data_ptr(), self.mids[1].data_ptr(), self.m_cap,
                                 self.mids[0].shape[1], cache.k.data_ptr(), cache.vt.data_ptr(), cache.capacity,
                                 aws.data_ptr(), aws.numel(), self.logits.data_ptr(), ld, self.part.data_ptr(),
                                 self.part.numel(), self.sync.data_ptr())
            self._native[key] = st
        return st, self.logits[: self.m_cap * ld].view(self.m_cap, ld)


class PrefillWorkspace:
    """Activation buffers of ssd_prefill for prompt chunks of up to ``m_cap`` rows."""

    def __init__(self, model: MI355XLlama, m_cap: int):
        s, dev = model.shape, model.device
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.m_cap = m_cap
        self.h = torch.zeros(m_cap, s.hidden, **bf)
        self.q = torch.zeros(m_cap, s.heads * s.head_dim, **bf)
        self.attn = torch.zeros(m_cap, s.heads * s.head_dim, **bf)
        self.act = torch.zeros(m_cap, s.inter, **bf)
        self.ids = torch.zeros(m_cap, dtype=torch.int32, device=dev)
        self.logits = torch.zeros(1, s.vocab, **bf)
        self._native: dict = {}

    def native(self, cache: KVCache) -> "_lib.SsdPrefillBuffers":
        key = (cache.k.data_ptr(), cache.vt.data_ptr(), cache.capacity)
        st = self._native.get(key)
        if st is None:
            if len(self._native) >= 8:
                self._native.pop(next(iter(self._native)))
            st = _lib.SsdPrefillBuffers(self.m_cap, self.h.data_ptr(), self.q.data_ptr(), self.attn.data_ptr(),
                                        self.act.data_ptr(), cache.k.data_ptr(), cache.vt.data_ptr(), cache.capacity,
                                        self.logits.data_ptr())
            self._native[key] = st
        return st


class _BaseRefs:
    """Plain holder so base weights are never registered as draft parameters."""

    def __init__(self, model: MI355XLlama, layer_indices: list):
        self.model = model
        self.layers = [model.layers[i] for i in layer_indices]
        self.embed_tokens = model.embed
        self.norm = model.norm
        self.lm_head = model.lm_head


class SubnetworkDraftModel(nn.Module):
    def __init__(self, base_model, layer_indices: list, bridge_config: Optional[BridgeConfig] = None,
                 freeze_base: bool = True):
        super().__init__()
        model = as_device_model(base_model)
        s = model.shape
        self.num_base_layers = s.layers
        self.layer_indices = validate_layer_indices(layer_indices, s.layers)
        self.d_model, self.num_heads, self.num_kv_heads, self.head_dim = s.hidden, s.heads, s.kv_heads, s.head_dim
        self.bridge_config = bridge_config or BridgeConfig()
        self.base = _BaseRefs(model, self.layer_indices)
        self.bridge_specs = plan_bridges(self.layer_indices, s.layers)
        by_tgt = {b.tgt_boundary: b.name for b in self.bridge_specs}
        self._pre_layer_bridge = [by_tgt.get(i) for i in self.layer_indices]
        self._pre_norm_bridge = by_tgt.get(s.layers)
        self.bridges = nn.ModuleDict({b.name: TransitionBridge.from_config(self.d_model, self.bridge_config)
                                      for b in self.bridge_specs})
        self.vocab_ids: Optional[torch.Tensor] = None
        self._vocab_ids_i32: Optional[torch.Tensor] = None
        self._vocab_inv: Optional[torch.Tensor] = None
        self._sub_head: Optional[torch.Tensor] = None
        self._ws: Optional[Workspace] = None
        self._pw: Optional[PrefillWorkspace] = None
        self._plan = None

    # ------------------------------------------------------------------ setup
    @property
    def model(self) -> MI355XLlama:
        return self.base.model

    @property
    def num_layers(self) -> int:
        return len(self.layer_indices)

    def set_vocab_subset(self, token_ids: Optional[torch.Tensor]) -> None:
        """Score only ``token_ids`` (sorted ascending) in this model's lm_head: a packed copy of
        those rows (|subset| x d) streamed by the same GEMM (reference :136-144)."""
        if token_ids is None:
            self.vocab_ids = self._sub_head = self._vocab_ids_i32 = self._vocab_inv = None
            return
        ids = token_ids.to(self.model.device).long()
        self.vocab_ids = ids
        self._vocab_ids_i32 = ids.to(torch.int32)
        # token -> subset column (-1 outside): the sampling warp zeroes q outside the subset
        inv = torch.full((self.model.shape.vocab,), -1, dtype=torch.int32, device=ids.device)
        inv[ids] = torch.arange(ids.numel(), dtype=torch.int32, device=ids.device)
        self._vocab_inv = inv
        self._sub_head = ops.pack_weight(self.model.lm_head_rows(ids))

    def place_bridges(self) -> None:
        """Single-GPU build: bridges run where the base weights live."""
        self.bridges.to(self.model.device)

    def new_cache(self, max_length: int) -> KVCache:
        s = self.model.shape
        return KVCache(s.layers, max_length, s.kv_heads, s.head_dim, self.model.device)

    def workspace(self, m_cap: int = CHUNK) -> Workspace:
        bh = max([b.hidden for b in self.bridges.values()] + [0])
        if self._ws is None or self._ws.m_cap < m_cap or self._ws.mids[0].shape[1] < bh:
            self._ws = Workspace(self.model, m_cap, bh)
        return self._ws

    def prefill_capable(self) -> bool:
        """The full target (every layer in order, no bridges) at shapes the prefill kernels take."""
        s = self.model.shape
        return (self.layer_indices == list(range(s.layers)) and not self.bridge_specs and s.head_dim in (64, 128)
                and s.hidden % 64 == 0 and s.inter % 64 == 0 and (s.heads * s.head_dim) % 64 == 0)

    def prefill_chunk(self, ids: list, pos0: int, cache: KVCache, logits: bool) -> Optional[torch.Tensor]:
        """ssd_prefill over prompt rows pos0 .. pos0 + len(ids) - 1 (at most PREFILL_CHUNK): K/V
        of every layer into the cache, the final residual stream in the prefill workspace's h, and
        with ``logits`` the last row's full-vocabulary logits ([1, V] view)."""
        m = len(ids)
        if m > PREFILL_CHUNK:
            raise ValueError(f"prefill chunk of {m} rows > {PREFILL_CHUNK}")
        pw = self._pw
        if pw is None or pw.m_cap < m:
            pw = self._pw = PrefillWorkspace(self.model, max(m, min(PREFILL_CHUNK, 1024)))
        pw.ids[:m].copy_(torch.tensor(ids, dtype=torch.int32))
        _lib.call("ssd_prefill", self.model.native(cache.capacity), self.model.lm_head.data_ptr() if logits else None,
                  pw.native(cache), pw.ids.data_ptr(), m, int(pos0), ops.stream())
        return pw.logits if logits else None

    def _packed_bridge(self, name: str):
        br = self.bridges[name]
        if br._packed is None and br.norm.weight.device != self.model.device:
            br.to(self.model.device)
        return br.packed(self.model.device)

    # ------------------------------------------------------- device forward
    def native_plan(self) -> "_lib.SsdPlan":
        """C descriptor (SsdPlan): selected layers, their bridges and the head; rebuilt when a
        bridge is repacked or the vocabulary subset changes."""
        pre = [self._packed_bridge(n) if n is not None else None for n in self._pre_layer_bridge]
        post = self._packed_bridge(self._pre_norm_bridge) if self._pre_norm_bridge is not None else None
        head = self._sub_head if self._sub_head is not None else self.model.lm_head
        key = (tuple(id(b) for b in pre), id(post), head.data_ptr())
        if self._plan is None or self._plan[0] != key:
            n = len(self.layer_indices)
            ids = (ctypes.c_int32 * n)(*self.layer_indices)
            BP = ctypes.POINTER(_lib.SsdBridgeW)
            natives = [b.native() if b is not None else None for b in pre]
            arr = (BP * n)(*[ctypes.pointer(x) if x is not None else BP() for x in natives])
            st = _lib.SsdPlan(n, ids, arr if any(natives) else None,
                              ctypes.pointer(post.native()) if post is not None else None, head.data_ptr(),
                              self._head_n())
            self._plan = (key, st, ids, arr, pre, post)
        return self._plan[1]

    def _head_n(self) -> int:
        return int(self.vocab_ids.numel()) if self._sub_head is not None else self.model.shape.vocab

    def forward_rows(self, rows, m: int, p_min: int, l_max: int, cache: KVCache, ws: Workspace,
                     head_first: int = 0, head_rows: Optional[int] = None) -> Optional[torch.Tensor]:
        """One ssd_forward call over rows [0, m) on the device: embedding, the selected layers and
        bridges (final residual stream in ws.h) and the head, with the final norm folded, over rows
        [head_first, head_first + head_rows) (default all). Returns the bf16 logits view
        [head_rows, n] (None if no rows)."""
        if head_rows is None:
            head_rows = m
        n = self._head_n()
        buf, logits = ws.native(self.model, cache, n)
        _lib.call("ssd_forward", self.model.native(cache.capacity), self.native_plan(), buf, rows.struct, m,
                  int(p_min), int(l_max), head_first, head_rows, ops.stream())
        return logits[:head_rows, :n] if head_rows else None

    def run_rows(self, rows: Rows, m: int, p_min: int, l_max: int, cache: KVCache, ws: Workspace,
                 bridge_states: Optional[dict] = None, ids_ready: bool = True) -> torch.Tensor:
        """The kernels of ssd_forward called one by one from Python, in the same order (used when
        bridge states are requested). Leaves the final residual stream in ws.h[:m] and returns it."""
        if m > ws.m_cap:
            raise ValueError(f"{m} rows > workspace {ws.m_cap}")
        model, s = self.model, self.model.shape
        cos, sin = model.rope(cache.capacity)
        aws = ws.attn_ws(model, cache.capacity)
        part = ws.part
        ops.embed(rows.ids, m, model.embed, ws.h)
        for slot, layer in enumerate(self.base.layers):
            li = self.layer_indices[slot]
            name = self._pre_layer_bridge[slot]
            if name is not None:
                self._packed_bridge(name).apply_(ws.h, m, ws.mids, part)
                if bridge_states is not None:
                    bridge_states[name] = ws.h[:m].clone()
            kc, vt = cache.layer(li)
            ops.qkv_rope(ws.h, m, layer.wqkv, s.hidden, s.heads, s.kv_heads, s.head_dim, cos, sin, rows.pos, rows.slot,
                         ws.q, kc, vt, cache.capacity, norm_eps=s.eps)
            ops.tree_attention(ws.q, m, s.heads, s.kv_heads, s.head_dim, kc, vt, cache.capacity, rows.prefix,
                               rows.depth, rows.anc, p_min, l_max, aws, ws.attn)
            ops.gemm_residual(ws.attn, m, layer.wo, s.hidden, s.heads * s.head_dim, ws.h, part)
            if layer.mlp_fused:
                ops.mlp(ws.h, m, layer.wgu, layer.wd, s.inter, s.hidden, s.eps, ws.mlp, part, ws.sync)
                continue
            ops.gemm_swiglu(ws.h, m, layer.wgu, s.inter, s.hidden, ws.mlp, norm_eps=s.eps)
            ops.gemm_residual(ws.mlp, m, layer.wd, s.hidden, s.inter, ws.h, part)
        if self._pre_norm_bridge is not None:
            self._packed_bridge(self._pre_norm_bridge).apply_(ws.h, m, ws.mids, part)
            if bridge_states is not None:
                bridge_states[self._pre_norm_bridge] = ws.h[:m].clone()
        return ws.h

    def head(self, h: torch.Tensor, m: int, ws: Workspace) -> torch.Tensor:
        """lm_head (or the vocab-subset head) over the final residual stream h[:m], final norm
        folded -> bf16 logits view [m, V]."""
        n = self._head_n()
        w = self._sub_head if self._sub_head is not None else self.model.lm_head
        out = ws.logits_buf(m, n)
        ops.gemm(h, m, w, n, self.d_model, out, norm_eps=self.model.shape.eps)
        return out[:, :n]

    def head_topk(self, h: torch.Tensor, m: int, k: int, parts: torch.Tensor, mode: int = 1) -> int:
        """The head over h[:m] (final norm folded) fused with its top-k chunk pass: ``parts`` gets
        each row's per-slab records (k best keys, max, sum of exp) for a merge; the logits are not
        stored. Returns the record count per row."""
        n = self._head_n()
        w = self._sub_head if self._sub_head is not None else self.model.lm_head
        return ops.gemm_topk(h, m, w, n, self.d_model, k, mode, parts, norm_eps=self.model.shape.eps)

    def final_norm(self, h: torch.Tensor, m: int, out: torch.Tensor) -> torch.Tensor:
        return ops.rmsnorm(h, m, self.model.norm, self.model.shape.eps, out)

    # ---------------------------------------------------------- generic API
    @staticmethod
    def mask_to_rows(q_len: int, past: int, mask: Optional[torch.Tensor]):
        """Reference mask semantics (subnetwork_draft.py:165-191) -> per-row (prefix, ancestors)."""
        if mask is None:
            if q_len == 1:
                return [past + 1], [[]]
            return [past + t + 1 for t in range(q_len)], [[] for _ in range(q_len)]
        mk = mask.detach().to("cpu", torch.bool)
        while mk.dim() > 2:
            if mk.shape[0] != 1:
                raise ValueError("batch size 1 only")
            mk = mk[0]
        if mk.shape[-1] == past + q_len and past > 0:
            full = mk
        else:
            if tuple(mk.shape[-2:]) != (q_len, q_len):
                raise ValueError(f"tree_attention_mask must be [.., {q_len}, {q_len}], got {tuple(mk.shape)}")
            full = torch.cat([torch.ones(q_len, past, dtype=torch.bool), mk], 1)
        prefix, anc = [], []
        for t in range(q_len):
            row = full[t]
            off = torch.nonzero(~row).flatten()
            p = int(off[0]) if off.numel() else int(row.numel())
            rest = (torch.nonzero(row[p:]).flatten() + p).tolist()
            if len(rest) > MAXD:
                raise ValueError(f"row {t} attends {len(rest)} non-prefix slots (max {MAXD})")
            if p == 0 and not rest:
                raise ValueError(f"row {t} attends nothing")
            prefix.append(p)
            anc.append(rest)
        return prefix, anc

    def forward(self, input_ids: Optional[torch.Tensor] = None, position_ids: Optional[torch.Tensor] = None,
                past_key_values: Optional[KVCache] = None, tree_attention_mask: Optional[torch.Tensor] = None,
                inputs_embeds: Optional[torch.Tensor] = None, logits_to_keep: int = 0, compute_logits: bool = True,
                output_bridge_states: bool = False, true_layer_inputs: Optional[dict] = None,
                output_layer_inputs: Optional[set] = None) -> DraftOutput:
        if true_layer_inputs is not None or output_layer_inputs:
            raise NotImplementedError("training-mode inputs are outside the decode path")
        if inputs_embeds is not None:
            raise NotImplementedError("inputs_embeds: pass token ids")
        ids = torch.as_tensor(input_ids)
        if ids.dim() == 1:
            ids = ids[None]
        if ids.shape[0] != 1:
            raise ValueError("batch size 1 only (speculative decoding is batch 1)")
        ids = ids[0].tolist()
        q = len(ids)
        cache = past_key_values
        if cache is None:
            cache = self.new_cache(q)
        cache.ensure(self.num_kv_heads, self.head_dim, self.model.device)
        past = cache.get_seq_length()
        cache.check_room(past + q)
        pos = list(range(past, past + q)) if position_ids is None else torch.as_tensor(position_ids).reshape(-1).tolist()
        prefix, anc = self.mask_to_rows(q, past, tree_attention_mask)
        ws = self.workspace(CHUNK)
        rows = Rows(CHUNK, self.model.device)
        hraw = torch.empty(q, self.d_model, dtype=torch.bfloat16, device=self.model.device)
        states: dict = {} if output_bridge_states else None
        causal = tree_attention_mask is None and pos == list(range(past, past + q))
        if causal and states is None and q >= PREFILL_MIN and self.prefill_capable():
            # a long causal prompt: the MFMA prefill kernels, PREFILL_CHUNK rows per call
            for c0 in range(0, q, PREFILL_CHUNK):
                c1 = min(q, c0 + PREFILL_CHUNK)
                self.prefill_chunk(ids[c0:c1], past + c0, cache, False)
                hraw[c0:c1].copy_(self._pw.h[:c1 - c0])
            q_done = q
        else:
            q_done = 0
        for c0 in range(q_done, q, CHUNK):
            c1 = min(q, c0 + CHUNK)
            seen = [a for lst in anc[c0:c1] for a in lst] + [p - 1 for p in prefix[c0:c1]]
            if max(seen) >= past + c1:
                raise ValueError("a row attends a slot written by a later chunk")
            rows.upload(ids[c0:c1], pos[c0:c1], list(range(past + c0, past + c1)), prefix[c0:c1],
                        [len(a) for a in anc[c0:c1]], anc[c0:c1])
            m = c1 - c0
            p_min = min(prefix[c0:c1])
            l_max = max(p + len(a) for p, a in zip(prefix[c0:c1], anc[c0:c1]))
            if states is None:
                self.forward_rows(rows, m, p_min, l_max, cache, ws, head_rows=0)
            else:
                self.run_rows(rows, m, p_min, l_max, cache, ws, states)
            hraw[c0:c1].copy_(ws.h[:m])
            torch.cuda.current_stream().synchronize()  # the pinned staging buffer is reused next chunk
        ws.check_faults()
        cache.advance(q)
        # hidden_states = the final-normed rows (reference :343); the decode path never needs
        # them (its head folds the norm), so they are computed here only
        hidden = torch.empty_like(hraw)
        for c0 in range(0, q, CHUNK):
            self.final_norm(hraw[c0:c0 + CHUNK], min(CHUNK, q - c0), hidden[c0:c0 + CHUNK])
        logits = None
        if compute_logits:
            keep = hraw[-logits_to_keep:] if logits_to_keep > 0 else hraw
            outs = []
            for c0 in range(0, keep.shape[0], CHUNK):
                part = keep[c0:c0 + CHUNK]
                outs.append(self.head(part, part.shape[0], ws).clone())
            logits = torch.cat(outs, 0)[None]
        return DraftOutput(logits=logits, hidden_states=hidden[None], past_key_values=past_key_values,
                           bridge_states={k: v[None] for k, v in (states or {}).items()},
                           vocab_ids=self.vocab_ids if compute_logits else None)

    # ------------------------------------------------------------ persistence
    def save_bridges(self, path: str, **meta) -> None:
        """Same file format as the reference (subnetwork_draft.py:455-466)."""
        os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
        torch.save({"layer_indices": self.layer_indices, "bridge_config": vars(self.bridge_config),
                    "state_dict": self.bridges.state_dict(), "meta": meta}, path)

    def load_bridges(self, path: str, strict: bool = True) -> None:
        ckpt = torch.load(path, map_location="cpu", weights_only=True)
        if list(ckpt["layer_indices"]) != self.layer_indices:
            raise ValueError(f"checkpoint layer_indices {ckpt['layer_indices']} != {self.layer_indices}")
        self.bridges.load_state_dict(ckpt["state_dict"], strict=strict)
        for b in self.bridges.values():
            b._packed = None
