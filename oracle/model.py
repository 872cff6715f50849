"""CPU restatement of the reference's model forward (test infrastructure only).

Follows, op for op and cast for cast:

* ``ssd/models/subnetwork_draft.py:249-357`` (``SubnetworkDraftModel.forward``):
  embed -> [bridge] -> selected layers -> [pre-norm bridge] -> norm -> lm_head
  (or the vocab-subset head, ``:345-349``);
* ``ssd/models/subnetwork_draft.py:193-246`` (``_layer_forward``): RMSNorm ->
  q/k/v -> RoPE -> cache write -> masked GQA attention -> o_proj + residual ->
  RMSNorm -> SwiGLU MLP + residual;
* ``ssd/models/subnetwork_draft.py:165-191`` (``_build_attn_mask``);
* ``ssd/models/subnetwork_draft.py:61-73`` (``plan_bridges``);
* ``ssd/models/bridges.py:27-37,40-65,131-135`` (bridge RMSNorm and MLPs);
* ``ssd/engine/kv_cache.py:21-73`` (``KVCache``);
* the transformers Llama pieces the reference calls into
  (``modeling_llama.py`` RMSNorm, rotary embedding and MLP): fp32 normalise,
  cast, then multiply by the weight; cos/sin computed in fp32 then cast to the
  activation dtype.

Weights are plain tensors keyed by the HF state-dict names; nothing from the
reference or from transformers is called at run time.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn.functional as F

ACTS = {"silu": F.silu, "gelu": F.gelu, "relu": F.relu}


@dataclass
class LlamaShape:
    hidden: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    inter: int
    vocab: int
    eps: float = 1e-6
    theta: float = 500000.0
    rope_scaling: Optional[tuple] = None  # llama3: (factor, low_freq_factor, high_freq_factor, original ctx)

    @classmethod
    def from_hf_config(cls, c) -> "LlamaShape":
        hd = getattr(c, "head_dim", None) or c.hidden_size // c.num_attention_heads
        rp = getattr(c, "rope_parameters", None) or {}
        theta = rp.get("rope_theta", getattr(c, "rope_theta", 10000.0))
        scaling = None
        if rp.get("rope_type", "default") == "llama3":
            scaling = (rp["factor"], rp["low_freq_factor"], rp["high_freq_factor"],
                       rp.get("original_max_position_embeddings") or c.max_position_embeddings)
        elif rp.get("rope_type", "default") != "default":
            raise ValueError(f"rope_type {rp['rope_type']!r}")
        return cls(c.hidden_size, c.num_hidden_layers, c.num_attention_heads, c.num_key_value_heads, hd,
                   c.intermediate_size, c.vocab_size, c.rms_norm_eps, float(theta), scaling)


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """HF LlamaRMSNorm: normalise in fp32, cast back, then scale (weight * x)."""
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return w * xf.to(x.dtype)


def bridge_rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """Bridge RMSNorm (ssd/models/bridges.py:33-37): same order as HF's."""
    return rms_norm(x, w, eps)


def llama3_inv_freq(inv: torch.Tensor, factor, low, high, ctx) -> torch.Tensor:
    """Llama 3.1 frequency scaling (transformers modeling_rope_utils._compute_llama3_parameters):
    frequencies whose wavelength exceeds ctx/low are divided by factor, those below ctx/high kept,
    the band between blended: (1 - s) w / factor + s w with s = (ctx / wavelength - low) / (high - low)."""
    out = inv.clone()
    for i in range(inv.numel()):
        w = inv[i:i + 1]
        wl = 2 * math.pi / w
        if wl.item() > ctx / low:
            out[i:i + 1] = w / factor
        elif wl.item() >= ctx / high:
            s = (ctx / wl - low) / (high - low)
            out[i:i + 1] = (1 - s) * w / factor + s * w
    return out


def rope_cos_sin(positions: torch.Tensor, head_dim: int, theta: float, dtype,
                 scaling: Optional[tuple] = None) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin [n, head_dim] for integer positions, computed in fp32 and cast."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))
    if scaling is not None:
        inv = llama3_inv_freq(inv, *scaling)
    freqs = positions.float()[:, None] * inv[None, :]
    emb = torch.cat([freqs, freqs], -1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], -1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [H, n, hd]; cos/sin [n, hd] (same dtype as x). Two rounded products, one rounded sum."""
    return x * cos + rotate_half(x) * sin


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: Optional[torch.Tensor]) -> torch.Tensor:
    """Masked GQA attention. q [Hq, M, hd], k/v [Hkv, S, hd], mask bool [M, S] (True = attend)
    or None (attend all). Computed in fp32 and returned in q's dtype (SDPA semantics)."""
    hq, m, hd = q.shape
    rep = hq // k.shape[0]
    kf = k.float().repeat_interleave(rep, 0)
    vf = v.float().repeat_interleave(rep, 0)
    s = (q.float() @ kf.transpose(1, 2)) / math.sqrt(hd)
    if mask is not None:
        s = s.masked_fill(~mask[None], float("-inf"))
    return (torch.softmax(s, -1) @ vf).to(q.dtype)


class KVCache:
    """Per-base-layer K/V buffers [Hkv, max_len, hd] (ssd/engine/kv_cache.py:21-73, batch 1)."""

    def __init__(self, num_slots: int, max_length: int):
        self.max_length = max_length
        self.seq_len = 0
        self.k: list[Optional[torch.Tensor]] = [None] * num_slots
        self.v: list[Optional[torch.Tensor]] = [None] * num_slots

    def get_seq_length(self) -> int:
        return self.seq_len

    def update(self, layer: int, k: torch.Tensor, v: torch.Tensor):
        n = k.shape[1]
        end = self.seq_len + n
        if end > self.max_length:  # kv_cache.py:35-36
            raise RuntimeError(f"KVCache overflow: {end} > max_length={self.max_length}")
        if self.k[layer] is None:
            self.k[layer] = torch.zeros(k.shape[0], self.max_length, k.shape[2], dtype=k.dtype)
            self.v[layer] = torch.zeros(v.shape[0], self.max_length, v.shape[2], dtype=v.dtype)
        self.k[layer][:, self.seq_len:end] = k
        self.v[layer][:, self.seq_len:end] = v
        return self.k[layer][:, :end], self.v[layer][:, :end]

    def advance(self, n: int) -> None:
        self.seq_len += n

    def crop(self, length: int) -> None:
        if length > self.seq_len:
            raise ValueError(f"cannot crop to {length} > current length {self.seq_len}")
        self.seq_len = length

    def keep_positions(self, start: int, positions: list[int]) -> None:
        """kv_cache.py:54-70: move ``positions`` to [start, start+n); a gather that reads
        every source before writing (index_select materialises first)."""
        n = len(positions)
        if n == 0 or list(positions) == list(range(start, start + n)):
            self.seq_len = start + n
            return
        idx = torch.tensor(positions, dtype=torch.long)
        for layer in range(len(self.k)):
            if self.k[layer] is None:
                continue
            self.k[layer][:, start:start + n] = self.k[layer].index_select(1, idx)
            self.v[layer][:, start:start + n] = self.v[layer].index_select(1, idx)
        self.seq_len = start + n


@dataclass
class BridgeSpec:
    name: str
    src_boundary: int
    tgt_boundary: int


def plan_bridges(layer_indices: list[int], num_base_layers: int) -> list[BridgeSpec]:
    """A bridge before every selected layer that does not follow its predecessor, plus
    ``into_norm`` when the last base layer is skipped (subnetwork_draft.py:61-73)."""
    specs, have = [], 0
    for idx in layer_indices:
        if have != idx:
            specs.append(BridgeSpec(f"into_{idx}", have, idx))
        have = idx + 1
    if have != num_base_layers:
        specs.append(BridgeSpec("into_norm", have, num_base_layers))
    return specs


class Bridge:
    """``x + MLP(RMSNorm(x))`` (bridges.py:68-135) from a state dict with the reference's key
    names (``norm.weight``, ``mlp.body.{0,2}.{weight,bias}``, ``mlp.out_proj.*`` or
    ``mlp.{gate,up}_proj.*``), evaluated in the parameters' dtype."""

    def __init__(self, sd: dict, mlp_type: str = "mlp", activation: str = "silu", eps: float = 1e-5):
        self.sd, self.mlp_type, self.act, self.eps = sd, mlp_type, ACTS[activation], eps

    def _lin(self, x, name):
        return F.linear(x, self.sd[name + ".weight"], self.sd.get(name + ".bias"))

    def mlp(self, x):
        if self.mlp_type == "swiglu":
            return self._lin(F.silu(self._lin(x, "mlp.gate_proj")) * self._lin(x, "mlp.up_proj"), "mlp.out_proj")
        i = 0
        while f"mlp.body.{i}.weight" in self.sd:
            x = self.act(self._lin(x, f"mlp.body.{i}"))
            i += 2
        return self._lin(x, "mlp.out_proj")

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        w = self.sd["norm.weight"]
        xi = x.to(w.dtype)
        return (xi + self.mlp(bridge_rms_norm(xi, w, self.eps))).to(x.dtype)


class Llama:
    """Weights of a Llama target, by HF state-dict name, in one dtype."""

    def __init__(self, sd: dict, shape: LlamaShape, dtype=None):
        self.shape = shape
        self.dtype = dtype or sd["model.embed_tokens.weight"].dtype
        self.sd = {k: v.detach().to("cpu", self.dtype) for k, v in sd.items()}

    @classmethod
    def from_hf(cls, model, dtype=None) -> "Llama":
        return cls(model.state_dict(), LlamaShape.from_hf_config(model.config), dtype)

    def w(self, name: str) -> torch.Tensor:
        return self.sd[name]

    def new_cache(self, max_length: int) -> KVCache:
        return KVCache(self.shape.layers, max_length)


def build_attn_mask(q_len: int, past_len: int, tree_mask: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    """bool [q, past+q] (True = attend) or None = attend all (subnetwork_draft.py:165-191)."""
    if tree_mask is not None and tree_mask.shape[-1] == past_len + q_len and past_len > 0:
        return tree_mask.bool()
    if tree_mask is None:
        if q_len == 1:
            return None
        causal = torch.ones(q_len, q_len, dtype=torch.bool).tril()
    else:
        causal = tree_mask.bool()
        if tuple(causal.shape[-2:]) != (q_len, q_len):
            raise ValueError(f"tree_attention_mask must be [.., {q_len}, {q_len}], got {tuple(causal.shape)}")
    return torch.cat([torch.ones(q_len, past_len, dtype=torch.bool), causal], -1)


class Subnetwork:
    """Draft (or, with every layer selected, the target) over a ``Llama``
    (subnetwork_draft.py:101-357). Bridges: ``{name: Bridge}``."""

    def __init__(self, base: Llama, layer_indices: list[int], bridges: Optional[dict] = None):
        n = base.shape.layers
        idx = [int(i) for i in layer_indices]
        if not idx or any(b <= a for a, b in zip(idx, idx[1:])) or idx[0] < 0 or idx[-1] >= n:
            raise ValueError(f"bad layer_indices {layer_indices} for {n} layers")
        self.base, self.layer_indices = base, idx
        self.specs = plan_bridges(idx, n)
        by_tgt = {s.tgt_boundary: s.name for s in self.specs}
        self.pre_layer = [by_tgt.get(i) for i in idx]
        self.pre_norm = by_tgt.get(n)
        self.bridges = bridges or {}
        missing = [s.name for s in self.specs if s.name not in self.bridges]
        if missing:
            raise ValueError(f"missing bridges {missing}")
        self.vocab_ids: Optional[torch.Tensor] = None
        self.sub_head: Optional[torch.Tensor] = None

    def set_vocab_subset(self, ids: Optional[torch.Tensor]) -> None:
        """subnetwork_draft.py:136-144: keep the lm_head rows of ``ids`` (sorted ascending)."""
        if ids is None:
            self.vocab_ids = self.sub_head = None
            return
        self.vocab_ids = ids.long()
        self.sub_head = self.base.w("lm_head.weight").index_select(0, self.vocab_ids).contiguous()

    def new_cache(self, max_length: int) -> KVCache:
        return self.base.new_cache(max_length)

    def _layer(self, li: int, h: torch.Tensor, cos, sin, mask, cache: Optional[KVCache]) -> torch.Tensor:
        s, w = self.base.shape, self.base.w
        p = f"model.layers.{li}."
        m = h.shape[0]
        x = rms_norm(h, w(p + "input_layernorm.weight"), s.eps)
        q = F.linear(x, w(p + "self_attn.q_proj.weight")).view(m, s.heads, s.head_dim).transpose(0, 1)
        k = F.linear(x, w(p + "self_attn.k_proj.weight")).view(m, s.kv_heads, s.head_dim).transpose(0, 1)
        v = F.linear(x, w(p + "self_attn.v_proj.weight")).view(m, s.kv_heads, s.head_dim).transpose(0, 1)
        q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
        if cache is not None:
            k, v = cache.update(li, k, v)
        if mask is None and m > 1:
            mask = torch.ones(m, m, dtype=torch.bool).tril()
        o = attention(q, k, v, mask).transpose(0, 1).reshape(m, s.heads * s.head_dim)
        h = h + F.linear(o, w(p + "self_attn.o_proj.weight"))
        x = rms_norm(h, w(p + "post_attention_layernorm.weight"), s.eps)
        g = F.silu(F.linear(x, w(p + "mlp.gate_proj.weight")))
        u = F.linear(x, w(p + "mlp.up_proj.weight"))
        return h + F.linear(g * u, w(p + "mlp.down_proj.weight"))

    def forward(self, input_ids, position_ids=None, cache: Optional[KVCache] = None, tree_attention_mask=None,
                logits_to_keep: int = 0, compute_logits: bool = True):
        """input_ids [M] or [1, M]; position_ids likewise. Returns (logits [M', V or V'], hidden [M, d])."""
        ids = torch.as_tensor(input_ids).reshape(-1).long()
        m = ids.numel()
        past = cache.get_seq_length() if cache is not None else 0
        pos = (torch.arange(past, past + m) if position_ids is None
               else torch.as_tensor(position_ids).reshape(-1).long())
        s = self.base.shape
        cos, sin = rope_cos_sin(pos, s.head_dim, s.theta, self.base.dtype, s.rope_scaling)
        mask = None if (cache is None and tree_attention_mask is None) else build_attn_mask(m, past, tree_attention_mask)
        h = self.base.w("model.embed_tokens.weight")[ids]
        for slot, li in enumerate(self.layer_indices):
            if self.pre_layer[slot] is not None:
                h = self.bridges[self.pre_layer[slot]](h)
            h = self._layer(li, h, cos, sin, mask, cache)
        if self.pre_norm is not None:
            h = self.bridges[self.pre_norm](h)
        if cache is not None:
            cache.advance(m)
        h = rms_norm(h, self.base.w("model.norm.weight"), s.eps)
        logits = None
        if compute_logits:
            hs = h[-logits_to_keep:] if logits_to_keep > 0 else h
            head = self.sub_head if self.sub_head is not None else self.base.w("lm_head.weight")
            logits = F.linear(hs, head)
        return logits, h

    __call__ = forward


class Target(Subnetwork):
    """Every layer, no bridges (ssd/engine/speculative.py:94-99)."""

    def __init__(self, base: Llama):
        super().__init__(base, list(range(base.shape.layers)))


def identity_bridges(specs: list[BridgeSpec], d: int, dtype=torch.float32, hidden: Optional[int] = None) -> dict:
    """Zero out_proj bridges (BridgeConfig(init_std=0), bridges.py:118-129): exact identity."""
    hid = hidden or d
    out = {}
    for s in specs:
        out[s.name] = Bridge({
            "norm.weight": torch.ones(d, dtype=dtype),
            "mlp.body.0.weight": torch.zeros(hid, d, dtype=dtype),
            "mlp.body.0.bias": torch.zeros(hid, dtype=dtype),
            "mlp.out_proj.weight": torch.zeros(d, hid, dtype=dtype),
            "mlp.out_proj.bias": torch.zeros(d, dtype=dtype),
        })
    return out


def random_bridges(specs: list[BridgeSpec], d: int, seed: int, init_std: float = 1e-3, dtype=torch.float32,
                   hidden: Optional[int] = None) -> dict:
    """Bridges initialised like bridges.py:118-129 (inner N(0,1/sqrt(fan_in)), out N(0,init_std),
    zero biases, norm 1) from a seeded CPU generator, as reference-named state dicts."""
    g = torch.Generator().manual_seed(seed)
    hid = hidden or d
    out = {}
    for s in specs:
        out[s.name] = Bridge({
            "norm.weight": torch.ones(d, dtype=dtype),
            "mlp.body.0.weight": (torch.randn(hid, d, generator=g) / math.sqrt(d)).to(dtype),
            "mlp.body.0.bias": torch.zeros(hid, dtype=dtype),
            "mlp.out_proj.weight": (torch.randn(d, hid, generator=g) * init_std).to(dtype),
            "mlp.out_proj.bias": torch.zeros(d, dtype=dtype),
        })
    return out
