"""Llama target weights in the MI355X layout.

The reference keeps HF ``LlamaForCausalLM`` modules and calls their ``nn.Linear`` layers
(ssd/models/subnetwork_draft.py:80-89, 193-246). Here the same weights live once in HBM in
the layout the gfx950 kernels stream:

* per layer: q/k/v fused into one packed matrix whose 16-row tiles pair rotary dims d and
  d + hd/2 (so RoPE and the KV-cache write run in the GEMM epilogue); gate/up fused with 8
  gate rows + the matching 8 up rows per tile (SwiGLU in the epilogue); o and down packed
  as-is. Each RMSNorm weight is folded into the columns of the projection that consumes it
  (ln1 into q/k/v, ln2 into gate/up, the final norm into the lm_head): those GEMMs take the
  residual stream itself and scale each row by its rsqrt(mean(h^2) + eps), so no separate
  norm kernel runs (the weights are also kept as plain bf16 vectors);
* the embedding table row-major (a gather), the lm_head packed (a weight-streaming GEMM);
* RoPE cos/sin tables [positions, hd/2] computed in fp32 and rounded to bf16 exactly as HF's
  rotary embedding does.

Packed weights are built from an HF model / state dict (copied once, layer by layer) or
generated directly on the GPU for synthetic benchmarks (``synthetic``), never duplicated.
"""

from __future__ import annotations

import types
from dataclasses import dataclass
from typing import Optional

import torch

from ssd import _lib, ops

BF16 = torch.bfloat16


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
    # Llama 3.1 frequency scaling (HF rope_type "llama3", used by Llama-3.1/3.2 checkpoints):
    # (factor, low_freq_factor, high_freq_factor, original_max_position_embeddings); None = plain RoPE
    rope_scaling: Optional[tuple] = None

    @classmethod
    def from_hf_config(cls, c) -> "LlamaShape":
        hd = getattr(c, "head_dim", None) or c.hidden_size // c.num_attention_heads
        theta, scaling = rope_config(c)
        return cls(c.hidden_size, c.num_hidden_layers, c.num_attention_heads, c.num_key_value_heads, hd,
                   c.intermediate_size, c.vocab_size, float(c.rms_norm_eps), theta, scaling)

    def validate(self) -> None:
        if self.heads % self.kv_heads:
            raise ValueError("heads must be a multiple of kv_heads")
        if self.head_dim not in (32, 64, 128):
            raise ValueError(f"head_dim {self.head_dim} unsupported (32, 64, 128)")
        for name in ("hidden", "inter"):
            if getattr(self, name) % 32:
                raise ValueError(f"{name}={getattr(self, name)} must be a multiple of 32")


class _Cfg:
    """HF-config-like view (num_hidden_layers, hidden_size, ...) for API compatibility."""

    def __init__(self, s: LlamaShape):
        self.num_hidden_layers = s.layers
        self.hidden_size = s.hidden
        self.num_attention_heads = s.heads
        self.num_key_value_heads = s.kv_heads
        self.head_dim = s.head_dim
        self.intermediate_size = s.inter
        self.vocab_size = s.vocab
        self.rms_norm_eps = s.eps
        self.rope_theta = s.theta
        self.rope_parameters = {"rope_type": "default", "rope_theta": s.theta}
        if s.rope_scaling is not None:
            f, lo, hi, ctx = s.rope_scaling
            self.rope_parameters.update(rope_type="llama3", factor=f, low_freq_factor=lo, high_freq_factor=hi,
                                        original_max_position_embeddings=ctx)


def qkv_row_map(heads: int, kv_heads: int, hd: int) -> torch.Tensor:
    """Packed row -> row of cat(q, k, v): per head, tiles of (8 dims of the first rotary half,
    the same 8 dims of the second half)."""
    half, rows = hd // 2, []
    for base, nh in ((0, heads), (heads * hd, kv_heads), ((heads + kv_heads) * hd, kv_heads)):
        for h in range(nh):
            for p in range(hd // 16):
                b = base + h * hd + p * 8
                rows += list(range(b, b + 8)) + list(range(b + half, b + half + 8))
    return torch.tensor(rows, dtype=torch.int32)


def gate_up_row_map(inter: int) -> torch.Tensor:
    """Packed row -> row of cat(gate, up): tile i = gate rows [8i, 8i+8) then up rows [8i, 8i+8)."""
    i = torch.arange(inter // 8, dtype=torch.int32)[:, None] * 8 + torch.arange(8, dtype=torch.int32)[None]
    return torch.cat([i, i + inter], 1).reshape(-1)


def rope_config(c) -> tuple:
    """(theta, llama3 scaling tuple or None) from an HF config: ``rope_parameters`` (transformers
    5) or ``rope_theta`` + ``rope_scaling`` (4.x). Other rope types raise ValueError."""
    rp = dict(getattr(c, "rope_parameters", None) or {})
    legacy = getattr(c, "rope_scaling", None)
    if legacy and not rp.get("rope_type"):
        rp.update(legacy)
    theta = float(rp.get("rope_theta", getattr(c, "rope_theta", None) or 10000.0))
    rtype = rp.get("rope_type", rp.get("type", "default"))
    if rtype == "default":
        return theta, None
    if rtype == "llama3":
        old = rp.get("original_max_position_embeddings") or getattr(c, "max_position_embeddings")
        return theta, (float(rp["factor"]), float(rp["low_freq_factor"]), float(rp["high_freq_factor"]), int(old))
    raise ValueError(f"rope_type {rtype!r} is not supported (default and llama3 RoPE)")


def rope_inv_freq(hd: int, theta: float, scaling: Optional[tuple] = None) -> torch.Tensor:
    """fp32 inverse frequencies theta^(-2i/hd); with Llama 3.1 scaling (factor f, low/high
    frequency factors l/h, original context C) the wavelength 2 pi / w decides per frequency:
    above C / l divide by f, below C / h keep, in between blend w / f and w linearly by
    s = (C / wavelength - l) / (h - l), all in fp32 as HF's rope init does."""
    inv = 1.0 / (theta ** (torch.arange(0, hd, 2, dtype=torch.int64).float() / hd))
    if scaling is None:
        return inv
    f, lo, hi, ctx = scaling
    wavelen = 2 * torch.pi / inv
    low_cut, high_cut = ctx / lo, ctx / hi  # long wavelengths are scaled, short ones kept
    scaled = torch.where(wavelen > low_cut, inv / f, inv)
    s = (ctx / wavelen - lo) / (hi - lo)
    blend = (1 - s) * scaled / f + s * scaled
    mid = (wavelen >= high_cut) & (wavelen <= low_cut)
    return torch.where(mid, blend, scaled)


def rope_tables(positions: int, hd: int, theta: float, device,
                scaling: Optional[tuple] = None) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin [positions, hd/2] as HF computes them (fp32 inv_freq and angles, then bf16)."""
    inv = rope_inv_freq(hd, theta, scaling)
    ang = torch.arange(positions, dtype=torch.float32)[:, None] * inv[None, :]
    return ang.cos().to(BF16).to(device).contiguous(), ang.sin().to(BF16).to(device).contiguous()


class Layer:
    __slots__ = ("wqkv", "wo", "wgu", "wd", "ln1", "ln2", "mlp_fused")


class MI355XLlama:
    """A Llama target resident in HBM in the kernels' layout. ``config`` mimics the HF config."""

    def __init__(self, shape: LlamaShape, device="cuda", fused_mlp: bool = True):
        shape.validate()
        self.shape = shape
        self.fused_mlp = fused_mlp  # pack gate/up for the one-launch MLP where the shape allows
        self.config = _Cfg(shape)
        self.generation_config = types.SimpleNamespace(eos_token_id=None)
        dev = torch.device(device)
        if dev.type == "cuda" and dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        self.device = dev
        self.embed: Optional[torch.Tensor] = None
        self.lm_head: Optional[torch.Tensor] = None
        self.norm: Optional[torch.Tensor] = None
        self.layers: list[Layer] = []
        self._cos = self._sin = None
        self._lm_head_rows: Optional[torch.Tensor] = None  # row-major lm_head kept only when requested
        self._native = None

    # ------------------------------------------------------------ construction
    def _put(self, t: torch.Tensor) -> torch.Tensor:
        return t.detach().to(device=self.device, dtype=BF16).contiguous()

    def _set_layer(self, get) -> None:
        s = self.shape
        L = Layer()
        L.ln1 = self._put(get("input_layernorm.weight"))
        L.ln2 = self._put(get("post_attention_layernorm.weight"))
        # each RMSNorm weight is folded into the columns of the projection that consumes it
        qkv = torch.cat([self._put(get("self_attn.q_proj.weight")), self._put(get("self_attn.k_proj.weight")),
                         self._put(get("self_attn.v_proj.weight"))], 0)
        L.wqkv = ops.pack_weight(qkv, qkv_row_map(s.heads, s.kv_heads, s.head_dim), col_scale=L.ln1)
        del qkv
        L.wo = ops.pack_weight(self._put(get("self_attn.o_proj.weight")), residual=True)
        gu = torch.cat([self._put(get("mlp.gate_proj.weight")), self._put(get("mlp.up_proj.weight"))], 0)
        # grouped for the fused MLP (one cooperative launch) where the shape has a plan for it
        g = ops.mlp_group(s.inter, s.hidden) if self.fused_mlp else 0
        L.wgu = ops.pack_weight(gu, gate_up_row_map(s.inter), col_scale=L.ln2, group=g or None)
        L.mlp_fused = g > 0
        del gu
        L.wd = ops.pack_weight(self._put(get("mlp.down_proj.weight")), residual=True)
        self.layers.append(L)

    @property
    def mlp_fused(self) -> bool:
        """Every layer's MLP runs as one cooperative launch (ops.mlp)."""
        return bool(self.layers) and all(L.mlp_fused for L in self.layers)

    @classmethod
    def from_state_dict(cls, sd: dict, shape: LlamaShape, device="cuda", keep_lm_head_rows: bool = False,
                        fused_mlp: bool = True):
        m = cls(shape, device, fused_mlp)
        m.embed = m._put(sd["model.embed_tokens.weight"])
        for i in range(shape.layers):
            m._set_layer(lambda n, i=i: sd[f"model.layers.{i}.{n}"])
        m.norm = m._put(sd["model.norm.weight"])
        head = sd.get("lm_head.weight", sd["model.embed_tokens.weight"])
        head = m._put(head)
        m.lm_head = ops.pack_weight(head, col_scale=m.norm)  # final norm folded
        if keep_lm_head_rows:
            m._lm_head_rows = head
        torch.cuda.synchronize(m.device)
        return m

    @classmethod
    def from_hf(cls, model, device="cuda", keep_lm_head_rows: bool = False, fused_mlp: bool = True) -> "MI355XLlama":
        m = cls.from_state_dict(model.state_dict(), LlamaShape.from_hf_config(model.config), device,
                                keep_lm_head_rows, fused_mlp)
        m.generation_config.eos_token_id = getattr(getattr(model, "generation_config", None), "eos_token_id", None)
        return m

    @classmethod
    def synthetic(cls, shape: LlamaShape, seed: int = 0, std: float = 0.02, device="cuda",
                  fused_mlp: bool = True) -> "MI355XLlama":
        """Random-init weights N(0, std) (norms = 1) generated on the GPU by ``synthetic_tensors``
        (one seeded generator per tensor), so the model is reproducible on one torch build."""
        m = cls(shape, device, fused_mlp)
        s = shape
        gen = synthetic_tensors(shape, seed, std, m.device)
        m.embed = next(gen)[1]
        for _ in range(s.layers):
            w = {n.split(".", 3)[3]: t for n, t in (next(gen) for _ in range(9))}
            m._set_layer(w.__getitem__)
            del w
        m.norm = next(gen)[1]
        m.lm_head = ops.pack_weight(next(gen)[1], col_scale=m.norm)
        torch.cuda.synchronize(m.device)
        return m

    # ---------------------------------------------------------------- helpers
    def rope(self, max_pos: int) -> tuple[torch.Tensor, torch.Tensor]:
        if self._cos is None or self._cos.shape[0] < max_pos:
            n = max(max_pos, 4096)
            self._cos, self._sin = rope_tables(n, self.shape.head_dim, self.shape.theta, self.device,
                                               self.shape.rope_scaling)
        return self._cos, self._sin

    def native(self, max_pos: int) -> "_lib.SsdModel":
        """C descriptor (SsdModel) of this model for ssd_forward; rebuilt only when the rotary
        tables grow. The struct and its layer array stay alive on this object."""
        cos, sin = self.rope(max_pos)
        if self._native is None or self._native[0] != cos.data_ptr():
            s = self.shape
            arr = (_lib.SsdLayerW * s.layers)(*[
                _lib.SsdLayerW(L.wqkv.data_ptr(), L.wo.data_ptr(), L.wgu.data_ptr(), L.wd.data_ptr(), L.ln1.data_ptr(),
                               L.ln2.data_ptr()) for L in self.layers])
            st = _lib.SsdModel(s.hidden, s.heads, s.kv_heads, s.head_dim, s.inter, s.vocab, s.layers, s.eps,
                               s.head_dim ** -0.5, self.embed.data_ptr(), self.norm.data_ptr(), cos.data_ptr(),
                               sin.data_ptr(), cos.shape[0], arr, int(self.mlp_fused))
            self._native = (cos.data_ptr(), st, arr)
        return self._native[1]

    def weight_bytes(self, layers=None) -> int:
        """Packed bytes streamed per forward for ``layers`` (default all) plus the full lm_head."""
        idx = range(self.shape.layers) if layers is None else layers
        b = sum(self.layers[i].wqkv.numel() + self.layers[i].wo.numel() + self.layers[i].wgu.numel()
                + self.layers[i].wd.numel() for i in idx)
        return 2 * (b + self.lm_head.numel())

    def lm_head_rows(self, ids: torch.Tensor) -> torch.Tensor:
        """Row-major lm_head rows ``ids`` as the packed head applies them (final-norm weight folded
        into the columns), for a vocabulary-subset head. Unpacks from the packed tiles when the
        row-major copy was not kept."""
        if self._lm_head_rows is not None:
            rows = self._lm_head_rows.index_select(0, ids.to(self.device))
            return (rows.float() * self.norm.float()).to(BF16)  # the fold of ssd_pack_weight_bf16
        return unpack_rows(self.lm_head, self.shape.vocab, self.shape.hidden, ids.to(self.device),
                           ops.weight_group(self.shape.vocab, self.shape.hidden))


def synthetic_tensors(shape: LlamaShape, seed: int = 0, std: float = 0.02, device="cuda"):
    """The synthetic model's tensors in HF state-dict naming, generated one at a time on
    ``device``: linear weights and the embedding N(0, std) in fp32 rounded to bf16, each from its
    own generator seeded seed * 1000 + index (index = order of generation), norm weights 1. Yields
    (name, tensor) in the order embed, per layer (q, k, v, o, gate, up, down, ln1, ln2), norm,
    lm_head, so a caller can rebuild any tensor of a model ``MI355XLlama.synthetic`` made."""
    counter = [0]

    def rnd(*size):
        g = torch.Generator(device=device).manual_seed(seed * 1000 + counter[0])
        counter[0] += 1
        return (torch.randn(*size, generator=g, device=device, dtype=torch.float32) * std).to(BF16)

    s = shape
    yield "model.embed_tokens.weight", rnd(s.vocab, s.hidden)
    for i in range(s.layers):
        p = f"model.layers.{i}."
        yield p + "self_attn.q_proj.weight", rnd(s.heads * s.head_dim, s.hidden)
        yield p + "self_attn.k_proj.weight", rnd(s.kv_heads * s.head_dim, s.hidden)
        yield p + "self_attn.v_proj.weight", rnd(s.kv_heads * s.head_dim, s.hidden)
        yield p + "self_attn.o_proj.weight", rnd(s.hidden, s.heads * s.head_dim)
        yield p + "mlp.gate_proj.weight", rnd(s.inter, s.hidden)
        yield p + "mlp.up_proj.weight", rnd(s.inter, s.hidden)
        yield p + "mlp.down_proj.weight", rnd(s.hidden, s.inter)
        yield p + "input_layernorm.weight", torch.ones(s.hidden, dtype=BF16, device=device)
        yield p + "post_attention_layernorm.weight", torch.ones(s.hidden, dtype=BF16, device=device)
    yield "model.norm.weight", torch.ones(s.hidden, dtype=BF16, device=device)
    yield "lm_head.weight", rnd(s.vocab, s.hidden)


def unpack_rows(packed: torch.Tensor, n: int, k: int, ids: torch.Tensor, group: int = 1) -> torch.Tensor:
    """Rows ``ids`` of the row-major matrix held in MFMA tiles (inverse of the identity packing
    with tiles grouped by ``group`` per k-block)."""
    kb = (k + 31) // 32
    t = packed.view(-1, kb, group, 4, 16, 8)  # [nb // group, kb, nb % group, lane/16, lane%16, 8]
    nb, r = ids // 16, ids % 16
    rows = t[(nb // group).long(), :, (nb % group).long(), :, r.long(), :]  # [len, kb, 4, 8]
    return rows.reshape(ids.numel(), kb * 32)[:, :k].contiguous()
