"""Torch-tensor wrappers over the C ABI (include/ssd_mi355x.h).

PyTorch only supplies device memory and the current HIP stream here; every computation is a
hand-written gfx950 kernel in ``libssd_mi355x.so``. Inputs are validated on the host (dtype,
device, alignment, shapes) before a launch, so a bad call raises instead of faulting.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from ssd import _lib

ACT = {None: 0, "none": 0, "silu": 1, "gelu": 2, "relu": 3}
BF16 = torch.bfloat16


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _p(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _check(t: torch.Tensor, name: str, dtype=BF16):
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError(f"{name} must be a CUDA (HIP) tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if dtype == BF16 and t.data_ptr() % 16:
        raise ValueError(f"{name} must be 16-byte aligned")


def _rows(t: torch.Tensor, name: str, cols: int, rows: int = 0) -> int:
    """Row stride of a 2-D row-major tensor with unit column stride and >= ``rows`` rows."""
    if t.dim() != 2 or t.stride(1) != 1 or t.shape[1] < cols or t.shape[0] < rows:
        raise ValueError(f"{name} must be [>={rows}, >={cols}] with unit column stride, got {tuple(t.shape)}")
    return t.stride(0)


def _len(t: Optional[torch.Tensor], name: str, n: int) -> None:
    if t is not None and t.numel() < n:
        raise ValueError(f"{name} has {t.numel()} elements, needs {n}")


def packed_elems(n: int, k: int) -> int:
    return int(_lib.load().ssd_packed_weight_elems(n, k))


def weight_group(n: int, k: int) -> int:
    """Tile grouping the single-pass GEMMs (gemm, gemm_swiglu, qkv_rope) expect for an [N, K] weight."""
    g = int(_lib.load().ssd_gemm_weight_group(n, k))
    if g < 1:
        raise ValueError(f"weight_group: bad shape N={n} K={k}")
    return g


def pack_weight(w: torch.Tensor, row_map: Optional[torch.Tensor] = None, split: bool = False,
                n_logical: Optional[int] = None, col_scale: Optional[torch.Tensor] = None,
                residual: bool = False, group: Optional[int] = None) -> torch.Tensor:
    """Row-major bf16 W[N, K] -> MFMA tile layout. row_map picks the source row of each packed
    row (-1 = zeros); default = identity. Rows are padded with zeros to a multiple of 128. Tiles
    are grouped for the single-pass GEMMs (group = weight_group(N_logical, K), N_logical = the
    GEMM's output width, default the row_map length); split=True packs for gemm_partial (group 1),
    residual=True for gemm_residual (group = residual_group(N, K)); group overrides all of these
    (mlp: gate/up packed with mlp_group(I, H)). col_scale [K] folds an RMSNorm weight into the
    columns (W * s, rounded once to bf16), for GEMMs called with norm_eps."""
    _check(w, "w")
    n, k = w.shape
    ld = _rows(w, "w", k)
    if row_map is None:
        row_map = torch.arange(n, dtype=torch.int32)
    row_map = row_map.to(torch.int32).cpu()
    n_log = n_logical if n_logical is not None else row_map.numel()
    n_packed = (row_map.numel() + 127) // 128 * 128
    if n_packed != row_map.numel():
        row_map = torch.cat([row_map, torch.full((n_packed - row_map.numel(),), -1, dtype=torch.int32)])
    rm = row_map.to(device=w.device)
    if group is None:
        group = 1 if split else residual_group(n_log, k) if residual else weight_group(n_log, k)
    if col_scale is not None:
        _check(col_scale, "col_scale")
        _len(col_scale, "col_scale", k)
    out = torch.empty(packed_elems(n_packed, k), dtype=BF16, device=w.device)
    _lib.call("ssd_pack_weight_bf16", w.data_ptr(), ld, n, k, rm.data_ptr(), n_packed, group, _p(col_scale),
              out.data_ptr(), stream())
    return out


def gemm(x: torch.Tensor, m: int, wp: torch.Tensor, n: int, k: int, out: torch.Tensor, bias=None, act=None,
         residual: Optional[torch.Tensor] = None, norm_eps: float = 0.0) -> torch.Tensor:
    """Y = act(X W^T + b) [+ residual]; norm_eps > 0: X is h and W was packed with the RMSNorm
    weight as col_scale (RMSNorm folded into the GEMM)."""
    _check(x, "x"); _check(wp, "w_packed"); _check(out, "out")
    if bias is not None:
        _check(bias, "bias")
    ldx = _rows(x, "x", k, m)
    ldy = _rows(out, "out", n, m)
    _len(bias, "bias", n)
    _len(wp, "w_packed", packed_elems(n, k))
    ldr = 0
    if residual is not None:
        _check(residual, "residual")
        ldr = _rows(residual, "residual", n, m)
    _lib.call("ssd_gemm_bf16", x.data_ptr(), ldx, m, wp.data_ptr(), n, k, float(norm_eps), out.data_ptr(), ldy,
              _p(bias), ACT[act], _p(residual), ldr, stream())
    return out


def gemm_swiglu(x: torch.Tensor, m: int, wp: torch.Tensor, inter: int, k: int, out: torch.Tensor, bias_gate=None,
                bias_up=None, norm_eps: float = 0.0) -> torch.Tensor:
    _check(x, "x"); _check(wp, "w_packed"); _check(out, "out")
    _len(bias_gate, "bias_gate", inter); _len(bias_up, "bias_up", inter)
    _len(wp, "w_packed", packed_elems(2 * inter, k))
    _lib.call("ssd_gemm_swiglu_bf16", x.data_ptr(), _rows(x, "x", k, m), m, wp.data_ptr(), inter, k, float(norm_eps),
              out.data_ptr(), _rows(out, "out", inter, m), _p(bias_gate), _p(bias_up), stream())
    return out


def qkv_rope(x, m, wp, k, heads, kv_heads, head_dim, cos, sin, pos, slot, q_out, k_cache, vt_cache, max_len,
             norm_eps: float = 0.0):
    _check(x, "x"); _check(wp, "w_packed"); _check(q_out, "q"); _check(k_cache, "k_cache"); _check(vt_cache, "vt")
    for t, nm in ((pos, "pos"), (slot, "slot")):
        _check(t, nm, torch.int32)
        _len(t, nm, m)
    _len(wp, "w_packed", packed_elems((heads + 2 * kv_heads) * head_dim, k))
    if k_cache.numel() < kv_heads * max_len * head_dim or vt_cache.numel() < kv_heads * max_len * head_dim:
        raise ValueError("qkv_rope: cache smaller than kv_heads * max_len * head_dim")
    if cos.shape != sin.shape or cos.dim() != 2 or cos.shape[1] != head_dim // 2:
        raise ValueError("qkv_rope: cos/sin must be [rows, head_dim/2]")
    _lib.call("ssd_gemm_qkv_rope_bf16", x.data_ptr(), _rows(x, "x", k, m), m, wp.data_ptr(), k, float(norm_eps), heads,
              kv_heads, head_dim, cos.data_ptr(), sin.data_ptr(), cos.shape[0], pos.data_ptr(), slot.data_ptr(),
              q_out.data_ptr(), _rows(q_out, "q", heads * head_dim, m), k_cache.data_ptr(), vt_cache.data_ptr(),
              max_len, stream())


# ------------------------------------------------------------------ prefill (long prompt chunks)
EPI = {"store": 0, "swiglu": 1, "qkv": 2}


def prefill_gemm(x, m, wp, group, n, k, out, epi="store", residual=None, norm_eps: float = 0.0, qkv=None):
    """Y = epilogue(X W^T) for prompt-length M on the LDS-tiled MFMA kernel; ``wp`` packed with
    ``group`` (as for the decode GEMM of the same weight). epi "store" (+ residual), "swiglu"
    (n = 2 * inter, out gets inter columns) or "qkv" (qkv = dict(heads, kv_heads, head_dim, cos, sin,
    pos0, k_cache, vt_cache, max_len); q goes to out, k/v to the cache at slots pos0 + row)."""
    _check(x, "x"); _check(wp, "w_packed"); _check(out, "out")
    _len(wp, "w_packed", packed_elems(n, k))
    cols = n // 2 if epi == "swiglu" else (qkv["heads"] * qkv["head_dim"] if epi == "qkv" else n)
    ldr = 0
    if residual is not None:
        _check(residual, "residual")
        ldr = _rows(residual, "residual", n, m)
    ep = None
    if epi == "qkv":
        c = qkv
        for t, nm in ((c["k_cache"], "k_cache"), (c["vt_cache"], "vt_cache"), (c["cos"], "cos"), (c["sin"], "sin")):
            _check(t, nm)
        if c["k_cache"].numel() < c["kv_heads"] * c["max_len"] * c["head_dim"]:
            raise ValueError("prefill_gemm: cache smaller than kv_heads * max_len * head_dim")
        ep = _lib.SsdQkvEpilogue(c["heads"], c["kv_heads"], c["head_dim"], c["cos"].data_ptr(), c["sin"].data_ptr(),
                                 c["cos"].shape[0], int(c["pos0"]), c["k_cache"].data_ptr(), c["vt_cache"].data_ptr(),
                                 int(c["max_len"]))
    ldx = _rows(x, "x", k, m)
    rs = None
    if norm_eps > 0:  # the folded RMSNorm's row scales, one pass before the GEMM
        rs = torch.empty(m, dtype=torch.float32, device=x.device)
        _lib.call("ssd_prefill_row_scale_bf16", x.data_ptr(), ldx, m, k, float(norm_eps), rs.data_ptr(), stream())
    _lib.call("ssd_prefill_gemm_bf16", x.data_ptr(), ldx, m, wp.data_ptr(), int(group), n, k, _p(rs), EPI[epi],
              out.data_ptr(), _rows(out, "out", cols, m), _p(residual), ldr,
              ctypes.byref(ep) if ep is not None else None, stream())
    return out


def prefill_attention(q, m, pos0, heads, kv_heads, head_dim, k_cache, vt_cache, max_len, out, scale=None):
    """Causal attention of prompt rows pos0 .. pos0 + m - 1 over cache slots [0, row position]."""
    _check(q, "q"); _check(k_cache, "k_cache"); _check(vt_cache, "vt_cache"); _check(out, "out")
    if k_cache.numel() < kv_heads * max_len * head_dim or vt_cache.numel() < kv_heads * max_len * head_dim:
        raise ValueError("prefill_attention: cache smaller than kv_heads * max_len * head_dim")
    scale = head_dim ** -0.5 if scale is None else scale
    _lib.call("ssd_prefill_attention_bf16", q.data_ptr(), _rows(q, "q", heads * head_dim, m), m, int(pos0), heads,
              kv_heads, head_dim, k_cache.data_ptr(), vt_cache.data_ptr(), int(max_len), float(scale), out.data_ptr(),
              _rows(out, "out", heads * head_dim, m), stream())
    return out


def attn_workspace_floats(m: int, heads: int, head_dim: int, max_len: int) -> int:
    return int(_lib.load().ssd_attn_workspace_floats(m, heads, head_dim, max_len))


def tree_attention(q, m, heads, kv_heads, head_dim, k_cache, vt_cache, max_len, prefix, depth, anc, p_min, l_max,
                   ws, out, scale=None):
    _check(q, "q"); _check(k_cache, "k_cache"); _check(vt_cache, "vt_cache"); _check(out, "out")
    _check(ws, "ws", torch.float32)
    for t, nm, n in ((prefix, "prefix", m), (depth, "depth", m), (anc, "anc", m * 32)):
        _check(t, nm, torch.int32)
        _len(t, nm, n)
    if k_cache.numel() < kv_heads * max_len * head_dim or vt_cache.numel() < kv_heads * max_len * head_dim:
        raise ValueError("tree_attention: cache smaller than kv_heads * max_len * head_dim")
    scale = head_dim ** -0.5 if scale is None else scale
    _lib.call("ssd_tree_attention_bf16", q.data_ptr(), _rows(q, "q", heads * head_dim, m), m, heads, kv_heads, head_dim,
              k_cache.data_ptr(), vt_cache.data_ptr(), max_len, prefix.data_ptr(), depth.data_ptr(), anc.data_ptr(),
              int(p_min), int(l_max), float(scale), ws.data_ptr(), ws.numel(), out.data_ptr(),
              _rows(out, "out", heads * head_dim, m), stream())


def rmsnorm(x, m, w, eps, out):
    _check(x, "x"); _check(w, "w"); _check(out, "out")
    d = w.numel()
    _lib.call("ssd_rmsnorm_bf16", x.data_ptr(), _rows(x, "x", d, m), m, d, w.data_ptr(), float(eps), out.data_ptr(),
              _rows(out, "out", d, m), stream())
    return out


def embed(ids, m, table, out):
    _check(ids, "ids", torch.int32); _check(table, "table"); _check(out, "out")
    v, d = table.shape
    _len(ids, "ids", m)
    _lib.call("ssd_embed_bf16", ids.data_ptr(), m, table.data_ptr(), v, d, out.data_ptr(), _rows(out, "out", d, m),
              stream())
    return out


# ------------------------------------------------------------------ KV-cache block layout
_KV_INDEX: dict = {}


def kv_block_index(cap: int, hd: int, device) -> tuple:
    """Element offsets (k_idx, v_idx), each [cap, hd] int64, of K[s][d] and V[s][d] inside one
    (layer, kv head) region of the cache's 64-slot block layout (csrc/common.h k_off / v_off):
    a 64-slot block of K is stored as the attention kernel's S = K Q^T operand tiles, one of V as
    its O = V^T P^T operand tiles, each tile in lane order. cap % 64 == 0, hd % 32 == 0."""
    if cap % 64 or hd % 32:
        raise ValueError(f"kv_block_index: cap {cap} / head_dim {hd} must be multiples of 64 / 32")
    key = (cap, hd, str(device))
    if key not in _KV_INDEX:
        s = torch.arange(cap, dtype=torch.int64, device=device)[:, None]
        d = torch.arange(hd, dtype=torch.int64, device=device)[None, :]
        o = s & 63
        kt = ((o >> 5) << 1) | ((o >> 2) & 1)
        i = (((o >> 3) & 3) << 2) | (o & 3)
        k_idx = ((((s >> 6) * 4 + kt) * (hd >> 5) + (d >> 5)) * 64 + ((d >> 3) & 3) * 16 + i) * 8 + (d & 7)
        v_idx = ((((s >> 6) * (hd >> 4) + (d >> 4)) * 2 + (o >> 5)) * 64 + ((o >> 3) & 3) * 16 + (d & 15)) * 8 + (o & 7)
        _KV_INDEX[key] = (k_idx, v_idx)
    return _KV_INDEX[key]


def kv_tile(x: torch.Tensor, which: str) -> torch.Tensor:
    """[..., cap, hd] K or V (``which`` = "k" / "v") -> [..., cap * hd] in the block layout."""
    cap, hd = x.shape[-2:]
    idx = kv_block_index(cap, hd, x.device)[0 if which == "k" else 1].reshape(-1)
    out = torch.empty(*x.shape[:-2], cap * hd, dtype=x.dtype, device=x.device)
    out[..., idx] = x.reshape(*x.shape[:-2], cap * hd)
    return out


def kv_untile(flat: torch.Tensor, cap: int, hd: int, which: str) -> torch.Tensor:
    """Inverse of kv_tile: [..., cap * hd] in the block layout -> [..., cap, hd]."""
    idx = kv_block_index(cap, hd, flat.device)[0 if which == "k" else 1]
    return flat[..., idx]


def kv_compact(k_arena, vt_arena, layers, kv_heads, head_dim, max_len, start, src, n_dev, n_max, pos_base=None):
    """ssd_kv_compact_bf16; with ``pos_base`` (a device int32 word) ``start`` is relative to it."""
    _check(k_arena, "k_arena"); _check(vt_arena, "vt_arena")
    if pos_base is not None:
        _check(pos_base, "pos_base", torch.int32)
    _check(src, "src", torch.int32); _check(n_dev, "n", torch.int32)
    _len(src, "src", n_max)
    if k_arena.numel() < layers * kv_heads * max_len * head_dim or vt_arena.numel() < k_arena.numel():
        raise ValueError("kv_compact: arenas smaller than layers * kv_heads * max_len * head_dim")
    _lib.call("ssd_kv_compact_bf16", k_arena.data_ptr(), vt_arena.data_ptr(), layers, kv_heads, head_dim, max_len,
              int(start), src.data_ptr(), n_dev.data_ptr(), int(n_max), _p(pos_base), stream())


_TOPK_WS: dict = {}


def _topk_ws(device, nbytes: int) -> torch.Tensor:
    """Per-device scratch for the row top-k partials (grown on demand, reused across calls)."""
    key = str(device)
    buf = _TOPK_WS.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _TOPK_WS[key] = buf
    return buf


def row_topk(logits, m, n, k, mode, vocab_ids, out_tok, out_val=None, out_lse=None):
    _check(logits, "logits"); _check(out_tok, "out_tok", torch.int32)
    if vocab_ids is not None:
        _check(vocab_ids, "vocab_ids", torch.int32)
        _len(vocab_ids, "vocab_ids", n)
    _len(out_tok, "out_tok", m * k)
    if out_val is not None:
        _check(out_val, "out_val", torch.float32)
        _len(out_val, "out_val", m * k)
    if out_lse is not None:
        _check(out_lse, "out_lse", torch.float32)
        _len(out_lse, "out_lse", m)
    nbytes = int(_lib.load().ssd_row_topk_ws_bytes(m, n))
    ws = _topk_ws(logits.device, nbytes)
    _lib.call("ssd_row_topk_bf16", logits.data_ptr(), _rows(logits, "logits", n, m), m, n, k, mode, _p(vocab_ids),
              out_tok.data_ptr(), _p(out_val), _p(out_lse), ws.data_ptr(), ws.numel(), stream())


def row_topk_ws_bytes(m: int, n: int) -> int:
    return int(_lib.load().ssd_row_topk_ws_bytes(m, n))


def row_topk_partial(logits, m, n, k, mode, parts):
    """The chunk pass of row_topk alone: each row's 4096-column chunk records into ``parts`` (a uint8
    tensor of row_topk_ws_bytes(m, n) bytes), for ssd_tree_level_topk to merge."""
    _check(logits, "logits"); _check(parts, "parts", torch.uint8)
    _len(parts, "parts", row_topk_ws_bytes(m, n))
    _lib.call("ssd_row_topk_partial_bf16", logits.data_ptr(), _rows(logits, "logits", n, m), m, n, k, mode,
              parts.data_ptr(), parts.numel(), stream())


def row_topk_merge(parts, m, s, k, mode, vocab_ids, out_tok, out_val=None, out_lse=None):
    """The merge pass alone over ``s`` records per row (ssd_row_topk_partial_bf16: ceil(n / 4096);
    ssd_gemm_topk_bf16: gemm_topk_parts(n))."""
    _check(parts, "parts", torch.uint8); _check(out_tok, "out_tok", torch.int32)
    if vocab_ids is not None:
        _check(vocab_ids, "vocab_ids", torch.int32)
    _len(out_tok, "out_tok", m * k)
    if out_val is not None:
        _check(out_val, "out_val", torch.float32)
        _len(out_val, "out_val", m * k)
    if out_lse is not None:
        _check(out_lse, "out_lse", torch.float32)
        _len(out_lse, "out_lse", m)
    _lib.call("ssd_row_topk_merge", parts.data_ptr(), parts.numel(), m, s, k, mode, _p(vocab_ids), out_tok.data_ptr(),
              _p(out_val), _p(out_lse), stream())


TOPK_PART_BYTES = 136  # room per record: max, sum of exp, up to 16 keys (stored packed for the call's k)


def gemm_topk_parts(n: int) -> int:
    """Records per row that gemm_topk writes for an n-column head."""
    s = int(_lib.load().ssd_gemm_topk_parts(n))
    if s < 1:
        raise ValueError(f"gemm_topk_parts: bad N={n}")
    return s


def gemm_topk_bytes(m: int, n: int) -> int:
    return m * gemm_topk_parts(n) * TOPK_PART_BYTES


def gemm_topk(x, m, wp, n, k_dim, k, mode, parts, norm_eps: float = 0.0, out=None) -> int:
    """Vocabulary head fused with its top-k chunk pass: ``parts`` (uint8, gemm_topk_bytes(m, n)) gets
    each row's per-slab records of X W^T (k best keys, max, mode 1: sum of exp), for row_topk_merge or
    ssd_tree_level_topk; ``out`` (optional) also receives the bf16 logits. Returns the record count
    per row."""
    _check(x, "x"); _check(wp, "w_packed"); _check(parts, "parts", torch.uint8)
    ldx = _rows(x, "x", k_dim, m)
    _len(wp, "w_packed", packed_elems(n, k_dim))
    _len(parts, "parts", gemm_topk_bytes(m, n))
    ldy = 0
    if out is not None:
        _check(out, "out")
        ldy = _rows(out, "out", n, m)
    _lib.call("ssd_gemm_topk_bf16", x.data_ptr(), ldx, m, wp.data_ptr(), n, k_dim, float(norm_eps), k, mode,
              parts.data_ptr(), parts.numel(), _p(out), ldy, stream())
    return gemm_topk_parts(n)


# ------------------------------------------------------------------ split-K GEMMs
def gemm_splits(n: int, k: int) -> int:
    s = int(_lib.load().ssd_gemm_splits(n, k))
    if s < 1:
        raise ValueError(f"gemm_splits: bad shape N={n} K={k}")
    return s


def part_ld(n: int) -> int:
    """Row stride of split-K partials for an N-column output."""
    return (n + 63) // 64 * 64


def partial_floats(m: int, n: int, k: int) -> int:
    return gemm_splits(n, k) * m * part_ld(n)


def gemm_partial(x, m, wp, n, k, part):
    """part[s*m*ldp + r*ldp + c] = sum over the s-th K range of x[r] . W[c] (fp32); returns (S, ldp)."""
    _check(x, "x"); _check(wp, "w_packed"); _check(part, "partials", torch.float32)
    _len(wp, "w_packed", packed_elems(n, k))
    s, ld = gemm_splits(n, k), part_ld(n)
    _len(part, "partials", s * m * ld)
    _lib.call("ssd_gemm_partial_bf16", x.data_ptr(), _rows(x, "x", k, m), m, wp.data_ptr(), n, k, part.data_ptr(), ld,
              m * ld, stream())
    return s, ld


def gemm_finalize(part, s, ld, m, n, out, bias=None, act=None, residual=None):
    _check(part, "partials", torch.float32); _check(out, "out")
    if bias is not None:
        _check(bias, "bias")
    if residual is not None:
        _check(residual, "residual")
    _len(part, "partials", s * m * ld)
    _lib.call("ssd_gemm_finalize_bf16", part.data_ptr(), ld, m * ld, s, m, n, out.data_ptr(), _rows(out, "out", n, m),
              _p(bias), ACT[act], _p(residual), 0 if residual is None else _rows(residual, "residual", n, m), stream())
    return out


def qkv_rope_finalize(part, s, ld, m, heads, kv_heads, head_dim, cos, sin, pos, slot, q_out, k_cache, vt_cache, max_len):
    _check(part, "partials", torch.float32); _check(q_out, "q"); _check(k_cache, "k_cache"); _check(vt_cache, "vt")
    for t, nm in ((pos, "pos"), (slot, "slot")):
        _check(t, nm, torch.int32)
        _len(t, nm, m)
    _len(part, "partials", s * m * ld)
    if k_cache.numel() < kv_heads * max_len * head_dim or vt_cache.numel() < kv_heads * max_len * head_dim:
        raise ValueError("qkv_rope_finalize: cache smaller than kv_heads * max_len * head_dim")
    if cos.shape != sin.shape or cos.dim() != 2 or cos.shape[1] != head_dim // 2:
        raise ValueError("qkv_rope_finalize: cos/sin must be [rows, head_dim/2]")
    _lib.call("ssd_qkv_rope_finalize_bf16", part.data_ptr(), ld, m * ld, s, m, heads, kv_heads, head_dim,
              cos.data_ptr(), sin.data_ptr(), cos.shape[0], pos.data_ptr(), slot.data_ptr(), q_out.data_ptr(),
              _rows(q_out, "q", heads * head_dim, m), k_cache.data_ptr(), vt_cache.data_ptr(), max_len, stream())


def residual_group(n: int, k: int) -> int:
    g = int(_lib.load().ssd_gemm_residual_group(n, k))
    if g < 1:
        raise ValueError(f"residual_group: bad shape N={n} K={k}")
    return g


def residual_floats(m: int, n: int, k: int) -> int:
    """fp32 scratch of gemm_residual for m rows of an [n, k] projection (0: none needed)."""
    return int(_lib.load().ssd_gemm_residual_floats(m, n, k))


def gemm_residual(x, m, wp, n, k, h, part, bias=None):
    """h[:m] <- bf16(h + bf16(x W^T + bias)) (W packed with residual=True)."""
    _check(x, "x"); _check(wp, "w_packed"); _check(h, "h")
    if bias is not None:
        _check(bias, "bias"); _len(bias, "bias", n)
    need = residual_floats(m, n, k)
    if need:
        _check(part, "part", torch.float32)
        _len(part, "part", need)
    _len(wp, "w_packed", packed_elems(n, k))
    _lib.call("ssd_gemm_residual_bf16", x.data_ptr(), _rows(x, "x", k, m), m, wp.data_ptr(), n, k, _p(bias),
              h.data_ptr(), _rows(h, "h", n, m), _p(part) if need else None, part.numel() if need else 0, stream())
    return h


def mlp_group(inter: int, hidden: int) -> int:
    """Packing group of the gate/up weight for the fused MLP (0: no fused plan for this shape)."""
    return int(_lib.load().ssd_mlp_group(inter, hidden))


def mlp_sync_words() -> int:
    return int(_lib.load().ssd_mlp_sync_words())


def mlp_timeout_word() -> int:
    """Index of the word in an mlp sync buffer that counts flag waits that gave up."""
    return int(_lib.load().ssd_mlp_timeout_word())


def mlp_sync(device) -> torch.Tensor:
    """Zeroed flag words for mlp (one buffer per stream; word mlp_timeout_word() counts timeouts)."""
    return torch.zeros(mlp_sync_words(), dtype=torch.int32, device=device)


def check_mlp_timeouts(count: int) -> None:
    """Raises SsdError for a nonzero timeout count read from an mlp sync buffer."""
    if count:
        raise _lib.SsdError(
            f"fused MLP: {count} flag waits gave up (the device did not run all 256 workgroups at once: "
            "another stream or process held compute units); results computed since the count was zero are invalid")


def mlp(h, m, wgu, wd, inter, hidden, eps, act, part, sync):
    """h[:m] <- h + down(SwiGLU(RMSNorm(h))) in one cooperative launch (wgu packed with
    group=mlp_group(inter, hidden) and the ln2 weight as col_scale, wd with residual=True)."""
    _check(h, "h"); _check(wgu, "wgu"); _check(wd, "wd"); _check(act, "act")
    _check(part, "part", torch.float32); _check(sync, "sync", torch.int32)
    need = residual_floats(min(m, 64), hidden, inter)
    _len(part, "part", need)
    _len(sync, "sync", int(_lib.load().ssd_mlp_sync_words()))
    _len(wgu, "wgu", packed_elems(2 * inter, hidden))
    _len(wd, "wd", packed_elems(hidden, inter))
    _lib.call("ssd_mlp_bf16", h.data_ptr(), _rows(h, "h", hidden, m), m, wgu.data_ptr(), wd.data_ptr(), inter, hidden,
              float(eps), act.data_ptr(), _rows(act, "act", inter, m), part.data_ptr(), part.numel(), sync.data_ptr(),
              stream())
    return h


def add_rmsnorm(part, s, ld, h, m, w, eps, out, bias=None):
    """h[:m] <- bf16(h + bf16(sum of the s partials + bias)) (s = 0: unchanged); out[:m] <- RMSNorm(h) * w."""
    _check(h, "h")
    d = h.shape[1]
    if s:
        _check(part, "partials", torch.float32)
        _len(part, "partials", s * m * ld)
    if bias is not None:
        _check(bias, "bias")
    if out is not None:
        _check(out, "out"); _check(w, "w")
    _lib.call("ssd_add_rmsnorm_bf16", part.data_ptr() if s else None, ld if s else 0, m * ld if s else 0, s, _p(bias),
              h.data_ptr(), _rows(h, "h", d, m), m, d, None if out is None else w.data_ptr(), float(eps),
              _p(out), 0 if out is None else _rows(out, "out", d, m), stream())
    return out


# ------------------------------------------------------------------------ sampling
def sample_ws_bytes(rows: int, n: int) -> int:
    b = int(_lib.load().ssd_sample_ws_bytes(rows, n))
    if b < 0:
        raise ValueError(f"sampling workspace: {n} columns beyond the compiled limit")
    return b


_SMP_WS: dict = {}


def sample_ws(device, rows: int, n: int) -> torch.Tensor:
    """A reusable workspace for the sampling kernels on ``device`` (grown on demand)."""
    need = sample_ws_bytes(rows, n)
    buf = _SMP_WS.get(str(device))
    if buf is None or buf.numel() < need:
        buf = torch.empty(need, dtype=torch.uint8, device=device)
        _SMP_WS[str(device)] = buf
    return buf


def warp_probs(logits, rows, n, temperature, top_p, out, V=None, vocab_ids=None, vocab_inv=None, tree_meta=None,
               level=0, ws=None):
    """softmax(logits / T) + nucleus cut per row into fp32 ``out`` [*, V] (ssd_warp_probs_bf16)."""
    _check(logits, "logits"); _check(out, "probs", torch.float32)
    V = n if V is None else V
    if vocab_ids is not None:
        _check(vocab_ids, "vocab_ids", torch.int32); _len(vocab_ids, "vocab_ids", n)
        _check(vocab_inv, "vocab_inv", torch.int32); _len(vocab_inv, "vocab_inv", V)
    if tree_meta is not None:
        _check(tree_meta, "tree_meta", torch.int32)
    elif out.shape[0] < rows:
        raise ValueError(f"probs has {out.shape[0]} rows < {rows}")
    ws = sample_ws(logits.device, rows, V) if ws is None else ws
    _lib.call("ssd_warp_probs_bf16", logits.data_ptr(), _rows(logits, "logits", n, rows), rows, n, _p(vocab_ids),
              _p(vocab_inv), V, float(temperature), float(top_p), _p(tree_meta), level, out.data_ptr(),
              _rows(out, "probs", V), ws.data_ptr(), ws.numel(), stream())
    return out


def gumbel_topk(probs, rows, V, k, seed, counter, out_tok, out_lp, tree_meta=None, level=0, ws=None):
    _check(probs, "probs", torch.float32); _check(out_tok, "out_tok", torch.int32)
    _check(out_lp, "out_lp", torch.float32)
    _len(out_tok, "out_tok", rows * k); _len(out_lp, "out_lp", rows * k)
    if tree_meta is not None:
        _check(tree_meta, "tree_meta", torch.int32)
    ws = sample_ws(probs.device, rows, V) if ws is None else ws
    _lib.call("ssd_gumbel_topk", probs.data_ptr(), _rows(probs, "probs", V), rows, V, k, _p(tree_meta), level,
              seed & (2**64 - 1), counter & (2**64 - 1), out_tok.data_ptr(), out_lp.data_ptr(), ws.data_ptr(),
              ws.numel(), stream())


def sample_rows(probs, rows, V, seed, counter, out_tok, ws=None):
    _check(probs, "probs", torch.float32); _check(out_tok, "out_tok", torch.int32)
    _len(out_tok, "out_tok", rows)
    ws = sample_ws(probs.device, rows, V) if ws is None else ws
    _lib.call("ssd_sample_rows", probs.data_ptr(), _rows(probs, "probs", V, rows), rows, V, seed & (2**64 - 1),
              counter & (2**64 - 1), out_tok.data_ptr(), ws.data_ptr(), ws.numel(), stream())
    return out_tok


def sample_top64(logits, rows, V, temperature, top_p, seed, counter, out_tok):
    """sample_next at temperature > 0 (ssd_sample_top64_bf16): per row, one draw among the 64
    largest logits after the temperature + nucleus warp of those 64."""
    _check(logits, "logits"); _check(out_tok, "out_tok", torch.int32)
    _len(out_tok, "out_tok", rows)
    need = int(_lib.load().ssd_sample_top64_ws_bytes(rows, V))
    if need < 0:
        raise RuntimeError(f"sample_next: top-64 needs 64 <= V <= 262144 columns, got V={V}")
    ws = _topk_ws(logits.device, need)
    _lib.call("ssd_sample_top64_bf16", logits.data_ptr(), _rows(logits, "logits", V, rows), rows, V,
              float(temperature), float(top_p), seed & (2**64 - 1), counter & (2**64 - 1), out_tok.data_ptr(),
              ws.data_ptr(), ws.numel(), stream())
    return out_tok


def accept_sample_trials(P, Q, rows, branch, seed, counter0, trials, out_tokens, out_n):
    """ssd_accept_sample_trials: ``trials`` independent proposal + acceptance rounds of the
    unpruned tree ``branch`` over the fixed per-node rows of P and Q (row 0 the root); the
    per-row supports are derived here (columns where P or Q is nonzero)."""
    _check(P, "P", torch.float32); _check(Q, "Q", torch.float32)
    _check(out_tokens, "out_tokens", torch.int32); _check(out_n, "out_n", torch.int32)
    depth = len(branch)
    _len(out_tokens, "out_tokens", trials * (depth + 1)); _len(out_n, "out_n", trials)
    nz = (P[:rows] > 0) | (Q[:rows] > 0)
    counts = nz.sum(1)
    off = torch.zeros(rows + 1, dtype=torch.int32, device=P.device)
    off[1:] = torch.cumsum(counts, 0).to(torch.int32)
    cols = torch.nonzero(nz)[:, 1].to(torch.int32).contiguous()  # row-major: ascending within a row
    br = (ctypes.c_int32 * depth)(*branch)
    _lib.call("ssd_accept_sample_trials", P.data_ptr(), P.stride(0), Q.data_ptr(), Q.stride(0), rows,
              cols.data_ptr(), off.data_ptr(), depth, br, int(seed), int(counter0), int(trials), out_tokens.data_ptr(),
              out_n.data_ptr(), stream())
    torch.cuda.current_stream().synchronize()  # cols / off are temporaries of this call


def accept_sample(tree_struct, P, Q, V, rows, max_kids, seed, counter, committed, result, keep_src, n_keep,
                  root_token, ws=None):
    """ssd_accept_sample: speculative-sampling walk over the finalized tree (P: warped target rows,
    Q: warped draft rows at 1 + draft node index, row 0 the root)."""
    _check(P, "P", torch.float32); _check(Q, "Q", torch.float32)
    for t, name in ((result, "result"), (keep_src, "keep_src"), (n_keep, "n_keep"), (root_token, "root_token")):
        _check(t, name, torch.int32)
    ws = sample_ws(P.device, rows, V) if ws is None else ws
    _lib.call("ssd_accept_sample", tree_struct, P.data_ptr(), _rows(P, "P", V, rows), Q.data_ptr(),
              _rows(Q, "Q", V), V, rows, max_kids, seed & (2**64 - 1), counter & (2**64 - 1), ws.data_ptr(),
              ws.numel(), committed, result.data_ptr(), keep_src.data_ptr(), n_keep.data_ptr(), root_token.data_ptr(),
              stream())
