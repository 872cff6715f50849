"""Per-kernel CPU references (test infrastructure only).

Each function states, in fp32 on the CPU, what one HIP entry point computes, with the
reference's bf16 rounding points (ssd/models/subnetwork_draft.py:209-245, bridges.py:131-135,
HF RMSNorm/RoPE/MLP). They are pinned through ``oracle.model``: the model forward composed
from them equals ``oracle.model.Subnetwork`` (itself pinned to transformers' Llama), see
tests/test_oracle_kernels.py.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from oracle.model import ACTS, rope_cos_sin


def rbf(x: torch.Tensor) -> torch.Tensor:
    """Round fp32 through bf16."""
    return x.to(torch.bfloat16).float()


def linear(x: torch.Tensor, w: torch.Tensor, bias=None, act=None, residual=None) -> torch.Tensor:
    """bf16 nn.Linear chain: rnd(x W^T + b) -> rnd(act(.)) -> rnd(residual + .). fp32 out."""
    y = x.float() @ w.float().T
    if bias is not None:
        y = y + bias.float()
    y = rbf(y)
    if act is not None:
        y = rbf(ACTS[act](y))
    if residual is not None:
        y = rbf(residual.float() + y)
    return y


def swiglu(x: torch.Tensor, wg: torch.Tensor, wu: torch.Tensor, bg=None, bu=None) -> torch.Tensor:
    """rnd(rnd(silu(rnd(x Wg^T + bg))) * rnd(x Wu^T + bu)) -- HF LlamaMLP before down_proj."""
    g = linear(x, wg, bg)
    u = linear(x, wu, bu)
    return rbf(rbf(F.silu(g)) * u)


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    r = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return rbf(w.float() * rbf(xf * r))


def rope(x: torch.Tensor, pos: torch.Tensor, theta: float) -> torch.Tensor:
    """x [M, H, hd] (bf16-valued fp32) at positions pos[M]: rnd(rnd(x cos) + rnd(rot(x) sin))."""
    hd = x.shape[-1]
    cos, sin = rope_cos_sin(pos, hd, theta, torch.bfloat16)
    cos, sin = cos.float()[:, None], sin.float()[:, None]
    h = hd // 2
    rot = torch.cat([-x[..., h:], x[..., :h]], -1)
    return rbf(rbf(x * cos) + rbf(rot * sin))


def qkv_rope(x, wq, wk, wv, heads, kv_heads, hd, pos, theta):
    """Returns q [M, heads, hd], k [M, kv, hd] (RoPE'd), v [M, kv, hd], all bf16-valued fp32."""
    m = x.shape[0]
    q = linear(x, wq).view(m, heads, hd)
    k = linear(x, wk).view(m, kv_heads, hd)
    v = linear(x, wv).view(m, kv_heads, hd)
    return rope(q, pos, theta), rope(k, pos, theta), v


def tree_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, prefix: list, anc: list,
                   scale: float = None) -> torch.Tensor:
    """q [M, Hq, hd]; k/v [Hkv, S, hd] (cache rows by slot). Row t attends slots [0, prefix[t])
    plus anc[t]. Exact fp32 softmax attention -> [M, Hq, hd] fp32."""
    m, hq, hd = q.shape
    hkv, s_len, _ = k.shape
    rep = hq // hkv
    scale = 1.0 / math.sqrt(hd) if scale is None else scale
    out = torch.empty(m, hq, hd)
    for t in range(m):
        slots = list(range(prefix[t])) + list(anc[t])
        idx = torch.tensor(slots, dtype=torch.long)
        kk = k.float()[:, idx].repeat_interleave(rep, 0)  # [Hq, n, hd]
        vv = v.float()[:, idx].repeat_interleave(rep, 0)
        s = torch.einsum("hd,hnd->hn", q[t].float(), kk) * scale
        out[t] = torch.einsum("hn,hnd->hd", torch.softmax(s, -1), vv)
    return out


def kv_compact(k: torch.Tensor, start: int, src: list) -> torch.Tensor:
    """Gather rows src -> [start, start+n) along dim -2 of k [..., S, hd] (all sources read first)."""
    out = k.clone()
    out[..., start:start + len(src), :] = k[..., torch.tensor(src, dtype=torch.long), :]
    return out


def log_softmax_topk(logits: torch.Tensor, k: int):
    """Per row: (values, columns) of the k best log-softmax entries, ties lower column first;
    plus the logsumexp."""
    x = logits.float()
    lp = F.log_softmax(x, -1)
    vals, idx = torch.sort(lp, dim=-1, descending=True, stable=True)
    return vals[:, :k], idx[:, :k], torch.logsumexp(x, -1)


def argmax_first(logits: torch.Tensor) -> torch.Tensor:
    """First index of the row maximum."""
    x = logits.float()
    mx = x.max(-1, keepdim=True).values
    ar = torch.arange(x.shape[-1]).expand_as(x)
    return torch.where(x == mx, ar, x.shape[-1]).min(-1).values
