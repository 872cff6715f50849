"""Sampling-path restatement with counter-based randomness (test infrastructure only).

The reference draws from torch's CPU generator (``exponential_`` in
ssd/engine/tree_drafter.py:141, ``torch.rand`` in ssd/engine/verify.py:80, ``multinomial`` in
verify.py:94 and ssd/engine/speculative.py:84). The HIP path draws from Philox4x32-10 instead,
so this module restates the same algorithms with the same Philox streams the kernels use:
given a seed and a round counter, every decision is then determined and the GPU can be
checked draw for draw. Pinning:

* ``philox4x32_10`` against the generator's published known-answer vectors (Random123
  ``kat_vectors``: counter/key all zero, all ones, and the pi-digit pattern);
* ``warp_probs`` is the reference's rule with a stable sort (equal probabilities keep lower
  columns first); it is checked against hand-derived nucleus cases and against
  ``oracle.engine.warp_probs`` wherever no two probabilities tie;
* ``sample_verify`` is the reference loop of verify.py:60-95 verbatim, with its three random
  sources replaced by Philox streams; the claim that it samples the warped target exactly
  (the speculative-sampling theorem) is checked by a chi-square test of the first committed
  token and by the brute-force V=8 joint of the reference's own test;
* ``sample_verify_states`` restates the GPU's formulation (all rejection states of a node
  precomputed, then a scalar walk) and is checked against ``sample_verify`` decision for
  decision on random trees.

Every function returns, next to its result, a ``fragile`` flag: true when a decision hinged
on a margin below ``MARGIN`` (a uniform within that relative distance of the acceptance
ratio, two Gumbel keys that close, a nucleus boundary that close to top_p). fp32 rounding
differences between the CPU and the GPU may flip such decisions and nothing else.
"""

from __future__ import annotations

from typing import Optional

import numpy as np
import torch

ROOT = -1
MARGIN = 1e-4

TAG_PROPOSE, TAG_ACCEPT, TAG_BONUS, TAG_DRAW, TAG_TOP64 = 1, 2, 3, 4, 5

_M0, _M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
_W0, _W1 = np.uint32(0x9E3779B9), np.uint32(0xBB67AE85)
_LO = np.uint64(0xFFFFFFFF)


def philox4x32_10(c0, c1, c2, c3, k0, k1):
    """Philox4x32 with 10 rounds (Salmon et al., SC 2011), vectorised over numpy uint32 arrays.
    Returns four uint32 arrays."""
    c = [np.asarray(x, dtype=np.uint64) & _LO for x in (c0, c1, c2, c3)]
    c0, c1, c2, c3 = np.broadcast_arrays(*c)
    c0, c1, c2, c3 = (x.copy() for x in (c0, c1, c2, c3))
    k0 = np.uint64(int(k0) & 0xFFFFFFFF)
    k1 = np.uint64(int(k1) & 0xFFFFFFFF)
    for _ in range(10):
        p0 = _M0 * c0
        p1 = _M1 * c2
        hi0, lo0 = p0 >> np.uint64(32), p0 & _LO
        hi1, lo1 = p1 >> np.uint64(32), p1 & _LO
        c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
        k0 = (k0 + np.uint64(0x9E3779B9)) & _LO
        k1 = (k1 + np.uint64(0xBB67AE85)) & _LO
    return tuple(x.astype(np.uint32) for x in (c0, c1, c2, c3))


class Stream:
    """The kernels' counter layout: key = seed; counter = (index, row | level << 16,
    round counter low word, round counter high bits << 8 | tag)."""

    def __init__(self, seed: int, counter: int):
        self.k0, self.k1 = seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF
        self.c2 = counter & 0xFFFFFFFF
        self.c3 = ((counter >> 32) << 8) & 0xFFFFFFFF

    def bits(self, idx, c1: int, tag: int):
        """uint32 words of counters (idx, c1, ...); returns a [len(idx), 4] array."""
        out = philox4x32_10(np.asarray(idx, dtype=np.uint32), np.uint32(c1), np.uint32(self.c2),
                            np.uint32(self.c3 | tag), self.k0, self.k1)
        return np.stack(out, -1)

    def element_bits(self, V: int, c1: int, tag: int) -> np.ndarray:
        """One 32-bit word per element y < V: word y % 4 of counter y // 4."""
        quads = np.arange((V + 3) // 4, dtype=np.uint32)
        return self.bits(quads, c1, tag).reshape(-1)[:V]


def exp1_from_bits(b: np.ndarray) -> np.ndarray:
    """-log(U), U = (b + 1/2) / 2^32, in fp32: the lower half of U directly, the upper half
    through 1 - U (the kernels' rule)."""
    b = np.asarray(b, dtype=np.uint32)
    lo = b < np.uint32(0x80000000)
    u = (b.astype(np.float32) + np.float32(0.5)) * np.float32(2.0 ** -32)
    v = ((~b).astype(np.float32) + np.float32(0.5)) * np.float32(2.0 ** -32)
    with np.errstate(divide="ignore"):
        return np.where(lo, -np.log(u), -np.log1p(-v)).astype(np.float32)


def uniform_from_bits(b) -> float:
    return (float(int(b)) + 0.5) * 2.0 ** -32


# ---------------------------------------------------------------------------- warp
def warp_probs(logits: torch.Tensor, temperature: float, top_p: float):
    """ssd/engine/tree_drafter.py:34-45 with a stable descending sort. Returns (probs, fragile)."""
    probs = torch.softmax(logits.float() / temperature, dim=-1)
    fragile = False
    if top_p < 1.0:
        sp, idx = probs.sort(dim=-1, descending=True, stable=True)
        before = sp.cumsum(-1) - sp
        drop = before > top_p
        gap = (before - top_p).abs()
        fragile = bool((gap < MARGIN).any())
        sp = sp.masked_fill(drop, 0.0)
        probs = torch.zeros_like(probs).scatter(-1, idx, sp)
        probs = probs / probs.sum(-1, keepdim=True)
    return probs, fragile


def warp_probs64(logits: torch.Tensor, temperature: float, top_p: float, band: float = 1e-5):
    """The same rule in float64 from the given (bf16-valued) logits, as the checker of a kernel
    that accumulates mass exactly: returns (probabilities, kept mask, boundary band mask). The band
    holds the entries whose preceding mass lies within ``band`` of top_p: fp32 rounding of p may
    move them across the cut, nothing else may differ. With top_p >= 1 nothing is cut and the
    probabilities are not renormalised (tree_drafter.py:39)."""
    p = torch.softmax(logits.double() / temperature, dim=-1)
    if top_p >= 1.0:
        return p, torch.ones_like(p, dtype=torch.bool), torch.zeros_like(p, dtype=torch.bool)
    sp, idx = p.sort(dim=-1, descending=True, stable=True)
    before = sp.cumsum(-1) - sp
    kept = torch.zeros_like(p, dtype=torch.bool).scatter(-1, idx, before <= top_p)
    near = torch.zeros_like(p, dtype=torch.bool).scatter(-1, idx, (before - top_p).abs() <= band)
    return p, kept, near


def scatter_vocab(probs: torch.Tensor, vocab_ids: Optional[torch.Tensor], V: int) -> torch.Tensor:
    """Draft-vocab columns back to the full vocabulary, zero elsewhere (tree_drafter.py:134-137)."""
    if vocab_ids is None:
        return probs
    full = torch.zeros(*probs.shape[:-1], V)
    return full.index_copy_(-1, vocab_ids.long(), probs)


# ------------------------------------------------------------------ Gumbel top-k
def gumbel_topk(q: torch.Tensor, k: int, stream: Stream, row: int, level: int):
    """min(k, |support|) draws without replacement from q in draw order (tree_drafter.py:138-144):
    the largest keys q(y) / E(y), E(y) = Exp(1) from the PROPOSE stream. Returns
    (tokens, log q of each, fragile)."""
    qn = q.float().numpy()
    V = qn.shape[0]
    e = exp1_from_bits(stream.element_bits(V, row | (level << 16), TAG_PROPOSE))
    support = int((qn > 0).sum())
    with np.errstate(divide="ignore", invalid="ignore"):
        keys = np.where(qn > 0, qn.astype(np.float32) / e, -1.0).astype(np.float32)
    order = np.lexsort((np.arange(V), -keys.astype(np.float64)))  # key desc, then index asc
    take = min(k, support)
    toks = order[:take].tolist()
    fragile = False
    if support > take:  # the k-th and (k+1)-th keys
        a, b = keys[order[take - 1]], keys[order[take]]
        fragile = abs(a - b) <= MARGIN * abs(a)
    for i in range(take - 1):
        a, b = keys[order[i]], keys[order[i + 1]]
        fragile |= abs(a - b) <= MARGIN * abs(a)
    lps = [float(np.log(np.float32(qn[t]))) for t in toks]
    return toks, lps, bool(fragile)


def categorical(p: torch.Tensor, stream: Stream, row: int, tag: int = TAG_DRAW, c1: Optional[int] = None):
    """One draw: argmax_y p(y) / E(y) over p(y) > 0, lower index first among equal keys
    (the Gumbel-max form of torch.multinomial(p, 1)). Returns (token, fragile)."""
    pn = p.float().numpy().astype(np.float32)
    V = pn.shape[0]
    e = exp1_from_bits(stream.element_bits(V, row if c1 is None else c1, tag))
    with np.errstate(divide="ignore", invalid="ignore"):
        keys = np.where(pn > 0, pn / e, -1.0)
    order = np.lexsort((np.arange(V), -keys.astype(np.float64)))
    a, b = keys[order[0]], keys[order[1]] if V > 1 else -1.0
    return int(order[0]), bool(V > 1 and b > 0 and abs(a - b) <= MARGIN * abs(a))


def sample_next_top64(logits: torch.Tensor, temperature: float, top_p: float, stream: Stream, row: int,
                      k: int = 64):
    """sample_next at temperature > 0 (ssd/data/generate_selfdistill.py:50-60): the k largest
    logits of the row (equal logits: lower column first), warp_probs over those k alone, one
    draw among them (Gumbel-max over the k ranks, Exp(1) of rank j from the TAG_TOP64 stream).
    Returns (column, fragile)."""
    x = logits.float()
    order = np.lexsort((np.arange(x.shape[0]), -x.numpy().astype(np.float64)))[:k]
    p, fr = warp_probs(x[torch.from_numpy(order)], temperature, top_p)
    j, fr2 = categorical(p, stream, row, TAG_TOP64)
    return int(order[j]), fr or fr2


def top64_probs(logits: torch.Tensor, temperature: float, top_p: float, k: int = 64) -> torch.Tensor:
    """The distribution sample_next draws from, over the full row: warp_probs of the k largest
    logits, zero elsewhere (float64)."""
    x = logits.double()
    order = np.lexsort((np.arange(x.shape[0]), -x.numpy()))[:k]
    idx = torch.from_numpy(order)
    p, _ = warp_probs(x[idx].float(), temperature, top_p)
    return torch.zeros(x.shape[0], dtype=torch.float64).index_copy_(0, idx, p.double())


# ---------------------------------------------------------------- acceptance
def children(tokens, parents, ranks) -> dict:
    out: dict = {}
    for i, p in enumerate(parents):
        out.setdefault(p, []).append(i)
    for kids in out.values():
        kids.sort(key=lambda i: ranks[i])
    return out


def sample_verify(tokens, parents, ranks, P: torch.Tensor, child_q: dict, stream: Stream, _residual: bool = True):
    """verify.py:60-95, loop for loop. Row r = cur + 1 of P is the warped target at node cur;
    child_q[cur] the warped draft distribution its children were drawn from. Random sources:
    the uniform for the j-th rejection test at row r is word 0 of counter (j, r, ACCEPT); the
    bonus is the Gumbel-max draw with the shared BONUS vector. Returns (accepted, bonus, fragile).
    ``_residual=False`` drops the residual update: a planted mistake for the negative control."""
    kids = children(tokens, parents, ranks)
    V = P.shape[1]
    e_bonus = torch.from_numpy(exp1_from_bits(stream.element_bits(V, 0, TAG_BONUS)))
    accepted, cur, fragile = [], ROOT, False
    while True:
        r = cur + 1
        p = P[r].float().clone()
        chosen, j = None, 0
        if kids.get(cur):
            q = child_q[cur].float().clone()
            for c in kids[cur]:
                x = tokens[c]
                if q[x] <= 0:
                    continue
                u = uniform_from_bits(stream.bits([j], r, TAG_ACCEPT)[0, 0])
                ratio = min(1.0, (p[x] / q[x]).item())
                fragile |= abs(u - ratio) <= MARGIN * max(ratio, 1e-30)
                if u < ratio:
                    chosen = c
                    break
                residual = (p - q).clamp_min(0)
                if _residual and residual.sum() > 0:
                    p = residual / residual.sum()
                q[x] = 0
                j += 1
                if q.sum() <= 0:
                    break
                q = q / q.sum()
            if chosen is not None:
                accepted.append(chosen)
                cur = chosen
                continue
        keys = torch.where(p > 0, p / e_bonus, torch.full_like(p, -1.0))
        top = torch.topk(keys, min(2, V))
        bonus = int(torch.nonzero(keys == top.values[0])[0])
        if V > 1 and top.values[1] > 0:
            fragile |= bool((top.values[0] - top.values[1]).abs() <= MARGIN * top.values[0].abs())
        return accepted, bonus, bool(fragile)


def sample_verify_states(tokens, parents, ranks, P: torch.Tensor, child_q: dict, stream: Stream):
    """The GPU formulation: for every node, the rejection states j = 0..n (p_j, q_j as scalars
    zr[j], zq[j] over q0 and p) and each state's bonus draw are precomputed; the walk then only
    evaluates p_j(x) / q_j(x) at the children. Same random sources as ``sample_verify``.
    Returns (accepted, bonus)."""
    kids = children(tokens, parents, ranks)
    V = P.shape[1]
    e_bonus = torch.from_numpy(exp1_from_bits(stream.element_bits(V, 0, TAG_BONUS)))

    def draw(w):
        keys = torch.where(w > 0, w / e_bonus, torch.full_like(w, -1.0))
        return int(torch.argmax(keys))  # first maximal index

    states = {}
    for cur in [ROOT] + list(range(len(tokens))):
        p0 = P[cur + 1].float()
        ks = [c for c in kids.get(cur, []) if child_q[cur][tokens[c]] > 0]
        st = {"kids": ks, "bonus": [draw(p0)], "zr": [0.0], "zq": [1.0], "supp": 0}
        if ks:
            q0 = child_q[cur].float()
            st["supp"] = int((q0 > 0).sum())
            s0 = q0.double().sum().item()
            rej = []
            pj, qj = p0, q0
            for c in ks:
                x = tokens[c]
                res = (pj - qj).clamp_min(0)
                z = res.double().sum().item()
                st["zr"].append(z)
                st["bonus"].append(draw(res) if z > 0 else st["bonus"][-1])
                pj = res / z if z > 0 else pj
                rej.append(x)
                s0 -= q0[x].item()
                st["zq"].append(s0)
                qj = q0.clone()
                qj[rej] = 0
                qj = qj / s0
        states[cur] = st
    accepted, cur = [], ROOT
    while True:
        st = states[cur]
        r = cur + 1
        q0 = child_q[cur].float() if st["kids"] else None
        chosen, j = None, 0
        for c in st["kids"]:
            x = tokens[c]
            # p_j(x): chain over the states (x itself was never rejected)
            pv = P[r, x].float().item()
            for i in range(1, j + 1):
                qv = q0[x].item() if i == 1 else q0[x].item() / st["zq"][i - 1]
                if st["zr"][i] > 0:
                    pv = max(pv - qv, 0.0) / st["zr"][i]
            qv = q0[x].item() if j == 0 else q0[x].item() / st["zq"][j]
            u = uniform_from_bits(stream.bits([j], r, TAG_ACCEPT)[0, 0])
            if u < min(1.0, pv / qv):
                chosen = c
                break
            j += 1
            if j >= st["supp"]:
                break
        if chosen is None:
            return accepted, st["bonus"][j]
        accepted.append(chosen)
        cur = chosen
