"""Tree verification API (reference ssd/engine/verify.py).

The round loop verifies on the device (``ssd_tree_finalize`` builds the verify rows,
``ssd_row_topk_bf16`` k=1 takes the first-index argmax, ``ssd_accept_greedy`` walks the
tree). These functions keep the reference's host-level signatures for callers that hold a
``DraftTree``.
"""

from __future__ import annotations

import torch

from ssd import ops
from ssd.engine.tree_drafter import ROOT, DraftTree


def verify_inputs(tree: DraftTree, root_token: int, root_pos: int, past_len: int, device) -> tuple:
    """ids [1, n+1], positions [1, n+1], bool mask [n+1, past+n+1]; row 0 is the root
    (reference verify.py:32-42)."""
    n = len(tree)
    ids = torch.tensor([[root_token] + tree.tokens], device=device)
    pos = torch.tensor([[root_pos] + [root_pos + d for d in tree.depths]], device=device)
    mask = torch.zeros(n + 1, past_len + n + 1, dtype=torch.bool)
    mask[:, : past_len + 1] = True
    for i in range(n):
        for a in tree.ancestors(i):
            mask[i + 1, past_len + 1 + a] = True
    return ids, pos, mask.to(device)


def row_argmax(logits: torch.Tensor) -> list:
    """First-index argmax of each row of bf16 logits [rows, V] on the device."""
    lg = logits.reshape(-1, logits.shape[-1])
    if lg.dtype != torch.bfloat16 or lg.stride(-1) != 1 or lg.shape[-1] % 8 or lg.stride(0) % 8:
        pad = (lg.shape[-1] + 7) // 8 * 8
        buf = torch.full((lg.shape[0], pad), float("-inf"), dtype=torch.bfloat16, device=lg.device)
        buf[:, : lg.shape[-1]] = lg
        lg = buf
    out = torch.zeros(lg.shape[0], dtype=torch.int32, device=lg.device)
    ops.row_topk(lg, lg.shape[0], logits.shape[-1], 1, 0, None, out)
    return out.tolist()


def greedy_verify(tree: DraftTree, target_logits: torch.Tensor) -> tuple:
    """Walk root -> child whose token is the target argmax; the first miss gives the bonus
    token (reference verify.py:45-57)."""
    argmax = row_argmax(target_logits)
    kids = tree.children()
    accepted, cur = [], ROOT
    while True:
        want = argmax[cur + 1]
        nxt = next((c for c in kids.get(cur, []) if tree.tokens[c] == want), None)
        if nxt is None:
            return accepted, want
        accepted.append(nxt)
        cur = nxt


def sample_verify(tree: DraftTree, target_logits: torch.Tensor, temperature: float, top_p: float,
                  generator=None) -> tuple:
    """Speculative sampling over the tree (reference verify.py:60-95) on the device: the target
    rows are warped by ``ssd_warp_probs_bf16`` and walked by ``ssd_accept_sample``. ``tree.child_q``
    maps each node with children (and the root, -1) to the warped draft distribution its children
    were drawn from (trees built by a sampled ``TreeDrafter.build`` carry them). The Philox seed is
    drawn from ``generator``. Returns (accepted node indices, bonus token)."""
    from ssd.engine.sampling import Sampler, seed_from_generator
    from ssd.engine.tree_drafter import DeviceTree

    V = target_logits.shape[-1]
    lg = target_logits.reshape(-1, V)
    n = len(tree)
    if lg.shape[0] < n + 1:
        raise ValueError(f"target_logits has {lg.shape[0]} rows, the tree needs {n + 1}")
    dev = lg.device
    sampler = Sampler(temperature, top_p, V, dev, 1 + n, n + 1, seed_from_generator(generator))
    sampler.max_kids = max([tree.parents.count(p) for p in set(tree.parents)] + [1])
    for p in set(tree.parents):
        sampler.Q[0 if p == ROOT else 1 + p, :V] = torch.as_tensor(tree.child_q[p], device=dev).float()
    dt = DeviceTree(dev, cap=max(n, 1))
    if n:
        i32 = dict(dtype=torch.int32, device=dev)
        dt.vtokens[:n] = torch.tensor(tree.tokens, **i32)
        dt.vparents[:n] = torch.tensor(tree.parents, **i32)
        dt.vranks[:n] = torch.tensor(tree.ranks, **i32)
        dt.vdepths[:n] = torch.tensor(tree.depths, **i32)
        dt.vorig[:n] = torch.arange(n, **i32)
    dt.vmeta[0] = n
    ld = (V + 7) // 8 * 8
    buf = torch.zeros(n + 1, ld, dtype=torch.bfloat16, device=dev)
    buf[:, :V] = lg[: n + 1]
    depth = max(tree.depths, default=0)
    result = torch.zeros(depth + 3, dtype=torch.int32, device=dev)
    keep_src = torch.zeros(depth + 2, dtype=torch.int32, device=dev)
    n_keep = torch.zeros(1, dtype=torch.int32, device=dev)
    root = torch.zeros(1, dtype=torch.int32, device=dev)
    sampler.accept(dt, buf[:, :V], n + 1, 0, result, keep_src, n_keep, root)
    r = result.tolist()
    n_new = r[0]
    accepted = [s - 1 for s in keep_src[1:n_new].tolist()]
    return accepted, r[n_new]
