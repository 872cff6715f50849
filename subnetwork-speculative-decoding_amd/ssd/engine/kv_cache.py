"""Shared KV cache for target and draft (reference ssd/engine/kv_cache.py).

One arena per cache in HBM, keyed by *base* layer index like the reference's slots:

* ``k``  [layers, kv_heads, max_len, head_dim]  bf16 -- rows are keys (QK^T operand);
* ``vt`` [layers, kv_heads, head_dim, max_len]  bf16 -- V transposed, so the P.V operand of
  the tree-attention MFMA is a contiguous 16-byte run of 8 keys.

Writes happen inside the fused q/k/v + RoPE GEMM epilogue; ``keep_positions`` (the
accepted-path compaction) is one kernel launch over every layer. ``seq_len`` bookkeeping,
``advance``/``crop``/``reset`` and the overflow ``RuntimeError`` follow the reference
(kv_cache.py:21-73). Batch size is 1, as in the reference's speculative decoding.
"""

from __future__ import annotations

from typing import Optional

import torch

from ssd import ops


class KVCache:
    def __init__(self, num_slots: int, max_length: int, kv_heads: Optional[int] = None,
                 head_dim: Optional[int] = None, device=None):
        self.num_slots = num_slots
        self.max_length = max_length
        # Slot capacity rounded up so every V^T row is 16-byte aligned for the vector loads.
        self.capacity = (max_length + 7) // 8 * 8
        self.seq_len = 0
        self.kv_heads, self.head_dim, self.device = kv_heads, head_dim, device
        self.k: Optional[torch.Tensor] = None
        self.vt: Optional[torch.Tensor] = None
        if kv_heads is not None and head_dim is not None and device is not None:
            self._alloc()

    def _alloc(self) -> None:
        shape_k = (self.num_slots, self.kv_heads, self.capacity, self.head_dim)
        shape_v = (self.num_slots, self.kv_heads, self.head_dim, self.capacity)
        self.k = torch.zeros(shape_k, dtype=torch.bfloat16, device=self.device)
        self.vt = torch.zeros(shape_v, dtype=torch.bfloat16, device=self.device)

    def ensure(self, kv_heads: int, head_dim: int, device) -> None:
        if self.k is None:
            self.kv_heads, self.head_dim, self.device = kv_heads, head_dim, torch.device(device)
            self._alloc()

    def get_seq_length(self) -> int:
        return self.seq_len

    def check_room(self, end: int) -> None:
        if end > self.max_length:
            raise RuntimeError(f"KVCache overflow: {end} > max_length={self.max_length}")

    def layer(self, i: int) -> tuple[torch.Tensor, torch.Tensor]:
        return self.k[i], self.vt[i]

    def update(self, slot: int, k: torch.Tensor, v: torch.Tensor):
        """Write k/v [1, kv_heads, q, hd] at [seq_len, seq_len+q) of base layer ``slot`` and return
        views of [0, seq_len+q) (API form of the reference's update; decoding writes in-kernel)."""
        q = k.shape[2]
        end = self.seq_len + q
        self.check_room(end)
        self.ensure(k.shape[1], k.shape[3], k.device)
        self.k[slot, :, self.seq_len:end] = k[0].to(torch.bfloat16)
        self.vt[slot, :, :, self.seq_len:end] = v[0].to(torch.bfloat16).transpose(1, 2)
        return self.k[slot, None, :, :end], self.vt[slot, None, :, :, :end].transpose(-1, -2)

    def advance(self, n: int) -> None:
        self.seq_len += n

    def crop(self, length: int) -> None:
        if length > self.seq_len:
            raise ValueError(f"cannot crop to {length} > current length {self.seq_len}")
        self.seq_len = length

    def keep_positions(self, start: int, positions) -> None:
        """Move entries ``positions`` (absolute, >= start) to [start, start+n) in every layer
        with one kernel launch; sources are all read before any destination is written."""
        pos = positions.tolist() if isinstance(positions, torch.Tensor) else list(positions)
        n = len(pos)
        if n == 0 or pos == list(range(start, start + n)) or self.k is None:
            self.seq_len = start + n
            return
        if min(pos) < start or max(pos) >= self.capacity:
            raise ValueError("keep_positions: positions out of range")
        src = torch.tensor(pos, dtype=torch.int32).to(self.device)
        n_dev = torch.tensor([n], dtype=torch.int32).to(self.device)
        ops.kv_compact(self.k, self.vt, self.num_slots, self.kv_heads, self.head_dim, self.capacity, start, src,
                       n_dev, n)
        self.seq_len = start + n

    def compact_device(self, start: int, src: torch.Tensor, n_dev: torch.Tensor, n_max: int) -> None:
        """Compaction with sources and count already on the device (the engine's path: no host sync)."""
        ops.kv_compact(self.k, self.vt, self.num_slots, self.kv_heads, self.head_dim, self.capacity, start, src,
                       n_dev, n_max)

    def reset(self) -> None:
        self.seq_len = 0
