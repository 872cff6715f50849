"""Shared KV cache for target and draft (reference ssd/engine/kv_cache.py).

One arena per cache in HBM, keyed by *base* layer index like the reference's slots:
``k`` and ``vt`` are each [layers, kv_heads, max_len * head_dim] bf16, max_len a multiple of 64,
in the 64-slot block layout of csrc/common.h (k_off / v_off): every 64-slot block of K is stored
as the tree-attention kernel's S = K Q^T operand tiles and every block of V as its O = V^T P^T
operand tiles, each tile in lane order, so the kernel reads a block as contiguous 1 KiB loads.
``read`` / ``ops.kv_untile`` give the plain [kv_heads, slots, head_dim] view.

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
        # Slot capacity in whole 64-slot blocks (the block layout's unit).
        self.capacity = (max_length + 63) // 64 * 64
        self.seq_len = 0
        self.kv_heads, self.head_dim, self.device = kv_heads, head_dim, device
        self.k: Optional[torch.Tensor] = None
        self.vt: Optional[torch.Tensor] = None
        if kv_heads is not None and head_dim is not None and device is not None:
            self._alloc()

    def _alloc(self) -> None:
        shape = (self.num_slots, self.kv_heads, self.capacity * self.head_dim)
        self.k = torch.zeros(shape, dtype=torch.bfloat16, device=self.device)
        self.vt = torch.zeros(shape, dtype=torch.bfloat16, device=self.device)

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
        plain copies [1, kv_heads, seq_len+q, hd] of K and V (API form of the reference's update;
        decoding writes in-kernel)."""
        q = k.shape[2]
        end = self.seq_len + q
        self.check_room(end)
        self.ensure(k.shape[1], k.shape[3], k.device)
        k_idx, v_idx = ops.kv_block_index(self.capacity, self.head_dim, self.k.device)
        self.k[slot][:, k_idx[self.seq_len:end]] = k[0].to(torch.bfloat16)
        self.vt[slot][:, v_idx[self.seq_len:end]] = v[0].to(torch.bfloat16)
        kk, vv = self.read(slot, end)
        return kk[None], vv[None]

    def read(self, slot: int, end: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Plain copies K, V [kv_heads, end, head_dim] of slots [0, end) of base layer ``slot``."""
        k_idx, v_idx = ops.kv_block_index(self.capacity, self.head_dim, self.k.device)
        return self.k[slot][:, k_idx[:end]], self.vt[slot][:, v_idx[:end]]

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

    def compact_device(self, start: int, src: torch.Tensor, n_dev: torch.Tensor, n_max: int,
                       pos_base: Optional[torch.Tensor] = None) -> None:
        """Compaction with sources and count already on the device (the engine's path: no host sync);
        with ``pos_base`` the destination start is relative to that device word."""
        ops.kv_compact(self.k, self.vt, self.num_slots, self.kv_heads, self.head_dim, self.capacity, start, src,
                       n_dev, n_max, pos_base)

    def reset(self) -> None:
        self.seq_len = 0
