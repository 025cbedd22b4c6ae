"""HybridMemoryPool -- the reference's slab pool API (serving/hybrid_memory_pool.h:40-85) over the native
slot bookkeeping of libkdn.so (kdn_pool_*) and one device slab of fp32 recurrent states.

Each stream owns one slot of [num_layers][num_heads][lifted_dim][val_dim] fp32 state (the layout the
decode and scan kernels read with unit stride); the pool allocates nothing after construction
(allocate / fork / release only move slots between the free stack and the active set; fork copies the
parent's slot on the device).  The softmax anchor pages the reference class also manages belong to the
attention layers, not to this path, and are not modelled.
"""
from __future__ import annotations

import torch

from kdn import ops


class HybridMemoryPool:
    def __init__(self, max_streams: int, max_seq_len: int, num_layers: int = 20, num_heads: int = 16,
                 val_dim: int = 64, lifted_dim: int = 512, device="cuda:0"):
        self.max_streams = max_streams
        self.max_seq_len = max_seq_len
        self.num_layers = num_layers
        self._pool = ops.StatePool(max_streams, num_layers, num_heads, lifted_dim, val_dim, device=device)
        self.recurrent_bytes_per_stream = self._pool.slot_bytes
        self.prompt_len = {}

    @property
    def slab(self) -> torch.Tensor:
        """[max_streams, num_layers, num_heads, lifted_dim, val_dim] fp32."""
        return self._pool.slab

    def layer_states(self, layer: int) -> torch.Tensor:
        """[max_streams, num_heads, lifted_dim, val_dim] view: the states argument of a layer's step."""
        return self._pool.layer_states(layer)

    def allocate_stream(self, prompt_len: int) -> int:
        slot = self._pool.allocate()
        if slot >= 0:
            self.prompt_len[slot] = prompt_len
        return slot

    def fork_stream(self, parent_stream_id: int) -> int:
        try:
            child = self._pool.fork(parent_stream_id)
        except RuntimeError:
            return -1
        if child >= 0:
            self.prompt_len[child] = self.prompt_len.get(parent_stream_id, 0)
        return child

    def release_stream(self, stream_id: int) -> None:
        try:
            self._pool.release(stream_id)
        except RuntimeError:
            return
        self.prompt_len.pop(stream_id, None)

    def get_total_allocated_bytes(self) -> int:
        return self._pool.allocated_bytes()

    def get_free_bytes(self) -> int:
        return self._pool.free_bytes()

    def print_memory_profile(self) -> None:
        active = self._pool.active
        total = self.max_streams * self.recurrent_bytes_per_stream
        used = self.get_total_allocated_bytes()
        print("[HybridMemoryPool]")
        print(f"  Active streams: {active} / {self.max_streams}")
        print(f"  Recurrent slab: {used / 2**20:.1f} MB / {total / 2**20:.1f} MB ({100.0 * used / max(total, 1):.1f}%)")
