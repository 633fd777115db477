"""Paged KV-cache physical memory pool in MI355X HBM.

Same layout and API as the reference (memforge_ml/runtime/kv_pool.py:27-211):
``key_pool`` / ``value_pool`` are ``(num_layers, num_blocks, block_size,
num_kv_heads, head_dim)`` tensors, public because callers index them
directly. Token position ``i`` of a sequence lives in physical block
``block_table[i // block_size]`` at slot ``i % block_size``. Reads and writes
run through the HIP copy kernels; the pool must live on the GPU.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Tuple

import torch

from memforge_amd import _native as nat
from memforge_amd.kernels import paged_gather


def _require_gpu_device(device) -> None:
    if torch.device(device).type != "cuda":
        raise ValueError(
            f"memforge_amd keeps the KV pool in GPU memory; got device {device!r} "
            "(there is no CPU path)"
        )


@dataclass(frozen=True)
class ModelKVSpec:
    """Per-token KV geometry derived from a Hugging Face model config
    (kv_pool.py:27-55)."""

    num_layers: int
    num_kv_heads: int
    head_dim: int
    dtype: torch.dtype
    device: str

    @classmethod
    def from_config(cls, config, dtype: torch.dtype, device: str) -> "ModelKVSpec":
        head_dim = getattr(config, "head_dim", None) or (config.hidden_size // config.num_attention_heads)
        num_kv_heads = getattr(config, "num_key_value_heads", None) or config.num_attention_heads
        return cls(num_layers=config.num_hidden_layers, num_kv_heads=num_kv_heads,
                   head_dim=head_dim, dtype=dtype, device=device)

    @property
    def bytes_per_token(self) -> int:
        """KV bytes of one token across all layers (K and V)."""
        elem = torch.empty(0, dtype=self.dtype).element_size()
        return 2 * self.num_layers * self.num_kv_heads * self.head_dim * elem


class PagedKVPool:
    """Fixed-size physical block pool backing the paged KV cache."""

    def __init__(self, spec: ModelKVSpec, num_blocks: int, block_size: int = 16):
        _require_gpu_device(spec.device)
        self.spec = spec
        self.num_blocks = num_blocks
        self.block_size = block_size
        shape = (spec.num_layers, num_blocks, block_size, spec.num_kv_heads, spec.head_dim)
        self.key_pool = torch.zeros(shape, dtype=spec.dtype, device=spec.device)
        self.value_pool = torch.zeros(shape, dtype=spec.dtype, device=spec.device)

    # ---------------------------------------------------------------- sizing

    @property
    def bytes_per_block(self) -> int:
        return self.spec.bytes_per_token * self.block_size

    @property
    def total_bytes(self) -> int:
        return self.bytes_per_block * self.num_blocks

    @property
    def capacity_tokens(self) -> int:
        return self.num_blocks * self.block_size

    @staticmethod
    def blocks_for_budget(spec: ModelKVSpec, block_size: int, budget_mb: float) -> int:
        """Largest number of physical blocks inside a memory budget (kv_pool.py:84-88)."""
        per_block = spec.bytes_per_token * block_size
        return max(1, int((budget_mb * 1024 * 1024) // per_block))

    # -------------------------------------------------------------- indexing

    def slot_indices(self, block_table: torch.Tensor, start: int, end: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """(physical block, slot) tensors for token range [start, end)
        (memforge_ml/runtime/kv_pool.py:92-110). The bound check is integer arithmetic on the host,
        so it costs no device synchronisation."""
        if end > start and (end - 1) // self.block_size >= block_table.numel():
            raise IndexError(
                f"logical block {(end - 1) // self.block_size} is outside a block table of "
                f"{block_table.numel()} entries (token range {start}:{end})"
            )
        positions = torch.arange(start, end, device=block_table.device)
        logical = torch.div(positions, self.block_size, rounding_mode="floor")
        slots = positions % self.block_size
        return block_table.reshape(-1)[logical], slots

    @staticmethod
    def block_table_tensor(block_table: List[int], device: str) -> torch.Tensor:
        return torch.tensor(block_table, dtype=torch.long, device=device)

    def flat_indices(self, block_table: torch.Tensor, start: int, end: int) -> torch.Tensor:
        """One flat offset per token into the pool viewed as (blocks*slots, ...)."""
        physical, slots = self.slot_indices(block_table, start, end)
        return paged_gather.flat_slot_index(physical, slots, self.block_size)

    # ----------------------------------------------------------------- I / O

    def layer_view(self, layer_idx: int) -> nat.PoolView:
        return nat.PoolView.from_bshd(self.key_pool[layer_idx], self.value_pool[layer_idx])

    def write(self, layer_idx: int, physical: torch.Tensor, slots: torch.Tensor,
              keys: torch.Tensor, values: torch.Tensor) -> None:
        """Scatter ``(1, num_kv_heads, T, head_dim)`` K/V to (physical, slot) (kv_pool.py:134-149)."""
        flat = paged_gather.flat_slot_index(physical, slots, self.block_size)
        nat.kv_write(keys[0].permute(1, 0, 2), values[0].permute(1, 0, 2), flat, self.layer_view(layer_idx))

    def gather(self, layer_idx: int, physical: torch.Tensor, slots: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """Contiguous ``(1, num_kv_heads, T, head_dim)`` K/V of (physical, slot) (kv_pool.py:151-169)."""
        flat = paged_gather.flat_slot_index(physical, slots, self.block_size)
        return self.gather_flat(layer_idx, flat)

    def gather_flat(self, layer_idx: int, flat_index: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        return paged_gather.gather_kv(self.key_pool, self.value_pool, layer_idx, flat_index, self.block_size)

    def write_flat(self, layer_idx: int, flat_index: torch.Tensor, keys: torch.Tensor,
                   values: torch.Tensor) -> None:
        paged_gather.scatter_kv(self.key_pool, self.value_pool, layer_idx, flat_index, keys, values,
                                self.block_size)

    def zero_(self) -> None:
        self.key_pool.zero_()
        self.value_pool.zero_()

    def describe(self) -> dict:
        return {
            "num_blocks": self.num_blocks,
            "block_size": self.block_size,
            "capacity_tokens": self.capacity_tokens,
            "bytes_per_token": self.spec.bytes_per_token,
            "bytes_per_block": self.bytes_per_block,
            "total_mb": round(self.total_bytes / (1024 * 1024), 2),
            "num_layers": self.spec.num_layers,
            "num_kv_heads": self.spec.num_kv_heads,
            "head_dim": self.spec.head_dim,
            "dtype": str(self.spec.dtype),
            "device": self.spec.device,
            # how the kernels address it: one layer of one pool tensor is
            # blocks x block_size x kv_heads x head_dim, head_dim contiguous
            "layout": "(layers, blocks, block_size, kv_heads, head_dim)",
            "element_bytes": self.key_pool.element_size(),
            "block_table_dtype": "int32",
            "slot_mapping_dtype": "int64",
        }
