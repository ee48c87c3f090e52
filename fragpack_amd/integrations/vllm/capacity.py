"""Host-only snapshot of the store's allocation, for the engine's statistics.

Reference: fragpack/integrations/vllm/capacity.py.  The backend publishes one
:class:`FragPackCapacity` per store binding; consumers read it without any
device access.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass
from typing import Any


@dataclass(frozen=True)
class FragPackCapacity:
    """Allocated capacity of one worker's FragPack store.

    Attributes:
        blocks: Blocks of the engine's cache (including its null block).
        block_tokens: Token slots per block.
        layers: Attention layers on this worker.
        kv_heads: KV heads per layer on this worker.
        page_bytes: Bytes per block and layer.
        raw_page_bytes: BF16 bytes of the same block-layer.
        memory: Persistent device bytes by component (arena, staging,
            scratch, overflow, metadata, codebooks, workspaces).
    """

    blocks: int
    block_tokens: int
    layers: int
    kv_heads: int
    page_bytes: int
    raw_page_bytes: int
    memory: dict[str, int]

    def to_dict(self) -> dict[str, Any]:
        """An independent, serialisable copy (the memory dict is copied)."""
        return asdict(self)


_CAPACITY: FragPackCapacity | None = None


def publish_capacity(capacity: FragPackCapacity) -> None:
    """Replace the process's published snapshot (after a store binding)."""
    global _CAPACITY
    _CAPACITY = capacity


def get_capacity() -> FragPackCapacity | None:
    """The published snapshot, or None before any store exists (None is not
    zero capacity)."""
    return _CAPACITY


__all__ = ["FragPackCapacity", "get_capacity", "publish_capacity"]
