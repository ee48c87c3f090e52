"""HBM-resident FragPack KV store over a paged KV cache (MI355X).

Reference: fragpack/ops/hbm_kv.py (module contract :1-47, page_bytes :87-99,
StoreStats / StoreError :102-123, register_store / active_store :126-159,
HbmKvStore :177-613) and fragpack/ops/hbm_kv.cu.

The engine's paged KV cache is the arena: row ``b`` of layer ``l`` is one
page shared by the block's ``2 H`` records, packed back to back in encode
order.  Records are located through ``rec_addr[L, NB, 2, H]`` (absolute
device addresses) and ``rec_len`` (bytes past the dense part; raw records use
``RAW_VAR_LEN``): a record lives in its block's page, in staging while its
block is open, or raw in the overflow pool when it does not code or its page
is full.

Per step: :meth:`HbmKvStore.prepare` (GC, staging claims, close list), then
per layer :meth:`write` / attention / :meth:`encode`, then :meth:`commit`
after the last layer.  Launch shapes depend only on host values fixed per
batch shape, so the per-layer calls are HIP-graph safe.  Block blobs move
closed blocks to and from an external tier (:meth:`export_blocks`,
:meth:`import_blocks`).
"""

from __future__ import annotations

from dataclasses import dataclass
import hashlib

import numpy as np
import torch

from fragpack_amd.compression import attn_page as ap
from fragpack_amd.compression.attn_tables import DeviceTables
from fragpack_amd.logging import init_logger
from fragpack_amd.ops.fragpack_ext import extension

logger = init_logger(__name__)

BLOCK_TOKENS = 128
HEAD_DIM = 128
# Page budget per record past the dense part (calibrated KV averages ~550 B
# of variable part; at 1280 a block-layer page spills essentially none).
VAR_SHARE = 1280
RAW_RECORD = 32768
RAW_VAR_LEN = RAW_RECORD - ap.DENSE_BYTES

# Counter slots (fp_store.hip, the reference's numbering).
_ERR_STAGING = 4
_ERR_OVERFLOW = 5
_FALLBACKS = 6
_ENCODED = 7
_SPILLS = 8
_N_COUNTERS = 16
_N_TAGS = 4
_BLOB_FAILURES = {1: "bad header", 2: "bad lengths", 4: "overflow full"}

_ACTIVE: HbmKvStore | None = None


def page_bytes(kv_heads: int) -> int:
    """Arena page bytes per block-layer: ``2 H * (DENSE_BYTES + VAR_SHARE)``."""
    return 2 * kv_heads * (ap.DENSE_BYTES + VAR_SHARE)


@dataclass(frozen=True)
class StoreStats:
    """Cumulative store counters.

    Attributes:
        encoded: Records encoded (all layers).
        fallbacks: Records stored raw in the overflow pool (includes spills).
        spills: Coded records stored raw because their page was full.
        err_staging: Claims dropped because staging was exhausted.
        err_overflow: Raw records dropped because the overflow pool was full.
    """

    encoded: int
    fallbacks: int
    spills: int
    err_staging: int
    err_overflow: int


class StoreError(RuntimeError):
    """Raised when the store dropped KV data (staging or overflow exhausted)."""


def register_store(store: HbmKvStore) -> None:
    """Publish the process's store to a KV connector."""
    global _ACTIVE
    _ACTIVE = store


def active_store() -> HbmKvStore:
    """The store published by :func:`register_store`.

    Raises:
        RuntimeError: If none was registered.
    """
    if _ACTIVE is None:
        raise RuntimeError("no FragPack KV store: the FragPack attention backend is not active")
    return _ACTIVE


def blob_failures(status: int) -> str:
    """Comma-separated names of an import status word's failure bits."""
    return ", ".join(name for bit, name in _BLOB_FAILURES.items() if status & bit)


class HbmKvStore:
    """FragPack KV store whose arena is the engine's paged KV cache.

    Args:
        kv_caches: One uint8-viewable tensor per layer; block ``b`` of layer
            ``l`` is row ``b`` (``stride(0) * element_size`` bytes, a 16-byte
            multiple, normally :func:`page_bytes`).
        kv_heads: KV heads ``H``.
        tables: Calibrated tables for every layer.
        max_tokens: Most tokens in one step (sizes the lists and scratch).
        staging_slots: Persistent staging slots (one per running request).
        overflow_records: Raw records the overflow pool holds
            (``FRAGPACK_OVERFLOW`` in the serving backend).
    """

    def __init__(
        self,
        kv_caches: list[torch.Tensor],
        kv_heads: int,
        tables: DeviceTables,
        max_tokens: int,
        staging_slots: int,
        overflow_records: int,
    ) -> None:
        dev = kv_caches[0].device
        self.num_layers = len(kv_caches)
        self.kv_heads = kv_heads
        self.num_blocks = kv_caches[0].shape[0]
        self.tables = tables
        if tables.rank_of.shape[:3] != (self.num_layers, 2, kv_heads):
            raise ValueError(
                f"tables {tuple(tables.rank_of.shape)} do not match L={self.num_layers}, H={kv_heads}"
            )
        self.arena_base: list[int] = []
        self.arena_stride: list[int] = []
        # Identifies the codec tables so blobs coded with others are rejected.
        self.table_digest = int.from_bytes(
            hashlib.blake2b(tables.rank_of.cpu().numpy().tobytes(), digest_size=8).digest(),
            "little",
            signed=True,
        )
        for cache in kv_caches:
            stride = cache.stride(0) * cache.element_size()
            if cache.shape[0] != self.num_blocks or stride % 16:
                raise ValueError(f"cache {tuple(cache.shape)} stride {stride} is not a 16-byte multiple")
            self.arena_base.append(cache.data_ptr())
            self.arena_stride.append(stride)

        L, NB, H = self.num_layers, self.num_blocks, kv_heads
        i32 = dict(dtype=torch.int32, device=dev)
        transient = max_tokens // BLOCK_TOKENS + 2 + staging_slots
        self.counters = torch.zeros(_N_COUNTERS, **i32)
        self.counters[0] = staging_slots
        self.wslot = torch.full((NB,), -1, **i32)
        self.tags = torch.zeros((_N_TAGS, NB), **i32)
        self.free_stack = torch.arange(staging_slots, **i32)
        words = -(-overflow_records // 32)
        bits = np.zeros(words * 32, dtype=bool)
        bits[overflow_records:] = True  # slots past the pool are never handed out
        self.ovf_bits = torch.from_numpy(np.packbits(bits, bitorder="little").view(np.int32).copy()).to(dev)
        self.claim_list = torch.zeros(2 * max_tokens, **i32)
        self.close_list = torch.zeros(2 * max_tokens, **i32)
        # Never-claimed blocks read one all-zero raw record.
        self.null_record = torch.zeros(RAW_RECORD, dtype=torch.uint8, device=dev)
        self.rec_addr = torch.full((L, NB, 2, H), self.null_record.data_ptr(), dtype=torch.int64, device=dev)
        self.rec_len = torch.full((L, NB, 2, H), RAW_VAR_LEN, **i32)
        self.staging = torch.zeros((staging_slots, L, 2, H, RAW_RECORD), dtype=torch.uint8, device=dev)
        self.scratch = torch.zeros((transient, 2, H, RAW_RECORD), dtype=torch.uint8, device=dev)
        self.overflow = torch.zeros((overflow_records, RAW_RECORD), dtype=torch.uint8, device=dev)
        self.fill = torch.zeros((L, NB), **i32)
        self.live = torch.zeros(NB, **i32)
        i64 = dict(dtype=torch.int64, device=dev)
        self.arena_base_dev = torch.tensor(self.arena_base, **i64)
        self.arena_stride_dev = torch.tensor(self.arena_stride, **i64)
        self._poll_host = torch.zeros(_N_COUNTERS, dtype=torch.int32, pin_memory=dev.type == "cuda")
        self._poll_event: torch.cuda.Event | None = None
        self._step = 0
        self._state = (
            self.counters,
            self.wslot,
            self.tags,
            self.free_stack,
            self.ovf_bits,
            self.claim_list,
            self.close_list,
            self.rec_addr,
            self.rec_len,
            self.staging,
            self.scratch,
            self.overflow,
            self.fill,
        )

    def memory_usage(self) -> dict[str, int]:
        """Persistent GPU bytes by component (arena rows at their real strides)."""
        metadata = (
            self.counters,
            self.wslot,
            self.tags,
            self.free_stack,
            self.ovf_bits,
            self.claim_list,
            self.close_list,
            self.null_record,
            self.rec_addr,
            self.rec_len,
            self.fill,
            self.live,
            self.arena_base_dev,
            self.arena_stride_dev,
        )
        return {
            "arena": self.num_blocks * sum(self.arena_stride),
            "staging": self.staging.numel() * self.staging.element_size(),
            "scratch": self.scratch.numel() * self.scratch.element_size(),
            "overflow": self.overflow.numel() * self.overflow.element_size(),
            "metadata": sum(t.numel() * t.element_size() for t in metadata),
            "codebooks": sum(
                t.numel() * t.element_size() for t in (self.tables.rank_of, self.tables.plut, self.tables.slut)
            ),
        }

    def prepare(self, slot_mapping: torch.Tensor, num_tokens: int, live_blocks: np.ndarray) -> None:
        """Start a step: GC, claim staging, list closing blocks.

        Args:
            slot_mapping: int64 ``[>= num_tokens]`` slot ids (negative = pad).
            num_tokens: Tokens to scan.
            live_blocks: int32 ids of blocks that keep their staging slot.
        """
        self._step = self._step % 0x7FFFFFFE + 1
        n_live = int(live_blocks.size)
        if n_live:
            host = torch.from_numpy(np.ascontiguousarray(live_blocks, dtype=np.int32)).pin_memory()
            self.live[:n_live].copy_(host, non_blocking=True)
        extension().hbm_prepare(*self._state, slot_mapping, num_tokens, self.live, n_live, self._step)

    def write(self, layer: int, key: torch.Tensor, value: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        """Store one layer's new K / V tokens (BF16 ``[N, H, 128]``) into staging."""
        extension().hbm_write(*self._state, key, value, slot_mapping, layer)

    def encode(self, layer: int, max_close: int, ordered: bool = False) -> None:
        """Code this layer's records of every block closed this step.

        ``ordered``: place each block's records in (kv, head) order, so that
        the arena bytes and which records spill depend only on the records
        (the reference places them as they arrive).
        """
        extension().hbm_encode(
            *self._state, self.tables.rank_of, layer, self.arena_base[layer], self.arena_stride[layer], max_close,
            ordered=ordered,
        )

    def commit(self) -> None:
        """Release the staging of blocks closed this step (after the last layer)."""
        extension().hbm_commit(*self._state)

    def gather(self, layer: int, blocks: torch.Tensor, wk: torch.Tensor, wv: torch.Tensor) -> None:
        """Decode blocks of one layer into token-major BF16 ``[P, 128, H, 128]`` pages."""
        extension().hbm_gather(
            blocks,
            self.rec_addr[layer],
            self.rec_len[layer],
            self.tables.plut[layer],
            self.tables.slut[layer],
            wk,
            wv,
            self.kv_heads,
        )

    def layer_tables(self, layer: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
        """``(rec_addr, rec_len, plut, slut)`` views of one layer."""
        return self.rec_addr[layer], self.rec_len[layer], self.tables.plut[layer], self.tables.slut[layer]

    @property
    def blob_stride(self) -> int:
        """Bytes reserved per block blob (all records raw)."""
        return ap.blob_slot_bytes(self.num_layers, self.kv_heads)

    def export_blocks(self, blocks: torch.Tensor, out: torch.Tensor, stride: int) -> torch.Tensor:
        """Copy closed blocks' records into block blobs; returns int64 ``[n]`` lengths."""
        lengths = torch.empty(blocks.numel(), dtype=torch.int64, device=out.device)
        extension().hbm_export(blocks, self.rec_addr, self.rec_len, out, stride, lengths, self.table_digest)
        return lengths

    def import_blocks(self, src: torch.Tensor, offsets: torch.Tensor, blocks: torch.Tensor) -> torch.Tensor:
        """Install block blobs into blocks; returns int32 ``[n]`` status (0 = installed)."""
        status = torch.zeros(blocks.numel(), dtype=torch.int32, device=src.device)
        extension().hbm_import(
            *self._state, src, offsets, blocks, status, self.arena_base_dev, self.arena_stride_dev, self.table_digest
        )
        return status

    def poll(self) -> StoreStats | None:
        """Non-blocking counter snapshot (the previous call's); raises on data loss."""
        stats = None
        if self._poll_event is not None:
            if not self._poll_event.query():
                return None
            stats = self._stats_from(self._poll_host.numpy())
        self._poll_host.copy_(self.counters, non_blocking=True)
        self._poll_event = torch.cuda.Event()
        self._poll_event.record()
        return stats

    def stats(self) -> StoreStats:
        """Synchronous counter read; raises :class:`StoreError` on data loss."""
        return self._stats_from(self.counters.cpu().numpy())

    def _stats_from(self, c: np.ndarray) -> StoreStats:
        stats = StoreStats(
            encoded=int(c[_ENCODED]),
            fallbacks=int(c[_FALLBACKS]),
            spills=int(c[_SPILLS]),
            err_staging=int(c[_ERR_STAGING]),
            err_overflow=int(c[_ERR_OVERFLOW]),
        )
        if stats.err_staging or stats.err_overflow:
            raise StoreError(
                f"FragPack store dropped KV: staging={stats.err_staging} overflow={stats.err_overflow} "
                "(staging must cover one open block per running request; overflow is sized by FRAGPACK_OVERFLOW)"
            )
        return stats


__all__ = [
    "BLOCK_TOKENS",
    "HEAD_DIM",
    "RAW_RECORD",
    "RAW_VAR_LEN",
    "VAR_SHARE",
    "HbmKvStore",
    "StoreError",
    "StoreStats",
    "active_store",
    "blob_failures",
    "page_bytes",
    "register_store",
]
