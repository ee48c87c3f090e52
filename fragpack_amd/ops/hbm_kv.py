"""HBM-resident FragPack KV store over an engine's paged KV cache (MI355X).

Reference interface: fragpack/ops/hbm_kv.py (page_bytes :87-99, StoreStats /
StoreError :102-123, register_store / active_store :126-159, HbmKvStore
:177-613) over the kernels of fragpack/ops/hbm_kv.cu.  Names, arguments,
the 13-tensor state order and the counter slots are that interface; the
class below is this package's own.

Model.  The engine's cache is the arena: row ``b`` of layer ``l`` is the
page of block ``b``, holding its ``2 H`` records packed back to back.  A
record is found through ``rec_addr[L, NB, 2, H]`` (absolute device address)
and ``rec_len`` (bytes past the 22528-byte dense part; ``RAW_VAR_LEN`` for a
raw record).  While a block is open its records are raw BF16 in a staging
slot -- persistent ``[S_p, L, 2, H, 32 KB]`` for blocks open across steps,
transient ``[S_t, 2, H, 32 KB]`` for blocks that open and close within one
step -- and a closed record that does not code, or no longer fits its page,
is raw in the overflow pool (``FRAGPACK_OVERFLOW`` records, a bitmap).

Step protocol: :meth:`HbmKvStore.prepare` once per step (GC, staging claims,
close list), then per layer :meth:`write`, attention, :meth:`encode`, and
:meth:`commit` after the last layer.  Launch shapes depend only on host
integers fixed by the batch shape, so the per-layer calls can be captured
in a HIP graph.  Closed blocks move to and from other tiers as block blobs
(:meth:`export_blocks` / :meth:`import_blocks`).
"""

from __future__ import annotations

from dataclasses import dataclass, fields
import enum
import hashlib
from typing import NamedTuple

import numpy as np
import torch

from fragpack_amd.compression import attn_page as ap
from fragpack_amd.compression.attn_tables import DeviceTables
from fragpack_amd.logging import init_logger
from fragpack_amd.ops.fragpack_ext import extension

logger = init_logger(__name__)

BLOCK_TOKENS = 128
HEAD_DIM = 128
# Arena budget per record past the dense part: calibrated KV needs ~550 B on
# average (VAR_CAP 2048), and at 1280 B per record a page spills almost never.
VAR_SHARE = 1280
RAW_RECORD = 32768
RAW_VAR_LEN = RAW_RECORD - ap.DENSE_BYTES


class _Counter(enum.IntEnum):
    """Slots of the int32 counter array (the kernels' numbering, hbm_kv.cu:14-26)."""

    FREE_TOP = 0
    TRANSIENT = 1
    CLAIMS = 2
    CLOSES = 3
    ERR_STAGING = 4
    ERR_OVERFLOW = 5
    FALLBACKS = 6
    ENCODED = 7
    SPILLS = 8
    HEIRS = 9
    DONORS = 10


_N_COUNTERS = 16
_N_TAGS = 4
# kept for callers that index the counter array directly
_ERR_STAGING, _ERR_OVERFLOW = int(_Counter.ERR_STAGING), int(_Counter.ERR_OVERFLOW)
_FALLBACKS, _ENCODED, _SPILLS = int(_Counter.FALLBACKS), int(_Counter.ENCODED), int(_Counter.SPILLS)
_IMPORT_FAILURES = ((1, "bad header"), (2, "bad lengths"), (4, "overflow full"))


def page_bytes(kv_heads: int) -> int:
    """Arena bytes of one block-layer page: ``2 H (DENSE_BYTES + VAR_SHARE)``."""
    return 2 * kv_heads * (ap.DENSE_BYTES + VAR_SHARE)


@dataclass(frozen=True)
class StoreStats:
    """Cumulative store counters.

    Attributes:
        encoded: Records encoded, all layers.
        fallbacks: Records stored raw in the overflow pool (spills included).
        spills: Coded records stored raw because their page was full.
        err_staging: Claims that found no staging slot (their KV is lost).
        err_overflow: Raw records the full overflow pool could not take.
    """

    encoded: int
    fallbacks: int
    spills: int
    err_staging: int
    err_overflow: int

    @classmethod
    def from_counters(cls, c: np.ndarray) -> StoreStats:
        return cls(encoded=int(c[_Counter.ENCODED]), fallbacks=int(c[_Counter.FALLBACKS]),
                   spills=int(c[_Counter.SPILLS]), err_staging=int(c[_Counter.ERR_STAGING]),
                   err_overflow=int(c[_Counter.ERR_OVERFLOW]))

    @property
    def lost(self) -> bool:
        return bool(self.err_staging or self.err_overflow)


class StoreError(RuntimeError):
    """KV data was dropped: staging or the overflow pool ran out."""


class _Registry:
    """The process's active store, handed from the attention backend to a
    KV connector without either importing the other."""

    store: HbmKvStore | None = None


def register_store(store: HbmKvStore) -> None:
    """Make ``store`` the process's active store (replacing any earlier one)."""
    _Registry.store = store


def active_store() -> HbmKvStore:
    """The active store.

    Raises:
        RuntimeError: If no store was registered (the backend is not in use).
    """
    if _Registry.store is None:
        raise RuntimeError("no FragPack KV store is registered: the FragPack attention backend is not active")
    return _Registry.store


def blob_failures(status: int) -> str:
    """Names of the failure bits in an import status word, comma separated."""
    return ", ".join(name for bit, name in _IMPORT_FAILURES if status & bit)


class _State(NamedTuple):
    """The 13 state tensors, in the order every store kernel takes them
    (hbm_kv.py:287-301)."""

    counters: torch.Tensor    # int32 [16]
    wslot: torch.Tensor       # int32 [NB] staging slot of each block, -1 none
    tags: torch.Tensor        # int32 [4, NB] per-block step stamps
    free_stack: torch.Tensor  # int32 [S_p] free persistent slots (first counters[0])
    ovf_bits: torch.Tensor    # int32 bitmap of overflow slots in use
    claim_list: torch.Tensor  # int32 [2, cap] claims | heirs
    close_list: torch.Tensor  # int32 [2, cap] closes | their heirs
    rec_addr: torch.Tensor    # int64 [L, NB, 2, H]
    rec_len: torch.Tensor     # int32 [L, NB, 2, H]
    staging: torch.Tensor     # uint8 [S_p, L, 2, H, 32 KB]
    scratch: torch.Tensor     # uint8 [S_t, 2, H, 32 KB]
    overflow: torch.Tensor    # uint8 [O, 32 KB]
    fill: torch.Tensor        # int32 [L, NB] page bytes in use


@dataclass(frozen=True)
class _Geometry:
    layers: int
    blocks: int
    heads: int
    max_tokens: int
    staging_slots: int
    overflow_records: int

    @property
    def scratch_slots(self) -> int:
        # blocks that can open and close within one step, plus heirs
        return self.max_tokens // BLOCK_TOKENS + 2 + self.staging_slots

    def allocate(self, dev: torch.device, null_addr: int) -> _State:
        L, NB, H = self.layers, self.blocks, self.heads
        i32 = dict(dtype=torch.int32, device=dev)
        u8 = dict(dtype=torch.uint8, device=dev)
        counters = torch.zeros(_N_COUNTERS, **i32)
        counters[_Counter.FREE_TOP] = self.staging_slots
        # overflow bitmap: bits past the pool start set, so they are never handed out
        words = -(-self.overflow_records // 32)
        in_use = np.arange(words * 32) >= self.overflow_records
        ovf = np.packbits(in_use, bitorder="little").view(np.int32)
        return _State(
            counters=counters,
            wslot=torch.full((NB,), -1, **i32),
            tags=torch.zeros((_N_TAGS, NB), **i32),
            free_stack=torch.arange(self.staging_slots, **i32),
            ovf_bits=torch.from_numpy(ovf.copy()).to(dev),
            claim_list=torch.zeros(2 * self.max_tokens, **i32),
            close_list=torch.zeros(2 * self.max_tokens, **i32),
            # a block never written reads one all-zero raw record
            rec_addr=torch.full((L, NB, 2, H), null_addr, dtype=torch.int64, device=dev),
            rec_len=torch.full((L, NB, 2, H), RAW_VAR_LEN, **i32),
            staging=torch.zeros((self.staging_slots, L, 2, H, RAW_RECORD), **u8),
            scratch=torch.zeros((self.scratch_slots, 2, H, RAW_RECORD), **u8),
            overflow=torch.zeros((self.overflow_records, RAW_RECORD), **u8),
            fill=torch.zeros((L, NB), **i32),
        )


def _digest(rank_of: torch.Tensor) -> int:
    """Identifies the codec tables in blob headers (blake2b-8 of ``rank_of``)."""
    h = hashlib.blake2b(rank_of.cpu().numpy().tobytes(), digest_size=8).digest()
    return int.from_bytes(h, "little", signed=True)


class HbmKvStore:
    """FragPack KV store whose arena is the engine's paged KV cache.

    Args:
        kv_caches: One tensor per layer, viewed as bytes: block ``b`` of layer
            ``l`` is row ``b`` (``stride(0) * element_size`` bytes, a multiple
            of 16, normally :func:`page_bytes`).
        kv_heads: KV heads ``H``.
        tables: Calibrated tables of every layer.
        max_tokens: Most tokens in one step (sizes the lists and scratch).
        staging_slots: Persistent staging slots (one per running request).
        overflow_records: Raw records the overflow pool holds.

    Raises:
        ValueError: If the caches disagree with each other or the tables.
    """

    def __init__(self, kv_caches: list[torch.Tensor], kv_heads: int, tables: DeviceTables, max_tokens: int,
                 staging_slots: int, overflow_records: int) -> None:
        first = kv_caches[0]
        geo = _Geometry(len(kv_caches), first.shape[0], kv_heads, max_tokens, staging_slots, overflow_records)
        want = (geo.layers, 2, kv_heads)
        if tuple(tables.rank_of.shape[:3]) != want:
            raise ValueError(f"tables {tuple(tables.rank_of.shape)} do not match L={geo.layers}, H={kv_heads}")
        self.arena_base: list[int] = []
        self.arena_stride: list[int] = []
        for layer, cache in enumerate(kv_caches):
            stride = cache.stride(0) * cache.element_size()
            if cache.shape[0] != geo.blocks or stride % 16:
                raise ValueError(f"layer {layer} cache {tuple(cache.shape)} (row stride {stride} B) must have "
                                 f"{geo.blocks} rows of a 16-byte multiple")
            self.arena_base.append(cache.data_ptr())
            self.arena_stride.append(stride)
        dev = first.device
        self._geo = geo
        self.num_layers, self.num_blocks, self.kv_heads = geo.layers, geo.blocks, kv_heads
        self.tables = tables
        self.table_digest = _digest(tables.rank_of)
        self.null_record = torch.zeros(RAW_RECORD, dtype=torch.uint8, device=dev)
        self._state = geo.allocate(dev, self.null_record.data_ptr())
        for name, t in self._state._asdict().items():
            setattr(self, name, t)
        self.live = torch.zeros(geo.blocks, dtype=torch.int32, device=dev)
        i64 = dict(dtype=torch.int64, device=dev)
        self.arena_base_dev = torch.tensor(self.arena_base, **i64)
        self.arena_stride_dev = torch.tensor(self.arena_stride, **i64)
        self._poll_host = torch.zeros(_N_COUNTERS, dtype=torch.int32, pin_memory=dev.type == "cuda")
        self._poll_event: torch.cuda.Event | None = None
        self._step = 0

    # ------------------------------------------------------------- accounting
    def memory_usage(self) -> dict[str, int]:
        """Persistent device bytes per component (arena rows at their strides)."""
        nbytes = lambda t: t.numel() * t.element_size()  # noqa: E731
        s = self._state
        bulk = {"staging": s.staging, "scratch": s.scratch, "overflow": s.overflow}
        meta = [t for name, t in s._asdict().items() if name not in bulk]
        meta += [self.null_record, self.live, self.arena_base_dev, self.arena_stride_dev]
        return {
            "arena": self.num_blocks * sum(self.arena_stride),
            **{name: nbytes(t) for name, t in bulk.items()},
            "metadata": sum(nbytes(t) for t in meta),
            "codebooks": sum(nbytes(getattr(self.tables, f.name)) for f in fields(self.tables)),
        }

    # ----------------------------------------------------------- step protocol
    def prepare(self, slot_mapping: torch.Tensor, num_tokens: int, live_blocks: np.ndarray) -> None:
        """Start a step: release unreferenced staging, claim staging for blocks
        receiving offset 0, list the blocks receiving offset 127.

        Args:
            slot_mapping: int64 ``[>= num_tokens]`` slots (negative: padding).
            num_tokens: Tokens of this step.
            live_blocks: int32 ids of the blocks still being written (they
                keep their staging).
        """
        self._step = self._step % 0x7FFFFFFE + 1
        n_live = int(np.size(live_blocks))
        if n_live:
            host = torch.from_numpy(np.ascontiguousarray(live_blocks, dtype=np.int32)).pin_memory()
            self.live[:n_live].copy_(host, non_blocking=True)
        extension().hbm_prepare(*self._state, slot_mapping, num_tokens, self.live, n_live, self._step)

    def write(self, layer: int, key: torch.Tensor, value: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        """Store one layer's new tokens (BF16 ``[N, H, 128]``, rows may be strided)."""
        extension().hbm_write(*self._state, key, value, slot_mapping, layer)

    def encode(self, layer: int, max_close: int, ordered: bool = False) -> None:
        """Code this layer's records of the blocks closed this step.

        ``ordered``: place each block's records in (kv, head) order, so the
        arena bytes and the spill set depend only on the records (the
        reference places records in arrival order).
        """
        extension().hbm_encode(*self._state, self.tables.rank_of, layer, self.arena_base[layer],
                               self.arena_stride[layer], max_close, ordered=ordered)

    def write_encode(self, layer: int, key: torch.Tensor, value: torch.Tensor, slot_mapping: torch.Tensor,
                     max_close: int, ordered: bool = False) -> None:
        """``write`` then ``encode`` of one layer in one launch (the decode-step
        fusion; fragpack_step_bench.py:472-610 times the two separately).

        Results equal the two calls'.  The encoders of closing blocks write
        those blocks' new rows themselves, scanning the whole slot mapping per
        record: meant for steps of few tokens (decode steps).
        """
        extension().hbm_write_encode(*self._state, key, value, slot_mapping, self.tables.rank_of, layer,
                                     self.arena_base[layer], self.arena_stride[layer], max_close, ordered=ordered)

    def commit(self) -> None:
        """After the last layer: release or hand over the closed blocks' staging."""
        extension().hbm_commit(*self._state)

    # ----------------------------------------------------------------- readers
    def layer_tables(self, layer: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
        """``(rec_addr, rec_len, plut, slut)`` of one layer, for decode attention."""
        return self._state.rec_addr[layer], self._state.rec_len[layer], self.tables.plut[layer], \
            self.tables.slut[layer]

    def gather(self, layer: int, blocks: torch.Tensor, wk: torch.Tensor, wv: torch.Tensor) -> None:
        """Decode blocks of one layer into token-major BF16 ``[P, 128, H, 128]`` pages."""
        addr, length, plut, slut = self.layer_tables(layer)
        extension().hbm_gather(blocks, addr, length, plut, slut, wk, wv, self.kv_heads)

    # ------------------------------------------------------------------ blobs
    @property
    def blob_stride(self) -> int:
        """Bytes to reserve per block blob (every record raw)."""
        return ap.blob_slot_bytes(self.num_layers, self.kv_heads)

    def export_blocks(self, blocks: torch.Tensor, out: torch.Tensor, stride: int) -> torch.Tensor:
        """Copy closed blocks into blobs at ``out[i * stride]``; returns int64 lengths."""
        lengths = torch.empty(blocks.numel(), dtype=torch.int64, device=out.device)
        extension().hbm_export(blocks, self._state.rec_addr, self._state.rec_len, out, stride, lengths,
                               self.table_digest)
        return lengths

    def import_blocks(self, src: torch.Tensor, offsets: torch.Tensor, blocks: torch.Tensor) -> torch.Tensor:
        """Install blobs into blocks; returns int32 status per blob (0: installed)."""
        status = torch.zeros(blocks.numel(), dtype=torch.int32, device=src.device)
        extension().hbm_import(*self._state, src, offsets, blocks, status, self.arena_base_dev,
                               self.arena_stride_dev, self.table_digest)
        return status

    # --------------------------------------------------------------- counters
    def poll(self) -> StoreStats | None:
        """Counters of the previous call, without waiting (None while the copy
        is in flight); raises :class:`StoreError` if KV was lost."""
        ready = None
        if self._poll_event is not None:
            if not self._poll_event.query():
                return None
            ready = self._checked(StoreStats.from_counters(self._poll_host.numpy()))
        self._poll_host.copy_(self._state.counters, non_blocking=True)
        self._poll_event = torch.cuda.Event()
        self._poll_event.record()
        return ready

    def stats(self) -> StoreStats:
        """Counters now (synchronises); raises :class:`StoreError` if KV was lost."""
        return self._checked(StoreStats.from_counters(self._state.counters.cpu().numpy()))

    @staticmethod
    def _checked(stats: StoreStats) -> StoreStats:
        if stats.lost:
            raise StoreError(
                f"FragPack store dropped KV: staging={stats.err_staging} overflow={stats.err_overflow} (size "
                "staging for one open block per running request, and the overflow pool with FRAGPACK_OVERFLOW)")
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
