"""Engine-independent per-step and per-layer work of the serving backend.

Reference: fragpack/integrations/vllm/backend.py.  The vLLM classes there
(metadata builder, attention impl) mix engine plumbing with the store's step
protocol; this module holds the protocol alone, on plain host arrays and
device tensors, so that it runs (and is tested) without vLLM:

- :func:`plan_step` — host-only: decode / prefill split, the encode grid bound
  (blocks closed this step) and the prefill groups that share the BF16
  workspace (backend.py:276-290, 398-446);
- :class:`FragPackRunner` — owns the store, the decode workspace and the
  prefill workspace; :meth:`~FragPackRunner.bind` makes the store over the
  engine's per-layer caches (backend.py:311-384), :meth:`~FragPackRunner.build`
  prepares one step (backend.py:269-309), :meth:`~FragPackRunner.layer_forward`
  writes, attends and encodes one layer (backend.py:537-578).

Per step the order is: ``prepare`` (once), then per layer ``write`` ->
decode attention over the compressed records (the first layer plans the
split-KV schedule, the others reuse it) -> per prefill group ``gather`` into
the workspace + MFMA prefill -> ``encode`` of the blocks closed this step; the
last layer ``commit``s.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
from numpy.typing import NDArray

from fragpack_amd.integrations.vllm.capacity import FragPackCapacity, publish_capacity
from fragpack_amd.logging import init_logger

BLOCK_TOKENS = 128
HEAD_DIM = 128
POLL_EVERY = 16
LOG_EVERY = 4096
# Raw (incompressible) records the overflow pool holds; FRAGPACK_OVERFLOW
# overrides it.  Real KV rarely falls back, but a degenerate prompt (one token
# repeated) falls back for most records: 8192 records (256 MiB) hold such a
# 2048-token prompt beside normal traffic.
OVERFLOW_RECORDS = 8192

logger = init_logger(__name__)


def split_decodes(query_lens: NDArray[np.int64]) -> int:
    """Leading single-token rows of a batch whose decodes come first (vLLM's
    ``split_decodes_and_prefills`` with threshold 1, backend.py:273).

    Returns:
        The number of decode rows: all rows when none has more than one
        query token, else the index of the first such row.
    """
    long_rows = np.flatnonzero(query_lens > 1)
    return int(query_lens.size if long_rows.size == 0 else long_rows[0])


@dataclass
class HostPrefillGroup:
    """One workspace pass of prefill rows, host side (backend.py:83-107).

    Attributes:
        r0, r1: Batch rows ``[r0, r1)``.
        src_rows, src_cols: ``[P]`` (row, page) of the engine's block table
            whose blocks are decoded into workspace pages ``0..P``.
        block_table: int32 ``[R, max_pages]`` workspace pages per row.
        cu_seqlens_q: int32 ``[R + 1]`` query offsets relative to ``tok0``.
        seqused_k: int32 ``[R]`` context lengths.
        tok0, tok1: The group's token range in the batch.
        max_seqlen_q, max_seqlen_k: Longest query / context.
    """

    r0: int
    r1: int
    src_rows: NDArray[np.int64]
    src_cols: NDArray[np.int64]
    block_table: NDArray[np.int32]
    cu_seqlens_q: NDArray[np.int32]
    seqused_k: NDArray[np.int32]
    tok0: int
    tok1: int
    max_seqlen_q: int
    max_seqlen_k: int


@dataclass
class HostStep:
    """Host-side plan of one step.

    Attributes:
        num_reqs: Rows of the batch.
        num_decodes: Leading single-token rows.
        num_tokens: Batch tokens that carry a slot.
        closes: Blocks receiving their last token this step.
        max_close: Grid bound of each layer's encode.
        prefills: Prefill groups (empty in a capture build).
    """

    num_reqs: int
    num_decodes: int
    num_tokens: int
    closes: int
    max_close: int
    prefills: list[HostPrefillGroup]


def plan_step(
    query_start_loc: NDArray[np.integer],
    seq_lens: NDArray[np.integer],
    slot_rows: int,
    workspace_pages: int,
    max_tokens: int,
    capture: bool = False,
) -> HostStep:
    """Plan one step from the batch's host metadata (backend.py:269-290).

    Args:
        query_start_loc: ``[R + 1]`` query offsets (decodes first).
        seq_lens: ``[R]`` context lengths including this step's tokens.
        slot_rows: Rows of the slot mapping (bounds ``num_tokens``).
        workspace_pages: Pages of the BF16 prefill workspace.
        max_tokens: Largest step the store was sized for.
        capture: A graph-capture build: no prefill groups, and an encode
            grid that covers every replay of the captured decode shape.

    Raises:
        ValueError: A prefill row needs more pages than the workspace holds.
    """
    qsl = np.asarray(query_start_loc, dtype=np.int64)
    num_reqs = qsl.size - 1
    seq = np.asarray(seq_lens, dtype=np.int64)[:num_reqs]
    qlen = qsl[1:] - qsl[:-1]
    nd = split_decodes(qlen)
    num_tokens = min(int(qsl[num_reqs]), slot_rows)
    # one close per 128-token boundary crossed by the row's new tokens
    closes = int(np.sum(seq // BLOCK_TOKENS - np.maximum(seq - qlen, 0) // BLOCK_TOKENS))
    # A captured decode shape encodes with a grid that covers every replay
    # (each decode closes at most one block).  Any other build is launched
    # as planned, so its grid is the exact close count and a step that
    # closes nothing launches no encode (the reference always sizes the grid
    # for capture, backend.py:287).
    max_close = min(max(closes, nd) if capture else closes, max_tokens)
    prefills: list[HostPrefillGroup] = []
    if not capture and nd < num_reqs:
        prefills = prefill_groups(qsl, seq, nd, workspace_pages)
    return HostStep(num_reqs, nd, num_tokens, closes, max_close, prefills)


def default_workspace_pages(max_model_len: int, max_tokens: int, max_reqs: int) -> int:
    """Pages of the BF16 prefill workspace: one max-length context, or a
    whole step of fresh prompts if that is more (every token of the step's
    budget plus one partial page per request).

    The reference sizes the workspace for one max-length context
    (backend.py:398-411), so a step of several fresh prompts prefills in one
    launch per workspace pass; sized for the step, the step's prefill is one
    launch, and the workspace stays a small fraction of the GPU's HBM.
    """
    return max(-(-max_model_len // BLOCK_TOKENS), -(-max_tokens // BLOCK_TOKENS) + max_reqs)


def prefill_groups(
    qsl: NDArray[np.int64], seq: NDArray[np.int64], first: int, workspace_pages: int
) -> list[HostPrefillGroup]:
    """Greedy in-order packing of prefill rows ``first..R`` into workspace
    passes of at most ``workspace_pages`` pages (backend.py:398-411)."""
    num_reqs = qsl.size - 1
    pages = -(-seq // BLOCK_TOKENS)
    if first < num_reqs and int(pages[first:num_reqs].max()) > workspace_pages:
        raise ValueError(f"a prefill context of {int(seq[first:num_reqs].max())} tokens exceeds the "
                         f"{workspace_pages}-page workspace")
    groups = []
    start, used = first, 0
    for r in range(first, num_reqs):
        if used + pages[r] > workspace_pages and r > start:
            groups.append(_group(qsl, seq, pages, start, r))
            start, used = r, 0
        used += int(pages[r])
    groups.append(_group(qsl, seq, pages, start, num_reqs))
    return groups


def _group(qsl, seq, pages, r0: int, r1: int) -> HostPrefillGroup:
    pg = pages[r0:r1]
    offs = np.concatenate(([0], np.cumsum(pg)))
    total, width = int(offs[-1]), max(1, int(pg.max()))
    table = np.zeros((r1 - r0, width), dtype=np.int32)
    for i in range(r1 - r0):
        table[i, : pg[i]] = np.arange(offs[i], offs[i + 1])
    qlen = qsl[r0 + 1 : r1 + 1] - qsl[r0:r1]
    return HostPrefillGroup(
        r0=r0,
        r1=r1,
        src_rows=np.repeat(np.arange(r0, r1), pg),
        src_cols=np.arange(total) - np.repeat(offs[:-1], pg),
        block_table=table,
        cu_seqlens_q=(qsl[r0 : r1 + 1] - qsl[r0]).astype(np.int32),
        seqused_k=seq[r0:r1].astype(np.int32),
        tok0=int(qsl[r0]),
        tok1=int(qsl[r1]),
        max_seqlen_q=int(qlen.max()),
        max_seqlen_k=int(seq[r0:r1].max()),
    )


@dataclass
class PrefillGroup:
    """A prefill group on the device (backend.py:83-107)."""

    src_blocks: object  # torch int32 [P]
    block_table: object  # torch int32 [R, max_pages]
    cu_seqlens_q: object  # torch int32 [R + 1]
    seqused_k: object  # torch int32 [R]
    tok0: int
    tok1: int
    max_seqlen_q: int
    max_seqlen_k: int


@dataclass
class FragPackMetadata:
    """Per-step metadata shared by every layer (backend.py:110-150).

    ``layer_index`` maps an engine layer name to its store layer; callers that
    have no names pass the index to :meth:`FragPackRunner.layer_forward`.
    """

    store: object
    layer_tables: list
    layer_index: dict[str, int]
    last_layer: int
    slot_mapping: object
    num_tokens: int
    num_decodes: int
    decode_block_table: object
    decode_seq_lens: object
    units: int
    decode_workspace: tuple
    max_close: int
    prefills: list[PrefillGroup]
    wk: object
    wv: object


class FragPackRunner:
    """The store, its tables and the attention workspaces of one worker.

    Args:
        kv_heads: KV heads on this worker.
        tables: Calibrated :class:`DeviceTables` for every layer.
        device: The GPU.
        max_tokens: Most tokens in a step (sizes store lists and scratch).
        max_reqs: Most running requests (staging slots, decode workspace).
        max_model_len: Longest sequence (sizes the prefill workspace).
        overflow_records: Raw-record overflow pool size.
        layer_names: Engine layer names in layer order (optional).
        workspace_pages: Pages of the BF16 prefill workspace (default: a
            step's whole token budget of fresh prompts, plus one partial
            page per request, and at least one ``max_model_len`` context).

    Used from the model-runner thread only; every method enqueues on the
    current stream.
    """

    def __init__(
        self,
        kv_heads: int,
        tables,
        device,
        max_tokens: int,
        max_reqs: int,
        max_model_len: int,
        overflow_records: int = OVERFLOW_RECORDS,
        layer_names: list[str] | None = None,
        workspace_pages: int | None = None,
    ) -> None:
        import torch

        from fragpack_amd.ops.fused_attn_decode import decode_units, workspace_elems

        self.kv_heads = kv_heads
        self.tables = tables
        self.device = torch.device(device)
        self.max_tokens = max_tokens
        self.max_reqs = max_reqs
        self.overflow_records = overflow_records
        self.layer_names = list(layer_names or [])
        self.layer_index = {name: i for i, name in enumerate(self.layer_names)}
        self.num_sms = torch.cuda.get_device_properties(self.device).multi_processor_count
        opart, ml, plan = workspace_elems(kv_heads, decode_units(max(max_reqs, 1), kv_heads, self.num_sms))
        self.decode_workspace = (
            torch.empty(opart, dtype=torch.float32, device=self.device),
            torch.empty(ml, dtype=torch.float32, device=self.device),
            torch.empty(plan, dtype=torch.int32, device=self.device),
        )
        if workspace_pages is None:
            workspace_pages = default_workspace_pages(max_model_len, max_tokens, max_reqs)
        if workspace_pages < -(-max_model_len // BLOCK_TOKENS):
            raise ValueError(f"workspace of {workspace_pages} pages cannot hold a {max_model_len}-token context")
        self.workspace_pages = workspace_pages
        shape = (self.workspace_pages, BLOCK_TOKENS, kv_heads, HEAD_DIM)
        self.wk = torch.empty(shape, dtype=torch.bfloat16, device=self.device)
        self.wv = torch.empty(shape, dtype=torch.bfloat16, device=self.device)
        self.store = None
        self.store_key: tuple[int, int] | None = None
        self.layer_tables: list = []
        self.steps = 0

    def bind(self, caches: list) -> object:
        """The store over ``caches`` (one uint8-viewable ``[blocks, page]``
        tensor per layer), made on first use and again whenever the engine
        re-binds its cache (backend.py:311-384).

        Raises:
            RuntimeError: The cache is not bound yet (empty tensor).
        """
        from fragpack_amd.ops.fused_attn_decode import RecordTables
        from fragpack_amd.ops.hbm_kv import HbmKvStore, register_store

        if not caches or caches[0].numel() == 0:
            raise RuntimeError("FragPack attention built metadata before the KV cache was bound")
        key = (caches[0].data_ptr(), caches[0].shape[0])
        if self.store is not None and key == self.store_key:
            return self.store
        # one staging slot per running request: a request holds at most one
        # open block across steps
        store = HbmKvStore(caches, self.kv_heads, self.tables, self.max_tokens, staging_slots=self.max_reqs,
                           overflow_records=self.overflow_records)
        self.store, self.store_key = store, key
        register_store(store)
        self.layer_tables = [RecordTables(*store.layer_tables(i)) for i in range(len(caches))]
        memory = store.memory_usage()
        memory["prefill_workspace"] = sum(t.numel() * t.element_size() for t in (self.wk, self.wv))
        memory["decode_workspace"] = sum(t.numel() * t.element_size() for t in self.decode_workspace)
        raw = 2 * self.kv_heads * BLOCK_TOKENS * HEAD_DIM * 2
        publish_capacity(FragPackCapacity(blocks=store.num_blocks, block_tokens=BLOCK_TOKENS, layers=store.num_layers,
                                          kv_heads=self.kv_heads, page_bytes=store.arena_stride[0],
                                          raw_page_bytes=raw, memory=memory))
        logger.info(
            "FragPack store: %d layers x %d blocks, %d B/block-layer (raw %d), %d staging slots, %d overflow "
            "records, %.0f MiB prefill workspace",
            store.num_layers, store.num_blocks, store.arena_stride[0], raw, self.max_reqs, self.overflow_records,
            memory["prefill_workspace"] / 2**20,
        )
        return store

    def build(
        self,
        caches: list,
        query_start_loc: NDArray[np.integer],
        seq_lens_host: NDArray[np.integer],
        seq_lens,
        block_table,
        slot_mapping,
        live_blocks: NDArray[np.int32],
        capture: bool = False,
    ) -> FragPackMetadata:
        """Prepare the store for one step and return the layers' metadata
        (backend.py:269-309).

        Args:
            caches: The engine's per-layer caches.
            query_start_loc: Host ``[R + 1]`` query offsets, decodes first.
            seq_lens_host: Host ``[R]`` context lengths (an upper bound is
                enough for planning).
            seq_lens: Device int32 ``[>= R]`` context lengths.
            block_table: Device int32 ``[>= R, pages]`` block ids.
            slot_mapping: Device int64 ``[>= tokens]`` slot ids.
            live_blocks: Blocks still being written (``OpenBlocks``).
            capture: Graph-capture build: launch shapes only, the store's
                state is not touched and no prefill groups are made.

        Raises:
            StoreError: The store dropped KV data since the last poll.
        """
        import torch

        from fragpack_amd.ops.fused_attn_decode import decode_units

        store = self.bind(caches)
        hs = plan_step(query_start_loc, seq_lens_host, slot_mapping.shape[0], self.workspace_pages,
                       self.max_tokens, capture=capture)
        if not capture:
            store.prepare(slot_mapping, hs.num_tokens, live_blocks)
            self.steps += 1
            if self.steps % POLL_EVERY == 0:
                stats = store.poll()
                if stats is not None and self.steps % LOG_EVERY == 0:
                    logger.info("FragPack store: %s", stats)
        prefills = []
        for g in hs.prefills:
            n, width = g.block_table.shape
            host = np.concatenate((g.src_rows, g.src_cols, g.block_table.ravel().astype(np.int64),
                                   g.cu_seqlens_q.astype(np.int64), g.seqused_k.astype(np.int64)))
            dev = torch.from_numpy(host).pin_memory().to(self.device, non_blocking=True)
            total = g.src_rows.size
            a, b, c, d = total, 2 * total, 2 * total + n * width, 2 * total + n * width + n + 1
            prefills.append(PrefillGroup(
                src_blocks=block_table[dev[:a], dev[a:b]].to(torch.int32),
                block_table=dev[b:c].view(n, width).to(torch.int32),
                cu_seqlens_q=dev[c:d].to(torch.int32),
                seqused_k=dev[d:].to(torch.int32),
                tok0=g.tok0, tok1=g.tok1, max_seqlen_q=g.max_seqlen_q, max_seqlen_k=g.max_seqlen_k,
            ))
        nd = hs.num_decodes
        return FragPackMetadata(
            store=store,
            layer_tables=self.layer_tables,
            layer_index=self.layer_index,
            last_layer=store.num_layers - 1,
            slot_mapping=slot_mapping,
            num_tokens=hs.num_tokens,
            num_decodes=nd,
            decode_block_table=block_table[:nd],
            decode_seq_lens=seq_lens[:nd],
            units=decode_units(max(nd, 1), self.kv_heads, self.num_sms),
            decode_workspace=self.decode_workspace,
            max_close=hs.max_close,
            prefills=prefills,
            wk=self.wk,
            wv=self.wv,
        )


# Steps of at most this many tokens write and encode each layer in one
# launch (fp_hbm_write_encode): each closing record's encoder scans the slot
# mapping, which stays cheap for decode-sized steps.
FUSED_STEP_TOKENS = 512


def layer_forward(md: FragPackMetadata, li: int, query, key, value, output, scale: float):
    """Write one layer's new KV, attend, encode the blocks closed this step,
    and commit after the last layer (backend.py:537-578); steps of up to
    ``FUSED_STEP_TOKENS`` tokens write and encode in one launch before
    attending.

    Args:
        md: The step's metadata; None in an engine's profiling run (the
            output is zeroed).
        li: Store layer index.
        query: BF16 ``[T, Hq, 128]``; key / value BF16 ``[T, H, 128]``.
        output: BF16 ``[T, Hq, 128]``.
        scale: Softmax scale.

    Returns:
        ``output``.
    """
    from fragpack_amd.ops.fused_attn_decode import decode_attention
    from fragpack_amd.ops.prefill_attn import flash_attn_varlen_func

    if md is None:
        return output.zero_()
    store = md.store
    n = md.num_tokens
    # A step of few tokens writes and encodes in one launch, before attention
    # rather than after it: the blocks it closes are then read back from
    # their coded records, which hold the same bits.
    fused = n <= FUSED_STEP_TOKENS
    if fused:
        store.write_encode(li, key[:n], value[:n], md.slot_mapping[:n], md.max_close)
    else:
        store.write(li, key[:n], value[:n], md.slot_mapping[:n])
    nd = md.num_decodes
    if nd:
        decode_attention(query[:nd], md.layer_tables[li], md.decode_block_table, md.decode_seq_lens, scale,
                         md.units, output[:nd], md.decode_workspace, replan=li == 0)
    for g in md.prefills:
        store.gather(li, g.src_blocks, md.wk, md.wv)
        flash_attn_varlen_func(q=query[g.tok0 : g.tok1], k=md.wk, v=md.wv, out=output[g.tok0 : g.tok1],
                               cu_seqlens_q=g.cu_seqlens_q, max_seqlen_q=g.max_seqlen_q, seqused_k=g.seqused_k,
                               max_seqlen_k=g.max_seqlen_k, softmax_scale=scale, causal=True,
                               block_table=g.block_table)
    if not fused:
        store.encode(li, md.max_close)
    if li == md.last_layer:
        store.commit()
    return output


__all__ = [
    "FragPackMetadata",
    "FragPackRunner",
    "HostPrefillGroup",
    "HostStep",
    "PrefillGroup",
    "default_workspace_pages",
    "layer_forward",
    "plan_step",
    "prefill_groups",
    "split_decodes",
]
