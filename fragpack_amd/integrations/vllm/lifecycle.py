"""Which KV block each running request is still writing, from scheduler outputs.

Reference interface: fragpack/integrations/vllm/lifecycle.py (OpenBlocks,
``update`` / ``live_blocks``).  The store keeps a staging slot for every block
a request may still append to; vLLM hands attention backends no request ids,
so the worker mirrors the scheduler's per-request block lists here (fed by the
runner wrapper in ``compat``).  Host-only: imports neither torch nor vLLM.

Design: one :class:`_Request` per tracked request (its block list and
computed length).  A step's scheduler output is applied as four passes in
the V2 runner's order -- forget finished / preempted requests, admit new
ones, install authoritative block-table replacements, advance cached ones --
and :meth:`OpenBlocks.live_blocks` asks each request for the block holding
its next token.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Iterable

import numpy as np
from numpy.typing import NDArray


@dataclass
class _Request:
    blocks: list[int] = field(default_factory=list)
    computed: int = 0

    def writing(self, block_tokens: int) -> int | None:
        """The allocated block that holds the next token, when the computed
        length stops inside a block; None otherwise."""
        index, offset = divmod(self.computed, block_tokens)
        if offset == 0 or index >= len(self.blocks):
            return None
        return self.blocks[index]


class OpenBlocks:
    """Per-request block lists and computed lengths, from scheduler outputs.

    Only a request's next-token block is ever reported live (and only when
    that position is not block-aligned): reporting more would let a block
    that was freed and re-allocated to another request ahead of its write
    position keep a stale staging slot.

    Args:
        block_tokens: Token slots per KV block.

    Thread-safety:
        One instance per worker, used from the model-runner thread only.
    """

    def __init__(self, block_tokens: int) -> None:
        if block_tokens <= 0:
            raise ValueError("block_tokens must be positive")
        self.block_tokens = block_tokens
        self._reqs: dict[str, _Request] = {}

    # views kept for callers that inspect the mirror
    @property
    def blocks(self) -> dict[str, list[int]]:
        return {rid: r.blocks for rid, r in self._reqs.items()}

    @property
    def computed(self) -> dict[str, int]:
        return {rid: r.computed for rid, r in self._reqs.items()}

    def _forget(self, ids: Iterable[str]) -> None:
        for rid in ids:
            self._reqs.pop(rid, None)

    def _admit(self, new_reqs: Iterable[Any]) -> None:
        for nr in new_reqs:
            self._reqs[nr.req_id] = _Request(list(nr.block_ids[0]), int(nr.num_computed_tokens))

    def _replace_tables(self, updates: dict) -> set[str]:
        for rid, ids in updates.items():
            req = self._reqs.get(rid)
            if req is not None:
                req.blocks = list(ids[0])
        return set(updates)

    def _advance(self, cached: Any, replaced: set[str]) -> None:
        rows = (cached.req_ids, cached.num_computed_tokens, cached.new_block_ids)
        if len({len(x) for x in rows}) != 1:
            raise ValueError("scheduled_cached_reqs fields differ in length")
        resumed = set(cached.resumed_req_ids)
        for rid, computed, new_ids in zip(*rows):
            req = self._reqs.get(rid)
            if req is None:  # preempted this step, or never admitted on this worker
                continue
            req.computed = int(computed)
            if new_ids is None or rid in replaced:
                continue  # no new blocks, or this step's replacement is authoritative
            req.blocks = list(new_ids[0]) if rid in resumed else req.blocks + list(new_ids[0])

    def update(self, so: Any) -> None:
        """Apply one step's scheduler output.

        Args:
            so: A SchedulerOutput-like object with ``finished_req_ids``,
                ``preempted_req_ids`` (may be None), ``scheduled_new_reqs``
                (``req_id``, ``block_ids``, ``num_computed_tokens``),
                ``block_table_updates`` (may be None) and
                ``scheduled_cached_reqs`` (``req_ids``, ``num_computed_tokens``,
                ``new_block_ids``, ``resumed_req_ids``).

        Raises:
            ValueError: If the cached-request fields differ in length.
        """
        self._forget(set(so.finished_req_ids) | set(so.preempted_req_ids or ()))
        self._admit(so.scheduled_new_reqs)
        replaced = self._replace_tables(dict(so.block_table_updates or {}))
        self._advance(so.scheduled_cached_reqs, replaced)

    def live_blocks(self) -> NDArray[np.int32]:
        """int32 ids of the blocks being written, at most one per request."""
        live = (r.writing(self.block_tokens) for r in self._reqs.values())
        return np.fromiter((b for b in live if b is not None), dtype=np.int32)


__all__ = ["OpenBlocks"]
