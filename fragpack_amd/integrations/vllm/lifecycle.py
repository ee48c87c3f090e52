"""Host-side tracking of each running request's writable KV block.

Reference: fragpack/integrations/vllm/lifecycle.py (OpenBlocks).  The store
keeps a staging slot for every block a request may still write; vLLM does not
pass those ids to attention backends, so the scheduler output is mirrored here
(the version-pinned runner wrapper in ``compat`` feeds it).  Imports neither
torch nor vLLM; no I/O, no device access.
"""

from __future__ import annotations

from typing import Any

import numpy as np
from numpy.typing import NDArray


class OpenBlocks:
    """Per-request block lists and computed lengths, from scheduler outputs.

    Only the block that holds a request's next token (its first uncomputed
    position, when that position is not block-aligned) is reported live: a
    larger set is unsafe, since a freed open block may be handed to a new
    request ahead of its write position and would keep an obsolete staging
    slot.

    Args:
        block_tokens: Token slots per KV block.

    Thread-safety:
        One instance per worker, used on the model-runner thread only.
    """

    def __init__(self, block_tokens: int) -> None:
        if block_tokens <= 0:
            raise ValueError("block_tokens must be positive")
        self.block_tokens = block_tokens
        self.blocks: dict[str, list[int]] = {}
        self.computed: dict[str, int] = {}

    def update(self, so: Any) -> None:
        """Apply one step's scheduler output, in the V2 runner's order:
        finished / preempted requests are dropped first (so a request
        re-admitted in the same step starts from its new allocation), then new
        requests are added, authoritative block-table replacements applied,
        and cached requests advanced (a resumed request replaces its list,
        others append their newly allocated blocks unless a replacement was
        given this step).

        Args:
            so: A SchedulerOutput-like object: ``finished_req_ids``,
                ``preempted_req_ids`` (may be None), ``scheduled_new_reqs``
                (``req_id``, ``block_ids``, ``num_computed_tokens``),
                ``block_table_updates`` (may be None),
                ``scheduled_cached_reqs`` (``req_ids``, ``num_computed_tokens``,
                ``new_block_ids``, ``resumed_req_ids``).
        """
        gone = set(so.finished_req_ids) | set(so.preempted_req_ids or ())
        for req in gone:
            self.blocks.pop(req, None)
            self.computed.pop(req, None)
        for new in so.scheduled_new_reqs:
            self.blocks[new.req_id] = list(new.block_ids[0])
            self.computed[new.req_id] = int(new.num_computed_tokens)
        replaced = dict(so.block_table_updates or {})
        for req, ids in replaced.items():
            if req in self.blocks:
                self.blocks[req] = list(ids[0])
        cached = so.scheduled_cached_reqs
        if len(cached.req_ids) != len(cached.num_computed_tokens) or len(cached.req_ids) != len(
            cached.new_block_ids
        ):
            raise ValueError("scheduled_cached_reqs fields differ in length")
        for req, computed, new_ids in zip(cached.req_ids, cached.num_computed_tokens, cached.new_block_ids):
            if req not in self.blocks:
                continue  # preempted this step, or never admitted here
            self.computed[req] = int(computed)
            if new_ids is None or req in replaced:
                continue
            if req in cached.resumed_req_ids:
                self.blocks[req] = list(new_ids[0])
            else:
                self.blocks[req].extend(new_ids[0])

    def live_blocks(self) -> NDArray[np.int32]:
        """Block ids being written: for each tracked request whose computed
        length is not block-aligned, the block holding its next token (if
        allocated).

        Returns:
            int32 array, at most one id per request.
        """
        live = []
        for req, blocks in self.blocks.items():
            index, offset = divmod(self.computed[req], self.block_tokens)
            if offset and index < len(blocks):
                live.append(blocks[index])
        return np.asarray(live, dtype=np.int32)


__all__ = ["OpenBlocks"]
