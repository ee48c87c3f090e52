"""CPU model of the HBM store's step bookkeeping -- TEST INFRASTRUCTURE ONLY.

Restates the reference's prepare / commit state machine
(fragpack/ops/hbm_kv.cu:110-219 prepare_kernel, :431-448 commit_kernel;
contract fragpack/ops/hbm_kv.py:1-47) over host arrays, with the order in
which the MI355X kernels build their lists (every list in input order, see
below), so a GPU store's state after each prepare / commit can be compared
with it exactly.  Loaded only by tests/.

Semantics (the reference's):
  * GC: a transient slot (index >= S_p) ends with its step; a persistent slot
    whose block is not in ``live`` returns to the free stack.
  * A block receiving offset 127 closes this step.
  * Claims (offset 0, one per block): a block that still holds a slot keeps
    it; a block that also closes takes transient scratch if any is left;
    otherwise the free stack's top; with the stack empty a block that stays
    open becomes an *heir* in transient scratch; anything else is a staging
    error.
  * Closes (offset 127, one per block holding staging): each closing block
    with a persistent slot is a donor, paired with the next heir.
  * Heirs left without a donor are staging errors.
  * Claimed blocks' records (every layer, kv, head) point at their staging,
    raw; overflow slots they held are freed; page fills reset.
  * commit: a donor's slot passes to its heir, other persistent slots of
    closing blocks return to the free stack, closing blocks drop their slot.

Order (the MI355X kernels' convention; the reference's atomics leave it
open): freed slots are pushed in block order; claims are taken in slot-
mapping order, closing claims first (transient scratch in order, the
overflow of those after the open claims on the free stack), open claims
popping the stack from its top; the claim list, heir list and close list
are in slot-mapping order; donors pair with heirs in close-list order;
commit pushes in close-list order.

Pinning: besides the exact comparison with the GPU, the tests check the
invariants that hold whatever the order -- every slot is held by at most one
block or is on the free stack exactly once, live blocks keep their slots,
counts of claims / closes / errors.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

RAW_RECORD = 32768
DENSE_BYTES = 22528
RAW_VAR_LEN = RAW_RECORD - DENSE_BYTES

# counter slots (hbm_kv.cu:14-26)
FREE_TOP, TRANS, CLAIMS, CLOSES, ERR_STAGING = 0, 1, 2, 3, 4
HEIRS, DONORS = 9, 10


@dataclass
class StoreModel:
    num_layers: int
    num_blocks: int
    kv_heads: int
    staging_slots: int
    scratch_slots: int
    staging_base: int = 0
    scratch_base: int = 0
    wslot: np.ndarray = field(init=False)
    free_stack: list = field(init=False)
    counters: np.ndarray = field(init=False)
    claims: list = field(default_factory=list)
    closes: list = field(default_factory=list)   # (block, heir or -1)
    heirs: list = field(default_factory=list)

    def __post_init__(self) -> None:
        self.wslot = np.full(self.num_blocks, -1, np.int64)
        self.free_stack = list(range(self.staging_slots))
        self.counters = np.zeros(16, np.int64)

    # ----------------------------------------------------------------- address
    def staging_addr(self, w: int, layer: int, kvh: int) -> int:
        """hbm_kv.cu:81-84 (staging_addr)."""
        H, L = self.kv_heads, self.num_layers
        if w < self.staging_slots:
            return self.staging_base + ((w * L + layer) * 2 * H + kvh) * RAW_RECORD
        return self.scratch_base + ((w - self.staging_slots) * 2 * H + kvh) * RAW_RECORD

    # ----------------------------------------------------------------- prepare
    def prepare(self, slots, live) -> None:
        S_p, S_t, NB = self.staging_slots, self.scratch_slots, self.num_blocks
        slots = [int(x) for x in slots]
        live_slots = {int(self.wslot[b]) for b in live if 0 <= b < NB and 0 <= self.wslot[b] < S_p}
        errors = 0
        for b in range(NB):  # GC in block order
            w = int(self.wslot[b])
            if w >= S_p:
                self.wslot[b] = -1
            elif w >= 0 and w not in live_slots:
                self.wslot[b] = -1
                self.free_stack.append(w)
        closing = {s >> 7 for s in slots if s >= 0 and s % 128 == 127 and (s >> 7) < NB}
        seen, cand = set(), []
        for s in slots:
            if s >= 0 and s % 128 == 0 and (s >> 7) < NB and (s >> 7) not in seen:
                seen.add(s >> 7)
                cand.append(s >> 7)
        close_claims = [b for b in cand if self.wslot[b] < 0 and b in closing]
        open_claims = [b for b in cand if self.wslot[b] < 0 and b not in closing]
        late = []
        for r, b in enumerate(close_claims):
            if r < S_t:
                self.wslot[b] = S_p + r
            else:
                late.append(b)
        trans = min(len(close_claims), S_t)
        self.heirs = []
        for b in open_claims:
            if self.free_stack:
                self.wslot[b] = self.free_stack.pop()
            elif trans < S_t:
                self.wslot[b] = S_p + trans
                trans += 1
                self.heirs.append(b)
            else:
                errors += 1
        for b in late:
            if self.free_stack:
                self.wslot[b] = self.free_stack.pop()
            else:
                errors += 1
        self.claims = [b for b in cand if self.wslot[b] >= 0]
        self.closes = []
        seen = set()
        donors = 0
        for s in slots:
            b = s >> 7
            if s < 0 or s % 128 != 127 or b >= NB or b in seen:
                continue
            seen.add(b)
            w = int(self.wslot[b])
            if w < 0:
                continue
            heir = -1
            if w < S_p:
                if donors < len(self.heirs):
                    heir = self.heirs[donors]
                donors += 1
            self.closes.append((b, heir))
        errors += max(len(self.heirs) - donors, 0)
        c = self.counters
        c[FREE_TOP] = len(self.free_stack)
        c[TRANS] = trans
        c[CLAIMS] = len(self.claims)
        c[CLOSES] = len(self.closes)
        c[HEIRS] = len(self.heirs)
        c[DONORS] = donors
        c[ERR_STAGING] += errors

    def claimed_records(self):
        """(layer, block, kvh) -> staging address of every claimed block's records."""
        out = {}
        for b in self.claims:
            for layer in range(self.num_layers):
                for kvh in range(2 * self.kv_heads):
                    out[(layer, b, kvh)] = self.staging_addr(int(self.wslot[b]), layer, kvh)
        return out

    # ------------------------------------------------------------------ commit
    def commit(self) -> None:
        for b, heir in self.closes:
            w = int(self.wslot[b])
            self.wslot[b] = -1
            if heir >= 0:
                self.wslot[heir] = w
            elif 0 <= w < self.staging_slots:
                self.free_stack.append(w)
        self.closes = []
        self.counters[FREE_TOP] = len(self.free_stack)
        self.counters[CLOSES] = 0
