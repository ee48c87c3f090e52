"""Pins the CPU store model (oracle/store_model.py) that the GPU store's
bookkeeping is compared with: hand-derived outcomes of the reference's
prepare / commit rules (fragpack/ops/hbm_kv.cu:110-219, 431-448;
hbm_kv.py:1-47) on small steps, and the invariants that hold whatever the
list order.  CPU only."""

from __future__ import annotations

import numpy as np

from oracle.store_model import CLAIMS, CLOSES, DONORS, ERR_STAGING, FREE_TOP, HEIRS, TRANS, StoreModel

T = 128


def _slots(block, start, n):
    return [block * T + p for p in range(start, start + n)]


def _invariants(m: StoreModel):
    held = [int(w) for w in m.wslot if 0 <= w < m.staging_slots]
    assert len(held) == len(set(held)), "a persistent slot held twice"
    assert sorted(held + m.free_stack) == list(range(m.staging_slots))


def test_open_block_claims_a_persistent_slot_and_keeps_it_while_live():
    m = StoreModel(1, 8, 1, staging_slots=2, scratch_slots=4)
    m.prepare(_slots(3, 0, 10), live=[])
    assert m.claims == [3] and m.wslot[3] == 1  # the stack's top (slots pushed 0, 1)
    assert m.closes == [] and m.counters[CLAIMS] == 1 and m.counters[FREE_TOP] == 1
    m.commit()
    m.prepare(_slots(3, 10, 1), live=[3])  # a decode token: no claim, the slot stays
    assert m.claims == [] and m.wslot[3] == 1
    _invariants(m)


def test_block_not_live_is_collected():
    m = StoreModel(1, 8, 1, staging_slots=1, scratch_slots=4)
    m.prepare(_slots(2, 0, 5), live=[])
    m.commit()
    m.prepare(_slots(4, 0, 5), live=[])  # block 2's request finished: its slot serves block 4
    assert m.wslot[2] == -1 and m.wslot[4] == 0 and m.counters[ERR_STAGING] == 0
    _invariants(m)


def test_block_opening_and_closing_in_one_step_uses_transient_scratch():
    m = StoreModel(2, 8, 2, staging_slots=1, scratch_slots=3)
    m.prepare(_slots(5, 0, T), live=[])
    assert m.wslot[5] == 1 and m.counters[TRANS] == 1  # S_p + 0
    assert m.closes == [(5, -1)] and m.counters[CLOSES] == 1
    # transient staging has no layer dimension: record (kv, head) of slot t
    assert m.staging_addr(1, 1, 3) == m.scratch_base + 3 * 32768
    m.commit()
    assert m.wslot[5] == -1 and m.free_stack == [0]
    _invariants(m)


def test_heir_takes_the_closing_blocks_slot():
    """A chunk that fills a request's open block and opens the next one
    while no persistent slot is free (hbm_kv.py:24-29)."""
    m = StoreModel(1, 8, 1, staging_slots=1, scratch_slots=3)
    m.prepare(_slots(0, 0, 100), live=[])
    m.commit()
    assert m.wslot[0] == 0
    m.prepare(_slots(0, 100, 28) + _slots(1, 0, 50), live=[0])
    assert m.wslot[1] == 1 and m.heirs == [1]  # staged in scratch as an heir
    assert m.closes == [(0, 1)] and m.counters[HEIRS] == 1 and m.counters[DONORS] == 1
    assert m.counters[ERR_STAGING] == 0
    m.commit()
    assert m.wslot[1] == 0 and m.wslot[0] == -1 and m.free_stack == []
    _invariants(m)


def test_staging_exhaustion_is_counted():
    m = StoreModel(1, 8, 1, staging_slots=1, scratch_slots=1)
    # two open blocks, one persistent slot, one scratch slot: the second is
    # an heir with no donor (error); a third open block has nothing left
    m.prepare(_slots(1, 0, 5) + _slots(2, 0, 5) + _slots(3, 0, 5), live=[])
    assert m.wslot[1] == 0 and m.heirs == [2] and m.wslot[3] == -1
    assert m.counters[ERR_STAGING] == 2  # block 3 unstaged, heir 2 unpaired
    assert m.claims == [1, 2]


def test_duplicate_and_padding_slots():
    m = StoreModel(1, 4, 1, staging_slots=2, scratch_slots=2)
    m.prepare([-1, 2 * T, 2 * T, -5, 9 * T], live=[])  # block 9 is past the store
    assert m.claims == [2] and m.counters[CLAIMS] == 1


def test_random_steps_keep_invariants():
    rng = np.random.default_rng(0)
    m = StoreModel(2, 64, 2, staging_slots=6, scratch_slots=10)
    pos = {}  # request -> (blocks, computed)
    free = list(range(64))
    for step in range(200):
        if len(pos) < 6 and rng.random() < 0.4:
            pos[step] = ([], 0)
        for r in list(pos):
            if rng.random() < 0.05:
                free.extend(pos.pop(r)[0])
        live = [bl[c // T] for bl, c in pos.values() if c % T and c // T < len(bl)]
        slots = []
        for r, (bl, c) in list(pos.items()):
            n = int(rng.integers(1, 200)) if rng.random() < 0.3 else 1
            need = -(-(c + n) // T) - len(bl)
            if need > len(free):
                continue
            bl = bl + [free.pop(0) for _ in range(need)]
            slots += [bl[p // T] * T + p % T for p in range(c, c + n)]
            pos[r] = (bl, c + n)
        m.prepare(slots, live)
        _invariants(m)
        assert all(m.wslot[b] >= 0 for b in live), "a live block lost its slot"
        m.commit()
        _invariants(m)
