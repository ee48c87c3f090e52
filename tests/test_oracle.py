"""Pins the CPU oracle before anything is checked against it.

* Golden vectors written by the reference codec itself
  (tests/golden/make_golden.py): exact record bytes for K and V records with
  escapes, raw bytes, VAR_CAP / MAX_WARP_RAW boundaries and fallbacks; the
  kernel order; LUTs; calibration including ties.
* Invariants the format fixes: decode(encode(x)) == x, the closed-form
  variable length, the fallback rule, the kernel order being a permutation.
* Attention: the oracle's fp32 paged attention against a float64 numpy
  softmax on the same KV, and the repetition identity (a page repeated n
  times == its logits + log n).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle
from tests import kvgen


def _records(golden):
    names = golden["record_names"]
    for i, name in enumerate(names):
        yield (str(name), golden[f"r{i}_raw"], golden[f"r{i}_table"], int(golden[f"r{i}_kv"]),
               golden[f"r{i}_enc"].tobytes())


def test_golden_encode_bytes(golden):
    n = 0
    for name, raw, table, kv, enc in _records(golden):
        assert oracle.encode_record(raw, table, kv) == enc, name
        n += 1
    assert n >= 30


def test_golden_decode(golden):
    for name, raw, table, kv, enc in _records(golden):
        assert np.array_equal(oracle.decode_record(enc, table, kv), raw), name


def test_golden_covers_boundaries(golden):
    lens = {name: len(enc) for name, _, _, _, enc in _records(golden)}
    assert lens["edge_ext4000_kv0"] == 22528 + 2048  # exactly VAR_CAP
    assert lens["edge_ext4001_kv0"] == 32768  # one nibble over -> raw
    assert lens["edge_raw32_kv1"] < 32768 and lens["edge_raw33_kv1"] == 32768  # warp raw cap
    assert lens["edge_rawcap_fit_kv0"] == 22528 + 2048 and lens["edge_rawcap_over_kv0"] == 32768
    assert lens["unit_incompressible_kv0"] == 32768


def test_kernel_order(golden):
    for kv in (0, 1):
        order = oracle.kernel_order(kv)
        assert np.array_equal(order, golden[f"kernel_order_kv{kv}"])
        assert np.array_equal(np.sort(order), np.arange(16384))


def test_luts_and_tables(golden):
    for i in range(2):
        table = golden[f"plut{i}_table"]
        rank_of, plut, slut = oracle.tables(table)
        assert np.array_equal(plut, golden[f"plut{i}"])
        assert np.array_equal(slut, golden[f"slut{i}"])
        assert np.array_equal(rank_of[table], np.arange(22))
        assert np.count_nonzero(rank_of != 255) == 22
    # device_tables of the calibrated dump
    tables = golden["cal_table"]
    for idx in np.ndindex(tables.shape[:3]):
        rank_of, plut, slut = oracle.tables(tables[idx])
        assert np.array_equal(rank_of, golden["cal_rank_of"][idx])
        assert np.array_equal(plut.view(np.int32), golden["cal_plut"][idx])
        assert np.array_equal(slut, golden["cal_slut"][idx])


def test_calibration(golden):
    assert np.array_equal(oracle.calibrate(golden["cal_dump"]), golden["cal_table"])
    assert np.array_equal(oracle.calibrate_table(golden["tie_input"]), golden["tie_table"])
    # brute force: top-22 by (-count, value)
    rng = np.random.default_rng(5)
    x = rng.integers(0, 40, 3000).astype(np.uint8)
    counts = np.bincount(x, minlength=256)
    want = sorted(range(256), key=lambda v: (-counts[v], v))[:22]
    assert list(oracle.calibrate_table(x)) == want


def _closed_form_len(raw, table, kv):
    """Record length from the format's arithmetic alone (attn_page.py:195-202)."""
    rank = np.full(256, 255, np.uint8)
    rank[table] = np.arange(22)
    vals = raw.reshape(-1)[oracle.kernel_order(kv)]
    r = rank[vals >> 8]
    esc = r >= 7
    raw_s = r >= 22
    n_esc, n_raw = int(esc.sum()), int(raw_s.sum())
    raw_offset = (48 + (n_esc + 1) // 2 + 3) & ~3
    var_len = (raw_offset + 4 * n_raw + 15) & ~15
    if var_len > 2048 or raw_s.reshape(8, 2048).sum(1).max() > 32:
        return 32768
    return 22528 + var_len


@pytest.mark.parametrize("kv", [0, 1])
@pytest.mark.parametrize("density", [0.0, 0.03, 0.2, 0.5])
def test_round_trip_and_length(kv, density):
    rng = np.random.default_rng(int(density * 100) + kv)
    table = rng.permutation(256)[:22].astype(np.uint8)
    absent = np.setdiff1d(np.arange(256), table)
    n = 16384
    high = table[rng.integers(0, 7, n)].astype(np.uint16)
    esc = rng.random(n) < density
    high[esc] = table[7 + rng.integers(0, 15, int(esc.sum()))]
    rawm = rng.random(n) < density / 40
    high[rawm] = absent[rng.integers(0, absent.size, int(rawm.sum()))]
    raw = ((high << 8) | rng.integers(0, 256, n).astype(np.uint16)).reshape(128, 128).astype(np.uint16)
    enc = oracle.encode_record(raw, table, kv)
    assert len(enc) == _closed_form_len(raw, table, kv)
    assert len(enc) % 16 == 0
    assert np.array_equal(oracle.decode_record(enc, table, kv), raw)
    # the raw form holds the same words in kernel order
    rr = np.frombuffer(oracle.raw_record(raw, kv), np.uint16).reshape(8, 256, 8).transpose(1, 0, 2).reshape(-1)
    assert np.array_equal(rr, raw.reshape(-1)[oracle.kernel_order(kv)])


def test_known_answer_incompressible():
    """test_attn_page.py:38-47: table arange(22), uniform u16 -> raw record."""
    rng = np.random.default_rng(2)
    record = rng.integers(0, 1 << 16, size=(128, 128), dtype=np.uint16)
    for kv in (0, 1):
        enc = oracle.encode_record(record, np.arange(22, dtype=np.uint8), kv)
        assert len(enc) == 32768
        assert np.array_equal(oracle.decode_record(enc, np.arange(22, dtype=np.uint8), kv), record)


def test_batch_matches_single():
    rng = np.random.default_rng(7)
    raw = kvgen.kv_bits(rng, (6, 128, 128), 0.05)
    tables = np.stack([oracle.calibrate_table((raw[i] >> 8).astype(np.uint8)) for i in range(2)])
    tab_idx = np.array([0, 1, 0, 1, 1, 0], np.int32)
    kv = np.array([0, 0, 1, 1, 0, 1], np.int32)
    recs, lens = oracle.encode_batch(raw, tables, tab_idx, kv, threads=2)
    for i in range(6):
        assert recs[i, : lens[i]].tobytes() == oracle.encode_record(raw[i], tables[tab_idx[i]], kv[i])
    back = oracle.decode_batch(recs, lens, tables, tab_idx, kv, threads=2)
    assert np.array_equal(back, raw)


@pytest.mark.parametrize("group", [1, 4, 8])
def test_paged_attention_oracle_vs_float64(group):
    case = kvgen.decode_case(seed=3 + group, batch=3, heads=2, group=group, lens=[1, 300, 129])
    got = kvgen.oracle_decode(case, threads=2)
    want = kvgen.reference_attention(case)
    np.testing.assert_allclose(got, want, atol=1e-4, rtol=1e-4)


def test_paged_attention_repetition_identity():
    """A block repeated n times in the table == adding log(n) to its logits
    (the reference's long-context check, test_fragpack_decode_schedule.py:118-147)."""
    case = kvgen.decode_case(seed=11, batch=1, heads=1, group=8, lens=[256], raw_tail=False)
    blk = case.block_table[0, :2]
    reps = np.array([blk[0]] * 3 + [blk[1]], np.int32)
    case.block_table = reps[None]
    case.lens = np.array([512], np.int32)
    got = kvgen.oracle_decode(case, threads=2)[0]
    q = kvgen.bits_to_f32(case.q_bits[0]).astype(np.float64)
    k = kvgen.bits_to_f32(case.kv[blk, 0, :, 0, :]).reshape(-1, 128).astype(np.float64)
    v = kvgen.bits_to_f32(case.kv[blk, 1, :, 0, :]).reshape(-1, 128).astype(np.float64)
    s = q @ k.T * case.scale + np.concatenate([np.full(128, np.log(3.0)), np.zeros(128)])
    p = np.exp(s - s.max(1, keepdims=True))
    want = (p / p.sum(1, keepdims=True)) @ v
    np.testing.assert_allclose(got, want, atol=1e-4, rtol=1e-4)


def _plan_cost(pages: np.ndarray, ppc: int, heads: int, slots: int) -> tuple[int, int]:
    """Modelled makespan of a chunk size: rounds of resident workgroups
    times (chunk pages + one page of fixed unit cost), by direct counting."""
    n = sum(-(-int(x) // ppc) for x in pages)
    return -(-n * heads // slots) * (ppc + 1), n


@pytest.mark.parametrize("seed", range(6))
def test_decode_plan_invariants(seed):
    """The planner restatement against brute force over its candidate set:
    the chosen chunk size fits the unit cap, no candidate has a lower
    modelled cost (ties: no larger chunk with the same cost), and the unit
    map tiles every sequence's pages exactly once."""
    rng = np.random.default_rng(seed)
    batch = int(rng.integers(1, 300))
    lens = rng.integers(0, 40000, batch).astype(np.int32)
    lens[rng.random(batch) < 0.2] = 0
    units = batch + int(rng.integers(0, 600))
    heads, slots = int(rng.choice([1, 4, 8, 32])), 768
    ppc, used, unit_map, seq_map = oracle.decode_plan(lens, units, heads, slots)
    pages = (lens.astype(np.int64) + 127) // 128
    longest = int(pages.max(initial=0))
    cost, n = _plan_cost(pages, ppc, heads, slots)
    assert n == used <= units
    for c in range(1, 65):
        cand = max(1, -(-longest // c))
        cc, cn = _plan_cost(pages, cand, heads, slots)
        if cn <= units:
            assert cc > cost or (cc == cost and cand <= ppc)
    covered = np.zeros(int(pages.sum()), np.int64)
    offs = np.concatenate([[0], np.cumsum(pages)])
    for u, (b, p0) in enumerate(unit_map):
        if b < 0:
            assert u >= seq_map[:, 1].sum()
            continue
        assert seq_map[b, 0] <= u < seq_map[b, 0] + seq_map[b, 1]
        n = min(int(pages[b]), p0 + ppc) - p0
        assert n > 0
        covered[offs[b] + p0 : offs[b] + p0 + n] += 1
    assert np.all(covered == 1)


def test_decode_plan_known_answers():
    """Hand-computed plans on a 768-slot device.  Config 1 (4 x 64 pages, 4
    heads): ppc 2 gives 128 units per head = 512 workgroups, one round, cost
    3; ppc 1 needs two rounds (cost 4).  Config 4's decode (64 x 256 pages, 8
    heads): ppc 86 gives 3 chunks per row, 1536 workgroups in two rounds,
    cost 174, against 257 for one chunk per row.  Units equal to the batch
    cap the chunks: pages [3, 0, 71, 1] with 4 units take ppc 36 (4 chunks,
    cost 37; ppc 24 would need 5).  An all-empty batch plans nothing."""
    ppc, used, unit_map, seq_map = oracle.decode_plan(np.full(4, 8192, np.int32), 4 + 4 * 192 - 1, 4, 768)
    assert (ppc, used) == (2, 128)
    assert seq_map.tolist() == [[0, 32], [32, 32], [64, 32], [96, 32]]
    assert unit_map[33].tolist() == [1, 2] and unit_map[128, 0] == -1
    ppc, used, _, seq_map = oracle.decode_plan(np.full(64, 32768, np.int32), 64 + 4 * 96 - 1, 8, 768)
    assert (ppc, used) == (86, 192) and np.all(seq_map[:, 1] == 3)
    lens = np.array([300, 0, 9000, 1], np.int32)
    ppc, used, _, seq_map = oracle.decode_plan(lens, 4, 4, 768)
    assert used == 4 and ppc == 36 and seq_map[:, 1].tolist() == [1, 0, 2, 1]
    ppc, used, unit_map, seq_map = oracle.decode_plan(np.zeros(5, np.int32), 7, 4, 768)
    assert used == 0 and ppc == 1 and np.all(unit_map[:, 0] == -1) and not seq_map[:, 1].any()

