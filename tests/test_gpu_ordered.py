"""Ordered encode (fp_hbm_encode_ordered) on the GPU vs the placement rule.

Both of its paths are covered: a step closing few blocks (two parallel
passes: measure, then place) and one closing enough blocks to fill the
device block by block (one workgroup walks each block's records).

The rule: each closed block's 2H records, in (kv, head) order, are coded
(the oracle's encode_record); a record that codes takes the block page's
next bytes if they fit, else it spills raw to the overflow pool; a record
that does not code goes raw to the pool.  Pages here are tight (room for the
dense parts and about three average variable regions) and the records'
sizes vary (per-head scale mismatch against the calibrated tables), so the
spill set depends on the order.  Checked on two fresh stores: every record's
placement (page offset or pool), the arena bytes against the oracle, the
counters, and gather bit-exactness -- the same on both runs.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests import kvgen
from tests.conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

H, D, T = 4, 128, 128
DENSE, RAW = 22528, 32768


def _case(seed, NB):
    from oracle import oracle

    rng = np.random.default_rng(seed)
    cal = kvgen.bf16_bits(rng.standard_normal((2, H, 4 * T, D)) * 0.5)
    table = np.empty((1, 2, H, 22), np.uint8)
    for kv in range(2):
        for h in range(H):
            table[0, kv, h] = oracle.calibrate_table((cal[kv, h] >> 8).astype(np.uint8))
    # per-record scale: some records escape much more than others
    scale = rng.choice([0.5, 1.0, 1.4, 2.0], size=(NB, 2, H), p=[0.35, 0.3, 0.3, 0.05])
    x = rng.standard_normal((NB, 2, T, H, D)) * scale[:, :, None, :, None]
    return table, kvgen.bf16_bits(x)  # [NB, 2, T, H, D]


def _expected(table, kv, page):
    NB = kv.shape[0]
    """Per (block, kv, head): page offset, or -1 for the pool; plus counts."""
    from oracle import oracle

    where = np.full((NB, 2, H), -1, np.int64)
    recs = {}
    spills = fallbacks = 0
    for b in range(NB):
        off = 0
        for k in range(2):
            for h in range(H):
                rec = oracle.encode_record(kv[b, k, :, h], table[0, k, h], k)
                recs[b, k, h] = rec
                if len(rec) == RAW:
                    fallbacks += 1
                elif off + len(rec) <= page:
                    where[b, k, h] = off
                    off += len(rec)
                else:
                    spills += 1
    return where, recs, spills, fallbacks


def _run(table, kv, page):
    NB = kv.shape[0]
    import torch

    from fragpack_amd.compression.attn_tables import device_tables
    from fragpack_amd.ops import hbm_kv
    from fragpack_amd.ops.hbm_kv import HbmKvStore

    arena = torch.randint(0, 256, (NB, page), dtype=torch.uint8, device="cuda")
    store = HbmKvStore([arena], H, device_tables(table, torch.device("cuda")), max_tokens=NB * T, staging_slots=1,
                       overflow_records=2 * NB * H)
    slots = torch.arange(NB * T, dtype=torch.int64, device="cuda")
    store.prepare(slots, NB * T, np.zeros(0, np.int32))
    kt = torch.from_numpy(np.ascontiguousarray(kv[:, 0]).reshape(NB * T, H, D).view(np.int16)).cuda()
    vt = torch.from_numpy(np.ascontiguousarray(kv[:, 1]).reshape(NB * T, H, D).view(np.int16)).cuda()
    store.write(0, kt.view(torch.bfloat16), vt.view(torch.bfloat16), slots)
    store.encode(0, NB, ordered=True)
    store.commit()
    torch.cuda.synchronize()
    c = store.counters.cpu().numpy()
    wk = torch.empty((NB, T, H, D), dtype=torch.bfloat16, device="cuda")
    wv = torch.empty_like(wk)
    store.gather(0, torch.arange(NB, dtype=torch.int32, device="cuda"), wk, wv)
    got = np.stack([wk.view(torch.int16).cpu().numpy(), wv.view(torch.int16).cpu().numpy()], 1).view(np.uint16)
    return (store.rec_addr[0].cpu().numpy(), store.rec_len[0].cpu().numpy(), arena.cpu().numpy(), arena.data_ptr(),
            store.overflow.data_ptr(), store.overflow.numel(),
            {k: int(c[i]) for k, i in (("encoded", hbm_kv._ENCODED), ("fallbacks", hbm_kv._FALLBACKS),
                                        ("spills", hbm_kv._SPILLS), ("err_overflow", hbm_kv._ERR_OVERFLOW))}, got)


# 24 blocks take the two-pass path, 400 the block-major one (2 x ceil(400 x 8
# records / 1024 workgroup slots) >= 8 records per block)
@pytest.mark.parametrize("seed,NB", [(1, 24), (2, 24), (3, 400)])
def test_ordered_encode_places_by_record_order(seed, NB):
    table, kv = _case(seed, NB)
    page = 2 * H * DENSE + 3 * 1280
    where, recs, spills, fallbacks = _expected(table, kv, page)
    print("ordered encode", seed, NB, "spills", spills, "fallbacks", fallbacks, flush=True)
    assert spills > 0  # the case must exercise the order
    runs = [_run(table, kv, page) for _ in range(2)]
    for addr, length, arena, abase, obase, osize, counters, got in runs:
        assert counters == {"encoded": NB * 2 * H, "fallbacks": spills + fallbacks, "spills": spills,
                            "err_overflow": 0}
        for (b, k, h), rec in recs.items():
            a = int(addr[b, k, h])
            if where[b, k, h] < 0:
                assert obase <= a < obase + osize and int(length[b, k, h]) == RAW - DENSE, (b, k, h)
            else:
                assert a - abase == b * page + int(where[b, k, h]), (b, k, h)
                assert int(length[b, k, h]) == len(rec) - DENSE
                o = a - abase
                assert arena[b].tobytes()[o - b * page : o - b * page + len(rec)] == rec, (b, k, h)
        np.testing.assert_array_equal(got.transpose(0, 1, 2, 3, 4), kv)
