"""Decode attention that appends the step's new tokens itself
(fp_fused_decode_append) against the store's write followed by decode
attention (the reference's two launches, fragpack_ext.cpp:5-23).

Two stores are filled identically from the same seeded KV; one step of
decode tokens then goes through either path.  Bar: attention outputs
bit-identical, and after the step's encode and commit every block of both
stores gathers back bit-identical to the written KV.  Cases: new tokens at
rows 0 (a freshly claimed block, a single-page unit), 31 / 32 (the K slab
boundary), 100 and 127 (the block closes and is encoded), sequences of one
to 71 pages (units of one page and units past the first 64 pages), GQA 1 and
8, a padding row (slot -1, length 0), and a table entry outside the store's
staging (left unwritten).
"""

from __future__ import annotations

import numpy as np
import pytest

from tests import workloads
from tests.conftest import gpu_available

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not gpu_available(), reason="needs a GPU"),
    pytest.mark.skip(reason="the fused append is switched off: the first GPU run of this file faulted the device "
                            "and the cause is not yet found"),
]

T, D = 128, 128


def _fill(torch, H, tables, lens, kv, pages):
    """A store whose sequence b holds tokens [0, lens[b]) of kv[:, b] in
    blocks b * pages + p; closed blocks are encoded."""
    from fragpack_amd.ops.hbm_kv import HbmKvStore, page_bytes

    B = len(lens)
    arena = torch.empty((B * pages, page_bytes(H)), dtype=torch.uint8, device="cuda")
    store = HbmKvStore([arena], H, tables, max_tokens=int(sum(lens)) + B + T, staging_slots=B, overflow_records=64)
    slots, rows = [], []
    for b, n in enumerate(lens):
        pos = np.arange(n)
        slots.append((b * pages + pos // T) * T + pos % T)
        rows.append(np.stack([np.full(n, b), pos], 1))
    slots = torch.from_numpy(np.concatenate(slots).astype(np.int64)).cuda()
    rows = torch.from_numpy(np.concatenate(rows).astype(np.int64)).cuda()
    k = kv[0][rows[:, 0], rows[:, 1]].contiguous()
    v = kv[1][rows[:, 0], rows[:, 1]].contiguous()
    store.prepare(slots, slots.numel(), np.zeros(0, np.int32))
    store.write(0, k, v, slots)
    closes = int(sum(n // T for n in lens))
    store.encode(0, closes)
    store.commit()
    return store, arena


def _run(lens, heads, group, seed, foreign_row=None):
    import torch

    from fragpack_amd.compression.attn_tables import device_tables
    from fragpack_amd.ops.fused_attn_decode import RecordTables, decode_attention, decode_units, workspace_elems

    B, H, G = len(lens), heads, group
    rng = np.random.default_rng(seed)
    scales = workloads.channel_scales(rng, H, 0.02)
    tables = device_tables(workloads.calibrated_tables(rng, H, scales), "cuda")
    gen = torch.Generator(device="cuda").manual_seed(seed)
    pages = max(1, -(-(max(lens) + 1) // T))
    kv = workloads.gen_kv(torch, gen, B * pages * T, H, torch.from_numpy(scales).float().cuda())
    kv = kv.view(2, B, pages * T, H, D)
    q = torch.randn((B, H * G, D), generator=gen, device="cuda").to(torch.bfloat16)
    lens = np.asarray(lens)
    pad = lens < 0  # padding rows: no token, length 0
    before = np.where(pad, 0, lens)
    after = np.where(pad, 0, lens + 1)
    bt = torch.from_numpy((np.arange(B)[:, None] * pages + np.arange(pages)[None]).astype(np.int32)).cuda()
    seq = torch.from_numpy(after.astype(np.int32)).cuda()
    step_slots = np.where(pad, -1, (np.arange(B) * pages + before // T) * T + before % T).astype(np.int64)
    slots_t = torch.from_numpy(step_slots).cuda()
    nk = kv[0][torch.arange(B), torch.from_numpy(before).cuda()].contiguous()  # [B, H, D]
    nv = kv[1][torch.arange(B), torch.from_numpy(before).cuda()].contiguous()
    sms = torch.cuda.get_device_properties(0).multi_processor_count
    units = decode_units(B, H, sms)
    outs, stores = [], []
    for fused in (False, True):
        store, arena = _fill(torch, H, tables, list(before), kv, pages)
        live = np.array([b * pages + before[b] // T for b in range(B) if not pad[b] and before[b] % T], np.int32)
        store.prepare(slots_t, B, live)
        tabs = RecordTables(*store.layer_tables(0))
        if foreign_row is not None:
            # the row's open block's K table entry points at a record outside
            # the store's staging: the fused write must leave it alone
            blk = int(step_slots[foreign_row]) >> 7
            foreign = torch.zeros(32768, dtype=torch.uint8, device="cuda")
            tabs.rec_addr[blk, 0, 0] = foreign.data_ptr()
        o_e, m_e, p_e = workspace_elems(H, units)
        ws = (torch.empty(o_e, device="cuda"), torch.empty(m_e, device="cuda"),
              torch.empty(p_e, dtype=torch.int32, device="cuda"))
        out = torch.full_like(q, float("nan"))
        print("append case", list(lens), H, G, "fused" if fused else "write", flush=True)
        if fused:
            decode_attention(q, tabs, bt, seq, D ** -0.5, units, out, ws, True,
                             append=(nk, nv, slots_t, store.staging, store.scratch))
        else:
            store.write(0, nk, nv, slots_t)
            decode_attention(q, tabs, bt, seq, D ** -0.5, units, out, ws, True)
        torch.cuda.synchronize()
        if foreign_row is not None:
            assert not foreign.any(), "a record outside the staging was written"
            continue
        store.encode(0, int(np.sum(after // T - before // T)))
        store.commit()
        torch.cuda.synchronize()
        outs.append(out)
        stores.append(store)
    if foreign_row is not None:
        return
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    assert torch.isfinite(outs[1].float()).all()
    blocks = torch.arange(B * pages, dtype=torch.int32, device="cuda")
    got = []
    for store in stores:
        wk = torch.empty((B * pages, T, H, D), dtype=torch.bfloat16, device="cuda")
        wv = torch.empty_like(wk)
        store.gather(0, blocks, wk, wv)
        got.append((wk.view(B, pages * T, H, D), wv.view(B, pages * T, H, D)))
    for b in range(B):
        n = int(after[b])
        for kvi in range(2):
            want = kv[kvi, b, :n].view(torch.int16)
            assert torch.equal(got[1][kvi][b, :n].view(torch.int16), want), (b, kvi)
            assert torch.equal(got[0][kvi][b, :n].view(torch.int16), want), (b, kvi)


@pytest.mark.parametrize("group", [1, 8])
def test_append_matches_write_then_attend(group):
    _run([0, 31, 32, 100, 127, 128, 255, 1000, 9000], heads=2, group=group, seed=3 + group)


def test_append_skips_padding_rows():
    _run([-1, 5, -1, 127], heads=2, group=4, seed=9)


def test_append_leaves_records_outside_the_staging_alone():
    _run([40, 300], heads=1, group=8, seed=11, foreign_row=1)
