"""HBM store steps (prepare / write / encode / commit) vs the oracle.

Follows the reference's store contract (tests/gpu/test_fragpack_hbm_store.py
in the reference repo): a few serving steps of a small batch through the
public API, then

* every closed block's coded records are byte-identical to the oracle's
  ``encode_record`` of the written tokens and packed disjointly in their
  block-layer page; raw records (the one incompressible "WIDE" record, and
  with a tight page the records that no longer fit) hold the written KV;
* counters: encoded / fallbacks / spills exact, no staging or overflow loss;
* gather returns the written tokens bit-exactly (zeros for a never-written
  block), decode attention over coded, raw and still-open blocks matches
  the fp32 reference for GQA 8/4/2/1;
* a request whose chunk closes its open block and opens a new tail inherits
  the closing block's staging slot;
* block blobs exported from one store install into another (same bytes,
  overflow accounting) and corrupt or foreign blobs are rejected untouched.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests import kvgen
from tests.conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

L, H, D, T = 2, 2, 128, 128
GQA = 8
HQ = H * GQA
NB = 12
SCALE = D ** -0.5
WIDE = (9, 0, 0, 1)  # (block, layer, kv, head) made incompressible
DENSE = 22528
RAW = 32768


def _bits(x):
    return kvgen.bf16_bits(x)


def _bf16(bits):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(torch.bfloat16)


def _overflow_used(store, records):
    bits = np.unpackbits(store.ovf_bits.cpu().numpy().view(np.uint8))
    return int(bits.sum()) - (bits.size - records)


class Harness:
    def __init__(self, seed: int, page: int, overflow_records: int = 16, staging_slots: int = 3):
        import torch

        from fragpack_amd.compression.attn_tables import device_tables
        from fragpack_amd.ops.hbm_kv import HbmKvStore
        from oracle import oracle

        self.rng = np.random.default_rng(seed)
        self.page = page
        cal = _bits(self.rng.standard_normal((L, 2, H, 4 * T, D)) * 0.5)
        self.table = np.empty((L, 2, H, 22), np.uint8)
        for idx in np.ndindex(L, 2, H):
            self.table[idx] = oracle.calibrate_table((cal[idx] >> 8).astype(np.uint8))
        # garbage, like an engine's uninitialised cache
        self.caches = [torch.randint(0, 256, (NB, page), dtype=torch.uint8, device="cuda") for _ in range(L)]
        self.store = HbmKvStore(self.caches, H, device_tables(self.table, torch.device("cuda")), max_tokens=1024,
                                staging_slots=staging_slots, overflow_records=overflow_records)
        self.overflow_records = overflow_records
        self.ref = np.zeros((L, 2, NB, T, H, D), np.uint16)

    def step(self, rows, live):
        """One engine step; a row is (blocks, first position, token count)."""
        import torch

        slots = [blocks[q // T] * T + q % T for blocks, start, n in rows for q in range(start, start + n)]
        n = len(slots)
        slot_t = torch.tensor(slots, dtype=torch.int64, device="cuda")
        closes = sum((st + cnt) // T - st // T for _, st, cnt in rows)
        self.store.prepare(slot_t, n, np.array(live, np.int32))
        blk, off = np.array(slots) // T, np.array(slots) % T
        for layer in range(L):
            kv = _bits(self.rng.standard_normal((2, n, H, D)) * 0.5)
            hit = blk == WIDE[0]
            if layer == WIDE[1] and hit.any():
                wide = np.exp2(self.rng.uniform(-40, 4, (int(hit.sum()), D)))
                kv[WIDE[2], hit, WIDE[3]] = _bits(wide)
            self.ref[layer, :, blk, off] = kv.transpose(1, 0, 2, 3)
            # K / V as strided slices of one fused qkv row, like a serving engine
            qkv = torch.empty(n, HQ + 2 * H, D, dtype=torch.bfloat16, device="cuda")
            qkv[:, HQ : HQ + H] = _bf16(kv[0])
            qkv[:, HQ + H :] = _bf16(kv[1])
            self.store.write(layer, qkv[:, HQ : HQ + H], qkv[:, HQ + H :], slot_t)
            self.store.encode(layer, closes)
        self.store.commit()

    def check_arena(self, blocks):
        """Closed blocks' records vs the oracle; returns (fallbacks, spills)."""
        from oracle import oracle

        addr = self.store.rec_addr.cpu().numpy()
        length = self.store.rec_len.cpu().numpy()
        overflow = self.store.overflow.cpu().numpy().reshape(-1)
        ovf_base = self.store.overflow.data_ptr()
        fallbacks = spills = 0
        for b in blocks:
            for layer in range(L):
                arena = self.caches[layer].cpu().numpy().reshape(-1)
                page = self.caches[layer].data_ptr() + b * self.page
                used = []
                for kv in range(2):
                    for h in range(H):
                        ref = self.ref[layer, kv, b, :, h]
                        table = self.table[layer, kv, h]
                        want = oracle.encode_record(ref, table, kv)
                        a = int(addr[layer, b, kv, h])
                        if ovf_base <= a < ovf_base + overflow.size:
                            got = overflow[a - ovf_base :][:RAW]
                            np.testing.assert_array_equal(oracle.decode_record(got.tobytes(), table, kv), ref)
                            assert int(length[layer, b, kv, h]) == RAW - DENSE
                            if len(want) == RAW:
                                fallbacks += 1
                                assert (b, layer, kv, h) == WIDE
                            else:
                                spills += 1
                            continue
                        n = len(want)
                        assert n < RAW, (b, layer, kv, h)
                        assert a % 16 == 0 and page <= a <= page + self.page - n
                        assert DENSE + int(length[layer, b, kv, h]) == n
                        o = a - self.caches[layer].data_ptr()
                        assert arena[o : o + n].tobytes() == want, (b, layer, kv, h)
                        used.append((a, a + n))
                used.sort()
                assert all(e <= s for (_, e), (s, _) in zip(used[:-1], used[1:]))
        return fallbacks, spills

    def check_gather(self, filled):
        import torch

        blocks = sorted(filled)
        src = torch.tensor(blocks, dtype=torch.int32, device="cuda")
        wk = torch.empty(len(blocks), T, H, D, dtype=torch.bfloat16, device="cuda")
        wv = torch.empty_like(wk)
        for layer in range(L):
            self.store.gather(layer, src, wk, wv)
            got = [x.view(torch.int16).cpu().numpy().view(np.uint16) for x in (wk, wv)]
            for i, b in enumerate(blocks):
                n = filled[b]
                for kv in range(2):
                    np.testing.assert_array_equal(got[kv][i, :n], self.ref[layer, kv, b, :n], err_msg=f"{b}")

    def check_decode(self, tables, seqs, group=GQA):
        import torch

        from fragpack_amd.ops.fused_attn_decode import RecordTables, decode_attention, decode_units, workspace_elems

        B = len(seqs)
        width = max(len(t) for t in tables)
        bt = np.zeros((B, width), np.int32)
        for i, t in enumerate(tables):
            bt[i, : len(t)] = t
        block_table = torch.from_numpy(bt).cuda()
        seq_lens = torch.tensor(seqs, dtype=torch.int32, device="cuda")
        sms = torch.cuda.get_device_properties(0).multi_processor_count
        for units in (decode_units(B, H, sms), B, B + 1):
            opart, ml, plan = workspace_elems(H, units)
            ws = (torch.empty(opart, device="cuda"), torch.empty(ml, device="cuda"),
                  torch.empty(plan, dtype=torch.int32, device="cuda"))
            for layer in range(L):
                q = torch.randn(B, H * group, D, dtype=torch.bfloat16, device="cuda")
                out = torch.empty_like(q)
                decode_attention(q, RecordTables(*self.store.layer_tables(layer)), block_table, seq_lens, SCALE,
                                 units, out, ws, layer == 0)
                kvf = _bf16(self.ref[layer]).float()  # [2, NB, T, H, D]
                ref = torch.empty(B, H * group, D, device="cuda")
                for i, (t, s) in enumerate(zip(tables, seqs)):
                    pg = torch.tensor(t, device="cuda")
                    for h in range(H):
                        k = kvf[0, pg, :, h].reshape(-1, D)[:s]
                        v = kvf[1, pg, :, h].reshape(-1, D)[:s]
                        qh = q[i, group * h : group * (h + 1)].float()
                        ref[i, group * h : group * (h + 1)] = torch.softmax(qh @ k.T * SCALE, -1) @ v
                torch.testing.assert_close(out.float(), ref, atol=2e-2, rtol=1e-2)


def _page_bytes():
    from fragpack_amd.ops.hbm_kv import page_bytes

    return page_bytes(H)


@pytest.mark.parametrize("tight", [False, True])
def test_store_steps_match_oracle(tight):
    page = 2 * H * DENSE - 16 if tight else _page_bytes()
    spills = 5 * L - 1 if tight else 0  # a tight page holds 3 of a block-layer's 4 records
    h = Harness(0, page)
    a, b, c, d = [0, 1, 4, 5], [8, 9, 10], [2], [3]
    print("prefill step", flush=True)
    h.step([(a, 0, 300), (b, 0, 256), (c, 0, 10)], a + b + c)
    h.step([(a, 300, 84), (b, 256, 1), (c, 10, 1)], a + b + c)
    import torch

    torch.cuda.synchronize()
    assert h.check_arena([0, 1, 4, 8, 9]) == (1, spills)
    # C finished: GC must free block 2's slot or D / A's claims overflow staging
    h.step([(a, 384, 1), (b, 257, 1), (d, 0, 10)], a + b + d)
    h.step([(a, 385, 1), (b, 258, 1), (d, 10, 1)], a + b + d)
    torch.cuda.synchronize()
    st = h.store.stats()
    assert st.encoded == 5 * L * 2 * H
    assert st.fallbacks == 1 + spills and st.spills == spills
    assert st.err_staging == 0 and st.err_overflow == 0
    # block 11 was never written: reads as zeros, not arena garbage
    h.check_gather({0: T, 1: T, 4: T, 5: 2, 8: T, 9: T, 10: 3, 3: 11, 11: T})
    for group in (GQA, 4, 2, 1):
        print("decode group", group, flush=True)
        h.check_decode([a, b, d, [11]], [386, 259, 11, T], group)


def test_chunk_reopening_tail_inherits_closing_slot():
    import torch

    h = Harness(1, _page_bytes(), staging_slots=2)
    a, b = [0, 1, 2], [3, 4, 5]
    h.step([(a, 0, 200), (b, 0, 200)], [])
    h.step([(a, 200, 100), (b, 200, 100)], [1, 4])
    torch.cuda.synchronize()
    assert h.store.stats().err_staging == 0
    assert h.check_arena([0, 1, 3, 4]) == (0, 0)
    h.check_gather({2: 44, 5: 44})
    h.step([(a, 300, 1), (b, 300, 1)], [2, 5])
    h.step([(a, 301, 83), (b, 301, 83)], [2, 5])
    torch.cuda.synchronize()
    st = h.store.stats()
    assert st.err_staging == 0 and st.err_overflow == 0
    assert st.encoded == 6 * L * 2 * H
    assert h.check_arena([0, 1, 2, 3, 4, 5]) == (0, 0)
    h.check_gather({b: T for b in range(6)})
    h.check_decode([a, b], [384, 384])


SRC, DST = [0, 1, 4, 8, 9], [6, 7, 2, 3, 9]


def _prefill(h):
    a, b, c = [0, 1, 4, 5], [8, 9, 10], [2]
    h.step([(a, 0, 300), (b, 0, 256), (c, 0, 10)], a + b + c)
    h.step([(a, 300, 84), (b, 256, 1), (c, 10, 1)], a + b + c)


def _export(h, blocks):
    import torch

    stride = h.store.blob_stride
    out = torch.zeros(len(blocks) * stride, dtype=torch.uint8, device="cuda")
    ids = torch.tensor(blocks, dtype=torch.int32, device="cuda")
    lengths = h.store.export_blocks(ids, out, stride).cpu().tolist()
    return out, lengths


def _import(h, src, offsets, blocks):
    import torch

    off = torch.tensor(offsets, dtype=torch.int64, device="cuda")
    ids = torch.tensor(blocks, dtype=torch.int32, device="cuda")
    return h.store.import_blocks(src, off, ids).cpu().tolist()


@pytest.mark.parametrize("tight", [False, True])
def test_blob_round_trip(tight):
    import torch

    from fragpack_amd.compression import attn_page as ap

    page = 2 * H * DENSE - 16 if tight else _page_bytes()
    spills = 5 * L - 1 if tight else 0
    src = Harness(0, page)
    _prefill(src)
    blobs, lengths = _export(src, SRC)
    stride = src.store.blob_stride
    assert stride == ap.blob_slot_bytes(L, H)
    head = ap.blob_head_bytes(L, H)
    rec_len = src.store.rec_len.cpu().numpy()
    for b, n in zip(SRC, lengths):
        body = sum(DENSE + int(v) for v in rec_len[:, b].ravel())
        assert n == -(-(head + body) // ap.BLOB_ALIGN) * ap.BLOB_ALIGN <= stride
    # blob header fields (hbm_kv.cu:496-500 layout): magic, version, L, H, bytes, digest
    hb = blobs[:64].cpu().numpy()
    assert int(hb[:4].view(np.uint32)[0]) == ap.BLOB_MAGIC
    assert tuple(hb[4:16].view(np.uint32)) == (1, L, H)
    assert int(hb[24:32].view(np.int64)[0]) == src.store.table_digest
    dst = Harness(0, page, overflow_records=32)
    for s_b, d_b in zip(SRC, DST):
        dst.ref[:, :, d_b] = src.ref[:, :, s_b]
    offsets = [i * stride for i in range(len(SRC))]
    assert _import(dst, blobs, offsets, DST) == [0] * len(DST)
    torch.cuda.synchronize()
    assert dst.check_arena(DST) == (1, spills)
    assert _overflow_used(dst.store, dst.overflow_records) == 1 + spills
    # re-importing frees the overflow records it replaces
    assert _import(dst, blobs, offsets, DST) == [0] * len(DST)
    assert _overflow_used(dst.store, dst.overflow_records) == 1 + spills
    dst.check_gather({b: T for b in DST})
    dst.check_decode([[6, 7], [2], [3, 9]], [256, 128, 256])


def test_blob_import_rejects_without_side_effects():
    import torch

    from fragpack_amd.compression import attn_page as ap

    src = Harness(0, _page_bytes())
    _prefill(src)
    blobs, _ = _export(src, [8, 9])
    stride = src.store.blob_stride
    dst = Harness(0, _page_bytes(), overflow_records=1)
    before = dst.store.rec_addr.clone(), dst.store.rec_len.clone()
    bad = blobs.clone()
    bad[0] ^= 1  # magic
    bad[stride + ap.BLOB_FIXED_BYTES] = 8  # a var length that is not a record size
    assert _import(dst, bad, [0, stride], [5, 6]) == [1, 2]
    other = Harness(1, _page_bytes())  # other calibration: other digest
    assert _import(other, blobs, [0], [5]) == [1]
    torch.cuda.synchronize()
    assert torch.equal(dst.store.rec_addr, before[0])
    assert torch.equal(dst.store.rec_len, before[1])
    # block 9's WIDE record takes the only overflow slot; a second copy finds
    # the pool full in that layer and must release what it took
    assert _import(dst, blobs, [stride], [9]) == [0]
    assert _import(dst, blobs, [stride], [10]) == [4]
    assert _overflow_used(dst.store, 1) == 1
    torch.cuda.synchronize()
    assert torch.equal(dst.store.rec_addr[WIDE[1], 10], before[0][WIDE[1], 10])


def test_store_errors_surface():
    """An exhausted overflow pool is reported (StoreError), not silent."""
    from fragpack_amd.ops.hbm_kv import StoreError

    h = Harness(0, 2 * H * DENSE - 16, overflow_records=2)
    _prefill(h)
    import torch

    torch.cuda.synchronize()
    with pytest.raises(StoreError):
        h.store.stats()
