"""The GPU store (HbmKvStore over libfragpack_hip.so) driven by a simulated
serving engine, checked against the CPU store model and the CPU oracle.

The contract is the reference's (fragpack/ops/hbm_kv.py:1-47, hbm_kv.cu):
after every ``prepare`` and ``commit`` the store's bookkeeping -- which
staging slot each block holds, the free stack, the claim / close / heir
lists and the counters -- equals ``oracle.store_model.StoreModel`` exactly
(the kernels build every list in input order, so the state is a function of
the steps); after the steps every closed block's records are the oracle
codec's bytes, placed disjointly in their page or raw in the overflow pool,
gather returns the written KV bit for bit, and decode attention over coded,
raw and open blocks matches fp32 softmax attention.  Scenarios: GC of a
finished request's slot, a tight page (spills), an incompressible record
(fallback), a chunk that closes its open block and opens a new one while
staging is full (heir inherits the donor's slot), staging and overflow
exhaustion surfacing as StoreError, and block blobs moving between stores.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle
from oracle.store_model import StoreModel
from tests import kvgen
from tests.conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

T, D = 128, 128
DENSE, RAW = 22528, 32768


def _dev_bits(bits):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(torch.bfloat16)


class SimEngine:
    """A serving engine in miniature: requests own block lists taken from a
    pool (lowest id first); each step schedules some tokens per request and
    runs prepare -> (write, encode) per layer -> commit on the GPU store and
    on the store model, keeping the written KV on the host.  ``fused``: each
    layer's write and encode go through the one-launch write_encode;
    ``ordered``: records are placed in (kv, head) order."""

    def __init__(self, seed, layers=2, heads=2, blocks=12, page=None, staging=3, overflow=16, noisy=(),
                 fused=False, ordered=False, max_tokens=1024):
        import torch

        from fragpack_amd.compression.attn_tables import calibrate, device_tables
        from fragpack_amd.ops.hbm_kv import HbmKvStore, page_bytes

        self.rng = np.random.default_rng(seed)
        self.L, self.H, self.NB = layers, heads, blocks
        self.page = page or page_bytes(heads)
        dump = kvgen.bf16_bits(self.rng.standard_normal((6, layers, 2, T, heads, D)) * 0.5)
        self.table = calibrate(dump)  # [L, 2, H, 22]
        # an engine's cache starts as garbage
        self.caches = [torch.randint(0, 256, (blocks, self.page), dtype=torch.uint8, device="cuda")
                       for _ in range(layers)]
        self.max_tokens = max_tokens
        self.store = HbmKvStore(self.caches, heads, device_tables(self.table, torch.device("cuda")),
                                max_tokens=self.max_tokens, staging_slots=staging, overflow_records=overflow)
        self.model = StoreModel(layers, blocks, heads, staging, self.store.scratch.shape[0],
                                self.store.staging.data_ptr(), self.store.scratch.data_ptr())
        self.kv = np.zeros((layers, 2, blocks, T, heads, D), np.uint16)  # written KV by block
        self.reqs: dict[str, list] = {}  # name -> [blocks, computed]
        self.pool = list(range(blocks))
        self.noisy = set(noisy)  # (block, layer, kv, head) written with values too spread to code
        self.filled: dict[int, int] = {}
        self.heirs_seen = 0
        self.fused, self.ordered = fused, ordered

    def _take(self, n):
        got = sorted(self.pool)[:n]
        for b in got:
            self.pool.remove(b)
        return got

    def finish(self, name):
        blocks, _ = self.reqs.pop(name)
        self.pool.extend(blocks)
        for b in blocks:
            self.filled.pop(b, None)

    def step(self, sched, pad=0):
        """``sched``: (request, tokens) pairs; unknown requests are admitted.
        ``pad``: slots of -1 (an engine's padding tokens) follow every
        ``pad``-th token of the GPU store's slot mapping."""
        import torch

        live = []
        for name, (blocks, computed) in self.reqs.items():
            if computed % T and computed // T < len(blocks):
                live.append(blocks[computed // T])
        slots, pos = [], []
        closes = 0
        for name, n in sched:
            blocks, computed = self.reqs.setdefault(name, [[], 0])
            need = -(-(computed + n) // T) - len(blocks)
            blocks.extend(self._take(need))
            for p in range(computed, computed + n):
                slots.append(blocks[p // T] * T + p % T)
                pos.append((blocks[p // T], p % T))
            closes += (computed + n) // T - computed // T
            self.reqs[name][1] = computed + n
        dev_slots = slots
        if pad:
            dev_slots = [x for i, sl in enumerate(slots) for x in ((sl, -1) if i % pad == 0 else (sl,))]
        real = np.array(dev_slots) >= 0
        slot_t = torch.tensor(dev_slots, dtype=torch.int64, device="cuda")
        self.store.prepare(slot_t, len(dev_slots), np.array(live, np.int32))
        self.model.prepare(slots, live)
        self.heirs_seen += len(self.model.heirs)
        self.check_bookkeeping(claims=True)
        blk = np.array([b for b, _ in pos])
        off = np.array([o for _, o in pos])
        n = len(slots)
        for layer in range(self.L):
            kv = kvgen.bf16_bits(self.rng.standard_normal((2, n, self.H, D)) * 0.5)
            for b, lyr, k, h in self.noisy:
                hit = blk == b
                if lyr == layer and hit.any():
                    # finite values over ~44 binary orders of magnitude: high bytes spread too wide to code
                    mag = np.exp2(self.rng.uniform(-40, 4, (int(hit.sum()), D)))
                    kv[k, hit, h] = kvgen.bf16_bits(mag * self.rng.choice([-1.0, 1.0], mag.shape))
            self.kv[layer, :, blk, off] = kv.transpose(1, 0, 2, 3)
            # K / V as strided views of a fused qkv row, as an engine hands them over
            qkv = torch.randn(len(dev_slots), 3 * self.H, D, device="cuda").to(torch.bfloat16)
            rows = torch.from_numpy(np.flatnonzero(real)).cuda()
            qkv[rows, self.H : 2 * self.H] = _dev_bits(kv[0])
            qkv[rows, 2 * self.H :] = _dev_bits(kv[1])
            key, value = qkv[:, self.H : 2 * self.H], qkv[:, 2 * self.H :]
            if self.fused:
                self.store.write_encode(layer, key, value, slot_t, closes, ordered=self.ordered)
            else:
                self.store.write(layer, key, value, slot_t)
                self.store.encode(layer, closes, ordered=self.ordered)
        self.store.commit()
        self.model.commit()
        self.check_bookkeeping(claims=False)
        for b, o in pos:
            self.filled[b] = max(self.filled.get(b, 0), o + 1)

    # ------------------------------------------------------------------ checks
    def check_bookkeeping(self, claims):
        st, m = self.store, self.model
        top = int(st.counters[0])
        assert np.array_equal(st.wslot.cpu().numpy(), m.wslot), "staging slot per block"
        assert st.free_stack[:top].cpu().tolist() == m.free_stack, "free stack"
        got = st.counters.cpu().numpy()
        for i in (0, 1, 2, 3, 4, 9, 10):
            assert got[i] == m.counters[i], f"counter {i}: {got[i]} vs {m.counters[i]}"
        # every persistent slot is held by one block or free, exactly once
        held = [int(w) for w in m.wslot if 0 <= w < m.staging_slots]
        assert sorted(held + m.free_stack) == list(range(m.staging_slots))
        if not claims:
            return
        cap = st.claim_list.numel() // 2
        assert st.claim_list[: len(m.claims)].cpu().tolist() == m.claims
        cl = st.close_list.cpu().numpy()
        assert [(int(cl[c]), int(cl[cap + c])) for c in range(len(m.closes))] == m.closes
        addr = st.rec_addr.cpu().numpy().reshape(self.L, self.NB, -1)
        ln = st.rec_len.cpu().numpy().reshape(self.L, self.NB, -1)
        for (layer, b, kvh), a in m.claimed_records().items():
            assert addr[layer, b, kvh] == a and ln[layer, b, kvh] == RAW - DENSE

    def check_records(self, blocks):
        """Closed blocks' records vs the oracle codec; returns (fallbacks, spills)."""
        addr = self.store.rec_addr.cpu().numpy()
        length = self.store.rec_len.cpu().numpy()
        pool = self.store.overflow.cpu().numpy().reshape(-1)
        pool0 = self.store.overflow.data_ptr()
        fallbacks = spills = 0
        for layer in range(self.L):
            arena = self.caches[layer].cpu().numpy().reshape(-1)
            base = self.caches[layer].data_ptr()
            for b in blocks:
                spans = []
                for k in range(2):
                    for h in range(self.H):
                        tok = self.kv[layer, k, b, :, h]
                        want = oracle.encode_record(tok, self.table[layer, k, h], k)
                        a = int(addr[layer, b, k, h])
                        if pool0 <= a < pool0 + pool.size:
                            assert int(length[layer, b, k, h]) == RAW - DENSE
                            assert pool[a - pool0 : a - pool0 + RAW].tobytes() == oracle.raw_record(tok, k)
                            if len(want) == RAW:
                                fallbacks += 1
                            else:
                                spills += 1
                            continue
                        assert len(want) < RAW, ("a record that does not code is not in the pool", b, layer, k, h)
                        o = a - base
                        assert o % 16 == 0 and b * self.page <= o <= (b + 1) * self.page - len(want)
                        assert DENSE + int(length[layer, b, k, h]) == len(want)
                        assert arena[o : o + len(want)].tobytes() == want, (b, layer, k, h)
                        spans.append((o, o + len(want)))
                spans.sort()
                assert all(e <= s for (_, e), (s, _) in zip(spans, spans[1:])), "records overlap in a page"
        return fallbacks, spills

    def check_gather(self, filled=None):
        import torch

        filled = dict(filled or self.filled)
        blocks = sorted(filled)
        ids = torch.tensor(blocks, dtype=torch.int32, device="cuda")
        wk = torch.empty(len(blocks), T, self.H, D, dtype=torch.bfloat16, device="cuda")
        wv = torch.empty_like(wk)
        for layer in range(self.L):
            self.store.gather(layer, ids, wk, wv)
            got = [x.view(torch.int16).cpu().numpy().view(np.uint16) for x in (wk, wv)]
            for i, b in enumerate(blocks):
                for k in range(2):
                    np.testing.assert_array_equal(got[k][i, : filled[b]], self.kv[layer, k, b, : filled[b]])

    def check_decode(self, names, group):
        import torch

        from fragpack_amd.ops.fused_attn_decode import RecordTables, decode_attention, decode_units, workspace_elems

        tables = [self.reqs[r][0] for r in names]
        lens = [self.reqs[r][1] for r in names]
        B, H = len(names), self.H
        bt = np.zeros((B, max(len(t) for t in tables)), np.int32)
        for i, t in enumerate(tables):
            bt[i, : len(t)] = t
        bt_t = torch.from_numpy(bt).cuda()
        lens_t = torch.tensor(lens, dtype=torch.int32, device="cuda")
        sms = torch.cuda.get_device_properties(0).multi_processor_count
        for units in (decode_units(B, H, sms), B):
            ws = tuple(torch.empty(n, dtype=dt, device="cuda")
                       for n, dt in zip(workspace_elems(H, units), (torch.float32, torch.float32, torch.int32)))
            for layer in range(self.L):
                q = torch.randn(B, H * group, D, device="cuda").to(torch.bfloat16)
                out = torch.empty_like(q)
                decode_attention(q, RecordTables(*self.store.layer_tables(layer)), bt_t, lens_t, D ** -0.5, units,
                                 out, ws, layer == 0)
                kvf = _dev_bits(self.kv[layer]).float()  # [2, NB, T, H, D]
                for i in range(B):
                    pg = torch.tensor(tables[i], device="cuda")
                    k = kvf[0, pg].reshape(-1, H, D)[: lens[i]]
                    v = kvf[1, pg].reshape(-1, H, D)[: lens[i]]
                    qi = q[i].float().view(H, group, D)
                    p = torch.softmax(torch.einsum("hgd,thd->hgt", qi, k) * D ** -0.5, -1)
                    ref = torch.einsum("hgt,thd->hgd", p, v).reshape(H * group, D)
                    torch.testing.assert_close(out[i].float(), ref, atol=2e-2, rtol=1e-2)


def _serve(eng):
    """Prefills of 300 / 256 / 10 tokens, then decodes; the 10-token request
    finishes and a new one is admitted (its slot must come from GC)."""
    eng.step([("a", 300), ("b", 256), ("c", 10)])
    eng.step([("a", 84), ("b", 1), ("c", 1)])
    eng.finish("c")
    eng.step([("a", 1), ("b", 1), ("d", 10)])
    eng.step([("a", 1), ("b", 1), ("d", 1)])


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("tight", [False, True])
def test_serving_steps_match_model_and_oracle(tight, fused):
    import torch

    from fragpack_amd.ops.hbm_kv import page_bytes

    H = 2
    # a tight page holds 3 of a block-layer's 4 records: one spills per block-layer
    page = 2 * H * DENSE - 16 if tight else page_bytes(H)
    eng = SimEngine(0, heads=H, page=page, noisy={(3, 0, 0, 1)}, fused=fused)
    _serve(eng)
    torch.cuda.synchronize()
    closed = [b for b, n in eng.filled.items() if n == T]
    assert len(closed) == 5
    fallbacks, spills = eng.check_records(closed)
    assert fallbacks == 1 and spills == (len(closed) * eng.L - 1 if tight else 0)
    st = eng.store.stats()
    assert st.encoded == len(closed) * eng.L * 2 * H
    assert (st.fallbacks, st.spills, st.err_staging, st.err_overflow) == (fallbacks + spills, spills, 0, 0)
    eng.check_gather()
    for group in (8, 4, 2, 1):
        print("decode group", group, flush=True)
        eng.check_decode(["a", "b", "d"], group)


@pytest.mark.parametrize("fused", [False, True])
def test_closing_chunk_hands_its_slot_to_the_new_tail(fused):
    """With every persistent slot held, a chunk that fills a request's open
    block and opens the next one stages the new tail as an heir, which takes
    the closing block's slot at commit (hbm_kv.py:24-29)."""
    import torch

    eng = SimEngine(1, staging=2, fused=fused)
    eng.step([("a", 200), ("b", 200)])
    eng.step([("a", 100), ("b", 100)])  # each closes block 1 and opens block 2
    assert eng.heirs_seen == 2
    torch.cuda.synchronize()
    assert eng.store.stats().err_staging == 0
    eng.step([("a", 1), ("b", 1)])
    eng.step([("a", 83), ("b", 83)])
    eng.step([("a", 250), ("b", 250)])  # closes a block, fills one, opens another
    torch.cuda.synchronize()
    st = eng.store.stats()
    assert (st.err_staging, st.err_overflow) == (0, 0)
    closed = sorted(b for b, n in eng.filled.items() if n == T)
    assert eng.check_records(closed) == (0, 0)
    eng.check_gather()
    eng.check_decode(["a", "b"], 8)


@pytest.mark.parametrize("fused", [False, True])
def test_staging_and_overflow_exhaustion_surface(fused):
    from fragpack_amd.ops.hbm_kv import StoreError

    eng = SimEngine(3, staging=1, fused=fused)
    eng.step([("a", 10), ("b", 10)])  # two open blocks, one slot
    with pytest.raises(StoreError, match="staging"):
        eng.store.stats()
    eng = SimEngine(3, heads=2, page=2 * 2 * DENSE - 16, overflow=2, fused=fused)
    eng.step([("a", 384)])  # 3 closed blocks x 2 layers: 6 spills, 2 slots
    with pytest.raises(StoreError, match="overflow"):
        eng.store.stats()


def _placed(eng):
    """Per layer: (rec_len, record offsets within the arena (-1 elsewhere),
    the arena bytes of the closed blocks' pages up to their fill)."""
    closed = sorted(b for b, n in eng.filled.items() if n == T)
    addr = eng.store.rec_addr.cpu().numpy()
    out = []
    for layer in range(eng.L):
        base, size = eng.caches[layer].data_ptr(), eng.caches[layer].numel()
        a = addr[layer]
        off = np.where((a >= base) & (a < base + size), a - base, -1)
        arena = eng.caches[layer].cpu().numpy()
        fill = eng.store.fill[layer].cpu().numpy()
        pages = [arena[b, : fill[b]].tobytes() for b in closed]
        out.append((eng.store.rec_len[layer].cpu().numpy(), off, pages))
    return out


def test_fused_write_encode_places_records_like_the_two_launches():
    """Ordered placement depends only on the records, so the one-launch
    write + encode must leave the same tables and arena bytes as write then
    encode, step for step -- decode steps (one token per block, some
    closing), a closing chunk with an heir, and mid-block steps."""
    import torch

    engines = [SimEngine(5, staging=2, ordered=True, fused=f) for f in (False, True)]
    # chunks closing a block and opening one with both staging slots held
    # (heirs), then decode steps, two of which close a block each
    sched = [[("a", 200), ("b", 200)], [("a", 100), ("b", 100)], [("a", 1), ("b", 1)], [("a", 82), ("b", 81)],
             [("a", 1), ("b", 1)], [("a", 1), ("b", 1)], [("a", 1), ("b", 1)]]
    for st in sched:
        for eng in engines:
            eng.step(st)
        torch.cuda.synchronize()
        got = [_placed(eng) for eng in engines]
        for (l0, o0, p0), (l1, o1, p1) in zip(*got):
            np.testing.assert_array_equal(l0, l1)
            np.testing.assert_array_equal(o0, o1)
            assert p0 == p1
        s0, s1 = (eng.store.stats() for eng in engines)
        assert s0 == s1
    assert engines[1].heirs_seen > 0
    for eng in engines:
        closed = sorted(b for b, n in eng.filled.items() if n == T)
        eng.check_records(closed)
        eng.check_gather()


# ---------------------------------------------------------------- block blobs
def _export(eng, blocks):
    import torch

    stride = eng.store.blob_stride
    out = torch.zeros(len(blocks) * stride, dtype=torch.uint8, device="cuda")
    ids = torch.tensor(blocks, dtype=torch.int32, device="cuda")
    return out, eng.store.export_blocks(ids, out, stride).cpu().tolist()


def _import(eng, src, offsets, blocks):
    import torch

    off = torch.tensor(offsets, dtype=torch.int64, device="cuda")
    ids = torch.tensor(blocks, dtype=torch.int32, device="cuda")
    return eng.store.import_blocks(src, off, ids).cpu().tolist()


def _overflow_in_use(eng):
    bits = np.unpackbits(eng.store.ovf_bits.cpu().numpy().view(np.uint8))
    return int(bits.sum()) - (bits.size - eng.store.overflow.shape[0])


@pytest.mark.parametrize("tight", [False, True])
def test_blobs_move_closed_blocks_between_stores(tight):
    import torch

    from fragpack_amd.compression import attn_page as ap
    from fragpack_amd.ops.hbm_kv import page_bytes

    H = 2
    page = 2 * H * DENSE - 16 if tight else page_bytes(H)
    src = SimEngine(0, heads=H, page=page, noisy={(3, 0, 0, 1)})
    _serve(src)
    closed = sorted(b for b, n in src.filled.items() if n == T)
    blobs, lengths = _export(src, closed)
    stride = src.store.blob_stride
    assert stride == ap.blob_slot_bytes(src.L, H)
    head = ap.blob_head_bytes(src.L, H)
    rec_len = src.store.rec_len.cpu().numpy()
    for b, n in zip(closed, lengths):
        body = sum(DENSE + int(v) for v in rec_len[:, b].ravel())
        assert n == -(-(head + body) // ap.BLOB_ALIGN) * ap.BLOB_ALIGN <= stride
    hdr = blobs[:64].cpu().numpy()
    assert int(hdr[:4].view(np.uint32)[0]) == ap.BLOB_MAGIC
    assert tuple(hdr[4:16].view(np.uint32)) == (1, src.L, H)
    assert int(hdr[24:32].view(np.int64)[0]) == src.store.table_digest
    # same seed: same calibration, so the destination accepts the digest
    dst = SimEngine(0, heads=H, page=page, overflow=32)
    targets = [11, 10, 9, 7, 6][: len(closed)]
    for s_b, d_b in zip(closed, targets):
        dst.kv[:, :, d_b] = src.kv[:, :, s_b]
    offsets = [i * stride for i in range(len(closed))]
    assert _import(dst, blobs, offsets, targets) == [0] * len(targets)
    torch.cuda.synchronize()
    fallbacks, spills = dst.check_records(targets)
    assert fallbacks == 1 and _overflow_in_use(dst) == fallbacks + spills
    assert _import(dst, blobs, offsets, targets) == [0] * len(targets)  # frees what it replaces
    assert _overflow_in_use(dst) == fallbacks + spills
    dst.check_gather({b: T for b in targets})


def test_blob_import_rejects_bad_blobs_untouched():
    import torch

    from fragpack_amd.compression import attn_page as ap

    src = SimEngine(0, noisy={(3, 0, 0, 1)})
    _serve(src)
    blobs, _ = _export(src, [3, 4])
    stride = src.store.blob_stride
    dst = SimEngine(0, overflow=1)
    before = dst.store.rec_addr.clone(), dst.store.rec_len.clone()
    bad = blobs.clone()
    bad[0] ^= 1  # magic
    bad[stride + ap.BLOB_FIXED_BYTES] = 8  # a length that is no record size
    assert _import(dst, bad, [0, stride], [5, 6]) == [1, 2]
    assert _import(SimEngine(1), blobs, [0], [5]) == [1]  # other tables: other digest
    torch.cuda.synchronize()
    assert torch.equal(dst.store.rec_addr, before[0]) and torch.equal(dst.store.rec_len, before[1])
    # block 3's incompressible record takes the only overflow slot; a second
    # copy finds the pool full and must release what it took
    assert _import(dst, blobs, [0], [9]) == [0]
    assert _import(dst, blobs, [0], [10]) == [4]
    assert _overflow_in_use(dst) == 1
    assert torch.equal(dst.store.rec_addr[0, 10], before[0][0, 10])


def test_blob_import_partial_overflow_claim_is_returned():
    """A layer needing two overflow slots finds one: the slot it won goes back
    to the pool and that layer's tables stay as they were, while the blob's
    other layer (coded records only) installs; the export's header words past
    the digest are zero."""
    import torch

    src = SimEngine(0, noisy={(3, 0, 0, 1), (3, 0, 1, 0)})
    _serve(src)
    blobs, _ = _export(src, [3])
    assert not blobs[32:64].any()
    dst = SimEngine(0, overflow=1)
    before = dst.store.rec_addr.clone(), dst.store.rec_len.clone()
    assert _import(dst, blobs, [0], [8]) == [4]
    torch.cuda.synchronize()
    assert _overflow_in_use(dst) == 0
    assert torch.equal(dst.store.rec_addr[0, 8], before[0][0, 8]) and torch.equal(dst.store.rec_len[0, 8], before[1][0, 8])
    assert torch.equal(dst.store.rec_len[1, 8], src.store.rec_len[1, 3])
    ids = torch.tensor([8], dtype=torch.int32, device="cuda")
    wk = torch.empty(1, T, dst.H, D, dtype=torch.bfloat16, device="cuda")
    wv = torch.empty_like(wk)
    dst.store.gather(1, ids, wk, wv)
    for k, x in enumerate((wk, wv)):
        np.testing.assert_array_equal(x.view(torch.int16).cpu().numpy().view(np.uint16)[0], src.kv[1, k, 3])


def test_fused_write_encode_degenerate_steps():
    """write_encode with nothing to close (the write alone), with no tokens
    (the encode alone) and with padding slots (-1) leaves the same records
    and counters as the separate calls on a twin store."""
    import torch

    from fragpack_amd.compression.attn_tables import device_tables
    from fragpack_amd.ops.hbm_kv import HbmKvStore, page_bytes

    H, NB = 2, 6
    rng = np.random.default_rng(77)
    dump = kvgen.bf16_bits(rng.standard_normal((4, 1, 2, T, H, D)) * 0.5)
    from fragpack_amd.compression.attn_tables import calibrate

    tables = device_tables(calibrate(dump), torch.device("cuda"))

    def twin():
        arena = torch.zeros((NB, page_bytes(H)), dtype=torch.uint8, device="cuda")
        return HbmKvStore([arena], H, tables, max_tokens=512, staging_slots=2, overflow_records=8), arena

    (a, arena_a), (b, arena_b) = twin(), twin()
    kv = torch.from_numpy(kvgen.bf16_bits(rng.standard_normal((2, 3 * T, H, D)) * 0.5).view(np.int16)).cuda()
    kv = kv.view(torch.bfloat16)
    # step 1: block 0 rows 0..99 and block 1 rows 0..4 (nothing closes), with padding
    slots = torch.tensor([-1] + list(range(100)) + [128 + r for r in range(5)] + [-1], dtype=torch.int64,
                         device="cuda")
    k, v = kv[0, : slots.numel()], kv[1, : slots.numel()]
    for st in (a, b):
        st.prepare(slots, slots.numel(), np.zeros(0, np.int32))
    a.write(0, k, v, slots)
    a.encode(0, 0)
    b.write_encode(0, k, v, slots, 0)
    for st in (a, b):
        st.commit()
    # step 2: block 0 rows 100..127 close it; block 1 row 5 stays open
    slots2 = torch.tensor(list(range(100, 128)) + [133, -1], dtype=torch.int64, device="cuda")
    k2, v2 = kv[0, 200 : 200 + slots2.numel()], kv[1, 200 : 200 + slots2.numel()]
    live = np.array([0, 1], np.int32)
    for st in (a, b):
        st.prepare(slots2, slots2.numel(), live)
    a.write(0, k2, v2, slots2)
    a.encode(0, 2)
    b.write_encode(0, k2, v2, slots2, 2)
    # step 3: no tokens; the fused call only encodes (nothing is left to close)
    for st in (a, b):
        st.commit()
        st.prepare(torch.empty(0, dtype=torch.int64, device="cuda"), 0, np.array([1], np.int32))
    a.encode(0, 1)
    b.write_encode(0, kv[0, :0], kv[1, :0], torch.empty(0, dtype=torch.int64, device="cuda"), 1)
    for st in (a, b):
        st.commit()
    torch.cuda.synchronize()
    assert a.stats() == b.stats() and a.stats().encoded == 2 * H
    ids = torch.arange(2, dtype=torch.int32, device="cuda")
    got = []
    for st in (a, b):
        wk = torch.empty((2, T, H, D), dtype=torch.bfloat16, device="cuda")
        wv = torch.empty_like(wk)
        st.gather(0, ids, wk, wv)
        got.append((wk.view(torch.int16).clone(), wv.view(torch.int16).clone()))
    want_k = torch.cat((kv[0, 1:101], kv[0, 200:228]))  # block 0: step 1 rows 0..99, step 2 rows 100..127
    assert torch.equal(got[1][0][0], want_k.view(torch.int16))
    assert torch.equal(got[0][0][:, :6], got[1][0][:, :6]) and torch.equal(got[0][1][:, :6], got[1][1][:, :6])
    assert torch.equal(got[0][0][0], got[1][0][0]) and torch.equal(got[0][1][0], got[1][1][0])
    # block 1: rows 0..4 from step 1, row 5 from step 2
    want_k1 = torch.cat((kv[0, 101:106], kv[0, 228:229]))
    assert torch.equal(got[1][0][1, :6], want_k1.view(torch.int16))


@pytest.mark.parametrize("heads", [8, 2])
def test_large_step_writes_batched_items(heads):
    """Steps of 16,384+ (token, head) items take the write's slab path:
    whole 16-token slabs leave as 16-byte chunks, the rest per token.  The
    first step's padding slots (-1 after every 37th token) leave slabs
    partly written; the second step's decodes put the prompt's tokens at
    odd step offsets.  Records vs the oracle, open blocks' rows through a
    gather, bookkeeping vs the store model."""
    k = 8 // heads  # the same number of (token, head) items at either head count
    eng = SimEngine(7, layers=1, heads=heads, blocks=48 * k, staging=6, overflow=64 * k, max_tokens=4096 * k)
    eng.step([("a", 1100 * k), ("b", 935 * k), ("c", 300 * k)], pad=37)
    eng.step([("a", 1), ("b", 1), ("c", 2000 * k)])
    closed = [b for b, f in eng.filled.items() if f == T]
    assert len(closed) >= 20
    eng.check_records(closed)
    eng.check_gather()


@pytest.mark.parametrize("fused", [False, True])
def test_random_serving_steps(fused):
    """Forty random serving steps: requests arrive with prompts of 2..4000
    tokens, prefill in chunks of up to 3000 tokens, then decode one token a
    step and finish at random; some steps carry padding slots, and steps of
    4096+ tokens take the slab write (or, fused, the one-launch write +
    encode at that size).  Bookkeeping equals the store model
    after every prepare and commit; at the end every closed block's records
    equal the oracle codec's and every written row gathers back."""
    import torch

    rng = np.random.default_rng(1234 + fused)
    eng = SimEngine(41, layers=1, heads=4, blocks=240, staging=8, overflow=256, fused=fused, max_tokens=8192)
    prompt: dict[str, int] = {}  # request -> prompt tokens not yet scheduled
    admitted, large_steps = 0, 0
    for step in range(40):
        while len(prompt) < 6 and rng.random() < 0.7:
            prompt[f"r{admitted}"] = int(rng.integers(2, 4000))
            admitted += 1
        free = len(eng.pool)
        sched, tokens = [], 0
        for name, rem in prompt.items():
            blocks, computed = eng.reqs.get(name, [[], 0])
            n = min(rem, int(rng.integers(1, 3000)), 7500 - tokens) if rem else 1
            n = max(n, 0)
            while n > 0 and -(-(computed + n) // T) - len(blocks) > free:
                n //= 2
            if n == 0:
                continue
            free -= -(-(computed + n) // T) - len(blocks)
            sched.append((name, n))
            tokens += n
        if not sched:
            continue
        large_steps += tokens * eng.H >= 1 << 14
        eng.step(sched, pad=int(rng.integers(20, 60)) if rng.random() < 0.3 else 0)
        for name, n in sched:
            prompt[name] = max(prompt[name] - n, 0) if prompt[name] else 0
        for name in [r for r, rem in prompt.items() if rem == 0 and r in eng.reqs and rng.random() < 0.25]:
            eng.finish(name)
            del prompt[name]
    assert large_steps >= 3
    torch.cuda.synchronize()
    st = eng.store.stats()
    assert (st.err_staging, st.err_overflow) == (0, 0)
    closed = sorted(b for b, n in eng.filled.items() if n == T)
    eng.check_records(closed)
    eng.check_gather()


def test_encode_dynamic_tail_across_launches():
    """A claim-mode encode of at least eight rounds per workgroup hands its
    last records out from a cursor that the launch's last workgroup resets:
    two layers of 1024 closed blocks (H 8: 16 rounds over MI355X's 1024
    encode workgroups) encoded one launch after the other both place every
    record (none left pointing at staging), the counts add up, both tail
    counters read zero after each launch, and every record gathers back
    bit for bit."""
    import torch

    from fragpack_amd.compression.attn_tables import device_tables
    from fragpack_amd.ops import hbm_kv
    from fragpack_amd.ops.hbm_kv import HbmKvStore, page_bytes
    from tests import workloads

    H, n, L = 8, 1024, 2
    rng = np.random.default_rng(77)
    scales = workloads.channel_scales(rng, H, 0.02)
    tables = np.repeat(workloads.calibrated_tables(rng, H, scales), L, axis=0)
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(77)
    scales_t = torch.from_numpy(scales).float().to(dev)
    arenas = [torch.empty((n, page_bytes(H)), dtype=torch.uint8, device=dev) for _ in range(L)]
    store = HbmKvStore(arenas, H, device_tables(tables, dev), max_tokens=n * T, staging_slots=1,
                       overflow_records=8192)
    slots = torch.arange(n * T, device=dev, dtype=torch.int64)
    store.prepare(slots, slots.numel(), np.zeros(0, np.int32))
    # blocks closing in their own step hold transient slots of one layer's
    # size: each layer is written and encoded in turn, as a forward does
    held = [(t.data_ptr(), t.data_ptr() + t.numel()) for t in (store.staging, store.scratch)]
    for layer in range(L):
        kv = workloads.gen_kv(torch, gen, n * T, H, scales_t)
        store.write(layer, kv[0], kv[1], slots)
        store.encode(layer, n)
        torch.cuda.synchronize()
        c = store.counters.cpu().numpy()
        print("layer", layer, "counters", c.tolist(), flush=True)
        assert int(c[hbm_kv._ENCODED]) == (layer + 1) * n * 2 * H
        assert int(c[11]) == 0 and int(c[12]) == 0, "the tail cursor is reset for the next launch"
        addr = store.rec_addr[layer].cpu().numpy()
        for lo, hi in held:
            assert not np.any((addr >= lo) & (addr < hi)), "a record was left in staging"
        blocks = torch.arange(n, dtype=torch.int32, device=dev)
        wk = torch.empty((n, T, H, D), dtype=torch.bfloat16, device=dev)
        wv = torch.empty_like(wk)
        store.gather(layer, blocks, wk, wv)
        ref = kv.view(2, n, T, H, D)
        assert torch.equal(wk.view(torch.int16), ref[0].view(torch.int16))
        assert torch.equal(wv.view(torch.int16), ref[1].view(torch.int16))


@pytest.mark.parametrize("read_bytes,write_bytes,wg", [(32768, 17408, 4), (32768, 0, 8), (4096, 4096, 1)])
def test_stream_probe_copies_the_written_prefix(read_bytes, write_bytes, wg):
    """The bench's streaming probe: each 32 KB record's first ``write_bytes``
    reach dst unchanged; the rest of dst is untouched."""
    import torch

    from fragpack_amd.ops.fragpack_ext import extension

    n = 37  # fewer records than workgroups, and not a multiple of the grid
    gen = torch.Generator(device="cuda").manual_seed(5)
    src = torch.randint(0, 256, (n * 32768,), generator=gen, device="cuda", dtype=torch.uint8)
    dst = torch.full_like(src, 0xA5)
    print("probe", read_bytes, write_bytes, wg, flush=True)
    extension().stream_probe(src, dst, read_bytes, write_bytes, wg)
    torch.cuda.synchronize()
    s, d = src.view(n, 32768), dst.view(n, 32768)
    assert torch.equal(d[:, :write_bytes], s[:, :write_bytes])
    assert bool((d[:, write_bytes:] == 0xA5).all())
    with pytest.raises(RuntimeError, match="write <= read"):
        extension().stream_probe(src, dst, 4096, 8192, wg)
