"""Fused decode attention (HIP) vs the fp32 reference on identical inputs.

Tolerance: 2e-2 abs + 1e-2 rel (BF16 out, fp32 accumulate), the target
stated for this path; the reference's own tests use 2e-2/2e-2 and
2e-3/1e-2 (test_fragpack_hbm_store.py:215, test_fragpack_decode_schedule.py:184).
Covers GQA groups 1/2/4/8, coded + raw-tail + fallback records, ragged and
zero-length rows, unit counts from the minimum to the automatic one, and
graph replay with changed lengths.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests import kvgen
from tests.conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

ATOL, RTOL = 2e-2, 1e-2


def _check(out, ref, lens=None):
    assert np.all(np.isfinite(out))
    np.testing.assert_allclose(out, ref, atol=ATOL, rtol=RTOL)
    if lens is not None:
        assert not np.any(out[np.asarray(lens) == 0])


def test_config0_shape(tmp_path):
    """1 seq, H4, G8, 1000 tokens (7 coded pages + a
    104-token raw tail), tables from the repository's calibration CLI on a
    seeded [64, 1, 2, 128, 4, 128] dump.  The GPU batch codec reconstructs
    every record bit-exactly, and decode attention matches float64."""
    from fragpack_amd.compression import attn_page as ap

    case = kvgen.config0_case(tmp_path)
    print("config0 case built", flush=True)
    blks = case.block_table[0, :8]
    recs, kvs, tabs, want = [], [], [], []
    for blk in blks:
        for kv in range(2):
            for h in range(4):
                off = int(case.rec_off[blk, kv, h])
                recs.append(case.recs[off : off + kvgen.DENSE + int(case.rec_len[blk, kv, h])].tobytes())
                kvs.append(kv)
                tabs.append(kv * 4 + h)
                want.append(case.kv[blk, kv, :, h, :])
    back = ap.decode_records(recs, case.tables.reshape(8, 22), np.array(kvs, np.int32), np.array(tabs, np.int32))
    np.testing.assert_array_equal(back, np.stack(want))
    out = kvgen.run_gpu_decode(case)
    _check(out, kvgen.reference_attention(case))


@pytest.mark.parametrize("group", [1, 2, 4, 8])
def test_groups_ragged(group):
    lens = [0, 1, 127, 128, 129, 8 * 128 + 13, 700]
    case = kvgen.decode_case(seed=10 + group, batch=len(lens), heads=2, group=group, lens=lens, outlier=0.05)
    print("group", group, flush=True)
    out = kvgen.run_gpu_decode(case)
    _check(out, kvgen.reference_attention(case), lens)


@pytest.mark.parametrize("units_policy", ["min", "min+1", "auto"])
def test_unit_counts(units_policy):
    lens = [300, 2000, 1, 513]
    case = kvgen.decode_case(seed=21, batch=4, heads=4, group=8, lens=lens)
    B = len(lens)
    units = {"min": B, "min+1": B + 1, "auto": None}[units_policy]
    print("units", units_policy, flush=True)
    out = kvgen.run_gpu_decode(case, units=units, repeat=2)
    _check(out, kvgen.reference_attention(case), lens)


def test_all_raw_records():
    """Every record raw (the BF16 paged baseline form)."""
    case = kvgen.decode_case(seed=5, batch=2, heads=2, group=4, lens=[640, 200])
    from oracle import oracle

    chunks, off = [], 0
    for blk in range(case.kv.shape[0]):
        for k in range(2):
            for h in range(case.heads):
                r = oracle.raw_record(case.kv[blk, k, :, h, :], k)
                case.rec_off[blk, k, h] = off
                case.rec_len[blk, k, h] = len(r) - kvgen.DENSE
                chunks.append(np.frombuffer(r, np.uint8))
                off += len(r)
    case.recs = np.concatenate(chunks)
    out = kvgen.run_gpu_decode(case)
    _check(out, kvgen.reference_attention(case))


def test_heavy_tail_records():
    """Outlier-heavy KV: many escapes / raw bytes, some fallbacks."""
    case = kvgen.decode_case(seed=6, batch=2, heads=2, group=8, lens=[1024, 777], outlier=0.3)
    n_raw = int((case.rec_len > 2048).sum())
    print("raw records", n_raw, "of", case.rec_len.size, flush=True)
    out = kvgen.run_gpu_decode(case)
    _check(out, kvgen.reference_attention(case))


def test_graph_replay_changed_lengths():
    import torch

    from fragpack_amd.ops.fused_attn_decode import RecordTables, decode_attention, decode_units, workspace_elems

    base = [300, 2000, 1, 513, 0, 129]
    case = kvgen.decode_case(seed=31, batch=len(base), heads=2, group=8, lens=base)
    q, rec_addr, rec_len, plut, slut, bt, lens, arena = kvgen.upload(case)
    sms = torch.cuda.get_device_properties(q.device).multi_processor_count
    units = decode_units(len(base), 2, sms)
    opart, ml, plan = workspace_elems(2, units)
    ws = (torch.empty(opart, device=q.device), torch.empty(ml, device=q.device),
          torch.empty(plan, dtype=torch.int32, device=q.device))
    out = torch.empty_like(q)
    tabs = RecordTables(rec_addr, rec_len, plut, slut)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            decode_attention(q, tabs, bt, lens, case.scale, units, out, ws, True)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        decode_attention(q, tabs, bt, lens, case.scale, units, out, ws, True)
    for trial in ([300, 2000, 1, 513, 0, 129], [0, 0, 0, 0, 0, 0], [1, 0, 2047, 5, 129, 0], [0, 1999, 0, 0, 0, 1]):
        lt = np.array(trial, np.int32)
        lens.copy_(torch.from_numpy(lt))
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        case.lens = lt
        _check(out.float().cpu().numpy(), kvgen.reference_attention(case), lt)
    del arena


def test_planning_launch_block_table_forms():
    """Planning inside the kernel with the block table read whole into LDS
    (a small table whose storage covers batch x stride entries) and read
    from global memory (a column view at a storage offset; a table past
    1024 entries) give bit-identical outputs, equal to fp32."""
    import torch

    from fragpack_amd.ops.fused_attn_decode import RecordTables, decode_attention, decode_units, workspace_elems

    lens = [300, 2000, 1, 513, 0, 129]
    case = kvgen.decode_case(seed=41, batch=len(lens), heads=2, group=8, lens=lens)
    q, rec_addr, rec_len, plut, slut, bt, lens_t, arena = kvgen.upload(case)
    B, width = bt.shape
    units = decode_units(B, 2, torch.cuda.get_device_properties(q.device).multi_processor_count)
    tabs = RecordTables(rec_addr, rec_len, plut, slut)
    view_parent = torch.zeros((B, width + 5), dtype=torch.int32, device=q.device)
    view_parent[:, 3 : 3 + width] = bt
    wide = torch.zeros((B, 1100 // B + width), dtype=torch.int32, device=q.device)
    wide[:, :width] = bt
    outs = []
    for name, table in (("whole table in LDS", bt.contiguous()), ("offset view", view_parent[:, 3 : 3 + width]),
                        ("wide table", wide)):
        print("block table form:", name, flush=True)
        opart, ml, plan = workspace_elems(2, units)
        ws = (torch.empty(opart, device=q.device), torch.empty(ml, device=q.device),
              torch.empty(plan, dtype=torch.int32, device=q.device))
        out = torch.full_like(q, float("nan"))
        for _ in range(3):  # the first call launches the planner; later ones plan in the kernel
            decode_attention(q, tabs, table, lens_t, case.scale, units, out, ws, True)
        torch.cuda.synchronize()
        outs.append(out.clone())
    ref = kvgen.reference_attention(case)
    for out in outs:
        _check(out.float().cpu().numpy(), ref, lens)
        assert torch.equal(out.view(torch.int16), outs[0].view(torch.int16))
    del arena
