"""Decode scheduling contracts for ragged and graph-padded batches.

Mirrors the reference's tests/gpu/test_fragpack_decode_schedule.py: three
physical pages of two layers are encoded through the store and repeated in
block tables, so contexts up to 1024 pages need no large KV allocation.  The
fp32 reference folds identical token copies into multiplicities
(``n * exp(l) == exp(l + log n)``).  Tolerance 2e-3 abs + 1e-2 rel, the
reference's own for this test.  In addition the device work plan (the
``plan`` workspace) must equal the oracle's restatement of the reference
planner, entry for entry, including for a batch too large for the planner's
LDS table.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle
from tests.conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

LAYERS, HEADS, BLOCKS = 2, 4, 3
TOKENS, DIM, GQA = 128, 128, 8
MAX_PAGES = 1024
SCALE = DIM ** -0.5


@pytest.fixture(scope="module")
def encoded_store():
    import torch

    from fragpack_amd.compression.attn_tables import calibrate, device_tables
    from fragpack_amd.ops.hbm_kv import HbmKvStore, page_bytes

    generator = torch.Generator().manual_seed(231)
    source = torch.randn(LAYERS, 2, BLOCKS, TOKENS, HEADS, DIM, generator=generator).mul_(0.5)
    # distinct page means make a missing or misassigned page visible
    source[:, 1] += torch.arange(BLOCKS)[None, :, None, None, None] - 1
    source = source.to(torch.bfloat16)
    bits = source.view(torch.int16).numpy().view(np.uint16)
    table = calibrate(bits.transpose(2, 0, 1, 3, 4, 5))
    dev = torch.device("cuda", torch.cuda.current_device())
    arenas = [torch.empty(BLOCKS, page_bytes(HEADS), dtype=torch.uint8, device=dev) for _ in range(LAYERS)]
    store = HbmKvStore(arenas, HEADS, device_tables(table, dev), max_tokens=BLOCKS * TOKENS, staging_slots=1,
                       overflow_records=LAYERS * BLOCKS * 2 * HEADS)
    source = source.to(dev)
    slots = torch.arange(BLOCKS * TOKENS, dtype=torch.int64, device=dev)
    store.prepare(slots, slots.numel(), np.arange(BLOCKS, dtype=np.int32))
    for layer in range(LAYERS):
        key, value = source[layer].reshape(2, BLOCKS * TOKENS, HEADS, DIM)
        store.write(layer, key, value, slots)
        store.encode(layer, BLOCKS)
    store.commit()
    stats = store.stats()
    assert stats.err_staging == 0 and stats.err_overflow == 0
    assert stats.encoded > stats.fallbacks
    print("schedule store encoded", stats, flush=True)
    return store, arenas, source


def _block_table(batch):
    return ((np.arange(batch)[:, None] + np.arange(MAX_PAGES)[None, :]) % BLOCKS).astype(np.int32)


def _ragged_lengths(batch):
    lengths = np.resize(np.array([1, TOKENS - 1, TOKENS, TOKENS + 1, 8 * TOKENS + 13], np.int32), batch)
    lengths[1::7] = 0
    lengths[0] = 63 * TOKENS + 1
    lengths[-1] = MAX_PAGES * TOKENS - 1
    return lengths


def _workspace(units, dev):
    import torch

    from fragpack_amd.ops.fused_attn_decode import workspace_elems

    opart, ml, plan = workspace_elems(HEADS, units)
    return (torch.empty(opart, dtype=torch.float32, device=dev), torch.empty(ml, dtype=torch.float32, device=dev),
            torch.empty(plan, dtype=torch.int32, device=dev))


def _reference(q, source, block_table, lengths):
    import torch

    counts = np.zeros((len(lengths), BLOCKS, TOKENS), np.float32)
    for row, length in enumerate(lengths):
        full, tail = divmod(int(length), TOKENS)
        counts[row] = np.bincount(block_table[row, :full], minlength=BLOCKS)[:, None]
        if tail:
            counts[row, block_table[row, full], :tail] += 1
    mult = torch.from_numpy(counts.reshape(len(lengths), -1)).to(q.device)
    key, value = source.permute(0, 3, 1, 2, 4).reshape(2, HEADS, BLOCKS * TOKENS, DIM).float()
    group = q.shape[1] // HEADS
    query = q.reshape(len(lengths), HEADS, group, DIM).float()
    logits = torch.einsum("bhgd,htd->bhgt", query, key) * SCALE
    logits += mult.log()[:, None, None, :]
    padding = torch.from_numpy(lengths == 0).to(q.device)
    logits[padding] = 0
    ref = torch.einsum("bhgt,htd->bhgd", logits.softmax(-1), value)
    ref[padding] = 0
    return ref.reshape_as(q)


def _decode_layers(store, queries, outputs, block_table, lengths, units, workspace):
    from fragpack_amd.ops.fused_attn_decode import RecordTables, decode_attention

    for layer in range(LAYERS):
        decode_attention(queries[layer], RecordTables(*store.layer_tables(layer)), block_table, lengths, SCALE, units,
                         outputs[layer], workspace, replan=layer == 0)


def _check_outputs(queries, outputs, source, block_table, lengths):
    import torch

    padding = torch.from_numpy(lengths == 0).to(source.device)
    for layer in range(LAYERS):
        ref = _reference(queries[layer], source[layer], block_table, lengths)
        torch.testing.assert_close(outputs[layer].float(), ref, atol=2e-3, rtol=1e-2)
        assert torch.count_nonzero(outputs[layer][padding]).item() == 0


def _check_plan(plan, lengths, units):
    import torch

    from fragpack_amd.ops.fused_attn_decode import UNITS_PER_CU

    slots = UNITS_PER_CU * torch.cuda.get_device_properties(plan.device).multi_processor_count
    ppc, used, unit_map, seq_map = oracle.decode_plan(lengths, units, HEADS, slots)
    got = plan.cpu().numpy()
    assert (int(got[0]), int(got[1])) == (ppc, used)
    umap = got[2 : 2 + 2 * units].reshape(units, 2).copy()
    umap[umap[:, 0] < 0, 1] = 0  # an idle unit's page entry is unspecified
    np.testing.assert_array_equal(umap, unit_map)
    np.testing.assert_array_equal(got[2 + 2 * units : 2 + 2 * units + 2 * len(lengths)].reshape(-1, 2), seq_map)


@pytest.mark.parametrize("batch_case", ["below_wave", "at_wave", "above_wave", "tiled"])
def test_ragged_batches_match_fp32_attention(encoded_store, batch_case):
    import torch

    from fragpack_amd.ops.fused_attn_decode import decode_units

    store, _arenas, source = encoded_store
    sms = torch.cuda.get_device_properties(source.device).multi_processor_count
    wave = max(1, 2 * sms // HEADS)
    batch = {"below_wave": max(1, wave - 1), "at_wave": wave, "above_wave": wave + 1,
             "tiled": max(269, wave + 1)}[batch_case]
    print("schedule batch", batch_case, batch, flush=True)
    table = _block_table(batch)
    lengths = _ragged_lengths(batch)
    units = decode_units(batch, HEADS, sms)
    gen = torch.Generator(device=source.device).manual_seed(325 + batch)
    queries = [torch.randn(batch, HEADS * GQA, DIM, dtype=torch.bfloat16, device=source.device, generator=gen)
               for _ in range(LAYERS)]
    outputs = [torch.full_like(q, float("nan")) for q in queries]
    ws = _workspace(units, source.device)
    _decode_layers(store, queries, outputs, torch.from_numpy(table).to(source.device),
                   torch.from_numpy(lengths).to(source.device), units, ws)
    _check_outputs(queries, outputs, source, table, lengths)
    _check_plan(ws[2], lengths, units)


@pytest.mark.parametrize("units_policy", ["auto", "minimum"])
@pytest.mark.parametrize("group", [1, 2, 4, GQA])
def test_graph_replans_padding_and_reuses_plan_across_layers(encoded_store, units_policy, group):
    import torch

    from fragpack_amd.ops.fused_attn_decode import decode_units

    store, _arenas, source = encoded_store
    print("schedule graph", units_policy, group, flush=True)
    batch = 269
    table = _block_table(batch)
    initial = _ragged_lengths(batch)
    changed = np.roll(initial, 17)
    changed[0] = changed[256] = 0
    changed[257] = MAX_PAGES * TOKENS - 11
    empty = np.zeros(batch, np.int32)
    sparse = empty.copy()
    sparse[[0, 256, batch - 1]] = [1, TOKENS + 1, MAX_PAGES * TOKENS - 17]
    dev_table = torch.from_numpy(table).to(source.device)
    dev_lengths = torch.from_numpy(initial).to(source.device)
    sms = torch.cuda.get_device_properties(source.device).multi_processor_count
    units = decode_units(batch, HEADS, sms) if units_policy == "auto" else batch
    ws = _workspace(units, source.device)
    gen = torch.Generator(device=source.device).manual_seed(401)
    queries = [torch.randn(batch, HEADS * group, DIM, dtype=torch.bfloat16, device=source.device, generator=gen)
               for _ in range(LAYERS)]
    outputs = [torch.full_like(q, float("nan")) for q in queries]
    args = store, queries, outputs, dev_table, dev_lengths, units, ws
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            _decode_layers(*args)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        _decode_layers(*args)
    for lengths in (initial, changed, empty, sparse):
        dev_lengths.copy_(torch.from_numpy(lengths))
        for out in outputs:
            out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        _check_outputs(queries, outputs, source, table, lengths)
        _check_plan(ws[2], lengths, units)


def test_plan_beyond_lds_table(encoded_store):
    """9000 short rows: the planner locates sequences through the plan in
    global memory instead of its LDS table."""
    import torch

    from fragpack_amd.ops.fused_attn_decode import decode_units

    store, _arenas, source = encoded_store
    batch = 9000
    rng = np.random.default_rng(9)
    lengths = rng.integers(0, 3 * TOKENS, batch).astype(np.int32)
    lengths[::5] = 0
    table = _block_table(batch)[:, :4].copy()
    sms = torch.cuda.get_device_properties(source.device).multi_processor_count
    units = decode_units(batch, HEADS, sms)
    print("schedule beyond lds", batch, units, flush=True)
    gen = torch.Generator(device=source.device).manual_seed(77)
    queries = [torch.randn(batch, HEADS * GQA, DIM, dtype=torch.bfloat16, device=source.device, generator=gen)
               for _ in range(LAYERS)]
    outputs = [torch.full_like(q, float("nan")) for q in queries]
    ws = _workspace(units, source.device)
    _decode_layers(store, queries, outputs, torch.from_numpy(table).to(source.device),
                   torch.from_numpy(lengths).to(source.device), units, ws)
    torch.cuda.synchronize()
    _check_plan(ws[2], lengths, units)
    _check_outputs(queries, outputs, source, table, lengths)


@pytest.mark.parametrize("group", [1, GQA])
def test_small_batch_plans_inside_the_attention_kernel(encoded_store, group):
    """Batches of at most 64 rows replan inside the attention kernel once the
    workspace's merge counters are known to be zero (after its first call).
    Successive calls with changed lengths, then a captured graph replayed
    over new lengths: outputs match fp32 attention and the plan words match
    the planner restatement every time."""
    import torch

    from fragpack_amd.ops.fused_attn_decode import decode_units

    store, _arenas, source = encoded_store
    batch = 40
    print("schedule inline plan", batch, group, flush=True)
    table = _block_table(batch)
    rng = np.random.default_rng(40 + group)
    sms = torch.cuda.get_device_properties(source.device).multi_processor_count
    units = decode_units(batch, HEADS, sms)
    ws = _workspace(units, source.device)
    dev_table = torch.from_numpy(table).to(source.device)
    gen = torch.Generator(device=source.device).manual_seed(4040 + group)
    queries = [torch.randn(batch, HEADS * group, DIM, dtype=torch.bfloat16, device=source.device, generator=gen)
               for _ in range(LAYERS)]
    outputs = [torch.full_like(q, float("nan")) for q in queries]
    cases = [_ragged_lengths(batch), rng.integers(0, 200 * TOKENS, batch).astype(np.int32),
             np.zeros(batch, np.int32), np.full(batch, 9 * TOKENS + 5, np.int32)]
    cases[1][::3] = 0
    dev_lengths = torch.from_numpy(cases[0]).to(source.device)
    for lengths in cases:
        dev_lengths.copy_(torch.from_numpy(lengths))
        for out in outputs:
            out.fill_(float("nan"))
        _decode_layers(store, queries, outputs, dev_table, dev_lengths, units, ws)
        torch.cuda.synchronize()
        _check_outputs(queries, outputs, source, table, lengths)
        _check_plan(ws[2], lengths, units)
    assert getattr(ws[2], "_fp_counters_zeroed", False)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        _decode_layers(store, queries, outputs, dev_table, dev_lengths, units, ws)
    for lengths in reversed(cases):
        dev_lengths.copy_(torch.from_numpy(lengths))
        for out in outputs:
            out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        _check_outputs(queries, outputs, source, table, lengths)
        _check_plan(ws[2], lengths, units)


def test_one_workspace_serves_steps_of_changing_batch(encoded_store):
    """A serving engine sizes one workspace for its largest batch and then
    decodes steps whose batch, and so unit count and plan layout, changes
    from step to step (first layer replans, the others reuse).  The merge
    counters sit at a place that does not move with the unit count, so every
    step's outputs match fp32 attention, inline planning included."""
    import torch

    from fragpack_amd.ops.fused_attn_decode import decode_units

    store, _arenas, source = encoded_store
    sms = torch.cuda.get_device_properties(source.device).multi_processor_count
    ws = _workspace(decode_units(96, HEADS, sms), source.device)  # batches above 64 use the planner launch
    gen = torch.Generator(device=source.device).manual_seed(77)
    rng = np.random.default_rng(77)
    for batch in (3, 2, 5, 64, 1, 40, 2, 80, 3):
        print("schedule batch", batch, flush=True)
        units = decode_units(batch, HEADS, sms)
        table = _block_table(batch)
        lengths = rng.integers(1, 20 * TOKENS, batch).astype(np.int32)
        queries = [torch.randn(batch, HEADS * 4, DIM, dtype=torch.bfloat16, device=source.device, generator=gen)
                   for _ in range(LAYERS)]
        outputs = [torch.full_like(q, float("nan")) for q in queries]
        _decode_layers(store, queries, outputs, torch.from_numpy(table).to(source.device),
                       torch.from_numpy(lengths).to(source.device), units, ws)
        torch.cuda.synchronize()
        _check_outputs(queries, outputs, source, table, lengths)
