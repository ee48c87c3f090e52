"""GPU record codec vs the golden vectors and the oracle (bit-exact).

The batch encoder / decoder kernels (fp_encode_records / fp_decode_records,
the GPU form of attn_page.encode_record / decode_record) must reproduce the
reference codec's bytes for every golden record, and round-trip random and
KV-shaped records bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests import kvgen
from tests.conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]


def _golden_records(golden):
    for i, name in enumerate(golden["record_names"]):
        yield (str(name), golden[f"r{i}_raw"], golden[f"r{i}_table"], int(golden[f"r{i}_kv"]),
               golden[f"r{i}_enc"].tobytes())


def test_encode_matches_golden(golden):
    from fragpack_amd.compression import attn_page as ap

    recs = list(_golden_records(golden))
    print("golden records:", len(recs), flush=True)
    raw = np.stack([r[1] for r in recs])
    tables = np.stack([r[2] for r in recs])
    kv = np.array([r[3] for r in recs], np.int32)
    got = ap.encode_records(raw, tables, kv, np.arange(len(recs), dtype=np.int32))
    for (name, _, _, _, enc), g in zip(recs, got):
        assert len(g) == len(enc), name
        assert g == enc, name


def test_decode_matches_golden(golden):
    from fragpack_amd.compression import attn_page as ap

    recs = list(_golden_records(golden))
    tables = np.stack([r[2] for r in recs])
    kv = np.array([r[3] for r in recs], np.int32)
    got = ap.decode_records([r[4] for r in recs], tables, kv, np.arange(len(recs), dtype=np.int32))
    for (name, raw, _, _, _), g in zip(recs, got):
        assert np.array_equal(g, raw), name


@pytest.mark.parametrize("outlier", [0.02, 0.05, 0.3])
def test_random_kv_records_vs_oracle(outlier):
    from fragpack_amd.compression import attn_page as ap
    from oracle import oracle

    rng = np.random.default_rng(int(outlier * 1000))
    n = 64
    raw = kvgen.kv_bits(rng, (n, 128, 128), outlier)
    cal = kvgen.kv_bits(rng, (4, 512, 128), outlier)
    tables = np.stack([oracle.calibrate_table((cal[i] >> 8).astype(np.uint8)) for i in range(4)])
    tab_idx = rng.integers(0, 4, n).astype(np.int32)
    kv = rng.integers(0, 2, n).astype(np.int32)
    got = ap.encode_records(raw, tables, kv, tab_idx)
    want_recs, want_lens = oracle.encode_batch(raw, tables, tab_idx, kv, threads=4)
    for i in range(n):
        assert got[i] == want_recs[i, : want_lens[i]].tobytes(), i
    back = ap.decode_records(got, tables, kv, tab_idx)
    assert np.array_equal(back, raw)


def test_gpu_batch_codec_equals_host_codec():
    """The GPU batch codec and the package's host codec give the same bytes
    and both decode each other's records."""
    from fragpack_amd.compression import attn_page as ap

    rng = np.random.default_rng(0)
    cal = kvgen.kv_bits(rng, (128, 128), 0.02)
    table = ap.calibrate_table((cal >> 8).astype(np.uint8))
    recs = np.stack([kvgen.kv_bits(rng, (128, 128), 0.02) for _ in range(4)])
    recs[1, 3, 5] = 0x7F00 | (recs[1, 3, 5] & 0xFF)
    recs[3] = rng.integers(0, 1 << 16, (128, 128), dtype=np.uint16)  # falls back to raw
    kv = np.array([0, 1, 0, 1], np.int32)
    got = ap.encode_records(recs, table[None], kv, np.zeros(4, np.int32))
    for i in range(4):
        host = ap.encode_record(recs[i], table, int(kv[i]))
        assert got[i] == host, i
        assert np.array_equal(ap.decode_record(got[i], table, int(kv[i])), recs[i])
    assert len(got[3]) == ap.RAW_RECORD_BYTES
    back = ap.decode_records(got, table[None], kv, np.zeros(4, np.int32))
    assert np.array_equal(back, recs)
