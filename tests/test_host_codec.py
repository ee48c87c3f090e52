"""The package's host codec (fragpack_amd.compression.attn_page
encode_record / decode_record, numpy, no GPU) against the reference codec's
own bytes (tests/golden/codec_golden.npz) and against the CPU oracle on
seeded KV records, including heavy tails that force escapes, raw bytes and
fallbacks (reference: attn_page.py:146-269, tests/unit/test_attn_page.py).
"""

from __future__ import annotations

import numpy as np
import pytest

from fragpack_amd.compression import attn_page as ap
from oracle import oracle
from tests import kvgen


def _records(golden):
    for i, name in enumerate(golden["record_names"]):
        yield (str(name), golden[f"r{i}_raw"], golden[f"r{i}_table"], int(golden[f"r{i}_kv"]),
               golden[f"r{i}_enc"].tobytes())


def test_host_encode_matches_golden_bytes(golden):
    for name, raw, table, kv, enc in _records(golden):
        assert ap.encode_record(raw, table, kv) == enc, name


def test_host_decode_matches_golden(golden):
    for name, raw, table, kv, enc in _records(golden):
        got = ap.decode_record(enc, table, kv)
        assert got.dtype == np.uint16 and got.shape == (128, 128)
        assert np.array_equal(got, raw), name


@pytest.mark.parametrize("heavy", [0.0, 0.01, 0.05, 0.3])
def test_host_codec_vs_oracle(heavy):
    rng = np.random.default_rng(int(heavy * 1000) + 7)
    cal = kvgen.kv_bits(rng, (512, 128), 0.02)
    table = ap.calibrate_table((cal >> 8).astype(np.uint8))
    for trial in range(6):
        rec = kvgen.kv_bits(rng, (128, 128), 0.02)
        pick = rng.random(rec.shape) < heavy
        wild = rng.integers(0, 1 << 16, rec.shape, dtype=np.uint16)
        rec = np.where(pick, wild, rec).astype(np.uint16)
        for kv in (0, 1):
            enc = ap.encode_record(rec, table, kv)
            assert enc == oracle.encode_record(rec, table, kv), (heavy, trial, kv)
            assert np.array_equal(ap.decode_record(enc, table, kv), rec)


def test_host_decode_rejects_malformed():
    table = np.arange(22, dtype=np.uint8)
    with pytest.raises(ValueError):
        ap.decode_record(b"\x00" * 100, table, 0)
    enc = bytearray(ap.encode_record(np.zeros((128, 128), np.uint16) + 0x0300, table, 0))
    enc[22528] = 5  # header claims escapes the symbols do not have
    with pytest.raises(ValueError):
        ap.decode_record(bytes(enc), table, 0)
    with pytest.raises(ValueError):
        ap.encode_record(np.zeros((128, 128), np.uint16), table, 2)
