"""BASELINE config 0 on the CPU: the reference's CPU round trip + decode
attention for one layer (1 sequence, 4 KV heads, GQA 8, 1000 tokens = 7
coded blocks + a 104-token raw tail, 2% outlier channels), with tables made
by the repository's calibration CLI from a seeded [64, 1, 2, 128, 4, 128]
dump.  Checks: the CLI's tables equal a brute-force top-22 of the dump's
high bytes (ties to the lower byte, attn_page.py:97-111), every record of the
7 closed blocks decodes bit-exactly with the host codec, the tail is raw,
and the CPU oracle's attention is within 2e-2 abs + 1e-2 rel of the float64
reference.  The GPU leg of the same case is in test_gpu_decode.py.
"""

from __future__ import annotations

import numpy as np

from fragpack_amd.compression import attn_page as ap
from tests import kvgen

DENSE = 22528


def test_config0_cli_tables_round_trip_and_attention(tmp_path):
    case = kvgen.config0_case(tmp_path)
    dump = np.load(tmp_path / "dump.npy")
    hi = (dump >> 8).astype(np.int64)
    for kv in range(2):
        for h in range(4):
            counts = np.bincount(hi[:, 0, kv, :, h, :].ravel(), minlength=256)
            want = sorted(range(256), key=lambda v: (-counts[v], v))[:22]
            assert case.tables[kv, h].tolist() == want
    pages = case.block_table[0, :8]
    for p_i, blk in enumerate(pages):
        for kv in range(2):
            for h in range(4):
                off, n = int(case.rec_off[blk, kv, h]), DENSE + int(case.rec_len[blk, kv, h])
                rec = case.recs[off : off + n].tobytes()
                if p_i == 7:
                    assert n == 32768  # the open block's raw record
                else:
                    assert n < 32768
                np.testing.assert_array_equal(ap.decode_record(rec, case.tables[kv, h], kv), case.kv[blk, kv, :, h, :])
    got = kvgen.oracle_decode(case)
    ref = kvgen.reference_attention(case)
    np.testing.assert_allclose(got, ref, atol=2e-2, rtol=1e-2)
