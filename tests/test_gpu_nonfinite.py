"""Decode attention over KV holding NaN and Inf bit patterns.

The codec is lossless for every BF16 bit pattern, so a stored K or V may be
NaN or +-Inf; attention must then give what IEEE arithmetic gives (the
reference computes softmax(QK^T)V in fp32 with these values as they are,
fragpack/ops/fused_attn_decode.cu:214-404).  Checked against the float64
reference softmax: the same positions NaN, the same signed infinities, and
every finite output within 2e-2 abs + 1e-2 rel.  One sequence per case: NaN
in V (one output dim NaN), NaN in K (every head of the group NaN), +Inf in K
(heads whose query makes the score +Inf are NaN, those where it is -Inf drop
that token), -Inf in V in the raw tail page (one dim -Inf), and a clean
sequence.  Records with the special values are coded through escapes or stay
raw, as the codec decides.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests import kvgen
from tests.conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

NAN, POS_INF, NEG_INF = 0x7FC0, 0x7F80, 0xFF80


def _poke(kv, bt):
    # (sequence, token, kv, head, dim, bits)
    for b, t, k, h, d, bits in ((0, 5, 1, 0, 7, NAN), (1, 130, 0, 1, 3, NAN), (2, 40, 0, 0, 0, POS_INF),
                                (3, 260, 1, 1, 100, NEG_INF)):
        kv[bt[b, t // 128], k, t % 128, h, d] = bits


@pytest.mark.parametrize("group", [1, 4, 8])
def test_nan_and_inf_kv_propagate_like_ieee(group):
    case = kvgen.decode_case(seed=21 + group, batch=5, heads=2, group=group, lens=[300, 300, 300, 300, 300],
                             poke=_poke)
    got = kvgen.run_gpu_decode(case)
    ref = kvgen.reference_attention(case)
    assert np.isnan(ref).any() and np.isinf(ref).any()
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    np.testing.assert_array_equal(np.isposinf(got), np.isposinf(ref))
    np.testing.assert_array_equal(np.isneginf(got), np.isneginf(ref))
    fin = np.isfinite(ref)
    err = np.abs(got[fin] - ref[fin]) - (2e-2 + 1e-2 * np.abs(ref[fin]))
    assert err.max() <= 0, f"finite outputs outside 2e-2 + 1e-2 rel (excess {err.max()})"
    # the +Inf key: heads whose query component is positive are NaN, the others finite
    G = group
    q = kvgen.bits_to_f32(case.q_bits)[2, :G, 0]
    assert np.array_equal(np.isnan(got[2, :G]).all(axis=1), q > 0)
