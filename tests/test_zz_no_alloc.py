"""fp_fused_decode_noalloc (decode attention whose split-KV workspace is a
static device array) against fp_fused_decode with caller workspaces, both
called through the C ABI: bit-identical outputs on two calls in a row, the
second with a smaller batch and shorter contexts (so the shared array holds
the first call's partials and plan when the second starts), plus the oracle
bar (2e-2 abs + 1e-2 rel) and the size limit's error."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from tests import kvgen
from tests.conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

_p, _i64 = ctypes.c_void_p, ctypes.c_int64


def _lib():
    from fragpack_amd.ops.fragpack_ext import LIB_PATH

    lib = ctypes.CDLL(str(LIB_PATH))
    f = lib.fp_fused_decode_noalloc
    f.argtypes = [_p, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _i64, _p, _p, _i64, _i64, ctypes.c_double, _p]
    f.restype = ctypes.c_int
    lib.fp_last_error.restype = ctypes.c_char_p
    lib.fp_fused_decode_noalloc_capacity.restype = _i64
    return lib


def _both(case, units):
    import torch

    from fragpack_amd.ops.fused_attn_decode import RecordTables, decode_attention, workspace_elems

    q, rec_addr, rec_len, plut, slut, bt, lens, arena = kvgen.upload(case)
    B, H = case.lens.size, case.heads
    ws = tuple(torch.empty(n, dtype=dt, device="cuda")
               for n, dt in zip(workspace_elems(H, units), (torch.float32, torch.float32, torch.int32)))
    want = torch.full_like(q, float("nan"))
    decode_attention(q, RecordTables(rec_addr, rec_len, plut, slut), bt, lens, case.scale, units, want, ws, True)
    got = torch.full_like(q, float("nan"))
    lib = _lib()
    print("noalloc call", B, H, case.group, units, flush=True)
    rc = lib.fp_fused_decode_noalloc(q.data_ptr(), q.stride(0), B, H, case.group, rec_addr.data_ptr(),
                                     rec_len.data_ptr(), plut.data_ptr(), slut.data_ptr(), bt.data_ptr(),
                                     bt.stride(0), lens.data_ptr(), got.data_ptr(), got.stride(0), units,
                                     case.scale, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.fp_last_error()
    torch.cuda.synchronize()
    del arena
    return want, got


def test_noalloc_matches_workspace_entry_on_consecutive_calls():
    import torch

    from fragpack_amd.ops.fused_attn_decode import decode_units

    sms = torch.cuda.get_device_properties(0).multi_processor_count
    big = kvgen.decode_case(seed=31, batch=6, heads=4, group=8, lens=[2000, 1, 700, 4096, 0, 129], outlier=0.02)
    small = kvgen.decode_case(seed=32, batch=2, heads=4, group=8, lens=[300, 1500], outlier=0.02)
    for case in (big, small):
        units = decode_units(case.lens.size, case.heads, sms)
        want, got = _both(case, units)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        ref = kvgen.oracle_decode(case)
        err = np.abs(got.float().cpu().numpy() - ref) - (2e-2 + 1e-2 * np.abs(ref))
        assert float(err.max()) <= 0


def test_noalloc_rejects_workspace_past_its_capacity():
    lib = _lib()
    cap = lib.fp_fused_decode_noalloc_capacity()
    units = cap // (8 * 128 * 4) + 1  # one KV head's partials alone exceed the array
    rc = lib.fp_fused_decode_noalloc(None, 1024, 1, 1, 8, None, None, None, None, None, 1, None, None, 1024, units,
                                     0.1, None)
    assert rc == -1 and b"exceeds" in lib.fp_last_error()
