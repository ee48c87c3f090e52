"""Host-side logic (no GPU work): the package's calibration / LUT / blob
arithmetic against the reference golden vectors, the decode workspace
contract, store memory accounting on CPU tensors, and the C-ABI library
exporting every entry point include/fragpack_hip.h declares."""

from __future__ import annotations

import ctypes
from pathlib import Path
import re

import numpy as np
import pytest
import torch

from fragpack_amd.compression import attn_page as ap
from fragpack_amd.compression import attn_tables as at
from fragpack_amd.ops import fused_attn_decode as fad
from fragpack_amd.ops.fragpack_ext import LIB_PATH

ROOT = Path(__file__).resolve().parent.parent


def test_constants():
    assert ap.DENSE_BYTES == 22528 and ap.RAW_RECORD_BYTES == 32768 and ap.VAR_CAP == 2048
    assert ap.TABLE_ENTRIES == 22 and ap.BLOB_MAGIC == 0x424B5046


def test_kernel_order_and_calibration_vs_golden(golden):
    for kv in (0, 1):
        assert np.array_equal(ap.kernel_order(kv), golden[f"kernel_order_kv{kv}"])
    assert np.array_equal(ap.calibrate_table(golden["tie_input"]), golden["tie_table"])
    assert np.array_equal(at.calibrate(golden["cal_dump"]), golden["cal_table"])


def test_luts_vs_golden(golden):
    for i in range(2):
        table = golden[f"plut{i}_table"]
        assert np.array_equal(np.array(ap.primary_lut(table), np.uint32), golden[f"plut{i}"])
        assert np.array_equal(np.frombuffer(ap.secondary_lut(table), np.uint8), golden[f"slut{i}"])
    dt = at.device_tables(golden["cal_table"], torch.device("cpu"))
    assert np.array_equal(dt.rank_of.numpy(), golden["cal_rank_of"])
    assert np.array_equal(dt.plut.numpy(), golden["cal_plut"])
    assert np.array_equal(dt.slut.numpy(), golden["cal_slut"])


def test_blob_sizes_vs_golden(golden):
    for (l, h), head, slot in zip(golden["blob_geo"], golden["blob_head"], golden["blob_slot"]):
        assert ap.blob_head_bytes(int(l), int(h)) == head
        assert ap.blob_slot_bytes(int(l), int(h)) == slot


def test_tables_npz_round_trip(tmp_path):
    rng = np.random.default_rng(0)
    dump = rng.integers(0, 1 << 16, size=(2, 3, 2, 128, 4, 128), dtype=np.uint16)
    table = at.calibrate(dump)
    assert table.shape == (3, 2, 4, 22)
    path = tmp_path / "t.npz"
    np.savez(path, table=table)
    dt = at.load_tables(str(path), torch.device("cpu"), slice(2, 4))
    assert dt.rank_of.shape == (3, 2, 2, 256)
    with pytest.raises(ValueError):
        at.load_tables(str(path), torch.device("cpu"), slice(4, 8))
    with pytest.raises(ValueError):
        at.device_tables(np.zeros((1, 2, 1, 21), np.uint8), torch.device("cpu"))


def test_decode_units_and_workspace():
    assert fad.decode_units(4, 4, 256) >= 4
    assert fad.decode_units(269, 4, 256) == 269 + fad.SPLIT_WAVES * (fad.UNITS_PER_CU * 256 // 4) - 1
    opart, ml, plan = fad.workspace_elems(4, 100)
    assert opart == 4 * 100 * 8 * 128 and ml == 4 * 100 * 16
    assert plan >= 2 + 4 * 100 + 8 * 100 + 4 * 100


def test_encode_record_rejects_bad_size():
    with pytest.raises(ValueError):
        ap.encode_record(np.zeros(10, np.uint16), np.arange(22, dtype=np.uint8), 0)


def test_memory_usage_counts_page_stride_and_separates_overflow():
    """Store accounting on CPU tensors (no kernels): padded arena rows are
    counted at their stride; only the overflow pool scales with its size."""
    from fragpack_amd.ops.hbm_kv import HbmKvStore, page_bytes

    layers, blocks, heads = 2, 3, 1
    payload = page_bytes(heads)
    strides = (payload + 16, payload + 48)
    owners = [torch.empty((blocks, s), dtype=torch.uint8) for s in strides]
    arenas = [o[:, :payload] for o in owners]
    table = np.broadcast_to(np.arange(22, dtype=np.uint8), (layers, 2, heads, 22)).copy()
    tables = at.device_tables(table, torch.device("cpu"))

    def build(n):
        return HbmKvStore(arenas, heads, tables, max_tokens=128, staging_slots=2, overflow_records=n)

    small, larger = build(1).memory_usage(), build(2).memory_usage()
    assert small["arena"] == sum(o.numel() for o in owners) > layers * blocks * payload
    assert small["staging"] > 0 and small["scratch"] > 0 and small["metadata"] > 0 and small["codebooks"] > 0
    assert larger["overflow"] == 2 * small["overflow"]
    assert {k: v for k, v in small.items() if k != "overflow"} == {k: v for k, v in larger.items() if k != "overflow"}


def test_store_rejects_mismatched_tables():
    from fragpack_amd.ops.hbm_kv import HbmKvStore

    tables = at.device_tables(np.zeros((1, 2, 2, 22), np.uint8) + np.arange(22, dtype=np.uint8), torch.device("cpu"))
    with pytest.raises(ValueError):
        HbmKvStore([torch.empty((2, 64), dtype=torch.uint8)] * 2, 2, tables, 128, 1, 1)


def _declared_symbols():
    text = (ROOT / "include" / "fragpack_hip.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(fp_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    assert LIB_PATH.exists(), "build the library first (__graft_entry__.build())"
    lib = ctypes.CDLL(str(LIB_PATH))
    syms = _declared_symbols()
    assert len(syms) >= 12
    for name in syms:
        assert hasattr(lib, name), name
    lib.fp_abi_version.restype = ctypes.c_int
    assert lib.fp_abi_version() == 1
    lib.fp_last_error.restype = ctypes.c_char_p
    assert isinstance(lib.fp_last_error(), bytes)


def test_c_abi_rejects_bad_arguments_without_gpu_work():
    """Argument checks run before any launch: errors come back as -1 + message."""
    lib = ctypes.CDLL(str(LIB_PATH))
    lib.fp_last_error.restype = ctypes.c_char_p
    f = lib.fp_fused_decode
    f.restype = ctypes.c_int
    p, i64 = ctypes.c_void_p, ctypes.c_int64
    f.argtypes = [p, i64, i64, i64, i64, p, p, p, p, p, i64, p, p, i64, p, i64, p, i64, p, i64, i64, ctypes.c_int,
                  ctypes.c_double, p]
    # group 3 does not divide 8
    rc = f(None, 1024, 1, 4, 3, None, None, None, None, None, 1, None, None, 0, None, 0, None, 0, None, 1024, 1, 1,
           0.1, None)
    assert rc == -1 and b"group" in lib.fp_last_error()
    # units < batch
    rc = f(None, 4096, 4, 4, 8, None, None, None, None, None, 1, None, None, 1 << 20, None, 1 << 20, None, 1 << 20,
           None, 4096, 2, 1, 0.1, None)
    assert rc == -1 and b"unit" in lib.fp_last_error()
    # empty batch is a no-op
    assert f(None, 4096, 0, 4, 8, None, None, None, None, None, 1, None, None, 0, None, 0, None, 0, None, 4096, 0, 1,
             0.1, None) == 0


def test_store_write_rejects_bad_steps_without_gpu_work():
    """The store write's argument checks (fp_store.hip write_args) return -1
    with a message before any launch: a step of 2^30+ (token, head) items,
    odd strides; an empty step is a no-op."""
    from fragpack_amd.ops.fragpack_ext import FpStore

    lib = ctypes.CDLL(str(LIB_PATH))
    lib.fp_last_error.restype = ctypes.c_char_p
    f = lib.fp_hbm_write
    f.restype = ctypes.c_int
    p, i64 = ctypes.c_void_p, ctypes.c_int64
    f.argtypes = [ctypes.POINTER(FpStore), p, i64, i64, p, i64, i64, p, i64, i64, p]
    d = FpStore(num_layers=1, num_blocks=4, kv_heads=8, staging_slots=2, scratch_slots=2, ovf_words=1, list_cap=64,
                overflow_records=32)
    dummy = p(256)  # never dereferenced: the checks fail first
    rc = f(ctypes.byref(d), dummy, 8 * 128, 128, dummy, 8 * 128, 128, dummy, 1 << 27, 0, None)
    assert rc == -1 and b"items" in lib.fp_last_error()
    rc = f(ctypes.byref(d), dummy, 8 * 128 + 1, 128, dummy, 8 * 128, 128, dummy, 16, 0, None)
    assert rc == -1 and b"strides" in lib.fp_last_error()
    rc = f(ctypes.byref(d), dummy, 8 * 128, 128, dummy, 8 * 128, 128, dummy, 16, 5, None)
    assert rc == -1 and b"layer" in lib.fp_last_error()
    assert f(ctypes.byref(d), dummy, 8 * 128, 128, dummy, 8 * 128, 128, dummy, 0, 0, None) == 0


def test_planner_reciprocal_division_is_exact_within_its_range():
    """The device planners divide x / d (0 <= x < 2^22, d >= 1) by a float
    product with the hardware reciprocal (relative error up to one ulp,
    2^-23) and one correction step each way (fp_attn.hip, ``Divider``).
    Restated in float32 with the reciprocal taken one ulp low, exact and one
    ulp high: the quotient equals x // d everywhere sampled, including
    multiples of d and their neighbours and the range's ends."""
    rng = np.random.default_rng(7)
    ds = np.concatenate([np.arange(1, 3000), rng.integers(3000, 1 << 22, 4000), [(1 << 22) - 1]]).astype(np.int64)
    for d in ds:
        k = rng.integers(0, ((1 << 22) - 1) // d + 1, 24)
        x = np.concatenate([k * d, k * d - 1, k * d + d - 1, rng.integers(0, 1 << 22, 24), [0, (1 << 22) - 1]])
        x = x[(x >= 0) & (x < (1 << 22))]
        exact = np.float32(1.0) / np.float32(d)
        for inv in (np.nextafter(exact, np.float32(0)), exact, np.nextafter(exact, np.float32(2))):
            q = np.trunc(x.astype(np.float32) * np.float32(inv)).astype(np.int64)
            q += (q + 1) * d <= x
            q -= q * d > x
            np.testing.assert_array_equal(q, x // d, err_msg=f"d={d}")


def test_plan_reuse_without_a_plan_is_refused():
    """A reusing decode call (replan=False) on a workspace no planning call
    has written is refused on the host, before any device pointer is taken:
    the kernel would follow whatever descriptors the buffer holds."""
    from fragpack_amd.ops.fragpack_ext import extension

    B, H, G, units = 2, 2, 8, 8
    q = torch.zeros((B, H * G, 128), dtype=torch.bfloat16)
    out = torch.zeros_like(q)
    opart, ml, plan = fad.workspace_elems(H, units)
    ws = (torch.zeros(opart), torch.zeros(ml), torch.zeros(plan, dtype=torch.int32))
    args = (q, torch.zeros((4, 2, H), dtype=torch.int64), torch.zeros((4, 2, H), dtype=torch.int32),
            torch.zeros((2, H, 2), dtype=torch.int32), torch.zeros((2, H, 16), dtype=torch.uint8),
            torch.zeros((B, 4), dtype=torch.int32), torch.ones(B, dtype=torch.int32), *ws, out, units)
    with pytest.raises(RuntimeError, match="plan first"):
        extension().fused_decode(*args, False, 0.1, G)
    # a key from another shape is refused too
    ws[2]._fp_plan_key = (units + 1, B, H)
    with pytest.raises(RuntimeError, match="plan first"):
        extension().fused_decode(*args, False, 0.1, G)
