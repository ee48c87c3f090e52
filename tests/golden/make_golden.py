"""Write the FragPack codec golden vectors from the reference implementation.

Run once, in the build container only (the reference tree is not present on
GPU boxes):

    python tests/golden/make_golden.py /root/reference

It imports the reference's ``fragpack.compression.attn_page`` and
``attn_tables`` (numpy codec, attn_page.py:146-269; calibration,
attn_tables.py:46-124) and records, for seeded inputs, the exact bytes they
produce. The byte layout of a coded record (nibble / word interleave, header
field order, raw-list and tail padding, chunk-major dense regions) is fixed
only by that code, so these vectors are what pins the oracle and the GPU
encoder byte for byte. The output, ``codec_golden.npz``, holds data only
(inputs and expected outputs); nothing from the reference source is kept.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

OUT = Path(__file__).with_name("codec_golden.npz")


def _bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> BF16 bit patterns."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def _trunc_bits(x: np.ndarray) -> np.ndarray:
    """Truncating fp32 -> BF16 (the reference unit tests' generator)."""
    return (np.ascontiguousarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(
        np.uint16
    )


def _kv_like(rng: np.random.Generator, shape: tuple, outlier: float) -> np.ndarray:
    """N(0,1) x per-channel lognormal(0, 0.5) scale, ``outlier`` channels x8."""
    dim = shape[-1]
    scale = rng.lognormal(0.0, 0.5, dim)
    scale[rng.random(dim) < outlier] *= 8.0
    return _bf16_bits(rng.standard_normal(shape) * scale)


def _escape_record(rng, table, n_ext: int, n_raw_per_slab: list[int], order) -> np.ndarray:
    """A record with ``n_ext`` extended-table escapes and the given raw counts
    per 2048-scalar kernel-order slab; everything else a primary entry."""
    tab = table.astype(np.uint16)
    absent = np.setdiff1d(np.arange(256, dtype=np.uint16), tab)
    n = 128 * 128
    high = tab[rng.integers(0, 7, n)]
    pos = rng.permutation(n)
    high[pos[:n_ext]] = tab[7 + rng.integers(0, 15, n_ext)]
    # raw scalars: choose kernel-order positions inside each slab
    used = set(pos[:n_ext].tolist())
    for slab, cnt in enumerate(n_raw_per_slab):
        cand = [p for p in rng.permutation(2048) + 2048 * slab if int(order[p]) not in used]
        for p in cand[:cnt]:
            tok_idx = int(order[p])
            high[tok_idx] = absent[rng.integers(0, absent.size)]
            used.add(tok_idx)
    low = rng.integers(0, 256, n).astype(np.uint16)
    return (low | (high << 8)).reshape(128, 128).astype(np.uint16)


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from fragpack.compression import attn_page as ap  # noqa: E402
    from fragpack.compression import attn_tables as at  # noqa: E402

    data: dict[str, np.ndarray] = {}
    records: list[tuple[str, np.ndarray, np.ndarray, int]] = []

    # 1. The reference unit tests' own inputs (test_attn_page.py:9-47).
    rng = np.random.default_rng(0)
    cal = _trunc_bits(rng.standard_normal((128, 128)) * 0.5)
    table0 = ap.calibrate_table((cal >> 8).astype(np.uint8))
    rec = _trunc_bits(rng.standard_normal((128, 128)) * 0.5)
    rec[3, 5] = 0x7F00 | (rec[3, 5] & 0xFF)
    rec[100, 127] = 0x0100
    for kv in (0, 1):
        records.append((f"unit_escapes_kv{kv}", rec, table0, kv))
    rng = np.random.default_rng(1)
    table1 = ap.calibrate_table((_trunc_bits(rng.standard_normal((128, 128)) * 0.1) >> 8).astype(np.uint8))
    records.append(("unit_compressible", _trunc_bits(rng.standard_normal((128, 128)) * 0.1), table1, 0))
    rng = np.random.default_rng(2)
    tab_ar = np.arange(22, dtype=np.uint8)
    rnd = rng.integers(0, 1 << 16, size=(128, 128), dtype=np.uint16)
    for kv in (0, 1):
        records.append((f"unit_incompressible_kv{kv}", rnd, tab_ar, kv))

    # 2. KV-shaped records (benchmark distribution), several seeds.
    for seed, outlier in ((10, 0.02), (11, 0.05), (12, 0.02)):
        rng = np.random.default_rng(seed)
        calk = _kv_like(rng, (512, 128), outlier)
        tab = ap.calibrate_table((calk >> 8).astype(np.uint8))
        for kv in (0, 1):
            records.append((f"kv_seed{seed}_kv{kv}", _kv_like(rng, (128, 128), outlier), tab, kv))

    # 3. Heavy-tail mix (encoder stress distribution): mostly fallbacks.
    rng = np.random.default_rng(20)
    tab = ap.calibrate_table((_kv_like(rng, (512, 128), 0.02) >> 8).astype(np.uint8))
    for frac in (0.002, 0.01, 0.1):
        base = rng.standard_normal((128, 128)) * rng.lognormal(0.0, 0.5, 128)
        heavy = rng.standard_t(2, (128, 128)) * 16
        mix = np.where(rng.random((128, 128)) < frac, heavy, base)
        for kv in (0, 1):
            records.append((f"heavy_{frac}_kv{kv}", _bf16_bits(mix), tab, kv))

    # 4. Boundary records around VAR_CAP and MAX_WARP_RAW.
    order = {kv: ap._kernel_order(kv) for kv in (0, 1)}
    rng = np.random.default_rng(30)
    tabb = ap.calibrate_table((_kv_like(rng, (512, 128), 0.02) >> 8).astype(np.uint8))
    for name, n_ext, raws in (
        ("ext4000", 4000, [0] * 8),  # var_len exactly VAR_CAP
        ("ext4001", 4001, [0] * 8),  # one nibble over: fallback
        ("ext3999", 3999, [0] * 8),
        ("raw32", 100, [32, 0, 0, 0, 0, 0, 0, 32]),  # warp cap met
        ("raw33", 100, [0, 0, 33, 0, 0, 0, 0, 0]),  # warp cap exceeded
        ("rawall", 50, [32] * 8),
        ("rawcap_fit", 1696, [32] * 8),  # 1952 escapes + 256 raws: var_len 2048
        ("rawcap_over", 1697, [32] * 8),  # one more escape: 2064, fallback
        ("none", 0, [0] * 8),
    ):
        for kv in (0, 1):
            r = _escape_record(rng, tabb, n_ext, raws, order[kv])
            records.append((f"edge_{name}_kv{kv}", r, tabb, kv))

    # 5. All-zero record (the store's null block) and constant records.
    z = np.zeros((128, 128), np.uint16)
    records.append(("zeros_kv0", z, tabb, 0))
    records.append(("const_absent_kv1", np.full((128, 128), 0xABCD, np.uint16), tabb, 1))

    names = []
    for i, (name, raw, table, kv) in enumerate(records):
        enc = ap.encode_record(raw, table, kv)
        dec = ap.decode_record(enc, table, kv)
        assert np.array_equal(dec, raw), name
        data[f"r{i}_raw"] = np.ascontiguousarray(raw, np.uint16)
        data[f"r{i}_table"] = np.ascontiguousarray(table, np.uint8)
        data[f"r{i}_kv"] = np.array(kv, np.int32)
        data[f"r{i}_enc"] = np.frombuffer(enc, np.uint8).copy()
        names.append(name)
    data["record_names"] = np.array(names)
    for kv in (0, 1):
        data[f"kernel_order_kv{kv}"] = ap._kernel_order(kv).astype(np.int32)
    for i, (_, _, table, _) in enumerate(records[:1] + records[5:6]):
        lo, hi = ap.primary_lut(table)
        data[f"plut{i}"] = np.array([lo, hi], np.uint32)
        data[f"slut{i}"] = np.frombuffer(ap.secondary_lut(table), np.uint8).copy()
        data[f"plut{i}_table"] = table

    # 6. Calibration: a seeded dump and a tie-heavy histogram.
    rng = np.random.default_rng(40)
    dump = _kv_like(rng, (2, 1, 2, 128, 2, 128), 0.02)
    data["cal_dump"] = dump
    tables = at.calibrate(dump)
    data["cal_table"] = tables
    dev = at.device_tables(tables, "cpu")
    data["cal_rank_of"] = dev.rank_of.numpy()
    data["cal_plut"] = dev.plut.numpy()
    data["cal_slut"] = dev.slut.numpy()
    ties = np.repeat(np.arange(40, dtype=np.uint8)[::-1], 3)  # 40 values, 3 each
    ties = np.concatenate([ties, np.full(5, 200, np.uint8), np.full(3, 7, np.uint8)])
    data["tie_input"] = ties
    data["tie_table"] = ap.calibrate_table(ties)

    # 7. Blob geometry.
    geo = [(l, h) for l in (1, 2, 48) for h in (1, 2, 4, 8)]
    data["blob_geo"] = np.array(geo, np.int64)
    data["blob_head"] = np.array([ap.blob_head_bytes(l, h) for l, h in geo], np.int64)
    data["blob_slot"] = np.array([ap.blob_slot_bytes(l, h) for l, h in geo], np.int64)

    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(records)} records)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
