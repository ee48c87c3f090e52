"""Codec tables for every (layer, kv, head): calibration, file format, kernel forms.

Reference interface: fragpack/compression/attn_tables.py (DeviceTables
:30-43, calibrate :46-67, load_tables :70-93, device_tables :96-124, CLI
:127-135).  The names, the ``.npz`` key ``table`` (uint8 ``[L, 2, H, 22]``,
most frequent high byte first) and the three kernel forms are that
interface; the implementation is this package's own:

* calibration builds one 256-bin histogram per (layer, kv, head) for all
  heads at once (``np.bincount`` over ``head_index * 256 + high_byte``),
  streaming the dump in slices of pages so a memory-mapped dump is never
  loaded whole, then ranks every histogram with the table rule of
  :func:`fragpack_amd.compression.attn_page.calibrate_table`;
* the kernel forms are derived for all heads in one vectorised pass.

CLI::

    python -m fragpack_amd.compression.attn_tables DUMP.npy OUT.npz

``DUMP.npy`` holds uint16 ``[S, L, 2, 128, H, 128]`` BF16 bit patterns
(S captured pages).
"""

from __future__ import annotations

import argparse
from dataclasses import dataclass
import sys

import numpy as np
from numpy.typing import NDArray
import torch

from fragpack_amd.compression import attn_page as ap
from fragpack_amd.logging import init_logger

logger = init_logger(__name__)

# elements of the dump read per histogram pass (bounds host memory for big dumps)
_PASS_ELEMS = 1 << 24


@dataclass(frozen=True)
class DeviceTables:
    """The kernels' lookup tables, for every layer, on one device.

    Attributes:
        rank_of: uint8 ``[L, 2, H, 256]``: table position of each high byte
            (255 when the byte is not in the table); read by the encoder.
        plut: int32 ``[L, 2, H, 2]``: table entries 0-6 and a zero byte as
            two little-endian words, the decoder's byte-permute source.
        slut: uint8 ``[L, 2, H, 16]``: entries 7-21 and a zero byte, indexed
            by escape nibble; read by the decoder.
    """

    rank_of: torch.Tensor
    plut: torch.Tensor
    slut: torch.Tensor


def _histograms(dump: NDArray[np.uint16]) -> NDArray[np.int64]:
    """int64 ``[L, 2, H, 256]`` counts of each high byte."""
    pages, n_layers, kv, _, heads, _ = dump.shape
    n_hist = n_layers * kv * heads
    counts = np.zeros(n_hist * 256, np.int64)
    # histogram id of each element of one page: (layer, kv, head) over [L, 2, 128, H, 128]
    hid = (np.arange(n_layers)[:, None, None, None, None] * kv + np.arange(kv)[None, :, None, None, None]) * heads
    hid = np.broadcast_to(hid + np.arange(heads)[None, None, None, :, None], (n_layers, kv, ap.PAGE_TOKENS, heads,
                                                                              ap.HEAD_DIM))
    base = (hid.astype(np.int64) << 8).reshape(-1)
    step = max(1, _PASS_ELEMS // base.size)
    for p0 in range(0, pages, step):
        part = np.asarray(dump[p0 : p0 + step]).reshape(-1, base.size)
        keys = (part >> 8).astype(np.int64) + base[None, :]
        counts += np.bincount(keys.reshape(-1), minlength=counts.size)
    return counts.reshape(n_layers, kv, heads, 256)


def calibrate(dump: NDArray[np.uint16]) -> NDArray[np.uint8]:
    """Calibrate one table per (layer, kv, head).

    Args:
        dump: uint16 ``[S, L, 2, 128, H, 128]`` captured pages (may be a
            memory map).

    Returns:
        uint8 ``[L, 2, H, 22]``: per head the 22 most frequent high bytes,
        most frequent first, equal counts in increasing byte order.

    Raises:
        ValueError: If ``dump`` does not have that shape.
    """
    if dump.ndim != 6 or dump.shape[2] != 2 or dump.shape[3] != ap.PAGE_TOKENS or dump.shape[5] != ap.HEAD_DIM:
        raise ValueError(f"dump must be uint16 [S, L, 2, 128, H, 128], got {tuple(dump.shape)}")
    hist = _histograms(dump)
    # rank by count descending, then byte value ascending (a stable sort of
    # -count over the byte values in increasing order)
    order = np.argsort(-hist, axis=-1, kind="stable")
    return order[..., : ap.TABLE_ENTRIES].astype(np.uint8)


def load_tables(path: str, device: torch.device, heads: slice = slice(None)) -> DeviceTables:
    """Kernel tables of a calibrated ``.npz`` for the KV heads ``heads`` (a
    tensor-parallel rank's slice).

    Raises:
        ValueError: If the file has no ``table`` of the right shape, or the
            slice selects no head.
    """
    with np.load(path, allow_pickle=False) as f:
        if "table" not in f.files:
            raise ValueError(f"{path} holds no FragPack 'table'")
        table = f["table"]
    if table.ndim != 4 or table.shape[1] != 2:
        raise ValueError(f"{path}: table must be [L, 2, H, 22], got {table.shape}")
    table = np.ascontiguousarray(table[:, :, heads])
    if table.shape[2] == 0:
        raise ValueError(f"FragPack tables {path} hold no head in {heads}")
    return device_tables(table, device)


def device_tables(table: NDArray[np.uint8], device: torch.device) -> DeviceTables:
    """The three kernel forms of calibrated tables ``[L, 2, H, 22]``.

    Raises:
        ValueError: If the last dimension is not 22 entries.
    """
    table = np.asarray(table, np.uint8)
    if table.ndim != 4 or table.shape[-1] != ap.TABLE_ENTRIES:
        raise ValueError(f"expected [L, 2, H, {ap.TABLE_ENTRIES}] tables, got {table.shape}")
    lead = table.shape[:3]
    flat = table.reshape(-1, ap.TABLE_ENTRIES)
    rank_of = np.full((flat.shape[0], 256), 255, np.uint8)
    rows = np.repeat(np.arange(flat.shape[0]), ap.TABLE_ENTRIES)
    rank_of[rows, flat.reshape(-1)] = np.tile(np.arange(ap.TABLE_ENTRIES, dtype=np.uint8), flat.shape[0])
    zero = np.zeros((flat.shape[0], 1), np.uint8)
    plut = np.ascontiguousarray(np.concatenate([flat[:, : ap.PRIMARY_DIRECT], zero], axis=1)).view("<i4")
    slut = np.concatenate([flat[:, ap.PRIMARY_DIRECT :], zero], axis=1)
    return DeviceTables(
        rank_of=torch.from_numpy(rank_of.reshape(*lead, 256)).to(device),
        plut=torch.from_numpy(plut.astype(np.int32).reshape(*lead, 2)).to(device),
        slut=torch.from_numpy(np.ascontiguousarray(slut).reshape(*lead, 16)).to(device),
    )


def _main(argv: list[str] | None = None) -> int:
    cli = argparse.ArgumentParser(prog="python -m fragpack_amd.compression.attn_tables",
                                  description="Calibrate FragPack codec tables from a captured KV dump.")
    cli.add_argument("dump", help=".npy of uint16 [S, L, 2, 128, H, 128] BF16 bit patterns")
    cli.add_argument("out", help="output .npz (key 'table', uint8 [L, 2, H, 22])")
    args = cli.parse_args(argv)
    dump = np.load(args.dump, mmap_mode="r", allow_pickle=False)
    if dump.dtype != np.uint16:
        cli.error(f"{args.dump} must hold uint16 BF16 bit patterns, not {dump.dtype}")
    table = calibrate(dump)
    np.savez(args.out, table=table)
    logger.info("calibrated %d tables from %d pages -> %s", table.shape[0] * table.shape[1] * table.shape[2],
                dump.shape[0], args.out)
    return 0


if __name__ == "__main__":
    sys.exit(_main())


__all__ = ["DeviceTables", "calibrate", "device_tables", "load_tables"]
