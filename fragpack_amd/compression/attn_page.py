"""FragPack record format: constants, calibration, LUTs and the record codec.

Reference: fragpack/compression/attn_page.py (format spec :1-44, constants
:51-80, calibrate_table :97-111, primary_lut / secondary_lut :114-143,
encode_record / decode_record :146-269, blob sizes :285-319).

A record holds one (page, kv, head) slice of 128 tokens x 128 dims of BF16
in the reference's "kernel order" (thread t = (w, g, c) of 256 owns scalars
[64t, 64t+64), scalar s = 8st + 4j + 2f + e; K: token 16w+8j+g, dim
16st+8f+2c+e; V swapped).  Coded records store every low byte verbatim and
the high byte as a 3-bit code into a calibrated 22-entry table (code 7 =
escape: a nibble into entries 7-21, or 15 = raw byte in a raw list).  A
record whose variable region exceeds ``VAR_CAP`` or with more than
``MAX_WARP_RAW`` raw scalars in a 2048-scalar slab is stored raw
(``RAW_RECORD_BYTES``).  The byte format is the reference's, unchanged.

``encode_record`` / ``decode_record`` run on the GPU (the batch codec
kernels of libfragpack_hip.so); there is no CPU codec in this package.
Table calibration and LUT packing are host-side numpy, as in the reference.
"""

from __future__ import annotations

import struct

import numpy as np
from numpy.typing import NDArray

PAGE_TOKENS = 128
HEAD_DIM = 128
RECORD_SCALARS = PAGE_TOKENS * HEAD_DIM
GROUP_SCALARS = 32
WARP_SCALARS = 2048
WARPS = RECORD_SCALARS // WARP_SCALARS
PRIMARY_DIRECT = 7
EXTENDED = 15
TABLE_ENTRIES = PRIMARY_DIRECT + EXTENDED
RAW_NIBBLE = 15
HEADER_BYTES = 48
LOW_BYTES = RECORD_SCALARS
SYMBOL_BYTES = RECORD_SCALARS * 3 // 8
DENSE_BYTES = LOW_BYTES + SYMBOL_BYTES
VAR_CAP = 2048
THREADS = 256
RAW_RECORD_BYTES = RECORD_SCALARS * 2
MAX_WARP_RAW = 32
BLOB_MAGIC = 0x424B5046  # "FPKB"
BLOB_FIXED_BYTES = 64
BLOB_ALIGN = 4096


def kernel_order(kv: int) -> NDArray[np.int64]:
    """Token-major scalar index of each kernel-order position (attn_page.py:83-91)."""
    t = np.arange(THREADS)[:, None]
    s = np.arange(RECORD_SCALARS // THREADS)[None, :]
    w, g, c = t >> 5, (t >> 2) & 7, t & 3
    st, j, f, e = s >> 3, (s >> 2) & 1, (s >> 1) & 1, s & 1
    rows = 16 * w + 8 * j + g
    cols = 16 * st + 8 * f + 2 * c + e
    tok, dim = (rows, cols) if kv == 0 else (cols, rows)
    return (tok * HEAD_DIM + dim).reshape(-1)


def calibrate_table(high_bytes: NDArray[np.uint8]) -> NDArray[np.uint8]:
    """The 22 most frequent high bytes, most frequent first; equal counts go
    to the smaller byte value (attn_page.py:97-111)."""
    counts = np.bincount(np.asarray(high_bytes, dtype=np.uint8).reshape(-1), minlength=256)
    # sort by (-count, byte): lexsort's last key is the primary one
    order = np.lexsort((np.arange(256), -counts))
    return order[:TABLE_ENTRIES].astype(np.uint8)


def primary_lut(table: NDArray[np.uint8]) -> tuple[int, int]:
    """The two little-endian u32 words of the 8-byte primary table: entries
    0-6 and a zero escape byte (attn_page.py:114-128)."""
    b = bytes(np.asarray(table, np.uint8)[:PRIMARY_DIRECT]) + b"\x00"
    lo, hi = struct.unpack("<II", b)
    return lo, hi


def secondary_lut(table: NDArray[np.uint8]) -> bytes:
    """Entries 7-21 then a zero byte, indexed by escape nibble (attn_page.py:131-143)."""
    return bytes(np.asarray(table, np.uint8)[PRIMARY_DIRECT:TABLE_ENTRIES]) + b"\x00"


def rank_of(table: NDArray[np.uint8]) -> NDArray[np.uint8]:
    """Table rank of every byte value, 255 if absent (attn_tables.py:112-117)."""
    r = np.full(256, 255, dtype=np.uint8)
    r[np.asarray(table, np.uint8)] = np.arange(TABLE_ENTRIES, dtype=np.uint8)
    return r


def _device():
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("the FragPack record codec runs on the GPU; no GPU is available")
    return torch.device("cuda", torch.cuda.current_device())


def encode_records(raw: NDArray[np.uint16], tables: NDArray[np.uint8], kv: NDArray[np.int32],
                   tab_idx: NDArray[np.int32]) -> list[bytes]:
    """Encode many token-major records on the GPU.

    Args:
        raw: uint16 ``[n, 128, 128]`` BF16 bit patterns.
        tables: uint8 ``[T, 22]`` head tables.
        kv: int32 ``[n]`` 0 (K) / 1 (V) per record.
        tab_idx: int32 ``[n]`` table of each record.

    Returns:
        The ``n`` records' bytes (each as :func:`encode_record` would return).
    """
    import torch

    from fragpack_amd.ops.fragpack_ext import extension

    dev = _device()
    raw = np.ascontiguousarray(raw, np.uint16).reshape(-1, PAGE_TOKENS, HEAD_DIM)
    n = raw.shape[0]
    ranks = np.stack([rank_of(t) for t in np.asarray(tables, np.uint8).reshape(-1, TABLE_ENTRIES)])
    t_raw = torch.from_numpy(raw.view(np.int16)).to(dev)
    out = torch.empty(n * RAW_RECORD_BYTES, dtype=torch.uint8, device=dev)
    lens = torch.empty(n, dtype=torch.int32, device=dev)
    extension().encode_records(
        t_raw,
        torch.from_numpy(np.ascontiguousarray(kv, np.int32)).to(dev),
        torch.from_numpy(ranks).to(dev),
        torch.from_numpy(np.ascontiguousarray(tab_idx, np.int32)).to(dev),
        out,
        lens,
    )
    host = out.view(n, RAW_RECORD_BYTES).cpu().numpy()
    ln = lens.cpu().numpy()
    return [host[i, : ln[i]].tobytes() for i in range(n)]


def encode_record(raw: NDArray[np.uint16], table: NDArray[np.uint8], kv: int) -> bytes:
    """Encode one token-major ``[128, 128]`` BF16 record (attn_page.py:146-209).

    Returns:
        The record (16-byte aligned length), coded, or the ``RAW_RECORD_BYTES``
        raw fallback.

    Raises:
        ValueError: If ``raw`` has the wrong size.
        RuntimeError: If no GPU (or the library) is available.
    """
    values = np.ascontiguousarray(raw, dtype=np.uint16).reshape(-1)
    if values.size != RECORD_SCALARS:
        raise ValueError("record must hold PAGE_TOKENS * HEAD_DIM scalars")
    return encode_records(values.reshape(1, PAGE_TOKENS, HEAD_DIM), np.asarray(table, np.uint8)[None],
                          np.array([kv], np.int32), np.zeros(1, np.int32))[0]


def decode_records(records: list[bytes], tables: NDArray[np.uint8], kv: NDArray[np.int32],
                   tab_idx: NDArray[np.int32]) -> NDArray[np.uint16]:
    """Decode many records on the GPU into uint16 ``[n, 128, 128]``."""
    import torch

    from fragpack_amd.ops.fragpack_ext import extension

    dev = _device()
    n = len(records)
    buf = np.zeros((max(n, 1), RAW_RECORD_BYTES), np.uint8)
    lens = np.empty(max(n, 1), np.int32)
    for i, r in enumerate(records):
        if len(r) != RAW_RECORD_BYTES and not (DENSE_BYTES + HEADER_BYTES <= len(r) <= DENSE_BYTES + VAR_CAP):
            raise ValueError(f"record {i} has an impossible length {len(r)}")
        buf[i, : len(r)] = np.frombuffer(r, np.uint8)
        lens[i] = len(r) - DENSE_BYTES
    tabs = np.asarray(tables, np.uint8).reshape(-1, TABLE_ENTRIES)
    plut = np.array([primary_lut(t) for t in tabs], np.uint32)
    slut = np.stack([np.frombuffer(secondary_lut(t), np.uint8) for t in tabs])
    d_buf = torch.from_numpy(buf).to(dev)
    addr = d_buf.data_ptr() + RAW_RECORD_BYTES * torch.arange(n, dtype=torch.int64)
    out = torch.empty((n, PAGE_TOKENS, HEAD_DIM), dtype=torch.int16, device=dev)
    extension().decode_records(
        addr.to(dev),
        torch.from_numpy(lens[:n]).to(dev),
        torch.from_numpy(np.ascontiguousarray(kv, np.int32)).to(dev),
        torch.from_numpy(plut.view(np.int32)).to(dev),
        torch.from_numpy(slut).to(dev),
        torch.from_numpy(np.ascontiguousarray(tab_idx, np.int32)).to(dev),
        out,
    )
    return out.cpu().numpy().view(np.uint16)


def decode_record(record: bytes, table: NDArray[np.uint8], kv: int) -> NDArray[np.uint16]:
    """Decode one record (attn_page.py:212-269) into uint16 ``[128, 128]``."""
    return decode_records([record], np.asarray(table, np.uint8)[None], np.array([kv], np.int32),
                          np.zeros(1, np.int32))[0]


def blob_head_bytes(num_layers: int, kv_heads: int) -> int:
    """Header + length table of a block blob, rounded up to ``BLOB_ALIGN``
    (attn_page.py:285-299)."""
    head = BLOB_FIXED_BYTES + 8 * num_layers * kv_heads
    return -(-head // BLOB_ALIGN) * BLOB_ALIGN


def blob_slot_bytes(num_layers: int, kv_heads: int) -> int:
    """Largest block blob (every record raw), aligned (attn_page.py:302-319)."""
    return blob_head_bytes(num_layers, kv_heads) + 2 * num_layers * kv_heads * RAW_RECORD_BYTES


__all__ = [
    "BLOB_ALIGN",
    "BLOB_FIXED_BYTES",
    "BLOB_MAGIC",
    "DENSE_BYTES",
    "HEAD_DIM",
    "PAGE_TOKENS",
    "RAW_RECORD_BYTES",
    "TABLE_ENTRIES",
    "VAR_CAP",
    "blob_head_bytes",
    "blob_slot_bytes",
    "calibrate_table",
    "decode_record",
    "decode_records",
    "encode_record",
    "encode_records",
    "kernel_order",
    "primary_lut",
    "rank_of",
    "secondary_lut",
]
