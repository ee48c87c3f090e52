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

``encode_record`` / ``decode_record`` are the host codec (numpy, no GPU
needed, as the reference's are): every byte of a record is placed through
index maps computed once per kv from the kernel order -- which token-major
scalar each dense low byte holds, which scalars feed each nibble of each
symbol word, which scalar each raw-form halfword holds -- so encode and
decode are gathers and scatters over those maps.  ``encode_records`` /
``decode_records`` are the GPU batch codec (libfragpack_hip.so kernels),
byte-identical to the host codec.  Table calibration and LUT packing are
host-side numpy, as in the reference.
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


# ---------------------------------------------------------------------------
# Host codec.  Byte placement of a coded record (attn_page.py:56-80 format):
#   low byte of kernel-order scalar 64 t + 16 j + i  -> byte 16 (256 j + t) + i
#   symbol word (group G = 2 t + gi, k)              -> u32 at LOW_BYTES +
#       8 (256 m + t) + 4 x with 2 m + x = 3 gi + k; nibble n of that word is
#       (code of scalar 32 G + 8 k + n) & 7 | (bit k of code 32 G + 24 + n) << 3
#   raw form: kernel-order scalar 64 t + 8 st + i    -> u16 at 16 (256 st + t) + 2 i
# The maps below give, for each output position, the token-major scalar it
# reads (composed with the kernel order of K or V).

_SYM_WORDS = SYMBOL_BYTES // 4  # 1536 u32 words: 3 per 32-scalar group


def _placement_maps(kv: int) -> dict[str, NDArray[np.int64]]:
    order = kernel_order(kv)  # kernel-order position -> token-major scalar
    pos = np.arange(LOW_BYTES)
    j, t, i = pos >> 12, (pos >> 4) & 255, pos & 15
    low = order[64 * t + 16 * j + i]
    q = np.arange(_SYM_WORDS)
    m, t, x = q // 512, (q >> 1) & 255, q & 1
    gk = 2 * m + x  # 3 gi + k
    group = 2 * t + gk // 3
    k = gk % 3
    n = np.arange(8)
    code_src = order[32 * group[:, None] + 8 * k[:, None] + n[None, :]]  # [word, nibble]: 3 code bits
    bit_src = order[32 * group[:, None] + 24 + n[None, :]]              # [word, nibble]: one bit of this code
    h = np.arange(RECORD_SCALARS)
    st, t, i = h >> 11, (h >> 3) & 255, h & 7
    raw = order[64 * t + 8 * st + i]
    return {"order": order, "low": low, "code_src": code_src, "bit_src": bit_src, "bit_k": k, "raw": raw}


_MAPS = (_placement_maps(0), _placement_maps(1))
_NIB_SHIFT = (4 * np.arange(8)).astype(np.uint32)
_HEADER = struct.Struct("<4I8H8H")


def _checked_kv(kv: int) -> int:
    if kv not in (0, 1):
        raise ValueError(f"kv must be 0 (K) or 1 (V), got {kv}")
    return int(kv)


def encode_record(raw: NDArray[np.uint16], table: NDArray[np.uint8], kv: int) -> bytes:
    """Encode one token-major ``[128, 128]`` BF16 record on the host
    (attn_page.py:146-209).

    Args:
        raw: BF16 bit patterns as uint16 (``PAGE_TOKENS * HEAD_DIM`` of them).
        table: The head's 22-entry table (:func:`calibrate_table`).
        kv: 0 for a K record, 1 for a V record (selects the kernel order).

    Returns:
        The record (16-byte aligned length), coded, or the ``RAW_RECORD_BYTES``
        raw form when the variable region would exceed ``VAR_CAP`` or a
        2048-scalar slab would hold more than ``MAX_WARP_RAW`` raw scalars.

    Raises:
        ValueError: If ``raw`` has the wrong size or ``kv`` is not 0 / 1.

    Async/thread-safety:
        Pure function.
    """
    tm = np.ascontiguousarray(raw, dtype=np.uint16).reshape(-1)
    if tm.size != RECORD_SCALARS:
        raise ValueError("record must hold PAGE_TOKENS * HEAD_DIM scalars")
    mp = _MAPS[_checked_kv(kv)]
    ranks = rank_of(table)[tm >> 8]  # per token-major scalar
    seq = ranks[mp["order"]]         # in kernel order
    esc = seq >= PRIMARY_DIRECT
    is_raw = seq >= TABLE_ENTRIES
    slab_raw = is_raw.reshape(WARPS, WARP_SCALARS).sum(axis=1)
    esc_ranks = seq[esc]
    n_esc, n_raw = int(esc_ranks.size), int(slab_raw.sum())
    raw_offset = (HEADER_BYTES + (n_esc + 1) // 2 + 3) & ~3
    var_len = (raw_offset + 4 * n_raw + 15) & ~15
    if var_len > VAR_CAP or int(slab_raw.max()) > MAX_WARP_RAW:
        return tm[mp["raw"]].astype("<u2").tobytes()
    out = np.zeros(DENSE_BYTES + var_len, np.uint8)
    out[:LOW_BYTES] = tm[mp["low"]] & 0xFF
    code = np.minimum(ranks, PRIMARY_DIRECT).astype(np.uint32)
    nib = (code[mp["code_src"]] & 7) | (((code[mp["bit_src"]] >> mp["bit_k"][:, None]) & 1) << 3)
    out[LOW_BYTES:DENSE_BYTES] = (nib << _NIB_SHIFT).sum(axis=1, dtype=np.uint32).astype("<u4").view(np.uint8)
    # variable region: header, escape nibbles (low nibble first), raw list
    slab_esc = esc.reshape(WARPS, WARP_SCALARS).sum(axis=1)
    esc_prefix = np.cumsum(slab_esc) - slab_esc
    raw_prefix = np.cumsum(slab_raw) - slab_raw
    var = out[DENSE_BYTES:]
    var[:HEADER_BYTES] = np.frombuffer(_HEADER.pack(n_esc, n_raw, raw_offset, 0, *esc_prefix, *raw_prefix), np.uint8)
    nibbles = np.where(esc_ranks < TABLE_ENTRIES, esc_ranks.astype(np.int32) - PRIMARY_DIRECT, RAW_NIBBLE)
    packed = np.zeros((n_esc + 1) // 2 * 2, np.uint8)
    packed[:n_esc] = nibbles
    var[HEADER_BYTES : HEADER_BYTES + packed.size // 2] = packed[0::2] | (packed[1::2] << 4)
    ordinals = np.flatnonzero(esc_ranks >= TABLE_ENTRIES).astype(np.uint32)
    highs = (tm[mp["order"]][is_raw] >> 8).astype(np.uint32)
    var[raw_offset : raw_offset + 4 * n_raw] = (ordinals | (highs << 16)).astype("<u4").view(np.uint8)
    return out.tobytes()


def decode_record(record: bytes, table: NDArray[np.uint8], kv: int) -> NDArray[np.uint16]:
    """Decode one record (coded or raw) on the host (attn_page.py:212-269).

    Args:
        record: Bytes from :func:`encode_record` (or the arena / overflow).
        table: The table it was coded with.
        kv: The ``kv`` it was coded with.

    Returns:
        uint16 ``[128, 128]`` token-major BF16 bit patterns.

    Raises:
        ValueError: If the length is impossible or the variable region is
            inconsistent with the symbols.

    Async/thread-safety:
        Pure function.
    """
    mp = _MAPS[_checked_kv(kv)]
    buf = np.frombuffer(record, np.uint8)
    out = np.empty(RECORD_SCALARS, np.uint16)
    if buf.size == RAW_RECORD_BYTES:
        out[mp["raw"]] = buf.view("<u2")
        return out.reshape(PAGE_TOKENS, HEAD_DIM)
    if not DENSE_BYTES + HEADER_BYTES <= buf.size <= DENSE_BYTES + VAR_CAP:
        raise ValueError(f"record length {buf.size} is neither raw nor coded")
    tab = np.asarray(table, np.uint8)
    words = buf[LOW_BYTES:DENSE_BYTES].view("<u4").astype(np.uint32)
    nib = (words[:, None] >> _NIB_SHIFT) & 15  # [word, nibble]
    code = np.zeros(RECORD_SCALARS, np.uint32)  # token-major
    code[mp["code_src"]] = nib & 7
    np.bitwise_or.at(code, mp["bit_src"], (nib >> 3) << mp["bit_k"][:, None].astype(np.uint32))
    var = buf[DENSE_BYTES:]
    n_esc, n_raw, raw_offset = _HEADER.unpack_from(var)[:3]
    if HEADER_BYTES + (n_esc + 1) // 2 > var.size or raw_offset + 4 * n_raw > var.size:
        raise ValueError("variable region overruns the record")
    seq_code = code[mp["order"]]
    escaped = seq_code == PRIMARY_DIRECT
    if int(escaped.sum()) != n_esc:
        raise ValueError("escape count does not match the symbols")
    packed = var[HEADER_BYTES : HEADER_BYTES + (n_esc + 1) // 2]
    nibbles = np.stack([packed & 15, packed >> 4], axis=1).reshape(-1)[:n_esc]
    highs = np.zeros(n_esc, np.uint16)
    ext = nibbles < RAW_NIBBLE
    highs[ext] = tab[PRIMARY_DIRECT + nibbles[ext]]
    entries = var[raw_offset : raw_offset + 4 * n_raw].view("<u4")
    ords = entries & 0xFFFF
    if np.any(ords >= n_esc):
        raise ValueError("raw entry names no escape")
    highs[ords] = entries >> 16
    high_seq = np.zeros(RECORD_SCALARS, np.uint16)
    high_seq[~escaped] = tab[seq_code[~escaped]]
    high_seq[escaped] = highs
    out[mp["low"]] = buf[:LOW_BYTES]
    out[mp["order"]] |= high_seq << 8
    return out.reshape(PAGE_TOKENS, HEAD_DIM)


def _device():
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("the GPU batch codec needs a GPU; encode_record / decode_record run on the host")
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
