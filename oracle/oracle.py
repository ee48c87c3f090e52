"""ctypes front end of the FragPack CPU oracle -- TEST INFRASTRUCTURE ONLY.

Loaded by tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` as the checker; the ``fragpack_amd`` package never imports it.
Each function names the reference code it restates (see fp_oracle.c).
"""

from __future__ import annotations

import ctypes
from pathlib import Path
import subprocess

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB_PATH = _DIR / "libfp_oracle.so"
_lib: ctypes.CDLL | None = None

RAW_RECORD_BYTES = 32768
DENSE_BYTES = 22528


def build() -> Path:
    """Compile libfp_oracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-B", "-C", str(_DIR), "CC=gcc"], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(_LIB_PATH))
        p = ctypes.c_void_p
        i64, i32, f32 = ctypes.c_int64, ctypes.c_int, ctypes.c_float
        _lib.fpo_kernel_order.argtypes = [i32, p]
        _lib.fpo_calibrate_table.argtypes = [p, i64, p]
        _lib.fpo_tables.argtypes = [p, p, p, p]
        _lib.fpo_encode_record.argtypes = [p, p, i32, p]
        _lib.fpo_encode_record.restype = i32
        _lib.fpo_decode_record.argtypes = [p, i32, p, i32, p]
        _lib.fpo_decode_record.restype = i32
        _lib.fpo_raw_record.argtypes = [p, i32, p]
        _lib.fpo_encode_batch.argtypes = [i64, p, p, p, p, p, p, i32]
        _lib.fpo_decode_batch.argtypes = [i64, p, p, p, p, p, p, i32]
        _lib.fpo_decode_batch.restype = i32
        _lib.fpo_paged_attention.argtypes = [
            p, i32, i32, i32, p, p, p, p, p, i64, p, f32, p, i32
        ]
        _lib.fpo_paged_attention.restype = i32
        _lib.fpo_num_threads.restype = i32
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags.c_contiguous
    return a.ctypes.data


def kernel_order(kv: int) -> np.ndarray:
    """attn_page.py:83-94."""
    out = np.empty(16384, np.int32)
    lib().fpo_kernel_order(kv, _ptr(out))
    return out


def calibrate_table(high: np.ndarray) -> np.ndarray:
    """attn_page.py:97-111."""
    h = np.ascontiguousarray(high, np.uint8).reshape(-1)
    out = np.empty(22, np.uint8)
    lib().fpo_calibrate_table(_ptr(h), h.size, _ptr(out))
    return out


def calibrate(dump: np.ndarray) -> np.ndarray:
    """attn_tables.py:46-67: dump uint16 [S, L, 2, 128, H, 128] -> [L, 2, H, 22]."""
    _, n_layers, kv, _, heads, _ = dump.shape
    out = np.empty((n_layers, kv, heads, 22), np.uint8)
    for idx in np.ndindex(n_layers, kv, heads):
        l, k, h = idx
        out[idx] = calibrate_table((np.asarray(dump[:, l, k, :, h, :]) >> 8).astype(np.uint8))
    return out


def tables(table: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(rank_of[256] u8, plut[2] u32, slut[16] u8) of one head table."""
    t = np.ascontiguousarray(table, np.uint8)
    rank_of = np.empty(256, np.uint8)
    plut = np.empty(2, np.uint32)
    slut = np.empty(16, np.uint8)
    lib().fpo_tables(_ptr(t), _ptr(rank_of), _ptr(plut), _ptr(slut))
    return rank_of, plut, slut


def encode_record(raw: np.ndarray, table: np.ndarray, kv: int) -> bytes:
    """attn_page.py:146-209."""
    r = np.ascontiguousarray(raw, np.uint16).reshape(-1)
    if r.size != 16384:
        raise ValueError("record must hold PAGE_TOKENS * HEAD_DIM scalars")
    t = np.ascontiguousarray(table, np.uint8)
    out = np.zeros(RAW_RECORD_BYTES, np.uint8)
    n = lib().fpo_encode_record(_ptr(r), _ptr(t), kv, _ptr(out))
    return out[:n].tobytes()


def raw_record(raw: np.ndarray, kv: int) -> bytes:
    """attn_page.py:279-282: the raw (kernel-order BF16) form of a record."""
    r = np.ascontiguousarray(raw, np.uint16).reshape(-1)
    out = np.zeros(RAW_RECORD_BYTES, np.uint8)
    lib().fpo_raw_record(_ptr(r), kv, _ptr(out))
    return out.tobytes()


def decode_record(record: bytes, table: np.ndarray, kv: int) -> np.ndarray:
    """attn_page.py:212-269."""
    buf = np.zeros(RAW_RECORD_BYTES, np.uint8)
    buf[: len(record)] = np.frombuffer(record, np.uint8)
    t = np.ascontiguousarray(table, np.uint8)
    out = np.empty(16384, np.uint16)
    if lib().fpo_decode_record(_ptr(buf), len(record), _ptr(t), kv, _ptr(out)) != 0:
        raise ValueError("malformed record")
    return out.reshape(128, 128)


def encode_batch(raw: np.ndarray, tables_: np.ndarray, tab_idx: np.ndarray, kv: np.ndarray,
                 threads: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """Encode ``raw`` [n,128,128] -> (records [n, 32768] u8, record byte lengths [n] i32)."""
    raw = np.ascontiguousarray(raw, np.uint16)
    n = raw.shape[0]
    out = np.zeros((n, RAW_RECORD_BYTES), np.uint8)
    lens = np.empty(n, np.int32)
    lib().fpo_encode_batch(
        n, _ptr(raw), _ptr(np.ascontiguousarray(tables_, np.uint8)),
        _ptr(np.ascontiguousarray(tab_idx, np.int32)), _ptr(np.ascontiguousarray(kv, np.int32)),
        _ptr(out), _ptr(lens), threads or lib().fpo_num_threads(),
    )
    return out, lens


def decode_batch(recs: np.ndarray, lens: np.ndarray, tables_: np.ndarray, tab_idx: np.ndarray,
                 kv: np.ndarray, threads: int = 0) -> np.ndarray:
    recs = np.ascontiguousarray(recs, np.uint8)
    n = recs.shape[0]
    out = np.empty((n, 128, 128), np.uint16)
    rc = lib().fpo_decode_batch(
        n, _ptr(recs), _ptr(np.ascontiguousarray(lens, np.int32)),
        _ptr(np.ascontiguousarray(tables_, np.uint8)), _ptr(np.ascontiguousarray(tab_idx, np.int32)),
        _ptr(np.ascontiguousarray(kv, np.int32)), _ptr(out), threads or lib().fpo_num_threads(),
    )
    if rc:
        raise ValueError("malformed record in batch")
    return out


def paged_attention(q_bits: np.ndarray, heads: int, rec: np.ndarray, rec_off: np.ndarray,
                    rec_len: np.ndarray, tables_: np.ndarray, block_table: np.ndarray,
                    seq_lens: np.ndarray, scale: float, threads: int = 0) -> np.ndarray:
    """fp32 attention over paged records; q_bits uint16 [B, H*G, 128]."""
    q = np.ascontiguousarray(q_bits, np.uint16)
    B, hq, _ = q.shape
    G = hq // heads
    bt = np.ascontiguousarray(block_table, np.int32)
    out = np.empty((B, hq, 128), np.float32)
    rc = lib().fpo_paged_attention(
        _ptr(q), B, heads, G, _ptr(np.ascontiguousarray(rec, np.uint8)),
        _ptr(np.ascontiguousarray(rec_off, np.int64)), _ptr(np.ascontiguousarray(rec_len, np.int32)),
        _ptr(np.ascontiguousarray(tables_, np.uint8)), _ptr(bt), bt.shape[1],
        _ptr(np.ascontiguousarray(seq_lens, np.int32)), scale, _ptr(out),
        threads or lib().fpo_num_threads(),
    )
    if rc:
        raise ValueError("malformed record")
    return out


def decode_plan(seq_lens: np.ndarray, units: int, kv_heads: int = 1,
                slots: int = 768) -> tuple[int, int, np.ndarray, np.ndarray]:
    """Split-KV work plan: the reference planner's layout
    (fused_attn_decode.cu:95-163) with this build's chunk-size policy.

    Every sequence is cut into chunks of ``ppc`` pages.  ``ppc`` minimises
    ``ceil(chunks * kv_heads / slots) * (ppc + 1)`` over the candidates
    ``ceil(longest / c)`` for c = 1..64 whose chunk count fits ``units``,
    ties going to the larger ``ppc`` (``slots``: workgroups the device runs
    at once over all heads).

    Returns ``(ppc, used, unit_map [units, 2], seq_map [B, 2])``: unit u
    covers pages from ``unit_map[u, 1]`` of sequence ``unit_map[u, 0]`` (-1
    when idle; an idle unit's page entry is left 0 here), sequence b owns
    ``seq_map[b, 1]`` units from ``seq_map[b, 0]``, ``used`` units in all.
    """
    lens = np.asarray(seq_lens, np.int64)
    batch = lens.size
    pages = (lens + 127) >> 7
    longest = int(pages.max(initial=0))

    def chunks(ppc: int) -> np.ndarray:
        return (pages + ppc - 1) // ppc

    best = None
    for c in range(1, 65):
        ppc = max(1, -(-longest // c))
        n = int(chunks(ppc).sum())
        if n > units:
            continue
        key = (-(-n * kv_heads // slots) * (ppc + 1), -ppc)
        if best is None or key < best:
            best = key
    ppc = -best[1]
    c = chunks(ppc)
    first = np.concatenate([[0], np.cumsum(c)[:-1]]).astype(np.int64) if batch else np.zeros(0, np.int64)
    unit_map = np.zeros((units, 2), np.int32)
    unit_map[:, 0] = -1
    for b in range(batch):
        for s in range(int(c[b])):
            unit_map[first[b] + s] = (b, s * ppc)
    seq_map = np.stack([first, c], axis=1).astype(np.int32) if batch else np.zeros((0, 2), np.int32)
    return ppc, int(c.sum()), unit_map, seq_map


def num_threads() -> int:
    return int(lib().fpo_num_threads())
