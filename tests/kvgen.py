"""Seeded synthetic KV, decode cases and reference attention for the tests.

Distribution (the benchmark's): K/V = N(0,1) x a per-channel
scale ~ lognormal(0, 0.5), a fraction of channels x8 (outliers), rounded to
BF16 (round-to-nearest-even).  Records are built with the CPU oracle (test
infrastructure), uploaded to one device arena and addressed through
``rec_addr`` / ``rec_len`` exactly as the store lays them out; the last,
partially filled page of a sequence is a raw record, as an open block's
staging record is.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from oracle import oracle

T = 128
D = 128
DENSE = 22528


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> BF16 bit patterns, round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def kv_bits(rng: np.random.Generator, shape: tuple, outlier: float, scale: np.ndarray | None = None) -> np.ndarray:
    """BF16 bits of N(0,1) x per-channel lognormal scale (channels = last axis)."""
    if scale is None:
        scale = channel_scale(rng, shape[-1], outlier)
    return bf16_bits(rng.standard_normal(shape) * scale)


def channel_scale(rng: np.random.Generator, dim: int, outlier: float) -> np.ndarray:
    scale = rng.lognormal(0.0, 0.5, dim)
    scale[rng.random(dim) < outlier] *= 8.0
    return scale


@dataclass
class DecodeCase:
    heads: int
    group: int
    lens: np.ndarray  # int32 [B]
    block_table: np.ndarray  # int32 [B, width]
    q_bits: np.ndarray  # uint16 [B, H*G, 128]
    kv: np.ndarray  # uint16 [NB, 2, T, H, D] (physical blocks, token-major)
    tables: np.ndarray  # uint8 [2, H, 22]
    recs: np.ndarray  # uint8 arena
    rec_off: np.ndarray  # int64 [NB, 2, H] byte offsets into recs
    rec_len: np.ndarray  # int32 [NB, 2, H]
    scale: float


def make_tables(rng: np.random.Generator, heads: int, outlier: float, scales: np.ndarray) -> np.ndarray:
    """Calibrated [2, H, 22] tables from a seeded dump [64, 1, 2, 128, H, 128]."""
    dump = np.empty((64, 1, 2, T, heads, D), np.uint16)
    for kv in range(2):
        for h in range(heads):
            dump[:, 0, kv, :, h, :] = kv_bits(rng, (64, T, D), outlier, scales[kv, h])
    return oracle.calibrate(dump)[0]


def decode_case(seed: int, batch: int, heads: int, group: int, lens, outlier: float = 0.02,
                raw_tail: bool = True, extra_blocks: int = 2, poke=None, scales=None, tables=None) -> DecodeCase:
    """A seeded decode case; ``poke(kv, block_table)`` may edit the token-major
    KV bits [NB, 2, T, H, D] before the records are built.  ``scales``
    ([2, H, 128]) and ``tables`` ([2, H, 22]) replace the drawn channel scales
    and the calibrated tables."""
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int32)
    assert lens.size == batch
    if scales is None:
        scales = np.stack([[channel_scale(rng, D, outlier) for _ in range(heads)] for _ in range(2)])
    if tables is None:
        tables = make_tables(rng, heads, outlier, scales)
    pages = [(int(n) + T - 1) // T for n in lens]
    nb = sum(pages) + extra_blocks
    perm = rng.permutation(nb).astype(np.int32)
    width = max(1, max(pages))
    bt = np.zeros((batch, width), np.int32)
    used = 0
    open_block = np.zeros(nb, bool)
    for b, p in enumerate(pages):
        bt[b, :p] = perm[used : used + p]
        if p and lens[b] % T and raw_tail:
            open_block[perm[used + p - 1]] = True
        used += p
    kv = np.empty((nb, 2, T, heads, D), np.uint16)
    for k in range(2):
        for h in range(heads):
            kv[:, k, :, h, :] = kv_bits(rng, (nb, T, D), outlier, scales[k, h])
    if poke is not None:
        poke(kv, bt)
    # records, 16-byte aligned, in one arena
    chunks = []
    rec_off = np.zeros((nb, 2, heads), np.int64)
    rec_len = np.zeros((nb, 2, heads), np.int32)
    off = 0
    for blk in range(nb):
        for k in range(2):
            for h in range(heads):
                tok_major = kv[blk, k, :, h, :]
                if open_block[blk]:
                    r = oracle.raw_record(tok_major, k)
                else:
                    r = oracle.encode_record(tok_major, tables[k, h], k)
                rec_off[blk, k, h] = off
                rec_len[blk, k, h] = len(r) - DENSE
                chunks.append(np.frombuffer(r, np.uint8))
                off += len(r)
    recs = np.concatenate(chunks)
    q = bf16_bits(rng.standard_normal((batch, heads * group, D)))
    return DecodeCase(heads, group, lens, bt, q, kv, tables, recs, rec_off, rec_len, D ** -0.5)


def reference_attention(case: DecodeCase) -> np.ndarray:
    """float64 softmax(q k^T * scale) v over the token-major KV, float32 out."""
    B = case.lens.size
    H, G = case.heads, case.group
    out = np.zeros((B, H * G, D), np.float32)
    q = bits_to_f32(case.q_bits).astype(np.float64)
    for b in range(B):
        n = int(case.lens[b])
        if n == 0:
            continue
        pages = (n + T - 1) // T
        blks = case.block_table[b, :pages]
        for h in range(H):
            k = bits_to_f32(case.kv[blks, 0, :, h, :]).reshape(-1, D)[:n].astype(np.float64)
            v = bits_to_f32(case.kv[blks, 1, :, h, :]).reshape(-1, D)[:n].astype(np.float64)
            qh = q[b, h * G : (h + 1) * G]
            with np.errstate(invalid="ignore", over="ignore"):
                # NaN / Inf bits propagate as IEEE arithmetic does
                s = qh @ k.T * case.scale
                s -= s.max(axis=1, keepdims=True)
                p = np.exp(s)
                p /= p.sum(axis=1, keepdims=True)
                out[b, h * G : (h + 1) * G] = (p @ v).astype(np.float32)
    return out


def oracle_decode(case: DecodeCase, threads: int = 0) -> np.ndarray:
    """The CPU oracle's fp32 paged attention (decodes every record itself)."""
    return oracle.paged_attention(case.q_bits, case.heads, case.recs, case.rec_off, case.rec_len,
                                  case.tables, case.block_table, case.lens, case.scale, threads)


def upload(case: DecodeCase, device=None):
    """Device tensors of a case: (q, rec_addr, rec_len, plut, slut, bt, lens, arena)."""
    import torch

    from fragpack_amd.compression.attn_tables import device_tables

    dev = device or torch.device("cuda", torch.cuda.current_device())
    arena = torch.from_numpy(case.recs).to(dev)
    rec_addr = (torch.from_numpy(case.rec_off) + arena.data_ptr()).to(dev)
    rec_len = torch.from_numpy(case.rec_len).to(dev)
    dt = device_tables(case.tables[None], dev)
    q = torch.from_numpy(case.q_bits.view(np.int16)).to(dev).view(torch.bfloat16)
    bt = torch.from_numpy(case.block_table).to(dev)
    lens = torch.from_numpy(case.lens).to(dev)
    return q, rec_addr, rec_len, dt.plut[0], dt.slut[0], bt, lens, arena


def run_gpu_decode(case: DecodeCase, units: int | None = None, repeat: int = 1) -> np.ndarray:
    import torch

    from fragpack_amd.ops.fused_attn_decode import RecordTables, decode_attention, decode_units, workspace_elems

    q, rec_addr, rec_len, plut, slut, bt, lens, arena = upload(case)
    B = case.lens.size
    if units is None:
        units = decode_units(B, case.heads, torch.cuda.get_device_properties(q.device).multi_processor_count)
    opart, ml, plan = workspace_elems(case.heads, units)
    ws = (torch.empty(opart, device=q.device), torch.empty(ml, device=q.device),
          torch.empty(plan, dtype=torch.int32, device=q.device))
    out = torch.full_like(q, float("nan"))
    tabs = RecordTables(rec_addr, rec_len, plut, slut)
    for i in range(repeat):
        decode_attention(q, tabs, bt, lens, case.scale, units, out, ws, i == 0)
    torch.cuda.synchronize()
    del arena
    return out.float().cpu().numpy()


def config0_case(workdir, seed: int = 0) -> DecodeCase:
    """1 sequence, 4 KV heads, GQA 8, 1000 tokens (7 coded
    blocks + a 104-token raw tail), 2% outlier channels; the tables come from
    the repository's calibration CLI (``python -m
    fragpack_amd.compression.attn_tables dump.npy tables.npz``) run on a seeded
    uint16 dump [64, 1, 2, 128, 4, 128] drawn from the same distribution."""
    import subprocess
    import sys
    from pathlib import Path

    H = 4
    rng = np.random.default_rng(seed)
    scales = np.stack([[channel_scale(rng, D, 0.02) for _ in range(H)] for _ in range(2)])
    dump = np.empty((64, 1, 2, T, H, D), np.uint16)
    for kv in range(2):
        for h in range(H):
            dump[:, 0, kv, :, h, :] = kv_bits(rng, (64, T, D), 0.02, scales[kv, h])
    workdir = Path(workdir)
    np.save(workdir / "dump.npy", dump)
    root = Path(__file__).resolve().parent.parent
    subprocess.run([sys.executable, "-m", "fragpack_amd.compression.attn_tables", str(workdir / "dump.npy"),
                    str(workdir / "tables.npz")], check=True, cwd=root, capture_output=True)
    with np.load(workdir / "tables.npz", allow_pickle=False) as f:
        tables = f["table"]
    assert tables.shape == (1, 2, H, 22)
    return decode_case(seed + 1, batch=1, heads=H, group=8, lens=[1000], scales=scales, tables=tables[0])
