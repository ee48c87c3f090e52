"""GPU-side synthetic workloads of the BASELINE configs, shared by bench.py
and the full-size GPU tests.

KV = N(0,1) x a per-channel scale ~ lognormal(0, 0.5), a fraction of channels
x8 (outliers), optionally a share of values replaced by Student-t(2) x 16
(config 3's heavy tail), rounded to BF16.  Tables are calibrated with the
package's calibration (attn_tables.calibrate) from a seeded
[64, 1, 2, 128, H, 128] dump drawn the same way.  Blocks are written and
encoded through the GPU block store (HbmKvStore), as a serving engine would.
"""

from __future__ import annotations

import math

import numpy as np

T = 128
D = 128


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> BF16 bit patterns, round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def channel_scales(rng, heads: int, outlier: float) -> np.ndarray:
    """[2, H, 128] per-channel scales: lognormal(0, 0.5), outliers x8."""
    s = rng.lognormal(0.0, 0.5, (2, heads, D))
    s[rng.random((2, heads, D)) < outlier] *= 8.0
    return s


def calibrated_tables(rng, heads: int, scales: np.ndarray):
    from fragpack_amd.compression.attn_tables import calibrate

    dump = np.empty((64, 1, 2, T, heads, D), np.uint16)
    for kv in range(2):
        for h in range(heads):
            dump[:, 0, kv, :, h, :] = bf16_bits(rng.standard_normal((64, T, D)) * scales[kv, h])
    return calibrate(dump)  # [1, 2, H, 22]


def gen_kv(torch, gen, n_tok: int, heads: int, scales_t, heavy: float = 0.0):
    """BF16 [2, n_tok, H, 128] on the GPU; ``heavy`` of the values replaced by
    Student-t(2) x 16 (config 3)."""
    x = torch.randn((2, n_tok, heads, D), generator=gen, device="cuda") * scales_t[:, None]
    if heavy > 0:
        z = torch.randn((2, n_tok, heads, D), generator=gen, device="cuda")
        chi = torch.randn((2, n_tok, heads, D, 2), generator=gen, device="cuda").pow(2).sum(-1)
        t2 = z / torch.sqrt(chi / 2) * 16
        pick = torch.rand((2, n_tok, heads, D), generator=gen, device="cuda") < heavy
        x = torch.where(pick, t2, x)
    return x.to(torch.bfloat16)


def build_store(torch, heads: int, n_blocks: int, tables, gen, scales_t, fill_blocks: int, heavy: float = 0.0,
                overflow: int = 8192, keep_kv: bool = False, layers: int = 1):
    """A store of ``layers`` layers whose blocks 0..n_blocks-1 are written and
    encoded, each layer with KV of its own (same distribution and tables);
    ``keep_kv`` returns layer 0's KV."""
    from fragpack_amd.compression.attn_tables import device_tables
    from fragpack_amd.ops.hbm_kv import HbmKvStore, page_bytes

    dev = torch.device("cuda")
    arenas = [torch.empty((n_blocks, page_bytes(heads)), dtype=torch.uint8, device=dev) for _ in range(layers)]
    tables = np.repeat(np.asarray(tables)[:1], layers, axis=0)
    store = HbmKvStore(arenas, heads, device_tables(tables, dev), max_tokens=fill_blocks * T, staging_slots=1,
                       overflow_records=overflow)
    kept = []
    no_live = np.zeros(0, np.int32)
    for b0 in range(0, n_blocks, fill_blocks):
        n = min(fill_blocks, n_blocks - b0)
        slots = (torch.arange(b0, b0 + n, device=dev)[:, None] * T + torch.arange(T, device=dev)).reshape(-1)
        store.prepare(slots, slots.numel(), no_live)
        for layer in range(layers):
            kv = gen_kv(torch, gen, n * T, heads, scales_t, heavy)
            store.write(layer, kv[0], kv[1], slots)
            store.encode(layer, n)
            if keep_kv and layer == 0:
                kept.append(kv)
        store.commit()
    torch.cuda.synchronize()
    return store, (arenas[0] if layers == 1 else arenas), (torch.cat(kept, dim=1) if keep_kv else None)


def reference_decode(torch, q, kv, block_table, lens, heads, group, scale):
    """fp32 torch attention over token-major KV [2, NB*128, H, 128]."""
    out = torch.zeros(q.shape, dtype=torch.float32, device=q.device)
    kvf = kv.float().view(2, -1, T, heads, D)
    for b in range(q.shape[0]):
        n = int(lens[b])
        pages = block_table[b, : math.ceil(n / T)].long().to(q.device)
        k = kvf[0, pages].reshape(-1, heads, D)[:n]
        v = kvf[1, pages].reshape(-1, heads, D)[:n]
        qb = q[b].float().view(heads, group, D)
        s = torch.einsum("hgd,thd->hgt", qb, k) * scale
        out[b] = torch.einsum("hgt,thd->hgd", s.softmax(-1), v).reshape(heads * group, D)
    return out
