"""Decode attention over a plain paged BF16 KV cache: the uncompressed
baseline the FragPack decode path is measured against.

Reference counterpart: the FA3 arm of the reference's step benchmark
(benchmarks/fragpack_step_bench.py:205-284, ``flash_attn_with_kvcache`` over
a token-major paged cache ``[blocks, 128, H, 128]``).  Here it is a
hand-written gfx950 kernel (``paged_decode_kernel``, C entry
``fp_paged_decode``): split-KV over the device's resident workgroups, K
straight into MFMA operands, V through LDS transposing reads, fp32 partials
merged by the last split of each (sequence, head).
"""

from __future__ import annotations

import torch

from fragpack_amd.ops.fragpack_ext import extension


def paged_splits(batch: int, kv_heads: int, max_seq_len: int) -> int:
    """Splits per (sequence, KV head) that fill the device (depends only on
    the shape, so a captured launch keeps it)."""
    return extension().paged_decode_splits(batch, kv_heads, max_seq_len)


def set_streaming_loads(on: bool) -> None:
    """Page loads with the non-temporal policy (default) or plain; which is
    faster depends on the shape.  Process-wide."""
    extension().paged_set_streaming(on)


def paged_workspace(batch: int, kv_heads: int, splits: int, device) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``(opart, ml, counters)`` for :func:`paged_decode_attention`; the
    counters start at zero and every completed call leaves them at zero."""
    rows = batch * kv_heads * splits * 8
    return (torch.empty(rows * 128, dtype=torch.float32, device=device),
            torch.empty(rows * 2, dtype=torch.float32, device=device),
            torch.zeros(batch * kv_heads, dtype=torch.int32, device=device))


def paged_decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, block_table: torch.Tensor,
                           seq_lens: torch.Tensor, max_seq_len: int, scale: float, out: torch.Tensor,
                           workspace: tuple[torch.Tensor, torch.Tensor, torch.Tensor], splits: int) -> None:
    """One query token per sequence over a paged BF16 cache.

    Args:
        q: BF16 ``[B, H * G, 128]`` (G in 1, 2, 4, 8).
        k_cache, v_cache: BF16 ``[blocks, 128, H, 128]``.
        block_table: int32 ``[B, >= ceil(max_seq_len / 128)]``.
        seq_lens: int32 ``[B]`` (each <= ``max_seq_len``; 0 gives a zero row).
        max_seq_len: Bound on ``seq_lens``.
        scale: Softmax scale.
        out: BF16 ``[B, H * G, 128]``.
        workspace: From :func:`paged_workspace` with the same ``splits``.
        splits: From :func:`paged_splits`.
    """
    opart, ml, counters = workspace
    extension().paged_decode(q, k_cache, v_cache, block_table, seq_lens, max_seq_len, splits, opart, ml, counters,
                             out, scale)


__all__ = ["paged_decode_attention", "paged_splits", "paged_workspace", "set_streaming_loads"]
