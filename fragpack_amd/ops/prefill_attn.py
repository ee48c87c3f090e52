"""Causal varlen prefill attention over the paged BF16 workspace.

The reference backend runs prefill through vLLM's FlashAttention on the
workspace that ``HbmKvStore.gather`` fills
(fragpack/integrations/vllm/backend.py:560-575)::

    flash_attn_varlen_func(q=query[tok0:tok1], k=wk, v=wv, out=output[tok0:tok1],
                           cu_seqlens_q=..., max_seqlen_q=..., seqused_k=..., max_seqlen_k=...,
                           softmax_scale=scale, causal=True, block_table=..., fa_version=...)

Here the same call runs a hand-written gfx950 MFMA kernel
(``fp_prefill_attention``).  Semantics follow FlashAttention's varlen
contract for a paged KV cache: sequence b has ``cu_seqlens_q[b+1] -
cu_seqlens_q[b]`` queries, which are its last positions, over
``seqused_k[b]`` keys (causal mask aligned bottom-right); key j of b is row
``j % 128`` of workspace page ``block_table[b, j // 128]``.
"""

from __future__ import annotations

import torch

from .fragpack_ext import extension


def flash_attn_varlen_func(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    out: torch.Tensor | None = None,
    cu_seqlens_q: torch.Tensor | None = None,
    max_seqlen_q: int = 0,
    seqused_k: torch.Tensor | None = None,
    max_seqlen_k: int = 0,
    softmax_scale: float | None = None,
    causal: bool = True,
    block_table: torch.Tensor | None = None,
    fa_version: int | None = None,
) -> torch.Tensor:
    """Paged varlen attention, keyword-compatible with the backend's call.

    Args:
        q: BF16 ``[Nq, Hq, 128]`` queries (token rows may be strided).
        k, v: BF16 ``[pages, 128, H, 128]`` workspace; ``Hq`` a multiple of
            ``H`` by 1, 2, 4 or 8.
        out: BF16 output like ``q`` (allocated when None).
        cu_seqlens_q: int32 ``[B + 1]`` query offsets.
        max_seqlen_q: Largest query count (sizes the launch grid).
        seqused_k: int32 ``[B]`` key counts.
        max_seqlen_k: Largest key count.
        softmax_scale: Defaults to ``128 ** -0.5``.
        causal: Bottom-right aligned causal mask.
        block_table: int32 ``[B, pages]`` workspace pages per sequence.
        fa_version: Accepted for call compatibility; ignored.

    Returns:
        ``out``.

    Raises:
        RuntimeError: On shape / dtype errors or a missing library.

    Async/thread-safety:
        Enqueues on the current stream; not synchronized.
    """
    del fa_version
    if cu_seqlens_q is None or seqused_k is None or block_table is None:
        raise ValueError("cu_seqlens_q, seqused_k and block_table are required (paged varlen form)")
    if out is None:
        out = torch.empty_like(q)
    scale = softmax_scale if softmax_scale is not None else q.size(-1) ** -0.5
    extension().prefill_attention(q, k, v, out, cu_seqlens_q, seqused_k, block_table, max_seqlen_q, max_seqlen_k,
                                  scale, causal)
    return out


__all__ = ["flash_attn_varlen_func"]
