"""Split-KV decode attention straight from FragPack KV records (MI355X).

Reference: fragpack/ops/fused_attn_decode.py:41-219 (RecordTables,
decode_units, workspace_elems, decode_attention, _launch) and
fragpack/ops/fused_attn_decode.cu.

One work unit handles a chunk of pages of one (sequence, KV head) pair for
all query heads of the group, with an online softmax; a small combine kernel
merges each sequence's chunks (here fused into the same kernel: the last
finished chunk of a (sequence, head) merges them).  On gfx950 a unit is one 256-thread workgroup:
its four wavefronts decode the four slabs of each record in parallel, straight into MFMA operands
(``S^T = K Q^T`` and ``O^T += V^T P^T`` with v_mfma_f32_16x16x32_bf16, the
group's query heads on the N side), so units never synchronise with each
other.  A one-workgroup planner picks the chunk size on device once per step
(``replan``) and every layer reuses it; the launch shape depends only on the
batch size and ``units``, so the call is HIP-graph safe.

Records are located through ``rec_addr[P, 2, H]`` (absolute device
addresses) and ``rec_len[P, 2, H]`` (bytes past the dense part; raw records
use ``RAW_VAR_LEN``).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from fragpack_amd.logging import init_logger
from fragpack_amd.ops.fragpack_ext import extension

logger = init_logger(__name__)

GQA = 8
# Split capacity per compute unit: a unit is one 256-thread workgroup and
# the decode kernel keeps 3 of them resident per CU (3 waves per SIMD).
UNITS_PER_CU = 3
# Waves of split capacity in decode_units: the planner may spread a step over
# up to this many rounds of resident workgroups.
SPLIT_WAVES = 4


@dataclass(frozen=True)
class RecordTables:
    """One layer's record tables for :func:`decode_attention`.

    Attributes:
        rec_addr: int64 ``[P, 2, H]`` record device addresses.
        rec_len: int32 ``[P, 2, H]`` record bytes minus ``DENSE_BYTES``.
        plut: int32 ``[2, H, 2]`` primary tables.
        slut: uint8 ``[2, H, 16]`` extended tables.
    """

    rec_addr: torch.Tensor
    rec_len: torch.Tensor
    plut: torch.Tensor
    slut: torch.Tensor


def decode_units(batch: int, kv_heads: int, num_sms: int) -> int:
    """Work-unit capacity per KV head of a decode launch.

    One unit per sequence plus ``SPLIT_WAVES`` waves of split capacity minus
    one (the reference has one wave, fused_attn_decode.py:58-85); a "wave"
    is the workgroups the device runs at once per KV head, ``UNITS_PER_CU``
    per compute unit.  The planner picks how many of them to use.  Depends
    only on the (padded) batch size, so the launch shape is fixed under graph
    capture.

    Args:
        batch: Number of sequences (padded batch size under graphs).
        kv_heads: KV heads per sequence.
        num_sms: Compute-unit count (``multi_processor_count``; 256 on MI355X).

    Returns:
        Unit count, at least ``batch``.
    """
    wave = max(1, (UNITS_PER_CU * num_sms) // max(1, kv_heads))
    return batch + SPLIT_WAVES * wave - 1


def workspace_elems(kv_heads: int, units: int) -> tuple[int, int, int]:
    """Element counts of the ``(opart, ml, plan)`` workspace (float, float, int32).

    ``plan`` holds the reference's ``2 + 4 * units`` planner words (padded to
    8), an 8-int descriptor per unit and ``units * kv_heads`` counters for the
    merge fused into the attention kernel.  The counters are the buffer's last
    words, so a workspace made for ``units`` serves calls with fewer units.
    """
    rows = kv_heads * units * GQA
    return rows * 128, rows * 2, ((2 + 4 * units + 7) & ~7) + 8 * units + units * kv_heads


def decode_attention(
    q: torch.Tensor,
    tables: RecordTables,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    scale: float,
    units: int,
    out: torch.Tensor,
    workspace: tuple[torch.Tensor, torch.Tensor, torch.Tensor],
    replan: bool,
    append: tuple | None = None,
) -> None:
    """Split-KV decode attention for one query token per sequence.

    Args:
        q: BF16 ``[B, H * G, 128]`` queries (rows may be strided); G in 1, 2, 4, 8.
        tables: Record tables of this layer.
        block_table: int32 ``[B, max_pages]`` page ids (rows may be strided).
        seq_lens: int32 ``[B]`` context lengths; 0 yields a zero output row.
        scale: Softmax scale.
        units: Work-unit capacity per KV head, at least ``B`` (e.g. from
            :func:`decode_units`).
        out: BF16 ``[B, H * G, 128]`` output (rows may be strided).
        workspace: ``(opart, ml, plan)`` sized by :func:`workspace_elems`.
        replan: Recompute the work plan from ``seq_lens`` and ``units``; later
            layers of the same step may pass False (the workspace must then
            hold a plan made for the same ``units``, batch and KV heads).
        append: None, or ``(new_k, new_v, slot_mapping, staging, scratch)``:
            write each sequence's new token (BF16 ``[B, H, 128]``, int64
            slot, negative = padding; the sequence's last position) into its
            open block's raw record first, in the same launch -- a
            decode-only step's ``HbmKvStore.write`` fused into attention
            (this build's addition; the reference writes with a launch of its
            own).  ``staging`` / ``scratch`` are the store's tensors; records
            outside them are never written.

    Raises:
        ValueError: If the query group does not divide ``GQA``.
        RuntimeError: If ``replan`` is False and no earlier call planned this
            workspace for the same units, batch and KV heads.

    Async/thread-safety:
        Enqueues on the current stream; not synchronized.  Unlike the
        reference, smaller groups run natively (no padded copies).
    """
    kv_heads = tables.rec_addr.shape[2]
    group = q.shape[1] // kv_heads
    if group * kv_heads != q.shape[1] or GQA % group:
        raise ValueError(f"query heads {q.shape[1]} need a group dividing {GQA}")
    _launch(q, tables, block_table, seq_lens, scale, units, out, workspace, replan, group, append)


def _launch(q, tables, block_table, seq_lens, scale, units, out, workspace, replan, group=GQA, append=None) -> None:
    extension().fused_decode(
        q,
        tables.rec_addr,
        tables.rec_len,
        tables.plut,
        tables.slut,
        block_table,
        seq_lens,
        workspace[0],
        workspace[1],
        workspace[2],
        out,
        units,
        replan,
        scale,
        group,
        append,
    )


__all__ = ["GQA", "RecordTables", "decode_attention", "decode_units", "workspace_elems"]
