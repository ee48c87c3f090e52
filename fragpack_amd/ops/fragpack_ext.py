"""Loader of the gfx950 FragPack library and its tensor-level entry points.

Reference: fragpack/ops/fragpack_ext.py:12-31 (JIT-built pybind module
``fragpack_cuda``) and fragpack/ops/fragpack_ext.cpp:5-66 (its 8 functions).
Here the native side is a plain C ABI (include/fragpack_hip.h) in
``fragpack_amd/_lib/libfragpack_hip.so``, built ahead of time by
``fragpack_amd.csrc.build`` for gfx950.  :func:`extension` returns an object
with the reference module's 8 functions, same names, argument order and
meaning; each validates its tensors like the reference's ``TORCH_CHECK``s
(``RuntimeError``), then calls the C entry point with raw device pointers on
the current stream.

There is no fallback: a missing library or a CPU tensor raises.
"""

from __future__ import annotations

import ctypes
import functools
from pathlib import Path

import torch

import os

# FRAGPACK_LIB overrides the library path (e.g. to compare builds).
LIB_PATH = Path(os.environ.get("FRAGPACK_LIB", Path(__file__).resolve().parent.parent / "_lib" / "libfragpack_hip.so"))

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f64 = ctypes.c_double


class FpStore(ctypes.Structure):
    """``fp_store_t``: the store's 13 state tensors plus geometry."""

    _fields_ = [
        ("counters", _p),
        ("wslot", _p),
        ("tags", _p),
        ("free_stack", _p),
        ("ovf_bits", _p),
        ("claim_list", _p),
        ("close_list", _p),
        ("rec_addr", _p),
        ("rec_len", _p),
        ("staging", _p),
        ("scratch", _p),
        ("overflow", _p),
        ("fill", _p),
        ("num_layers", _i64),
        ("num_blocks", _i64),
        ("kv_heads", _i64),
        ("staging_slots", _i64),
        ("scratch_slots", _i64),
        ("ovf_words", _i64),
        ("list_cap", _i64),
        ("overflow_records", _i64),
    ]


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _dev(t: torch.Tensor, name: str) -> int:
    _check(t.is_cuda, f"{name} must be a GPU tensor")
    return t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _store_desc(state: tuple[torch.Tensor, ...]) -> FpStore:
    (counters, wslot, tags, free_stack, ovf_bits, claim_list, close_list, rec_addr, rec_len, staging, scratch,
     overflow, fill) = state
    _check(rec_addr.dim() == 4 and rec_addr.dtype == torch.int64, "rec_addr must be int64 [L, NB, 2, H]")
    _check(rec_len.shape == rec_addr.shape and rec_len.dtype == torch.int32, "rec_len must be int32 [L, NB, 2, H]")
    _check(counters.dtype == torch.int32 and counters.numel() >= 16, "counters must be int32 [16]")
    _check(claim_list.numel() == close_list.numel(), "block lists must match")
    L, NB, _, H = rec_addr.shape
    d = FpStore()
    for name, t in zip(
        ("counters", "wslot", "tags", "free_stack", "ovf_bits", "claim_list", "close_list", "rec_addr",
         "rec_len", "staging", "scratch", "overflow", "fill"),
        state,
    ):
        setattr(d, name, _dev(t, name) if t.numel() else 0)
    d.num_layers, d.num_blocks, d.kv_heads = L, NB, H
    d.staging_slots = free_stack.numel()
    d.scratch_slots = scratch.numel() // (2 * H * 32768)
    d.ovf_words = ovf_bits.numel()
    d.list_cap = claim_list.numel() // 2
    d.overflow_records = overflow.numel() // 32768
    return d


class Extension:
    """The reference module's functions over the C ABI."""

    def __init__(self, lib: ctypes.CDLL) -> None:
        self._lib = lib
        sp = ctypes.POINTER(FpStore)
        sigs = {
            "fp_fused_decode": [_p, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _i64, _p, _p, _i64, _p, _i64, _p,
                                _i64, _p, _i64, _i64, _i32, _f64, _p],
            "fp_fused_decode_append": [_p, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _i64, _p, _p, _i64, _p, _i64,
                                       _p, _i64, _p, _i64, _i64, _i32, _f64, _p, _i64, _i64, _p, _i64, _i64, _p,
                                       _p, _i64, _p, _i64, _p],
            "fp_hbm_prepare": [sp, _p, _i64, _p, _i64, _i64, _p],
            "fp_hbm_write": [sp, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p],
            "fp_hbm_encode": [sp, _p, _i64, _i64, _i64, _i64, _i64, _p],
            "fp_hbm_encode_ordered": [sp, _p, _i64, _i64, _i64, _i64, _i64, _p],
            "fp_hbm_write_encode": [sp, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64,
                                    _i32, _p],
            "fp_hbm_commit": [sp, _p],
            "fp_hbm_gather": [_p, _i64, _p, _p, _p, _p, _p, _p, _i64, _i64, _p],
            "fp_stream_probe": [_p, _p, _i64, _i64, _i64, _i64, _p],
            "fp_hbm_export": [_p, _i64, _p, _p, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _p],
            "fp_hbm_import": [sp, _p, _i64, _p, _p, _i64, _p, _p, _p, _i64, _p],
            "fp_encode_records": [_p, _i64, _p, _p, _p, _i64, _p, _p, _p],
            "fp_decode_records": [_p, _p, _i64, _p, _p, _p, _p, _i64, _p, _p],
            "fp_paged_decode": [_p, _i64, _i64, _i64, _i64, _p, _p, _i64, _p, _i64, _p, _i64, _i64, _p, _i64, _p,
                                _i64, _p, _i64, _p, _i64, _f64, _p],
            "fp_paged_decode_splits": [_i64, _i64, _i64],
            "fp_paged_set_streaming": [_i32],
            "fp_prefill_attention": [_p, _i64, _p, _p, _i64, _i64, _i64, _p, _p, _p, _i64, _i64, _i64, _i64, _f64,
                                     _i32, _p, _i64, _p],
        }
        for name, args in sigs.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = _i32
        self._fused = lib.fp_fused_decode
        self._fused_append = lib.fp_fused_decode_append
        lib.fp_last_error.restype = ctypes.c_char_p
        lib.fp_abi_version.restype = _i32

    def _call(self, name: str, *args) -> None:
        if getattr(self._lib, name)(*args) != 0:
            raise RuntimeError(f"{name}: {self._lib.fp_last_error().decode()}")

    # -- fused_decode (fragpack_ext.cpp:5-9, fused_attn_decode.cu:429-478) --
    def fused_decode(self, q, rec_addr, rec_len, plut, slut, block_table, seq_lens, opart, ml, plan, out,
                     units: int, replan: bool, scale: float, group: int = 8, append=None) -> None:
        """``append``: None, or ``(new_k, new_v, slot_mapping, staging,
        scratch)`` -- each sequence's new token (BF16 ``[B, H, 128]``, int64
        slot, negative = padding) is written into its open block's raw record
        inside the attention launch (the store's ``write`` for a decode-only
        step); records outside the ``staging`` / ``scratch`` tensors are left
        alone."""
        # one tuple read per tensor property: this runs once per decode layer
        qsh, qst, ost, bst = q.shape, q.stride(), out.stride(), block_table.stride()
        bf16, i32 = torch.bfloat16, torch.int32
        _check(len(qsh) == 3 and qsh[2] == 128 and qst[2] == 1 and qst[1] == 128 and qst[0] % 8 == 0
               and q.dtype == bf16, "q must be [B, H, 128] with contiguous heads")
        _check(len(ost) == 3 and ost[2] == 1 and ost[1] == 128 and out.dtype == bf16 and out.shape[1] == qsh[1],
               "out must be [B, H, 128] with contiguous heads")
        _check(block_table.dtype == i32 and bst[1] == 1, "block_table rows must be contiguous")
        _check(seq_lens.dtype == i32, "seq_lens must be int32")
        _check(rec_addr.dtype == torch.int64 and rec_len.dtype == i32, "record tables must be int64 / int32")
        _check(plan.dtype == i32, "decode plan must be int32 with 2 + 4 * units + units * kv_heads elements")
        _check(opart.dtype == torch.float32 and ml.dtype == torch.float32, "decode workspace must be float32")
        B = qsh[0]
        kvh = qsh[1] // group
        _check(kvh * group == qsh[1], "query heads must be a multiple of the group")
        if B == 0:
            return
        # A reusing call reads the unit descriptors an earlier planning call
        # wrote: without one (same units, batch and heads) they are whatever
        # the buffer holds, and the kernel would follow them anywhere.
        _check(replan or getattr(plan, "_fp_plan_key", None) == (units, B, kvh),
               "replan=False reuses the plan of an earlier call on this workspace with the same units, batch "
               "and kv heads: plan first")
        # Replanning runs inside the attention kernel (no plan launch) once a
        # call has left this workspace's merge counters at zero; the first
        # call on a workspace launches the planner, which zeroes them.
        mode = 0
        if replan:
            mode = 2 if getattr(plan, "_fp_counters_zeroed", False) else 1
            # 3: the kernel may read the whole (small) block table -- only if
            # its storage holds B rows of stride entries from the view's start
            if mode == 2 and B * bst[0] <= 1024 and \
                    block_table.untyped_storage().nbytes() >= (block_table.storage_offset() + B * bst[0]) * 4:
                mode = 3
        args = (
            _dev(q, "q"), qst[0], B, kvh, group, _dev(rec_addr, "rec_addr"), _dev(rec_len, "rec_len"),
            _dev(plut, "plut"), _dev(slut, "slut"), _dev(block_table, "block_table"), bst[0],
            _dev(seq_lens, "seq_lens"), _dev(opart, "opart"), opart.numel(), _dev(ml, "ml"), ml.numel(),
            _dev(plan, "plan"), plan.numel(), _dev(out, "out"), ost[0], units, mode, scale,
        )
        if append is None:
            if self._fused(*args, torch.cuda.current_stream().cuda_stream):
                raise RuntimeError(f"fp_fused_decode: {self._lib.fp_last_error().decode()}")
        else:
            raise NotImplementedError("the fused append (fp_fused_decode_append) is disabled: its first GPU run "
                                      "faulted and the cause is not yet found; write with HbmKvStore.write")
        if mode:
            plan._fp_counters_zeroed = True
            plan._fp_plan_key = (units, B, kvh)

    # -- store (fragpack_ext.cpp:11-39, hbm_kv.cu:669-734) --
    def hbm_prepare(self, *args) -> None:
        state, (slot_mapping, n_tok, live, n_live, step) = args[:13], args[13:]
        _check(slot_mapping.dtype == torch.int64, "slot_mapping must be int64")
        d = _store_desc(state)
        _check(2 * int(n_tok) <= state[5].numel(), "block lists too small")
        self._call("fp_hbm_prepare", ctypes.byref(d), _dev(slot_mapping, "slot_mapping"), int(n_tok),
                   _dev(live, "live"), int(n_live), int(step), _stream(slot_mapping))

    def hbm_write(self, *args) -> None:
        state, (key, value, slot_mapping, layer) = args[:13], args[13:]
        n = key.size(0)
        if n == 0:
            return
        _check(key.stride(2) == 1 and value.stride(2) == 1, "head dim must be contiguous")
        _check(key.dtype == torch.bfloat16 and value.dtype == torch.bfloat16, "K / V must be BF16")
        _check(slot_mapping.dtype == torch.int64 and slot_mapping.numel() >= n, "slot_mapping must be int64 [N]")
        d = _store_desc(state)
        _check(key.size(1) == d.kv_heads and key.size(2) == 128 and value.shape == key.shape,
               "K / V must be [N, H, 128]")
        self._call("fp_hbm_write", ctypes.byref(d), _dev(key, "key"), key.stride(0), key.stride(1),
                   _dev(value, "value"), value.stride(0), value.stride(1), _dev(slot_mapping, "slot_mapping"), n,
                   int(layer), _stream(key))

    def hbm_encode(self, *args, ordered: bool = False) -> None:
        """``ordered``: place each block's records in (kv, head) order
        (fp_hbm_encode_ordered) instead of by arrival."""
        state, (rank_of, layer, arena, page_bytes, max_close) = args[:13], args[13:]
        if int(max_close) == 0:
            return
        d = _store_desc(state)
        _check(2 * int(max_close) <= state[6].numel(), "close list too small")
        _check(rank_of.numel() == d.num_layers * 2 * d.kv_heads * 256, "rank_of must hold every layer")
        _check(int(page_bytes) % 16 == 0 and int(page_bytes) < (1 << 31), "bad arena page size")
        self._call("fp_hbm_encode_ordered" if ordered else "fp_hbm_encode", ctypes.byref(d), _dev(rank_of, "rank_of"),
                   rank_of.numel(), int(layer), int(arena), int(page_bytes), int(max_close), _stream(rank_of))

    def hbm_write_encode(self, *args, ordered: bool = False) -> None:
        """hbm_write then hbm_encode of one layer in one launch
        (fp_hbm_write_encode); same arguments as the two calls."""
        state, (key, value, slot_mapping, rank_of, layer, arena, page_bytes, max_close) = args[:13], args[13:]
        n = key.size(0)
        if int(max_close) == 0:
            self.hbm_write(*state, key, value, slot_mapping, layer)
            return
        if n == 0:
            self.hbm_encode(*state, rank_of, layer, arena, page_bytes, max_close, ordered=ordered)
            return
        _check(key.stride(2) == 1 and value.stride(2) == 1, "head dim must be contiguous")
        _check(key.dtype == torch.bfloat16 and value.dtype == torch.bfloat16, "K / V must be BF16")
        _check(slot_mapping.dtype == torch.int64 and slot_mapping.numel() >= n, "slot_mapping must be int64 [N]")
        d = _store_desc(state)
        _check(key.size(1) == d.kv_heads and key.size(2) == 128 and value.shape == key.shape,
               "K / V must be [N, H, 128]")
        _check(2 * int(max_close) <= state[6].numel(), "close list too small")
        _check(rank_of.numel() == d.num_layers * 2 * d.kv_heads * 256, "rank_of must hold every layer")
        _check(int(page_bytes) % 16 == 0 and int(page_bytes) < (1 << 31), "bad arena page size")
        self._call("fp_hbm_write_encode", ctypes.byref(d), _dev(key, "key"), key.stride(0), key.stride(1),
                   _dev(value, "value"), value.stride(0), value.stride(1), _dev(slot_mapping, "slot_mapping"), n,
                   int(layer), _dev(rank_of, "rank_of"), rank_of.numel(), int(arena), int(page_bytes),
                   int(max_close), int(bool(ordered)), _stream(key))

    def hbm_commit(self, *state) -> None:
        d = _store_desc(state)
        self._call("fp_hbm_commit", ctypes.byref(d), _stream(state[0]))

    def hbm_gather(self, src_blocks, rec_addr, rec_len, plut, slut, wk, wv, kv_heads: int) -> None:
        n = src_blocks.numel()
        if n == 0:
            return
        _check(src_blocks.dtype == torch.int32, "src_blocks must be int32")
        _check(wk.is_contiguous() and wv.is_contiguous() and wk.numel() == wv.numel(), "workspaces must be contiguous")
        ws = wk.numel() * wk.element_size()
        _check(ws >= n * 128 * kv_heads * 256, "workspace too small")
        self._call("fp_hbm_gather", _dev(src_blocks, "src_blocks"), n, _dev(rec_addr, "rec_addr"),
                   _dev(rec_len, "rec_len"), _dev(plut, "plut"), _dev(slut, "slut"), _dev(wk, "wk"),
                   _dev(wv, "wv"), ws, int(kv_heads), _stream(wk))

    def stream_probe(self, src, dst, read_bytes: int, write_bytes: int, wg_per_cu: int) -> None:
        """Streaming probe (measurement only): per 32 KB record of ``src``
        read ``read_bytes`` and write the first ``write_bytes`` of them to
        ``dst``."""
        _check(src.dtype == torch.uint8 and dst.dtype == torch.uint8 and src.is_contiguous() and dst.is_contiguous()
               and src.numel() == dst.numel() and src.numel() % 32768 == 0, "probe buffers: equal uint8 [n * 32768]")
        self._call("fp_stream_probe", _dev(src, "src"), _dev(dst, "dst"), src.numel() // 32768, int(read_bytes),
                   int(write_bytes), int(wg_per_cu), _stream(src))

    def hbm_export(self, blocks, rec_addr, rec_len, out, stride: int, lengths, digest: int) -> None:
        n = blocks.numel()
        if n == 0:
            return
        _check(blocks.dtype == torch.int32 and lengths.dtype == torch.int64 and lengths.numel() >= n,
               "export blocks must be int32 and lengths int64 [>= n]")
        _check(out.dtype == torch.uint8 and out.is_contiguous() and out.data_ptr() % 16 == 0,
               "export buffer must be contiguous 16-byte aligned uint8")
        L, NB, _, H = rec_addr.shape
        self._call("fp_hbm_export", _dev(blocks, "blocks"), n, _dev(rec_addr, "rec_addr"), _dev(rec_len, "rec_len"),
                   L, NB, H, _dev(out, "out"), out.numel(), int(stride), _dev(lengths, "lengths"), int(digest),
                   _stream(out))

    def hbm_import(self, *args) -> None:
        state = args[:13]
        src, offsets, blocks, status, arena_base, arena_stride, digest = args[13:]
        n = blocks.numel()
        if n == 0:
            return
        _check(src.dtype == torch.uint8 and src.is_contiguous() and src.data_ptr() % 16 == 0,
               "import buffer must be contiguous 16-byte aligned uint8")
        _check(offsets.dtype == torch.int64 and offsets.numel() == n and blocks.dtype == torch.int32
               and status.dtype == torch.int32 and status.numel() >= n,
               "import metadata must be int64 offsets, int32 blocks / status")
        d = _store_desc(state)
        _check(d.kv_heads <= 16, "too many KV heads")
        _check(arena_base.numel() == d.num_layers and arena_stride.numel() == d.num_layers,
               "arena tables must hold every layer")
        self._call("fp_hbm_import", ctypes.byref(d), _dev(src, "src"), src.numel(), _dev(offsets, "offsets"),
                   _dev(blocks, "blocks"), n, _dev(status, "status"), _dev(arena_base, "arena_base"),
                   _dev(arena_stride, "arena_stride"), int(digest), _stream(src))

    # -- batch record codec (GPU form of attn_page.encode_record / decode_record) --
    def encode_records(self, raw, kv, rank_of, tab_idx, out, lens) -> None:
        n = raw.size(0)
        if n == 0:
            return
        _check(raw.dtype in (torch.int16, torch.bfloat16, torch.uint16) and raw.is_contiguous()
               and raw[0].numel() == 16384, "raw must be contiguous 16-bit [n, 128, 128]")
        _check(out.dtype == torch.uint8 and out.is_contiguous() and out.numel() >= n * 32768, "out too small")
        _check(kv.dtype == torch.int32 and tab_idx.dtype == torch.int32 and lens.dtype == torch.int32,
               "kv / tab_idx / lens must be int32")
        _check(rank_of.dtype == torch.uint8 and rank_of.numel() % 256 == 0, "rank_of must be uint8 [T, 256]")
        self._call("fp_encode_records", _dev(raw, "raw"), n, _dev(kv, "kv"), _dev(rank_of, "rank_of"),
                   _dev(tab_idx, "tab_idx"), rank_of.numel() // 256, _dev(out, "out"), _dev(lens, "lens"),
                   _stream(raw))

    def decode_records(self, rec_addr, rec_len, kv, plut, slut, tab_idx, out) -> None:
        n = rec_addr.numel()
        if n == 0:
            return
        _check(out.is_contiguous() and out.numel() * out.element_size() >= n * 32768, "out too small")
        self._call("fp_decode_records", _dev(rec_addr, "rec_addr"), _dev(rec_len, "rec_len"), n, _dev(kv, "kv"),
                   _dev(plut, "plut"), _dev(slut, "slut"), _dev(tab_idx, "tab_idx"), slut.numel() // 16,
                   _dev(out, "out"), _stream(out))

    # -- plain BF16 paged decode (the baseline arm; the FA3 call of fragpack_step_bench.py:205-284) --
    def paged_decode_splits(self, batch: int, kv_heads: int, max_seq_len: int) -> int:
        return int(self._lib.fp_paged_decode_splits(int(batch), int(kv_heads), int(max_seq_len)))

    def paged_set_streaming(self, on: bool) -> None:
        self._lib.fp_paged_set_streaming(1 if on else 0)

    def paged_decode(self, q, k_cache, v_cache, block_table, seq_lens, max_seq_len: int, splits: int, opart, ml,
                     counters, out, scale: float) -> None:
        B = q.size(0)
        if B == 0:
            return
        _check(q.dtype == torch.bfloat16 and q.dim() == 3 and q.size(2) == 128 and q.stride(2) == 1
               and q.stride(1) == 128, "q must be BF16 [B, Hq, 128] with contiguous heads")
        _check(k_cache.dtype == torch.bfloat16 and k_cache.dim() == 4 and k_cache.size(1) == 128
               and k_cache.size(3) == 128 and k_cache.is_contiguous() and v_cache.shape == k_cache.shape
               and v_cache.dtype == torch.bfloat16 and v_cache.is_contiguous(),
               "k / v caches must be contiguous BF16 [blocks, 128, H, 128]")
        _check(out.shape == q.shape and out.dtype == torch.bfloat16 and out.stride(2) == 1 and out.stride(1) == 128,
               "out must match q")
        _check(block_table.dtype == torch.int32 and block_table.stride(1) == 1 and seq_lens.dtype == torch.int32,
               "block_table int32 [B, pages] with contiguous rows, seq_lens int32 [B]")
        kvh = k_cache.size(2)
        group = q.size(1) // kvh
        _check(group * kvh == q.size(1), "query heads must be a multiple of the KV heads")
        self._call("fp_paged_decode", _dev(q, "q"), q.stride(0), B, kvh, group, _dev(k_cache, "k_cache"),
                   _dev(v_cache, "v_cache"), k_cache.size(0), _dev(block_table, "block_table"), block_table.stride(0),
                   _dev(seq_lens, "seq_lens"), int(max_seq_len), int(splits), _dev(opart, "opart"), opart.numel(),
                   _dev(ml, "ml"), ml.numel(), _dev(counters, "counters"), counters.numel(), _dev(out, "out"),
                   out.stride(0), float(scale), _stream(q))

    # -- prefill (the FlashAttention call of backend.py:560-575) --
    def prefill_attention(self, q, wk, wv, out, cu_seqlens_q, seqused_k, block_table, max_seqlen_q: int,
                          max_seqlen_k: int, scale: float, causal: bool) -> None:
        n_seqs = seqused_k.numel()
        if n_seqs == 0 or q.size(0) == 0:
            return
        _check(q.dtype == torch.bfloat16 and out.dtype == torch.bfloat16 and wk.dtype == torch.bfloat16
               and wv.dtype == torch.bfloat16, "q / k / v / out must be BF16")
        _check(q.dim() == 3 and q.size(2) == 128 and q.stride(2) == 1 and q.stride(1) == 128,
               "q must be [N, Hq, 128] with contiguous heads")
        _check(out.shape == q.shape and out.stride(2) == 1 and out.stride(1) == 128, "out must match q")
        _check(wk.dim() == 4 and wk.size(1) == 128 and wk.size(3) == 128 and wk.is_contiguous()
               and wv.shape == wk.shape and wv.is_contiguous(), "k / v must be contiguous [P, 128, H, 128]")
        kvh = wk.size(2)
        group = q.size(1) // kvh
        _check(group * kvh == q.size(1), "query heads must be a multiple of the KV heads")
        _check(cu_seqlens_q.dtype == torch.int32 and seqused_k.dtype == torch.int32
               and cu_seqlens_q.numel() == n_seqs + 1, "cu_seqlens_q int32 [B + 1], seqused_k int32 [B]")
        _check(block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.stride(1) == 1
               and block_table.size(0) == n_seqs, "block_table must be int32 [B, pages] with contiguous rows")
        self._call("fp_prefill_attention", _dev(q, "q"), q.stride(0), _dev(wk, "k"), _dev(wv, "v"), wk.size(0), kvh,
                   group, _dev(cu_seqlens_q, "cu_seqlens_q"), _dev(seqused_k, "seqused_k"),
                   _dev(block_table, "block_table"), block_table.stride(0), n_seqs, int(max_seqlen_q),
                   int(max_seqlen_k), float(scale), int(bool(causal)), _dev(out, "out"), out.stride(0), _stream(q))


@functools.cache
def extension() -> Extension:
    """Load (once per process) the gfx950 library.

    Raises:
        RuntimeError: if the library has not been built or cannot be loaded.
    """
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m fragpack_amd.csrc.build` "
            "(or __graft_entry__.build()); there is no CPU fallback"
        )
    return Extension(ctypes.CDLL(str(LIB_PATH)))


__all__ = ["Extension", "FpStore", "LIB_PATH", "extension"]
