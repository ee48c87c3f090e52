/*
 * fragpack_hip.h -- C ABI of the MI355X FragPack hot path
 * (libfragpack_hip.so, built from fragpack_amd/csrc/ for gfx950).
 *
 * Every entry point enqueues work on ``stream`` and returns without
 * synchronising.  Return value: 0 on success, -1 on a rejected argument or a
 * launch failure; fp_last_error() then holds the message (per host thread).
 * All pointers are device pointers unless stated otherwise.  The library
 * allocates no device memory.
 *
 * Each function replaces one function of the reference's pybind module
 * (fragpack/ops/fragpack_ext.cpp:5-66), which the reference's Python layer
 * calls with torch tensors; here the tensors are flattened to pointers,
 * element strides and sizes.  The Python mirror
 * (fragpack_amd/ops/fragpack_ext.py) keeps the reference's tensor signatures
 * and calls these.
 */
#ifndef FRAGPACK_HIP_H_
#define FRAGPACK_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* fp_stream_t; /* hipStream_t */

/* The HBM store's state, i.e. the 13 tensors the reference passes to every
 * hbm_* call, in its order (fragpack/ops/hbm_kv.py:287-301; struct Store in
 * fragpack/ops/hbm_kv.cu:32-78), plus their geometry. */
typedef struct fp_store {
  int32_t* counters;   /* int32 [16]                                   */
  int32_t* wslot;      /* int32 [NB] staging slot of an open block      */
  int32_t* tags;       /* int32 [4, NB] per-block step stamps           */
  int32_t* free_stack; /* int32 [S_p]                                   */
  uint32_t* ovf_bits;  /* [ovf_words] overflow slots in use             */
  int32_t* claim_list; /* int32 [2, list_cap]                           */
  int32_t* close_list; /* int32 [2, list_cap]                           */
  int64_t* rec_addr;   /* int64 [L, NB, 2, H] record device addresses  */
  int32_t* rec_len;    /* int32 [L, NB, 2, H] bytes past the dense part */
  uint8_t* staging;    /* [S_p, L, 2, H, 32768] persistent staging      */
  uint8_t* scratch;    /* [S_t, 2, H, 32768] transient staging          */
  uint8_t* overflow;   /* [O, 32768] raw overflow records               */
  int32_t* fill;       /* int32 [L, NB] arena bytes used per page       */
  int64_t num_layers, num_blocks, kv_heads;
  int64_t staging_slots, scratch_slots, ovf_words, list_cap, overflow_records;
} fp_store_t;

/* Last error message of this host thread ("" if none). */
const char* fp_last_error(void);
/* ABI version (bumped on any signature change). */
int fp_abi_version(void);

/*
 * Split-KV decode attention over FragPack records.
 * Replaces fused_decode (fragpack/ops/fragpack_ext.cpp:5-9,
 * fragpack/ops/fused_attn_decode.cu:429-478).
 *   q           BF16 [B, H * group, 128], q_stride elements between rows
 *   rec_addr    int64 [P, 2, H], rec_len int32 [P, 2, H] (one layer)
 *   plut        uint32 [2, H, 2], slut uint8 [2, H, 16]
 *   block_table int32 [B, bt_stride], seq_lens int32 [B]
 *   opart/ml/plan  workspace (float, float, int32) of at least
 *               H*units*8*128, H*units*16 and
 *               ((2 + 4*units + 7) & ~7) + 8*units + H*units elements; the
 *               plan buffer's last H*units words are the merge counters, so
 *               one workspace serves calls of any unit count it fits (same H)
 *   out         BF16 [B, H * group, 128], out_stride elements between rows
 *   group       query heads per KV head: 1, 2, 4 or 8 (the reference pads
 *               smaller groups to 8 on the host; this kernel takes them as is)
 *   replan      0: reuse the plan in the workspace (written by an earlier
 *               planning call with the same units, batch and kv_heads; the
 *               kernel follows its unit descriptors, so anything else is
 *               undefined -- the Python mirror refuses such a call); 1: plan with a planner
 *               launch (also zeroes the merge counters); 2: plan inside the
 *               attention kernel when batch <= 64 (else as 1) -- the merge
 *               counters must be zero, as any completed call leaves them;
 *               3: as 2, and block_table holds batch * bt_stride readable
 *               entries (the kernel may read all of them when there are at
 *               most 1024)
 */
int fp_fused_decode(const void* q, int64_t q_stride, int64_t batch, int64_t kv_heads, int64_t group,
                    const int64_t* rec_addr, const int32_t* rec_len, const uint32_t* plut,
                    const uint8_t* slut, const int32_t* block_table, int64_t bt_stride,
                    const int32_t* seq_lens, float* opart, int64_t opart_elems, float* ml,
                    int64_t ml_elems, int32_t* plan, int64_t plan_elems, void* out, int64_t out_stride,
                    int64_t units, int replan, double scale, fp_stream_t stream);

/*
 * fp_fused_decode plus the store's write of a decode-only step, in one
 * launch.  No counterpart in the reference, which writes with hbm_write
 * (fragpack_ext.cpp:19-23, hbm_kv.cu:221-255) before fused_decode: here the
 * unit that owns each sequence's last page first writes that sequence's new
 * token -- new_k / new_v row b -- into slot slot_mapping[b] (block * 128 +
 * row, negative: padding, nothing written) of the raw record the block's
 * table entry names, then attends.  Only records that lie inside
 * [staging, staging + staging_bytes) or [scratch, scratch + scratch_bytes)
 * are written (a table entry elsewhere is skipped, as hbm_write skips a block
 * without a staging slot).  Every row must be a decode row: one new token,
 * the sequence's last (seq_lens[b] - 1), in its last block.
 *   new_k, new_v  BF16 [B, H, 128]: token / head strides in elements (even)
 *   slot_mapping  int64 [B]
 * Currently disabled: the call records an error (fp_last_error) and returns
 * -1 without launching anything, because its first GPU run faulted and the
 * cause has not been shown.  Callers write with fp_hbm_write (or the fused
 * fp_hbm_write_encode) and then call fp_fused_decode.
 */
int fp_fused_decode_append(const void* q, int64_t q_stride, int64_t batch, int64_t kv_heads, int64_t group,
                           const int64_t* rec_addr, const int32_t* rec_len, const uint32_t* plut,
                           const uint8_t* slut, const int32_t* block_table, int64_t bt_stride,
                           const int32_t* seq_lens, float* opart, int64_t opart_elems, float* ml,
                           int64_t ml_elems, int32_t* plan, int64_t plan_elems, void* out, int64_t out_stride,
                           int64_t units, int replan, double scale, const void* new_k, int64_t nk_token_stride,
                           int64_t nk_head_stride, const void* new_v, int64_t nv_token_stride,
                           int64_t nv_head_stride, const int64_t* slot_mapping, const void* staging,
                           int64_t staging_bytes, const void* scratch, int64_t scratch_bytes,
                           fp_stream_t stream);

/*
 * fp_fused_decode without caller workspaces, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * split-KV partials, (m, l) pairs and plan live in a static device array of
 * fp_fused_decode_noalloc_capacity() bytes (32 MiB) that each device holds
 * for the life of the process; a call needing more (about
 * 4 KiB x kv_heads x units) returns -1 with an error.  Every call launches
 * the planner (replan 1), which also zeroes the merge counters.  Calls that
 * overlap on one device share the array and race: serialise them (one
 * stream).  Arguments as fp_fused_decode minus the workspace and replan.
 */
int fp_fused_decode_noalloc(const void* q, int64_t q_stride, int64_t batch, int64_t kv_heads, int64_t group,
                            const int64_t* rec_addr, const int32_t* rec_len, const uint32_t* plut,
                            const uint8_t* slut, const int32_t* block_table, int64_t bt_stride,
                            const int32_t* seq_lens, void* out, int64_t out_stride, int64_t units, double scale,
                            fp_stream_t stream);
/* Bytes of the static workspace behind fp_fused_decode_noalloc. */
int64_t fp_fused_decode_noalloc_capacity(void);

/*
 * Decode attention over a plain paged BF16 cache: the uncompressed baseline
 * arm.  Replaces the FA3 call the reference benchmarks against
 * (benchmarks/fragpack_step_bench.py:205-284, flash_attn_with_kvcache).
 *   k_cache, v_cache BF16 [num_blocks, 128, kv_heads, 128] (contiguous);
 *   block_table int32 [batch, bt_stride]; seq_lens int32 [batch], each
 *   <= max_seq_len.  splits (from fp_paged_decode_splits) workgroups share
 *   each (sequence, head); with splits > 1 the workspace is opart float
 *   [batch * kv_heads * splits * 8 * 128], ml float [... * 8 * 2] and
 *   counters int32 [batch * kv_heads], zero before the first call (every
 *   completed call leaves them zero).
 */
int fp_paged_decode(const void* q, int64_t q_stride, int64_t batch, int64_t kv_heads, int64_t group,
                    const void* k_cache, const void* v_cache, int64_t num_blocks, const int32_t* block_table,
                    int64_t bt_stride, const int32_t* seq_lens, int64_t max_seq_len, int64_t splits, float* opart,
                    int64_t opart_elems, float* ml, int64_t ml_elems, int32_t* counters, int64_t counter_elems,
                    void* out, int64_t out_stride, double scale, fp_stream_t stream);
/* Splits per (sequence, head) that fill the current device. */
int fp_paged_decode_splits(int64_t batch, int64_t kv_heads, int64_t max_seq_len);
/* Load policy of fp_paged_decode's page loads: 1 non-temporal (default), 0
 * plain.  The faster one depends on the shape, so the baseline is measured
 * with both.  Process-wide, not for concurrent callers.  No counterpart in
 * the reference (FA3 chooses its own loads). */
int fp_paged_set_streaming(int on);

/* Step start: GC, staging claims, close list.  Replaces hbm_prepare
 * (fragpack_ext.cpp:11-17, hbm_kv.cu:669-686). */
int fp_hbm_prepare(const fp_store_t* s, const int64_t* slot_mapping, int64_t n_tok, const int32_t* live,
                   int64_t n_live, int64_t step, fp_stream_t stream);

/* New K/V tokens into kernel-order staging.  key/value BF16 [n, H, 128]
 * with element strides (k_s0, k_s1), (v_s0, v_s1); head dim contiguous.
 * Replaces hbm_write (fragpack_ext.cpp:19-25, hbm_kv.cu:688-705). */
int fp_hbm_write(const fp_store_t* s, const void* key, int64_t k_s0, int64_t k_s1, const void* value,
                 int64_t v_s0, int64_t v_s1, const int64_t* slot_mapping, int64_t n, int64_t layer,
                 fp_stream_t stream);

/* Encode this layer's records of the blocks closed this step into their
 * arena pages (rank_of uint8 [L, 2, H, 256]).  Replaces hbm_encode
 * (fragpack_ext.cpp:27-33, hbm_kv.cu:707-723). */
int fp_hbm_encode(const fp_store_t* s, const uint8_t* rank_of, int64_t rank_of_elems, int64_t layer,
                  int64_t arena, int64_t page_bytes, int64_t max_close, fp_stream_t stream);

/* fp_hbm_encode with placement by record order (deterministic page packing;
 * no counterpart in the reference, whose encode claims page space in arrival
 * order, hbm_kv.cu:352-363): each closed block's 2H records are placed in
 * (kv, head) order, a coded record taking the page's next bytes if they fit
 * and spilling to the overflow pool if not, so the arena bytes and the spill
 * set depend only on the records.  For few closing blocks this runs two
 * launches and uses the closing records' rec_addr / rec_len entries between
 * them: nothing may read those entries before the call's work completes. */
int fp_hbm_encode_ordered(const fp_store_t* s, const uint8_t* rank_of, int64_t rank_of_elems, int64_t layer,
                          int64_t arena, int64_t page_bytes, int64_t max_close, fp_stream_t stream);

/* fp_hbm_write followed by fp_hbm_encode (ordered = 0) or
 * fp_hbm_encode_ordered (ordered = 1) of the same layer, in one launch: the
 * decode-step fusion the reference's step benchmark measures as separate
 * launches (fragpack_step_bench.py:472-610, write hbm_kv.cu:223-255 then
 * encode :262-429).  The workgroups that encode a closing block's records
 * write that block's (and its heir's) new rows themselves before reading
 * them; the others write every token of the other blocks.  Same results as
 * the two calls.  Each closing record's encoder scans the whole slot
 * mapping, so this suits steps of few tokens (decode steps). */
int fp_hbm_write_encode(const fp_store_t* s, const void* key, int64_t k_s0, int64_t k_s1, const void* value,
                        int64_t v_s0, int64_t v_s1, const int64_t* slot_mapping, int64_t n, int64_t layer,
                        const uint8_t* rank_of, int64_t rank_of_elems, int64_t arena, int64_t page_bytes,
                        int64_t max_close, int ordered, fp_stream_t stream);

/* Release closed blocks' staging.  Replaces hbm_commit
 * (fragpack_ext.cpp:35-39, hbm_kv.cu:725-734). */
int fp_hbm_commit(const fp_store_t* s, fp_stream_t stream);

/* Streaming probe, no counterpart in the reference: for r < records, reads
 * the first read_bytes of src + 32768 r and writes the first write_bytes of
 * them to dst + 32768 r (non-temporal, wg_per_cu 256-thread workgroups per
 * CU, each with 32 KB of loads in flight).  bench.py times it as the HBM
 * ceiling for the encoder's read / write mix.  Buffers: records x 32768
 * bytes each, 16-byte aligned; bytes multiples of 16, write <= read <= 32768. */
int fp_stream_probe(const void* src, void* dst, int64_t records, int64_t read_bytes, int64_t write_bytes,
                    int64_t wg_per_cu, fp_stream_t stream);

/* Decode records of blocks src_blocks[i] (one layer's rec tables, [NB, 2, H])
 * into token-major BF16 pages wk / wv [>= n, 128, H, 128] (ws_bytes each).
 * Replaces hbm_gather (fragpack_ext.cpp:41-43, hbm_kv.cu:736-753). */
int fp_hbm_gather(const int32_t* src_blocks, int64_t n, const int64_t* rec_addr, const int32_t* rec_len,
                  const uint32_t* plut, const uint8_t* slut, void* wk, void* wv, int64_t ws_bytes,
                  int64_t kv_heads, fp_stream_t stream);

/* Closed blocks -> block blobs at out + i * stride; lengths int64 [n].
 * Replaces hbm_export (fragpack_ext.cpp:45-46, hbm_kv.cu:755-774). */
int fp_hbm_export(const int32_t* blocks, int64_t n, const int64_t* rec_addr, const int32_t* rec_len,
                  int64_t num_layers, int64_t num_blocks, int64_t kv_heads, uint8_t* out, int64_t out_bytes,
                  int64_t stride, int64_t* lengths, int64_t digest, fp_stream_t stream);

/* Validate and install block blobs (src, src_bytes) at offsets[i] into
 * blocks[i]; status int32 [n] gets failure bits.  arena_base / arena_stride
 * int64 [L].  Replaces hbm_import (fragpack_ext.cpp:48-55,
 * hbm_kv.cu:776-802). */
int fp_hbm_import(const fp_store_t* s, const uint8_t* src, int64_t src_bytes, const int64_t* offsets,
                  const int32_t* blocks, int64_t n, int32_t* status, const int64_t* arena_base,
                  const int64_t* arena_stride, int64_t digest, fp_stream_t stream);

/*
 * Batch record codec (device): the GPU form of the reference's CPU codec
 * attn_page.encode_record / decode_record (fragpack/compression/
 * attn_page.py:146-269), byte-identical to it.
 *   fp_encode_records: raw BF16 token-major [n, 128, 128] -> out [n, 32768]
 *     (record i in the first lens[i] bytes of row i); kv[i] in {0, 1};
 *     rank_of uint8 [n_tables, 256], tab_idx[i] selects the table.
 *   fp_decode_records: records (rec_addr[i], DENSE + rec_len[i] bytes) ->
 *     token-major [n, 128, 128]; plut [n_tables, 2], slut [n_tables, 16].
 */
int fp_encode_records(const void* raw, int64_t n, const int32_t* kv, const uint8_t* rank_of,
                      const int32_t* tab_idx, int64_t n_tables, uint8_t* out, int32_t* lens,
                      fp_stream_t stream);
int fp_decode_records(const int64_t* rec_addr, const int32_t* rec_len, int64_t n, const int32_t* kv,
                      const uint32_t* plut, const uint8_t* slut, const int32_t* tab_idx, int64_t n_tables,
                      void* out, fp_stream_t stream);

/*
 * Causal varlen prefill attention over the paged BF16 workspace (the
 * workspace HbmKvStore.gather fills): replaces the vLLM FlashAttention call
 * flash_attn_varlen_func(q, k, v, out, cu_seqlens_q, max_seqlen_q,
 * seqused_k, max_seqlen_k, softmax_scale, causal=True, block_table) of
 * fragpack/integrations/vllm/backend.py:560-575.
 *   q, out: BF16 [Nq, kv_heads * group, 128], heads contiguous, token
 *     strides q_stride / out_stride (elements).
 *   wk, wv: BF16 [num_pages, 128, kv_heads, 128]; sequence b's key j is row
 *     j % 128 of page block_table[b * bt_stride + j / 128].
 *   cu_seqlens_q int32 [num_seqs + 1]; seqused_k int32 [num_seqs] (>= the
 *     sequence's query count: queries are its last positions, causal mask
 *     aligned bottom-right).  group in {1, 2, 4, 8}.
 */
int fp_prefill_attention(const void* q, int64_t q_stride, const void* wk, const void* wv, int64_t num_pages,
                         int64_t kv_heads, int64_t group, const int32_t* cu_seqlens_q, const int32_t* seqused_k,
                         const int32_t* block_table, int64_t bt_stride, int64_t num_seqs, int64_t max_seqlen_q,
                         int64_t max_seqlen_k, double scale, int causal, void* out, int64_t out_stride,
                         fp_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FRAGPACK_HIP_H_ */
