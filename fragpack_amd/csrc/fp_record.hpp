// FragPack record format: constants and gfx950 device helpers shared by the
// decode-attention, gather, codec and store kernels.
//
// Record format (reference: fragpack/compression/attn_page.py:1-44): one
// (page, kv, head) slice of 128 tokens x 128 dims of BF16, permuted into the
// reference's "kernel order": thread t = (w = t>>5, g = (t>>2)&7, c = t&3)
// of a 256-wide group owns positions [64t, 64t+64); its scalar
// s = 8 st + 4 j + 2 f + e is
//   K: token 16w + 8j + g, dim 16st + 8f + 2c + e
//   V: token 16st + 8f + 2c + e, dim 16w + 8j + g.
// Coded records: low bytes (chunk j of thread t at 16 (256 j + t)), 3-bit
// symbols (three u32 words per 32-scalar group, thread t's six words as three
// 8-byte chunks at 16384 + 8 (256 m + t)), then a variable region of a 48-byte
// header, escape nibbles and a raw list.  Raw records: thread t's word st at
// 16 (256 st + t).  The format is the reference's wire format and is kept
// byte for byte; everything below is this build's own gfx950 code.
//
// A "slab" here is 64 consecutive kernel-order threads (4096 scalars): the
// unit one wavefront decodes per pass.  A lane may decode any thread of the
// slab (the decode-attention kernel permutes them to suit MFMA operand
// layouts); escape offsets are found with a scan in kernel order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace fp {

constexpr int kTokens = 128;
constexpr int kDim = 128;
constexpr int kLowBytes = 16384;
constexpr int kSymBytes = 6144;
constexpr int kDenseBytes = kLowBytes + kSymBytes;  // 22528
constexpr int kVarCap = 2048;
constexpr int kRawRecord = 32768;
constexpr int kRawVarLen = kRawRecord - kDenseBytes;  // 10240: rec_len of a raw record
constexpr int kHeaderBytes = 48;
constexpr int kPrimaryDirect = 7;
constexpr int kTableEntries = 22;
constexpr int kMaxWarpRaw = 32;
constexpr int kRawNibble = 15;
// Largest escape count of a coded record (VAR_CAP bounds the nibble bytes).
constexpr int kMaxEscapes = 2 * (kVarCap - kHeaderBytes);  // 4000
// Per-wave LDS bytes for one slab's expanded escape bytes (window reads may
// run up to 12 bytes past the last escape, and the region starts 8-aligned).
constexpr int kEscLds = kMaxEscapes + 64;

// ---------------------------------------------------------------------------
// Small helpers.

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).  Used
// where an index must stay a constant so arrays stay in registers.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// Two floats -> BF16 pair (x low), round to nearest even: one v_cvt_pk_bf16_f32.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float x, float y) {
  const f32x2_t v = {x, y};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  // v_perm_b32: byte i of the result is byte sel.byte[i] of {hi:lo}
  // (0-3 from lo, 4-7 from hi, 12 -> 0x00).
  return __builtin_amdgcn_perm(hi, lo, sel);
}

__device__ __forceinline__ uint32_t alignbyte(uint32_t hi, uint32_t lo, uint32_t shift) {
  return __builtin_amdgcn_alignbyte(hi, lo, shift);
}

__device__ __forceinline__ int wave_lane() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

template <typename T>
__device__ __forceinline__ T uniform(T v) {
  return (T)__builtin_amdgcn_readfirstlane((int)v);
}

__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Wavefront-wide inclusive scan with DPP (row shifts within 16-lane rows,
// then row broadcasts), no LDS round trips.  ``Op`` is + or max over values
// whose identity is 0.
template <bool kMax>
__device__ __forceinline__ int dpp_op(int a, int b) {
  return kMax ? max(a, b) : a + b;
}
template <bool kMax>
__device__ __forceinline__ int wave_scan_dpp(int x) {
  x = dpp_op<kMax>(x, __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true));  // row_shr:1
  x = dpp_op<kMax>(x, __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true));  // row_shr:2
  x = dpp_op<kMax>(x, __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true));  // row_shr:4
  x = dpp_op<kMax>(x, __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true));  // row_shr:8
  x = dpp_op<kMax>(x, __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false));  // row_bcast:15
  x = dpp_op<kMax>(x, __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false));  // row_bcast:31
  return x;
}
template <bool kMax>
__device__ __forceinline__ int wave_total(int x) {
  return __builtin_amdgcn_readlane(wave_scan_dpp<kMax>(x), 63);
}

// Inclusive prefix sum over the 64 lanes of a wavefront.
__device__ __forceinline__ int wave_incl_scan(int v) { return wave_scan_dpp<false>(v); }

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int o = 32; o; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Orders this wave's earlier LDS writes before its later LDS reads made by
// other lanes (DS instructions of one wave complete in order; this only
// stops the compiler from moving accesses across it).
// Workgroup barrier for LDS traffic only: waits for this wave's LDS (and
// scalar) operations, not for its global loads / stores, so prefetches stay
// in flight across it.  Use only where no global memory written before the
// barrier is read by another wave after it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt, expcnt unconstrained
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Sets this wave's instruction-issue priority to ``step`` mod 4 (wave-uniform).
// The workgroups resident on one CU issue in age order when their priorities
// are equal, so in a long-running launch the first-dispatched workgroup runs
// ahead and the CU spends the end of the launch with fewer workgroups than it
// can hold; kernels whose workgroups do equal work rotate the priority with
// their loop step (offset by the workgroup id) to even out their progress.
__device__ __forceinline__ void rotate_priority(int step) {
  switch (step & 3) {
    case 0: __builtin_amdgcn_s_setprio(0); break;
    case 1: __builtin_amdgcn_s_setprio(1); break;
    case 2: __builtin_amdgcn_s_setprio(2); break;
    default: __builtin_amdgcn_s_setprio(3); break;
  }
}

// ---------------------------------------------------------------------------
// Dense data of one kernel-order thread, as a lane holds it before decoding:
//   coded: v[0..3] = low-byte chunks 0..3, v[4] = symbol words 0..3,
//          v[5].x/y = symbol words 4..5;
//   raw:   v[st] = word st (8 BF16 scalars) for st < 6; words 6 and 7 are
//          read when decoded (raw records are rare: tails and fallbacks).
// Both forms are loaded by the same instructions (four 16-byte loads, four
// 8-byte loads) at offsets chosen by the form, so a caller's wait counts do
// not depend on it.
struct SlabBuf {
  uint4 v[6];
};

// Loads through the global address space (record pointers arrive as plain
// 64-bit addresses; generic pointers would compile to flat loads).
#define FP_GLOBAL __attribute__((address_space(1)))
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ld16(const uint8_t* p) {
  const u32x4_t v = *reinterpret_cast<const FP_GLOBAL u32x4_t*>(reinterpret_cast<uintptr_t>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld8(const uint8_t* p) {
  const u32x2_t v = *reinterpret_cast<const FP_GLOBAL u32x2_t*>(reinterpret_cast<uintptr_t>(p));
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ld4(const uint8_t* p) {
  return *reinterpret_cast<const FP_GLOBAL uint32_t*>(reinterpret_cast<uintptr_t>(p));
}
// The same with the non-temporal policy, for record data read once.
__device__ __forceinline__ uint4 ld16_nt(const uint8_t* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const FP_GLOBAL u32x4_t*>(reinterpret_cast<uintptr_t>(p)));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld8_nt(const uint8_t* p) {
  const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const FP_GLOBAL u32x2_t*>(reinterpret_cast<uintptr_t>(p)));
  return make_uint2(v.x, v.y);
}

// Buffer-resource loads: a wave-uniform record base in SGPRs, a per-lane
// 32-bit byte offset and a wave-uniform SGPR offset; out-of-range reads
// (past ``bytes``) return zero.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bld16(rsrc_t r, int voff, int soff) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 bld8(rsrc_t r, int voff, int soff) {
  const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
  return make_uint2(v.x, v.y);
}
// Record data is streamed: a launch reads each record once, so its loads
// carry the non-temporal policy bit (measured on MI355X: a plain streaming
// read of 8 GB runs at 6.2 TB/s, with the bit at 7.0 TB/s).
constexpr int kNt = 2;
__device__ __forceinline__ uint4 rld16(rsrc_t r, int voff, int soff) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kNt);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 rld8(rsrc_t r, int voff, int soff) {
  const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, kNt);
  return make_uint2(v.x, v.y);
}

typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float2vv __attribute__((ext_vector_type(2)));
// Split-KV partials are handed between workgroups (possibly on different
// XCDs, each with its own L2) through per-location coherent accesses:
// agent-scope relaxed atomic stores and loads (sc1: written through to, and
// read from, the device coherence point).  A writer waits for its stores to
// be acknowledged (s_waitcnt) before bumping the group counter, and a reader
// issues its loads only after seeing the counter complete.  This avoids the
// whole-L2 writeback / invalidate an agent-scope fence costs on a multi-XCD
// part once per workgroup.
// Coherent (sc1) 16- / 8-byte accesses through a buffer resource over a
// float array of < 2^31 bytes; ``i`` is the float index.
constexpr int kSc1 = 16;  // cache-policy bit of buffer instructions: sc1
__device__ __forceinline__ rsrc_t coh_rsrc(const float* base) { return make_rsrc(base, 0x7fffffff); }
__device__ __forceinline__ void st_coh4(rsrc_t r, int64_t i, float a, float b, float c, float d) {
  const float4v v = {a, b, c, d};
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, (int)(4 * i), 0, kSc1);
}
__device__ __forceinline__ void st_coh2(rsrc_t r, int64_t i, float a, float b) {
  const float2vv v = {a, b};
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, v), r, (int)(4 * i), 0, kSc1);
}
__device__ __forceinline__ float4 ld_coh4(rsrc_t r, int64_t i) {
  const float4v v = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(4 * i), 0, kSc1));
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ float2 ld_coh2(rsrc_t r, int64_t i) {
  const float2vv v = __builtin_bit_cast(float2vv, __builtin_amdgcn_raw_buffer_load_b64(r, (int)(4 * i), 0, kSc1));
  return make_float2(v[0], v[1]);
}
// Waits until every store this wave issued is acknowledged.
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0); }

// Loads dense data of kernel-order thread 64 * slab + nt (nt < 64) of the
// record behind ``r`` (``raw`` wave-uniform): no branch, eight loads.
__device__ __forceinline__ void load_slab(rsrc_t r, bool raw, int slab, int nt, SlabBuf& b) {
  const int v16 = 16 * nt;
#pragma unroll
  for (int j = 0; j < 4; ++j) b.v[j] = rld16(r, v16, 4096 * j + 1024 * slab);
  // symbol chunks m = 0..2 at 8 (256 m + t) and, past the record (zeros, no
  // memory access), a fourth piece; or words 4 and 5 in 8-byte halves
  const int vo = raw ? v16 : 8 * nt;
  const uint2 s0 = rld8(r, vo, raw ? 4096 * 4 + 1024 * slab : kLowBytes + 512 * slab);
  const uint2 s1 = rld8(r, vo, raw ? 4096 * 4 + 1024 * slab + 8 : kLowBytes + 2048 + 512 * slab);
  const uint2 s2 = rld8(r, vo, raw ? 4096 * 5 + 1024 * slab : kLowBytes + 4096 + 512 * slab);
  const uint2 s3 = rld8(r, vo, raw ? 4096 * 5 + 1024 * slab + 8 : kRawRecord);
  b.v[4] = make_uint4(s0.x, s0.y, s1.x, s1.y);
  b.v[5] = make_uint4(s2.x, s2.y, s3.x, s3.y);
}

// Loads thread ``t``'s (0..255) dense data of a record.
__device__ __forceinline__ void load_thread(const uint8_t* rec, bool raw, int t, SlabBuf& b) {
#pragma unroll
  for (int j = 0; j < 4; ++j) b.v[j] = ld16_nt(rec + 16 * (256 * j + t));
  if (raw) {
    b.v[4] = ld16_nt(rec + 16 * (256 * 4 + t));
    b.v[5] = ld16_nt(rec + 16 * (256 * 5 + t));
  } else {
    const uint2 s0 = ld8_nt(rec + kLowBytes + 8 * t), s1 = ld8_nt(rec + kLowBytes + 8 * (256 + t));
    const uint2 s2 = ld8_nt(rec + kLowBytes + 8 * (512 + t));
    b.v[4] = make_uint4(s0.x, s0.y, s1.x, s1.y);
    b.v[5] = make_uint4(s2.x, s2.y, 0u, 0u);
  }
}

__device__ __forceinline__ uint32_t u4(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

__device__ __forceinline__ uint32_t sym_dword(const SlabBuf& b, int i) {
  return i == 0 ? b.v[4].x : i == 1 ? b.v[4].y : i == 2 ? b.v[4].z : i == 3 ? b.v[4].w : i == 4 ? b.v[5].x : b.v[5].y;
}

// Symbol word (eight 4-bit nibbles, code in the low 3 bits) of word st
// (st must be a compile-time constant after inlining).
__device__ __forceinline__ uint32_t sym_word(const SlabBuf& b, int st) {
  const int gi = st >> 2, k = st & 3;
  if (k < 3) return sym_dword(b, 3 * gi + k) & 0x77777777u;
  const uint32_t w0 = sym_dword(b, 3 * gi), w1 = sym_dword(b, 3 * gi + 1), w2 = sym_dword(b, 3 * gi + 2);
  return ((w0 >> 3) & 0x11111111u) | ((w1 >> 2) & 0x22222222u) | ((w2 >> 1) & 0x44444444u);
}

// Bit 0 of nibble i set iff scalar i of the word is an escape (code 7).
__device__ __forceinline__ uint32_t esc_bits(uint32_t sk) { return ((sk + 0x11111111u) >> 3) & 0x11111111u; }

// Looks up four nibble values (one per byte, 0..15) in the 16-byte table
// {t3:t2:t1:t0}.
__device__ __forceinline__ uint32_t lut16(uint32_t sel, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
  const uint32_t s7 = sel & 0x07070707u;
  const uint32_t lo = perm(t1, t0, s7), hi = perm(t3, t2, s7);
  // byte k from lo (selector k) or hi (k + 4) by bit 3 of selector byte k
  return perm(hi, lo, ((sel >> 1) & 0x04040404u) | 0x03020100u);
}

// Eight nibbles (escape stream order, low nibble first) -> eight bytes
// through the extended table (nibble 15 -> 0, patched by the raw list).
__device__ __forceinline__ uint2 expand_nibbles(uint32_t n, const uint32_t (&sl)[4]) {
  const uint32_t ev = lut16(n & 0x0F0F0F0Fu, sl[0], sl[1], sl[2], sl[3]);
  const uint32_t od = lut16((n >> 4) & 0x0F0F0F0Fu, sl[0], sl[1], sl[2], sl[3]);
  return make_uint2(perm(od, ev, 0x05010400u), perm(od, ev, 0x07030602u));
}

// Record header fields one slab needs.
struct SlabHdr {
  int e0, e1;       // escape ordinals [e0, e1) of the slab's threads
  int r0, r1;       // raw-list entries [r0, r1)
  int raw_offset;   // byte offset of the raw list in the variable region
};

// ``rd4(offset)`` reads the u32 at byte ``offset`` of the variable region
// (global memory or an LDS copy).
// Slab ``slab`` (threads 64 slab .. 64 slab + 63) spans the header's
// 2048-scalar prefix entries 2 slab and 2 slab + 1; the low u16 of dword
// 4 + slab (8 + slab) is esc_prefix[2 slab] (raw_prefix[2 slab]).
template <typename Rd4>
__device__ __forceinline__ SlabHdr slab_header(Rd4&& rd4, int slab) {
  SlabHdr h;
  h.e0 = (int)(rd4(16 + 4 * slab) & 0xFFFF);
  h.r0 = (int)(rd4(32 + 4 * slab) & 0xFFFF);
  if (slab < 3) {
    h.e1 = (int)(rd4(16 + 4 * (slab + 1)) & 0xFFFF);
    h.r1 = (int)(rd4(32 + 4 * (slab + 1)) & 0xFFFF);
  } else {
    h.e1 = (int)rd4(0);
    h.r1 = (int)rd4(4);
  }
  h.raw_offset = (int)rd4(8);
  return h;
}

// Expands the slab's escape nibbles through the extended table into ``esc``
// (wave-private LDS, kEscLds bytes) and patches raw scalars' high bytes from
// the raw list.  Byte k of ``esc`` is escape ordinal (e0 & ~7) + k.  All 64
// lanes of the wave must call this together.
template <typename Rd4>
__device__ __forceinline__ void stage_escapes(Rd4&& rd4, const SlabHdr& h, const uint32_t (&sl)[4], uint8_t* esc,
                                              int lane) {
  const int d0 = h.e0 >> 3;
  const int nd = min(((h.e1 + 7) >> 3) - d0, kMaxEscapes / 8 + 1);
  for (int k = lane; k < nd; k += 64) {
    const uint2 b = expand_nibbles(rd4(kHeaderBytes + 4 * (d0 + k)), sl);
    *reinterpret_cast<uint2*>(esc + 8 * k) = b;
  }
  wave_lds_sync();
  for (int k = h.r0 + lane; k < h.r1; k += 64) {
    const uint32_t e = rd4(h.raw_offset + 4 * k);
    const int x = (int)(e & 0xFFFFu) - 8 * d0;
    if (x >= 0 && x < kEscLds) esc[x] = (uint8_t)(e >> 16);
  }
  wave_lds_sync();
}

// Decodes the 64 scalars of one kernel-order thread of a coded record and
// calls emit(st, word) for st = 0..7, word = 4 dwords = 8 BF16 (little-endian
// pairs).  ``eo`` is the LDS byte index (relative to ``esc``) of this
// thread's first escape.  ``lut0``, ``lut1``: primary table bytes 0-3 / 4-6
// (byte 7 = 0).  Scalar order within a word: natural (dwords hold scalars
// 0,1 | 2,3 | 4,5 | 6,7) or, with kEvenOdd, (0,2 | 1,3 | 4,6 | 5,7), which
// takes two byte permutes fewer (the attention kernel's tiles follow it).
//
// Per word: the high bytes come from the primary table by code, escapes
// (code 7) from the next 8 bytes of the expanded escape stream at this
// thread's running byte position (three aligned dword reads and two byte
// alignments: one unaligned 8-byte LDS read measured slower); the escape
// of scalar i takes stream byte rank(i), the number of escapes among
// scalars < i.
template <bool kEvenOdd = false, typename Emit>
__device__ __forceinline__ void decode_words(const SlabBuf& b, const uint8_t* esc, int eo, uint32_t lut0,
                                             uint32_t lut1, Emit&& emit) {
  // 0x0C0C0C0C in an SGPR, so each selector below is one v_bitop3 (a
  // literal operand would cost a separate v_xor)
  uint32_t c0c;
  asm("s_mov_b32 %0, 0x0c0c0c0c" : "=s"(c0c));
  // the running escape position as an LDS byte address (``esc`` is 4-byte
  // aligned, so its low two bits are those of eo)
  typedef __attribute__((address_space(3))) const uint8_t lds_u8;
  typedef __attribute__((address_space(3))) const uint32_t lds_u32;
  uint32_t ea = (uint32_t)(uintptr_t)(lds_u8*)esc + (uint32_t)eo;
  static_for<0, 8>([&](auto st_c) {
    constexpr int st = decltype(st_c)::value;
    const uint32_t sk = sym_word(b, st);
    const uint32_t b8 = (sk + 0x11111111u) & 0x88888888u;  // bit 3 of each escape nibble
    const uint32_t s_ev = sk & 0x07070707u, s_od = (sk >> 4) & 0x07070707u;
    // primary high bytes of scalars 0,2,4,6 / 1,3,5,7 (escape code 7 -> 0)
    const uint32_t hp_ev = perm(lut1, lut0, s_ev);
    const uint32_t hp_od = perm(lut1, lut0, s_od);
    lds_u32* ew = (lds_u32*)(uintptr_t)(ea & ~3u);
    const uint32_t d0 = ew[0], d1 = ew[1], d2 = ew[2];
    // v_alignbyte_b32 shifts by 8 x bits [1:0] of its last operand: ea as is
    const uint2 win = make_uint2(alignbyte(d1, d0, ea), alignbyte(d2, d1, ea));
    ea += __builtin_popcount(b8);
    // nibble i of rank: escapes among nibbles < i (b8 = 8 x the escape bits)
    const uint32_t rank = b8 * 0x02222222u;
    // selector byte per scalar: its rank for an escape, 0x0C (-> byte 0x00)
    // otherwise; the code-indexed mask is 0xF0 for an escape (keeping the
    // scalar's rank nibble, the low one of the byte), 0xFF otherwise
    const uint32_t m_ev = perm(0xF0FFFFFFu, 0xFFFFFFFFu, s_ev), m_od = perm(0xF0FFFFFFu, 0xFFFFFFFFu, s_od);
    const uint32_t sel_ev = (rank & ~m_ev) | (c0c & m_ev);
    const uint32_t sel_od = ((rank >> 4) & ~m_od) | (c0c & m_od);
    const uint32_t h_ev = hp_ev | perm(win.y, win.x, sel_ev);
    const uint32_t h_od = hp_od | perm(win.y, win.x, sel_od);
    const uint4 lw = b.v[st >> 1];
    const uint32_t la = (st & 1) ? lw.z : lw.x, lb = (st & 1) ? lw.w : lw.y;  // low bytes of 0..3 / 4..7
    if constexpr (kEvenOdd) {
      emit(st_c, make_uint4(perm(h_ev, la, 0x05020400u), perm(h_od, la, 0x05030401u), perm(h_ev, lb, 0x07020600u),
                            perm(h_od, lb, 0x07030601u)));
    } else {
      const uint32_t h01 = perm(h_od, h_ev, 0x05010400u);  // high bytes of scalars 0..3
      const uint32_t h23 = perm(h_od, h_ev, 0x07030602u);  // 4..7
      emit(st_c, make_uint4(perm(h01, la, 0x05010400u), perm(h01, la, 0x07030602u), perm(h23, lb, 0x05010400u),
                            perm(h23, lb, 0x07030602u)));
    }
  });
}

// Escape count of one thread's 64 scalars.
__device__ __forceinline__ int thread_escapes(const SlabBuf& b) {
  int n = 0;
  // same expression as decode_words' escape bits, so the two share it
  static_for<0, 8>([&](auto st) { n += __builtin_popcount((sym_word(b, st) + 0x11111111u) & 0x88888888u); });
  return n;
}

// Raw-record data is already the BF16 words: words 0..5 come from the
// SlabBuf, words 6 and 7 are read here.
template <typename Emit>
__device__ __forceinline__ void raw_tail(const SlabBuf& b, uint4 w6, uint4 w7, Emit&& emit) {
  static_for<0, 6>([&](auto st) { emit(st, b.v[st]); });
  emit(std::integral_constant<int, 6>{}, w6);
  emit(std::integral_constant<int, 7>{}, w7);
}

template <typename Emit>
__device__ __forceinline__ void raw_words(const SlabBuf& b, const uint8_t* rec, int t, Emit&& emit) {
  raw_tail(b, ld16_nt(rec + 16 * (256 * 6 + t)), ld16_nt(rec + 16 * (256 * 7 + t)), emit);
}

template <typename Emit>
__device__ __forceinline__ void raw_words(const SlabBuf& b, rsrc_t r, int slab, int nt, Emit&& emit) {
  raw_tail(b, rld16(r, 16 * nt, 4096 * 6 + 1024 * slab), rld16(r, 16 * nt, 4096 * 7 + 1024 * slab), emit);
}

// Butterfly partner values across 16- and 32-lane halves with the gfx950
// lane-swap instructions (VALU, no LDS round trip): v_permlane16_swap swaps
// the odd 16-lane rows of its first operand with the even rows of its
// second, v_permlane32_swap the upper half of the first with the lower half
// of the second; with both operands x, each lane ends up holding its own
// value in one result and its partner's (lane ^ 16, lane ^ 32) in the other,
// so a symmetric op of the two results is the butterfly step.
__device__ __forceinline__ float xor16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Table words of one (kv, head): primary bytes and the 16-byte extended table.
struct HeadLut {
  uint32_t p0, p1;
  uint32_t s[4];
};

__device__ __forceinline__ HeadLut load_lut(const uint32_t* plut, const uint8_t* slut, int idx) {
  HeadLut t;
  t.p0 = plut[2 * idx];
  t.p1 = plut[2 * idx + 1];
  const uint4 s = *reinterpret_cast<const uint4*>(slut + 16 * idx);
  t.s[0] = s.x;
  t.s[1] = s.y;
  t.s[2] = s.z;
  t.s[3] = s.w;
  return t;
}

}  // namespace fp
