// Split-KV decode attention straight from FragPack records (gfx950).
//
// Reference path: fragpack/ops/fused_attn_decode.cu (plan_decode :94-163,
// decode_attn :214-404, combine :407-425, host fused_decode :429-478) and the
// Python contract fragpack/ops/fused_attn_decode.py:41-219.
//
// Design (MI355X):
// * One work unit = one 256-thread workgroup (4 wavefronts) walking a chunk
//   of pages of one (sequence, KV head) with an online softmax.  Per page,
//   wave w decodes slab w (kernel-order threads 64w..64w+63) of the K record
//   -- tokens 32w..32w+31 -- and then slab w of the V record -- dims
//   32w..32w+31 --, so a page costs each wave two decode passes.  Two
//   workgroup barriers per page: (1) escapes staged and the previous page's
//   V pass done, (2) page maxima known and P tile written (the softmax runs
//   speculatively against the running max; a third barrier only when the
//   page max outruns it).
// * Lane l decodes kernel-order thread nt = 32 hh + 4 g + c of its slab, with
//   c = l >> 4, hh = (l >> 3) & 1, g = l & 7.  With that assignment the
//   decoded words are directly the A operands of v_mfma_f32_16x16x32_bf16:
//   MFMA row = l % 16 indexes the token (K) or dim (V) and the four 16-lane
//   groups (= c) hold disjoint dim (K) or token (V) sets, so KV data never
//   moves between lanes.
// * S^T = K Q^T and O^T += V^T P^T with the group's query heads in the MFMA
//   N = 16 columns (heads >= G are zero).  Q and P pass through LDS fragment
//   tiles; each wave keeps O for its 32 dims.
// * Escape bytes of a slab are expanded into wave-private LDS; each lane
//   finds its escapes with a kernel-order prefix scan across the wave.
// * Split-KV partials are merged in the same kernel: the last workgroup to
//   finish a (sequence, head) merges all its chunks.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include <mutex>

#include "../../include/fragpack_hip.h"
#include "fp_capi_internal.hpp"
#include "fp_record.hpp"

namespace fp {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float float2v __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;     // wavefronts per workgroup = slabs per record
constexpr int kBtLds = 1024;  // block-table entries a planning launch may hold in LDS
constexpr int kAttnPerCu = 3;  // resident workgroups per CU (kWaves = SIMDs per CU; VGPR budget 512 / 3)
// Launches with few (sequence, KV head) pairs split every sequence into many
// chunks, and the merge of a pair's partials (one workgroup reading 4 KB per
// chunk through one CU) sets their tail.  They run workgroups of two halves
// (8 waves, one workgroup per CU): each half is a 4-wave unit walking every
// other page of the workgroup's chunk, the halves combine in LDS, and a pair
// has half the chunks to merge.
constexpr int kHalvesPairs = 32;  // batch x kv_heads up to which launches use two halves
constexpr float kLazyMax = 8.f;    // log2 headroom of the speculative softmax reference
constexpr int kTileRow = 4 * 4 * 16 + 16;   // one head's row of a fragment tile, padded by a chunk
constexpr int kTileBytes = 8 * kTileRow;    // Q / P fragment tile: [head 8][a 4][c 4] x 16 B

struct AttnParams {
  const uint16_t* q;
  const int64_t* rec_addr;
  const int32_t* rec_len;
  const uint32_t* plut;
  const uint8_t* slut;
  const int32_t* block_table;
  const int32_t* seq_lens;
  int32_t* plan;
  float* opart;
  float* ml;
  uint16_t* out;
  int32_t* done;      // [kvh, units] merge-group counters (zero between launches)
  int64_t q_stride;   // BF16 elements between sequences
  int64_t out_stride;
  int64_t bt_stride;  // entries between block-table rows
  int kvh, group, units, batch;
  int ud_off;  // int32 offset of the unit descriptors in plan
  int slots;   // resident workgroups of this kernel on the device
  int halves;  // 2: two 4-wave halves per workgroup, each taking every other page
  int inline_plan;  // 1: every workgroup plans for itself (batch <= 64)
  int bt_lds;       // inline plan and the whole block table (batch x bt_stride <= kBtLds) read into LDS
  float scale_log2;
  float lazy;  // kLazyMax / scale_log2: the softmax reference's headroom in score units
};

// Plan layout (int32): [0] ppc, [1] units in use, [2, 2 + 2 units) (sequence, first
// page) per unit (sequence -1: idle), [2 + 2 units, 2 + 4 units) (first
// unit, chunks) per sequence -- the reference's layout --, then at
// ud_offset(units) 8 ints per unit (sequence, first page, pages, context,
// first unit, chunks, block of page 0, block of page 1).  The units * kvh
// merge counters are the last words of the plan buffer: their place does not
// depend on ``units``, so counters left at zero by a call stay zero for the
// next one even when its unit count (and so its plan layout) differs.
__host__ __device__ __forceinline__ int ud_offset(int units) { return (2 + 4 * units + 7) & ~7; }

__device__ __forceinline__ int pages_of(const int32_t* seq_lens, int b) { return (seq_lens[b] + 127) >> 7; }

// Work plan (layout of the reference planner, fused_attn_decode.cu:48-163;
// policy of this build).  Every sequence is cut into chunks of ``ppc``
// pages.  The reference takes the smallest ``ppc`` whose chunks fit one wave
// of units; on gfx950 the attention grid is persistent (``slots`` resident
// workgroups over all KV heads), so ``ppc`` is chosen to minimise the
// modelled makespan instead:
//   cost(ppc) = ceil(chunks(ppc) * kvh / slots) * (ppc + kUnitCost)
// over the candidates ppc = ceil(longest / c), c = 1..kPlanCands, with
// chunks(ppc) <= units; ties go to the larger ppc.  Each wave scores
// kPlanCands / 16 candidates with the page counts in registers (one DPP
// reduction per candidate, division by a reciprocal); wave 0 then writes
// each sequence's first unit and every thread fills the descriptors of its
// units, locating the sequence by binary search over the first units (in LDS
// up to kPlanLds sequences).  The descriptors also carry the first two block
// ids of each chunk.  plan[1] holds the number of units in use.
constexpr int kPlanCache = 16;  // page counts of batch <= 64 * 16 kept in registers
constexpr int kPlanThreads = 1024;
constexpr int kPlanWaves = kPlanThreads / 64;
constexpr int kPlanLds = 8192;
constexpr int kPlanCands = 64;
constexpr int kUnitCost = 1;  // fixed cost of a unit (metadata, Q, merge) in pages

// x / d for 0 <= x < 2^22, 1 <= d.  inv is the hardware reciprocal (relative
// error <= 2^-23), so x * inv is within 1.5 * 2^-23 * x / d < 0.75 of x / d:
// its truncation is off by at most one, which div's two steps correct.
struct Divider {
  int d;
  float inv;
  __device__ explicit Divider(int d_) : d(d_), inv(__builtin_amdgcn_rcpf((float)d_)) {}
  __device__ __forceinline__ int div(int x) const {
    int q = (int)((float)x * inv);
    q += (q + 1) * d <= x;
    q -= q * d > x;
    return q;
  }
  __device__ __forceinline__ int chunks(int pages) const { return div(pages + d - 1); }
};

__global__ void __launch_bounds__(kPlanThreads) plan_kernel(const int32_t* __restrict__ seq_lens,
                                                            const int32_t* __restrict__ block_table, int64_t bt_stride,
                                                            int32_t* __restrict__ plan, int64_t plan_elems, int batch,
                                                            int units, int kvh, int slots, int halves) {
  __shared__ int firsts[kPlanLds + 1];
  __shared__ unsigned long long best;
  __shared__ int shared_used;
  int32_t* seq_plan = plan + 2 + 2 * units;
  const bool lds = batch <= kPlanLds;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (threadIdx.x == 0) best = ~0ull;
  int pg[kPlanCache];
  int longest = 0;
  static_for<0, kPlanCache>([&](auto k) {
    pg[k] = 0;
    if (64 * k < batch) {
      const int b = lane + 64 * k;
      pg[k] = b < batch ? pages_of(seq_lens, b) : 0;
      longest = max(longest, pg[k]);
    }
  });
  for (int b = lane + 64 * kPlanCache; b < batch; b += 64) longest = max(longest, pages_of(seq_lens, b));
  longest = wave_total<true>(longest);
  auto count_chunks = [&](int ppc) {
    const Divider dv(ppc);
    int c = 0;
    static_for<0, kPlanCache>([&](auto k) {
      if (64 * k < batch) c += dv.chunks(pg[k]);
    });
    for (int b = lane + 64 * kPlanCache; b < batch; b += 64) c += dv.chunks(pages_of(seq_lens, b));
    return wave_total<false>(c);
  };
  __syncthreads();  // best initialised
  for (int k = 0; k < kPlanCands / kPlanWaves; ++k) {
    const int c = wave * (kPlanCands / kPlanWaves) + k + 1;
    const int ppc = max(1, (longest + c - 1) / c);
    const int n = count_chunks(ppc);
    if (n <= units && lane == 0) {
      const int64_t rounds = ((int64_t)n * kvh + slots - 1) / slots;
      const uint64_t cost = (uint64_t)(rounds * ((ppc + halves - 1) / halves + kUnitCost));
      atomicMin(&best, (cost << 24) | (uint64_t)(0xFFFFFF - ppc));
    }
  }
  __syncthreads();
  const int ppc = 0xFFFFFF - (int)(best & 0xFFFFFFu);
  if (wave == 0) {
    const Divider dv(ppc);
    int used = 0;
    auto place = [&](int b, int n) {
      const int c = dv.chunks(n);
      const int incl = wave_scan_dpp<false>(c);
      const int first = used + incl - c;
      if (b < batch) {
        seq_plan[2 * b] = first;
        seq_plan[2 * b + 1] = c;
        if (lds) firsts[b] = first;
      }
      used += __builtin_amdgcn_readlane(incl, 63);
    };
    static_for<0, kPlanCache>([&](auto k) {
      if (64 * k < batch) place(lane + 64 * k, pg[k]);
    });
    for (int base = 64 * kPlanCache; base < batch; base += 64) {
      const int b = base + lane;
      place(b, b < batch ? pages_of(seq_lens, b) : 0);
    }
    if (lane == 0) {
      if (lds) firsts[batch] = used;
      shared_used = used;
      plan[0] = ppc;
      plan[1] = used;
    }
  }
  __syncthreads();
  const int used = shared_used;
  const int ud0 = ud_offset(units);
  auto first_of = [&](int b) { return b == batch ? used : lds ? firsts[b] : seq_plan[2 * b]; };
  for (int u = threadIdx.x; u < units; u += kPlanThreads) {
    int4* ud = reinterpret_cast<int4*>(plan + ud0 + 8 * u);
    if (u >= used) {
      plan[2 + 2 * u] = -1;
      plan[ud0 + 8 * u] = -1;
      continue;
    }
    // the last sequence whose first unit is <= u owns u (empty sequences
    // share their successor's first unit)
    int lo = 0, hi = batch - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (first_of(mid) <= u)
        lo = mid;
      else
        hi = mid - 1;
    }
    const int b = lo, first = first_of(b), c = first_of(b + 1) - first;
    const int seq = seq_lens[b], n = (seq + 127) >> 7;
    const int p0 = (u - first) * ppc, np = min(n, p0 + ppc) - p0;
    const int32_t* bt = block_table + (int64_t)b * bt_stride;
    plan[2 + 2 * u] = b;
    plan[3 + 2 * u] = p0;
    ud[0] = make_int4(b, p0, np, seq);
    ud[1] = make_int4(first, c, bt[p0], np > 1 ? bt[p0 + 1] : 0);
  }
  // merge counters of the fused merge, for every unit count the buffer
  // holds: everything past this plan's words.  The last arrival of a
  // (sequence, head) resets its counter, so zeroing is needed only here.
  for (int64_t x = ud0 + 8 * units + threadIdx.x; x < plan_elems; x += kPlanThreads) plan[x] = 0;
}

__device__ __forceinline__ f32x4 mfma(const uint4& a, const uint4& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}


// A operand of MFMA (j, a) from words 2a (w0) and 2a+1 (w1) of a lane's
// decoded thread: slots (x, f, e) = word 2a + x, dword 2j + f, half e.
__device__ __forceinline__ uint4 a_frag(const uint4& w0, const uint4& w1, int j) {
  return j == 0 ? make_uint4(w0.x, w0.y, w1.x, w1.y) : make_uint4(w0.z, w0.w, w1.z, w1.w);
}

// Lane of the natural (kernel-order) thread ``nt`` of a slab.
__device__ __forceinline__ int lane_of_natural(int nt) { return 16 * (nt & 3) + 8 * (nt >> 5) + ((nt >> 2) & 7); }

// A record as the workgroup sees it (uniform values): its address and length;
// the 32 KB buffer resource over it is built at each use (two of its four
// words are constants), which keeps three scalar registers per live record.
struct RecRef {
  uint32_t lo, hi;
  int vlen;  // bytes past the dense part; > kVarCap marks a raw record
  __device__ __forceinline__ rsrc_t rs(int bytes = kRawRecord) const {
    return make_rsrc(reinterpret_cast<const uint8_t*>((uint64_t)lo | ((uint64_t)hi << 32)), bytes);
  }
};

__device__ __forceinline__ RecRef make_ref(uint32_t lo, uint32_t hi, int vlen) { return RecRef{lo, hi, vlen}; }

// Record metadata of up to 64 pages of a unit, page i in lane i: K / V
// record address (lo, hi) and length.
struct PageMeta {
  uint32_t klo, khi, vlo, vhi;
  int klen, vlen;
};

// Block id of page base + lane of the unit (-1 past its pages).
__device__ __forceinline__ int load_block(const int32_t* bt, int base, int npages, int lane) {
  return base + lane < npages ? bt[base + lane] : -1;
}

__device__ __forceinline__ PageMeta load_meta(const AttnParams& p, int blk, int h) {
  PageMeta m{0u, 0u, 0u, 0u, kRawVarLen, kRawVarLen};
  if (blk >= 0) {
    const int64_t kidx = ((int64_t)blk * 2) * p.kvh + h;
    const uint64_t ka = (uint64_t)p.rec_addr[kidx], va = (uint64_t)p.rec_addr[kidx + p.kvh];
    m.klo = (uint32_t)ka;
    m.khi = (uint32_t)(ka >> 32);
    m.vlo = (uint32_t)va;
    m.vhi = (uint32_t)(va >> 32);
    m.klen = p.rec_len[kidx];
    m.vlen = p.rec_len[kidx + p.kvh];
  }
  return m;
}

__device__ __forceinline__ RecRef page_ref(const PageMeta& m, int i, int kv) {
  const int l = i & 63;
  return kv == 0 ? make_ref(__builtin_amdgcn_readlane(m.klo, l), __builtin_amdgcn_readlane(m.khi, l),
                            __builtin_amdgcn_readlane(m.klen, l))
                 : make_ref(__builtin_amdgcn_readlane(m.vlo, l), __builtin_amdgcn_readlane(m.vhi, l),
                            __builtin_amdgcn_readlane(m.vlen, l));
}

// Prefetches are issued on every path through the page loop, the same
// instructions whether a record is coded or raw, present or not (``live``
// false: the loads run against an empty range, return zeros and move no
// data).  The compiler's wait before a decode then names exactly the loads
// of the slab it reads; with a path that issues fewer loads it would also
// wait on the prefetches issued after that slab (up to a memory round trip
// per page).

// Dense words of the wave's slab ``slab`` of record ``r``.
__device__ __forceinline__ void prefetch_dense(const RecRef& r, int slab, int nt, SlabBuf& b, bool live = true) {
  load_slab(r.rs(live ? kRawRecord : 0), live && r.vlen > kVarCap, slab, nt, b);
}

// This lane's 8 bytes (at 512 w + 8 lane) of the record's variable region;
// zeros for a wave whose quarter lies past the region (or a raw record).
__device__ __forceinline__ bool quarter_used(const RecRef& r, int w) { return r.vlen <= kVarCap && 512 * w < r.vlen; }

__device__ __forceinline__ uint2 prefetch_var(const RecRef& r, int w, int lane, bool live = true) {
  return rld8(r.rs(live && quarter_used(r, w) ? kRawRecord : 0), 8 * lane, kDenseBytes + 512 * w);
}

// Per-record escape staging, done by all four waves from their prefetched
// quarters of the variable region: (1) nibble bytes -> table bytes into the
// record's LDS escape area (byte k = escape ordinal k) and the header into
// LDS; then, after a barrier, (2) raw-list entries patch their escapes.
__device__ __forceinline__ void expand_var(const RecRef& r, uint2 v, int w, int lane, const uint32_t (&sl)[4],
                                           uint8_t* esc, uint32_t* hdr) {
  if (!quarter_used(r, w)) return;
  const int o = 512 * w + 8 * lane;
  if (o >= kHeaderBytes) {
    const uint2 e0 = expand_nibbles(v.x, sl), e1 = expand_nibbles(v.y, sl);
    *reinterpret_cast<uint4*>(esc + 2 * (o - kHeaderBytes)) = make_uint4(e0.x, e0.y, e1.x, e1.y);
  } else {
    hdr[o >> 2] = v.x;
    hdr[(o >> 2) + 1] = v.y;
  }
}

__device__ __forceinline__ void patch_raw(const RecRef& r, uint2 v, int w, int lane, uint8_t* esc,
                                          const uint32_t* hdr) {
  if (!quarter_used(r, w)) return;
  const int n_raw = (int)hdr[1], raw_offset = (int)hdr[2];
  const int o = 512 * w + 8 * lane;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int off = o + 4 * q;
    if (off >= raw_offset && ((off - raw_offset) >> 2) < n_raw) {
      const uint32_t e = q ? v.y : v.x;
      const int x = (int)(e & 0xFFFFu);
      if (x < kEscLds) esc[x] = (uint8_t)(e >> 16);
    }
  }
}

// Byte addresses for ds_bpermute between lane order and kernel order
// (natural index 32 hh + 4 g + c <-> lane 16 c + 8 hh + g): ``to_nat`` makes
// lane i read the lane holding kernel-order thread i, ``from_nat`` makes a
// lane read position ``nt``.
struct NatPerm {
  int to_nat, from_nat;
};

// Exclusive prefix (in kernel order) of ``cnt`` over the wave: counts moved
// into kernel order, a DPP inclusive scan, and moved back.
__device__ __forceinline__ int natural_prefix(int cnt, NatPerm np) {
  const int y = __builtin_amdgcn_ds_bpermute(np.to_nat, cnt);
  const int incl = wave_scan_dpp<false>(y);
  return __builtin_amdgcn_ds_bpermute(np.from_nat, incl) - cnt;
}

// Fragment tile [head 8][a 4][c 4] x 16 B: lane (c, n) reads its 8 BF16 of
// k-chunk a from chunk (a * 4 + c) of head row n & 7.  Used for Q (dims) and
// P (tokens).  Head rows are kTileRow = 272 B apart, one LDS bank row (256 B)
// plus one chunk, so the eight heads' chunks of one (a, c), which lanes read
// together, start four banks apart instead of all in the same four banks;
// the k-chunk stays an immediate offset (a * 64).
__device__ __forceinline__ int tile_chunk(int n, int a, int c) { return (n & 7) * kTileRow + (a * 4 + c) * 16; }
__device__ __forceinline__ uint4 tile_frag(const uint8_t* tile, int n, int a, int c) {
  return *reinterpret_cast<const uint4*>(tile + tile_chunk(n, a, c));
}

// Decodes this lane's kernel-order thread ``nt`` of the wave's slab ``w`` of
// record ``r`` (escapes staged in ``esc``, header in ``hdr``) and calls
// pair(a, word 2a, word 2a + 1, fragment a of ``tile``) for a = 0..3.  A raw
// record's words come in natural slot order, a coded record's in even-odd
// order (decode_words<true>): ``tile`` must be laid out in the same order,
// or, with kTileEvenOdd, is always in even-odd order and is permuted here for
// a raw record.
template <bool kTileEvenOdd = false, typename Pair>
__device__ __forceinline__ void decode_slab(const RecRef& r, const SlabBuf& b, int w, int nt, NatPerm np,
                                            const HeadLut& lut, const uint8_t* esc, const uint32_t* hdr,
                                            const uint8_t* tile, int n, int c, Pair&& pair) {
  uint4 fr[4];
#pragma unroll
  for (int a = 0; a < 4; ++a) fr[a] = tile_frag(tile, n, a, c);
  if (kTileEvenOdd && r.vlen > kVarCap) {
    // slots (4x + 2e + f) -> (4x + 2f + e): dwords (e0f0, e0f1), (e1f0, e1f1)
    // become (f0e0, f0e1), (f1e0, f1e1)
#pragma unroll
    for (int a = 0; a < 4; ++a)
      fr[a] = make_uint4(perm(fr[a].y, fr[a].x, 0x05040100u), perm(fr[a].y, fr[a].x, 0x07060302u),
                         perm(fr[a].w, fr[a].z, 0x05040100u), perm(fr[a].w, fr[a].z, 0x07060302u));
  }
  uint4 prev;
  auto emit = [&](auto st_c, const uint4& wd) {
    constexpr int st = decltype(st_c)::value;
    if constexpr (st & 1)
      pair(std::integral_constant<int, (st >> 1)>{}, prev, wd, fr[st >> 1]);
    else
      prev = wd;
  };
  if (r.vlen > kVarCap) {
    raw_words(b, r.rs(), w, nt, emit);
    return;
  }
  const int e0 = (int)(hdr[4 + w] & 0xFFFFu);  // esc_prefix[2 w]
  const int excl = natural_prefix(thread_escapes(b), np);
  decode_words<true>(b, esc, e0 + excl, lut.p0, lut.p1, emit);
}

struct alignas(16) AttnShared {
  uint8_t esc[2][2][kEscLds];  // [page parity][K, V] expanded escape bytes
  uint32_t hdr[2][2][12];      // [page parity][K, V] record headers
  uint8_t pt[kTileBytes];      // P tile
  uint8_t qt[kTileBytes];      // Q tile, even-odd slot order
  float red[kWaves][8];        // per-wave page max / final l per head
  float mrun[8];               // the running max per head before this page (two-half workgroups)
  int last;
};

// The planner of plan_kernel, run by a single wavefront for batch <= 64
// (sequence b in lane b): lane c scores candidate ppc = ceil(longest / (c+1))
// with the same cost and tie rule, then every lane holds its sequence's page
// count, first unit and chunk count.  Used when the attention kernel plans
// for itself (no separate plan launch).
struct InlinePlan {
  int len, n, first, cnt;  // per lane (sequence = lane)
  int ppc, used;           // uniform
};

// One step of a wavefront prefix minimum of u64 keys by DPP: both halves
// move with the same control; lanes without a source (shifted in, or rows
// masked off) read all ones, the identity.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint64_t dpp_min_u64(uint64_t x) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)(uint32_t)x, kCtrl, kRowMask, 0xf, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)(uint32_t)(x >> 32), kCtrl, kRowMask, 0xf, false);
  const uint64_t y = ((uint64_t)hi << 32) | lo;
  return y < x ? y : x;
}

// Minimum over the wavefront (uniform), by a DPP prefix scan (row shifts,
// then row broadcasts; lane 63 ends with the minimum): VALU only, where a
// butterfly of lane shuffles costs an LDS round trip per step.
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t x) {
  x = dpp_min_u64<0x111, 0xf>(x);  // row_shr:1
  x = dpp_min_u64<0x112, 0xf>(x);  // row_shr:2
  x = dpp_min_u64<0x114, 0xf>(x);  // row_shr:4
  x = dpp_min_u64<0x118, 0xf>(x);  // row_shr:8
  x = dpp_min_u64<0x142, 0xa>(x);  // row_bcast:15
  x = dpp_min_u64<0x143, 0xc>(x);  // row_bcast:31
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)x, 63);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(x >> 32), 63);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ InlinePlan inline_plan(const AttnParams& p, int lane, int len) {
  InlinePlan r;
  r.len = len;
  r.n = (r.len + 127) >> 7;
  const int longest = wave_total<true>(r.n);
  const int cand = max(1, Divider(lane + 1).div(longest + lane));
  const Divider dv(cand);
  int chunks = 0;
  for (int b = 0; b < p.batch; ++b) chunks += dv.chunks(__builtin_amdgcn_readlane(r.n, b));
  uint64_t key = ~0ull;
  if (chunks <= p.units) {
    // (chunks * kvh + slots < 2^22 for an inline-planning launch: Divider's range)
    const int rounds = Divider(p.slots).div(chunks * p.kvh + p.slots - 1);
    key = ((uint64_t)(rounds * ((cand + p.halves - 1) >> (p.halves - 1)) + rounds * kUnitCost) << 24) |
          (uint64_t)(0xFFFFFF - cand);
  }
  key = wave_min_u64(key);
  r.ppc = uniform(0xFFFFFF - (int)(key & 0xFFFFFFu));
  r.cnt = Divider(r.ppc).chunks(r.n);
  const int incl = wave_scan_dpp<false>(r.cnt);
  r.first = incl - r.cnt;
  r.used = __builtin_amdgcn_readlane(incl, 63);
  return r;
}

// Split-KV merge of (b, h) after this workgroup wrote the partial of one of
// its ``chunks`` units (``first`` .. ``first + chunks - 1``): the last
// workgroup to arrive merges all of them with the online-softmax merge in the
// log2 domain (the reference's combine, fused_attn_decode.cu:407-425) and
// writes the BF16 output rows.  One level: partials are read in batches of
// kMergeBatch with every load of a batch issued before any is used.  Thread t
// covers row t >> 5 (query head), dims 4 (t & 31) .. + 3.  The counter
// p.done[h * units + first] is left at zero.
constexpr int kMergeBatch = 16;
__device__ __forceinline__ void merge_chunks(const AttnParams& p, AttnShared& sh, int b, int h, int first, int chunks) {
  wait_stores();  // this workgroup's partial is at the coherence point
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t* cnt = p.done + (int64_t)h * p.units + first;
    const int last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == chunks - 1;
    if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sh.last = last;
  }
  __syncthreads();
  if (!sh.last) return;
  const int t = threadIdx.x, g = t >> 5, d = 4 * (t & 31);
  if (g >= p.group) return;
  const rsrc_t ro = coh_rsrc(p.opart), rm = coh_rsrc(p.ml);
  const int64_t row0 = ((int64_t)h * p.units + first) * 8 + g;
  float gm = -INFINITY, l = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int k0 = 0; k0 < chunks; k0 += kMergeBatch) {
    float2 ms[kMergeBatch];
    float4 o[kMergeBatch];
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      if (k0 + k < chunks) {
        const int64_t r = row0 + (int64_t)(k0 + k) * 8;
        ms[k] = ld_coh2(rm, r * 2);
        o[k] = ld_coh4(ro, r * kDim + d);
      }
    }
    float bm = -INFINITY;
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k)
      if (k0 + k < chunks) bm = fmaxf(bm, ms[k].x);
    const float nm = fmaxf(gm, bm);
    if (nm == -INFINITY) continue;
    const float alpha = __builtin_amdgcn_exp2f(gm - nm);
    l *= alpha;
    acc.x *= alpha;
    acc.y *= alpha;
    acc.z *= alpha;
    acc.w *= alpha;
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      if (k0 + k < chunks) {
        const float w = __builtin_amdgcn_exp2f(ms[k].x - nm);
        l += w * ms[k].y;
        acc.x += w * o[k].x;
        acc.y += w * o[k].y;
        acc.z += w * o[k].z;
        acc.w += w * o[k].w;
      }
    }
    gm = nm;
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const uint32_t lo = pack_bf16x2(acc.x * inv, acc.y * inv);
  const uint32_t hi = pack_bf16x2(acc.z * inv, acc.w * inv);
  *reinterpret_cast<uint2*>(p.out + (int64_t)b * p.out_stride + (int64_t)(h * p.group + g) * kDim + d) =
      make_uint2(lo, hi);
}

// (a two-half workgroup runs alone on its CU, two waves per SIMD: it may use
// the whole 256-register budget)
template <bool kInlinePlan, int kHalves>
__global__ void __launch_bounds__(64 * kWaves * kHalves) __attribute__((amdgpu_waves_per_eu(kHalves == 2 ? 2 : kAttnPerCu)))
attn_kernel(AttnParams pk) {
  // Two-half launches pass the scalar parameters through an empty asm once,
  // at entry, so the compiler keeps them in SGPRs instead of reloading them
  // from the kernel arguments (dependent scalar-load round trips) where they
  // are used: in a planning launch those reloads sat between the plan and the
  // first unit.  The pointers stay as they are (an asm operand would lose
  // their address space and turn their loads into flat loads).  One-half
  // launches skip it: the longer-lived SGPRs would spill VGPRs there.
  AttnParams p = pk;
  if constexpr (kHalves == 2) {
    asm volatile("" : "+s"(p.q_stride), "+s"(p.out_stride), "+s"(p.bt_stride), "+s"(p.kvh), "+s"(p.group), "+s"(p.units),
                 "+s"(p.batch), "+s"(p.ud_off), "+s"(p.slots), "+s"(p.halves), "+s"(p.bt_lds), "+s"(p.scale_log2), "+s"(p.lazy));
  }
  __shared__ AttnShared shs[kHalves];
  const int lane = wave_lane();
  const int wave = uniform((int)(threadIdx.x >> 6));
  const int w = wave & (kWaves - 1);          // this wave's slab of every record (wave-uniform)
  const int half = kHalves == 2 ? wave >> 2 : 0;  // this wave's half of the workgroup
  AttnShared& sh = shs[half];
  const int h = blockIdx.y;
  const int c = lane >> 4, hh = (lane >> 3) & 1, g = lane & 7;
  const int nt = 32 * hh + 4 * g + c;
  const NatPerm np{4 * lane_of_natural(lane), 4 * nt};
  const int n = lane & 15;  // MFMA column = query head within the group
  const HeadLut klut = load_lut(p.plut, p.slut, h);
  const HeadLut vlut = load_lut(p.plut, p.slut, p.kvh + h);

  // the work plan: planned here (inline) or read from the plan workspace
  InlinePlan ip{0, 0, 0, 0, 1, 0};
  // Planning launches with a small block table read all of it into LDS
  // beside the plan's sequence lengths, so a unit's page ids need no
  // global round trip after the plan is known.
  __shared__ int bt_s[kInlinePlan ? kBtLds : 1];
  // the inline plan per wave: first unit, chunks, context, pages by sequence
  __shared__ int plan_s[kInlinePlan ? kWaves * kHalves : 1][4][64];
  int(&wplan)[4][64] = plan_s[kInlinePlan ? wave : 0];  // this wave's rows
  const bool bt_lds = kInlinePlan && p.bt_lds;
  // A planning launch's first global hop carries the sequence lengths and the
  // block table together (the table's LDS stores wait only for its own loads).
  const int len0 = kInlinePlan && lane < p.batch ? p.seq_lens[lane] : 0;
  if (bt_lds) {
    constexpr int kStride = 64 * kWaves * kHalves;
    int v[(kBtLds + kStride - 1) / kStride];
#pragma unroll
    for (int k = 0; k < (kBtLds + kStride - 1) / kStride; ++k) {
      const int i = threadIdx.x + k * kStride;
      v[k] = i < p.batch * (int)p.bt_stride ? p.block_table[i] : 0;
    }
#pragma unroll
    for (int k = 0; k < (kBtLds + kStride - 1) / kStride; ++k) {
      const int i = threadIdx.x + k * kStride;
      if (i < p.batch * (int)p.bt_stride) bt_s[i] = v[k];
    }
  }
  if constexpr (kInlinePlan) ip = inline_plan(p, lane, len0);
  if (bt_lds) __syncthreads();
  // units in use; a launch reusing the plan walks its units until the first
  // idle one instead (every planner marks units [used, units) idle), so its
  // first hop is the unit descriptor itself, not the plan's unit count
  const int used = kInlinePlan ? ip.used : p.units;
  const int ppc = ip.ppc;
  if constexpr (kInlinePlan) {
    // the per-sequence plan goes to this wave's LDS rows (read back by
    // sequence), so its four registers are free during the page loop
    wplan[0][lane] = ip.first;
    wplan[1][lane] = ip.cnt;
    wplan[2][lane] = ip.len;
    wplan[3][lane] = ip.n;
    // lanes read each other's rows below: order the stores before those
    // reads for the compiler too (the wave's LDS accesses are in order)
    wave_lds_sync();
  }
  for (int unit = blockIdx.x; unit < used; unit += gridDim.x) {
    int b, p0, npages, seq, first, chunks, blk0, blk1;
    if constexpr (kInlinePlan) {
      // the last live sequence whose first unit is <= unit owns it
      const uint64_t own = __ballot(lane < p.batch && wplan[1][lane] > 0 && wplan[0][lane] <= unit);
      b = 63 - __builtin_clzll(own);
      first = uniform(wplan[0][b]);
      chunks = uniform(wplan[1][b]);
      seq = uniform(wplan[2][b]);
      p0 = (unit - first) * ppc;
      npages = min(uniform(wplan[3][b]), p0 + ppc) - p0;
      // the first two block ids: LDS and global reads in separate branches
      // (one read through a generic pointer would be a flat load, whose
      // wait also waits for every store in flight)
      if (bt_lds) {
        const int bt0 = b * (int)p.bt_stride + p0;  // < batch x bt_stride <= kBtLds
        blk0 = uniform(bt_s[bt0]);
        blk1 = npages > 1 ? uniform(bt_s[bt0 + 1]) : 0;
      } else {
        asm volatile("" ::: "memory");
        const int32_t* row = p.block_table + (int64_t)b * p.bt_stride + p0;
        blk0 = uniform(row[0]);
        blk1 = npages > 1 ? uniform(row[1]) : 0;
      }
    } else {
      // unit descriptor: b, first page, pages, context, first unit of b,
      // chunks of b, block of page 0 (both halves loaded together)
      const int4* udp = reinterpret_cast<const int4*>(p.plan + p.ud_off + 8 * unit);
      const int4 u0 = udp[0], u1 = udp[1];
      asm volatile("" ::"v"(u0.x), "v"(u0.y), "v"(u0.z), "v"(u0.w), "v"(u1.x), "v"(u1.y), "v"(u1.z), "v"(u1.w));  // one hop
      b = uniform(u0.x);
      if (b < 0) break;  // idle: so are this workgroup's later units
      p0 = uniform(u0.y);
      npages = uniform(u0.z);
      seq = uniform(u0.w);
      first = uniform(u1.x);
      chunks = uniform(u1.y);
      blk0 = uniform(u1.z);
      blk1 = uniform(u1.w);
    }
    // a two-half workgroup: half 1 starts at page 1 (with a single page it
    // runs page 0 with every key masked)
    const int ipage0 = kHalves == 2 ? min(half, npages - 1) : 0;
    const int blkf = ipage0 == 1 ? blk1 : blk0;
    const int32_t* bt = p.block_table + (int64_t)b * p.bt_stride + p0;
    // Q rows of the group, issued first so they overlap the record-table
    // hop: wave 0 loads 16-byte pieces L = lane, lane + 64 (row L / 16, u32
    // pairs 4 (L % 16) .. + 3); rows >= group are zero.
    uint4 qv[2];
    if (w == 0) {
      // a buffer resource over the group's rows: pieces past them read zero
      const rsrc_t rq = make_rsrc(p.q + (int64_t)b * p.q_stride + (int64_t)h * p.group * kDim, p.group * kDim * 2);
      qv[0] = bld16(rq, 16 * lane, 0);
      qv[1] = bld16(rq, 16 * lane, 1024);
    }
    // block ids of the unit's first 64 pages (one per lane), in the same hop
    // as page 0's record tables, which come straight from the descriptor's
    // block id
    const int blk = bt_lds && kInlinePlan ? (lane < npages ? bt_s[(b * (int)p.bt_stride + p0 + lane) % kBtLds] : -1)
                                          : load_block(bt, 0, npages, lane);
    RecRef kr, vr;
    {
      const int64_t kidx = ((int64_t)blkf * 2) * p.kvh + h;
      const int64_t ka = p.rec_addr[kidx], va = p.rec_addr[kidx + p.kvh];
      const int kl = p.rec_len[kidx], vl = p.rec_len[kidx + p.kvh];
      asm volatile("" ::"v"(ka), "v"(va), "v"(kl), "v"(vl));  // all four in one hop
      kr = make_ref((uint32_t)uniform64(ka), (uint32_t)((uint64_t)uniform64(ka) >> 32), uniform(kl));
      vr = make_ref((uint32_t)uniform64(va), (uint32_t)((uint64_t)uniform64(va) >> 32), uniform(vl));
    }
    // page 0: dense K slab and both variable regions, in flight before the
    // workgroup synchronises; then the metadata of the unit's other pages
    SlabBuf fk, fv;
    prefetch_dense(kr, w, nt, fk);
    uint2 vk = prefetch_var(kr, w, lane), vv = prefetch_var(vr, w, lane);
    PageMeta meta = load_meta(p, blk, h);

    __syncthreads();  // the previous unit is done with every tile
    // Q into the fragment tile: u32 pair j of row r (dims 2j, 2j + 1 =
    // 32a + 16x + 8f + 2c + e, e = 0, 1) belongs to fragment (r, a, c) at
    // slot 4x + 2e + f (even-odd order; raw K records permute the fragments
    // to natural order 4x + 2f + e in registers).
    if (w == 0) {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int L = lane + 64 * k, row = L >> 4;
        const uint32_t v[4] = {qv[k].x, qv[k].y, qv[k].z, qv[k].w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int j = 4 * (L & 15) + t;
          const int frag = tile_chunk(row, j >> 4, j & 3), x = (j >> 3) & 1, f = (j >> 2) & 1;
          // lanes L and L ^ 1 hold f = 0 and f = 1 of the same (a, c, x):
          // each writes the dword of e = its own f
          const uint32_t o = __shfl_xor(v[t], 1, 64);
          *reinterpret_cast<uint32_t*>(sh.qt + frag + 8 * x + 4 * f) =
              f ? perm(v[t], o, 0x07060302u) : perm(o, v[t], 0x05040100u);
        }
      }
    }
    float m_run = -INFINITY, l_run = 0.f;  // m_run: unscaled score units
    const float lazy = p.lazy;
    f32x4 o0 = {0.f, 0.f, 0.f, 0.f}, o1 = {0.f, 0.f, 0.f, 0.f};
    expand_var(kr, vk, w, lane, klut.s, sh.esc[0][0], sh.hdr[0][0]);
    expand_var(vr, vv, w, lane, vlut.s, sh.esc[0][1], sh.hdr[0][1]);
    // the next page's variable regions: each page's are in flight a page
    // before they are expanded
    RecRef nkr = kr, nvr = vr;
    const bool second = half + kHalves < npages;
    if (second) {
      nkr = page_ref(meta, half + kHalves, 0);
      nvr = page_ref(meta, half + kHalves, 1);
    }
    __syncthreads();
    patch_raw(kr, vk, w, lane, sh.esc[0][0], sh.hdr[0][0]);
    patch_raw(vr, vv, w, lane, sh.esc[0][1], sh.hdr[0][1]);
    vk = prefetch_var(nkr, w, lane, second);
    vv = prefetch_var(nvr, w, lane, second);

    // Workgroups L, L + cus, L + 2 cus (linear id L, cus = slots / kAttnPerCu)
    // share a CU, dispatched in that order; at equal issue priority the
    // oldest runs ahead (measured at config 4's shape: the three finished
    // their units ~30% apart, the CU idling at the end).  Each page step sets
    // the priority to (t + age rank) mod 4, t the device clock
    // (s_memrealtime, 100 MHz) in 5.12 us quanta: at any moment the three
    // hold different priorities, rotating in step.  (Rotating by the page
    // step instead left the oldest a few percent ahead: a workgroup one step
    // ahead of the next-younger shares its priority and wins the tie by age.
    // Measured at config 4: 927-933 us against 935-941 by step; 2.56 and
    // 1.28 us quanta were slower, 10.24 us no faster.)
    const int age = kHalves == 1 ? (int)(blockIdx.y * gridDim.x + blockIdx.x) / max(1, p.slots / kAttnPerCu) : 0;
    // a half takes pages half, half + 2, ...; both halves run the same
    // number of steps (and barriers): a step past a half's pages repeats its
    // last page with every key masked
    const int nsteps = kHalves == 2 ? (npages + 1) >> 1 : npages;
    for (int j = 0; j < nsteps; ++j) {
      rotate_priority(kHalves == 1 ? (int)(((uint32_t)(__builtin_amdgcn_s_memrealtime() >> 9) + (uint32_t)age) & 3u) : j);
      const int i = kHalves == 2 ? min(2 * j + half, npages - 1) : j;  // page of the unit
      const bool act = kHalves == 1 || 2 * j + half < npages;
      const int seq_m = act ? seq : 0;  // context this step's keys are masked against
      const int par = j & 1;
      const bool more = act && i + kHalves < npages, more2 = act && i + 2 * kHalves < npages;
      const int tok0 = (p0 + i) * kTokens;
      // the page after next starts a new window of 64 block ids
      if (more2 && ((i + 2 * kHalves) & 63) < kHalves) {
        meta = load_meta(p, load_block(bt, (i + 2 * kHalves) & ~63, npages, lane), h);
        // read below: waited for here, so that no wait for it reaches the
        // common path (where it would also wait on this page's K slab)
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      }
      // V slab of this page in flight while K is decoded; the variable
      // regions of the page after next in flight for a whole page
      prefetch_dense(vr, w, nt, fv);
      RecRef nnkr = nkr, nnvr = nvr;
      if (more2) {
        nnkr = page_ref(meta, i + 2 * kHalves, 0);
        nnvr = page_ref(meta, i + 2 * kHalves, 1);
      }
      const uint2 vk2 = prefetch_var(nnkr, w, lane, more2), vv2 = prefetch_var(nnvr, w, lane, more2);
      __syncthreads();  // B1: this page's escapes patched; the previous page's V pass done everywhere

      // ---- S^T = K Q^T for tokens 32w .. 32w + 31 ----
      f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
      // (a step past the half's pages decodes nothing: its keys are masked
      // and its V pass is skipped, so no stale escape data reaches O)
      if (act)
        decode_slab<true>(kr, fk, w, nt, np, klut, sh.esc[par][0], sh.hdr[par][0], sh.qt, n, c,
                    [&](auto, const uint4& w0, const uint4& w1, const uint4& qa) {
                      s0 = mfma(a_frag(w0, w1, 0), qa, s0);
                      s1 = mfma(a_frag(w0, w1, 1), qa, s1);
                    });
      // token of s_j[r] = 32 w + 16 (c >> 1) + 8 j + 4 (c & 1) + r
      // Scores stay unscaled (scale > 0 keeps their order; P = exp2(s c - m c)
      // is one FMA and one exp); the page past the context is masked in a
      // wave-uniform branch.
      if (tok0 + kTokens > seq_m) {
        const int tb = tok0 + 32 * w + 16 * (c >> 1) + 4 * (c & 1);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (tb + r >= seq_m) s0[r] = -INFINITY;
          if (tb + 8 + r >= seq_m) s1[r] = -INFINITY;
        }
      }
      float mloc = -INFINITY;
#pragma unroll
      for (int r = 0; r < 4; ++r) mloc = fmaxf(mloc, fmaxf(s0[r], s1[r]));
      mloc = xor32_max(xor16_max(mloc));
      if (lane < 8) sh.red[w][lane] = mloc;
      if (kHalves == 2 && w == 0 && lane < 8) sh.mrun[lane] = m_run;
      // Softmax against the running max m_run, speculatively: the page max is
      // known only after the barrier.  P = exp2((s - m_run) c) stays exact
      // while the page max exceeds m_run by at most kLazyMax / c (P <= 2^kLazyMax);
      // otherwise (and on the first page) P is recomputed below with a new
      // reference max, at the cost of one more barrier.
      float e0[4], e1[4], psum = 0.f;
      const bool spec = m_run != -INFINITY;  // the same in every wave
      auto softmax_tile = [&](float m_ref) {
        psum = 0.f;
        const float nm = -m_ref * p.scale_log2;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          e0[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[r], p.scale_log2, nm));
          e1[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[r], p.scale_log2, nm));
          psum += e0[r] + e1[r];
        }
        // P[n][token] -> tile[n][a = w][c' = 2 (c & 1) + r / 2][x = c >> 1]
        // at slot 4x + 2e + f (f = j, e = r & 1): the even-odd order coded
        // words decode in (a raw V record permutes the fragments)
        if (hh == 0) {
          uint8_t* c0 = sh.pt + tile_chunk(n, w, 2 * (c & 1)) + 8 * (c >> 1);
          uint8_t* c1 = sh.pt + tile_chunk(n, w, 2 * (c & 1) + 1) + 8 * (c >> 1);
          auto pk = pack_bf16x2;
          *reinterpret_cast<uint32_t*>(c0) = pk(e0[0], e1[0]);
          *reinterpret_cast<uint32_t*>(c0 + 4) = pk(e0[1], e1[1]);
          *reinterpret_cast<uint32_t*>(c1) = pk(e0[2], e1[2]);
          *reinterpret_cast<uint32_t*>(c1 + 4) = pk(e0[3], e1[3]);
        }
      };
      if (spec) softmax_tile(m_run);
      prefetch_dense(nkr, w, nt, fk, more);
      if (more) {
        expand_var(nkr, vk, w, lane, klut.s, sh.esc[par ^ 1][0], sh.hdr[par ^ 1][0]);
        expand_var(nvr, vv, w, lane, vlut.s, sh.esc[par ^ 1][1], sh.hdr[par ^ 1][1]);
      }
      __syncthreads();  // B2: page max per wave known; P tile written; next page's escapes expanded
      const float mpage = fmaxf(fmaxf(sh.red[0][n & 7], sh.red[1][n & 7]), fmaxf(sh.red[2][n & 7], sh.red[3][n & 7]));
      // the same decision in every wave: all read the same page maxima (and
      // in a two-half workgroup, each half also works out the other's, so
      // that both meet the extra barrier together)
      const bool renorm = !spec || __ballot(mpage > m_run + lazy) != 0;
      bool extra = renorm;
      if constexpr (kHalves == 2) {
        const AttnShared& ot = shs[half ^ 1];
        const float mp_o = fmaxf(fmaxf(ot.red[0][n & 7], ot.red[1][n & 7]), fmaxf(ot.red[2][n & 7], ot.red[3][n & 7]));
        const float mr_o = ot.mrun[n & 7];
        extra = extra || mr_o == -INFINITY || __ballot(mp_o > mr_o + lazy) != 0;
      }
      if (extra) {
        if (renorm) {
          const float m_new = fmaxf(m_run, mpage);
          const float m_use = m_new == -INFINITY ? 0.f : m_new;
          const float alpha = __builtin_amdgcn_exp2f((m_run - m_use) * p.scale_log2);
          m_run = m_new;
          l_run *= alpha;
          o0 *= alpha;
          o1 *= alpha;
          softmax_tile(m_use);
        }
        __syncthreads();  // rewritten P tile complete
      }
      l_run += psum;
      if (more) {
        patch_raw(nkr, vk, w, lane, sh.esc[par ^ 1][0], sh.hdr[par ^ 1][0]);
        patch_raw(nvr, vv, w, lane, sh.esc[par ^ 1][1], sh.hdr[par ^ 1][1]);
      }

      // ---- O^T += V^T P^T for dims 32w .. 32w + 31 ----
      if (act)
        decode_slab<true>(vr, fv, w, nt, np, vlut, sh.esc[par][1], sh.hdr[par][1], sh.pt, n, c,
                    [&](auto, const uint4& w0, const uint4& w1, const uint4& pa) {
                      o0 = mfma(a_frag(w0, w1, 0), pa, o0);
                      o1 = mfma(a_frag(w0, w1, 1), pa, o1);
                    });
      kr = nkr;
      vr = nvr;
      nkr = nnkr;
      nvr = nnvr;
      vk = vk2;
      vv = vv2;
    }

    // ---- this unit's result: O of the wave's 32 dims, m, and l summed over waves ----
    float l_tot = l_run;
    l_tot = xor32_sum(xor16_sum(l_tot));
    __syncthreads();  // everyone is past B2's reads of red
    if (lane < 8) sh.red[w][lane] = l_tot;
    __syncthreads();
    float l_all = sh.red[0][n & 7] + sh.red[1][n & 7] + sh.red[2][n & 7] + sh.red[3][n & 7];
    if (kInlinePlan && h == 0 && threadIdx.x == 0) {
      // this unit's plan entries for later calls (stored after the page loop:
      // the first waits for loads would otherwise also wait for these stores)
      int32_t* plan = p.plan;
      plan[2 + 2 * unit] = b;
      plan[3 + 2 * unit] = p0;
      int4* ud = reinterpret_cast<int4*>(plan + p.ud_off + 8 * unit);
      ud[0] = make_int4(b, p0, npages, seq);
      ud[1] = make_int4(first, chunks, blk0, blk1);
    }
    if constexpr (kHalves == 2) {
      // half 1 hands its (O, m, l) to half 0 through LDS (its escape area,
      // free now); half 0 merges them into its registers
      float* xo = reinterpret_cast<float*>(&shs[1].esc[0][0][0]);  // [head 8][dim 128], then m[8], l[8]
      const int d0 = 32 * w + 16 * (c >> 1) + 4 * (c & 1);
      if (half == 1 && hh == 0) {
        *reinterpret_cast<float4*>(xo + n * kDim + d0) = make_float4(o0[0], o0[1], o0[2], o0[3]);
        *reinterpret_cast<float4*>(xo + n * kDim + d0 + 8) = make_float4(o1[0], o1[1], o1[2], o1[3]);
        if (w == 0 && c == 0) {
          xo[8 * kDim + n] = m_run;
          xo[8 * kDim + 8 + n] = l_all;
        }
      }
      __syncthreads();
      if (half == 0) {
        const float m1 = xo[8 * kDim + (n & 7)], l1 = xo[8 * kDim + 8 + (n & 7)];
        const float m_new = fmaxf(m_run, m1);
        const float a0 = __builtin_amdgcn_exp2f((m_run - m_new) * p.scale_log2);
        const float a1 = __builtin_amdgcn_exp2f((m1 - m_new) * p.scale_log2);
        const float4 x0 = *reinterpret_cast<const float4*>(xo + (n & 7) * kDim + d0);
        const float4 x1 = *reinterpret_cast<const float4*>(xo + (n & 7) * kDim + d0 + 8);
        o0 = o0 * a0 + f32x4{x0.x, x0.y, x0.z, x0.w} * a1;
        o1 = o1 * a0 + f32x4{x1.x, x1.y, x1.z, x1.w} * a1;
        l_all = l_all * a0 + l1 * a1;
        m_run = m_new;
      }
    }
    if (chunks == 1) {
      // the whole sequence in one unit: normalise and write the output rows
      if (half == 0 && hh == 0 && n < p.group) {
        const float inv = l_all > 0.f ? 1.f / l_all : 0.f;
        auto pk = pack_bf16x2;
        uint16_t* orow = p.out + (int64_t)b * p.out_stride + (int64_t)(h * p.group + n) * kDim + 32 * w +
                         16 * (c >> 1) + 4 * (c & 1);
        *reinterpret_cast<uint2*>(orow) = make_uint2(pk(o0[0] * inv, o0[1] * inv), pk(o0[2] * inv, o0[3] * inv));
        *reinterpret_cast<uint2*>(orow + 8) = make_uint2(pk(o1[0] * inv, o1[1] * inv), pk(o1[2] * inv, o1[3] * inv));
      }
      continue;
    }
    const int64_t row = ((int64_t)h * p.units + unit) * 8 + n;
    if (half == 0 && hh == 0) {
      const rsrc_t ro = coh_rsrc(p.opart);
      const int64_t i0 = row * kDim + 32 * w + 16 * (c >> 1) + 4 * (c & 1);
      st_coh4(ro, i0, o0[0], o0[1], o0[2], o0[3]);
      st_coh4(ro, i0 + 8, o1[0], o1[1], o1[2], o1[3]);
      if (w == 0 && c == 0) st_coh2(coh_rsrc(p.ml), row * 2, m_run * p.scale_log2, l_all);
    }
    merge_chunks(p, shs[0], b, h, first, chunks);
  }
  // the plan words for later calls that reuse this plan (at the end, after
  // every load of the kernel)
  if (kInlinePlan && blockIdx.x == 0 && h == 0 && wave == 0) {
    int32_t* plan = p.plan;
    if (lane < p.batch) {
      plan[2 + 2 * p.units + 2 * lane] = ip.first;
      plan[3 + 2 * p.units + 2 * lane] = ip.cnt;
    }
    if (lane == 0) {
      plan[0] = ip.ppc;
      plan[1] = ip.used;
    }
  }
  if (kInlinePlan && h == 0) {
    // idle units of this workgroup's stride
    int32_t* plan = p.plan;
    for (int u = blockIdx.x + gridDim.x * (int)threadIdx.x; u < p.units; u += gridDim.x * 64 * kWaves * kHalves)
      if (u >= used) {
        plan[2 + 2 * u] = -1;
        plan[p.ud_off + 8 * u] = -1;
      }
  }
  // rows with no context produce zeros (workgroup 0 of each head)
  if (blockIdx.x == 0) {
    for (int b = wave; b < p.batch; b += kWaves * kHalves) {
      const int cnt = kInlinePlan ? wplan[1][b] : p.plan[3 + 2 * p.units + 2 * b];
      if (cnt != 0) continue;
      uint32_t* orow = reinterpret_cast<uint32_t*>(p.out + (int64_t)b * p.out_stride + (int64_t)h * p.group * kDim);
      for (int x = lane; x < p.group * kDim / 2; x += 64) orow[x] = 0u;
    }
  }
}

}  // namespace
}  // namespace fp

using namespace fp;


namespace fp {
namespace {
int decode_launch(AttnParams& p, const void* q, int64_t q_stride, int64_t batch, int64_t kv_heads, int64_t group,
                  const int64_t* rec_addr, const int32_t* rec_len, const uint32_t* plut, const uint8_t* slut,
                  const int32_t* block_table, int64_t bt_stride, const int32_t* seq_lens, float* opart,
                  int64_t opart_elems, float* ml, int64_t ml_elems, int32_t* plan, int64_t plan_elems, void* out,
                  int64_t out_stride, int64_t units, int replan, double scale, fp_stream_t stream) {
  FP_CHECK(batch >= 0 && kv_heads > 0, "decode needs batch >= 0 and kv_heads > 0");
  FP_CHECK(group == 1 || group == 2 || group == 4 || group == 8, "query heads need a group dividing 8");
  FP_CHECK(scale > 0, "softmax scale must be positive");
  if (batch == 0) return 0;
  FP_CHECK(units >= batch, "decode needs at least one unit per sequence");
  FP_CHECK(q_stride % 8 == 0 && q_stride >= kv_heads * group * kDim && reinterpret_cast<uintptr_t>(q) % 16 == 0,
           "q must be [B, H, 128] with contiguous heads, 16-byte aligned rows");
  FP_CHECK(out_stride % 2 == 0 && out_stride >= kv_heads * group * kDim && reinterpret_cast<uintptr_t>(out) % 4 == 0,
           "out must be [B, H, 128] with contiguous heads");
  FP_CHECK(opart_elems >= kv_heads * units * 8 * kDim && ml_elems >= kv_heads * units * 16,
           "decode workspace too small");
  FP_CHECK(units < (1 << 24) && batch < (1 << 24), "batch too large");
  // (page counts and their chunk arithmetic stay inside the planners' 2^22 range)
  FP_CHECK(bt_stride >= 0 && bt_stride < (1 << 21), "block table rows must hold fewer than 2^21 pages");
  FP_CHECK(kv_heads * units * 8 * kDim * 4 < (1LL << 31), "decode workspace must stay below 2 GiB");
  FP_CHECK(plan_elems >= ud_offset((int)units) + 8 * units + units * kv_heads,
           "decode plan workspace too small (see workspace_elems)");
  p.q = static_cast<const uint16_t*>(q);
  p.rec_addr = rec_addr;
  p.rec_len = rec_len;
  p.plut = plut;
  p.slut = slut;
  p.block_table = block_table;
  p.seq_lens = seq_lens;
  p.plan = plan;
  p.opart = opart;
  p.ml = ml;
  p.q_stride = q_stride;
  p.bt_stride = bt_stride;
  p.kvh = (int)kv_heads;
  p.group = (int)group;
  p.units = (int)units;
  p.batch = (int)batch;
  p.out = static_cast<uint16_t*>(out);
  p.out_stride = out_stride;
  p.ud_off = ud_offset((int)units);
  p.done = plan + plan_elems - units * kv_heads;
  p.scale_log2 = (float)(scale * 1.4426950408889634);
  p.lazy = kLazyMax / p.scale_log2;
  const int cus = device_cus();
  FP_CHECK(cus > 0, "cannot query the device's compute-unit count");
  // resident workgroups: kAttnPerCu 4-wave ones per CU, or one two-half
  // (8-wave) workgroup per CU for launches with few (sequence, head) pairs
  const int halves = batch * kv_heads <= kHalvesPairs ? 2 : 1;
  const int slots = halves == 2 ? cus : kAttnPerCu * cus;
  p.slots = slots;
  p.halves = halves;
  // replan 2 / 3: plan inside the attention kernel (batch <= 64; the merge
  // counters must be as a previous completed call left them, i.e. zero)
  FP_CHECK(replan >= 0 && replan <= 3, "replan must be 0, 1, 2 or 3");
  p.inline_plan = (replan == 2 || replan == 3) && batch <= 64 && units * kv_heads + slots < (1 << 22);
  p.bt_lds = replan == 3 && p.inline_plan && batch * bt_stride <= kBtLds;
  if (replan && !p.inline_plan) {
    hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, seq_lens, block_table, bt_stride, plan,
                       plan_elems, (int)batch, (int)units, (int)kv_heads, slots, halves);
    FP_LAUNCH_CHECK();
  }
  // persistent grid: one resident wave of workgroups (slots over all KV
  // heads) walks the units in use
  const int64_t per_head = std::min<int64_t>(units, (slots + kv_heads - 1) / kv_heads);
  const dim3 grid((unsigned)per_head, (unsigned)kv_heads), block(64 * kWaves * halves);
  if (halves == 2) {
    if (p.inline_plan)
      hipLaunchKernelGGL((attn_kernel<true, 2>), grid, block, 0, stream, p);
    else
      hipLaunchKernelGGL((attn_kernel<false, 2>), grid, block, 0, stream, p);
  } else if (p.inline_plan) {
    hipLaunchKernelGGL((attn_kernel<true, 1>), grid, block, 0, stream, p);
  } else {
    hipLaunchKernelGGL((attn_kernel<false, 1>), grid, block, 0, stream, p);
  }
  FP_LAUNCH_CHECK();
  return 0;
}
}  // namespace
}  // namespace fp

extern "C" int fp_fused_decode(const void* q, int64_t q_stride, int64_t batch, int64_t kv_heads, int64_t group,
                               const int64_t* rec_addr, const int32_t* rec_len, const uint32_t* plut,
                               const uint8_t* slut, const int32_t* block_table, int64_t bt_stride,
                               const int32_t* seq_lens, float* opart, int64_t opart_elems, float* ml,
                               int64_t ml_elems, int32_t* plan, int64_t plan_elems, void* out, int64_t out_stride,
                               int64_t units, int replan, double scale, fp_stream_t stream) {
  AttnParams p{};
  return decode_launch(p, q, q_stride, batch, kv_heads, group, rec_addr, rec_len, plut, slut, block_table, bt_stride,
                       seq_lens, opart, opart_elems, ml, ml_elems, plan, plan_elems, out, out_stride, units, replan,
                       scale, stream);
}

extern "C" int fp_fused_decode_append(const void* q, int64_t q_stride, int64_t batch, int64_t kv_heads,
                                      int64_t group, const int64_t* rec_addr, const int32_t* rec_len,
                                      const uint32_t* plut, const uint8_t* slut, const int32_t* block_table,
                                      int64_t bt_stride, const int32_t* seq_lens, float* opart, int64_t opart_elems,
                                      float* ml, int64_t ml_elems, int32_t* plan, int64_t plan_elems, void* out,
                                      int64_t out_stride, int64_t units, int replan, double scale,
                                      const void* new_k, int64_t nk_token_stride, int64_t nk_head_stride,
                                      const void* new_v, int64_t nv_token_stride, int64_t nv_head_stride,
                                      const int64_t* slot_mapping, const void* staging, int64_t staging_bytes,
                                      const void* scratch, int64_t scratch_bytes, fp_stream_t stream) {
  // Switched off: the first GPU run of its tests faulted the device and the
  // cause has not been shown; the device code is removed and the entry
  // stays declared so that callers fail loudly.
  (void)q, (void)q_stride, (void)batch, (void)kv_heads, (void)group, (void)rec_addr, (void)rec_len, (void)plut;
  (void)slut, (void)block_table, (void)bt_stride, (void)seq_lens, (void)opart, (void)opart_elems, (void)ml;
  (void)ml_elems, (void)plan, (void)plan_elems, (void)out, (void)out_stride, (void)units, (void)replan, (void)scale;
  (void)new_k, (void)nk_token_stride, (void)nk_head_stride, (void)new_v, (void)nv_token_stride, (void)nv_head_stride;
  (void)slot_mapping, (void)staging, (void)staging_bytes, (void)scratch, (void)scratch_bytes, (void)stream;
  fp::set_error("fp_fused_decode_append is disabled: its first GPU run faulted and the cause has not been shown");
  return -1;
}

// ---------------------------------------------------------------------------
// fp_fused_decode_noalloc: fp_fused_decode with its split-KV workspace (the
// partials, their (m, l) pairs and the plan with its merge counters) in a
// static device array instead of caller buffers, for callers that cannot
// allocate device memory.  Each device holds its own copy of ``scratch`` for
// the life of the process; its address is looked up once per device (with
// that device current) and kept.  Every call launches the planner, which
// rewrites the plan and zeroes the merge counters, so no state is carried
// between calls; calls that overlap on one device share the array and race.
constexpr int64_t kNoAllocBytes = 32LL << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];


namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
uint8_t* g_scratch_ptr[kMaxDevices] = {nullptr};

// The calling device's copy of ``scratch`` (nullptr with the error set).
uint8_t* device_scratch() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fp::set_error("fp_fused_decode_noalloc: no current HIP device");
    return nullptr;
  }
  std::lock_guard<std::mutex> guard(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (rc != hipSuccess || ptr == nullptr) {
      fp::set_error("fp_fused_decode_noalloc: hipGetSymbolAddress(scratch) failed");
      return nullptr;
    }
    g_scratch_ptr[dev] = static_cast<uint8_t*>(ptr);
  }
  return g_scratch_ptr[dev];
}

constexpr int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }
}  // namespace

extern "C" int64_t fp_fused_decode_noalloc_capacity(void) { return kNoAllocBytes; }

extern "C" int fp_fused_decode_noalloc(const void* q, int64_t q_stride, int64_t batch, int64_t kv_heads,
                                       int64_t group, const int64_t* rec_addr, const int32_t* rec_len,
                                       const uint32_t* plut, const uint8_t* slut, const int32_t* block_table,
                                       int64_t bt_stride, const int32_t* seq_lens, void* out, int64_t out_stride,
                                       int64_t units, double scale, fp_stream_t stream) {
  FP_CHECK(kv_heads > 0 && units > 0 && units < (1 << 24), "noalloc decode needs kv_heads > 0 and 0 < units < 2^24");
  const int64_t opart_elems = kv_heads * units * 8 * fp::kDim;
  const int64_t ml_elems = kv_heads * units * 16;
  const int64_t plan_elems = fp::ud_offset((int)units) + 8 * units + units * kv_heads;
  const int64_t ml_off = align256(opart_elems * 4), plan_off = ml_off + align256(ml_elems * 4);
  const int64_t need = plan_off + plan_elems * 4;
  if (need > kNoAllocBytes) {
    char msg[200];
    snprintf(msg, sizeof msg, "fp_fused_decode_noalloc: workspace of %lld bytes (kv_heads %lld x units %lld) exceeds the "
             "static scratch of %lld bytes", (long long)need, (long long)kv_heads, (long long)units,
             (long long)kNoAllocBytes);
    fp::set_error(msg);
    return -1;
  }
  uint8_t* base = device_scratch();
  if (base == nullptr) return -1;
  fp::AttnParams p{};
  return fp::decode_launch(p, q, q_stride, batch, kv_heads, group, rec_addr, rec_len, plut, slut, block_table,
                           bt_stride, seq_lens, reinterpret_cast<float*>(base), opart_elems,
                           reinterpret_cast<float*>(base + ml_off), ml_elems,
                           reinterpret_cast<int32_t*>(base + plan_off), plan_elems, out, out_stride, units,
                           /*replan=*/1, scale, stream);
}
