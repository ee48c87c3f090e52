// HBM-resident FragPack KV store on gfx950: per-step bookkeeping, the
// kernel-order staging writer, the record encoder, the decode-to-workspace
// gather, block-blob export/import and the batch record codec.
//
// Reference: fragpack/ops/hbm_kv.cu (prepare :110-219, write :221-255,
// encode :257-429, commit :431-448, gather :450-494, blobs :496-665) and the
// state machine in fragpack/ops/hbm_kv.py:1-47.  The bookkeeping kernels keep
// the reference's state layout and counter semantics, since the Python host
// side and the tests read them; the encoder produces the reference codec's
// exact bytes (fragpack/compression/attn_page.py:146-209).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <stdint.h>

#include "../../include/fragpack_hip.h"
#include "fp_capi_internal.hpp"
#include "fp_record.hpp"

namespace fp {
namespace {

// Counter slots (int32[16]), the reference's numbering (hbm_kv.cu:14-26).
enum : int {
  kFreeTop = 0,
  kTrans = 1,
  kClaims = 2,
  kCloses = 3,
  kErrStaging = 4,
  kErrOverflow = 5,
  kFallbacks = 6,
  kEncoded = 7,
  kSpills = 8,
  kHeirs = 9,
  kDonors = 10,
  // this build's: the claim-mode encode's dynamic tail (record cursor and
  // finished workgroups), both zero between launches
  kEncCursor = 11,
  kEncDone = 12,
};
// tags rows: [0] prepare's list of late closing claims (<= NB entries), [1..3] per-block step stamps
enum : int { kLateList = 0, kTagClose = 1, kTagClaim = 2, kTagCloseDedupe = 3 };

constexpr int kThreads = 256;
constexpr int kXcds = 8;    // XCDs of an MI355X (each with its own L2)
constexpr int kWriteSlabItems = 1 << 14;  // from this many (token, head) items a write takes the slab path
constexpr int kEncodeWgPerCu = 4;  // resident encode workgroups per CU (LDS: 32 KB stage + 6 KB each)

struct Store {
  int32_t* counters;
  int32_t* wslot;
  int32_t* tags;
  int32_t* free_stack;
  uint32_t* ovf_bits;
  int32_t* claim_list;
  int32_t* close_list;
  int64_t* rec_addr;
  int32_t* rec_len;
  uint8_t* staging;
  uint8_t* scratch;
  uint8_t* ovf_base;
  int32_t* fill;
  int64_t ovf_bytes;
  int L, H, NB, S_p, S_t, ovf_words, cap;
};

Store make_store(const fp_store_t* d) {
  Store s;
  s.counters = d->counters;
  s.wslot = d->wslot;
  s.tags = d->tags;
  s.free_stack = d->free_stack;
  s.ovf_bits = d->ovf_bits;
  s.claim_list = d->claim_list;
  s.close_list = d->close_list;
  s.rec_addr = d->rec_addr;
  s.rec_len = d->rec_len;
  s.staging = d->staging;
  s.scratch = d->scratch;
  s.ovf_base = d->overflow;
  s.fill = d->fill;
  s.ovf_bytes = d->overflow_records * (int64_t)kRawRecord;
  s.L = (int)d->num_layers;
  s.H = (int)d->kv_heads;
  s.NB = (int)d->num_blocks;
  s.S_p = (int)d->staging_slots;
  s.S_t = (int)d->scratch_slots;
  s.ovf_words = (int)d->ovf_words;
  s.cap = (int)d->list_cap;
  return s;
}

int check_store(const fp_store_t* d) {
  FP_CHECK(d != nullptr, "store descriptor is null");
  FP_CHECK(d->num_layers > 0 && d->num_blocks > 0 && d->kv_heads > 0, "store geometry must be positive");
  FP_CHECK(d->num_blocks < (1 << 30) && d->list_cap >= 0 && d->list_cap < (1 << 30), "store too large");
  return 0;
}

// Record (kv * H + h) of the block staged in slot ``w`` at ``layer``.
__device__ __forceinline__ uint8_t* staging_addr(const Store& s, int w, int layer, int kvh) {
  return w < s.S_p ? s.staging + (((int64_t)w * s.L + layer) * 2 * s.H + kvh) * kRawRecord
                   : s.scratch + ((int64_t)(w - s.S_p) * 2 * s.H + kvh) * kRawRecord;
}

// Overflow slot allocator over a bitmap (set = in use), safe against a
// concurrent allocator on another stream.  Returns -1 when full.  Called by
// one whole wavefront: 64 bitmap words are read per round (in scan order from
// the hint word, like the reference's serial probe, hbm_kv.cu:89-101) and the
// earliest word with a free bit is claimed by atomicOr, so a full pool costs
// ovf_words / 64 load rounds rather than ovf_words dependent loads.
__device__ int ovf_alloc_wave(const Store& s, uint32_t hint, int lane) {
  const uint32_t nw = (uint32_t)s.ovf_words;
  for (uint32_t base = 0; base < nw; base += 64) {
    const uint32_t i = base + (uint32_t)lane;
    int w = -1;
    uint32_t cur = 0xffffffffu;
    if (i < nw) {
      w = (int)((hint + i) % nw);
      cur = __hip_atomic_load(&s.ovf_bits[w], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    uint64_t avail = __ballot(cur != 0xffffffffu);
    while (avail) {
      const int src = __builtin_ctzll(avail);
      int got = -1;
      if (lane == src) {
        while (cur != 0xffffffffu) {
          const int bit = __builtin_ctz(~cur);
          const uint32_t prev = atomicOr(&s.ovf_bits[w], 1u << bit);
          if (!(prev & (1u << bit))) {
            got = 32 * w + bit;
            break;
          }
          cur = prev | (1u << bit);
        }
      }
      got = __shfl(got, src, 64);
      if (got >= 0) return got;
      avail &= avail - 1;
    }
  }
  return -1;
}

__device__ __forceinline__ void ovf_free(const Store& s, int64_t addr) {
  const int64_t off = addr - reinterpret_cast<int64_t>(s.ovf_base);
  if (off < 0 || off >= s.ovf_bytes) return;
  const int slot = (int)(off / kRawRecord);
  atomicAnd(&s.ovf_bits[slot >> 5], ~(1u << (slot & 31)));
}

// ---------------------------------------------------------------------------
// prepare / commit: a step's staging bookkeeping on one 1024-thread workgroup,
// with the semantics of the reference's prepare and commit
// (hbm_kv.cu:110-219, 431-448): GC of staging no live block holds, close
// marks (offset 127), claims (offset 0) served from transient scratch, the
// free stack or -- when it is empty -- transient scratch as an heir of a
// closing block, the close list with heirs paired to donors, and the claimed
// blocks' records pointed at their staging.
//
// Every list is built by workgroup stream compaction in input order: a
// thread takes kCompactPer consecutive items per round, its count is scanned
// across the wave with DPP and across the 16 waves through LDS, and each
// item lands at its rank.  All counters stay in registers / LDS until one
// store at the end -- no per-item global atomics -- and the outcome is a
// function of the state and the step: the same step on the same state gives
// the same slot assignment, list order and heir pairing.  Liveness is an LDS
// bitmap over persistent slots (a live block's slot bit), so GC needs no tag
// round trip.  The lists borrow the close list as scratch before the close
// phase writes it: deduplicated claims at close_list[0 ..), claims past the
// transient scratch at close_list[cap ..).
constexpr int kPrepThreads = 1024;
constexpr int kPrepWaves = kPrepThreads / 64;
constexpr int kCompactPer = 8;
constexpr int kScanPer = 8;   // slot-mapping entries per thread and round of prepare's first pass
constexpr int kLiveWords = 8192;  // persistent-slot liveness bitmap: up to 262144 slots

struct PrepShared {
  uint32_t live[kLiveWords];
  int wcnt[kPrepWaves];
};

// Stream compaction of items [0, n): ``load(i)`` fetches what item i's
// decision needs (a plain load, issued for all of a thread's items before
// any is decided, so they are in flight together), ``pick(i, v)`` returns a
// payload >= 0 to keep item i (or < 0), ``emit(i, rank, payload)`` receives
// each kept item's rank in input order.  Called by the whole workgroup;
// returns the count, with every emit's stores done before it returns.
template <typename Load, typename Pick, typename Emit>
__device__ int wg_compact(int n, PrepShared& sh, Load load, Pick pick, Emit emit) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  int total = 0;
  for (int r0 = 0; r0 < n; r0 += kCompactPer * kPrepThreads) {
    const int i0 = r0 + kCompactPer * tid;
    decltype(load(0)) v[kCompactPer];
#pragma unroll
    for (int k = 0; k < kCompactPer; ++k)
      if (i0 + k < n) v[k] = load(i0 + k);
    int pay[kCompactPer], cnt = 0;
#pragma unroll
    for (int k = 0; k < kCompactPer; ++k) {
      pay[k] = i0 + k < n ? pick(i0 + k, v[k]) : -1;
      cnt += pay[k] >= 0;
    }
    const int incl = wave_incl_scan(cnt);
    if (lane == 63) sh.wcnt[wave] = incl;
    __syncthreads();
    int before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kPrepWaves; ++w) {
      const int c = sh.wcnt[w];
      before += w < wave ? c : 0;
      all += c;
    }
    __syncthreads();  // wcnt is rewritten by the next round
    int rank = total + before + incl - cnt;
#pragma unroll
    for (int k = 0; k < kCompactPer; ++k)
      if (pay[k] >= 0) emit(i0 + k, rank++, pay[k]);
    total += all;
  }
  __syncthreads();  // every emit is visible to the workgroup's next phase
  return total;
}

__device__ __forceinline__ int slot_block(const Store& s, int64_t sl, int offset) {
  return sl >= 0 && (int)(sl & 127) == offset && (sl >> 7) < s.NB ? (int)(sl >> 7) : -1;
}

__global__ void __launch_bounds__(kPrepThreads) prepare_kernel(Store s, const int64_t* slots, int n_tok,
                                                               const int32_t* live, int n_live, int32_t step) {
  __shared__ PrepShared sh;
  const int tid = threadIdx.x;
  int32_t* close_tag = s.tags + kTagClose * s.NB;
  int32_t* claim_tag = s.tags + kTagClaim * s.NB;
  int32_t* dedupe_tag = s.tags + kTagCloseDedupe * s.NB;
  // Lists of this step, in space the state already has (every list holds at
  // most n_tok <= list_cap entries, or at most NB once deduplicated):
  int32_t* tmp = s.close_list;                // offset-0 blocks, then the deduplicated claims (until the closes)
  int32_t* ccand = s.close_list + s.cap;      // offset-127 blocks, compacted in place into the closes' heir column
  int32_t* late = s.tags + kLateList * s.NB;  // closing claims past the transient scratch
  int32_t* heirs = s.claim_list + s.cap;      // claims staged as heirs, in order
  const int top0 = s.counters[kFreeTop];

  // liveness of persistent slots (the round's loads in flight together)
  for (int i = tid; i < (s.S_p + 31) / 32; i += kPrepThreads) sh.live[i] = 0;
  __syncthreads();
  for (int r0 = 0; r0 < n_live; r0 += kCompactPer * kPrepThreads) {
    int bl[kCompactPer], w[kCompactPer];
#pragma unroll
    for (int k = 0; k < kCompactPer; ++k) {
      const int i = r0 + k * kPrepThreads + tid;
      bl[k] = i < n_live ? live[i] : -1;
    }
#pragma unroll
    for (int k = 0; k < kCompactPer; ++k) w[k] = bl[k] >= 0 && bl[k] < s.NB ? s.wslot[bl[k]] : -1;
#pragma unroll
    for (int k = 0; k < kCompactPer; ++k)
      if (w[k] >= 0 && w[k] < s.S_p) atomicOr(&sh.live[w[k] >> 5], 1u << (w[k] & 31));
  }

  // One pass over the slot mapping, no atomics: close marks (offset 127),
  // and two lists compacted together in input order -- the block of every
  // offset-0 token into tmp, of every offset-127 token into ccand.  Counts
  // are packed in one scan (each below 2^16: kScanPer * kPrepThreads
  // items per round); the next round's slots load while a round is scanned
  // (the round's barriers wait for LDS only).
  int n_raw0 = 0, n_raw1 = 0;
  {
    const int wave = tid >> 6, lane = tid & 63;
    int64_t nv[kScanPer];
#pragma unroll
    for (int k = 0; k < kScanPer; ++k) nv[k] = kScanPer * tid + k < n_tok ? slots[kScanPer * tid + k] : -1;
    for (int r0 = 0; r0 < n_tok; r0 += kScanPer * kPrepThreads) {
      int b0[kScanPer], b1[kScanPer], c = 0;
#pragma unroll
      for (int k = 0; k < kScanPer; ++k) {
        b0[k] = slot_block(s, nv[k], 0);
        b1[k] = slot_block(s, nv[k], 127);
        c += (b0[k] >= 0) + ((b1[k] >= 0) << 16);
      }
      const int i1 = r0 + kScanPer * (kPrepThreads + tid);
#pragma unroll
      for (int k = 0; k < kScanPer; ++k) nv[k] = i1 + k < n_tok ? slots[i1 + k] : -1;
      const int incl = wave_incl_scan(c);
      if (lane == 63) sh.wcnt[wave] = incl;
      lds_barrier();
      int before = 0, all = 0;
#pragma unroll
      for (int q = 0; q < kPrepWaves; ++q) {
        const int x = sh.wcnt[q];
        before += q < wave ? x : 0;
        all += x;
      }
      lds_barrier();  // wcnt is rewritten by the next round
      const int ex = before + incl - c;
      int r0c = n_raw0 + (ex & 0xFFFF), r1c = n_raw1 + (ex >> 16);
#pragma unroll
      for (int k = 0; k < kScanPer; ++k) {
        if (b0[k] >= 0) tmp[r0c++] = b0[k];
        if (b1[k] >= 0) {
          ccand[r1c++] = b1[k];
          close_tag[b1[k]] = step;
        }
      }
      n_raw0 += all & 0xFFFF;
      n_raw1 += all >> 16;
    }
  }
  __syncthreads();  // the lists and close marks are visible to the next phases

  // claims: one per block, the first offset-0 token to stamp claim_tag
  // (compacted in place: a round's items are loaded before any is written)
  const int n_cand = wg_compact(
      n_raw0, sh, [&](int i) { return tmp[i]; },
      [&](int, int b) { return atomicExch(&claim_tag[b], step) != step ? b : -1; },
      [&](int, int r, int b) { tmp[r] = b; });

  // GC: transient slots end with their step; persistent slots of blocks not
  // live go back on the free stack (pushed in block order)
  const int freed = wg_compact(
      s.NB, sh, [&](int b) { return s.wslot[b]; },
      [&](int b, int w) {
        if (w >= s.S_p) s.wslot[b] = -1;
        if (w < 0 || w >= s.S_p || ((sh.live[w >> 5] >> (w & 31)) & 1u)) return -1;
        s.wslot[b] = -1;
        return w;
      },
      [&](int, int r, int w) { s.free_stack[top0 + r] = w; });
  const int top = top0 + freed;

  // blocks that open and close within the step: transient scratch in order
  const int n_close_claims = wg_compact(
      n_cand, sh, [&](int i) { return tmp[i]; },
      [&](int, int b) {
        return s.wslot[b] < 0 && close_tag[b] == step ? b : -1;
      },
      [&](int, int r, int b) {
        if (r < s.S_t)
          s.wslot[b] = s.S_p + r;
        else
          late[r - s.S_t] = b;
      });
  const int trans0 = min(n_close_claims, s.S_t);
  // blocks that stay open: the free stack from its top, then heirs in scratch
  int errors = 0;
  const int n_open_claims = wg_compact(
      n_cand, sh, [&](int i) { return tmp[i]; },
      [&](int, int b) {
        return s.wslot[b] < 0 && close_tag[b] != step ? b : -1;
      },
      [&](int, int r, int b) {
        if (r < top) {
          s.wslot[b] = s.free_stack[top - 1 - r];
        } else if (trans0 + r - top < s.S_t) {
          s.wslot[b] = s.S_p + trans0 + r - top;
          heirs[r - top] = b;
        }
      });
  const int n_heirs = min(max(n_open_claims - top, 0), s.S_t - trans0);
  errors += max(n_open_claims - top, 0) - n_heirs;
  // closing blocks the scratch could not hold take what the stack has left
  const int n_late = n_close_claims - trans0;
  for (int q = tid; q < n_late; q += kPrepThreads) {
    const int d = n_open_claims + q;
    if (d < top) s.wslot[late[q]] = s.free_stack[top - 1 - d];
  }
  errors += max(n_late - max(top - n_open_claims, 0), 0);
  __syncthreads();

  const int n_claims = wg_compact(
      n_cand, sh, [&](int i) { return tmp[i]; }, [&](int, int b) { return s.wslot[b] >= 0 ? b : -1; },
      [&](int, int r, int b) { s.claim_list[r] = b; });

  // closes (offset 127), one per block holding staging (the first token to
  // stamp dedupe_tag); persistent donors hand their slot to the heirs in
  // order.  The candidates lie in the heirs half of the close list and are
  // compacted in place (rank <= index, a round's items loaded first).
  const int n_closes = wg_compact(
      n_raw1, sh, [&](int c) { return ccand[c]; },
      [&](int, int b) { return atomicExch(&dedupe_tag[b], step) != step && s.wslot[b] >= 0 ? b : -1; },
      [&](int, int r, int b) {
        s.close_list[r] = b;
        s.close_list[s.cap + r] = -1;
      });
  const int n_donors = wg_compact(
      n_closes, sh, [&](int c) { return s.close_list[c]; }, [&](int c, int b) { return s.wslot[b] < s.S_p ? c : -1; },
      [&](int, int d, int c) {
        if (d < n_heirs) s.close_list[s.cap + c] = heirs[d];
      });
  errors += max(n_heirs - n_donors, 0);

  // claimed blocks' records -> their staging, raw; freed overflow slots; page fill reset
  const int per = s.L * 2 * s.H;
  const int64_t n_ent = (int64_t)n_claims * per;
  for (int64_t x0 = 0; x0 < n_ent; x0 += kCompactPer * kPrepThreads) {
    // each level's loads for the round's entries in flight together
    int b[kCompactPer], w[kCompactPer];
    int64_t old[kCompactPer];
#pragma unroll
    for (int k = 0; k < kCompactPer; ++k) {
      const int64_t x = x0 + k * kPrepThreads + tid;
      b[k] = x < n_ent ? s.claim_list[x / per] : -1;
    }
#pragma unroll
    for (int k = 0; k < kCompactPer; ++k) {
      const int64_t x = x0 + k * kPrepThreads + tid;
      const int r = (int)(x % per), layer = r / (2 * s.H), kvh = r % (2 * s.H);
      w[k] = b[k] >= 0 ? s.wslot[b[k]] : -1;
      old[k] = b[k] >= 0 ? s.rec_addr[((int64_t)layer * s.NB + b[k]) * 2 * s.H + kvh] : 0;
    }
#pragma unroll
    for (int k = 0; k < kCompactPer; ++k) {
      if (b[k] < 0) continue;
      const int64_t x = x0 + k * kPrepThreads + tid;
      const int r = (int)(x % per), layer = r / (2 * s.H), kvh = r % (2 * s.H);
      const int64_t idx = ((int64_t)layer * s.NB + b[k]) * 2 * s.H + kvh;
      ovf_free(s, old[k]);
      s.rec_addr[idx] = reinterpret_cast<int64_t>(staging_addr(s, w[k], layer, kvh));
      s.rec_len[idx] = kRawVarLen;
      if (kvh == 0) s.fill[(int64_t)layer * s.NB + b[k]] = 0;
    }
  }
  if (tid == 0) {
    const int popped = min(top, n_open_claims + n_late);
    s.counters[kFreeTop] = top - popped;
    s.counters[kTrans] = trans0 + n_heirs;
    s.counters[kClaims] = n_claims;
    s.counters[kCloses] = n_closes;
    s.counters[kHeirs] = n_heirs;
    s.counters[kDonors] = n_donors;
    if (errors) s.counters[kErrStaging] += errors;
  }
}

// ---------------------------------------------------------------------------
// write: one wavefront per (token, head).  Lane p (0..63) moves the dim pair
// (2p, 2p+1) of K (one u32: both scalars are in the same kernel-order word)
// and of V (two u16: a V pair belongs to two threads) into the raw
// kernel-order staging record.
__device__ __forceinline__ void store_k_pair(uint8_t* rec, uint32_t val, int off, int p) {
  // K: token off = 16 tw + 8 j + g, dim 2p = 16 st + 8 f + 2 c
  const int st = p >> 3, f = (p >> 2) & 1, c = p & 3;
  const int tw = off >> 4, j = (off >> 3) & 1, g = off & 7;
  const int t = 32 * tw + 4 * g + c;
  *reinterpret_cast<uint32_t*>(rec + 16 * (256 * st + t) + 2 * (4 * j + 2 * f)) = val;
}

__device__ __forceinline__ void store_v_pair(uint8_t* rec, uint32_t val, int off, int p) {
  // V: token off = 16 st + 8 f + 2 c + e, dim d = 16 tw + 8 j + g
  const int st = off >> 4, f = (off >> 3) & 1, c = (off >> 1) & 3, e = off & 1;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int d = 2 * p + q;
    const int tw = d >> 4, j = (d >> 3) & 1, g = d & 7;
    const int t = 32 * tw + 4 * g + c;
    *reinterpret_cast<uint16_t*>(rec + 16 * (256 * st + t) + 2 * (4 * j + 2 * f + e)) = (uint16_t)(val >> (16 * q));
  }
}

__device__ __forceinline__ void put_k_row(uint8_t* rec, const uint16_t* krow, int off, int p) {
  store_k_pair(rec, *reinterpret_cast<const uint32_t*>(krow + 2 * p), off, p);
}

__device__ __forceinline__ void put_v_row(uint8_t* rec, const uint16_t* vrow, int off, int p) {
  store_v_pair(rec, *reinterpret_cast<const uint32_t*>(vrow + 2 * p), off, p);
}

// The step's new tokens as the write hands them over (element strides).
struct StepTokens {
  const uint16_t* k;
  const uint16_t* v;
  int64_t ks0, ks1, vs0, vs1;
  const int64_t* slots;
  int n;
  int enc_grid;  // write + encode in one launch: workgroups [0, enc_grid) encode, the rest write
};

// (token, head) item ``item`` of the write: K and V rows of token item / H,
// head item % H, into the staging of the token's block.  With
// ``skip_closing``, tokens of blocks on the close list are left to the
// encoders of those blocks (the fused write + encode).
__device__ __forceinline__ void write_item(const Store& s, const StepTokens& tk, int layer, int item,
                                           bool skip_closing) {
  if (item >= tk.n * s.H) return;
  const int tok = item / s.H, h = item % s.H;
  const int64_t sl = tk.slots[tok];
  if (sl < 0) return;
  const int b = (int)(sl >> 7), off = (int)(sl & 127);
  if (b >= s.NB) return;
  const int w = s.wslot[b];
  if (w < 0) return;
  const int p = threadIdx.x & 63;
  if (skip_closing) {
    const int n_closes = s.counters[kCloses];
    for (int c0 = 0; c0 < n_closes; c0 += 64) {
      const int c = c0 + p;
      if (__ballot(c < n_closes && s.close_list[c] == b) != 0) return;
    }
  }
  put_k_row(staging_addr(s, w, layer, h), tk.k + tok * tk.ks0 + h * tk.ks1, off, p);
  put_v_row(staging_addr(s, w, layer, s.H + h), tk.v + tok * tk.vs0 + h * tk.vs1, off, p);
}

// Workgroups are dealt to the 8 XCDs round-robin; the grid is a multiple of
// 8 and XCD x takes the x-th contiguous eighth of the grid.
__device__ __forceinline__ int xcd_contiguous_wg() {
  const int per = (int)gridDim.x / kXcds;
  return ((int)blockIdx.x % kXcds) * per + (int)blockIdx.x / kXcds;
}

// One wave per (token, head) item: steps of few tokens.
__global__ void __launch_bounds__(kThreads) write_kernel(Store s, StepTokens tk, int layer) {
  write_item(s, tk, layer, xcd_contiguous_wg() * (kThreads / 64) + (threadIdx.x >> 6), false);
}

// Large steps.  A 16-byte chunk of a kernel-order record holds two K tokens
// x 4 dims or four V tokens x 2 dims, all of one 16-token slab (token
// offsets 16 st .. 16 st + 15), so per-token stores are 2- and 4-byte
// pieces scattered over 8 (K) or 32 (V) lines.  Here each wave owns 16
// consecutive tokens of the step.  A token whose whole slab the step writes
// (16 tokens with consecutive slots from an offset that is a multiple of 16)
// is written by the wave owning the slab's first token: per record, the 16
// rows are loaded coalesced into LDS and leave as whole 16-byte chunks, 4 KB
// contiguous (V) or 8 runs of 512 B (K).  Other tokens go through the
// per-(token, head) path.  Each wave handles one record (kv, head) of its
// 16 tokens: the 2H waves of a window are neighbours, on one XCD.  The
// step's K and V rows must be 16-byte aligned.
constexpr int kSlab = 16;
constexpr int kSlabRow = 2 * kDim + 16;  // bytes per staged row (padded: 68 dwords)

__device__ __forceinline__ void wave_lds_sync() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done
  asm volatile("" ::: "memory");
}

__global__ void __launch_bounds__(kThreads) write_slab_kernel(Store s, StepTokens tk, int layer) {
  __shared__ __align__(16) uint8_t stage[kThreads / 64][kSlab * kSlabRow];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int job = xcd_contiguous_wg() * (kThreads / 64) + wave;
  const int rec = job % (2 * s.H);
  const int t0 = job / (2 * s.H) * kSlab;
  if (t0 >= tk.n) return;
  const bool is_v = rec >= s.H;
  const int h = is_v ? rec - s.H : rec;
  // slots of tokens t0 - 16 .. t0 + 31 (lanes 0..47); -1 past either end
  const int ti = t0 - kSlab + lane;
  const int64_t sl = lane < 3 * kSlab && ti >= 0 && ti < tk.n ? tk.slots[ti] : -1;
  const int64_t nxt = __shfl_down(sl, 1, 64);
  const uint64_t run = __ballot(lane < 3 * kSlab - 1 && sl >= 0 && nxt == sl + 1);  // bit i: i -> i+1 consecutive
  // a token is covered when its slab's first token s0 and the 15 steps after it are consecutive
  const int r = (int)(sl & (kSlab - 1));
  const int s0 = lane - r;
  const bool covered = sl >= 0 && s0 >= 0 && ((run >> s0) & 0x7fffull) == 0x7fffull;
  const bool mine = lane >= kSlab && lane < 2 * kSlab && ti < tk.n;
  uint64_t loose = __ballot(mine && sl >= 0 && !covered);
  const uint64_t start = __ballot(mine && covered && r == 0);
  uint8_t* lds = stage[wave];
  const int p = lane;
  // per-(token, head) path for tokens of partly written slabs
  while (loose) {
    const int bit = __builtin_ctzll(loose);
    loose &= loose - 1;
    const int64_t tsl = __shfl(sl, bit, 64);
    const int b = (int)(tsl >> 7), off = (int)(tsl & 127);
    if (b >= s.NB) continue;
    const int w = s.wslot[b];
    if (w < 0) continue;
    const int tok = t0 - kSlab + bit;
    if (is_v)
      put_v_row(staging_addr(s, w, layer, rec), tk.v + tok * tk.vs0 + h * tk.vs1, off, p);
    else
      put_k_row(staging_addr(s, w, layer, rec), tk.k + tok * tk.ks0 + h * tk.ks1, off, p);
  }
  if (!start) return;
  const int bit = __builtin_ctzll(start);  // at most one slab starts among 16 tokens
  const int64_t ssl = __shfl(sl, bit, 64);
  const int b = (int)(ssl >> 7), st = (int)((ssl & 127) >> 4);
  if (b >= s.NB) return;
  const int w = s.wslot[b];
  if (w < 0) return;
  const int tok0 = t0 - kSlab + bit;
  const int lrow = lane >> 4, lcol = (lane & 15) * 16;  // load: 16 lanes per 256-byte row
  // chunk ci = lane + 64 m of the slab's 256: k = ci & 31 and half = ci >> 5
  const int k = lane & 31, g = k >> 2, c = k & 3;
  const uint16_t* src = is_v ? tk.v + tok0 * tk.vs0 + h * tk.vs1 : tk.k + tok0 * tk.ks0 + h * tk.ks1;
  const int64_t rs = is_v ? tk.vs0 : tk.ks0;
  uint4 row[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    row[i] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(src + (lrow + 4 * i) * rs) + lcol);
#pragma unroll
  for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(lds + (lrow + 4 * i) * kSlabRow + lcol) = row[i];
  wave_lds_sync();
  uint8_t* dst = staging_addr(s, w, layer, rec);
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int half = (lane >> 5) + 2 * m;  // K: dim slab st'; V: dim group tw
    uint32_t q[4];
    if (!is_v) {
      // K chunk (st', t = 32 st + 4 g + c): u32 (2 j + f) = token 8 j + g, dims 16 st' + 8 f + 2 c, +1
#pragma unroll
      for (int jf = 0; jf < 4; ++jf)
        q[jf] = *reinterpret_cast<const uint32_t*>(lds + (8 * (jf >> 1) + g) * kSlabRow +
                                                   2 * (16 * half + 8 * (jf & 1) + 2 * c));
      *reinterpret_cast<uint4*>(dst + 16 * (256 * half + 32 * st + k)) = make_uint4(q[0], q[1], q[2], q[3]);
    } else {
      // V chunk (st, t = 32 tw + 4 g + c): u16 (4 j + 2 f + e) = token 8 f + 2 c + e, dim 16 tw + 8 j + g
#pragma unroll
      for (int jf = 0; jf < 4; ++jf) {
        const int j = jf >> 1, f = jf & 1, d = 16 * half + 8 * j + g;
        const uint32_t lo = *reinterpret_cast<const uint16_t*>(lds + (8 * f + 2 * c) * kSlabRow + 2 * d);
        const uint32_t hi = *reinterpret_cast<const uint16_t*>(lds + (8 * f + 2 * c + 1) * kSlabRow + 2 * d);
        q[jf] = lo | (hi << 16);
      }
      *reinterpret_cast<uint4*>(dst + 16 * (256 * st + 32 * half + k)) = make_uint4(q[0], q[1], q[2], q[3]);
    }
  }
}

// The fused write + encode's encoder side: before a workgroup reads record
// ``kvh`` of closing block ``b``, it writes that record's rows of every
// token of this step in block ``b`` -- and in the block's heir, whose
// staging the encoder copies -- itself, so no write of another workgroup
// has to land first.  The write workgroups skip closing blocks; a heir's
// rows may be written by both sides, with the same bytes.  Whole workgroup;
// the rows are stored and visible to the workgroup's later loads on return.
__device__ void write_own_rows(const Store& s, const StepTokens& tk, int layer, int b, int heir, int kvh) {
  const int tid = threadIdx.x, p = tid & 63, wave = tid >> 6;
  const bool is_k = kvh < s.H;
  const int h = is_k ? kvh : kvh - s.H;
  for (int i0 = 0; i0 < tk.n; i0 += kThreads) {
    const int i = i0 + tid;
    const int64_t sl = i < tk.n ? tk.slots[i] : -1;
    const int blk = sl >= 0 ? (int)(sl >> 7) : -1;
    uint64_t m = __ballot(blk >= 0 && (blk == b || blk == heir));
    while (m != 0) {
      const int bit = __builtin_ctzll(m);
      m &= m - 1;
      const int tok = i0 + 64 * wave + bit;
      const int tb = __shfl(blk, bit, 64), off = (int)(__shfl((int)(sl & 127), bit, 64));
      const int w = s.wslot[tb];
      if (w < 0) continue;
      uint8_t* rec = staging_addr(s, w, layer, kvh);
      if (is_k)
        put_k_row(rec, tk.k + tok * tk.ks0 + h * tk.ks1, off, p);
      else
        put_v_row(rec, tk.v + tok * tk.vs0 + h * tk.vs1, off, p);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // the rows are stored
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Record encoder core: one 256-thread workgroup, thread t holding the 8
// kernel-order words of thread t.  Computes codes, counts, the variable
// region (in LDS) and whether the record codes.
//
// The per-(kv, head) lookup table in LDS maps a high byte to
// code | nib << 4: code = min(rank, 7) (7 = escape), nib = the escape nibble
// (extended-table index rank - 7, or 15 for a raw scalar; 0 for a primary).
// A word's eight table bytes are read two per VGPR (16-bit halves) and
// rearranged with two v_perm into code and nibble words whose nibble j
// belongs to scalar j, so the rest of the analysis runs 8 scalars per op.

struct EncShared {
  uint8_t tb[256];                 // high byte -> code | nib << 4
  uint8_t esc[kMaxEscapes + 16];   // escape nibbles as bytes, by ordinal
  uint32_t var32[kVarCap / 4];
  int wsum[2][8];  // per 32-thread slab: escapes, raws
  int s_off, s_ovf;
  int dyn_start;  // claim-mode tail: the start of the batch thread 0 grabbed last
};

// LDS table entry of rank r (the store's rank_of byte: 0..21, 255 absent).
__device__ __forceinline__ uint8_t table_byte(uint32_t r) {
  return r < (uint32_t)kPrimaryDirect ? (uint8_t)r
                                      : (uint8_t)(kPrimaryDirect | (min(r - kPrimaryDirect, (uint32_t)kRawNibble) << 4));
}

struct EncResult {
  bool codes;
  int var_len;
  int raw_offset;
  int etot, rtot;
};

typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));

// Code and escape-nibble words of word ``st`` (nibble j = scalar j).
__device__ __forceinline__ void enc_word(const uint4& w, const uint8_t* tb, uint32_t& code, uint32_t& nib) {
  // scalar e is the half e & 1 of dword e >> 1; high byte = bits 8..15 / 24..31
  u16x2_t x0, x1, x2, x3;  // [t0, t2], [t4, t6], [t1, t3], [t5, t7]
  x0.x = tb[(w.x >> 8) & 0xFF];
  x0.y = tb[(w.y >> 8) & 0xFF];
  x1.x = tb[(w.z >> 8) & 0xFF];
  x1.y = tb[(w.w >> 8) & 0xFF];
  x2.x = tb[w.x >> 24];
  x2.y = tb[w.y >> 24];
  x3.x = tb[w.z >> 24];
  x3.y = tb[w.w >> 24];
  const uint32_t g = perm(__builtin_bit_cast(uint32_t, x1), __builtin_bit_cast(uint32_t, x0), 0x06040200u);
  const uint32_t h = perm(__builtin_bit_cast(uint32_t, x3), __builtin_bit_cast(uint32_t, x2), 0x06040200u);
  // g = [t0, t2, t4, t6], h = [t1, t3, t5, t7]
  code = (g & 0x0F0F0F0Fu) | ((h << 4) & 0xF0F0F0F0u);
  nib = ((g >> 4) & 0x0F0F0F0Fu) | (h & 0xF0F0F0F0u);
}

// Escape bits (bit 4j set iff scalar j escapes) of a code word.
__device__ __forceinline__ uint32_t esc_nibbles(uint32_t code) { return ((code + 0x11111111u) >> 3) & 0x11111111u; }
// Raw bits (bit 4j set iff scalar j's escape nibble is 15) of a nibble word.
__device__ __forceinline__ uint32_t raw_nibbles(uint32_t nib) {
  const uint32_t t = nib & (nib >> 2);
  return t & (t >> 1) & 0x11111111u;
}

// Per-thread code / nibble words and symbol words; totals across the
// workgroup.  Leaves the escape / raw exclusive prefixes of this thread in
// eo / ro.
__device__ __forceinline__ EncResult enc_analyse(const uint4 (&wd)[8], EncShared& sh, uint32_t (&sym)[6],
                                                 uint32_t (&code)[8], uint32_t (&nib)[8], int& eo, int& ro) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int ne = 0, nr = 0;
#pragma unroll
  for (int st = 0; st < 8; ++st) {
    enc_word(wd[st], sh.tb, code[st], nib[st]);
    ne += __builtin_popcount(esc_nibbles(code[st]));
    nr += __builtin_popcount(raw_nibbles(nib[st]));
  }
  // symbol words of group gi: words 4 gi + k (k < 3), bit 3 of nibble j =
  // bit k of the code of scalar 24 + j (word 4 gi + 3)
#pragma unroll
  for (int gi = 0; gi < 2; ++gi)
#pragma unroll
    for (int k = 0; k < 3; ++k) sym[3 * gi + k] = code[4 * gi + k] | ((code[4 * gi + 3] << (3 - k)) & 0x88888888u);
  const int ei = wave_incl_scan(ne), ri = wave_incl_scan(nr);
  // per 32-thread slab totals (two per wavefront)
  const int e31 = __shfl(ei, 31, 64), e63 = __shfl(ei, 63, 64);
  const int r31 = __shfl(ri, 31, 64), r63 = __shfl(ri, 63, 64);
  if (lane == 0) {
    sh.wsum[0][2 * wave] = e31;
    sh.wsum[0][2 * wave + 1] = e63 - e31;
    sh.wsum[1][2 * wave] = r31;
    sh.wsum[1][2 * wave + 1] = r63 - r31;
  }
  lds_barrier();
  int ebase = 0, rbase = 0, etot = 0, rtot = 0, rmax = 0;
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    if (w < 2 * wave) {
      ebase += sh.wsum[0][w];
      rbase += sh.wsum[1][w];
    }
    etot += sh.wsum[0][w];
    rtot += sh.wsum[1][w];
    rmax = max(rmax, sh.wsum[1][w]);
  }
  eo = ebase + ei - ne;
  ro = rbase + ri - nr;
  EncResult res;
  res.etot = etot;
  res.rtot = rtot;
  res.raw_offset = (kHeaderBytes + ((etot + 1) >> 1) + 3) & ~3;
  res.var_len = (res.raw_offset + 4 * rtot + 15) & ~15;
  res.codes = res.var_len <= kVarCap && rmax <= kMaxWarpRaw;
  return res;
}

// Builds the variable region in sh.var32 (coded records only).  Caller
// zeroed sh.var32 before enc_analyse's barrier.  Each thread writes its
// escape nibbles as bytes at their ordinals (sh.esc) and its raw-list
// entries; after a barrier the byte stream is packed two nibbles per byte
// into the region.  Ends with the region complete (barrier).
__device__ __forceinline__ void enc_var(const uint4 (&wd)[8], const uint32_t (&code)[8], const uint32_t (&nib)[8],
                                        EncShared& sh, const EncResult& res, int eo, int ro) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int st = 0; st < 8; ++st) {
    uint32_t m = esc_nibbles(code[st]);
    const uint32_t nw = nib[st];
    while (m) {
      const int j4 = __builtin_ctz(m);  // 4 j
      m &= m - 1;
      const uint32_t nv = (nw >> j4) & 0xFu;
      sh.esc[eo] = (uint8_t)nv;
      if (nv == (uint32_t)kRawNibble) {
        // high byte of scalar j: byte 2 (j & 1) + 1 of dword j >> 1
        const int j = j4 >> 2;
        const uint32_t d = u4(wd[st], j >> 1);
        const uint32_t hb = (d >> (8 + 16 * (j & 1))) & 0xFFu;
        sh.var32[(res.raw_offset >> 2) + ro++] = (uint32_t)eo | (hb << 16);
      }
      ++eo;
    }
  }
  if (threadIdx.x == 0) {
    sh.var32[0] = res.etot;
    sh.var32[1] = res.rtot;
    sh.var32[2] = res.raw_offset;
    sh.var32[3] = 0;
    int ep = 0, rp = 0;
    for (int w = 0; w < 8; ++w) {
      const int e16 = ep & 0xFFFF, r16 = rp & 0xFFFF;
      // u16 esc_prefix[8] at byte 16, raw_prefix[8] at byte 32
      if (w & 1) {
        sh.var32[4 + (w >> 1)] |= (uint32_t)e16 << 16;
        sh.var32[8 + (w >> 1)] |= (uint32_t)r16 << 16;
      } else {
        sh.var32[4 + (w >> 1)] = (uint32_t)e16;
        sh.var32[8 + (w >> 1)] = (uint32_t)r16;
      }
      ep += sh.wsum[0][w];
      rp += sh.wsum[1][w];
    }
  }
  lds_barrier();
  // pack: region dword 12 + k holds escape ordinals 8k .. 8k + 7 (nibble 2i
  // low, 2i + 1 high in byte i); ordinals past etot are zero
  for (int k = tid; 8 * k < res.etot; k += kThreads) {
    const uint2 b = *reinterpret_cast<const uint2*>(sh.esc + 8 * k);
    const int left = res.etot - 8 * k;  // > 0
    const uint32_t keep_lo = left >= 4 ? 0xFFFFFFFFu : (1u << (8 * left)) - 1u;
    const uint32_t keep_hi = left >= 8 ? 0xFFFFFFFFu : left <= 4 ? 0u : (1u << (8 * (left - 4))) - 1u;
    const uint32_t lo = b.x & keep_lo, hi = b.y & keep_hi;
    const uint32_t ev = perm(hi, lo, 0x06040200u), od = perm(hi, lo, 0x07050301u);
    sh.var32[(kHeaderBytes >> 2) + k] = ev | (od << 4);
  }
  lds_barrier();
}

// Streaming stores (the non-temporal policy: a record is written once and
// read by a later launch).
// (through the global address space: a generic pointer would make flat
// stores, which every later LDS wait would also wait for)
__device__ __forceinline__ void st16_nt(uint8_t* p, uint4 v) {
  const u32x4_t x = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(x, reinterpret_cast<FP_GLOBAL u32x4_t*>(reinterpret_cast<uintptr_t>(p)));
}
__device__ __forceinline__ void st8_nt(uint8_t* p, uint32_t a, uint32_t b) {
  __builtin_nontemporal_store(u32x2_t{a, b}, reinterpret_cast<FP_GLOBAL u32x2_t*>(reinterpret_cast<uintptr_t>(p)));
}

// Writes a coded record (dense part from registers, variable part from LDS)
// at ``dst`` (16-byte aligned).
__device__ __forceinline__ void enc_store(uint8_t* dst, const uint4 (&wd)[8], const uint32_t (&sym)[6],
                                          const EncShared& sh, int var_len) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint4 a = wd[2 * j], c = wd[2 * j + 1];
    // low bytes of the 16 scalars of chunk j
    st16_nt(dst + 16 * (256 * j + tid), make_uint4(perm(a.y, a.x, 0x06040200u), perm(a.w, a.z, 0x06040200u),
                                                   perm(c.y, c.x, 0x06040200u), perm(c.w, c.z, 0x06040200u)));
  }
#pragma unroll
  for (int m = 0; m < 3; ++m) st8_nt(dst + kLowBytes + 8 * (256 * m + tid), sym[2 * m], sym[2 * m + 1]);
  for (int i = tid; i < var_len / 16; i += kThreads)
    st16_nt(dst + kDenseBytes + 16 * i, reinterpret_cast<const uint4*>(sh.var32)[i]);
}

// Persistent encoder: workgroup g encodes records r = g, g + grid, ... of
// the n_closes * 2H records of this step (record r: kvh = r / n_closes of
// block close_list[r % n_closes]) from staging into the block's arena page (each record
// takes the next kDenseBytes + var_len bytes, claimed by CAS on fill), or raw
// into the overflow pool when it does not code or no longer fits; and hands
// the slot's record to the block's heir (hbm_kv.cu:262-429).  While record r
// is encoded from registers, record r + grid streams from HBM straight into
// this workgroup's LDS stage (global_load_lds: no registers held), each wave
// loading exactly the 16-byte words its own lanes read back.
struct EncStage {
  uint4 w[8][kThreads];  // record words: [st][thread], the staging layout
};

__device__ __forceinline__ void stage_record(EncStage& st_buf, const uint8_t* src) {
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  typedef const void __attribute__((address_space(1)))* gptr_t;
  typedef void __attribute__((address_space(3)))* lptr_t;
#pragma unroll
  for (int st = 0; st < 8; ++st)
    __builtin_amdgcn_global_load_lds((gptr_t)(src + 16 * (256 * st + tid)), (lptr_t)&st_buf.w[st][64 * wave], 16, 0,
                                     kNt);
}


// kBlockMajor (the ordered encode): workgroup g encodes whole blocks
// close_list[g], close_list[g + grid], ..., each block's 2H records in
// (kv, head) order, and places them itself: a record that codes takes the
// block's next kDenseBytes + var_len bytes if they fit in the page, else it
// spills to the overflow pool; later records of the block still try.  The
// placement then depends only on the records' sizes -- the same spill set on
// every run (the reference's encode claims page space in arrival order, so
// which record spills can change from run to run; its import places by a
// prefix over the lengths, hbm_kv.cu:628-642).
//
// The same placement in two parallel passes, for steps that close too few
// blocks to fill the device block by block: kMeasure analyses every record
// (no stores) and leaves in its table entries the variable length it codes
// to (rec_len; the raw length if it does not code) and the block's page fill
// (rec_addr); kPlaced then encodes every record in parallel, thread 0 of
// each workgroup walking the block's earlier records' lengths to find its
// offset by the rule above.  An earlier record of the same block may already
// have been finished by kPlaced: its entry then holds its final length --
// the same variable length if it was placed, the raw length if it spilled
// -- and either value leads to the same walk.  The block's last record
// writes the page fill.
enum EncMode { kEncClaim = 0, kEncBlockMajor = 1, kEncMeasure = 2, kEncPlaced = 3 };

template <int kMode, bool kWrite>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(kEncodeWgPerCu)))
encode_kernel(Store s, int layer, uint8_t* arena, int64_t page_bytes, const uint8_t* rank_of, StepTokens tk) {
  constexpr bool kBlockMajor = kMode == kEncBlockMajor;
  __shared__ EncShared sh;
  __shared__ EncStage stage;
  const int tid = threadIdx.x;
  const int per = 2 * s.H;
  const int n_closes = s.counters[kCloses];
  const int n_rec = n_closes * per;
  if constexpr (kWrite) {
    // the step's write: workgroups past the encoders, one wave per (token, head)
    if ((int)blockIdx.x >= tk.enc_grid) {
      write_item(s, tk, layer, ((int)blockIdx.x - tk.enc_grid) * (kThreads / 64) + (tid >> 6), true);
      return;
    }
  }
  int r = kBlockMajor ? (int)blockIdx.x * per : (int)blockIdx.x;
  if (r >= n_rec) return;
  // Claim-mode encode: each workgroup takes records x, x + grid, ... for the
  // first 7/8 of the rounds; the rest go out kDynBatch consecutive records at
  // a time from a cursor in the counters, so that workgroups that run faster
  // (the first dispatched on each CU; some XCDs) take more of them and the
  // launch ends when the average workgroup does (measured on MI355X with
  // static rounds only: workgroups ended within 4.9-5.7 ms of a 5.7 ms
  // launch).  A batch is grabbed one batch ahead (thread 0; published
  // through LDS at the end of the iteration) and its records' metadata
  // loaded when it is published.  The last workgroup to finish resets both
  // counters.
  constexpr bool kDyn = kMode == kEncClaim;
  constexpr int kDynBatch = 4;
  // Record metadata (block, heir, staging slot) of this workgroup's records
  // in batches of 64 (record r + j grid in lane j), loaded with vector loads
  // one batch ahead: scalar loads would be waited for at every LDS barrier.
  // The stage streams record r + grid while r is encoded.
  const int g = kWrite ? tk.enc_grid : (int)gridDim.x;
  const int lane = tid & 63;
  // (with fewer than 8 rounds the launch stays static: every workgroup then
  // has records, so every one reaches the counter that ends the tail)
  const int rounds = n_rec / g;
  const bool dyn = kDyn && rounds >= 8;
  const int k_static = dyn ? rounds - rounds / 8 : (1 << 30);
  const int n_static = dyn ? k_static * g : n_rec;
  // the k-th record of this workgroup: its block (close index) and (kv, head)
  auto rec_kvh = [&](int rr) { return kBlockMajor ? rr % per : rr / n_closes; };
  auto next_rec = [&](int rr) { return kBlockMajor ? (rr % per == per - 1 ? rr + 1 + (g - 1) * per : rr + 1) : rr + g; };
  auto load_meta = [&](int k0, int& mb, int& mh, int& mw) {
    mb = 0;
    mh = -1;
    mw = 0;
    const int kk = k0 + lane;
    const int ci = kBlockMajor ? (int)blockIdx.x + (kk / per) * g : ((int)blockIdx.x + kk * g) % n_closes;
    const bool ok = kBlockMajor ? ci < n_closes : (int)blockIdx.x + kk * g < n_rec;
    if (ok) {
      mb = s.close_list[ci];
      mh = s.close_list[s.cap + ci];
      mw = s.wslot[mb];
    }
  };
  int cb, ch, cw, nb, nh, nw;  // current / next batch
  load_meta(0, cb, ch, cw);
  load_meta(64, nb, nh, nw);
  // dynamic tail: the current batch [dyn_end - kDynBatch, dyn_end) and the
  // next one (start dyn_next, metadata of its record j in lane j of dn*)
  int dyn_end = 0, dyn_next = 0, dmb = 0, dmh = -1, dmw = 0, dnb = 0, dnh = -1, dnw = 0;
  int grabbed = 0;  // thread 0: the batch start to publish at the end of the iteration
  auto load_dyn_meta = [&](int start, int& mb, int& mh, int& mw) {
    mb = 0;
    mh = -1;
    mw = 0;
    const int rr = start + lane;
    if (lane < kDynBatch && rr < n_rec) {
      const int ci = rr % n_closes;
      mb = s.close_list[ci];
      mh = s.close_list[s.cap + ci];
      mw = s.wslot[mb];
    }
  };
  int b = __builtin_amdgcn_readfirstlane(cb);
  int heir = __builtin_amdgcn_readfirstlane(ch);
  uint8_t* src = staging_addr(s, __builtin_amdgcn_readfirstlane(cw), layer, rec_kvh(r));
  if constexpr (kWrite) write_own_rows(s, tk, layer, b, heir, rec_kvh(r));
  stage_record(stage, src);
  int rank_kvh = -1;
  // counter increments of this workgroup (thread 0), added once at the end:
  // one hot counter hit by every record serialises at its memory channel
  int n_enc = 0, n_fall = 0, n_err = 0, n_spill = 0;
  bool ovf_full = false;  // this workgroup found the overflow pool full
  int boff = 0;           // ordered encode: the block's next free page byte (thread 0)
  int r_next = r;
  for (int k = 0; r < n_rec; r = r_next, ++k) {
    const int kvh = rec_kvh(r);
    const int64_t idx = ((int64_t)layer * s.NB + b) * per + kvh;
    int32_t* fill = s.fill + (int64_t)layer * s.NB + b;
    if (kvh != rank_kvh) {  // consecutive records mostly share (layer, kvh)
      sh.tb[tid] = table_byte(rank_of[((int64_t)layer * per + kvh) * 256 + tid]);
      rank_kvh = kvh;
    }
    if (kMode != kEncMeasure)
      for (int i = tid; i < kVarCap / 4; i += kThreads) sh.var32[i] = 0;
    // the fill value is only a first guess for the claim: fetch it early
    int cur = 0;
    if (kBlockMajor) {
      if (tid == 0 && kvh == 0) boff = *fill;  // only this workgroup places this block's records
    } else if (kMode == kEncMeasure) {
      if (tid == 0) cur = *fill;  // no pass writes it before kPlaced's last record
    } else if (kMode == kEncPlaced) {
      if (tid == 0) cur = (int)s.rec_addr[idx];  // the fill kMeasure left here
    } else if (tid == 0) {
      cur = __hip_atomic_load(fill, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // this record's words: the wave's own LDS loads, then into registers
    __builtin_amdgcn_s_waitcnt(0);
    uint4 wd[8];
#pragma unroll
    for (int st = 0; st < 8; ++st) wd[st] = stage.w[st][tid];
    __builtin_amdgcn_s_waitcnt(0);  // reads done before the stage is refilled
    // the next record's metadata: lane (k + 1) % 64 of the current or next batch
    const int k1 = (k + 1) & 63;
    const bool nbatch = k1 == 0;
    int b1 = __builtin_amdgcn_readlane(nbatch ? nb : cb, k1);
    int heir1 = __builtin_amdgcn_readlane(nbatch ? nh : ch, k1);
    int w1 = __builtin_amdgcn_readlane(nbatch ? nw : cw, k1);
    uint8_t* src1 = src;
    int r1 = next_rec(r);
    bool new_batch = false;
    if (dyn && k + 1 >= k_static) {
      if (r + 1 < dyn_end) {  // the current tail batch goes on
        r1 = r + 1;
        const int j = r1 - (dyn_end - kDynBatch);
        b1 = __builtin_amdgcn_readlane(dmb, j);
        heir1 = __builtin_amdgcn_readlane(dmh, j);
        w1 = __builtin_amdgcn_readlane(dmw, j);
      } else {  // the next batch: grabbed one batch ago, metadata loaded
        r1 = dyn_next;
        dyn_end = dyn_next + kDynBatch;
        dmb = dnb;
        dmh = dnh;
        dmw = dnw;
        b1 = __builtin_amdgcn_readlane(dmb, 0);
        heir1 = __builtin_amdgcn_readlane(dmh, 0);
        w1 = __builtin_amdgcn_readlane(dmw, 0);
        new_batch = r1 < n_rec;
      }
      r1 = min(r1, n_rec);
    }
    // the first tail batch is grabbed three records before the static rounds
    // end (workgroups get there at different times, so the grabs spread out),
    // each later one when the batch before it starts
    if (dyn && k == k_static - 3) new_batch = true;
    if (new_batch && tid == 0) grabbed = n_static + atomicAdd(&s.counters[kEncCursor], kDynBatch);
    r_next = r1;
    if (r1 < n_rec) {
      src1 = staging_addr(s, w1, layer, rec_kvh(r1));
      if constexpr (kWrite) write_own_rows(s, tk, layer, b1, heir1, rec_kvh(r1));
      stage_record(stage, src1);
    }
    if (nbatch) {  // the next batch becomes current; load the one after
      cb = nb;
      ch = nh;
      cw = nw;
      load_meta(k + 65, nb, nh, nw);
    }
    if (kMode != kEncMeasure && heir >= 0) {
      const uint8_t* from = staging_addr(s, s.wslot[heir], layer, kvh);
#pragma unroll
      for (int st = 0; st < 8; ++st)
        *reinterpret_cast<uint4*>(src + 16 * (256 * st + tid)) = ld16(from + 16 * (256 * st + tid));
      if (tid == 0) s.rec_addr[((int64_t)layer * s.NB + heir) * per + kvh] = reinterpret_cast<int64_t>(src);
    }
    lds_barrier();
    uint32_t sym[6], code[8], nib[8];
    int eo, ro;
    const EncResult res = enc_analyse(wd, sh, sym, code, nib, eo, ro);
    if (kMode == kEncMeasure) {
      if (tid == 0) {
        s.rec_len[idx] = res.codes ? res.var_len : kRawVarLen;
        s.rec_addr[idx] = cur;
      }
      lds_barrier();  // sh (wsum; rank on a head change) is reused by the next record
      b = b1;
      heir = heir1;
      src = src1;
      continue;
    }
    if (kMode == kEncPlaced) {
      if (tid == 0) {
        // the block's earlier records in (kv, head) order
        const int32_t* lens = s.rec_len + ((int64_t)layer * s.NB + b) * per;
        int off = cur;
        for (int q = 0; q < kvh; ++q) {
          const int l = lens[q];
          if (l <= kVarCap && off + kDenseBytes + l <= page_bytes) off += kDenseBytes + l;
        }
        const int need = kDenseBytes + res.var_len;
        const bool fits = res.codes && off + need <= page_bytes;
        sh.s_off = fits ? off : -1;
        n_spill += res.codes && !fits;
        if (kvh == per - 1) *fill = fits ? off + need : off;  // the block's records are placed
      }
      if (res.codes) enc_var(wd, code, nib, sh, res, eo, ro);
    } else if (kBlockMajor && res.codes) {
      const int need = kDenseBytes + res.var_len;
      enc_var(wd, code, nib, sh, res, eo, ro);
      if (tid == 0) {
        const bool fits = boff + need <= page_bytes;
        sh.s_off = fits ? boff : -1;
        n_spill += !fits;
        if (fits) boff += need;
      }
    } else if (res.codes) {
      // first claim attempt in flight while the variable region is built
      const int need = kDenseBytes + res.var_len;
      int prev = -1;
      if (tid == 0 && cur + need <= page_bytes) prev = atomicCAS(fill, cur, cur + need);
      enc_var(wd, code, nib, sh, res, eo, ro);
      if (tid == 0) {
        int off = -1;
        if (cur + need <= page_bytes) {
          if (prev == cur) {
            off = cur;
          } else {
            cur = prev;
            while (cur + need <= page_bytes) {
              prev = atomicCAS(fill, cur, cur + need);
              if (prev == cur) {
                off = cur;
                break;
              }
              cur = prev;
            }
          }
        }
        n_spill += off < 0;
        sh.s_off = off;
      }
    } else if (tid == 0) {
      sh.s_off = -1;
    }
    lds_barrier();
    if (sh.s_off < 0) {
      if (tid < 64) {
        // Nothing frees overflow slots while an encode runs (frees happen in
        // prepare, on the same stream), so once this workgroup finds the pool
        // full every later allocation of the launch fails too: skip the scan.
        const int slot = ovf_full ? -1 : ovf_alloc_wave(s, (uint32_t)(b * per + kvh), tid);
        if (tid == 0) {
          n_err += slot < 0;
          ++n_fall;
          ++n_enc;
          sh.s_ovf = slot;
        }
      }
      lds_barrier();
      const int slot = sh.s_ovf;
      ovf_full = slot < 0;
      if (slot >= 0) {  // else the record stays in staging (data loss is counted)
        uint8_t* dst = s.ovf_base + (int64_t)slot * kRawRecord;
#pragma unroll
        for (int st = 0; st < 8; ++st) st16_nt(dst + 16 * (256 * st + tid), wd[st]);
        if (tid == 0) {
          s.rec_addr[idx] = reinterpret_cast<int64_t>(dst);
          s.rec_len[idx] = kRawVarLen;
        }
      }
    } else {
      uint8_t* dst = arena + (int64_t)b * page_bytes + sh.s_off;
      enc_store(dst, wd, sym, sh, res.var_len);
      if (tid == 0) {
        s.rec_addr[idx] = reinterpret_cast<int64_t>(dst);
        s.rec_len[idx] = res.var_len;
        ++n_enc;
      }
    }
    if (kBlockMajor && tid == 0 && kvh == per - 1) *fill = boff;  // the block's records are placed
    if (new_batch && tid == 0) sh.dyn_start = grabbed;
    lds_barrier();  // sh (var32, s_off, s_ovf; rank on a head change) is reused by the next record
    if (new_batch) {
      dyn_next = __builtin_amdgcn_readfirstlane(sh.dyn_start);
      load_dyn_meta(dyn_next, dnb, dnh, dnw);
    }
    b = b1;
    heir = heir1;
    src = src1;
  }
  if (dyn && tid == 0) {
    // every workgroup has made its last grab: the last one out resets the tail
    if (atomicAdd(&s.counters[kEncDone], 1) == g - 1) {
      s.counters[kEncCursor] = 0;
      s.counters[kEncDone] = 0;
    }
  }
  if (tid == 0) {
    if (n_enc) atomicAdd(&s.counters[kEncoded], n_enc);
    if (n_fall) atomicAdd(&s.counters[kFallbacks], n_fall);
    if (n_err) atomicAdd(&s.counters[kErrOverflow], n_err);
    if (n_spill) atomicAdd(&s.counters[kSpills], n_spill);
  }
}

// commit: closed blocks hand their slot to their heir or push a persistent
// slot back on the free stack (in close-list order); the close count is
// reset so a forward without a fresh prepare encodes nothing.
__global__ void __launch_bounds__(kPrepThreads) commit_kernel(Store s) {
  __shared__ PrepShared sh;
  const int n = s.counters[kCloses];
  const int top = s.counters[kFreeTop];
  const int pushed = wg_compact(
      n, sh, [&](int c) { return make_int2(s.close_list[c], s.close_list[s.cap + c]); },
      [&](int, int2 e) {
        const int b = e.x, heir = e.y;
        const int w = s.wslot[b];
        s.wslot[b] = -1;
        if (heir >= 0) s.wslot[heir] = w;
        return heir < 0 && w >= 0 && w < s.S_p ? w : -1;
      },
      [&](int, int r, int w) { s.free_stack[top + r] = w; });
  if (threadIdx.x == 0) {
    s.counters[kFreeTop] = top + pushed;
    s.counters[kCloses] = 0;
  }
}

// ---------------------------------------------------------------------------
// Decode of whole records into token-major BF16 (gather / batch decode).
// One 256-thread workgroup per record: wave W decodes slab W (kernel-order
// threads 64W..64W+63, lane = thread) into an LDS tile [128 tok][128 dim],
// then the tile is stored with 16-byte coalesced writes.

constexpr int kTileRow = 256;  // bytes per token row in the tile
struct DecShared {
  uint8_t tile[kTokens * kTileRow];
  uint8_t esc[4][kEscLds];
};

__device__ __forceinline__ int tile_off(int tok, int dim) {
  // 16-byte chunk of the row swizzled by the token so that the column
  // writes of V records spread over banks.
  return tok * kTileRow + ((((dim >> 3) ^ (tok & 15)) & 15) << 4) + 2 * (dim & 7);
}

__device__ void decode_record_to_tile(const uint8_t* rec, int vlen, int kv, const HeadLut& lut, DecShared& sh) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int w = tid >> 5, g = (tid >> 2) & 7, c = tid & 3;
  auto put = [&](int st, const uint4& wd) {
    const uint32_t d[4] = {wd.x, wd.y, wd.z, wd.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = i >> 1, f = i & 1;
      const int row = 16 * w + 8 * j + g, col = 16 * st + 8 * f + 2 * c;
      if (kv == 0) {
        *reinterpret_cast<uint32_t*>(sh.tile + tile_off(row, col)) = d[i];
      } else {
        *reinterpret_cast<uint16_t*>(sh.tile + tile_off(col, row)) = (uint16_t)d[i];
        *reinterpret_cast<uint16_t*>(sh.tile + tile_off(col + 1, row)) = (uint16_t)(d[i] >> 16);
      }
    }
  };
  auto emit = [&](auto st, const uint4& wd) { put(decltype(st)::value, wd); };
  SlabBuf b;
  const bool raw = vlen > kVarCap;
  load_thread(rec, raw, tid, b);
  if (raw) {
    raw_words(b, rec, tid, emit);
    return;
  }
  const uint8_t* var = rec + kDenseBytes;
  auto rd4 = [&](int off) { return ld4(var + off); };
  const SlabHdr h = slab_header(rd4, wave);
  stage_escapes(rd4, h, lut.s, sh.esc[wave], lane);
  const int cnt = thread_escapes(b);
  const int incl = wave_incl_scan(cnt);
  decode_words(b, sh.esc[wave], (h.e0 & 7) + incl - cnt, lut.p0, lut.p1, emit);
}

// Stores the tile: token row r to out + r * row_stride (bytes).
__device__ __forceinline__ void store_tile(const DecShared& sh, uint8_t* out, int64_t row_stride) {
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int x = q * kThreads + threadIdx.x, r = x >> 4, jj = x & 15;
    const uint4 val = *reinterpret_cast<const uint4*>(sh.tile + r * kTileRow + (((jj ^ (r & 15)) & 15) << 4));
    st16_nt(out + r * row_stride + jj * 16, val);
  }
}

// grid (P, 2H): record kvh of block src[i] at one layer -> workspace page i.
__global__ void __launch_bounds__(kThreads) gather_kernel(const int32_t* src, const int64_t* rec_addr,
                                                         const int32_t* rec_len, const uint32_t* plut,
                                                         const uint8_t* slut, uint8_t* wk, uint8_t* wv, int H) {
  extern __shared__ __align__(16) uint8_t smem[];
  DecShared& sh = *reinterpret_cast<DecShared*>(smem);
  const int kvh = blockIdx.y, kv = kvh / H, h = kvh % H;
  const int64_t idx = (int64_t)src[blockIdx.x] * 2 * H + kvh;
  const uint8_t* rec = reinterpret_cast<const uint8_t*>(rec_addr[idx]);
  decode_record_to_tile(rec, rec_len[idx], kv, load_lut(plut, slut, kvh), sh);
  __syncthreads();
  uint8_t* out = (kv == 0 ? wk : wv) + ((int64_t)blockIdx.x * kTokens * H + h) * kTileRow;
  store_tile(sh, out, (int64_t)H * kTileRow);
}

// Streaming probe: record r (32 KB-strided in src and dst) reads its first
// rb bytes and writes its first wb of them back to dst, records r =
// blockIdx.x, + gridDim.x, ...; eight 16-byte non-temporal loads per thread
// in flight, then the stores.  No computation: the HBM rate of a given
// read / write mix at a given number of bytes in flight per CU, for reading
// the encoder's rate against.
__global__ void __launch_bounds__(kThreads) stream_probe_kernel(const uint8_t* src, uint8_t* dst, int64_t n, int rb,
                                                               int wb) {
  const int tid = threadIdx.x;
  for (int64_t r = blockIdx.x; r < n; r += gridDim.x) {
    const uint8_t* from = src + r * kRawRecord;
    uint8_t* to = dst + r * kRawRecord;
    uint4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int o = 16 * (tid + kThreads * k);
      v[k] = o < rb ? ld16_nt(from + o) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int o = 16 * (tid + kThreads * k);
      if (o < wb) st16_nt(to + o, v[k]);
    }
  }
}

// grid (n): record i (any table, K or V) -> out [i, 128, 128].
__global__ void __launch_bounds__(kThreads) decode_records_kernel(const int64_t* rec_addr, const int32_t* rec_len,
                                                                 const int32_t* kv, const uint32_t* plut,
                                                                 const uint8_t* slut, const int32_t* tab_idx,
                                                                 uint8_t* out) {
  extern __shared__ __align__(16) uint8_t smem[];
  DecShared& sh = *reinterpret_cast<DecShared*>(smem);
  const int i = blockIdx.x;
  const uint8_t* rec = reinterpret_cast<const uint8_t*>(rec_addr[i]);
  decode_record_to_tile(rec, rec_len[i], kv[i], load_lut(plut, slut, tab_idx[i]), sh);
  __syncthreads();
  store_tile(sh, out + (int64_t)i * kRawRecord, kTileRow);
}

// grid (n): token-major record i -> coded bytes in out row i, lens[i].
__global__ void __launch_bounds__(kThreads) encode_records_kernel(const uint16_t* raw, const int32_t* kvs,
                                                                 const uint8_t* rank_of, const int32_t* tab_idx,
                                                                 uint8_t* out, int32_t* lens) {
  __shared__ EncShared sh;
  // the token-major record, staged with coalesced 16-byte loads; rows padded
  // by 8 bytes so the column reads of V records spread over the banks
  constexpr int kRowElems = kDim + 4;
  __shared__ __align__(16) uint16_t rec[kTokens * kRowElems];
  const int i = blockIdx.x, tid = threadIdx.x;
  const int kv = kvs[i];
  const uint16_t* src = raw + (int64_t)i * kTokens * kDim;
  sh.tb[tid] = table_byte(rank_of[(int64_t)tab_idx[i] * 256 + tid]);
  for (int x = tid; x < kVarCap / 4; x += kThreads) sh.var32[x] = 0;
#pragma unroll
  for (int k = 0; k < kTokens * kDim / 8 / kThreads; ++k) {
    const int e = 8 * (k * kThreads + tid), row = e / kDim, col = e % kDim;  // 16-byte piece
    const uint4 v = *reinterpret_cast<const uint4*>(src + e);
    uint2* d = reinterpret_cast<uint2*>(rec + row * kRowElems + col);  // 8-byte aligned (padded rows)
    d[0] = make_uint2(v.x, v.y);
    d[1] = make_uint2(v.z, v.w);
  }
  __syncthreads();
  // thread tid's kernel-order words
  const int w = tid >> 5, g = (tid >> 2) & 7, c = tid & 3;
  uint4 wd[8];
#pragma unroll
  for (int st = 0; st < 8; ++st) {
    uint32_t d[4];
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const int j = i4 >> 1, f = i4 & 1;
      const int row = 16 * w + 8 * j + g, col = 16 * st + 8 * f + 2 * c;
      if (kv == 0) {
        d[i4] = *reinterpret_cast<const uint32_t*>(rec + row * kRowElems + col);
      } else {
        d[i4] = (uint32_t)rec[col * kRowElems + row] | ((uint32_t)rec[(col + 1) * kRowElems + row] << 16);
      }
    }
    wd[st] = make_uint4(d[0], d[1], d[2], d[3]);
  }
  __syncthreads();
  uint32_t sym[6], code[8], nib[8];
  int eo, ro;
  const EncResult res = enc_analyse(wd, sh, sym, code, nib, eo, ro);
  uint8_t* dst = out + (int64_t)i * kRawRecord;
  if (!res.codes) {
#pragma unroll
    for (int st = 0; st < 8; ++st) *reinterpret_cast<uint4*>(dst + 16 * (256 * st + tid)) = wd[st];
    if (tid == 0) lens[i] = kRawRecord;
    return;
  }
  enc_var(wd, code, nib, sh, res, eo, ro);
  enc_store(dst, wd, sym, sh, res.var_len);
  if (tid == 0) lens[i] = kDenseBytes + res.var_len;
}

// ---------------------------------------------------------------------------
// Block blobs: the on-wire form of a closed block (hbm_kv.cu:496-665).  The
// byte format is kept exactly, since blobs travel between stores and tiers:
// a 64-byte header (u32 magic "FPKB", version, L, H; i64 declared bytes,
// table digest; the rest zero), the i32 rec_len table [L, 2, H], padding to
// a 4096-byte head, then every record in (layer, kv, head) order, each
// DENSE + var_len bytes (raw: 32 KB).
//
// The kernels move one record per wavefront.  A wave finds its record's place
// in the blob by summing the sizes before it 64 table entries at a time (one
// DPP reduction per 64), then streams the record through two buffer
// resources with kCopyDepth 16-byte loads per lane in flight before the first
// store; the resources' bounds end the record, so lanes past its end neither
// load nor store and nothing is predicated.
constexpr uint32_t kBlobMagic = 0x424B5046u;  // "FPKB"
constexpr uint32_t kBlobVersion = 1;
constexpr int kBlobFixed = 64;
constexpr int64_t kBlobAlign = 4096;
constexpr int kMaxHeads = 16;
enum : int { kBlobBadHeader = 1, kBlobBadLengths = 2, kBlobNoOverflow = 4 };
constexpr int kCopyDepth = 8;       // 16-byte loads in flight per lane: 8 KB per wave
constexpr int kExportWaves = 4;     // records per export workgroup
constexpr int kImportWaves = 8;     // waves of an import workgroup (one blob layer)

__host__ __device__ __forceinline__ int64_t blob_head_bytes(int L, int H) {
  return (kBlobFixed + 8LL * L * H + kBlobAlign - 1) / kBlobAlign * kBlobAlign;
}

// Copies ``bytes`` (a 16-byte multiple, at most 32 KB) from ``src`` to
// ``dst`` with the whole wave: each round issues kCopyDepth 16-byte loads per
// lane (1 KB apart per load), then their stores.  The whole offset is in the
// lane's offset (with the instruction's immediate), the part the bounds
// check covers; the wave-uniform offset register stays 0.
__device__ __forceinline__ void wave_copy_record(uint8_t* dst, const uint8_t* src, int bytes, int lane) {
  const rsrc_t rs = make_rsrc(src, bytes), rd = make_rsrc(dst, bytes);
  for (int base = 16 * lane; base < bytes + 16 * lane; base += 1024 * kCopyDepth) {
    u32x4_t v[kCopyDepth];
#pragma unroll
    for (int k = 0; k < kCopyDepth; ++k) v[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, base + 1024 * k, 0, kNt);
#pragma unroll
    for (int k = 0; k < kCopyDepth; ++k) __builtin_amdgcn_raw_buffer_store_b128(v[k], rd, base + 1024 * k, 0, kNt);
  }
}

// Sum over entries [0, upto) of ``size(g)`` (each at most 32 KB), 64 entries
// per step across the wave.
template <class Size>
__device__ __forceinline__ int64_t wave_bytes_before(const Size& size, int upto, int lane) {
  int64_t sum = 0;
  for (int c = 0; c < upto; c += 64) sum += wave_total<false>(c + lane < upto ? size(c + lane) : 0);
  return sum;
}

// grid n x ceil(L * 2H / kExportWaves), blob-major (neighbouring workgroups
// write neighbouring records): wave w of the blob's workgroup y copies
// record g = y * kExportWaves + w (layer g / 2H, kv-head g % 2H); the
// wave of record 0 also writes the header, the length table and the blob's
// aligned length.
__global__ void __launch_bounds__(64 * kExportWaves) blob_export_kernel(const int32_t* blocks, const int64_t* rec_addr,
                                                                       const int32_t* rec_len, uint8_t* out,
                                                                       int64_t stride, int64_t* lengths, int L, int H,
                                                                       int NB, int64_t digest) {
  const int lane = wave_lane(), w = uniform((int)(threadIdx.x >> 6));
  const int per = 2 * H, count = L * per, groups = (count + kExportWaves - 1) / kExportWaves;
  const int i = (int)(blockIdx.x / groups);  // blob
  const int g = (int)(blockIdx.x % groups) * kExportWaves + w;
  const int b = uniform(blocks[i]);
  // table entry of record gg: rec_len[layer][b][kv-head]
  auto entry = [&](int gg) { return ((int64_t)(gg / per) * NB + b) * per + gg % per; };
  auto size = [&](int gg) { return kDenseBytes + rec_len[entry(gg)]; };
  uint8_t* blob = out + (int64_t)i * stride;
  const int64_t head = blob_head_bytes(L, H);
  if (g == 0) {
    int64_t total = 0;
    int32_t* table = reinterpret_cast<int32_t*>(blob + kBlobFixed);
    for (int c = 0; c < count; c += 64) {
      int n = 0;
      if (c + lane < count) {
        const int len = rec_len[entry(c + lane)];
        table[c + lane] = len;
        n = kDenseBytes + len;
      }
      total += wave_total<false>(n);
    }
    if (lane < kBlobFixed / 8) {
      // header words as eight u64 lanes: (magic, version), (L, H), bytes, digest, zeros
      const uint64_t word[4] = {(uint64_t)kBlobVersion << 32 | kBlobMagic, (uint64_t)(uint32_t)H << 32 | (uint32_t)L,
                                (uint64_t)(head + total), (uint64_t)digest};
      reinterpret_cast<uint64_t*>(blob)[lane] = lane < 4 ? word[lane] : 0;
    }
    if (lane == 0) lengths[i] = (head + total + kBlobAlign - 1) / kBlobAlign * kBlobAlign;
  }
  if (g >= count) return;
  const int64_t at = head + wave_bytes_before(size, g, lane);
  const int64_t e = entry(g);
  const int n = uniform(kDenseBytes + rec_len[e]);
  wave_copy_record(blob + at, reinterpret_cast<const uint8_t*>(uniform64(rec_addr[e])), n, lane);
}

// Claims one overflow slot for every lane with ``want`` set (a wave claims
// for up to 64 records at once).  Lanes read 64 consecutive bitmap words from
// word ``hint`` on; the wave ranks their free bits, each lane takes with one
// atomicOr the free bits that serve the next unserved claims, and the bits
// won are handed to the claiming lanes in rank order.  Bits another caller
// took meanwhile are retried while the window still shows free bits, then
// the next 64 words are read.  Returns the lane's slot, or -1 if the pool
// ran out (slots won for other lanes are kept: the caller frees them).
__device__ int ovf_alloc_many(const Store& s, uint32_t hint, bool want, int lane) {
  const uint64_t wanting = __ballot(want);
  const int need = __popcll(wanting);
  const int rank = __popcll(wanting & ((1ull << lane) - 1));
  const uint32_t nw = (uint32_t)s.ovf_words;
  int got = 0, slot = -1;
  for (uint32_t base = 0; base < nw && got < need; base += 64) {
    const uint32_t wi = base + (uint32_t)lane;
    const int word = wi < nw ? (int)((hint + wi) % nw) : 0;
    uint32_t cur = wi < nw ? __hip_atomic_load(&s.ovf_bits[word], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                           : 0xffffffffu;
    while (got < need && __ballot(cur != 0xffffffffu)) {
      const int free_n = __popc(~cur);
      const int before = wave_incl_scan(free_n) - free_n;
      const int take = max(0, min(free_n, need - got - before));
      uint32_t mask = 0, avail = ~cur;
      for (int k = 0; k < take; ++k) {
        mask |= avail & (0u - avail);  // lowest free bit
        avail &= avail - 1;
      }
      const uint32_t prev = mask ? atomicOr(&s.ovf_bits[word], mask) : cur;
      const uint32_t won = mask & ~prev;
      cur = prev | mask;
      // hand the won bits to the claiming lanes in rank order
      for (uint64_t owners = __ballot(won != 0); owners; owners &= owners - 1) {
        const int j = __builtin_ctzll(owners);
        uint32_t bits = __builtin_amdgcn_readlane(won, j);
        const int wj = __builtin_amdgcn_readlane(word, j);
        for (; bits; bits &= bits - 1, ++got)
          if (want && rank == got) slot = 32 * wj + __builtin_ctz(bits);
      }
    }
  }
  return slot;
}

// Checks blob i's header and whole length table; every wave of every layer's
// workgroup runs it on its own (scalar loads and one pass over the table),
// so no workgroup waits for another.  Returns the failure bit (0: valid) and
// the bytes of the layers before ``l``.
__device__ int blob_check(const uint8_t* src, int64_t src_bytes, int64_t off, int L, int H, int l, int64_t digest,
                          int lane, int64_t& before_layer) {
  const int per = 2 * H, count = L * per;
  const int64_t head = blob_head_bytes(L, H);
  if (off < 0 || off % 16 || off + head > src_bytes) return kBlobBadHeader;
  const uint8_t* blob = src + off;
  const uint32_t magic = uniform(ld4(blob)), version = uniform(ld4(blob + 4));
  const int bl = uniform((int)ld4(blob + 8)), bh = uniform((int)ld4(blob + 12));
  const uint2 d0 = ld8(blob + 16), d1 = ld8(blob + 24);
  const int64_t declared = (int64_t)((uint64_t)uniform(d0.y) << 32 | uniform(d0.x));
  const int64_t dig = (int64_t)((uint64_t)uniform(d1.y) << 32 | uniform(d1.x));
  if (magic != kBlobMagic || version != kBlobVersion || bl != L || bh != H || dig != digest || declared < head ||
      off + declared > src_bytes)
    return kBlobBadHeader;
  const int32_t* table = reinterpret_cast<const int32_t*>(blob + kBlobFixed);
  int64_t total = 0;
  before_layer = 0;
  bool bad = false;
  for (int c = 0; c < count; c += 64) {
    int n = 0, nb = 0;
    if (c + lane < count) {
      const int v = table[c + lane];
      if (v == kRawVarLen || (v >= kHeaderBytes && v <= kVarCap && v % 16 == 0))
        n = kDenseBytes + v;
      else
        bad = true;
      nb = (c + lane) / per < l ? n : 0;
    }
    total += wave_total<false>(n);
    before_layer += wave_total<false>(nb);
  }
  if (__ballot(bad) || head + total != declared) return kBlobBadLengths;
  return 0;
}

// grid (n, L), kImportWaves waves: workgroup (i, l) validates blob i and
// installs its layer-l records into blocks[i].  In (kv, head) order a coded
// record goes to the block's arena page at the page's running fill if it
// fits, otherwise -- and every raw record -- to an overflow slot; wave 0
// decides the placement (lanes = records), claims all its overflow slots at
// once, and on a full pool returns them and fails the layer, whose tables
// stay untouched.  Every wave then copies its records (one per wave at a
// time) and wave 0 installs the tables, freeing overflow slots the block's
// old records held.
__global__ void __launch_bounds__(64 * kImportWaves) blob_import_kernel(Store s, const uint8_t* src, int64_t src_bytes,
                                                                       const int64_t* offsets, const int32_t* blocks,
                                                                       int32_t* status, const int64_t* arena_base,
                                                                       const int64_t* arena_stride, int64_t digest) {
  __shared__ int64_t s_from[2 * kMaxHeads], s_to[2 * kMaxHeads];
  __shared__ int s_ok;
  const int lane = wave_lane(), w = uniform((int)(threadIdx.x >> 6));
  const int i = blockIdx.x, l = blockIdx.y, L = s.L, H = s.H, per = 2 * H;
  const int b = uniform(blocks[i]);
  const int64_t off = uniform64(offsets[i]);
  int64_t before_layer = 0;
  const int fail = blob_check(src, src_bytes, off, L, H, l, digest, lane, before_layer);
  if (fail) {
    if (threadIdx.x == 0) atomicOr(&status[i], fail);
    return;
  }
  const uint8_t* blob = src + off;
  const int32_t* lens = reinterpret_cast<const int32_t*>(blob + kBlobFixed) + l * per;
  if (w == 0) {
    const int len = lane < per ? lens[lane] : 0;
    const int n = kDenseBytes + len;
    // page placement in (kv, head) order: a coded record takes the page's
    // running fill when it fits (the rule is sequential: a record that does
    // not fit leaves the fill for the smaller ones after it)
    const int64_t page = uniform64(arena_stride[l]);
    int fill = 0, at = -1;
    for (int k = 0; k < per; ++k) {
      const int nk = __builtin_amdgcn_readlane(n, k);
      if (__builtin_amdgcn_readlane(len, k) != kRawVarLen && fill + nk <= page) {
        if (lane == k) at = fill;
        fill += nk;
      }
    }
    const int from = wave_incl_scan(lane < per ? n : 0) - n;  // the record's bytes past the layer's first
    const bool ovf = lane < per && at < 0;
    const int slot = ovf_alloc_many(s, (uint32_t)(b * per), ovf, lane);
    const bool ok = !__ballot(ovf && slot < 0);
    if (!ok) {
      if (ovf && slot >= 0) ovf_free(s, reinterpret_cast<int64_t>(s.ovf_base) + (int64_t)slot * kRawRecord);
      if (lane == 0) atomicOr(&status[i], kBlobNoOverflow);
    } else if (lane < per) {
      s_from[lane] = blob_head_bytes(L, H) + before_layer + from;
      s_to[lane] = ovf ? reinterpret_cast<int64_t>(s.ovf_base) + (int64_t)slot * kRawRecord
                       : uniform64(arena_base[l]) + (int64_t)b * page + at;
    }
    if (lane == 0) {
      s_ok = ok;
      if (ok) s.fill[(int64_t)l * s.NB + b] = fill;
    }
  }
  __syncthreads();
  if (!s_ok) return;
  for (int k = w; k < per; k += kImportWaves)
    wave_copy_record(reinterpret_cast<uint8_t*>(s_to[k]), blob + s_from[k], uniform(kDenseBytes + lens[k]), lane);
  if (w == 0 && lane < per) {
    const int64_t e = ((int64_t)l * s.NB + b) * per + lane;
    ovf_free(s, s.rec_addr[e]);
    s.rec_addr[e] = s_to[lane];
    s.rec_len[e] = lens[lane];
  }
}

}  // namespace
}  // namespace fp

using namespace fp;

extern "C" int fp_hbm_prepare(const fp_store_t* d, const int64_t* slot_mapping, int64_t n_tok, const int32_t* live,
                              int64_t n_live, int64_t step, fp_stream_t stream) {
  if (check_store(d)) return -1;
  FP_CHECK(n_tok >= 0 && n_live >= 0, "negative token or live count");
  FP_CHECK(2 * n_tok <= 2 * d->list_cap, "block lists too small");
  FP_CHECK(n_live <= d->num_blocks, "more live blocks than blocks");
  FP_CHECK(d->staging_slots <= 32LL * kLiveWords, "too many persistent staging slots (at most 262144)");
  FP_CHECK(n_tok < (1LL << 30), "too many tokens in one step");
  const Store s = make_store(d);
  hipLaunchKernelGGL(prepare_kernel, dim3(1), dim3(kPrepThreads), 0, stream, s, slot_mapping, (int)n_tok, live,
                     (int)n_live, (int32_t)step);
  FP_LAUNCH_CHECK();
  return 0;
}

// Checks of a write's arguments; fills ``tk`` (enc_grid 0).
static int write_args(const fp_store_t* d, const void* key, int64_t k_s0, int64_t k_s1, const void* value,
                      int64_t v_s0, int64_t v_s1, const int64_t* slot_mapping, int64_t n, int64_t layer,
                      StepTokens& tk, int64_t& write_grid) {
  FP_CHECK(n > 0 && layer >= 0 && layer < d->num_layers, "bad token count or layer");
  FP_CHECK(key && value && slot_mapping, "write needs K, V and the slot mapping");
  FP_CHECK(k_s0 % 2 == 0 && k_s1 % 2 == 0 && v_s0 % 2 == 0 && v_s1 % 2 == 0,
           "K/V strides must keep dim pairs 4-byte aligned");
  FP_CHECK(n < (1LL << 30), "too many tokens in one step");
  tk = StepTokens{static_cast<const uint16_t*>(key), static_cast<const uint16_t*>(value), k_s0, k_s1, v_s0, v_s1,
                  slot_mapping, (int)n, 0};
  const int64_t items = n * d->kv_heads;
  FP_CHECK(items < (1LL << 30), "too many (token, head) items in one step");  // int item indices
  write_grid = (items + kThreads / 64 - 1) / (kThreads / 64);
  return 0;
}

extern "C" int fp_hbm_write(const fp_store_t* d, const void* key, int64_t k_s0, int64_t k_s1, const void* value,
                            int64_t v_s0, int64_t v_s1, const int64_t* slot_mapping, int64_t n, int64_t layer,
                            fp_stream_t stream) {
  if (n == 0) return 0;
  if (check_store(d)) return -1;
  StepTokens tk;
  int64_t grid = 0;
  if (write_args(d, key, k_s0, k_s1, value, v_s0, v_s1, slot_mapping, n, layer, tk, grid)) return -1;
  const Store s = make_store(d);
  // Large steps with 16-byte aligned K and V rows take the slab path: one
  // wave per 16 tokens and record.  Either grid is a multiple of 8 (XCD-contiguous).
  const bool aligned = ((reinterpret_cast<uintptr_t>(key) | reinterpret_cast<uintptr_t>(value)) & 15) == 0 &&
                       ((k_s0 | k_s1 | v_s0 | v_s1) & 7) == 0;
  if (n * d->kv_heads >= kWriteSlabItems && aligned) {
    grid = ((n + kSlab - 1) / kSlab * 2 * d->kv_heads + kThreads / 64 - 1) / (kThreads / 64);
    grid = (grid + kXcds - 1) / kXcds * kXcds;
    hipLaunchKernelGGL(write_slab_kernel, dim3((unsigned)grid), dim3(kThreads), 0, stream, s, tk, (int)layer);
  } else {
    grid = (grid + kXcds - 1) / kXcds * kXcds;
    hipLaunchKernelGGL(write_kernel, dim3((unsigned)grid), dim3(kThreads), 0, stream, s, tk, (int)layer);
  }
  FP_LAUNCH_CHECK();
  return 0;
}

// The encode launches; with ``tk`` (non-null) the first one also performs
// the step's write (write_grid workgroups appended to its grid).
static int encode_launch(const fp_store_t* d, const uint8_t* rank_of, int64_t rank_of_elems, int64_t layer,
                         int64_t arena, int64_t page_bytes, int64_t max_close, bool ordered, fp_stream_t stream,
                         StepTokens* tk = nullptr, int64_t write_grid = 0) {
  if (max_close == 0) return 0;
  if (check_store(d)) return -1;
  FP_CHECK(max_close > 0 && max_close <= d->list_cap, "close list too small");
  FP_CHECK(rank_of_elems == d->num_layers * 2 * d->kv_heads * 256, "rank_of must hold every layer");
  FP_CHECK(page_bytes % 16 == 0 && page_bytes > 0 && page_bytes < (1LL << 31), "bad arena page size");
  FP_CHECK(layer >= 0 && layer < d->num_layers && arena % 16 == 0, "bad layer or arena address");
  FP_CHECK(max_close < (1LL << 31), "too many closing blocks");
  const Store s = make_store(d);
  // persistent grid: a few workgroups per CU, capped by the records there can be
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    FP_CHECK(hipGetDevice(&dev) == hipSuccess &&
                 hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0,
             "cannot query the CU count");
    cus = n;
  }
  const int64_t records = max_close * 2 * d->kv_heads;
  const int64_t slots = (int64_t)cus * kEncodeWgPerCu;
  uint8_t* arena_p = reinterpret_cast<uint8_t*>(arena);
  // the first launch's grid: its encoders, plus the write's workgroups when fused
  StepTokens none{nullptr, nullptr, 0, 0, 0, 0, nullptr, 0, 0};
  auto launch_first = [&](auto kernel_w, auto kernel, int64_t enc_grid) {
    if (tk) {
      tk->enc_grid = (int)enc_grid;
      hipLaunchKernelGGL(kernel_w, dim3((unsigned)(enc_grid + write_grid)), dim3(kThreads), 0, stream, s,
                         (int)layer, arena_p, page_bytes, rank_of, *tk);
    } else {
      hipLaunchKernelGGL(kernel, dim3((unsigned)enc_grid), dim3(kThreads), 0, stream, s, (int)layer, arena_p,
                         page_bytes, rank_of, none);
    }
  };
  const int64_t grid = std::min<int64_t>(records, slots);
  if (!ordered) {
    launch_first(encode_kernel<kEncClaim, true>, encode_kernel<kEncClaim, false>, grid);
  } else if (2 * ((records + slots - 1) / slots) < 2 * d->kv_heads) {
    // few blocks: two parallel passes (each record read twice) finish
    // before one workgroup per block has walked its 2H records
    launch_first(encode_kernel<kEncMeasure, true>, encode_kernel<kEncMeasure, false>, grid);
    FP_LAUNCH_CHECK();
    hipLaunchKernelGGL((encode_kernel<kEncPlaced, false>), dim3((unsigned)grid), dim3(kThreads), 0, stream, s,
                       (int)layer, arena_p, page_bytes, rank_of, none);
  } else {
    launch_first(encode_kernel<kEncBlockMajor, true>, encode_kernel<kEncBlockMajor, false>,
                 std::min<int64_t>(max_close, slots));
  }
  FP_LAUNCH_CHECK();
  return 0;
}

extern "C" int fp_hbm_encode(const fp_store_t* d, const uint8_t* rank_of, int64_t rank_of_elems, int64_t layer,
                             int64_t arena, int64_t page_bytes, int64_t max_close, fp_stream_t stream) {
  return encode_launch(d, rank_of, rank_of_elems, layer, arena, page_bytes, max_close, false, stream);
}

extern "C" int fp_hbm_encode_ordered(const fp_store_t* d, const uint8_t* rank_of, int64_t rank_of_elems,
                                     int64_t layer, int64_t arena, int64_t page_bytes, int64_t max_close,
                                     fp_stream_t stream) {
  return encode_launch(d, rank_of, rank_of_elems, layer, arena, page_bytes, max_close, true, stream);
}

extern "C" int fp_hbm_write_encode(const fp_store_t* d, const void* key, int64_t k_s0, int64_t k_s1,
                                   const void* value, int64_t v_s0, int64_t v_s1, const int64_t* slot_mapping,
                                   int64_t n, int64_t layer, const uint8_t* rank_of, int64_t rank_of_elems,
                                   int64_t arena, int64_t page_bytes, int64_t max_close, int ordered,
                                   fp_stream_t stream) {
  if (n == 0) return encode_launch(d, rank_of, rank_of_elems, layer, arena, page_bytes, max_close, ordered != 0, stream);
  if (max_close == 0) return fp_hbm_write(d, key, k_s0, k_s1, value, v_s0, v_s1, slot_mapping, n, layer, stream);
  if (check_store(d)) return -1;
  StepTokens tk;
  int64_t write_grid = 0;
  if (write_args(d, key, k_s0, k_s1, value, v_s0, v_s1, slot_mapping, n, layer, tk, write_grid)) return -1;
  return encode_launch(d, rank_of, rank_of_elems, layer, arena, page_bytes, max_close, ordered != 0, stream, &tk,
                       write_grid);
}

extern "C" int fp_hbm_commit(const fp_store_t* d, fp_stream_t stream) {
  if (check_store(d)) return -1;
  const Store s = make_store(d);
  hipLaunchKernelGGL(commit_kernel, dim3(1), dim3(kPrepThreads), 0, stream, s);
  FP_LAUNCH_CHECK();
  return 0;
}

static int set_dec_smem() {
  static bool done = false;
  if (!done) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(gather_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(DecShared)) != hipSuccess ||
        hipFuncSetAttribute(reinterpret_cast<const void*>(decode_records_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(DecShared)) != hipSuccess) {
      set_error("cannot raise the decode kernels' LDS limit");
      return -1;
    }
    done = true;
  }
  return 0;
}

extern "C" int fp_hbm_gather(const int32_t* src_blocks, int64_t n, const int64_t* rec_addr, const int32_t* rec_len,
                             const uint32_t* plut, const uint8_t* slut, void* wk, void* wv, int64_t ws_bytes,
                             int64_t kv_heads, fp_stream_t stream) {
  if (n == 0) return 0;
  FP_CHECK(n > 0 && kv_heads > 0 && kv_heads <= 64, "bad block count or kv_heads");
  FP_CHECK(ws_bytes >= n * kTokens * kv_heads * kTileRow, "workspace too small");
  FP_CHECK(n < (1LL << 31), "too many blocks");
  if (set_dec_smem()) return -1;
  hipLaunchKernelGGL(gather_kernel, dim3((unsigned)n, (unsigned)(2 * kv_heads)), dim3(kThreads), sizeof(DecShared),
                     stream, src_blocks, rec_addr, rec_len, plut, slut, static_cast<uint8_t*>(wk),
                     static_cast<uint8_t*>(wv), (int)kv_heads);
  FP_LAUNCH_CHECK();
  return 0;
}

extern "C" int fp_stream_probe(const void* src, void* dst, int64_t records, int64_t read_bytes, int64_t write_bytes,
                               int64_t wg_per_cu, fp_stream_t stream) {
  if (records == 0) return 0;
  FP_CHECK(records > 0 && wg_per_cu > 0 && wg_per_cu <= 8, "bad probe geometry");
  FP_CHECK(read_bytes >= 0 && read_bytes <= kRawRecord && read_bytes % 16 == 0 && write_bytes >= 0 &&
               write_bytes <= read_bytes && write_bytes % 16 == 0,
           "probe bytes must be multiples of 16 with write <= read <= 32768");
  FP_CHECK(reinterpret_cast<uintptr_t>(src) % 16 == 0 && reinterpret_cast<uintptr_t>(dst) % 16 == 0,
           "probe buffers must be 16-byte aligned");
  const int cus = device_cus();
  FP_CHECK(cus > 0, "cannot query the device's compute-unit count");
  const int64_t grid = std::min<int64_t>(records, wg_per_cu * cus);
  hipLaunchKernelGGL(stream_probe_kernel, dim3((unsigned)grid), dim3(kThreads), 0, stream,
                     static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst), records, (int)read_bytes,
                     (int)write_bytes);
  FP_LAUNCH_CHECK();
  return 0;
}

extern "C" int fp_hbm_export(const int32_t* blocks, int64_t n, const int64_t* rec_addr, const int32_t* rec_len,
                             int64_t num_layers, int64_t num_blocks, int64_t kv_heads, uint8_t* out,
                             int64_t out_bytes, int64_t stride, int64_t* lengths, int64_t digest,
                             fp_stream_t stream) {
  if (n == 0) return 0;
  FP_CHECK(n > 0 && num_layers > 0 && kv_heads > 0 && num_blocks > 0, "bad export geometry");
  FP_CHECK(reinterpret_cast<uintptr_t>(out) % 16 == 0, "export buffer must be contiguous 16-byte aligned uint8");
  FP_CHECK(stride % 16 == 0 &&
               stride >= blob_head_bytes((int)num_layers, (int)kv_heads) + 2LL * num_layers * kv_heads * kRawRecord &&
               out_bytes >= n * stride,
           "export stride or buffer too small");
  const int64_t count = 2 * num_layers * kv_heads;
  const int64_t groups = (count + kExportWaves - 1) / kExportWaves;
  FP_CHECK(n * groups < (1LL << 31), "too many blobs or records per blob in one export");
  hipLaunchKernelGGL(blob_export_kernel, dim3((unsigned)(n * groups)),
                     dim3(64 * kExportWaves), 0, stream, blocks,
                     rec_addr, rec_len, out, stride, lengths, (int)num_layers, (int)kv_heads, (int)num_blocks, digest);
  FP_LAUNCH_CHECK();
  return 0;
}

extern "C" int fp_hbm_import(const fp_store_t* d, const uint8_t* src, int64_t src_bytes, const int64_t* offsets,
                             const int32_t* blocks, int64_t n, int32_t* status, const int64_t* arena_base,
                             const int64_t* arena_stride, int64_t digest, fp_stream_t stream) {
  if (n == 0) return 0;
  if (check_store(d)) return -1;
  FP_CHECK(d->kv_heads <= kMaxHeads, "too many KV heads");
  FP_CHECK(reinterpret_cast<uintptr_t>(src) % 16 == 0, "import buffer must be contiguous 16-byte aligned uint8");
  const Store s = make_store(d);
  FP_CHECK(d->num_layers < 65536, "too many layers for one import launch");
  hipLaunchKernelGGL(blob_import_kernel, dim3((unsigned)n, (unsigned)d->num_layers), dim3(64 * kImportWaves), 0, stream, s,
                     src, src_bytes, offsets, blocks, status, arena_base, arena_stride, digest);
  FP_LAUNCH_CHECK();
  return 0;
}

extern "C" int fp_encode_records(const void* raw, int64_t n, const int32_t* kv, const uint8_t* rank_of,
                                 const int32_t* tab_idx, int64_t n_tables, uint8_t* out, int32_t* lens,
                                 fp_stream_t stream) {
  if (n == 0) return 0;
  FP_CHECK(n > 0 && n < (1LL << 31) && n_tables > 0, "bad record or table count");
  hipLaunchKernelGGL(encode_records_kernel, dim3((unsigned)n), dim3(kThreads), 0, stream,
                     static_cast<const uint16_t*>(raw), kv, rank_of, tab_idx, out, lens);
  FP_LAUNCH_CHECK();
  return 0;
}

extern "C" int fp_decode_records(const int64_t* rec_addr, const int32_t* rec_len, int64_t n, const int32_t* kv,
                                 const uint32_t* plut, const uint8_t* slut, const int32_t* tab_idx,
                                 int64_t n_tables, void* out, fp_stream_t stream) {
  if (n == 0) return 0;
  FP_CHECK(n > 0 && n < (1LL << 31) && n_tables > 0, "bad record or table count");
  if (set_dec_smem()) return -1;
  hipLaunchKernelGGL(decode_records_kernel, dim3((unsigned)n), dim3(kThreads), sizeof(DecShared), stream, rec_addr,
                     rec_len, kv, plut, slut, tab_idx, static_cast<uint8_t*>(out));
  FP_LAUNCH_CHECK();
  return 0;
}
