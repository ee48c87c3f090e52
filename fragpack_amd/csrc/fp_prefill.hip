// Causal varlen prefill attention over the paged BF16 workspace (gfx950).
//
// Reference path: the vLLM FlashAttention call of the FragPack backend
// (fragpack/integrations/vllm/backend.py:560-575, prefill groups :387-444):
// flash_attn_varlen_func(q, k = wk, v = wv, out, cu_seqlens_q, max_seqlen_q,
// seqused_k, max_seqlen_k, softmax_scale, causal=True, block_table).  The
// workspace is what HbmKvStore.gather writes: token-major BF16
// [pages, 128, H, 128]; sequence b's key j lives in page
// block_table[b][j / 128], row j % 128.  Queries are the last
// q_len = cu[b+1] - cu[b] positions of the sequence (causal mask aligned
// bottom-right: query i sees keys j <= i + seqused_k - q_len).
//
// Design (MI355X):
// * One 512-thread workgroup (8 wavefronts) per (256-row query tile, KV head).
//   The 256 rows are T = 256 / G tokens x G query heads of the KV head
//   (head-major), so every K / V tile read serves the whole GQA group and
//   eight waves.  Wave w owns rows 32w .. 32w + 31 as two 16-column MFMA
//   tiles.
// * Keys stream in 64-key tiles through double-buffered LDS, K and V both
//   key-major and loaded straight from HBM into LDS (buffer_load ... lds, no
//   registers).  K fragments are plain 16-byte reads; V^T fragments come
//   from ds_read_b64_tr_b16 transposing reads.
// * S^T = K Q^T and O^T += V^T P^T with v_mfma_f32_16x16x32_bf16.  The
//   accumulator layout of S^T (lane = query column, 4 consecutive keys per
//   16-lane group) is, after BF16 packing, exactly the B operand of the PV
//   product once the PV contraction visits keys in the matching order
//   {4q..4q+3, 16+4q..16+4q+3} -- P never leaves registers.
// * Online softmax in the log2 domain (exp2), P rounded to BF16 for PV while
//   l sums the fp32 P -- the arithmetic FlashAttention uses.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/fragpack_hip.h"
#include "fp_capi_internal.hpp"

namespace fp {
namespace {

typedef __bf16 pf_bf16x8 __attribute__((ext_vector_type(8)));
typedef float pf_f32x4 __attribute__((ext_vector_type(4)));

constexpr int kPfQt = 2;           // 16-row query tiles per wavefront
constexpr int kPfWaves = 8;        // wavefronts per workgroup
constexpr int kPfWavesPerEu = 2;
constexpr int kPfThreads = 64 * kPfWaves;
constexpr int kPfRows = 16 * kPfQt * kPfWaves;  // query rows (token x head) per workgroup
constexpr int kPfKeys = 64;        // keys per LDS tile
constexpr int kPfDim = 128;
// K and V tiles in LDS: key-major rows of 256 bytes whose 16-byte chunks
// are XOR-swizzled by the row (chunk c of row r at slot c ^ (r & 15)), so
// the fragment reads of 16 consecutive rows cover all banks.
constexpr int kKRow = 256;
constexpr int kKBytes = kPfKeys * kKRow;   // 16384 (K or V)
constexpr float kLazyMax = 8.f;  // log2 headroom of the softmax reference max

struct PrefillParams {
  const uint16_t* q;
  const uint16_t* wk;
  const uint16_t* wv;
  const int32_t* cu_q;
  const int32_t* seq_k;
  const int32_t* block_table;
  uint16_t* out;
  int64_t q_stride;    // elements between consecutive query tokens
  int64_t out_stride;  // elements between consecutive output tokens
  int64_t bt_stride;
  int64_t num_pages;
  int kvh, group, num_seqs, tiles_per_seq;
  float scale_log2;
  int causal;
};

__device__ __forceinline__ pf_f32x4 pf_mfma(const uint4& a, const uint4& b, pf_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(pf_bf16x8, a), __builtin_bit_cast(pf_bf16x8, b),
                                                  c, 0, 0, 0);
}

// Two floats -> BF16 pair (x low), round to nearest even: one v_cvt_pk_bf16_f32.
typedef float pf_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 pf_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_bf16(float x, float y) {
  const pf_f32x2 v = {x, y};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, pf_bf16x2));
}


// Butterfly partners across 16- and 32-lane halves with the gfx950 lane
// swaps (VALU, no LDS round trip): with both operands x, one result holds
// the lane's own value and the other its partner's (lane ^ 16 / lane ^ 32).
__device__ __forceinline__ float pf_xor16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pf_xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pf_xor16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pf_xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

typedef __amdgpu_buffer_rsrc_t pf_rsrc_t;
typedef __attribute__((address_space(3))) void* pf_lds_ptr_t;

// A 64-key tile lies in one 128-token page (tiles start at multiples of 64):
// rows key0 .. key0 + 63 of head h are ``kvh * 256`` bytes apart, starting
// at the tile's first row.
__device__ __forceinline__ pf_rsrc_t tile_rsrc(const uint16_t* base, int64_t page, int key0, int h, int kvh) {
  const uint16_t* first = base + ((page * 128 + (key0 & 127)) * kvh + h) * kPfDim;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(first), (short)0, 64 * kvh * kPfDim * 2,
                                           0x00020000);
}

// Loads a 64-key tile of K and of V straight into LDS (buffer_load ... lds):
// rows of 256 bytes, 16-byte chunk c of row r at slot c ^ (r & 15).  Each
// wave instruction fills 1 KB = four rows, lane L the slot L % 16 of row
// L / 16, so lane L fetches chunk (L % 16) ^ (row & 15).  Rows past the
// tile's ``nkeys`` repeat its last row: V rows stay finite (their P is 0)
// and every load stays inside the page.
__device__ __forceinline__ void load_tile(const PrefillParams& p, int64_t page, int key0, int nkeys, int h,
                                          uint8_t* kst, uint8_t* vst) {
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row = p.kvh * kPfDim * 2;  // bytes between consecutive keys
  const pf_rsrc_t rk = tile_rsrc(p.wk, page, key0, h, p.kvh);
  const pf_rsrc_t rv = tile_rsrc(p.wv, page, key0, h, p.kvh);
  constexpr int kRows = kPfKeys / kPfWaves;  // rows per wave, four per instruction
#pragma unroll
  for (int i = 0; i < kRows / 4; ++i) {
    const int r0 = kRows * w + 4 * i, r = r0 + (lane >> 4);
    const int off = min(r, nkeys - 1) * row + 16 * ((lane & 15) ^ (r & 15));
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (pf_lds_ptr_t)(kst + r0 * kKRow), 16, off, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (pf_lds_ptr_t)(vst + r0 * kKRow), 16, off, 0, 0, 0);
  }
}

typedef short pf_i16x4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16 (gfx950): within each 16-lane group, lane i receives
// element i % 4 of the 8-byte pieces addressed by lanes 4 e + i / 4,
// e = 0..3 -- a 4 x 4 transpose of 16-bit elements across lanes.
__device__ __forceinline__ uint2 lds_tr16(const uint8_t* a) {
  const pf_i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) pf_i16x4*)a);
  return __builtin_bit_cast(uint2, v);
}

__global__ void __launch_bounds__(kPfThreads) __attribute__((amdgpu_waves_per_eu(kPfWavesPerEu))) prefill_kernel(PrefillParams p) {
  // K stages are two separate LDS objects and each trip of the tile loop
  // below names them statically: the counter pass then sees that the next
  // tile's K transfer into one cannot alias this tile's reads of the other
  // (one LDS object with computed stage offsets makes every K read wait for
  // the transfer just issued).  The V stages likewise: reads of the dynamic
  // LDS block are not known to miss the K objects.
  __shared__ __align__(16) uint8_t pf_k0[kKBytes];
  __shared__ __align__(16) uint8_t pf_k1[kKBytes];
  __shared__ __align__(16) uint8_t pf_v0[kKBytes];
  __shared__ __align__(16) uint8_t pf_v1[kKBytes];
  const int h = blockIdx.y;
  // longest query tiles first: later tiles see more keys under the causal mask
  const int b = blockIdx.x % p.num_seqs;
  const int qtile = p.tiles_per_seq - 1 - (int)(blockIdx.x / p.num_seqs);
  const int q0 = p.cu_q[b], qlen = p.cu_q[b + 1] - q0;
  const int T = kPfRows / p.group;  // query tokens per tile
  const int t0 = qtile * T;
  if (t0 >= qlen) return;
  const int klen = p.seq_k[b];
  const int shift = klen - qlen;  // query i sees keys <= i + shift (causal)
  const int32_t* bt = p.block_table + (int64_t)b * p.bt_stride;

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, q4 = lane >> 4;
  // this lane's query columns (tiles qt): row -> (head g, token t)
  int tok[kPfQt], hq[kPfQt];
  bool rvalid[kPfQt];
#pragma unroll
  for (int qt = 0; qt < kPfQt; ++qt) {
    const int row = 16 * kPfQt * w + 16 * qt + j;
    const int g = row / T, t = row - g * T;
    tok[qt] = t0 + t;
    hq[qt] = h * p.group + g;
    rvalid[qt] = tok[qt] < qlen;
  }
  // Q^T fragments (B operands): lane (j, q4) holds dims 32 ks + 8 q4 .. + 7
  uint4 qf[kPfQt][4];
#pragma unroll
  for (int qt = 0; qt < kPfQt; ++qt) {
    const uint16_t* qrow = p.q + (int64_t)(q0 + (rvalid[qt] ? tok[qt] : 0)) * p.q_stride + (int64_t)hq[qt] * kPfDim;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qf[qt][ks] = rvalid[qt] ? *reinterpret_cast<const uint4*>(qrow + 32 * ks + 8 * q4) : make_uint4(0u, 0u, 0u, 0u);
  }
  // keys this tile needs: up to the last valid query's causal limit
  const int last_tok = min(t0 + T, qlen) - 1;
  const int kend = p.causal ? min(klen, last_tok + shift + 1) : klen;
  const int ntiles = (kend + kPfKeys - 1) / kPfKeys;
  // causal limit per query column
  int kmax[kPfQt];
#pragma unroll
  for (int qt = 0; qt < kPfQt; ++qt) kmax[qt] = p.causal ? min(klen, tok[qt] + shift + 1) : klen;

  float m[kPfQt], l[kPfQt];
#pragma unroll
  for (int qt = 0; qt < kPfQt; ++qt) {
    m[qt] = -INFINITY;
    l[qt] = 0.f;
  }
  pf_f32x4 o[8][kPfQt];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int qt = 0; qt < kPfQt; ++qt) o[dt][qt] = pf_f32x4{0.f, 0.f, 0.f, 0.f};

  // page ids of the tiles: lane j holds block_table entry 64 pb + j
  int pages = 0, pbase = -1;
  auto page_of = [&](int key0) -> int64_t {
    const int pi = key0 >> 7;
    if ((pi & ~63) != pbase) {
      pbase = pi & ~63;
      pages = pbase + lane < (kend + 127) / 128 ? bt[pbase + lane] : 0;
    }
    return __builtin_amdgcn_readlane(pages, pi & 63);
  };
  if (ntiles > 0) load_tile(p, page_of(0), 0, min(kPfKeys, kend), h, pf_k0, pf_v0);
  __syncthreads();
  // Nothing in flight at the loop entry (Q and the first tile have landed):
  // without this explicit wait the counter pass, merging the entry path,
  // puts a vmcnt(0) before the first MFMA of every tile, i.e. waits for the
  // next tile's loads right after issuing them.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  // V fragment lanes: row x = 4 q4 + j / 4 of each 16-row block, byte
  // 8 (j & 1) of the chunk; the chunk's slot term 16 ((j >> 1 & 1) ^ x)
  const int vx = 4 * q4 + (j >> 2);
  const int vlane = vx * kKRow + 8 * (j & 1), vsw = 16 * (((j >> 1) & 1) ^ vx);
  auto tile = [&](int it, const uint8_t* stage, uint8_t* knext, const uint8_t* vstage, uint8_t* vnext)
                  __attribute__((always_inline)) {
    const int key0 = it * kPfKeys;
    const bool more = it + 1 < ntiles;
    if (more)
      load_tile(p, page_of(key0 + kPfKeys), key0 + kPfKeys, min(kPfKeys, kend - key0 - kPfKeys), h, knext, vnext);

    // ---- S^T = K Q^T: s[kt][qt], keys key0 + 16 kt + 4 q4 + r ----
    // The tile runs in halves so that one half's exponentials overlap the
    // other half's MFMAs within the wave: keys 0..31 are scored, then keys
    // 32..63 are scored while P of keys 0..31 is formed (speculatively,
    // against the running max); P of keys 32..63 is formed while the PV
    // product of keys 0..31 runs.
    //
    // Scores stay unscaled (scale > 0 keeps the order); P = exp2(s c - m c)
    // is one FMA and one exp per score.  The reference max m only moves when
    // some column's max outgrows it by more than 2^kLazyMax (log2 domain), so
    // O and l are rescaled on few tiles -- and only then is the speculative P
    // of keys 0..31 recomputed; P <= 2^kLazyMax is exact enough in BF16 and
    // fp32.
    pf_f32x4 s[4][kPfQt];
    auto qk = [&](int kt) {
#pragma unroll
      for (int qt = 0; qt < kPfQt; ++qt) s[kt][qt] = pf_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const uint4 kf = *reinterpret_cast<const uint4*>(stage + (16 * kt + j) * kKRow + 16 * ((4 * ks + q4) ^ j));
#pragma unroll
        for (int qt = 0; qt < kPfQt; ++qt) s[kt][qt] = pf_mfma(kf, qf[qt][ks], s[kt][qt]);
      }
    };
    // causal / length mask: only on tiles that reach some column's limit
    // (a wave-uniform branch; other tiles skip the compares)
    int kmin = kmax[0];
#pragma unroll
    for (int qt = 1; qt < kPfQt; ++qt) kmin = min(kmin, kmax[qt]);
    const bool mask_tile = __ballot(key0 + kPfKeys > kmin) != 0;
    auto mask = [&](int kt) {
#pragma unroll
      for (int qt = 0; qt < kPfQt; ++qt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (key0 + 16 * kt + 4 * q4 + r >= kmax[qt]) s[kt][qt][r] = -INFINITY;
    };
    float e[4][kPfQt][4];
    auto expo = [&](int kt, int qt, float nm) {
#pragma unroll
      for (int r = 0; r < 4; ++r) e[kt][qt][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][qt][r], p.scale_log2, nm));
    };
    auto neg_m = [&](int qt) { return m[qt] == -INFINITY ? 0.f : -m[qt] * p.scale_log2; };
    qk(0);
    qk(1);
    if (mask_tile) {
      mask(0);
      mask(1);
    }
    // keys 32..63 scored in four k-steps; after each, a quarter of the
    // exponentials of keys 0..31 (pinned there: they run while the step's
    // MFMAs execute)
    {
      float nm[kPfQt];
#pragma unroll
      for (int qt = 0; qt < kPfQt; ++qt) {
        nm[qt] = neg_m(qt);
        s[2][qt] = s[3][qt] = pf_f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const uint4 k2 = *reinterpret_cast<const uint4*>(stage + (32 + j) * kKRow + 16 * ((4 * ks + q4) ^ j));
        const uint4 k3 = *reinterpret_cast<const uint4*>(stage + (48 + j) * kKRow + 16 * ((4 * ks + q4) ^ j));
#pragma unroll
        for (int qt = 0; qt < kPfQt; ++qt) {
          s[2][qt] = pf_mfma(k2, qf[qt][ks], s[2][qt]);
          s[3][qt] = pf_mfma(k3, qf[qt][ks], s[3][qt]);
        }
        // (kt, qt) pairs ks * kPerStep .. of keys 0..31 (2 kPfQt pairs over
        // the four k-steps): kt = pair / kPfQt
        constexpr int kPerStep = (2 * kPfQt + 3) / 4;
#pragma unroll
        for (int u = 0; u < kPerStep; ++u) {
          const int pr = ks * kPerStep + u, kt = pr / kPfQt, qt = pr % kPfQt;
          if (pr >= 2 * kPfQt) continue;
#pragma unroll
          for (int r = 0; r < 4; ++r)
            e[kt][qt][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][qt][r], p.scale_log2, nm[qt]));
#pragma unroll
          for (int r = 0; r < 4; ++r) asm volatile("" ::"v"(e[kt][qt][r]));  // not sunk into a later block
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (mask_tile) {
      mask(2);
      mask(3);
    }
    float mloc[kPfQt];
#pragma unroll
    for (int qt = 0; qt < kPfQt; ++qt) {
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[kt][qt][r]);
      mx = pf_xor32_max(pf_xor16_max(mx));
      mloc[qt] = mx;
    }
    bool grow = false;
#pragma unroll
    for (int qt = 0; qt < kPfQt; ++qt)
      grow |= mloc[qt] > m[qt] && (m[qt] == -INFINITY || (mloc[qt] - m[qt]) * p.scale_log2 > kLazyMax);
    if (__ballot(grow) != 0) {
#pragma unroll
      for (int qt = 0; qt < kPfQt; ++qt) {
        const float m_new = fmaxf(m[qt], mloc[qt]);
        const float alpha = m[qt] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((m[qt] - m_new) * p.scale_log2);
        m[qt] = m_new;
        l[qt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[dt][qt] *= alpha;
        const float nm = neg_m(qt);
        expo(0, qt, nm);
        expo(1, qt, nm);
      }
    }
    // B operand of k-step kk: keys 32 kk + {4 q4 .. 4 q4 + 3} (tile 2 kk) and
    // 32 kk + 16 + {4 q4 ..} (tile 2 kk + 1)
    auto pfrag = [&](int kk, int qt) {
      return make_uint4(pk_bf16(e[2 * kk][qt][0], e[2 * kk][qt][1]), pk_bf16(e[2 * kk][qt][2], e[2 * kk][qt][3]),
                        pk_bf16(e[2 * kk + 1][qt][0], e[2 * kk + 1][qt][1]),
                        pk_bf16(e[2 * kk + 1][qt][2], e[2 * kk + 1][qt][3]));
    };
    uint4 p0[kPfQt];
#pragma unroll
    for (int qt = 0; qt < kPfQt; ++qt) p0[qt] = pfrag(0, qt);
#pragma unroll
    for (int qt = 0; qt < kPfQt; ++qt) {
      const float nm = neg_m(qt);
      expo(2, qt, nm);
      expo(3, qt, nm);
    }
    // ---- O^T += V^T P^T: o[dt][qt], dims 16 dt + 4 q4 + r ----
    // V^T fragment (dims 16 dt + j, keys 32 kk + {4 q4 .. 4 q4 + 3} and
    // 32 kk + 16 + {4 q4 ..}) by two transposing reads: lane (s = j, g = q4)
    // addresses row 32 kk (+ 16) + 4 g + s / 4, dims 16 dt + 4 (s % 4) ..,
    // so lane j receives dim 16 dt + j of rows 32 kk (+ 16) + 4 g + e.
    auto pv = [&](int kk, const uint4 (&pa)[kPfQt]) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        // chunk 2 dt + (j >> 1 & 1) of row x = 4 q4 + j / 4 (mod 16) sits at
        // slot chunk ^ x
        const uint8_t* base = vstage + (vsw ^ (32 * dt)) + vlane;
        const uint2 lo = lds_tr16(base + 32 * kk * kKRow);
        const uint2 hi = lds_tr16(base + (32 * kk + 16) * kKRow);
        const uint4 vf = make_uint4(lo.x, lo.y, hi.x, hi.y);
#pragma unroll
        for (int qt = 0; qt < kPfQt; ++qt) o[dt][qt] = pf_mfma(vf, pa[qt], o[dt][qt]);
      }
    };
    pv(0, p0);
    {
      uint4 p1[kPfQt];
#pragma unroll
      for (int qt = 0; qt < kPfQt; ++qt) p1[qt] = pfrag(1, qt);
      pv(1, p1);
    }
#pragma unroll
    for (int qt = 0; qt < kPfQt; ++qt) {
      float psum = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) psum += e[kt][qt][r];
      l[qt] += psum;
    }
    __syncthreads();
  };
  for (int it = 0; it < ntiles; it += 2) {
    tile(it, pf_k0, pf_k1, pf_v0, pf_v1);
    if (it + 1 < ntiles) tile(it + 1, pf_k1, pf_k0, pf_v1, pf_v0);
  }
  // ---- normalise and store: lane holds dims 16 dt + 4 q4 + r of query j ----
#pragma unroll
  for (int qt = 0; qt < kPfQt; ++qt) {
    float lt = l[qt];
    lt = pf_xor32_sum(pf_xor16_sum(lt));
    if (!rvalid[qt]) continue;
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    uint16_t* orow = p.out + (int64_t)(q0 + tok[qt]) * p.out_stride + (int64_t)hq[qt] * kPfDim;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      *reinterpret_cast<uint2*>(orow + 16 * dt + 4 * q4) =
          make_uint2(pk_bf16(o[dt][qt][0] * inv, o[dt][qt][1] * inv), pk_bf16(o[dt][qt][2] * inv, o[dt][qt][3] * inv));
  }
}

}  // namespace
}  // namespace fp

using namespace fp;

extern "C" int fp_prefill_attention(const void* q, int64_t q_stride, const void* wk, const void* wv, int64_t num_pages,
                                    int64_t kv_heads, int64_t group, const int32_t* cu_seqlens_q,
                                    const int32_t* seqused_k, const int32_t* block_table, int64_t bt_stride,
                                    int64_t num_seqs, int64_t max_seqlen_q, int64_t max_seqlen_k, double scale,
                                    int causal, void* out, int64_t out_stride, fp_stream_t stream) {
  FP_CHECK(num_seqs >= 0 && max_seqlen_q >= 0 && max_seqlen_k >= 0, "negative sizes");
  if (num_seqs == 0 || max_seqlen_q == 0) return 0;
  FP_CHECK(group == 1 || group == 2 || group == 4 || group == 8, "query heads per KV head must be 1, 2, 4 or 8");
  FP_CHECK(kv_heads >= 1 && kv_heads <= 65535, "kv_heads out of range");
  FP_CHECK(q && wk && wv && cu_seqlens_q && seqused_k && block_table && out, "null pointer");
  FP_CHECK(q_stride >= kv_heads * group * kPfDim && out_stride >= kv_heads * group * kPfDim,
           "token strides must cover all query heads");
  FP_CHECK(bt_stride >= (max_seqlen_k + 127) / 128, "block table narrower than max_seqlen_k");
  FP_CHECK(((uintptr_t)q | (uintptr_t)out | (uintptr_t)wk | (uintptr_t)wv) % 16 == 0 && q_stride % 8 == 0 &&
               out_stride % 8 == 0,
           "q / out / workspace must be 16-byte aligned with 8-element token strides");
  const int64_t rows_per_tile = kPfRows / group;
  const int64_t tiles = (max_seqlen_q + rows_per_tile - 1) / rows_per_tile;
  FP_CHECK(tiles * num_seqs < (1LL << 31), "grid too large");
  PrefillParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.wk = static_cast<const uint16_t*>(wk);
  p.wv = static_cast<const uint16_t*>(wv);
  p.cu_q = cu_seqlens_q;
  p.seq_k = seqused_k;
  p.block_table = block_table;
  p.out = static_cast<uint16_t*>(out);
  p.q_stride = q_stride;
  p.out_stride = out_stride;
  p.bt_stride = bt_stride;
  p.num_pages = num_pages;
  p.kvh = (int)kv_heads;
  p.group = (int)group;
  p.num_seqs = (int)num_seqs;
  p.tiles_per_seq = (int)tiles;
  p.scale_log2 = (float)(scale * 1.4426950408889634);
  p.causal = causal ? 1 : 0;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // all LDS is static (two K and two V stages, 64 KB)
  hipLaunchKernelGGL(prefill_kernel, dim3((unsigned)(tiles * num_seqs), (unsigned)kv_heads), dim3(kPfThreads), 0, s, p);
  FP_LAUNCH_CHECK();
  return 0;
}
