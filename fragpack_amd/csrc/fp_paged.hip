// Split-KV decode attention over a plain paged BF16 KV cache (gfx950): the
// uncompressed baseline the FragPack decode kernel is measured against.
//
// Reference counterpart: the FA3 arm of the reference's step benchmark
// (benchmarks/fragpack_step_bench.py:205-284: flash_attn_with_kvcache over a
// token-major paged BF16 cache [blocks, 128, H, 128]).  Same cache layout
// and arguments (q, paged K / V, block table, sequence lengths, scale).
//
// Design (MI355X):
// * Workgroup (c, h, b) = split c of sequence b's pages for KV head h; the
//   host picks ``splits`` so that B x H x splits is about one workgroup per
//   CU, and each split covers ``ppc`` consecutive pages.
// * Four wavefronts, each its own stream with its own online softmax: wave
//   w takes keys 32 w .. 32 w + 31 of every page, so no barrier runs inside
//   the page loop.  Its K rows go straight into registers as MFMA A operands
//   (16-byte loads: key row j, dims 32 ks + 8 q4 ..), its V rows into
//   wave-private LDS (buffer_load ... lds, 16-byte chunks XOR-swizzled by
//   row) and come back as V^T operands through ds_read_b64_tr_b16; the next
//   page's K and V are in flight while this page is computed.
// * S^T = K Q^T and O^T += V^T P^T with v_mfma_f32_16x16x32_bf16, query
//   heads in the N columns; the S^T accumulator is, packed to BF16, the B
//   operand of the PV product (keys visited in the order {4 q4 ..} and
//   {16 + 4 q4 ..}), so P stays in registers.  Softmax in the log2 domain
//   with a lazily moved reference max; P rounded to BF16 for PV, l summed in
//   fp32 -- the arithmetic of FlashAttention.
// * The four waves combine through LDS; splits combine through fp32
//   partials written to the device coherence point, the last workgroup of a
//   (sequence, head) merging them (a per-(b, h) counter, left at zero).
// * Rows past a sequence's length repeat its last valid row (the cache may
//   hold anything there), and their scores are masked.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <algorithm>

#include "../../include/fragpack_hip.h"
#include "fp_capi_internal.hpp"
#include "fp_record.hpp"

namespace fp {
namespace {

typedef __bf16 pg_bf16x8 __attribute__((ext_vector_type(8)));
typedef float pg_f32x4 __attribute__((ext_vector_type(4)));
typedef short pg_i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* pg_lds_ptr_t;

constexpr int kPgWaves = 4;
constexpr int kPgThreads = 64 * kPgWaves;
constexpr int kPgPerCu = 2;          // resident workgroups per CU (64 KB of V stages each)
constexpr int kPgRow = 256;          // bytes of one key row of one head
constexpr int kPgWaveKeys = 32;      // keys per wave per page
constexpr int kPgStage = kPgWaveKeys * kPgRow;  // 8 KB: one wave's V rows of one page
constexpr float kPgLazy = 8.f;       // log2 headroom of the reference max
// s_waitcnt immediates (gfx9 layout: vmcnt bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8; the other counters left unconstrained)
constexpr int kVmcnt0 = 0x0F70;
constexpr int kVmcnt16 = 0x4F70;

struct PagedParams {
  const uint16_t* q;
  const uint16_t* kc;
  const uint16_t* vc;
  const int32_t* block_table;
  const int32_t* seq_lens;
  float* opart;   // [B, H, splits, 8, 128]
  float* ml;      // [B, H, splits, 8, 2]
  int32_t* done;  // [B, H] merge counters (zero between launches)
  uint16_t* out;
  int64_t q_stride, out_stride, bt_stride;
  int64_t num_blocks;  // pages in the caches: block ids outside [0, num_blocks) are skipped
  int kvh, group, splits, ppc;
  int cus;  // compute units of the device
  float scale_log2;
};

__device__ __forceinline__ pg_f32x4 pg_mfma(const uint4& a, const uint4& b, pg_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(pg_bf16x8, a), __builtin_bit_cast(pg_bf16x8, b),
                                                  c, 0, 0, 0);
}

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element
// i % 4 of the 8-byte pieces addressed by lanes 4 e + i / 4, e = 0..3.
__device__ __forceinline__ uint2 pg_tr16(const uint8_t* a) {
  const pg_i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) pg_i16x4*)a);
  return __builtin_bit_cast(uint2, v);
}

// One wave's share of a page: K fragments in registers, V rows on their way
// into the wave's LDS stage.  Rows past ``valid`` keys of the page repeat row
// valid - 1.
struct KFrag {
  uint4 k[2][4];  // [16-key tile][k-step]: key 16 t + j, dims 32 ks + 8 q4 .. + 7
};

// Pages are streamed with the non-temporal load policy, as the compressed
// kernel streams its records.  A block id outside the caches reads as an empty page (zero-sized
// resources: every load returns zero) and the caller masks all its keys;
// returns whether the page is inside.
template <int kPolicy>
__device__ __forceinline__ bool load_page(const PagedParams& p, int64_t blk, int h, int w, int valid, int lane,
                                          KFrag& kf, uint8_t* vstage) {
  const int j = lane & 15, q4 = lane >> 4;
  const int row = p.kvh * kPgRow;  // bytes between consecutive keys of one head
  const bool inside = blk >= 0 && blk < p.num_blocks;
  if (!inside) blk = 0;
  const uint8_t* kpage = reinterpret_cast<const uint8_t*>(p.kc) + (blk * 128 * p.kvh + h) * kPgRow;
  const uint8_t* vpage = reinterpret_cast<const uint8_t*>(p.vc) + (blk * 128 * p.kvh + h) * kPgRow;
  const rsrc_t rk = make_rsrc(kpage, inside ? 128 * row : 0);
  const rsrc_t rv = make_rsrc(vpage, inside ? 128 * row : 0);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int key = min(kPgWaveKeys * w + 16 * t + j, valid - 1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rk, key * row + 64 * ks + 16 * q4, 0, kPolicy);
      kf.k[t][ks] = make_uint4(v.x, v.y, v.z, v.w);
    }
  }
  // V: each instruction fills 1 KB of the stage (four rows), lane L slot L % 16
  // of row L / 16, i.e. chunk (L % 16) ^ (row & 15)
#pragma unroll
  for (int i = 0; i < kPgWaveKeys / 4; ++i) {
    const int r = 4 * i + (lane >> 4);
    const int key = min(kPgWaveKeys * w + r, valid - 1);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (pg_lds_ptr_t)(vstage + 4 * i * kPgRow), 16,
                                             key * row + 16 * ((lane & 15) ^ (r & 15)), 0, 0, kPolicy);
  }
  return inside;
}

struct WaveState {
  float m, l;          // reference max (score units) and row sum of this lane's query column
  pg_f32x4 o[8];       // O^T: dims 16 dt + 4 q4 + r of query column j
};

// One page for one wave: scores of its 32 keys, softmax update, PV.
__device__ __forceinline__ void page_step(const PagedParams& p, const uint4 (&qf)[4], const KFrag& kf,
                                          const uint8_t* vstage, int key0, int len, int lane, WaveState& st) {
  const int j = lane & 15, q4 = lane >> 4;
  pg_f32x4 s[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    s[t] = pg_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) s[t] = pg_mfma(kf.k[t][ks], qf[ks], s[t]);
  }
  // keys key0 + 16 t + 4 q4 + r
  if (key0 + kPgWaveKeys > len) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (key0 + 16 * t + 4 * q4 + r >= len) s[t][r] = -INFINITY;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[t][r]);
  mx = xor32_max(xor16_max(mx));
  const bool grow = mx > st.m && (st.m == -INFINITY || (mx - st.m) * p.scale_log2 > kPgLazy);
  if (__ballot(grow) != 0) {
    const float m_new = fmaxf(st.m, mx);
    const float alpha = st.m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((st.m - m_new) * p.scale_log2);
    st.m = m_new;
    st.l *= alpha;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) st.o[dt] *= alpha;
  }
  const float nm = st.m == -INFINITY ? 0.f : -st.m * p.scale_log2;
  float e[2][4], psum = 0.f;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      e[t][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][r], p.scale_log2, nm));
      psum += e[t][r];
    }
  st.l += psum;
  const uint4 pf = make_uint4(pack_bf16x2(e[0][0], e[0][1]), pack_bf16x2(e[0][2], e[0][3]),
                              pack_bf16x2(e[1][0], e[1][1]), pack_bf16x2(e[1][2], e[1][3]));
  // V^T fragment (dims 16 dt + j, keys {4 q4 ..} and {16 + 4 q4 ..}): lane
  // (j, q4) addresses row x = 4 q4 + j / 4 (+ 16), dims 16 dt + 4 (j % 4) ..;
  // that chunk 2 dt + (j >> 1 & 1) of row x sits at slot chunk ^ (x & 15)
  const int x = 4 * q4 + (j >> 2);
  const uint8_t* base = vstage + x * kPgRow + 8 * (j & 1);
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    const int slot = 16 * (((2 * dt) | ((j >> 1) & 1)) ^ x);
    const uint2 lo = pg_tr16(base + slot);
    const uint2 hi = pg_tr16(base + 16 * kPgRow + slot);
    st.o[dt] = pg_mfma(make_uint4(lo.x, lo.y, hi.x, hi.y), pf, st.o[dt]);
  }
}

struct CombineShared {
  float o[kPgWaves][8][128];
  float m[kPgWaves][8], l[kPgWaves][8];
  int last;
};
static_assert(sizeof(CombineShared) <= kPgWaves * kPgStage, "combine reuses the first V stage");

constexpr int kPgMergeBatch = 16;

template <int kPolicy>
__global__ void __launch_bounds__(kPgThreads) __attribute__((amdgpu_waves_per_eu(kPgPerCu)))
paged_decode_kernel(PagedParams p) {
  // The two V stages are separate LDS objects, named statically in the
  // page loop, so the compiler's wait for the transfer into one stage never
  // covers reads of the other.
  __shared__ __align__(16) uint8_t stage0[kPgWaves][kPgStage];
  __shared__ __align__(16) uint8_t stage1[kPgWaves][kPgStage];
  CombineShared& cs = *reinterpret_cast<CombineShared*>(&stage0[0][0]);
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, q4 = lane >> 4;
  // pages past the block table's width are not read (a length beyond it is
  // cut to the table)
  const int n_pages = min((p.seq_lens[b] + 127) >> 7, (int)p.bt_stride);
  const int len = min(p.seq_lens[b], 128 * n_pages);
  const int pg0 = c * p.ppc, pg1 = min(n_pages, pg0 + p.ppc);
  const int32_t* bt = p.block_table + (int64_t)b * p.bt_stride;

  // Q^T fragments: lane (j, q4) holds head j's dims 32 ks + 8 q4 .. + 7 (zero past the group)
  uint4 qf[4];
  {
    const rsrc_t rq = make_rsrc(p.q + (int64_t)b * p.q_stride + (int64_t)h * p.group * kDim, p.group * kDim * 2);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[ks] = bld16(rq, j * 256 + 64 * ks + 16 * q4, 0);
  }
  WaveState st;
  st.m = -INFINITY;
  st.l = 0.f;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) st.o[dt] = pg_f32x4{0.f, 0.f, 0.f, 0.f};

  if (pg0 < pg1) {
    // workgroups L and L + cus (linear id L) share a CU, the older issuing
    // first at equal priority: the priority rotates with the page pair,
    // offset by the dispatch round, so the two progress evenly
    const int age = (int)(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z)) / max(1, p.cus);
    KFrag ka, kb;
    auto valid_of = [&](int pg) { return min(128, len - pg * 128); };
    bool in_a = load_page<kPolicy>(p, bt[pg0], h, w, valid_of(pg0), lane, ka, stage0[w]), in_b = false;
    // two pages per trip so that each stage and fragment set is named statically
    for (int pg = pg0; pg < pg1; pg += 2) {
      rotate_priority((pg >> 1) + age);
      if (pg + 1 < pg1) in_b = load_page<kPolicy>(p, bt[pg + 1], h, w, valid_of(pg + 1), lane, kb, stage1[w]);
      // page pg landed: only the next page's 16 transfers may still be in flight
      if (pg + 1 < pg1)
        __builtin_amdgcn_s_waitcnt(kVmcnt16);
      else
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
      page_step(p, qf, ka, stage0[w], pg * 128 + kPgWaveKeys * w, in_a ? len : 0, lane, st);
      if (pg + 1 >= pg1) break;
      if (pg + 2 < pg1) in_a = load_page<kPolicy>(p, bt[pg + 2], h, w, valid_of(pg + 2), lane, ka, stage0[w]);
      if (pg + 2 < pg1)
        __builtin_amdgcn_s_waitcnt(kVmcnt16);
      else
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
      page_step(p, qf, kb, stage1[w], (pg + 1) * 128 + kPgWaveKeys * w, in_b ? len : 0, lane, st);
    }
  }
  // ---- combine the four waves: thread t -> query head g = t / 32, dims 4 (t % 32) .. ----
  float lt = xor32_sum(xor16_sum(st.l));
  __syncthreads();  // every wave is done with the V stages
  if (j < 8) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      *reinterpret_cast<float4*>(&cs.o[w][j][16 * dt + 4 * q4]) =
          make_float4(st.o[dt][0], st.o[dt][1], st.o[dt][2], st.o[dt][3]);
    if (q4 == 0) {
      cs.m[w][j] = st.m == -INFINITY ? -INFINITY : st.m * p.scale_log2;
      cs.l[w][j] = lt;
    }
  }
  __syncthreads();
  const int t = threadIdx.x, g = t >> 5, d = 4 * (t & 31);
  float M = -INFINITY;
#pragma unroll
  for (int v = 0; v < kPgWaves; ++v) M = fmaxf(M, cs.m[v][g]);
  float L = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (M != -INFINITY) {
#pragma unroll
    for (int v = 0; v < kPgWaves; ++v) {
      const float a = __builtin_amdgcn_exp2f(cs.m[v][g] - M);
      const float4 ov = *reinterpret_cast<const float4*>(&cs.o[v][g][d]);
      L += a * cs.l[v][g];
      acc.x += a * ov.x;
      acc.y += a * ov.y;
      acc.z += a * ov.z;
      acc.w += a * ov.w;
    }
  }
  uint16_t* orow = p.out + (int64_t)b * p.out_stride + (int64_t)(h * p.group + g) * kDim + d;
  if (p.splits == 1) {
    if (g < p.group) {
      const float inv = L > 0.f ? 1.f / L : 0.f;
      *reinterpret_cast<uint2*>(orow) =
          make_uint2(pack_bf16x2(acc.x * inv, acc.y * inv), pack_bf16x2(acc.z * inv, acc.w * inv));
    }
    return;
  }
  // ---- split-KV: partial to the coherence point, the last split merges ----
  const int64_t bh = (int64_t)b * p.kvh + h;
  const rsrc_t ro = coh_rsrc(p.opart), rm = coh_rsrc(p.ml);
  const int64_t row = (bh * p.splits + c) * 8 + g;
  st_coh4(ro, row * kDim + d, acc.x, acc.y, acc.z, acc.w);
  if ((t & 31) == 0) st_coh2(rm, row * 2, M, L);
  wait_stores();
  __syncthreads();
  if (t == 0) {
    int32_t* cnt = p.done + bh;
    const int last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == p.splits - 1;
    if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    cs.last = last;
  }
  __syncthreads();
  if (!cs.last || g >= p.group) return;
  const int64_t row0 = bh * p.splits * 8 + g;
  float gm = -INFINITY, gl = 0.f;
  float4 go = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int k0 = 0; k0 < p.splits; k0 += kPgMergeBatch) {
    float2 ms[kPgMergeBatch];
    float4 ov[kPgMergeBatch];
#pragma unroll
    for (int k = 0; k < kPgMergeBatch; ++k)
      if (k0 + k < p.splits) {
        const int64_t r = row0 + (int64_t)(k0 + k) * 8;
        ms[k] = ld_coh2(rm, r * 2);
        ov[k] = ld_coh4(ro, r * kDim + d);
      }
    float bm = -INFINITY;
#pragma unroll
    for (int k = 0; k < kPgMergeBatch; ++k)
      if (k0 + k < p.splits) bm = fmaxf(bm, ms[k].x);
    const float nmax = fmaxf(gm, bm);
    if (nmax == -INFINITY) continue;
    const float a = __builtin_amdgcn_exp2f(gm - nmax);
    gl *= a;
    go.x *= a;
    go.y *= a;
    go.z *= a;
    go.w *= a;
#pragma unroll
    for (int k = 0; k < kPgMergeBatch; ++k)
      if (k0 + k < p.splits) {
        const float wgt = __builtin_amdgcn_exp2f(ms[k].x - nmax);
        gl += wgt * ms[k].y;
        go.x += wgt * ov[k].x;
        go.y += wgt * ov[k].y;
        go.z += wgt * ov[k].z;
        go.w += wgt * ov[k].w;
      }
    gm = nmax;
  }
  const float inv = gl > 0.f ? 1.f / gl : 0.f;
  *reinterpret_cast<uint2*>(orow) = make_uint2(pack_bf16x2(go.x * inv, go.y * inv), pack_bf16x2(go.z * inv, go.w * inv));
}

}  // namespace
}  // namespace fp

using namespace fp;

// Load policy of the paged kernel's K and V page loads: non-temporal
// (default) or plain.  Which is faster depends on the shape (measured: the
// non-temporal policy is faster at batch 4 x 8K, slower at 16 x 32 heads
// ragged), so a baseline measurement tries both.  Process-wide; not for
// concurrent callers.
static int g_paged_streaming = 1;

extern "C" int fp_paged_set_streaming(int on) {
  g_paged_streaming = on ? 1 : 0;
  return 0;
}

extern "C" int fp_paged_decode_splits(int64_t batch, int64_t kv_heads, int64_t max_seq_len) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus = 256;
  const int64_t pages = std::max<int64_t>(1, (max_seq_len + 127) / 128);
  // one workgroup per CU: more splits than that lose more to the merge of
  // their partials than they gain in parallel pages (measured at B4 x H4 x
  // 8K: 16 splits 17.7 us, 32 splits 22.4 us)
  const int64_t slots = cus;
  const int64_t want = std::max<int64_t>(1, (slots + batch * kv_heads - 1) / std::max<int64_t>(1, batch * kv_heads));
  const int64_t ppc = (pages + std::min(want, pages) - 1) / std::min(want, pages);
  return (int)((pages + ppc - 1) / ppc);
}

extern "C" int fp_paged_decode(const void* q, int64_t q_stride, int64_t batch, int64_t kv_heads, int64_t group,
                               const void* k_cache, const void* v_cache, int64_t num_blocks,
                               const int32_t* block_table, int64_t bt_stride, const int32_t* seq_lens,
                               int64_t max_seq_len, int64_t splits, float* opart, int64_t opart_elems, float* ml,
                               int64_t ml_elems, int32_t* counters, int64_t counter_elems, void* out,
                               int64_t out_stride, double scale, fp_stream_t stream) {
  FP_CHECK(batch >= 0 && kv_heads > 0 && kv_heads <= 1024 && num_blocks > 0, "bad batch / kv_heads / cache size");
  FP_CHECK(group == 1 || group == 2 || group == 4 || group == 8, "query heads per KV head must be 1, 2, 4 or 8");
  FP_CHECK(scale > 0 && max_seq_len >= 0, "scale must be positive and max_seq_len non-negative");
  if (batch == 0) return 0;
  FP_CHECK(batch < 65536, "batch too large");
  FP_CHECK(q && k_cache && v_cache && block_table && seq_lens && out, "null pointer");
  FP_CHECK(((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 == 0 && q_stride % 8 == 0 &&
               q_stride >= kv_heads * group * kDim,
           "q and the caches must be 16-byte aligned, q rows cover every head");
  FP_CHECK((uintptr_t)out % 8 == 0 && out_stride % 4 == 0 && out_stride >= kv_heads * group * kDim,
           "out rows must be 8-byte aligned and cover every head");
  const int64_t pages = std::max<int64_t>(1, (max_seq_len + 127) / 128);
  FP_CHECK(splits >= 1 && splits <= pages, "splits must be in [1, pages of max_seq_len]");
  FP_CHECK(bt_stride >= pages, "block table narrower than max_seq_len");
  const int64_t rows = batch * kv_heads * splits * 8;
  if (splits > 1) {
    FP_CHECK(opart && ml && counters && opart_elems >= rows * kDim && ml_elems >= rows * 2 &&
                 counter_elems >= batch * kv_heads,
             "split workspace too small (opart B*H*splits*8*128, ml B*H*splits*16, counters B*H, zeroed)");
    FP_CHECK(rows * kDim * 4 < (1LL << 31), "split workspace must stay below 2 GiB");
  }
  PagedParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.kc = static_cast<const uint16_t*>(k_cache);
  p.vc = static_cast<const uint16_t*>(v_cache);
  p.block_table = block_table;
  p.seq_lens = seq_lens;
  p.opart = opart;
  p.ml = ml;
  p.done = counters;
  p.out = static_cast<uint16_t*>(out);
  p.q_stride = q_stride;
  p.out_stride = out_stride;
  p.bt_stride = bt_stride;
  p.num_blocks = num_blocks;
  p.kvh = (int)kv_heads;
  p.group = (int)group;
  p.splits = (int)splits;
  p.ppc = (int)((pages + splits - 1) / splits);
  p.scale_log2 = (float)(scale * 1.4426950408889634);
  p.cus = device_cus();
  const dim3 grid((unsigned)splits, (unsigned)kv_heads, (unsigned)batch);
  if (g_paged_streaming)
    hipLaunchKernelGGL(paged_decode_kernel<kNt>, grid, dim3(kPgThreads), 0, reinterpret_cast<hipStream_t>(stream), p);
  else
    hipLaunchKernelGGL(paged_decode_kernel<0>, grid, dim3(kPgThreads), 0, reinterpret_cast<hipStream_t>(stream), p);
  FP_LAUNCH_CHECK();
  return 0;
}
