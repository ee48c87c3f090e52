// Split-KV decode attention straight from FragPack records (gfx950).
//
// Reference path: fragpack/ops/fused_attn_decode.cu (plan_decode :94-163,
// decode_attn :214-404, combine :407-425, host fused_decode :429-478) and the
// Python contract fragpack/ops/fused_attn_decode.py:41-219.
//
// Design (MI355X):
// * One work unit = one wavefront (64 lanes).  It walks a chunk of pages of
//   one (sequence, KV head) with an online softmax; four independent
//   wavefronts share a 256-thread workgroup and never synchronise with each
//   other.  No block-level barrier appears in the page loop.
// * Per page the wave decodes each record in four passes ("slabs" of 64
//   kernel-order threads).  Lane l decodes kernel-order thread
//   nt = 32 hh + 4 g + c of the slab, with c = l >> 4, hh = (l >> 3) & 1,
//   g = l & 7.  With that assignment the decoded words are directly the A
//   operands of v_mfma_f32_16x16x32_bf16: MFMA row = l % 16 indexes the token
//   (K) or dim (V), and the four 16-lane groups (= c) hold four disjoint dim
//   (K) or token (V) sets, so no cross-lane shuffle of KV data is needed.
// * S^T = K Q^T and O^T += V^T P^T, with the GQA heads in the MFMA N=16
//   columns (heads >= G are zero).  Softmax reductions are two cross-row
//   lane exchanges per page; P goes through 2 KB of wave-private LDS.
// * Escape bytes of a slab are expanded once into wave-private LDS; each lane
//   finds its escapes with a kernel-order prefix scan across the wave.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/fragpack_hip.h"
#include "fp_capi_internal.hpp"
#include "fp_record.hpp"

namespace fp {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;  // independent wavefronts per workgroup
constexpr int kTileBytes = 8 * 4 * 4 * 16;  // Q / P fragment tile: [head 8][a 4][c 4] x 16 B
constexpr int kWaveLds = kEscLds + kVarCap + 2 * kTileBytes;  // escapes, variable region, P, Q
constexpr int kPlanThreads = 256;

struct AttnParams {
  const uint16_t* q;
  const int64_t* rec_addr;
  const int32_t* rec_len;
  const uint32_t* plut;
  const uint8_t* slut;
  const int32_t* block_table;
  const int32_t* seq_lens;
  const int32_t* plan;
  float* opart;
  float* ml;
  int64_t q_stride;   // BF16 elements between sequences
  int64_t bt_stride;  // entries between block-table rows
  int kvh, group, units;
  float scale_log2;
};

__device__ __forceinline__ int pages_of(const int32_t* seq_lens, int b) { return (seq_lens[b] + 127) >> 7; }

__device__ __forceinline__ int chunks_of(int pages, int ppc) { return (pages + ppc - 1) / ppc; }

template <bool kMax>
__device__ __forceinline__ int block_reduce(int v, int* sh) {
#pragma unroll
  for (int o = 32; o; o >>= 1) {
    const int x = __shfl_xor(v, o, 64);
    v = kMax ? max(v, x) : v + x;
  }
  __syncthreads();
  if (wave_lane() == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  v = sh[0];
#pragma unroll
  for (int w = 1; w < kPlanThreads / 64; ++w) v = kMax ? max(v, sh[w]) : v + sh[w];
  return v;
}

// Work plan, one workgroup.  Same policy and layout as the reference planner
// (fused_attn_decode.cu:48-163): every sequence is cut into chunks of ``ppc``
// pages, ``ppc`` the smallest for which the live rows fit ``budget`` units;
// plan = [ppc, budget, (seq, first page) x units, (first unit, chunks) x B].
__global__ void __launch_bounds__(kPlanThreads) plan_kernel(const int32_t* seq_lens, int32_t* plan, int batch,
                                                            int units) {
  __shared__ int sh[kPlanThreads / 64];
  __shared__ int wtot[kPlanThreads / 64];
  const int tid = threadIdx.x;
  int total = 0, longest = 0, active = 0;
  for (int b = tid; b < batch; b += kPlanThreads) {
    const int n = pages_of(seq_lens, b);
    total += n;
    longest = max(longest, n);
    active += n > 0;
  }
  total = block_reduce<false>(total, sh);
  longest = block_reduce<true>(longest, sh);
  active = block_reduce<false>(active, sh);
  const int capacity = max(1, units - batch + active);
  const int wave = units - batch + 1;
  int budget = min(capacity, max(active, wave));
  if (capacity > budget) {
    const int tail_bound = 2 * max(1, (total + budget - 1) / budget);
    int c = 0;
    for (int b = tid; b < batch; b += kPlanThreads) c += chunks_of(pages_of(seq_lens, b), tail_bound);
    if (block_reduce<false>(c, sh) > budget) budget = capacity;
  }
  int lo = max(1, (total + budget - 1) / budget), hi = max(1, longest);
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    int c = 0;
    for (int b = tid; b < batch; b += kPlanThreads) c += chunks_of(pages_of(seq_lens, b), mid);
    if (block_reduce<false>(c, sh) <= budget)
      hi = mid;
    else
      lo = mid + 1;
  }
  const int ppc = lo;
  int32_t* seq_plan = plan + 2 + 2 * units;
  int used = 0;
  for (int base = 0; base < batch; base += kPlanThreads) {
    const int b = base + tid;
    const int c = b < batch ? chunks_of(pages_of(seq_lens, b), ppc) : 0;
    // block exclusive scan of c
    const int incl = wave_incl_scan(c);
    __syncthreads();
    if (wave_lane() == 63) wtot[tid >> 6] = incl;
    __syncthreads();
    int first = incl - c, tile = 0;
    for (int w = 0; w < kPlanThreads / 64; ++w) {
      if (w < (tid >> 6)) first += wtot[w];
      tile += wtot[w];
    }
    first += used;
    if (b < batch) {
      seq_plan[2 * b] = first;
      seq_plan[2 * b + 1] = c;
      for (int s = 0; s < c; ++s) {
        plan[2 + 2 * (first + s)] = b;
        plan[3 + 2 * (first + s)] = s * ppc;
      }
    }
    used += tile;
  }
  for (int u = used + tid; u < units; u += kPlanThreads) plan[2 + 2 * u] = -1;
  if (tid == 0) {
    plan[0] = ppc;
    plan[1] = budget;
  }
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

// Ends a slab step: nothing is scheduled across it, so exactly one slab of
// loads is in flight while the previous slab is decoded.
__device__ __forceinline__ void slab_fence() {
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Lane of the natural (kernel-order) thread ``nt`` of a slab.
__device__ __forceinline__ int lane_of_natural(int nt) { return 16 * (nt & 3) + 8 * (nt >> 5) + ((nt >> 2) & 7); }

// A record as the wave sees it (wave-uniform values).
struct RecRef {
  rsrc_t rs;
  int vlen;  // bytes past the dense part; > kVarCap marks a raw record
};

__device__ __forceinline__ RecRef rec_ref(const AttnParams& p, int64_t blk, int kv, int h) {
  const int64_t idx = (blk * 2 + kv) * p.kvh + h;
  RecRef r;
  r.rs = make_rsrc(reinterpret_cast<const uint8_t*>(uniform64(p.rec_addr[idx])), kRawRecord);
  r.vlen = uniform(p.rec_len[idx]);
  return r;
}

// The first 32 bytes per lane of a coded record's variable region, loaded
// with the record's first slab.
struct VarPref {
  uint4 v0, v1;
};

template <int SLAB>
__device__ __forceinline__ void prefetch(const RecRef& r, int nt, int lane, SlabBuf& b, VarPref& vp) {
  const bool raw = r.vlen > kVarCap;
  load_slab(r.rs, raw, SLAB, nt, b);
  if constexpr (SLAB == 0) {
    // Bytes past the record (a short variable region) read as zero.
    if (!raw) {
      vp.v0 = bld16(r.rs, 16 * lane, kDenseBytes);
      vp.v1 = r.vlen > 1024 ? bld16(r.rs, 16 * lane, kDenseBytes + 1024) : make_uint4(0u, 0u, 0u, 0u);
    }
  }
}

// Decodes this lane's kernel-order thread ``nt`` of slab SLAB of record ``r``
// from prefetched data and calls pair(a, word 2a, word 2a + 1), a = 0..3.
// ``var`` is the wave's LDS copy of the record's variable region (written
// here at slab 0), ``esc`` its escape-byte area.
template <int SLAB, typename Pair>
__device__ __forceinline__ void decode_slab(const RecRef& r, const SlabBuf& b, const VarPref& vp, int nt, int lane,
                                            const HeadLut& lut, uint8_t* var, uint8_t* esc, Pair&& pair) {
  uint4 prev;
  auto emit = [&](auto st_c, const uint4& wd) {
    constexpr int st = decltype(st_c)::value;
    if constexpr (st & 1)
      pair(std::integral_constant<int, (st >> 1)>{}, prev, wd);
    else
      prev = wd;
  };
  if (r.vlen > kVarCap) {
    raw_words(b, r.rs, SLAB, nt, emit);
    return;
  }
  if constexpr (SLAB == 0) {
    *reinterpret_cast<uint4*>(var + 16 * lane) = vp.v0;
    *reinterpret_cast<uint4*>(var + 1024 + 16 * lane) = vp.v1;
    wave_lds_sync();
  }
  auto rd4 = [&](int off) { return *reinterpret_cast<const uint32_t*>(var + off); };
  const SlabHdr h = slab_header(rd4, SLAB);
  stage_escapes(rd4, h, lut.s, esc, lane);
  // kernel-order exclusive prefix of the escape counts
  const int cnt = thread_escapes(b);
  const int v_nat = __shfl(cnt, lane_of_natural(lane), 64);
  const int incl = wave_incl_scan(v_nat);
  const int excl = __shfl(incl - v_nat, nt, 64);
  decode_words(b, esc, (h.e0 & 7) + excl, lut.p0, lut.p1, emit);
}

// Fragment tile [head 8][a 4][c 4] x 16 B: lane (c, n) reads its 8 BF16 of
// k-chunk a at ((n * 4 + a) * 4 + c) * 16.  Used for Q (dims) and P (tokens).
__device__ __forceinline__ uint4 tile_frag(const uint8_t* tile, int n, int a, int c) {
  return *reinterpret_cast<const uint4*>(tile + (((n & 7) * 4 + a) * 4 + c) * 16);
}

__global__ void __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(2))) attn_kernel(AttnParams p) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int lane = wave_lane();
  const int wv = threadIdx.x >> 6;
  uint8_t* esc = lds + wv * kWaveLds;
  uint8_t* var = esc + kEscLds;
  uint8_t* pt = var + kVarCap;
  uint8_t* qt = pt + kTileBytes;
  const int h = blockIdx.y;
  const int c = lane >> 4, hh = (lane >> 3) & 1, g = lane & 7;
  const int nt = 32 * hh + 4 * g + c;
  const int n = lane & 15;  // MFMA column = query head within the group
  const int budget = uniform(p.plan[1]);
  const int ppc = uniform(p.plan[0]);
  const HeadLut klut = load_lut(p.plut, p.slut, h);
  const HeadLut vlut = load_lut(p.plut, p.slut, p.kvh + h);

  for (int unit = blockIdx.x * kWaves + wv; unit < budget; unit += gridDim.x * kWaves) {
    const int b = uniform(p.plan[2 + 2 * unit]);
    if (b < 0) continue;
    const int p0 = uniform(p.plan[3 + 2 * unit]);
    const int seq = uniform(p.seq_lens[b]);
    const int npages = max(0, min((seq + 127) >> 7, p0 + ppc) - p0);
    if (npages == 0) continue;
    const int32_t* bt = p.block_table + (int64_t)b * p.bt_stride + p0;

    // Q tile: element (n, dim) at tile position (n, a = dim / 32, c, slot);
    // the dims of slot i = 4x + 2f + e of (a, c) are 32a + 16x + 8f + 2c + e.
    // Lane (c, n < 8) writes its four 16-byte fragments; heads >= G are zero.
    wave_lds_sync();
    if (hh == 0) {
      const bool valid = n < p.group;
      const uint32_t* q = reinterpret_cast<const uint32_t*>(p.q + (int64_t)b * p.q_stride +
                                                            (int64_t)(h * p.group + (valid ? n : 0)) * kDim);
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d = 16 * a + c;
        const uint4 v = valid ? make_uint4(q[d], q[d + 4], q[d + 8], q[d + 12]) : make_uint4(0u, 0u, 0u, 0u);
        *reinterpret_cast<uint4*>(qt + ((n * 4 + a) * 4 + c) * 16) = v;
      }
    }
    wave_lds_sync();
    float m_run = -INFINITY, l_run = 0.f;
    f32x4 o[4][2];
#pragma unroll
    for (int s = 0; s < 4; ++s) o[s][0] = o[s][1] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int64_t blk0 = uniform(bt[0]);
    RecRef kr = rec_ref(p, blk0, 0, h), vr = rec_ref(p, blk0, 1, h);
    SlabBuf fa, fb;  // double buffer: even slabs of a page in fa, odd in fb
    VarPref vp;
    prefetch<0>(kr, nt, lane, fa, vp);
    for (int i = 0; i < npages; ++i) {
      const bool more = i + 1 < npages;
      const int64_t nblk = more ? (int64_t)uniform(bt[i + 1]) : 0;
      const RecRef nkr = more ? rec_ref(p, nblk, 0, h) : kr;
      const RecRef nvr = more ? rec_ref(p, nblk, 1, h) : vr;
      const int tok0 = (p0 + i) * kTokens;

      // ---- S^T = K Q^T: s[slab][j] rows = tokens, column = head n ----
      f32x4 s[4][2];
      static_for<0, 4>([&](auto sl_c) {
        constexpr int sl = decltype(sl_c)::value;
        slab_fence();
        SlabBuf& cur = (sl & 1) ? fb : fa;
        SlabBuf& nxt = (sl & 1) ? fa : fb;
        if constexpr (sl < 3)
          prefetch<sl + 1>(kr, nt, lane, nxt, vp);
        const VarPref vcur = vp;
        if constexpr (sl == 3) prefetch<0>(vr, nt, lane, nxt, vp);
        f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
        decode_slab<sl>(kr, cur, vcur, nt, lane, klut, var, esc, [&](auto a, const uint4& w0, const uint4& w1) {
          const uint4 qa = tile_frag(qt, n, a, c);
          acc0 = mfma(a_frag(w0, w1, 0), qa, acc0);
          acc1 = mfma(a_frag(w0, w1, 1), qa, acc1);
        });
        s[sl][0] = acc0;
        s[sl][1] = acc1;
      });
      // token of s[sl][j][r] = 32 sl + 16 (c >> 1) + 8 j + 4 (c & 1) + r
      float mloc = -INFINITY;
#pragma unroll
      for (int sl = 0; sl < 4; ++sl)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int tok = tok0 + 32 * sl + 16 * (c >> 1) + 8 * j + 4 * (c & 1) + r;
            const float v = tok < seq ? s[sl][j][r] * p.scale_log2 : -INFINITY;
            s[sl][j][r] = v;
            mloc = fmaxf(mloc, v);
          }
      mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
      const float m_new = fmaxf(m_run, mloc);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
      m_run = m_new;
      float psum = 0.f;
#pragma unroll
      for (int sl = 0; sl < 4; ++sl)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          float e[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            e[r] = __builtin_amdgcn_exp2f(s[sl][j][r] - m_use);
            psum += e[r];
          }
          // P[n][token] -> tile[n][a = sl][c' = 2 (c & 1) + r / 2][x = c >> 1][f = j][e = r & 1]
          if (hh == 0) {
            const uint32_t p01 = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)e[0]) |
                                 ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)e[1]) << 16);
            const uint32_t p23 = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)e[2]) |
                                 ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)e[3]) << 16);
            uint8_t* base = pt + ((n * 4 + sl) * 4 + 2 * (c & 1)) * 16 + 8 * (c >> 1) + 4 * j;
            *reinterpret_cast<uint32_t*>(base) = p01;
            *reinterpret_cast<uint32_t*>(base + 16) = p23;
          }
        }
      l_run = l_run * alpha + psum;
#pragma unroll
      for (int sl = 0; sl < 4; ++sl)
#pragma unroll
        for (int j = 0; j < 2; ++j) o[sl][j] *= alpha;
      wave_lds_sync();
      uint4 pf[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) pf[a] = tile_frag(pt, n, a, c);

      // ---- O^T += V^T P^T: o[slab][j] rows = dims, column = head n ----
      static_for<0, 4>([&](auto sl_c) {
        constexpr int sl = decltype(sl_c)::value;
        slab_fence();
        SlabBuf& cur = (sl & 1) ? fb : fa;
        SlabBuf& nxt = (sl & 1) ? fa : fb;
        if constexpr (sl < 3)
          prefetch<sl + 1>(vr, nt, lane, nxt, vp);
        const VarPref vcur = vp;
        if constexpr (sl == 3) {
          if (more) prefetch<0>(nkr, nt, lane, nxt, vp);
        }
        decode_slab<sl>(vr, cur, vcur, nt, lane, vlut, var, esc, [&](auto a, const uint4& w0, const uint4& w1) {
          o[sl][0] = mfma(a_frag(w0, w1, 0), pf[a], o[sl][0]);
          o[sl][1] = mfma(a_frag(w0, w1, 1), pf[a], o[sl][1]);
        });
      });
      wave_lds_sync();  // P is rewritten next page
      kr = nkr;
      vr = nvr;
    }

    // ---- partial results of this unit ----
    float l_tot = l_run;
    l_tot += __shfl_xor(l_tot, 16, 64);
    l_tot += __shfl_xor(l_tot, 32, 64);
    if (hh == 0) {
      const int64_t row = ((int64_t)h * p.units + unit) * 8 + n;
      float* orow = p.opart + row * kDim;
#pragma unroll
      for (int sl = 0; sl < 4; ++sl)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int d = 32 * sl + 16 * (c >> 1) + 8 * j + 4 * (c & 1);
          *reinterpret_cast<float4*>(orow + d) = make_float4(o[sl][j][0], o[sl][j][1], o[sl][j][2], o[sl][j][3]);
        }
      if (c == 0) {
        p.ml[row * 2] = m_run;
        p.ml[row * 2 + 1] = l_tot;
      }
    }
  }
}

// Merges each sequence's chunk partials; rows with no context are zero.
__global__ void __launch_bounds__(128) combine_kernel(const float* opart, const float* ml, const int32_t* plan,
                                                     uint16_t* out, int64_t out_stride, int units, int group) {
  const int b = blockIdx.x, qh = blockIdx.y, d = threadIdx.x;
  const int h = qh / group, g = qh % group;
  const int first = plan[2 + 2 * units + 2 * b], chunks = plan[3 + 2 * units + 2 * b];
  const int64_t base = (int64_t)h * units + first;
  float gm = -INFINITY;
  for (int s = 0; s < chunks; ++s) gm = fmaxf(gm, ml[((base + s) * 8 + g) * 2]);
  float den = 0.f, acc = 0.f;
  if (gm != -INFINITY) {
    for (int s = 0; s < chunks; ++s) {
      const int64_t r = (base + s) * 8 + g;
      const float w = __builtin_amdgcn_exp2f(ml[r * 2] - gm);
      den += w * ml[r * 2 + 1];
      acc += w * opart[r * kDim + d];
    }
  }
  const float v = den > 0.f ? acc / den : 0.f;
  out[(int64_t)b * out_stride + (int64_t)qh * kDim + d] = __builtin_bit_cast(uint16_t, (__bf16)v);
}

}  // namespace
}  // namespace fp

using namespace fp;

extern "C" int fp_fused_decode(const void* q, int64_t q_stride, int64_t batch, int64_t kv_heads, int64_t group,
                               const int64_t* rec_addr, const int32_t* rec_len, const uint32_t* plut,
                               const uint8_t* slut, const int32_t* block_table, int64_t bt_stride,
                               const int32_t* seq_lens, float* opart, int64_t opart_elems, float* ml,
                               int64_t ml_elems, int32_t* plan, int64_t plan_elems, void* out, int64_t out_stride,
                               int64_t units, int replan, double scale, fp_stream_t stream) {
  FP_CHECK(batch >= 0 && kv_heads > 0, "decode needs batch >= 0 and kv_heads > 0");
  FP_CHECK(group == 1 || group == 2 || group == 4 || group == 8, "query heads need a group dividing 8");
  if (batch == 0) return 0;
  FP_CHECK(units >= batch, "decode needs at least one unit per sequence");
  FP_CHECK(q_stride % 2 == 0 && q_stride >= kv_heads * group * kDim, "q must be [B, H, 128] with contiguous heads");
  FP_CHECK(out_stride >= kv_heads * group * kDim, "out must be [B, H, 128] with contiguous heads");
  FP_CHECK(opart_elems >= kv_heads * units * 8 * kDim && ml_elems >= kv_heads * units * 16,
           "decode workspace too small");
  FP_CHECK(plan_elems >= 2 + 4 * units, "decode plan must be int32 with 2 + 4 * units elements");
  FP_CHECK(units < (1 << 24) && batch < (1 << 24), "batch too large");
  AttnParams p;
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
  p.scale_log2 = (float)(scale * 1.4426950408889634);
  if (replan) {
    hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, seq_lens, plan, (int)batch, (int)units);
    FP_LAUNCH_CHECK();
  }
  const int grid_x = (int)((units + kWaves - 1) / kWaves);
  const size_t lds = (size_t)kWaves * kWaveLds;
  hipLaunchKernelGGL(attn_kernel, dim3(grid_x, (unsigned)kv_heads), dim3(64 * kWaves), lds, stream, p);
  FP_LAUNCH_CHECK();
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)batch, (unsigned)(kv_heads * group)), dim3(kDim), 0, stream,
                     opart, ml, plan, static_cast<uint16_t*>(out), out_stride, (int)units, (int)group);
  FP_LAUNCH_CHECK();
  return 0;
}
