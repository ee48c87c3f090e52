/*
 * FragPack CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's record codec and of the fp32
 * attention its tests compare against. Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load this library, and only as the
 * checker (or the timed CPU baseline); the product package never calls it.
 *
 * Functions and the reference code each one restates:
 *   fpo_kernel_order      attn_page.py:83-94   (_kernel_order)
 *   fpo_calibrate_table   attn_page.py:97-111  (calibrate_table, stable top-22)
 *   fpo_tables            attn_page.py:114-143 (primary_lut / secondary_lut) and
 *                         attn_tables.py:96-124 (rank_of of device_tables)
 *   fpo_encode_record     attn_page.py:146-209, 272-282 (encode_record,
 *                         _interleave_dense, _raw_words)
 *   fpo_decode_record     attn_page.py:212-269 (decode_record)
 *   fpo_raw_record        attn_page.py:279-282 (_raw_words, the raw form)
 *   fpo_encode_batch /
 *   fpo_decode_batch      the two above over many records (OpenMP)
 *   fpo_paged_attention   fp32 softmax(q k^T * scale) v over paged records, as
 *                         in tests/gpu/test_fragpack_hbm_store.py:204-215
 *                         (reference decode path fused_attn_decode.cu:214-425)
 *
 * Pinning (how each is checked, tests/test_oracle.py):
 *   kernel order, LUTs, calibration, encode bytes, decode: golden vectors
 *   written by tests/golden/make_golden.py from the reference codec itself;
 *   plus round-trip / permutation / closed-form var_len invariants.
 *   paged attention: a float64 numpy softmax on the same decoded KV, and the
 *   identity that repeating a page n times equals adding log(n) to its logits.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum {
  PAGE_TOKENS = 128,
  HEAD_DIM = 128,
  RECORD_SCALARS = 16384,
  GROUP_SCALARS = 32,
  WARP_SCALARS = 2048,
  WARPS = 8,
  PRIMARY_DIRECT = 7,
  TABLE_ENTRIES = 22,
  RAW_NIBBLE = 15,
  HEADER_BYTES = 48,
  LOW_BYTES = 16384,
  SYMBOL_BYTES = 6144,
  DENSE_BYTES = 22528,
  VAR_CAP = 2048,
  THREADS = 256,
  RAW_RECORD_BYTES = 32768,
  MAX_WARP_RAW = 32,
};

static int32_t g_order[2][RECORD_SCALARS];
static int g_order_ready = 0;

/* attn_page.py:83-94: thread t = (w, g, c) owns kernel positions 64t..64t+63;
 * scalar s = 8 st + 4 j + 2 f + e.  K: row = token, col = dim; V swapped. */
void fpo_kernel_order(int kv, int32_t* out) {
  for (int t = 0; t < THREADS; ++t) {
    const int w = t >> 5, g = (t >> 2) & 7, c = t & 3;
    for (int s = 0; s < 64; ++s) {
      const int st = s >> 3, j = (s >> 2) & 1, f = (s >> 1) & 1, e = s & 1;
      const int row = 16 * w + 8 * j + g, col = 16 * st + 8 * f + 2 * c + e;
      const int tok = kv == 0 ? row : col, dim = kv == 0 ? col : row;
      out[64 * t + s] = tok * HEAD_DIM + dim;
    }
  }
}

static void ensure_order(void) {
  if (g_order_ready) return;
#ifdef _OPENMP
#pragma omp critical(fpo_order)
#endif
  {
    if (!g_order_ready) {
      fpo_kernel_order(0, g_order[0]);
      fpo_kernel_order(1, g_order[1]);
      g_order_ready = 1;
    }
  }
}

/* attn_page.py:97-111: the 22 most frequent bytes, ties broken toward the
 * smaller byte value (numpy's stable argsort of -count). */
void fpo_calibrate_table(const uint8_t* high, int64_t n, uint8_t* out) {
  int64_t count[256];
  memset(count, 0, sizeof(count));
  for (int64_t i = 0; i < n; ++i) count[high[i]]++;
  int order[256];
  for (int i = 0; i < 256; ++i) order[i] = i;
  /* insertion sort, stable, descending count */
  for (int i = 1; i < 256; ++i) {
    const int v = order[i];
    int k = i - 1;
    while (k >= 0 && count[order[k]] < count[v]) {
      order[k + 1] = order[k];
      --k;
    }
    order[k + 1] = v;
  }
  for (int i = 0; i < TABLE_ENTRIES; ++i) out[i] = (uint8_t)order[i];
}

/* attn_page.py:114-143 and attn_tables.py:112-119. */
void fpo_tables(const uint8_t* table, uint8_t* rank_of, uint32_t* plut, uint8_t* slut) {
  if (rank_of) {
    memset(rank_of, 255, 256);
    for (int i = 0; i < TABLE_ENTRIES; ++i) rank_of[table[i]] = (uint8_t)i;
  }
  if (plut) {
    uint8_t b[8];
    for (int i = 0; i < 7; ++i) b[i] = table[i];
    b[7] = 0;
    plut[0] = b[0] | (b[1] << 8) | (b[2] << 16) | ((uint32_t)b[3] << 24);
    plut[1] = b[4] | (b[5] << 8) | (b[6] << 16) | ((uint32_t)b[7] << 24);
  }
  if (slut) {
    for (int i = 0; i < 15; ++i) slut[i] = table[PRIMARY_DIRECT + i];
    slut[15] = 0;
  }
}

static inline void put_u32(uint8_t* p, uint32_t v) {
  p[0] = v & 0xFF;
  p[1] = (v >> 8) & 0xFF;
  p[2] = (v >> 16) & 0xFF;
  p[3] = (v >> 24) & 0xFF;
}
static inline void put_u16(uint8_t* p, uint32_t v) {
  p[0] = v & 0xFF;
  p[1] = (v >> 8) & 0xFF;
}
static inline uint32_t get_u32(const uint8_t* p) {
  return p[0] | (p[1] << 8) | (p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* attn_page.py:146-209.  raw: token-major [128,128] BF16 bits.  out must hold
 * RAW_RECORD_BYTES.  Returns the record length in bytes. */
int fpo_encode_record(const uint16_t* raw, const uint8_t* table, int kv, uint8_t* out) {
  ensure_order();
  uint8_t rank_of[256];
  fpo_tables(table, rank_of, NULL, NULL);
  uint16_t vals[RECORD_SCALARS];
  uint8_t rank[RECORD_SCALARS];
  const int32_t* ord = g_order[kv ? 1 : 0];
  for (int p = 0; p < RECORD_SCALARS; ++p) {
    vals[p] = raw[ord[p]];
    rank[p] = rank_of[vals[p] >> 8];
  }
  /* escapes in kernel order, per-slab prefixes, raw list */
  int n_esc = 0, n_raw = 0, warp_raw_max = 0;
  uint16_t esc_prefix[WARPS], raw_prefix[WARPS];
  static const int kNibCap = 2 * VAR_CAP;
  uint8_t nib[2 * VAR_CAP + 2];
  uint32_t rawlist[RECORD_SCALARS];
  for (int w = 0; w < WARPS; ++w) {
    esc_prefix[w] = (uint16_t)n_esc;
    raw_prefix[w] = (uint16_t)n_raw;
    int wr = 0;
    for (int p = w * WARP_SCALARS; p < (w + 1) * WARP_SCALARS; ++p) {
      const int r = rank[p];
      if (r >= PRIMARY_DIRECT) {
        if (n_esc < kNibCap) nib[n_esc] = (uint8_t)(r < TABLE_ENTRIES ? r - PRIMARY_DIRECT : RAW_NIBBLE);
        if (r >= TABLE_ENTRIES) {
          rawlist[n_raw++] = (uint32_t)n_esc | ((uint32_t)(vals[p] >> 8) << 16);
          ++wr;
        }
        ++n_esc;
      }
    }
    if (wr > warp_raw_max) warp_raw_max = wr;
  }
  const int nib_bytes = (n_esc + 1) / 2;
  const int raw_offset = (HEADER_BYTES + nib_bytes + 3) & ~3;
  const int var_len = (raw_offset + 4 * n_raw + 15) & ~15;
  if (var_len > VAR_CAP || warp_raw_max > MAX_WARP_RAW) {
    /* _raw_words: thread t's word st (8 scalars) at 16 (256 st + t). */
    for (int t = 0; t < THREADS; ++t)
      for (int st = 0; st < 8; ++st)
        for (int i = 0; i < 8; ++i)
          put_u16(out + 16 * (256 * st + t) + 2 * i, vals[64 * t + 8 * st + i]);
    return RAW_RECORD_BYTES;
  }
  /* dense low bytes: thread t's chunk j (16 scalars) at 16 (256 j + t) */
  for (int t = 0; t < THREADS; ++t)
    for (int j = 0; j < 4; ++j)
      for (int i = 0; i < 16; ++i) out[16 * (256 * j + t) + i] = vals[64 * t + 16 * j + i] & 0xFF;
  /* symbols: group G (32 scalars) -> 3 words; thread t's six words (groups
   * 2t, 2t+1) as three 8-byte chunks m at LOW + 8 (256 m + t). */
  for (int t = 0; t < THREADS; ++t) {
    uint32_t w6[6];
    for (int gi = 0; gi < 2; ++gi) {
      const int base = 64 * t + 32 * gi;
      uint32_t prim[32];
      for (int i = 0; i < 32; ++i) prim[i] = rank[base + i] < PRIMARY_DIRECT ? rank[base + i] : PRIMARY_DIRECT;
      for (int k = 0; k < 3; ++k) {
        uint32_t word = 0;
        for (int j = 0; j < 8; ++j) {
          word |= (prim[8 * k + j] & 7u) << (4 * j);
          word |= ((prim[24 + j] >> k) & 1u) << (4 * j + 3);
        }
        w6[3 * gi + k] = word;
      }
    }
    for (int m = 0; m < 3; ++m) {
      put_u32(out + LOW_BYTES + 8 * (256 * m + t), w6[2 * m]);
      put_u32(out + LOW_BYTES + 8 * (256 * m + t) + 4, w6[2 * m + 1]);
    }
  }
  /* variable region: <4I8H8H> header, nibbles, raw list, zero padding. */
  uint8_t* var = out + DENSE_BYTES;
  memset(var, 0, var_len);
  put_u32(var + 0, n_esc);
  put_u32(var + 4, n_raw);
  put_u32(var + 8, raw_offset);
  put_u32(var + 12, 0);
  for (int w = 0; w < WARPS; ++w) {
    put_u16(var + 16 + 2 * w, esc_prefix[w]);
    put_u16(var + 32 + 2 * w, raw_prefix[w]);
  }
  for (int i = 0; i < n_esc; ++i) var[HEADER_BYTES + i / 2] |= (uint8_t)(nib[i] << (4 * (i & 1)));
  for (int i = 0; i < n_raw; ++i) put_u32(var + raw_offset + 4 * i, rawlist[i]);
  return DENSE_BYTES + var_len;
}

/* attn_page.py:279-282 (_raw_words): the raw (fallback / open-block) form of
 * a token-major record, thread t's word st at 16 (256 st + t). */
void fpo_raw_record(const uint16_t* raw, int kv, uint8_t* out) {
  ensure_order();
  const int32_t* ord = g_order[kv ? 1 : 0];
  for (int t = 0; t < THREADS; ++t)
    for (int st = 0; st < 8; ++st)
      for (int i = 0; i < 8; ++i) put_u16(out + 16 * (256 * st + t) + 2 * i, raw[ord[64 * t + 8 * st + i]]);
}

/* attn_page.py:212-269.  Returns 0, or -1 for a malformed record. */
int fpo_decode_record(const uint8_t* rec, int len, const uint8_t* table, int kv, uint16_t* out) {
  ensure_order();
  const int32_t* ord = g_order[kv ? 1 : 0];
  if (len == RAW_RECORD_BYTES) {
    for (int t = 0; t < THREADS; ++t)
      for (int st = 0; st < 8; ++st)
        for (int i = 0; i < 8; ++i) {
          const uint8_t* p = rec + 16 * (256 * st + t) + 2 * i;
          out[ord[64 * t + 8 * st + i]] = (uint16_t)(p[0] | (p[1] << 8));
        }
    return 0;
  }
  if (len < DENSE_BYTES + HEADER_BYTES || len > DENSE_BYTES + VAR_CAP) return -1;
  const uint8_t* var = rec + DENSE_BYTES;
  const int var_len = len - DENSE_BYTES;
  const uint32_t n_esc = get_u32(var), n_raw = get_u32(var + 4), raw_offset = get_u32(var + 8);
  if (HEADER_BYTES + (n_esc + 1) / 2 > (uint32_t)var_len || raw_offset + 4 * n_raw > (uint32_t)var_len) return -1;
  /* escape values, in kernel order of the escapes */
  uint16_t esc_val[2 * VAR_CAP];
  for (uint32_t i = 0; i < n_esc; ++i) {
    const int nb = (var[HEADER_BYTES + i / 2] >> (4 * (i & 1))) & 15;
    esc_val[i] = nb < RAW_NIBBLE ? table[PRIMARY_DIRECT + nb] : 0;
  }
  for (uint32_t i = 0; i < n_raw; ++i) {
    const uint32_t e = get_u32(var + raw_offset + 4 * i);
    if ((e & 0xFFFF) < n_esc) esc_val[e & 0xFFFF] = (uint16_t)(e >> 16);
  }
  uint32_t x = 0;
  for (int t = 0; t < THREADS; ++t) {
    uint32_t w6[6];
    uint8_t low[64];
    for (int m = 0; m < 3; ++m) {
      w6[2 * m] = get_u32(rec + LOW_BYTES + 8 * (256 * m + t));
      w6[2 * m + 1] = get_u32(rec + LOW_BYTES + 8 * (256 * m + t) + 4);
    }
    for (int j = 0; j < 4; ++j)
      for (int i = 0; i < 16; ++i) low[16 * j + i] = rec[16 * (256 * j + t) + i];
    for (int gi = 0; gi < 2; ++gi) {
      uint32_t codes[32];
      memset(codes, 0, sizeof(codes));
      for (int k = 0; k < 3; ++k)
        for (int j = 0; j < 8; ++j) {
          const uint32_t word = w6[3 * gi + k];
          codes[8 * k + j] = (word >> (4 * j)) & 7;
          codes[24 + j] |= ((word >> (4 * j + 3)) & 1) << k;
        }
      for (int i = 0; i < 32; ++i) {
        const int s = 32 * gi + i;
        uint32_t high;
        if (codes[i] < PRIMARY_DIRECT) {
          high = table[codes[i]];
        } else {
          if (x >= n_esc) return -1;
          high = esc_val[x++];
        }
        out[ord[64 * t + s]] = (uint16_t)(low[s] | (high << 8));
      }
    }
  }
  return x == n_esc ? 0 : -1;
}

/* Many records: raw [n,128,128], tables [n_tab,22] selected by tab_idx[i],
 * kv[i]; out [n, RAW_RECORD_BYTES], lens[n]. */
void fpo_encode_batch(int64_t n, const uint16_t* raw, const uint8_t* tables, const int32_t* tab_idx,
                      const int32_t* kv, uint8_t* out, int32_t* lens, int threads) {
  ensure_order();
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 16) num_threads(threads > 0 ? threads : 1)
#endif
  for (int64_t i = 0; i < n; ++i)
    lens[i] = fpo_encode_record(raw + i * RECORD_SCALARS, tables + 22 * (int64_t)tab_idx[i], kv[i],
                                out + i * (int64_t)RAW_RECORD_BYTES);
  (void)threads;
}

int fpo_decode_batch(int64_t n, const uint8_t* recs, const int32_t* lens, const uint8_t* tables,
                     const int32_t* tab_idx, const int32_t* kv, uint16_t* out, int threads) {
  ensure_order();
  int bad = 0;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 16) reduction(| : bad) num_threads(threads > 0 ? threads : 1)
#endif
  for (int64_t i = 0; i < n; ++i)
    bad |= fpo_decode_record(recs + i * (int64_t)RAW_RECORD_BYTES, lens[i], tables + 22 * (int64_t)tab_idx[i],
                             kv[i], out + i * RECORD_SCALARS) != 0;
  (void)threads;
  return bad ? -1 : 0;
}

static inline float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/*
 * fp32 decode attention over paged records (one query token per sequence).
 *   q        BF16 bits [B, H*G, 128] (contiguous)
 *   rec      record bytes, addressed by rec_off[(page*2 + kv)*H + h] (byte
 *            offset into rec) with length DENSE_BYTES + rec_len[...]
 *   tables   [2, H, 22] codec tables of this layer
 *   block_table [B, bt_stride] int32, seq_lens [B]
 *   out      fp32 [B, H*G, 128]; rows with seq_len 0 are zero.
 * Every referenced record is decoded per (b, h) (the CPU baseline pays the
 * codec like the GPU path does).
 */
int fpo_paged_attention(const uint16_t* q, int B, int H, int G, const uint8_t* rec, const int64_t* rec_off,
                        const int32_t* rec_len, const uint8_t* tables, const int32_t* block_table,
                        int64_t bt_stride, const int32_t* seq_lens, float scale, float* out, int threads) {
  ensure_order();
  int bad = 0;
#ifdef _OPENMP
#pragma omp parallel for collapse(2) schedule(dynamic, 1) reduction(| : bad) num_threads(threads > 0 ? threads : 1)
#endif
  for (int b = 0; b < B; ++b) {
    for (int h = 0; h < H; ++h) {
      const int seq = seq_lens[b];
      float* o = out + ((int64_t)b * H * G + (int64_t)h * G) * HEAD_DIM;
      memset(o, 0, sizeof(float) * G * HEAD_DIM);
      if (seq <= 0) continue;
      const int pages = (seq + PAGE_TOKENS - 1) / PAGE_TOKENS;
      float* logits = (float*)malloc(sizeof(float) * (size_t)G * pages * PAGE_TOKENS);
      uint16_t* kbuf = (uint16_t*)malloc(sizeof(uint16_t) * RECORD_SCALARS);
      uint16_t* vbuf = (uint16_t*)malloc(sizeof(uint16_t) * RECORD_SCALARS);
      float qf[8][HEAD_DIM];
      for (int g = 0; g < G; ++g)
        for (int d = 0; d < HEAD_DIM; ++d)
          qf[g][d] = bf16_to_f32(q[((int64_t)b * H * G + (int64_t)h * G + g) * HEAD_DIM + d]);
      float mx[8];
      for (int g = 0; g < G; ++g) mx[g] = -INFINITY;
      for (int p = 0; p < pages; ++p) {
        const int64_t blk = block_table[(int64_t)b * bt_stride + p];
        const int64_t ki = (blk * 2 + 0) * H + h;
        bad |= fpo_decode_record(rec + rec_off[ki], DENSE_BYTES + rec_len[ki], tables + (0 * H + h) * 22, 0, kbuf);
        const int ntok = (p == pages - 1) ? seq - p * PAGE_TOKENS : PAGE_TOKENS;
        for (int t = 0; t < ntok; ++t)
          for (int g = 0; g < G; ++g) {
            float s = 0.f;
            for (int d = 0; d < HEAD_DIM; ++d) s += qf[g][d] * bf16_to_f32(kbuf[t * HEAD_DIM + d]);
            s *= scale;
            logits[(int64_t)g * pages * PAGE_TOKENS + p * PAGE_TOKENS + t] = s;
            if (s > mx[g]) mx[g] = s;
          }
      }
      float den[8];
      for (int g = 0; g < G; ++g) {
        den[g] = 0.f;
        for (int x = 0; x < seq; ++x) {
          float* l = &logits[(int64_t)g * pages * PAGE_TOKENS + x];
          *l = expf(*l - mx[g]);
          den[g] += *l;
        }
      }
      for (int p = 0; p < pages; ++p) {
        const int64_t blk = block_table[(int64_t)b * bt_stride + p];
        const int64_t vi = (blk * 2 + 1) * H + h;
        bad |= fpo_decode_record(rec + rec_off[vi], DENSE_BYTES + rec_len[vi], tables + (1 * H + h) * 22, 1, vbuf);
        const int ntok = (p == pages - 1) ? seq - p * PAGE_TOKENS : PAGE_TOKENS;
        for (int t = 0; t < ntok; ++t)
          for (int g = 0; g < G; ++g) {
            const float w = logits[(int64_t)g * pages * PAGE_TOKENS + p * PAGE_TOKENS + t] / den[g];
            for (int d = 0; d < HEAD_DIM; ++d) o[g * HEAD_DIM + d] += w * bf16_to_f32(vbuf[t * HEAD_DIM + d]);
          }
      }
      free(logits);
      free(kbuf);
      free(vbuf);
    }
  }
  return bad ? -1 : 0;
}

int fpo_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
