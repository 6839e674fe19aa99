/*
 * pdm_oracle.c — CPU restatement of the reference's embedding-lookup
 * semantics.  TEST INFRASTRUCTURE ONLY: the parity tests, the smoke check
 * and the benchmark's CPU-baseline leg call it as the checker.  Nothing in
 * the product links or calls it.
 *
 * Plain C, fp32 arithmetic in the order stated for every output, compiled
 * with -ffp-contract=off so that no multiply-add is fused.
 *
 * Functions and what each follows:
 *   oracle_tbe_pooled      pooled sum/mean per (table, bag):
 *                          primus_dlrm/models/sharded_embedding.py:220-227
 *                          (sum = sum of masked rows, mean = sum /
 *                          clamp(count, 1)); padding filter of
 *                          primus_dlrm/models/embedding.py:188-194;
 *                          table-major offsets of the TBE op
 *                          (tests/test_fbgemm_tbe.py:33-35).
 *   oracle_int8_quantize   int8 rowwise quantizer (no reference counterpart;
 *                          the reference has no quantized path) restating
 *                          FBGEMM's fused rowwise SB-half method.
 *   oracle_seq_gather      jagged -> padded per-pool gather: keep the last
 *                          max_len events, left pad with id 0
 *                          (primus_dlrm/data/dataset.py:604-626), look up
 *                          every feature table and concat per event
 *                          (primus_dlrm/models/onetrans.py:515-520), pools
 *                          concatenated along the sequence (:553-558).
 *   oracle_cross_hash      cross-feature ids: xxHash64 (seed = salt) of the
 *                          little-endian concatenation of n int64 keys,
 *                          modulo table_size (primus_dlrm/data/hashing.py:
 *                          23-52, struct "<{n}q" pack + xxhash.xxh64 +
 *                          intdigest() % table_size).  XXH64 is restated
 *                          from its published specification, byte by byte
 *                          over the packed buffer (any length), not from
 *                          the word structure the GPU kernel uses.
 *   oracle_tbe_backward    pooled-lookup backward with the fused embedding
 *                          optimizer TorchRec substitutes for the
 *                          reference's choice (primus_dlrm/distributed/
 *                          wrapper.py:151-174): the row gradient summed in
 *                          lookup order, then FBGEMM's ADAM or
 *                          EXACT_ROWWISE_ADAGRAD update rule per distinct
 *                          row (formulas at the function).
 *   f32_to_f16 / f32_to_bf16 / f16_to_f32: IEEE round-to-nearest-even.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { O_F32 = 0, O_F16 = 1, O_BF16 = 2, O_I8 = 3 };

/* ---- conversions ------------------------------------------------------ */

static inline uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float oracle_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ff;
  if (exp == 0) {
    /* zero or subnormal: value = man * 2^-24, exact in fp32 */
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  if (exp == 31) return bits_f(sign | 0x7f800000u | (man << 13));
  return bits_f(sign | ((exp + 112) << 23) | (man << 13));
}

uint16_t oracle_f32_to_f16(float f) {
  uint32_t u = f_bits(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000);
  uint32_t a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) /* inf or nan */
    return sign | (a > 0x7f800000u ? 0x7e00 : 0x7c00);
  if (a >= 0x477ff000u) /* rounds to >= 65520 -> inf */
    return sign | 0x7c00;
  if (a < 0x38800000u) {
    /* result is subnormal in fp16 (or zero): quantum 2^-24 */
    float m = bits_f(a) * 16777216.0f;     /* exact scaling by 2^24 */
    float r = rintf(m);                    /* ties to even */
    return sign | (uint16_t)r;
  }
  /* normal: keep 10 mantissa bits, round to nearest even */
  uint32_t lsb = (a >> 13) & 1u;
  uint32_t r = a + 0xfffu + lsb;
  r >>= 13;
  r -= (112u << 10);
  return sign | (uint16_t)r;
}

uint16_t oracle_f32_to_bf16(float f) {
  uint32_t u = f_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

static inline float bf16_to_f32(uint16_t b) { return bits_f((uint32_t)b << 16); }

/* ---- pooled lookup ------------------------------------------------------ */

typedef struct {
  int64_t rows;
  int64_t weights_offset; /* bytes */
  int32_t dim;
  int32_t dtype;
  int32_t pooling; /* 0 sum, 1 mean */
  int32_t row_bytes;
  int32_t out_offset;
  int32_t reserved;
} oracle_table;

static inline float decode(const uint8_t* row, int32_t dtype, int32_t d) {
  switch (dtype) {
    case O_F32: { float v; memcpy(&v, row + 4 * (size_t)d, 4); return v; }
    case O_F16: { uint16_t h; memcpy(&h, row + 2 * (size_t)d, 2); return oracle_f16_to_f32(h); }
    case O_BF16: { uint16_t h; memcpy(&h, row + 2 * (size_t)d, 2); return bf16_to_f32(h); }
    default: {
      uint16_t s16, b16;
      memcpy(&s16, row, 2);
      memcpy(&b16, row + 2, 2);
      volatile float prod = (float)row[4 + d] * oracle_f16_to_f32(s16);
      return prod + oracle_f16_to_f32(b16);
    }
  }
}

static inline int32_t default_row_bytes(int32_t dtype, int32_t dim) {
  switch (dtype) {
    case O_F32: return 4 * dim;
    case O_F16: case O_BF16: return 2 * dim;
    default: return (4 + dim + 3) & ~3;
  }
}

static inline void store_out(void* out, int32_t out_dtype, size_t pos, float v) {
  if (out_dtype == O_F32) ((float*)out)[pos] = v;
  else if (out_dtype == O_F16) ((uint16_t*)out)[pos] = oracle_f32_to_f16(v);
  else ((uint16_t*)out)[pos] = oracle_f32_to_bf16(v);
}

/* Returns the number of invalid entries met (out-of-range indices and bags
 * with bad offsets); those are skipped exactly as the device kernel does. */
int64_t oracle_tbe_pooled(const oracle_table* tables, int32_t T, int64_t B,
                          const uint8_t* weights, const void* indices,
                          int32_t index_bits, int64_t num_indices,
                          const int64_t* offsets, int64_t padding_idx,
                          void* out, int32_t out_dtype, int64_t out_stride,
                          int32_t num_threads) {
  int64_t bad = 0;
  (void)num_threads;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : bad) num_threads(num_threads > 0 ? num_threads : 1)
  for (int64_t g = 0; g < (int64_t)T * B; ++g) {
    const int32_t t = (int32_t)(g / B);
    const int64_t b = g % B;
    const oracle_table* tb = &tables[t];
    const int32_t D = tb->dim;
    const int32_t rb = tb->row_bytes > 0 ? tb->row_bytes : default_row_bytes(tb->dtype, D);
    float acc[4096];
    for (int32_t d = 0; d < D; ++d) acc[d] = 0.0f;
    int64_t start = offsets[g], end = offsets[g + 1];
    if (start < 0 || end < start || end > num_indices) {
      ++bad;
      start = end = 0;
    }
    int64_t count = 0;
    for (int64_t i = start; i < end; ++i) {
      const int64_t idx = index_bits == 32 ? (int64_t)((const int32_t*)indices)[i]
                                           : ((const int64_t*)indices)[i];
      if (padding_idx >= 0 && idx == padding_idx) continue;
      if (idx < 0 || idx >= tb->rows) { ++bad; continue; }
      const uint8_t* row = weights + tb->weights_offset + (size_t)idx * (size_t)rb;
      for (int32_t d = 0; d < D; ++d) acc[d] += decode(row, tb->dtype, d);
      ++count;
    }
    if (tb->pooling == 1 && count > 0) {
      const float c = (float)count;
      for (int32_t d = 0; d < D; ++d) acc[d] = acc[d] / c;
    }
    for (int32_t d = 0; d < D; ++d)
      store_out(out, out_dtype, (size_t)b * (size_t)out_stride + (size_t)tb->out_offset + (size_t)d, acc[d]);
  }
  return bad;
}

/* ---- int8 rowwise quantizer ------------------------------------------- */

void oracle_int8_quantize(const float* src, int64_t rows, int32_t dim,
                          uint8_t* dst, int32_t row_bytes, int32_t num_threads) {
  (void)num_threads;
#pragma omp parallel for schedule(static) num_threads(num_threads > 0 ? num_threads : 1)
  for (int64_t r = 0; r < rows; ++r) {
    const float* x = src + (size_t)r * (size_t)dim;
    uint8_t* o = dst + (size_t)r * (size_t)row_bytes;
    float mn = x[0], mx = x[0];
    for (int32_t d = 1; d < dim; ++d) {
      mn = x[d] < mn ? x[d] : mn;
      mx = x[d] > mx ? x[d] : mx;
    }
    const uint16_t bias16 = oracle_f32_to_f16(mn);
    const float bias = oracle_f16_to_f32(bias16);
    const float range = mx - bias;
    uint16_t scale16 = oracle_f32_to_f16(range == 0.0f ? 1.0f : range / 255.0f);
    float scale = oracle_f16_to_f32(scale16);
    if (scale == 0.0f || isinf(1.0f / scale)) {
      scale16 = 0x3c00; /* 1.0 */
      scale = 1.0f;
    }
    const float inv = 1.0f / scale;
    memcpy(o, &scale16, 2);
    memcpy(o + 2, &bias16, 2);
    for (int32_t d = 0; d < dim; ++d) {
      volatile float diff = x[d] - bias;
      float q = rintf(diff * inv);
      q = q < 0.0f ? 0.0f : (q > 255.0f ? 255.0f : q);
      o[4 + d] = (uint8_t)q;
    }
    for (int32_t d = 4 + dim; d < row_bytes; ++d) o[d] = 0;
  }
}

/* ---- jagged -> padded sequence gather --------------------------------- */

/* tables[f]: dense [rows[f], dim[f]] of element size esize; ids[p*F+f];
 * offsets[p] = [B+1].  out [B, S, sum dim] with S = sum max_len; mask [B, S].
 * pad_mode 0 = row 0 of each table, 1 = zeros; align 0 = right (left pad),
 * 1 = left.  Returns the count of invalid ids / offsets met. */
int64_t oracle_seq_gather(int32_t P, int32_t F, int32_t esize, int64_t B,
                          const int32_t* max_len, const int32_t* dim,
                          const int64_t* rows, const uint8_t* const* tables,
                          const int64_t* const* ids,
                          const int64_t* const* offsets,
                          const int64_t* num_ids, int32_t pad_mode,
                          int32_t align, uint8_t* out, uint8_t* mask) {
  int64_t S = 0, row_elems = 0, bad = 0;
  for (int32_t p = 0; p < P; ++p) S += max_len[p];
  for (int32_t f = 0; f < F; ++f) row_elems += dim[f];
  const size_t tok_bytes = (size_t)row_elems * (size_t)esize;
  for (int64_t b = 0; b < B; ++b) {
    int64_t s0 = 0;
    for (int32_t p = 0; p < P; ++p) {
      const int64_t L = max_len[p];
      int64_t beg = offsets[p][b], end = offsets[p][b + 1];
      if (beg < 0 || end < beg || end > num_ids[p]) { ++bad; beg = end = 0; }
      const int64_t len = end - beg;
      const int64_t n = len < L ? len : L;
      for (int64_t pos = 0; pos < L; ++pos) {
        int64_t ev = -1;
        if (align == 0) {
          if (pos >= L - n) ev = end - n + (pos - (L - n));
        } else {
          if (pos < n) ev = end - n + pos;
        }
        uint8_t* tok = out + ((size_t)b * (size_t)S + (size_t)(s0 + pos)) * tok_bytes;
        if (mask) mask[b * S + s0 + pos] = (uint8_t)(ev >= 0);
        size_t col = 0;
        for (int32_t f = 0; f < F; ++f) {
          const size_t fb = (size_t)dim[f] * (size_t)esize;
          int64_t id = ev >= 0 ? ids[p * F + f][ev] : 0;
          int zero = (ev < 0 && pad_mode == 1);
          if (id < 0 || id >= rows[f]) { ++bad; zero = 1; }
          if (zero) memset(tok + col, 0, fb);
          else memcpy(tok + col, tables[f] + (size_t)id * fb, fb);
          col += fb;
        }
      }
      s0 += L;
    }
  }
  return bad;
}

/* ---- cross-feature ids (xxHash64) --------------------------------------- */

static const uint64_t XP1 = 0x9E3779B185EBCA87ull, XP2 = 0xC2B2AE3D27D4EB4Full,
                      XP3 = 0x165667B19E3779F9ull, XP4 = 0x85EBCA77C2B2AE63ull,
                      XP5 = 0x27D4EB2F165667C5ull;

static inline uint64_t xrotl(uint64_t x, int r) { return (x << r) | (x >> (64 - r)); }
static inline uint64_t xread64(const uint8_t* p) {
  uint64_t v = 0;
  for (int i = 7; i >= 0; --i) v = (v << 8) | p[i];  /* little endian */
  return v;
}
static inline uint32_t xread32(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static inline uint64_t xround(uint64_t acc, uint64_t lane) { return xrotl(acc + lane * XP2, 31) * XP1; }
static inline uint64_t xmerge(uint64_t acc, uint64_t v) { return (acc ^ xround(0, v)) * XP1 + XP4; }

/* XXH64 of len bytes at p with seed (the specification's algorithm). */
uint64_t oracle_xxh64(const uint8_t* p, size_t len, uint64_t seed) {
  const uint8_t* end = p + len;
  uint64_t acc;
  if (len >= 32) {
    uint64_t v1 = seed + XP1 + XP2, v2 = seed + XP2, v3 = seed, v4 = seed - XP1;
    const uint8_t* limit = end - 32;
    do {
      v1 = xround(v1, xread64(p));
      v2 = xround(v2, xread64(p + 8));
      v3 = xround(v3, xread64(p + 16));
      v4 = xround(v4, xread64(p + 24));
      p += 32;
    } while (p <= limit);
    acc = xrotl(v1, 1) + xrotl(v2, 7) + xrotl(v3, 12) + xrotl(v4, 18);
    acc = xmerge(acc, v1);
    acc = xmerge(acc, v2);
    acc = xmerge(acc, v3);
    acc = xmerge(acc, v4);
  } else {
    acc = seed + XP5;
  }
  acc += (uint64_t)len;
  while (p + 8 <= end) {
    acc ^= xround(0, xread64(p));
    acc = xrotl(acc, 27) * XP1 + XP4;
    p += 8;
  }
  if (p + 4 <= end) {
    acc ^= (uint64_t)xread32(p) * XP1;
    acc = xrotl(acc, 23) * XP2 + XP3;
    p += 4;
  }
  while (p < end) {
    acc ^= (uint64_t)(*p) * XP5;
    acc = xrotl(acc, 11) * XP1;
    ++p;
  }
  acc ^= acc >> 33;
  acc *= XP2;
  acc ^= acc >> 29;
  acc *= XP3;
  acc ^= acc >> 32;
  return acc;
}

/* out[i] = xxh64(pack("<nq", keys[0][i*s0], ..., keys[n-1][i*s_{n-1}]), salt) % table_size. */
void oracle_cross_hash(const int64_t* const* keys, const int64_t* strides, int32_t n_keys, int64_t n,
                       uint64_t table_size, uint64_t salt, int64_t* out) {
#pragma omp parallel for schedule(static) if (n > 65536)
  for (int64_t i = 0; i < n; ++i) {
    uint8_t buf[8 * 64];
    for (int32_t k = 0; k < n_keys; ++k) {
      uint64_t v = (uint64_t)keys[k][i * strides[k]];
      for (int b = 0; b < 8; ++b) buf[8 * k + b] = (uint8_t)(v >> (8 * b));
    }
    out[i] = (int64_t)(oracle_xxh64(buf, (size_t)(8 * n_keys), salt) % table_size);
  }
}

/* ---- pooled TBE backward + fused optimizer ---------------------------- */

/* Same field layout as the library's pdm_optim_params. */
typedef struct {
  int32_t optimizer; /* 0 Adam, 1 row-wise Adagrad, 2 gradient only */
  int32_t wd_mode;   /* row-wise Adagrad: 0 none, 1 L2 */
  float lr, eps, beta1, beta2, weight_decay;
  int32_t reserved;
  int64_t step;
} oracle_optim;

typedef struct {
  int64_t key;   /* row id: row_off[slot] + index */
  int64_t pos;   /* lookup position (tie order) */
  int64_t goff;  /* first grad element of the lookup's bag slice */
  float scale;   /* 1, or 1 / pooled count for mean */
  int32_t slot;
} bwd_entry;

static int cmp_bwd_entry(const void* pa, const void* pb) {
  const bwd_entry* a = (const bwd_entry*)pa;
  const bwd_entry* b = (const bwd_entry*)pb;
  if (a->key != b->key) return a->key < b->key ? -1 : 1;
  return a->pos < b->pos ? -1 : (a->pos > b->pos ? 1 : 0);
}

/* The gradient of each looked-up row is the sum, in lookup-position order,
 * of scale * grad[b, out_offset + d] over the row's lookups (fmaf per term);
 * padding ids and out-of-range ids contribute nothing; the mean scale is
 * 1 / (pooled ids of the bag), the derivative of the pooled mean
 * (primus_dlrm/models/sharded_embedding.py:220-227).  The optimizer is then
 * applied once per distinct row (sparse update), with the formulas of the
 * fused FBGEMM optimizers TorchRec maps the reference's choice to
 * (primus_dlrm/distributed/wrapper.py:151-174; fbgemm_gpu 2026.4.29, absent
 * here, restated from its published update rules):
 *   Adam (EmbOptimType.ADAM, the reference's default optimizer):
 *     m = b1 m + (1 - b1) g;  v = b2 v + (1 - b2) g^2
 *     w = w - lr ((m / (1 - b1^t)) / (sqrt(v / (1 - b2^t)) + eps) + wd w)
 *   row-wise Adagrad (EXACT_ROWWISE_ADAGRAD, weight_decay_mode L2 or none):
 *     g' = g + wd w (L2);  G = G + mean_d(g'^2)
 *     mu = lr / (sqrt(G) + eps);  w = (1 - mu wd) w - mu g   (L2)
 *                                 w = w - mu g              (none)
 * row_off[t]: row id of row 0 of slot t's table (slots of one table share
 * it).  Adam state m1/m2 is laid out like the fp32 weights; row-wise state
 * m1 is indexed by row id.  ids_out / grads_out (optional; rows of
 * grads_stride floats) receive the distinct row ids, ascending, and their
 * gradients.  Returns the
 * number of distinct rows; *bad counts skipped entries (out-of-range ids,
 * bags with malformed offsets).  entries is scratch of num_indices. */
int64_t oracle_tbe_backward(const oracle_table* tables, const int64_t* row_off, int32_t T, int64_t B,
                            const void* indices, int32_t index_bits, int64_t num_indices,
                            const int64_t* offsets, int64_t padding_idx, const float* grad, int64_t grad_stride,
                            int64_t* ids_out, float* grads_out, int32_t grads_stride, const oracle_optim* opt,
                            float* weights,
                            float* m1, float* m2, bwd_entry* entries, int64_t* bad) {
  int64_t n = 0, nbad = 0;
  for (int64_t g = 0; g < (int64_t)T * B; ++g) {
    const int32_t t = (int32_t)(g / B);
    const int64_t b = g % B;
    const oracle_table* tb = &tables[t];
    const int64_t start = offsets[g], end = offsets[g + 1];
    if (start < 0 || end < start || end > num_indices) {
      ++nbad;
      continue;
    }
    int64_t count = 0;
    for (int64_t i = start; i < end; ++i) {
      const int64_t idx = index_bits == 32 ? (int64_t)((const int32_t*)indices)[i] : ((const int64_t*)indices)[i];
      if (padding_idx >= 0 && idx == padding_idx) continue;
      if (idx < 0 || idx >= tb->rows) {
        ++nbad;
        continue;
      }
      ++count;
    }
    const float scale = tb->pooling == 1 ? 1.0f / (float)count : 1.0f;
    for (int64_t i = start; i < end; ++i) {
      const int64_t idx = index_bits == 32 ? (int64_t)((const int32_t*)indices)[i] : ((const int64_t*)indices)[i];
      if ((padding_idx >= 0 && idx == padding_idx) || idx < 0 || idx >= tb->rows) continue;
      bwd_entry e = {row_off[t] + idx, i, b * grad_stride + tb->out_offset, scale, t};
      entries[n++] = e;
    }
  }
  if (bad) *bad = nbad;
  qsort(entries, (size_t)n, sizeof(bwd_entry), cmp_bwd_entry);
  int64_t u = 0;
  float gsum[4096];
  for (int64_t i = 0; i < n;) {
    int64_t j = i;
    const oracle_table* tb = &tables[entries[i].slot];
    const int32_t D = tb->dim;
    for (int32_t d = 0; d < D; ++d) gsum[d] = 0.0f;
    for (; j < n && entries[j].key == entries[i].key; ++j)
      for (int32_t d = 0; d < D; ++d) gsum[d] = fmaf(entries[j].scale, grad[entries[j].goff + d], gsum[d]);
    const int64_t key = entries[i].key;
    if (ids_out) ids_out[u] = key;
    if (grads_out)
      for (int32_t d = 0; d < D; ++d) grads_out[u * grads_stride + d] = gsum[d];
    if (opt && opt->optimizer != 2) {
      const int64_t e0 = tb->weights_offset / 4 + (key - row_off[entries[i].slot]) * D;
      float* w = weights + e0;
      if (opt->optimizer == 0) {
        const float b1 = opt->beta1, b2 = opt->beta2, omb1 = 1.0f - b1, omb2 = 1.0f - b2;
        const float bc1 = 1.0f - powf(b1, (float)opt->step), bc2 = 1.0f - powf(b2, (float)opt->step);
        float* m = m1 + e0;
        float* v = m2 + e0;
        for (int32_t d = 0; d < D; ++d) {
          const float g = gsum[d];
          m[d] = fmaf(g, omb1, m[d] * b1);
          v[d] = fmaf(g * g, omb2, v[d] * b2);
          w[d] = w[d] - opt->lr * ((m[d] / bc1) / (sqrtf(v[d] / bc2) + opt->eps) + opt->weight_decay * w[d]);
        }
      } else {
        const int l2 = opt->wd_mode == 1;
        float ss = 0.0f;
        for (int32_t d = 0; d < D; ++d) {
          const float gg = l2 ? gsum[d] + opt->weight_decay * w[d] : gsum[d];
          ss += gg * gg;
        }
        const float state = m1[key] + ss / (float)D;
        const float mult = opt->lr / (sqrtf(state) + opt->eps);
        const float corr = l2 ? 1.0f - mult * opt->weight_decay : 1.0f;
        for (int32_t d = 0; d < D; ++d) w[d] = corr * w[d] - mult * gsum[d];
        m1[key] = state;
      }
    }
    ++u;
    i = j;
  }
  return u;
}
