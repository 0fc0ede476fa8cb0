/*
 * pa_oracle.c -- float64 CPU oracle of paged GQA decode attention.
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (and nothing in the product) to
 * check oracle/reference.py and, through it, the HIP kernels.
 *
 * An independent second restatement of the reference's algorithm
 * (ParamThakkar123/paged-decode-attention) that shares no code with the torch
 * oracle: it walks the block table page by page instead of gathering, decodes
 * the stored bit patterns itself instead of calling torch casts, and works in
 * double precision throughout.
 *
 *   dequant            pagedattn/cache.py:51-62  (e5m2 -> fp16 exact; int8 ->
 *                      fp16(int8 * scale), product formed in the scale's type;
 *                      bf16 -> fp16 rounded to nearest even)
 *   pa_oracle_decode   pagedattn/reference.py:28-49 (softmax(q.K^T * scale) V
 *                      over positions [0, seq_len), kv head = q head / group)
 *   pa_oracle_split    pagedattn/triton_decode.py:78-85 (split ranges) and
 *                      :169-188 (normalised partial, log2-sum-exp, empty = -inf)
 *
 * Every buffer is dense and row-major:
 *   q    [B, Hq, D]           fp16 bits
 *   k, v [NB, P, Hkv, D]      fp16 bits | e5m2 bytes | int8
 *   ks,vs[NB, P, Hkv]         fp16 bits | fp32 (int8 only, else NULL)
 *   bt   [B, max_blocks]      int32
 *   out  [B, Hq, D]           double
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { KV_FP16 = 0, KV_FP8_E5M2 = 1, KV_INT8 = 2, KV_BF16 = 3 };
enum { SC_NONE = 0, SC_FP16 = 1, SC_FP32 = 2 };

/* IEEE binary16: 1 sign, 5 exponent (bias 15), 10 mantissa bits. */
double pa_oracle_half_to_double(uint16_t h) {
  const int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
  double v;
  if (e == 0) {
    v = ldexp((double)m, -24);
  } else if (e == 31) {
    v = m ? NAN : INFINITY;
  } else {
    v = ldexp(1.0 + m / 1024.0, e - 15);
  }
  return s ? -v : v;
}

/* OCP fp8 e5m2: 1 sign, 5 exponent (bias 15), 2 mantissa bits. */
double pa_oracle_e5m2_to_double(uint8_t b) {
  const int s = b >> 7, e = (b >> 2) & 31, m = b & 3;
  double v;
  if (e == 0) {
    v = ldexp((double)m, -16);
  } else if (e == 31) {
    v = m ? NAN : INFINITY;
  } else {
    v = ldexp(1.0 + m / 4.0, e - 15);
  }
  return s ? -v : v;
}

/* Round a double to the nearest binary16 value, ties to even. */
double pa_oracle_round_half(double x) {
  if (x != x) return x;
  const double a = fabs(x);
  if (a >= 65520.0) return copysign(INFINITY, x);
  int e;
  frexp(a, &e); /* a = f * 2^e, f in [0.5, 1) */
  int lead = e - 1;
  if (lead < -14) lead = -14; /* subnormal spacing 2^-24 */
  const double ulp = ldexp(1.0, lead - 10);
  return copysign(nearbyint(a / ulp) * ulp, x);
}

typedef struct {
  const uint8_t *k, *v, *ks, *vs;
  const int32_t *bt, *seq_lens;
  int hkv, d, page, max_blocks, kv_dtype, scale_dtype;
} cache_t;

static double scale_at(const uint8_t *s, int dtype, int64_t idx) {
  if (dtype == SC_FP32) {
    float f;
    memcpy(&f, s + 4 * idx, 4);
    return (double)f;
  }
  uint16_t h;
  memcpy(&h, s + 2 * idx, 2);
  return pa_oracle_half_to_double(h);
}

/* Dequantised row of one (physical block, slot, kv head) into dst[d]. */
static void load_row(const cache_t *c, const uint8_t *base, const uint8_t *sbase, int blk,
                     int slot, int kvh, double *dst) {
  const int64_t row = ((int64_t)blk * c->page + slot) * c->hkv + kvh;
  if (c->kv_dtype == KV_FP16) {
    const uint8_t *p = base + row * c->d * 2;
    for (int i = 0; i < c->d; ++i) {
      uint16_t h;
      memcpy(&h, p + 2 * i, 2);
      dst[i] = pa_oracle_half_to_double(h);
    }
  } else if (c->kv_dtype == KV_BF16) {
    const uint8_t *p = base + row * c->d * 2;
    for (int i = 0; i < c->d; ++i) {
      uint16_t h;
      memcpy(&h, p + 2 * i, 2);
      const uint32_t u = (uint32_t)h << 16;
      float f;
      memcpy(&f, &u, 4);
      dst[i] = pa_oracle_round_half((double)f);
    }
  } else if (c->kv_dtype == KV_FP8_E5M2) {
    const uint8_t *p = base + row * c->d;
    for (int i = 0; i < c->d; ++i) dst[i] = pa_oracle_e5m2_to_double(p[i]);
  } else {
    const int8_t *p = (const int8_t *)(base + row * c->d);
    const double s = scale_at(sbase, c->scale_dtype, row);
    for (int i = 0; i < c->d; ++i) {
      double prod = (double)p[i] * s;
      if (c->scale_dtype == SC_FP32) prod = (double)(float)prod; /* fp32 multiply */
      dst[i] = pa_oracle_round_half(prod);
    }
  }
}

static int physical_block(const cache_t *c, int b, int pos) {
  return c->bt[(int64_t)b * c->max_blocks + pos / c->page];
}

/* softmax(q.K^T * sm_scale) V over tokens [lo, hi) of sequence b for one head.
 * Writes the normalised output to out[d] and returns the natural-log sum-exp
 * (-inf for an empty range, out = 0 then). */
static double attend(const cache_t *c, const double *q, int b, int kvh, int lo, int hi,
                     double sm_scale, double *out, double *krow, double *logits) {
  const int n = hi - lo;
  for (int i = 0; i < c->d; ++i) out[i] = 0.0;
  if (n <= 0) return -INFINITY;
  double m = -INFINITY;
  for (int t = 0; t < n; ++t) {
    const int pos = lo + t;
    load_row(c, c->k, c->ks, physical_block(c, b, pos), pos % c->page, kvh, krow);
    double dot = 0.0;
    for (int i = 0; i < c->d; ++i) dot += q[i] * krow[i];
    logits[t] = dot * sm_scale;
    if (logits[t] > m) m = logits[t];
  }
  double den = 0.0;
  for (int t = 0; t < n; ++t) {
    const double p = exp(logits[t] - m);
    den += p;
    const int pos = lo + t;
    load_row(c, c->v, c->vs, physical_block(c, b, pos), pos % c->page, kvh, krow);
    for (int i = 0; i < c->d; ++i) out[i] += p * krow[i];
  }
  for (int i = 0; i < c->d; ++i) out[i] /= den;
  return m + log(den);
}

static void load_q(const uint16_t *q, int64_t off, int d, double *dst) {
  for (int i = 0; i < d; ++i) dst[i] = pa_oracle_half_to_double(q[off + i]);
}

/* Returns 0, or -1 on a bad argument / allocation failure. A sequence with
 * seq_len 0 gives NaN (0/0), as the reference does. */
int pa_oracle_decode(const uint16_t *q, const void *k, const void *v, const void *ks,
                     const void *vs, const int32_t *bt, const int32_t *seq_lens, int batch,
                     int hq, int hkv, int d, int page, int max_blocks, int kv_dtype,
                     int scale_dtype, double sm_scale, double *out) {
  if (batch < 0 || hq <= 0 || hkv <= 0 || hq % hkv || d <= 0 || page <= 0) return -1;
  cache_t c = {(const uint8_t *)k, (const uint8_t *)v, (const uint8_t *)ks,
               (const uint8_t *)vs, bt, seq_lens, hkv, d, page, max_blocks, kv_dtype,
               scale_dtype};
  const int group = hq / hkv;
  int smax = 1;
  for (int b = 0; b < batch; ++b)
    if (seq_lens[b] > smax) smax = seq_lens[b];
  double *qrow = malloc(sizeof(double) * d);
  double *krow = malloc(sizeof(double) * d);
  double *logits = malloc(sizeof(double) * smax);
  if (!qrow || !krow || !logits) {
    free(qrow), free(krow), free(logits);
    return -1;
  }
  for (int b = 0; b < batch; ++b) {
    for (int h = 0; h < hq; ++h) {
      double *o = out + ((int64_t)b * hq + h) * d;
      load_q(q, ((int64_t)b * hq + h) * d, d, qrow);
      if (seq_lens[b] <= 0) {
        for (int i = 0; i < d; ++i) o[i] = NAN;
        continue;
      }
      attend(&c, qrow, b, h / group, 0, seq_lens[b], sm_scale, o, krow, logits);
    }
  }
  free(qrow), free(krow), free(logits);
  return 0;
}

/* Per-split partials: part [B, Hq, S, D] (normalised output of the split) and
 * lse2 [B, Hq, S] = log2 of the split's sum of exp2(q.k * sm_scale * log2 e).
 * Split s covers [s*chunk, min((s+1)*chunk, T)), chunk = ceil(ceil(T/align)/S)*align,
 * or, with max_seq_len > 0, the larger of that and the chunk of max_seq_len. */
int pa_oracle_split(const uint16_t *q, const void *k, const void *v, const void *ks,
                    const void *vs, const int32_t *bt, const int32_t *seq_lens, int batch,
                    int hq, int hkv, int d, int page, int max_blocks, int kv_dtype,
                    int scale_dtype, double sm_scale, int num_splits, int align,
                    int max_seq_len, double *part, double *lse2) {
  if (batch < 0 || hq <= 0 || hkv <= 0 || hq % hkv || d <= 0 || page <= 0 || num_splits < 1 ||
      align < 1)
    return -1;
  cache_t c = {(const uint8_t *)k, (const uint8_t *)v, (const uint8_t *)ks,
               (const uint8_t *)vs, bt, seq_lens, hkv, d, page, max_blocks, kv_dtype,
               scale_dtype};
  const int group = hq / hkv;
  int smax = 1;
  for (int b = 0; b < batch; ++b)
    if (seq_lens[b] > smax) smax = seq_lens[b];
  double *qrow = malloc(sizeof(double) * d);
  double *krow = malloc(sizeof(double) * d);
  double *logits = malloc(sizeof(double) * smax);
  if (!qrow || !krow || !logits) {
    free(qrow), free(krow), free(logits);
    return -1;
  }
  for (int b = 0; b < batch; ++b) {
    const int T = seq_lens[b] > 0 ? seq_lens[b] : 0;
    const int64_t tiles = (T + align - 1) / align;
    int64_t chunk = ((tiles + num_splits - 1) / num_splits) * align;
    if (max_seq_len > 0) { /* balanced mode: the longest sequence's chunk, never less than own */
      const int64_t longest = ((int64_t)max_seq_len + align - 1) / align;
      const int64_t c2 = ((longest + num_splits - 1) / num_splits) * align;
      if (c2 > chunk) chunk = c2;
    }
    for (int h = 0; h < hq; ++h) {
      load_q(q, ((int64_t)b * hq + h) * d, d, qrow);
      for (int s = 0; s < num_splits; ++s) {
        int64_t lo = s * chunk, hi = lo + chunk;
        if (lo > T) lo = T;
        if (hi > T) hi = T;
        const int64_t idx = ((int64_t)b * hq + h) * num_splits + s;
        const double lse = attend(&c, qrow, b, h / group, (int)lo, (int)(lo < hi ? hi : lo),
                                  sm_scale, part + idx * d, krow, logits);
        lse2[idx] = lse / log(2.0);
      }
    }
  }
  free(qrow), free(krow), free(logits);
  return 0;
}
