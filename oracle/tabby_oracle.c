/*
 * CPU oracle for the token-sampling path -- TEST INFRASTRUCTURE ONLY (see tabby_oracle.h).
 *
 * Parity status of each function (what pins it, beyond this file):
 *   mulberry32      closed form; checked against the Node restatement (V8 integer semantics)
 *                   on >= 1e6 outputs per seed in tests/test_oracle.py
 *   exp             bit-for-bit against V8's Math.exp: 6,000 committed vectors and 1e6 live
 *                   arguments; within 1 ulp of glibc's exp
 *   argmax / topk   brute force over every tie-heavy tiny row (values -inf, -1, -0, 0, .5, 1;
 *                   lengths 1-5), numpy's stable argsort on large rows, special cases (all
 *                   equal, all -inf, +-0)
 *   sum_exp         definition (sequential f64 sum), checked against math.fsum
 *   sample_from_topk  closed forms on the reference's hand fixture
 *                   (tests/sampling.test.ts:206-250), inverse-CDF counting over a u grid,
 *                   shift invariance, and the Node restatement on committed and live rows
 * tests/test_oracle_mutants.py builds broken copies of this file (a flipped comparison, a
 * dropped term, a wrong constant) and requires these pins to reject every one.
 * Built with -ffp-contract=off: every f64 operation below must round exactly once, in the
 * order written, as V8 evaluates the reference's JavaScript.
 */
#include "tabby_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------------------
 * mulberry32 -- src/engine/sampler.ts:105-119. u32 wrap-around arithmetic throughout;
 * Math.imul is the low 32 bits of the product, `>>> 0` reinterprets as unsigned.
 * ------------------------------------------------------------------------------------- */
double tabby_oracle_mulberry32(uint32_t *state) {
  uint32_t s = *state + 0x6d2b79f5u;
  *state = s;
  uint32_t t = (s ^ (s >> 15)) * (s | 1u);
  t ^= t + (t ^ (t >> 7)) * (t | 61u);
  return (double)(t ^ (t >> 14)) / 4294967296.0;
}

void tabby_oracle_mulberry32_fill(uint32_t seed, double *out, int64_t n) {
  uint32_t state = seed;
  for (int64_t i = 0; i < n; ++i) out[i] = tabby_oracle_mulberry32(&state);
}

/* ---------------------------------------------------------------------------------------
 * exp(x) in f64, by the method of Sun's fdlibm e_exp.c (Copyright (C) 1993 Sun
 * Microsystems; freely distributable), which is what V8 ships as Math.exp (its
 * base::ieee754::exp, including the special case that returns the correctly rounded e
 * for x == 1). Reduction x = k*ln2 + r with ln2 split in a 32-bit-exact high part and a
 * low part, then a degree-5 Remez approximation R(r^2) of r*(e^r+1)/(e^r-1), then
 * exp(r) = 1 + 2r/(R - r), and a final exact scaling by 2^k.
 * ------------------------------------------------------------------------------------- */
static inline uint64_t bits_of(double x) {
  uint64_t b;
  memcpy(&b, &x, sizeof b);
  return b;
}

static inline double double_of(uint64_t b) {
  double x;
  memcpy(&x, &b, sizeof x);
  return x;
}

double tabby_oracle_exp(double x) {
  static const double kLn2Hi = 6.93147180369123816490e-01;   /* 0x3fe62e42 fee00000 */
  static const double kLn2Lo = 1.90821492927058770002e-10;   /* 0x3dea39ef 35793c76 */
  static const double kInvLn2 = 1.44269504088896338700e+00;  /* 0x3ff71547 652b82fe */
  static const double kP1 = 1.66666666666666019037e-01;
  static const double kP2 = -2.77777777770155933842e-03;
  static const double kP3 = 6.61375632143793436117e-05;
  static const double kP4 = -1.65339022054652515390e-06;
  static const double kP5 = 4.13813679705723846039e-08;
  static const double kOverflow = 7.09782712893383973096e+02;
  static const double kUnderflow = -7.45133219101941108420e+02;
  static const double kTwoM1000 = 9.33263618503218878990e-302; /* 2^-1000 */
  static const double kTwo1023 = 8.98846567431157953865e+307;  /* 2^1023 */
  static const double kE = 2.718281828459045;                  /* 0x4005bf0a 8b145769 */

  uint64_t b = bits_of(x);
  uint32_t hx = (uint32_t)(b >> 32);
  const int negative = (int)(hx >> 31);
  hx &= 0x7fffffffu;

  if (hx >= 0x40862e42u) { /* |x| >= 709.78 */
    if (hx >= 0x7ff00000u) {
      if (((hx & 0xfffffu) | (uint32_t)b) != 0) return x + x; /* NaN */
      return negative ? 0.0 : x;                               /* exp(+-inf) */
    }
    if (x > kOverflow) return INFINITY;
    if (x < kUnderflow) return 0.0;
  }

  double hi = 0.0, lo = 0.0;
  int k = 0;
  if (hx > 0x3fd62e42u) {   /* |x| > 0.5 ln2 */
    if (hx < 0x3ff0a2b2u) { /* |x| < 1.5 ln2: k = +-1 */
      if (x == 1.0) return kE;
      if (negative) {
        hi = x + kLn2Hi;
        lo = -kLn2Lo;
        k = -1;
      } else {
        hi = x - kLn2Hi;
        lo = kLn2Lo;
        k = 1;
      }
    } else {
      k = (int)(kInvLn2 * x + (negative ? -0.5 : 0.5)); /* truncation toward zero */
      const double t = (double)k;
      hi = x - t * kLn2Hi; /* exact: kLn2Hi has 32 significant bits */
      lo = t * kLn2Lo;
    }
    x = hi - lo;
  } else if (hx < 0x3e300000u) { /* |x| < 2^-28 */
    return 1.0 + x;
  }

  const double t = x * x;
  const double c = x - t * (kP1 + t * (kP2 + t * (kP3 + t * (kP4 + t * kP5))));
  if (k == 0) return 1.0 - ((x * c) / (c - 2.0) - x);
  const double y = 1.0 - ((lo - (x * c) / (2.0 - c)) - hi);
  if (k >= -1021) {
    if (k == 1024) return y * 2.0 * kTwo1023;
    return y * double_of((uint64_t)(0x3ff00000u + ((uint32_t)k << 20)) << 32);
  }
  return y * double_of((uint64_t)(0x3ff00000u + ((uint32_t)(k + 1000) << 20)) << 32) *
         kTwoM1000;
}

/* ---------------------------------------------------------------------------------------
 * Exact f16 -> f32 widening -- tests/support.ts:67-74.
 * ------------------------------------------------------------------------------------- */
float tabby_oracle_f16_to_f32(uint16_t bits) {
  const int negative = (bits & 0x8000) != 0;
  const int exponent = (bits >> 10) & 0x1f;
  const int mantissa = bits & 0x3ff;
  double v;
  if (exponent == 0) {
    v = ldexp((double)mantissa / 1024.0, -14);
  } else if (exponent == 31) {
    if (mantissa) return NAN;
    v = INFINITY;
  } else {
    v = ldexp(1.0 + (double)mantissa / 1024.0, exponent - 15);
  }
  return (float)(negative ? -v : v);
}

/* ---------------------------------------------------------------------------------------
 * argmax / topK -- src/engine/sampler.ts:13-30.
 * ------------------------------------------------------------------------------------- */
int32_t tabby_oracle_argmax(const float *row, int32_t n) {
  int32_t best = 0;
  float best_value = row[0];
  for (int32_t i = 1; i < n; ++i) {
    if (row[i] > best_value) { /* strict: the lowest index keeps a tie */
      best_value = row[i];
      best = i;
    }
  }
  return best;
}

typedef struct {
  float value;
  int32_t id;
} entry;

/* (b.value - a.value) || (a.id - b.id): value descending; equal values -- which includes
 * +0 vs -0 and -inf vs -inf (NaN difference in JS, equality here) -- fall back to id. */
static int entry_cmp(const void *pa, const void *pb) {
  const entry *a = (const entry *)pa;
  const entry *b = (const entry *)pb;
  if (a->value > b->value) return -1;
  if (a->value < b->value) return 1;
  return (a->id > b->id) - (a->id < b->id);
}

int32_t tabby_oracle_topk(const float *row, int32_t n, int32_t k, int32_t *ids,
                          float *values) {
  if (n <= 0 || k <= 0) return 0;
  entry *all = (entry *)malloc((size_t)n * sizeof(entry));
  if (!all) return -1;
  for (int32_t i = 0; i < n; ++i) {
    all[i].value = row[i];
    all[i].id = i;
  }
  qsort(all, (size_t)n, sizeof(entry), entry_cmp);
  const int32_t count = k < n ? k : n;
  for (int32_t i = 0; i < count; ++i) {
    if (ids) ids[i] = all[i].id;
    if (values) values[i] = all[i].value;
  }
  free(all);
  return count;
}

/* tests/sampling.test.ts:74-75: for (const value of full) sum += Math.exp(value - max). */
double tabby_oracle_sum_exp(const float *row, int32_t n, float max_logit) {
  double sum = 0.0;
  for (int32_t i = 0; i < n; ++i) sum += tabby_oracle_exp((double)row[i] - (double)max_logit);
  return sum;
}

/* ---------------------------------------------------------------------------------------
 * sampleFromTopK -- src/engine/sampler.ts:147-212, in its exact order of f64 operations.
 * ------------------------------------------------------------------------------------- */
int tabby_oracle_sample_from_topk(const int32_t *ids, const float *logits, int32_t count,
                                  double max_logit, double sum_exp, double temperature,
                                  double top_p, double uniform, tabby_oracle_outcome *out) {
  memset(out, 0, sizeof *out);
  if (count <= 0) { /* sampler.ts:153 -- 'sampleFromTopK: empty candidate set' */
    out->status = 3;
    return 3;
  }
  double *exact = (double *)malloc((size_t)count * sizeof(double));
  double *weights = (double *)malloc((size_t)count * sizeof(double));
  if (!exact || !weights) {
    free(exact);
    free(weights);
    out->status = 2;
    return 2;
  }

  /* sampler.ts:156-157 */
  for (int32_t i = 0; i < count; ++i)
    exact[i] = tabby_oracle_exp((double)logits[i] - max_logit) / sum_exp;
  double pool_mass = 0.0;
  for (int32_t i = 0; i < count; ++i) pool_mass += exact[i];

  /* sampler.ts:159-167 -- greedy; the uniform is not consumed */
  if (temperature <= 0.0) {
    out->id = ids[0];
    out->probability = exact[0];
    out->considered = 1;
    out->pool_mass = pool_mass;
    out->pool_exhausted = 0;
    free(exact);
    free(weights);
    return 0;
  }

  /* sampler.ts:170-172 */
  double scaled_total = 0.0;
  for (int32_t i = 0; i < count; ++i) {
    weights[i] = tabby_oracle_exp(((double)logits[i] - max_logit) / temperature);
  }
  for (int32_t i = 0; i < count; ++i) scaled_total += weights[i];
  for (int32_t i = 0; i < count; ++i) weights[i] = weights[i] / scaled_total;

  /* sampler.ts:175-189 */
  int32_t cut = count;
  int exhausted = 0;
  if (top_p < 1.0) {
    double cumulative = 0.0;
    for (int32_t i = 0; i < count; ++i) {
      cumulative += weights[i];
      if (cumulative >= top_p) {
        cut = i + 1;
        break;
      }
    }
    if (pool_mass < top_p) exhausted = 1;
  }

  /* sampler.ts:191-203 */
  double total = 0.0;
  for (int32_t i = 0; i < cut; ++i) total += weights[i];
  const double target = uniform * total;
  double running = 0.0;
  int32_t chosen = cut - 1;
  for (int32_t i = 0; i < cut; ++i) {
    running += weights[i];
    if (target < running) {
      chosen = i;
      break;
    }
  }

  out->id = ids[chosen];
  out->probability = exact[chosen];
  out->considered = (uint32_t)cut;
  out->pool_mass = pool_mass;
  out->pool_exhausted = exhausted;
  free(exact);
  free(weights);
  return 0;
}

/* ---------------------------------------------------------------------------------------
 * The whole path for one row: GPU head (maxLogit, sumExp, exact top-k) then the CPU tail.
 * ------------------------------------------------------------------------------------- */
int tabby_oracle_sample_row(const float *row, int32_t n, int32_t top_k, double temperature,
                            double top_p, double uniform, tabby_oracle_outcome *out,
                            int32_t *topk_ids, float *topk_values, int32_t topk_cap,
                            float *max_out, double *sum_exp_out) {
  memset(out, 0, sizeof *out);
  if (n <= 0) {
    out->status = 3;
    return 3;
  }
  for (int32_t i = 0; i < n; ++i) {
    if (isnan(row[i])) { /* NaN logits are outside the contract */
      out->status = 4;
      return 4;
    }
  }
  const int32_t k = (top_k <= 0 || top_k >= n) ? n : top_k;
  int32_t *ids = (int32_t *)malloc((size_t)k * sizeof(int32_t));
  float *vals = (float *)malloc((size_t)k * sizeof(float));
  if (!ids || !vals) {
    free(ids);
    free(vals);
    out->status = 2;
    return 2;
  }
  tabby_oracle_topk(row, n, k, ids, vals);
  const float max_logit = vals[0];
  if (!isfinite(max_logit)) { /* all -inf, or +inf present: exp(x - max) is NaN */
    free(ids);
    free(vals);
    out->status = 4;
    return 4;
  }
  const double sum_exp = tabby_oracle_sum_exp(row, n, max_logit);
  if (max_out) *max_out = max_logit;
  if (sum_exp_out) *sum_exp_out = sum_exp;
  if (topk_ids || topk_values) {
    const int32_t m = k < topk_cap ? k : topk_cap;
    for (int32_t i = 0; i < m; ++i) {
      if (topk_ids) topk_ids[i] = ids[i];
      if (topk_values) topk_values[i] = vals[i];
    }
  }
  const int rc = tabby_oracle_sample_from_topk(ids, vals, k, (double)max_logit, sum_exp,
                                               temperature, top_p, uniform, out);
  free(ids);
  free(vals);
  return rc;
}

int tabby_oracle_sample_batch(const float *logits, int32_t rows, int32_t n,
                              const int32_t *top_k, const double *temperature,
                              const double *top_p, const double *uniform,
                              tabby_oracle_outcome *out) {
  int worst = 0;
  for (int32_t r = 0; r < rows; ++r) {
    const int rc = tabby_oracle_sample_row(logits + (int64_t)r * n, n, top_k[r], temperature[r],
                                           top_p[r], uniform[r], &out[r], NULL, NULL, 0, NULL,
                                           NULL);
    if (rc && !worst) worst = rc;
  }
  return worst;
}

/* Math.max(a, b) (ECMAScript): NaN if either is NaN; +0 over -0; else the larger. */
static float js_max_f32(float a, float b) {
  if (a != a || b != b) return NAN;
  if (a == 0.0f && b == 0.0f) return (signbit(a) && signbit(b)) ? -0.0f : 0.0f;
  return a > b ? a : b;
}

/*
 * softmaxRows, src/reference/cpu.ts:238-264. The reference's f32(v) is Math.fround: each f32
 * step below is the f64 operation of two f32 values rounded to f32, written out as such.
 * out may equal x (the reference works on a copy, `out = Float32Array.from(x)`).
 */
void tabby_oracle_softmax_rows(const float *x, float *out, int32_t n_rows, int32_t row_len,
                               int32_t causal_period, int32_t causal_offset) {
  if (out != x) memcpy(out, x, (size_t)n_rows * (size_t)row_len * sizeof(float));
  for (int32_t row = 0; row < n_rows; ++row) {
    const int32_t valid =
        causal_period != 0 ? causal_offset + (row % causal_period) + 1 : row_len;
    float *o = out + (int64_t)row * row_len;
    float max_v = o[0];
    for (int32_t i = 1; i < valid; ++i) max_v = js_max_f32(max_v, o[i]);
    float sum = 0.0f;
    for (int32_t i = 0; i < valid; ++i) {
      const float d = (float)((double)o[i] - (double)max_v);
      const float e = (float)tabby_oracle_exp((double)d);
      o[i] = e;
      sum = (float)((double)sum + (double)e);
    }
    const float inv = (float)(1.0 / (double)sum);
    for (int32_t i = 0; i < valid; ++i) o[i] = (float)((double)o[i] * (double)inv);
    for (int32_t i = valid; i < row_len; ++i) o[i] = 0.0f;
  }
}

/*
 * matmulQuantized, src/reference/cpu.ts:352-393: y[t, m] = sum_k dequant(w[m, k]) * x[t, k]
 * + bias[m] with block-quantized weights (bits 4: eight values per u32 word, nibble j at bits
 * 4j, dequant(q) = (q - 8) * scale; bits 8: four signed bytes per word). Each word's partial
 * sum is taken in f32 over its values in order, then scaled by its block's scale and added to
 * the row's f32 accumulator -- the reference's order, every step rounded to f32.
 */
void tabby_oracle_matmul_quantized(const uint32_t *words, const float *scales, const float *x,
                                   int32_t n_tokens, int32_t out_dim, int32_t in_dim,
                                   int32_t bits, int32_t block_size, const float *bias,
                                   float *y) {
  const int32_t per_word = bits == 4 ? 8 : 4;
  const int32_t shift = 32 / per_word;
  const uint32_t mask = (1u << shift) - 1u;
  const int32_t words_per_row = in_dim / per_word;
  const int32_t words_per_block = block_size / per_word;
  const int32_t blocks_per_row = in_dim / block_size;
  for (int32_t t = 0; t < n_tokens; ++t) {
    const float *xt = x + (int64_t)t * in_dim;
    for (int32_t m = 0; m < out_dim; ++m) {
      const uint32_t *wrow = words + (int64_t)m * words_per_row;
      const float *srow = scales + (int64_t)m * blocks_per_row;
      float acc = 0.0f;
      for (int32_t w = 0; w < words_per_row; ++w) {
        const uint32_t word = wrow[w];
        const float scale = srow[w / words_per_block];
        const int32_t k0 = w * per_word;
        float block_sum = 0.0f;
        for (int32_t lane = 0; lane < per_word; ++lane) {
          const uint32_t raw = (word >> (lane * shift)) & mask;
          const int32_t centred = bits == 4 ? (int32_t)raw - 8 : (raw > 127 ? (int32_t)raw - 256 : (int32_t)raw);
          const float prod = (float)((double)centred * (double)xt[k0 + lane]);
          block_sum = (float)((double)block_sum + (double)prod);
        }
        acc = (float)((double)acc + (double)(float)((double)block_sum * (double)scale));
      }
      if (bias) acc = (float)((double)acc + (double)bias[m]);
      y[(int64_t)t * out_dim + m] = acc;
    }
  }
}
