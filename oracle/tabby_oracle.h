/*
 * CPU oracle for the token-sampling path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this.
 * The product path (tabby_amd/) never calls it; it is the checker, not the thing shipped.
 *
 * It restates the semantics of the reference CPU sampler, function by function:
 *   tabby_oracle_mulberry32     <- src/engine/sampler.ts:105-119 (SeededRandom),
 *                                  tests/support.ts:7-16 (rng)
 *   tabby_oracle_exp            <- V8's Math.exp, which sampler.ts:156,170 call; V8 implements it
 *                                  with the Sun fdlibm e_exp.c method (see tabby_oracle.c)
 *   tabby_oracle_argmax         <- src/engine/sampler.ts:13-23
 *   tabby_oracle_topk           <- src/engine/sampler.ts:25-30 (value desc, id asc)
 *   tabby_oracle_sum_exp        <- tests/sampling.test.ts:73-77 (f64 sum in index order)
 *   tabby_oracle_sample_from_topk <- src/engine/sampler.ts:147-212 (sampleFromTopK)
 *   tabby_oracle_sample_row     <- encodeSampling (src/engine/forward.ts:522-601) followed by
 *                                  sampleFromTopK (src/worker/inference.worker.ts:162-168),
 *                                  with top_k = 0 meaning the whole vocabulary
 *   tabby_oracle_f16_to_f32     <- tests/support.ts:67-74 (exact widening)
 *   tabby_oracle_softmax_rows   <- src/reference/cpu.ts:238-264 (softmaxRows: f32 steps,
 *                                  Math.exp, causal prefix)
 *   tabby_oracle_matmul_quantized <- src/reference/cpu.ts:352-393 (matmulQuantized: the
 *                                  lm_head's block-quantized matmul, f32 steps)
 */
#ifndef TABBY_ORACLE_H
#define TABBY_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
  int32_t id;
  uint32_t considered;
  double probability;
  double pool_mass;
  int32_t pool_exhausted;
  int32_t status; /* 0 ok, nonzero: row out of contract (non-finite max, empty pool) */
} tabby_oracle_outcome;

/* Advances *state once and returns u in [0,1) (u32 / 2^32, exact in f64). */
double tabby_oracle_mulberry32(uint32_t *state);
/* Fills out[0..n) with consecutive draws from a generator seeded with `seed`. */
void tabby_oracle_mulberry32_fill(uint32_t seed, double *out, int64_t n);

double tabby_oracle_exp(double x);

float tabby_oracle_f16_to_f32(uint16_t bits);

int32_t tabby_oracle_argmax(const float *row, int32_t n);

/* Exact top-k; writes min(k, n) entries. Returns the count written. */
int32_t tabby_oracle_topk(const float *row, int32_t n, int32_t k, int32_t *ids, float *values);

/* sum_i exp(row[i] - max) in index order, f64. */
double tabby_oracle_sum_exp(const float *row, int32_t n, float max_logit);

/* sampleFromTopK over `count` candidates (ids/logits highest first). */
int tabby_oracle_sample_from_topk(const int32_t *ids, const float *logits, int32_t count,
                                  double max_logit, double sum_exp, double temperature,
                                  double top_p, double uniform, tabby_oracle_outcome *out);

/*
 * Whole-row composition. top_k = 0 (or >= n) uses every entry of the row. When topk_ids /
 * topk_values are non-null they receive the first min(k_eff, topk_cap) sorted candidates.
 * *max_out / *sum_exp_out (if non-null) receive maxLogit and the f64 sumExp.
 */
int tabby_oracle_sample_row(const float *row, int32_t n, int32_t top_k, double temperature,
                            double top_p, double uniform, tabby_oracle_outcome *out,
                            int32_t *topk_ids, float *topk_values, int32_t topk_cap,
                            float *max_out, double *sum_exp_out);

/* Batched form over rows of a row-major [rows, n] f32 matrix, one thread per call. */
int tabby_oracle_sample_batch(const float *logits, int32_t rows, int32_t n,
                              const int32_t *top_k, const double *temperature,
                              const double *top_p, const double *uniform,
                              tabby_oracle_outcome *out);

/* softmaxRows over [n_rows, row_len] f32; out may equal x. */
void tabby_oracle_softmax_rows(const float *x, float *out, int32_t n_rows, int32_t row_len,
                               int32_t causal_period, int32_t causal_offset);

/* matmulQuantized over n_tokens rows of x [n_tokens, in_dim]; y [n_tokens, out_dim];
 * bias may be NULL; bits 4 or 8. */
void tabby_oracle_matmul_quantized(const uint32_t *words, const float *scales, const float *x,
                                   int32_t n_tokens, int32_t out_dim, int32_t in_dim,
                                   int32_t bits, int32_t block_size, const float *bias,
                                   float *y);

#ifdef __cplusplus
}
#endif

#endif
