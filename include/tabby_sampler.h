/*
 * tabby_sampler -- C ABI of the MI355X (gfx950) token sampler.
 *
 * For each row of logits it computes, in one stream-ordered launch sequence:
 *   maxLogit, sumExp = sum exp(x - maxLogit) over the whole row, the exact top-k
 *   (value descending, ties to the lower index), and then sampleFromTopK's temperature /
 *   top-p / categorical draw from a caller-supplied uniform.
 *
 * It replaces, in the reference (xOAviOx/tabby):
 *   - ForwardPass.encodeSampling            src/engine/forward.ts:522-601   (GPU head)
 *   - the sample-block readback + decode    src/engine/forward.ts:142-157, 442-451
 *   - sampleFromTopK                        src/engine/sampler.ts:147-212   (CPU tail)
 * composed as the worker does (src/worker/inference.worker.ts:162-168), for many rows at once.
 *
 * Conventions: plain C types only; every function returns a tabby_status; device pointers
 * are owned by the caller, scratch is owned by the handle; one handle per host thread and
 * stream (calls on one handle must not overlap). tabby_last_error() gives the message of
 * the calling thread's most recent failure.
 */
#ifndef TABBY_SAMPLER_H
#define TABBY_SAMPLER_H

#include <stdint.h>

#if defined(__GNUC__)
#define TABBY_API __attribute__((visibility("default")))
#else
#define TABBY_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  TABBY_OK = 0,
  TABBY_EINVAL = 1,    /* bad argument; e.g. topK outside [0, k_max] (forward.ts:348-351) */
  TABBY_EHIP = 2,      /* HIP runtime / launch failure */
  TABBY_EEMPTY = 3,    /* empty candidate pool (sampler.ts:153) */
  TABBY_EDOMAIN = 4,   /* row outside the contract: NaN, +inf, or every entry -inf */
  TABBY_ECAPACITY = 5  /* request exceeds what the handle was created for */
} tabby_status;

typedef enum { TABBY_F32 = 0, TABBY_F16 = 1 } tabby_dtype;

/* Per-row sampling parameters: SamplingParams (sampler.ts:83-98) plus the uniform that
 * SeededRandom.next() (sampler.ts:112-118) would return for this row. All f64, as JS
 * numbers are: 0.9 as f32 is not 0.9, and a mulberry32 draw has 32 significant bits. */
typedef struct {
  double temperature; /* <= 0 (-0, -inf included): greedy, the uniform is not used
                         (sampler.ts:159-167); NaN and +inf are refused (TABBY_EINVAL) */
  double top_p;       /* any value, as sampler.ts:177-186 takes it: >= 1 or NaN, no nucleus
                         cut; <= 0 keeps the first candidate */
  double uniform;     /* in [0, 1) */
  int32_t top_k;      /* 1..k_max candidates; 0 = the whole vocabulary */
  int32_t reserved;   /* must be 0 */
} tabby_row_params;

/* Per-row result: SampleOutcome (sampler.ts:121-135) plus the TopKResult header
 * (forward.ts:93-103). */
typedef struct {
  int32_t id;            /* chosen token id */
  uint32_t considered;   /* consideredCount: candidates that survived top-p */
  double probability;    /* exp(l - maxLogit) / sumExp of the chosen id */
  double pool_mass;      /* full-vocabulary mass of the k candidates */
  float max_logit;       /* largest logit of the row */
  int32_t pool_exhausted;/* 1 when poolMass < topP (top-p clipped by k) */
  double sum_exp;        /* sum over the row of exp(x - maxLogit) */
  int32_t status;        /* tabby_status of this row */
  int32_t topk_count;    /* entries written to the row's top-k output, if requested */
} tabby_row_result;

typedef struct tabby_sampler tabby_sampler;

/* Allocates the scratch a ForwardPass allocates for sampling (forward.ts:243-248), sized
 * for up to rows_max rows of up to vocab_max entries and top_k up to k_max (<= 1024).
 * `device` is a HIP device ordinal. */
TABBY_API int tabby_sampler_create(int device, int32_t vocab_max, int32_t rows_max, int32_t k_max,
                         tabby_sampler **out);

/* Frees the handle's scratch (ForwardPass.destroy, forward.ts:309-315). NULL is a no-op. */
TABBY_API int tabby_sampler_destroy(tabby_sampler *sampler);

/*
 * Device-resident form: logits_dev is [rows, vocab] row-major of `dtype`; params_dev and
 * results_dev have `rows` entries in device memory. If topk_cap > 0, topk_ids_dev and
 * topk_logits_dev ([rows, topk_cap]) receive each row's candidates, highest first (the
 * TopKResult ids/logits, forward.ts:93-103). Asynchronous on `stream` (a hipStream_t, NULL
 * for the default stream). Parameters are validated on the device: a bad row gets a
 * nonzero status and the other rows are still sampled.
 * `flags`: TABBY_FLAG_FULL_VOCAB must be set if any row may have top_k = 0 (or >= vocab)
 * with vocab above the pool capacity; such a row's pool is the whole vocabulary, and its
 * top-k output holds the first min(topk_cap, vocab) entries of it (topk_cap <= k_max).
 */
#define TABBY_FLAG_FULL_VOCAB 1u
TABBY_API int tabby_sampler_sample_device(tabby_sampler *sampler, const void *logits_dev, int32_t dtype,
                                int32_t rows, int32_t vocab, const tabby_row_params *params_dev,
                                tabby_row_result *results_dev, int32_t *topk_ids_dev,
                                float *topk_logits_dev, int32_t topk_cap, uint32_t flags,
                                void *stream);

/*
 * Host-parameter form, the decode-loop entry (forward.ts:430-451 + inference.worker.ts:162-168):
 * params_host are validated before any GPU work (TABBY_EINVAL with the reference's
 * "topK must be between 0 and <k_max>, got <k>" message), uploaded, sampled, and
 * results_host (and the optional top-k arrays, host memory) are filled when it returns.
 * Returns the first nonzero row status, if any.
 */
TABBY_API int tabby_sampler_sample(tabby_sampler *sampler, const void *logits_dev, int32_t dtype,
                         int32_t rows, int32_t vocab, const tabby_row_params *params_host,
                         tabby_row_result *results_host, int32_t *topk_ids_host,
                         float *topk_logits_host, int32_t topk_cap, void *stream);

/*
 * Allocation-free form of tabby_sampler_sample_device. It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). It takes no handle and
 * calls no hipMalloc, hipFree or allocating routine; its scratch is a fixed 16 MiB array in
 * the library's device image, one per GPU, kept until the process ends (the first call on a
 * device looks up its address). The 16 MiB are taken on every device the library's code is
 * loaded on, whether or not this entry is ever called. The caller passes inputs and outputs as for
 * tabby_sampler_sample_device, with flags = 0, on the current device. Limits: k_max <= 256,
 * and rows whose pool is the whole vocabulary (top_k = 0 or >= vocab, vocab > 256) get
 * status TABBY_EINVAL; a batch whose scratch would exceed 16 MiB returns TABBY_ECAPACITY
 * (batches of the sizes of the reference's configurations need at most ~10 MiB). Calls that
 * overlap on one GPU share that scratch and race: serialise them (one stream).
 */
TABBY_API int tabby_sampler_sample_device_noalloc(const void *logits_dev, int32_t dtype, int32_t rows,
                                                  int32_t vocab, int32_t k_max,
                                                  const tabby_row_params *params_dev,
                                                  tabby_row_result *results_dev, int32_t *topk_ids_dev,
                                                  float *topk_logits_dev, int32_t topk_cap, void *stream);

/*
 * Greedy fast path: ids_dev[r] = argmax of row r (src/engine/sampler.ts:13-23: the lowest
 * index among equal maxima, +0 equal to -0, NaN never chosen; 0 when the row's first entry
 * is NaN or nothing lies above -inf), for logits_dev [rows, vocab] of `dtype` in device
 * memory. max_logits_dev (may be NULL) receives the chosen entry's value. It replaces the
 * one-candidate sampling pass the reference's greedy and profile paths make
 * (forward.runSegment with {topK: 1}, src/worker/inference.worker.ts:216-229, read back by
 * argmaxOf) and generateGreedy's host argmax (sampler.ts:54-76): one read of the logits, no
 * pool, no uniform. Uses the handle's scratch; asynchronous on `stream`.
 */
TABBY_API int tabby_argmax_device(tabby_sampler *sampler, const void *logits_dev, int32_t dtype,
                                  int32_t rows, int32_t vocab, int32_t *ids_dev,
                                  float *max_logits_dev, void *stream);
/*
 * Row softmax of attention scores, replacing the softmax_rows kernel
 * (src/shaders/softmax_rows.wgsl:1-55, dispatched at src/engine/forward.ts:912-926) with the
 * results of its CPU reference softmaxRows (src/reference/cpu.ts:238-264) bit for bit.
 * x_dev and out_dev are [n_rows, row_len] f32 in device memory; out_dev may be x_dev (in
 * place, as the reference runs it) or a buffer that does not overlap it. With
 * causal_period > 0, row r covers its first causal_offset + (r % causal_period) + 1 entries
 * and the rest of the row is written 0; causal_period = 0 softmaxes whole rows.
 * causal_offset + causal_period must not exceed row_len. Asynchronous on `stream`; no
 * scratch.
 */
TABBY_API int tabby_softmax_rows_device(const float *x_dev, float *out_dev, int32_t n_rows,
                                        int32_t row_len, int32_t causal_period,
                                        int32_t causal_offset, void *stream);
/*
 * The lm_head's int4 weights (src/engine/forward.ts:408-428, encodeQuantMatmul :732-770;
 * src/shaders/matvec_q4.wgsl), repacked once into this library's layout. Input: the
 * reference's layout (tools/convert.py): words_dev u32 [vocab][hidden / 8] (eight 4-bit
 * values per word, value j at bits 4j, dequant(q) = (q - 8) * scale) and scales_dev f16 bits
 * [vocab][hidden / block_size]. Output: packed_dev u32 [hidden / 32][vocab][4] and
 * packed_scales_dev f16 bits [hidden / block_size][vocab] (a wave's 64 output rows read
 * contiguous bytes). hidden and block_size are multiples of 32, block_size divides hidden;
 * word arrays 16-byte aligned. Asynchronous on `stream`.
 */
TABBY_API int tabby_lmhead_q4_pack_device(const uint32_t *words_dev, const uint16_t *scales_dev,
                                          int32_t vocab, int32_t hidden, int32_t block_size,
                                          uint32_t *packed_dev, uint16_t *packed_scales_dev,
                                          void *stream);
/*
 * The lm_head matmul on its own (matvec_q4.wgsl's contract): logits_dev [rows][vocab] f32 =
 * hidden_dev [rows][hidden] f32 times the packed weights (+ bias_dev [vocab], may be NULL),
 * bit for bit the CPU reference matmulQuantized (src/reference/cpu.ts:352-393). Any number of
 * rows (weights re-read per eight rows). Asynchronous on `stream`.
 */
TABBY_API int tabby_lmhead_q4_device(const uint32_t *packed_dev, const uint16_t *packed_scales_dev,
                                     const float *bias_dev, const float *hidden_dev, int32_t rows,
                                     int32_t vocab, int32_t hidden, int32_t block_size,
                                     float *logits_dev, void *stream);
/*
 * The lm_head fused with sampling: for each of `rows` (1..8) hidden states, the logits of
 * tabby_lmhead_q4_device are computed and sampled without being written to memory -- the
 * composition of the reference's lm_head (forward.ts:408-428), encodeSampling
 * (forward.ts:522-601) and sampleFromTopK (sampler.ts:147-212) in one pass over the weights.
 * params_dev / results_dev as for tabby_sampler_sample_device. Pools of at most 64 (the
 * reference's topK bound, forward.ts:348-351; top_k 0 or above 64 gives the row TABBY_EINVAL);
 * no top-k lists. Uses the handle's scratch (vocab <= vocab_max, rows <= rows_max).
 * Asynchronous on `stream`.
 */
TABBY_API int tabby_sampler_sample_lmhead_q4_device(tabby_sampler *sampler, const uint32_t *packed_dev,
                                                    const uint16_t *packed_scales_dev,
                                                    const float *bias_dev, const float *hidden_dev,
                                                    int32_t rows, int32_t vocab, int32_t hidden,
                                                    int32_t block_size,
                                                    const tabby_row_params *params_dev,
                                                    tabby_row_result *results_dev, void *stream);
/* Message of the calling thread's last failure ("" if none). */
TABBY_API const char *tabby_last_error(void);

/* Library version string. */
TABBY_API const char *tabby_version(void);

/*
 * Diagnostic: y[i] = exp(x[i]) over device arrays with the device's f64 exp, the fdlibm
 * method that V8's Math.exp uses (the exp of sampler.ts:156,170). For parity tests.
 */
TABBY_API int tabby_debug_exp(const double *x_dev, double *y_dev, int64_t n, void *stream);

/*
 * Diagnostic: y[i] = fround(Math.exp(x[i])) for x[i] <= 0 (or NaN), the f32 exps of the row
 * softmax (src/reference/cpu.ts:253), as tabby_softmax_rows_device computes them. For
 * parity tests.
 */
TABBY_API int tabby_debug_exp_f32(const float *x_dev, float *y_dev, int64_t n, void *stream);
/*
 * Diagnostic: the device's bit-exact sequential f64 sum (the left-to-right sums of
 * sampler.ts:156-203: poolMass, the scaled total, the running sums), computed in parallel by
 * one wave. terms_dev[0..n) must be >= 0 with terms_dev[0] > 0; prefix_dev[j] receives the
 * j-th partial sum up to the first that is >= stop_at (INFINITY: none), and *count_dev the
 * number of partial sums written. wide = 1 selects the form used for long sums (16 terms per
 * lane per step), wide = 2 the same taken by a four-wave workgroup, wide = 3 by an eight-wave
 * workgroup (the form that finishes whole-vocabulary heads), wide = 4 the register form for
 * n <= 64 (term i in lane i: the form that finishes pools of at most 64). prefix_dev may be terms_dev
 * itself (the sums are then written over their terms, as whole-vocabulary heads run them).
 * For parity tests.
 */
TABBY_API int tabby_debug_seq_sum(const double *terms_dev, int32_t n, double stop_at,
                                  double *prefix_dev, int32_t *count_dev, int32_t wide,
                                  void *stream);

/*
 * Diagnostic: the draw of sampleFromTopK (sampler.ts:195-203) as whole-vocabulary rows run
 * it, a 64-ary search by one wave: for each of the m targets, out_dev[j] = the first i in
 * [0, n) with targets_dev[j] < c_dev[i] (c non-decreasing), or n - 1 when there is none.
 * For parity tests.
 */
TABBY_API int tabby_debug_first_above(const double *c_dev, int32_t n, const double *targets_dev,
                                      int32_t m, int32_t *out_dev, void *stream);
/*
 * Diagnostic with no counterpart in the reference, for measurements (bench.py
 * --read-ceiling and the FETCH_SIZE calibration): reads src_dev ([rows, row_floats] f32,
 * 16-byte aligned, row_floats a multiple of 4) once with the sampling kernels' 16-byte
 * nontemporal loads in their launch shape (one 1,024-lane workgroup per row) and does nothing
 * else with it -- the read ceiling of those bytes on this GPU, and a kernel whose FETCH_SIZE
 * per dispatch must equal a known byte count. sink_dev ([rows] u32) is almost never written.
 */
TABBY_API int tabby_debug_stream_read(const float *src_dev, int32_t rows, int64_t row_floats,
                                      uint32_t *sink_dev, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TABBY_SAMPLER_H */
