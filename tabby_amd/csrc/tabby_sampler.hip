// MI355X (gfx950) token sampler: kernels and the C ABI declared in include/tabby_sampler.h.
//
// The reference (xOAviOx/tabby) computes, for one row, max and sum-exp with two two-stage
// tree reductions (src/shaders/reduce_max.wgsl, reduce_sumexp.wgsl) and the top-k with k
// rounds of a full argmax pass plus a single-workgroup select-and-mask
// (src/shaders/topk_partial.wgsl, topk_select.wgsl), orchestrated by encodeSampling
// (src/engine/forward.ts:522-601); the f64 tail runs on the CPU (src/engine/sampler.ts:147-212).
//
// Here one call samples a whole batch on the caller's stream. A batch of at least as many
// rows as the device has CUs (pools up to 256) takes one kernel, row_kernel: one workgroup
// per row, whose waves stream the row and then merge in LDS what the two kernels below
// exchange through global memory. A batch of up to half as many rows as CUs runs row_kernel
// on parts of each row (one workgroup per part) and merges the parts' lists with
// wave_merge_kernel, or, where that would give two or three parts, one workgroup per row.
// Other batches, and pools above 256, take two kernels:
//   * wave_kernel (slice_kernel for pools above 256): grid = rows x splits; each wave
//     (workgroup) owns one slice of one row and reads it from HBM exactly once with 16-byte
//     nontemporal loads into registers. From registers it keeps the slice max, the slice sum
//     of exp(x - max) (f32 terms, f64 accumulation), and a superset of the slice's top-k: every
//     element at or above a bound that never exceeds the slice's k-th largest value, held in a
//     wave-private LDS list (pruned by histogram when it fills) and written unsorted to the
//     slice's candidate region. Waves of a row share the best bound any of them has proven.
//   * merge_kernel: grid = rows; each 256-lane workgroup combines its row's slices: max,
//     sum-exp (slice sums rescaled in f64, in slice order), an exact radix select over the
//     64-bit (value key, ~index) composites -- the lower index wins ties, as in sampler.ts:28 --
//     a sort, and sampleFromTopK's f64 tail in the reference's exact order of operations
//     (sequential sums; V8's exp by the fdlibm method).
// The kernel boundary orders the first kernel's writes before the second's reads; no
// workgroup waits on another. Rows whose pool is the whole vocabulary (top_k = 0 beyond the
// pool capacity) are finished by two more kernels that collect and sort the row's head
// (see head_kernel).

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <type_traits>

#include "block_ops.h"
#include "device_math.h"
#include "loads.h"
#include "q4_gemv.h"
#include "seqsum.h"
#include "wave_ops.h"
#include "tabby_sampler.h"
#include "abi_internal.h"

// Phase timestamps of row_kernel, compiled in only for the timeline library (TABBY_TIMELINE,
// read by tabby_debug_timeline): per workgroup, kTimelineSlots 64-bit stamps, s_memtime
// (shader clock) or s_memrealtime (100 MHz). Slots 0-15: each wave's stream end; 16/24: the
// workgroup's start (shader clock / real time); 22: the first bound ready (wave 0); 29: the
// last wave's take selection done; 30: the second-to-last wave's statistics done; 17: past
// the first tail barrier, 18: the take done, 19: past the second barrier (wave 0); 20: the
// sort done; in the register tail (reg_tail), 23: the terms computed, 26: their scans, 27:
// the cut and the draw, 28: the margins checked; 21/25: the row finished (shader clock / real
// time). pool_row_kernel (pools above 256) uses slots 0-15, 16/24, 22 and 21/25 the same way,
// 17 for the barrier after the stream, 23 for the selection's key passes done, 18 for the
// selection done, 19 for the pool gathered, 20 for the pool sorted, and records its candidate
// count in slot 31, its key passes in slot 26, where it ran in slot 30 and whether it took
// its candidates again at the certain first bound in slot 29 (TABBY_RECORD).
#ifdef TABBY_TIMELINE
namespace tabby {
constexpr int kTimelineSlots = 32;
constexpr int kTimelineGroups = 1024;
__device__ unsigned long long g_timeline[kTimelineGroups * kTimelineSlots];
}  // namespace tabby
#define TABBY_STAMP(slot)                                                                        \
  do {                                                                                           \
    if (wave_lane() == 0 && blockIdx.x < kTimelineGroups)                                        \
      g_timeline[(size_t)blockIdx.x * kTimelineSlots + (slot)] = __builtin_amdgcn_s_memtime();   \
  } while (0)
#define TABBY_STAMP_REAL(slot)                                                                   \
  do {                                                                                           \
    if (wave_lane() == 0 && blockIdx.x < kTimelineGroups)                                        \
      g_timeline[(size_t)blockIdx.x * kTimelineSlots + (slot)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#define TABBY_RECORD(slot, value)                                                                \
  do {                                                                                           \
    if (wave_lane() == 0 && blockIdx.x < kTimelineGroups)                                        \
      g_timeline[(size_t)blockIdx.x * kTimelineSlots + (slot)] = (unsigned long long)(value);    \
  } while (0)
#else
#define TABBY_RECORD(slot, value) \
  do {                            \
  } while (0)
#define TABBY_STAMP(slot) \
  do {                    \
  } while (0)
#define TABBY_STAMP_REAL(slot) \
  do {                         \
  } while (0)
#endif

namespace tabby {

constexpr float kLog2e = 1.44269504088896340736f;
constexpr int kMaxSplits = kBlock;  // one merge lane per slice

// A lane's sum-exp is kept as the sum of 2^(x*L - ml) (L = kLog2e) against its own
// reference ml = fl(lane_max * L). Rebased on a max m it is sum * 2^(ml - m*L), with m*L
// formed exactly in f64 (two 24-bit significands): the exponent difference has no error
// proportional to |m|, so the sum's accuracy does not depend on where the logits sit.
__device__ __forceinline__ double rebase_sum(double sum, float lane_max, float ml, float m) {
  if (lane_max == -INFINITY) return 0.0;
  const double d = (double)ml - (double)m * (double)kLog2e;
  return sum * (double)__builtin_amdgcn_exp2f((float)d);
}
constexpr int kKcapSmall = 256;
constexpr int kKcapLarge = 1024;

struct SliceStat {
  float max;      // slice max (f32, exact)
  uint32_t count; // candidates written
  double sum;     // sum over the slice of exp(x - max)
};
// SliceStat.count of a row that pool_row_kernel ended itself (sampled, or its status written):
// merge_kernel skips the row.
constexpr uint32_t kPoolRowDone = 0xffffffffu;

// Per-row hand-over from the sampling kernel to the head kernel (whole-vocabulary rows).
struct RowState {
  float max;
  uint32_t head_key;  // elements with key >= head_key form the row's head
  double sum_exp;
  int32_t status;
  uint32_t handoff;   // bits 16..: length N of the row's sorted top list in head_sorted (0: none);
                      // bit 0: head_fast_kernel finished the row
  double list_sum;    // T > 0: the sequential sum of the list's terms exp((l_i - M)/T)
};

// Whole-vocabulary rows hand at least this many of their largest composites, sorted, from the
// merge to head_fast_kernel.
constexpr int kHeadList = 32;

struct Workspace {
  uint32_t *head_count;     // [rows_cap] head sizes
  SliceStat *stats;         // [rows_cap * kMaxSplits]
  uint64_t *cands;          // [rows_cap * row_cand_stride]
  RowState *row_state;      // [rows_cap]
  uint64_t *head;           // [head_rows * head_stride] whole-vocabulary rows: the head, slice s
                            // of head_kernel at [s * h_slice_len, + head_slice_count)
  uint64_t *head_sorted;    // [head_rows * head_stride] the head, sorted
  double *head_s;           // [head_rows * head_stride] exp((l - max)/T) in sorted order
  double *head_c;           // [head_rows * head_stride] running sums of the weights
  uint32_t *head_plan;      // [head_rows * plan_stride] segment offsets of the sorted head
  double *head_part;        // [head_rows * 2 * (plan_stride - 2)] per-segment exp sums
  double *head_acc;         // [head_rows * 3 * acc_stride] head_kernel's per-slice ulp counts
  uint32_t *head_slice_count;  // [head_rows * acc_stride] head entries each slice stored
  int32_t plan_stride;
  int32_t acc_stride;       // >= the head kernel's slices per row
  int64_t row_cand_stride;  // composites per row in cands
  int32_t head_stride;
};

struct Launch {
  const void *logits;
  const tabby_row_params *params;
  tabby_row_result *results;
  int32_t *topk_ids;
  float *topk_logits;
  int32_t rows;
  int32_t vocab;
  int32_t splits;
  int32_t slice_len;
  int32_t topk_cap;
  int32_t k_max;     // largest top_k the handle accepts
  int32_t kcap;      // largest pool the sampling kernel finishes itself
  int32_t head_pass; // 1 when the head kernels run after this launch
  int32_t h_splits;  // slices per row of the head kernel
  int32_t h_slice_len;
  int32_t parts;      // row_kernel: 1 = one workgroup per row; > 1 = workgroups per row (each
                      // a part of slice_len elements, finished by wave_merge_kernel); 0 = unused
  int32_t row_waves;  // row_kernel: waves per workgroup
  int32_t pool_rows;  // 1: pool_row_kernel streams each row (pools above 256, rows >= CUs)
  int32_t list_stride;  // pools <= 256: entries between the sorted lists of consecutive slices
                        // (or parts) of a row in cands -- slice_len, or kWaveKcap when the
                        // lists are packed (a list never holds more than the pool)
};

// The (row, slice) of workgroup b of a grid of rows x splits. Workgroup b runs on XCD b % 8
// (round-robin dispatch over the eight XCDs), and so does the merge's workgroup for row b:
// when rows is a multiple of 8, row r's slices go to XCD r % 8 too, so that the merge
// finds their lists and statistics in its own XCD's L2. Otherwise row-major.
__device__ __forceinline__ void row_slice_of(int b, int rows, int splits, int &row, int &slice) {
  if (rows % 8 == 0) {
    const int x = b & 7, i = b >> 3;
    const int k = i / splits;
    row = x + 8 * k;
    slice = i - k * splits;
  } else {
    row = b / splits;
    slice = b - row * splits;
  }
}


__device__ __forceinline__ int32_t effective_k(const tabby_row_params &p, int vocab) {
  return (p.top_k <= 0 || p.top_k >= vocab) ? vocab : p.top_k;
}

// A row's parameters as the sampler accepts them: top_k in [0, k_max], the uniform in [0, 1),
// and a temperature below +inf that is not NaN. sampler.ts would sample a NaN temperature
// (`NaN <= 0` is false: every weight NaN, the draw falling to the pool's last entry) and turn
// +inf into a uniform draw whose -inf entries poison the sums; here both are TABBY_EINVAL on
// every path (the hosts throw before drawing a uniform). top_p is taken as sampler.ts takes
// it, any value: below 1 cuts at the first running sum reaching it (the first, for top_p <= 0),
// NaN or >= 1 never cuts.
__device__ __forceinline__ bool params_valid(const tabby_row_params &p, int k_max) {
  return p.top_k >= 0 && p.top_k <= k_max && p.reserved == 0 && !(p.uniform < 0.0) &&
         !(p.uniform >= 1.0) && p.uniform == p.uniform && p.temperature < INFINITY;
}

// sampleFromTopK's greedy branch (src/engine/sampler.ts:159): T <= 0 (-0 and -inf included)
// takes the pool's first entry and leaves the uniform unused. Every tail tests this one
// predicate; params_valid has already rejected NaN, so it is the complement of T > 0.
__device__ __forceinline__ bool greedy_temp(double T) { return T <= 0.0; }

// How many of its largest elements a slice keeps as candidates: the row's pool for a row
// whose pool fits the kernels (keff <= kcap); for a whole-vocabulary row, the top-k list the
// caller asked for (topk_cap <= k_max <= kcap) and at least kHeadList, which the merge uses
// to lower the row's head threshold far enough that the head holds that list, and hands on
// sorted to head_fast_kernel.
__device__ __forceinline__ int slice_keep(bool valid, int keff, int n, int kcap, int head_pass,
                                          int topk_cap) {
  if (!valid) return 0;
  if (keff <= kcap) return min(keff, n);
  return head_pass ? min(max(topk_cap, kHeadList), n) : 0;
}

// The first active lane's f64, bit for bit (the readfirstlane builtin takes 32-bit ints).
__device__ __forceinline__ double readfirstlane_f64(double v) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
  const long long b = __double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)b, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(b >> 32), lane);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// The fast form of finish_row for pools of 257..KCAP (as reg_tail for pools up to 64): terms
// from exp_nonpos (within 8 ulp of exp), the running sums of the scaled terms a workgroup scan
// divided by their total (each partial sum a tree of at most 12 roundings, then one
// division). Against the reference's sequential sums of its exact terms -- whose own rounding
// is at most n * 2^-53 relative -- the running sums then differ by less than 2^-42 of their
// value for n <= 1024, so when every comparison that decides the cut and the draw clears its
// threshold by more than 2^-36 relative, the reference decides the same way: returns true with
// the result written. Otherwise (or for a greedy row) returns false and finish_row computes the
// row bit for bit. poolMass and the probability (compared within 1e-5) take the fast terms.
// Three barriers: one exchange of the waves' totals, then one per first-index search (one LDS
// atomic per wave: the first lane that holds a match).
template <int KCAP, typename In, class Smem, int NW = kWaves>
__device__ __forceinline__ bool finish_row_fast(Smem &sm, const Launch &L, int row, const In *row_src, int count,
                                float max_logit, double sum_exp, const tabby_row_params &P) {
  constexpr int kThreads = NW * kWaveSize;
  static_assert(KCAP % kThreads == 0, "whole entries per thread");
  constexpr int PER = KCAP / kThreads;
  const double T = P.temperature, top_p = P.top_p;
  if (greedy_temp(T)) return false;
  const int lane = lane_id(), wave = wave_id();
  double *run = sm.u.tail.w;  // running sums, by index
  double c[PER], ex[PER], e_sum = 0.0, acc = 0.0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = (int)threadIdx.x * PER + j;
    const bool in = i < count;
    const double d = in ? (double)value_of(composite_key(sm.sorted[i])) - (double)max_logit : 0.0;
    const double e = in ? exp_nonpos(d) : 0.0;
    ex[j] = e;  // the exact term: the probability if this entry is drawn
    e_sum += e;
    acc += !in ? 0.0 : T == 1.0 ? e : exp_nonpos(d / T);
    c[j] = acc;  // the thread's running sum of the scaled terms
  }
  // At T = 1 the scaled terms are the exact ones: their total serves poolMass too (a different
  // summation order, within poolMass's 1e-5), and the exact terms need no reduction of their own.
  const bool t1 = T == 1.0;
  const double incl = wave_inclusive_scan(acc);
  if (lane == kWaveSize - 1) sm.bs.d[wave] = incl;
  if (!t1) {
    const double e_wave = wave_sum(e_sum);
    if (lane == 0) sm.bs.d2[wave] = e_wave;
  }
  if (threadIdx.x == 0) {
    sm.bs.slot = (uint32_t)count;
    sm.bs.slot2 = (uint32_t)count;
  }
  __syncthreads();
  double scaled = 0.0, e_total = 0.0, base = incl - acc;
  if constexpr (NW <= kWaves) {
#pragma unroll
    for (int k = 0; k < NW; ++k) {
      scaled += sm.bs.d[k];
      if (!t1) e_total += sm.bs.d2[k];
      if (k < wave) base += sm.bs.d[k];
    }
  } else {
    // Many waves: lane k takes wave k's totals, and a wave scan gives every prefix (the
    // unrolled loop above held too many of them in registers).
    const double waves_incl = wave_inclusive_scan(lane < NW ? sm.bs.d[lane] : 0.0);
    scaled = readlane_f64(waves_incl, NW - 1);
    if (!t1) e_total = wave_sum(lane < NW ? sm.bs.d2[lane] : 0.0);
    if (wave > 0) base += readlane_f64(waves_incl, wave - 1);
  }
  if (t1) e_total = scaled;
  const double pool = e_total / sum_exp;
  double r[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = (int)threadIdx.x * PER + j;
    r[j] = (base + c[j]) / scaled;
    if (i < count) run[i] = r[j];
  }
  // The first index whose running sum satisfies pred: the thread's first, the wave's first
  // lane with one, one atomic per wave.
  auto first_of = [&](uint32_t *slot, int n, auto pred) {
    int mine = n;
#pragma unroll
    for (int j = PER - 1; j >= 0; --j) {
      const int i = (int)threadIdx.x * PER + j;
      if (i < n && pred(r[j])) mine = i;
    }
    const uint64_t m = __ballot(mine < n);
    if (m && lane == __ffsll((unsigned long long)m) - 1) atomicMin(slot, (uint32_t)mine);
  };
  if (top_p < 1.0) first_of(&sm.bs.slot, count, [&](double x) { return x >= top_p; });
  __syncthreads();
  const int cut_at = (int)sm.bs.slot;
  const int cut = cut_at < count ? cut_at + 1 : count;
  const double total = run[cut - 1];
  const double target = P.uniform * total;
  first_of(&sm.bs.slot2, cut, [&](double x) { return target < x; });
  __syncthreads();
  const int hit = (int)sm.bs.slot2;
  const int chosen = hit < cut ? hit : cut - 1;
  // Margins of every comparison that fixed the cut and the draw (running sums are
  // non-decreasing, so the neighbours of each boundary are the only ones to check).
  constexpr double kMargin = 1.0 / 68719476736.0;  // 2^-36
  bool clear = true;
  if (top_p < 1.0) {
    const double m = kMargin * top_p;
    const double r_cut = run[cut - 1], r_before = cut >= 2 ? run[cut - 2] : 0.0;
    clear = (cut < count || r_cut < top_p - m) &&
            (cut == count || (r_cut >= top_p + m && (cut == 1 || r_before < top_p - m)));
  }
  const double m2 = kMargin * total;
  clear = clear && run[chosen] > target + m2 && (chosen == 0 || run[chosen - 1] < target - m2);
  if (!clear) {
    __syncthreads();  // finish_row reuses the arrays
    return false;
  }
  // The thread that holds the drawn entry writes the result with its own term.
  if ((int)threadIdx.x == chosen / PER) {
    double e = ex[0];
#pragma unroll
    for (int j = 1; j < PER; ++j)
      if (j == chosen % PER) e = ex[j];
    tabby_row_result res;
    res.max_logit = max_logit;
    res.sum_exp = sum_exp;
    res.pool_mass = pool;
    res.status = TABBY_OK;
    res.topk_count = min(count, L.topk_cap);
    res.considered = (uint32_t)cut;
    res.pool_exhausted = (top_p < 1.0 && pool < top_p) ? 1 : 0;
    res.id = (int32_t)composite_index(sm.sorted[chosen]);
    res.probability = e / sum_exp;
    L.results[row] = res;
  }
  if (L.topk_cap > 0) {
    const int m = min(count, L.topk_cap);
    for (int i = threadIdx.x; i < m; i += kThreads) {
      const uint32_t idx = composite_index(sm.sorted[i]);
      L.topk_ids[(size_t)row * L.topk_cap + i] = (int32_t)idx;
      L.topk_logits[(size_t)row * L.topk_cap + i] = load_one(row_src + min(idx, (uint32_t)(L.vocab - 1)));
    }
  }
  return true;
}

// sampleFromTopK (src/engine/sampler.ts:147-212) over the `count` sorted candidates in
// sm.sorted, f64 throughout, in the reference's order of operations: the per-element terms
// are independent and computed by all lanes; the sums are sequential left-to-right f64 sums,
// evaluated bit for bit by a wave (seqsum.h). The running sums of the draw (sampler.ts:195-203)
// are the top-p cumulative sums (sampler.ts:178-185), and `total` (:191-192) is the last of
// them. The fast form above is tried first.
template <int KCAP, typename In, class Smem, int NW = kWaves>
__device__ __forceinline__ void finish_row(Smem &sm, const Launch &L, int row, const In *row_src,
                           int count, float max_logit, double sum_exp,
                           const tabby_row_params &P) {
  constexpr int kThreads = NW * kWaveSize;
  if (finish_row_fast<KCAP, In, Smem, NW>(sm, L, row, row_src, count, max_logit, sum_exp, P)) return;
  const double T = P.temperature;
  double *exact = sm.u.tail.exact;
  double *w = sm.u.tail.w;
  for (int i = threadIdx.x; i < count; i += kThreads) {
    const float l = value_of(composite_key(sm.sorted[i]));
    const double d = (double)l - (double)max_logit;
    exact[i] = fdlibm_exp(d) / sum_exp;
    w[i] = !greedy_temp(T) ? fdlibm_exp(d / T) : 0.0;
  }
  __syncthreads();
  // Sequential sums (bit-exact; see seqsum.h): poolMass on wave 0 and the scaled total on
  // wave 1 at the same time. (The 16-terms-per-lane form reads 16 consecutive entries per
  // lane, which these unpadded LDS arrays serve with bank conflicts: slower here.)
  if (wave_id() == 0) {
    const double pool = wave_seq_sum(exact, count, nullptr, INFINITY).total;
    if (lane_id() == 0) sm.pool_mass = pool;
  } else if (wave_id() == 1) {
    const double scaled = !greedy_temp(T) ? wave_seq_sum(w, count, nullptr, INFINITY).total : 0.0;
    if (lane_id() == 0) sm.scaled_total = scaled;
  }
  __syncthreads();
  const double pool_mass = sm.pool_mass;
  const double scaled_total = sm.scaled_total;
  if (!greedy_temp(T)) {
    for (int i = threadIdx.x; i < count; i += kThreads) w[i] = w[i] / scaled_total;
    __syncthreads();
  }
  if (wave_id() == 0) {
    tabby_row_result r;
    r.max_logit = max_logit;
    r.sum_exp = sum_exp;
    r.pool_mass = pool_mass;
    r.status = TABBY_OK;
    r.topk_count = min(count, L.topk_cap);
    int chosen = 0;
    if (greedy_temp(T)) {
      r.considered = 1;
      r.pool_exhausted = 0;
    } else {
      // The running sums of the weights (in place), up to the first that reaches top-p.
      const double top_p = P.top_p;
      const SeqSum run = wave_seq_sum(w, count, w, top_p < 1.0 ? top_p : INFINITY);
      wave_lds_sync();
      const int cut = run.count;
      const double target = P.uniform * run.total;
      chosen = cut - 1;
      for (int base = 0; base < cut; base += kWaveSize) {
        const int i = base + lane_id();
        const uint64_t hit = __ballot(i < cut && target < w[min(i, cut - 1)]);
        if (hit) {
          chosen = base + __ffsll((unsigned long long)hit) - 1;
          break;
        }
      }
      r.considered = (uint32_t)cut;
      r.pool_exhausted = (top_p < 1.0 && pool_mass < top_p) ? 1 : 0;
    }
    r.id = (int32_t)composite_index(sm.sorted[chosen]);
    r.probability = exact[chosen];
    if (lane_id() == 0) L.results[row] = r;
  }
  if (L.topk_cap > 0) {
    const int m = min(count, L.topk_cap);
    for (int i = threadIdx.x; i < m; i += kThreads) {
      const uint32_t idx = composite_index(sm.sorted[i]);
      L.topk_ids[(size_t)row * L.topk_cap + i] = (int32_t)idx;
      L.topk_logits[(size_t)row * L.topk_cap + i] = load_one(row_src + min(idx, (uint32_t)(L.vocab - 1)));
    }
  }
}

// sampleFromTopK (src/engine/sampler.ts:147-212) for a pool of at most 64*R candidates, by
// one wave, in registers: element i of the pool is register i/64 of lane i%64. The
// per-element terms are computed lane-parallel; each sum is sequential in index order,
// lane by lane through readlane, as the reference's left-to-right reduce. The running sums
// of the draw equal the top-p cumulative sums, so they are kept (writelane) from the
// top-p scan (each lane keeps its own element's) and the draw is a ballot over
// "target < running".
template <int R, typename In>
__device__ __forceinline__ void wave_finish(const uint64_t *pool_in, int count, const Launch &L, int row,
                            const In *row_src, float max_logit, double sum_exp,
                            const tabby_row_params &P) {
  const int lane = wave_lane();
  uint64_t v[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * kWaveSize + lane;
    v[r] = i < count ? pool_in[i] : 0ull;
  }
  wave_sort_desc<R>(v);
  const double T = P.temperature;
  double exact[R], w[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    exact[r] = 0.0;
    w[r] = 0.0;
    if (r * kWaveSize + lane < count) {
      const double d = (double)value_of(composite_key(v[r])) - (double)max_logit;
      exact[r] = fdlibm_exp(d) / sum_exp;
      if (!greedy_temp(T)) w[r] = fdlibm_exp(d / T);
    }
  }
  double pool = 0.0, scaled = 0.0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int m = min(kWaveSize, count - r * kWaveSize);
    for (int j = 0; j < m; ++j) {
      pool += readlane_f64(exact[r], j);
      scaled += readlane_f64(w[r], j);
    }
  }
  tabby_row_result res;
  res.max_logit = max_logit;
  res.sum_exp = sum_exp;
  res.pool_mass = pool;
  res.status = TABBY_OK;
  res.topk_count = min(count, L.topk_cap);
  int chosen = 0;
  if (greedy_temp(T)) {
    res.considered = 1;
    res.pool_exhausted = 0;
  } else {
#pragma unroll
    for (int r = 0; r < R; ++r) w[r] = w[r] / scaled;
    const double top_p = P.top_p;
    double c = 0.0, running[R];
    int cut = count;
    bool cut_found = false;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      running[r] = 0.0;
      const int m = min(kWaveSize, count - r * kWaveSize);
      for (int j = 0; j < m && !cut_found; ++j) {
        c += readlane_f64(w[r], j);
        running[r] = lane == j ? c : running[r];
        if (top_p < 1.0 && c >= top_p) {
          cut = r * kWaveSize + j + 1;
          cut_found = true;
        }
      }
    }
    const double target = P.uniform * c;  // c is the running sum at cut - 1: the reference's total
    chosen = cut - 1;
    bool done = false;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = r * kWaveSize + lane;
      const uint64_t hit = __ballot(i < cut && target < running[r]);
      if (!done && hit) {
        chosen = r * kWaveSize + __ffsll((unsigned long long)hit) - 1;
        done = true;
      }
    }
    res.considered = (uint32_t)cut;
    res.pool_exhausted = (top_p < 1.0 && pool < top_p) ? 1 : 0;
  }
  // The chosen candidate's id and probability live in lane chosen%64, register chosen/64.
  uint64_t cv = 0;
  double cp = 0.0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r == chosen / kWaveSize) {
      cv = (uint64_t)__builtin_amdgcn_readlane((int)v[r], chosen % kWaveSize) |
           ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(v[r] >> 32), chosen % kWaveSize) << 32);
      cp = readlane_f64(exact[r], chosen % kWaveSize);
    }
  }
  res.id = (int32_t)composite_index(cv);
  res.probability = cp;
  if (lane == 0) L.results[row] = res;
  if (L.topk_cap > 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = r * kWaveSize + lane;
      if (i < count && i < L.topk_cap) {
        const uint32_t idx = composite_index(v[r]);
        L.topk_ids[(size_t)row * L.topk_cap + i] = (int32_t)idx;
        L.topk_logits[(size_t)row * L.topk_cap + i] = load_one(row_src + min(idx, (uint32_t)(L.vocab - 1)));
      }
    }
  }
}

__device__ __forceinline__ void write_status(const Launch &L, int row, int32_t status, float mx,
                                             double se) {
  tabby_row_result r;
  memset(&r, 0, sizeof r);
  r.id = -1;
  r.max_logit = mx;
  r.sum_exp = se;
  r.status = status;
  L.results[row] = r;
}

// ---------------------------------------------------------------------------------------
// Kernel 1 (slices): grid = rows x splits; each workgroup streams one slice of a row from
// HBM exactly once, in chunks of 16 elements per lane (4096 per workgroup) with the next
// chunk's loads in flight while the current one is processed. Per lane it keeps an online
// max and an f64 sum of exp(x - max). It also collects the slice's candidates: every
// element >= theta, where theta starts at a lower bound on the first chunk's kk-th largest
// element (a radix select on the top 22 bits of the key) -- so at least kk distinct elements
// reach it, and it never exceeds the slice's kk-th largest value. Candidates go to an LDS list with one atomic per
// wave; a list that would overflow is flushed to the slice's region of global memory. The
// exact selection happens once per row, in the merge.
//
// There is no cross-workgroup communication: the merge is the next kernel on the stream,
// so the kernel boundary orders these writes before its reads (an agent-scope fence per
// workgroup costs an L2 writeback + invalidate each, measured slower than the whole read).
// ---------------------------------------------------------------------------------------
constexpr int kChunkPerLane = 16;
constexpr int kChunk = kChunkPerLane * kBlock;
constexpr int kListCap = kChunk;  // a whole chunk always fits after a flush

struct SliceSmem {
  BlockScratch bs;
  uint32_t list_count;  // list length after a prune or flush
  uint32_t committed;   // list_count as of the last chunk boundary (stable between barriers)
  uint32_t flushed;     // candidates already written to global memory
  uint32_t wave_count[2][kWaves];  // by chunk parity: chunk c+1 writes while c is read
  float theta;
  uint32_t hist[kBins];       // radix-select histograms (first-chunk theta, list pruning)
  uint64_t list[kListCap];
};

// theta from a selection threshold key, clamped to [-inf, +inf]: an early-exit prefix can
// fall below the key of -inf (or above +inf), where keys decode to NaN.
__device__ __forceinline__ float theta_of(uint64_t prefix) {
  const uint32_t k = (uint32_t)(prefix >> 32);
  return value_of(min(max(k, kNegInfKey), 0xff800000u));
}

__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// This lane's position in a buffer filled through the LDS counter *slot, for lanes that
// take: one atomic per wave for all of its taking lanes (a counter that every lane
// increments serialises them -- 4,096 in a row cost a config-5 list prune ~5 us). Callers
// may be divergent: only active lanes count.
__device__ __forceinline__ uint32_t wave_slot(bool take, uint32_t *slot) {
  const uint64_t mask = __ballot(take);
  if (!mask) return 0u;
  const int leader = __ffsll((unsigned long long)mask) - 1;
  uint32_t base = 0u;
  if ((int)lane_id() == leader) base = atomicAdd(slot, (uint32_t)__popcll(mask));
  base = (uint32_t)__builtin_amdgcn_readlane((int)base, leader);
  return base + lanes_below(mask);
}

// Raw loads of chunk `chunk` (no masking, so nothing consumes them until the next
// iteration and they stay in flight). Lanes past the end reread the slice's last vector.
template <typename In, int VEC>
__device__ __forceinline__ void load_chunk(const In *src, int n, int chunk, float (&x)[kChunkPerLane]) {
  constexpr int ITEMS = kChunkPerLane / VEC;
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const int le = chunk * kChunk + (j * kBlock + (int)threadIdx.x) * VEC;
    float v[VEC];
    Loader<In, VEC>::load(src + min(le, n - VEC), v);
#pragma unroll
    for (int c = 0; c < VEC; ++c) x[j * VEC + c] = v[c];
  }
}

// Padding lanes of chunk `chunk` become -inf, which no statistic or candidate test admits.
template <int VEC>
__device__ __forceinline__ void mask_chunk(int n, int chunk, float (&x)[kChunkPerLane]) {
  constexpr int ITEMS = kChunkPerLane / VEC;
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const bool valid = chunk * kChunk + (j * kBlock + (int)threadIdx.x) * VEC < n;
#pragma unroll
    for (int c = 0; c < VEC; ++c) x[j * VEC + c] = valid ? x[j * VEC + c] : -INFINITY;
  }
}

template <int VEC>
__device__ __forceinline__ int chunk_local(int chunk, int e) {
  // Slice-local index of register element e of this lane in chunk `chunk`.
  return chunk * kChunk + ((e / VEC) * kBlock + (int)threadIdx.x) * VEC + e % VEC;
}

// Copies the LDS list to the slice's global region and empties it. Whole workgroup.
__device__ __forceinline__ void flush_list(SliceSmem &sm, uint64_t *region, uint32_t count) {
  const uint32_t at = sm.flushed;
  for (uint32_t i = threadIdx.x; i < count; i += kBlock) region[at + i] = sm.list[i];
  __syncthreads();
  if (threadIdx.x == 0) {
    sm.flushed = at + count;
    sm.list_count = 0u;
    sm.committed = 0u;
  }
  __syncthreads();
}

// Drops from the LDS list every entry below the key of its kk-th largest composite and
// raises sm.theta to that key. Whole workgroup; returns the new length (>= kk).
__device__ __forceinline__ uint32_t prune_list(SliceSmem &sm, uint32_t have, uint32_t kk) {
  auto each = [&](auto &&f) {
    for (uint32_t i = threadIdx.x; i < have; i += kBlock) f(sm.list[i]);
  };
  // Two radix passes (the key's top 22 bits) suffice: entries tied on the key are kept anyway.
  const SelectResult r = radix_select(each, kk, sm.hist, sm.bs, 2);
  const uint32_t key = min(max((uint32_t)(r.prefix >> 32), kNegInfKey), 0xff800000u);
  constexpr int kPer = kListCap / kBlock;
  uint64_t v[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const uint32_t i = (uint32_t)(q * kBlock) + threadIdx.x;
    v[q] = i < have ? sm.list[i] : 0ull;
  }
  if (threadIdx.x == 0) sm.bs.slot = 0u;
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const uint32_t i = (uint32_t)(q * kBlock) + threadIdx.x;
    const bool keep = i < have && composite_key(v[q]) >= key;
    const uint32_t at = wave_slot(keep, &sm.bs.slot);
    if (keep) sm.list[at] = v[q];
  }
  __syncthreads();
  const uint32_t kept = sm.bs.slot;
  if (threadIdx.x == 0) {
    sm.theta = fmaxf(sm.theta, value_of(key));
    sm.list_count = kept;
    sm.committed = kept;
  }
  __syncthreads();
  return kept;
}

template <typename In, int VEC>
__global__ __launch_bounds__(kBlock) void slice_kernel(Launch L, Workspace W) {
  constexpr int ITEMS = kChunkPerLane / VEC;
  __shared__ SliceSmem sm;

  int row, slice;
  row_slice_of((int)blockIdx.x, L.rows, L.splits, row, slice);
  const int V = L.vocab;
  const int begin = slice * L.slice_len;
  const int n = min(L.slice_len, V - begin);
  const int nchunks = (n + kChunk - 1) / kChunk;
  const tabby_row_params P = L.params[row];
  const bool valid_params = params_valid(P, L.k_max);
  const int keff = effective_k(P, V);
  const int kk = slice_keep(valid_params, keff, n, L.kcap, L.head_pass, L.topk_cap);
  const In *src = reinterpret_cast<const In *>(L.logits) + (size_t)row * V + begin;
  // The slice's candidate region: room for every element of the slice.
  uint64_t *region = W.cands + (size_t)row * W.row_cand_stride + (size_t)begin;

  if (threadIdx.x == 0) {
    sm.list_count = 0u;
    sm.committed = 0u;
    sm.flushed = 0u;
    sm.theta = -INFINITY;
  }
  __syncthreads();
  float lane_max = -INFINITY;
  float lane_ml = 0.0f;   // fl(lane_max * L): the reference of lane_sum's terms (rebase_sum)
  double lane_sum = 0.0;  // sum of 2^(x*L - lane_ml) over this lane's elements so far

  // Chunk c held in x, with the next chunk's loads in flight (issued unconditionally on each
  // path of the loop below and into their own registers, so the compiler's wait before
  // chunk c leaves them in flight).
  auto body = [&](int c, float(&x)[kChunkPerLane]) {
    mask_chunk<VEC>(n, c, x);

    // Online max / sum-exp for this lane.
    float cm = x[0];
#pragma unroll
    for (int e = 1; e < kChunkPerLane; ++e) cm = fmaxf(cm, x[e]);
    const float nm = fmaxf(lane_max, cm);
    if (nm != -INFINITY) {
      const float ml = nm * kLog2e;
      float t[kChunkPerLane];  // summed pairwise, as in the wave kernel
#pragma unroll
      for (int e = 0; e < kChunkPerLane; ++e) t[e] = __builtin_amdgcn_exp2f(fmaf(x[e], kLog2e, -ml));
#pragma unroll
      for (int h = kChunkPerLane / 2; h > 0; h >>= 1) {
#pragma unroll
        for (int e = 0; e < h; ++e) t[e] += t[e + h];
      }
      const float part = t[0];
      const double rescale = lane_max == -INFINITY ? 0.0 : (double)__builtin_amdgcn_exp2f(lane_ml - ml);
      lane_sum = lane_sum * rescale + (double)part;
      lane_max = nm;
      lane_ml = ml;
    }

    if (kk > 0) {
      if (c == 0 && kk < min(n, kChunk)) {
        // theta: a lower bound on the kk-th largest element of the first chunk (its padding
        // excluded).
        auto elems = [&](auto &&f) {
#pragma unroll
          for (int e = 0; e < kChunkPerLane; ++e) {
            const int local = chunk_local<VEC>(0, e);
            if (local < n) f(composite(key_of(x[e]), (uint32_t)local));
          }
        };
        // Two passes: the top 22 bits of the key. The bin's lower edge still has kk
        // elements at or above it (ties on the key would need the index digits).
        const SelectResult r = radix_select(elems, (uint32_t)kk, sm.hist, sm.bs, 2);
        if (threadIdx.x == 0) sm.theta = theta_of(r.prefix);
        __syncthreads();
      }
      const float theta = sm.theta;
      const bool check_index = !(theta > -INFINITY);
      // Count first (ballots, kept for the appends), so that a list that would overflow is
      // pruned or flushed before anything is appended; each wave's slots then follow from
      // the per-wave counts, with no atomics.
      uint64_t masks[kChunkPerLane];
      uint32_t mine = 0;
#pragma unroll
      for (int e = 0; e < kChunkPerLane; ++e) {
        masks[e] = __ballot(x[e] >= theta && (!check_index || chunk_local<VEC>(c, e) < n));
        mine += (uint32_t)__popcll(masks[e]);
      }
      if (lane_id() == 0) sm.wave_count[c & 1][wave_id()] = mine;
      __syncthreads();
      uint32_t incoming = 0, before = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const uint32_t wc = sm.wave_count[c & 1][w];
        before += w < wave_id() ? wc : 0u;
        incoming += wc;
      }
      uint32_t have = sm.committed;
      if (incoming > 0) {
        if (have + incoming > (uint32_t)kListCap && have >= (uint32_t)kk) {
          // Prune: keep the entries whose key reaches the list's kk-th largest, and raise
          // theta to it. Only massive ties can leave the list too full; it is then flushed.
          have = prune_list(sm, have, (uint32_t)kk);
        }
        if (have + incoming > (uint32_t)kListCap) {
          flush_list(sm, region, have);
          have = 0;
        }
        uint32_t at = have + before;  // a chunk holds at most kChunk <= kListCap candidates
#pragma unroll
        for (int e = 0; e < kChunkPerLane; ++e) {
          const uint64_t mask = masks[e];
          if (mask) {
            if ((mask >> lane_id()) & 1ull)
              sm.list[at + lanes_below(mask)] =
                  composite(key_of(x[e]), (uint32_t)(begin + chunk_local<VEC>(c, e)));
            at += (uint32_t)__popcll(mask);
          }
        }
        __syncthreads();
        if (threadIdx.x == 0) sm.committed = have + incoming;  // read after the next barrier
      }
    }
  };
  float x[kChunkPerLane], y[kChunkPerLane];
  load_chunk<In, VEC>(src, n, 0, x);
  for (int c = 0; c < nchunks; c += 2) {
    if (c + 1 >= nchunks) {
      body(c, x);
      break;
    }
    load_chunk<In, VEC>(src, n, c + 1, y);
    body(c, x);
    if (c + 2 >= nchunks) {
      body(c + 1, y);
      break;
    }
    load_chunk<In, VEC>(src, n, c + 2, x);
    body(c + 1, y);
  }

  // Slice statistics (their barriers also publish `committed`).
  const float ms = block_max(lane_max, sm.bs);
  const double ss = block_sum(rebase_sum(lane_sum, lane_max, lane_ml, ms), sm.bs);
  uint32_t total = 0;
  if (kk > 0) {
    uint32_t have = sm.committed;
    // A last prune keeps the merge's candidate set small (about kk plus ties per slice).
    if (have > (uint32_t)kk + (uint32_t)kk / 4u) have = prune_list(sm, have, (uint32_t)kk);
    total = sm.flushed + have;
    const uint32_t at = sm.flushed;
    for (uint32_t i = threadIdx.x; i < have; i += kBlock) region[at + i] = sm.list[i];
  }
  if (threadIdx.x == 0) {
    SliceStat st_out;
    st_out.max = ms;
    st_out.count = total;
    st_out.sum = ss;
    W.stats[(size_t)row * kMaxSplits + slice] = st_out;
  }
}

// ---------------------------------------------------------------------------------------
// Kernel 1 for pools of at most 256 (wave_kernel): grid = rows x splits, one wave per
// workgroup, so nothing in it waits at a barrier. Each wave streams its slice of a row from
// HBM exactly once, 1024 elements (16 per lane) per chunk, with the next chunk's loads in
// flight while the current one is processed; keeps the lane max and f64 sum-exp online; and
// keeps in a wave-private LDS list every element >= theta, where theta never exceeds the
// kk-th largest value seen so far. theta starts at the kk-th largest lane maximum of the
// first chunk (kk <= 64). When the list is nearly full it is pruned: its keys
// are binned by distance below the list's largest key (256 bins, width chosen from the key
// range), theta rises to the lower edge of the bin that holds the kk-th largest entry, and
// the entries below are dropped -- no sort. (Only massive ties can keep a bin from
// shrinking the list; then it is sorted in registers and cut to kk.)
// At the end the list is sorted in registers and the slice's top min(count, kk) go to its
// candidate region, so the merge works on sorted lists.
// ---------------------------------------------------------------------------------------
constexpr int kWChunkPerLane = 16;
constexpr int kWChunk = kWaveSize * kWChunkPerLane;
constexpr int kWListCap = 512;
constexpr int kWaveKcap = 256;
constexpr int kPruneBins = 256;

template <typename In, int VEC>
__device__ __forceinline__ void wave_load(const In *src, int n, int chunk, float (&x)[kWChunkPerLane]) {
  constexpr int ITEMS = kWChunkPerLane / VEC;
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const int le = chunk * kWChunk + (j * kWaveSize + wave_lane()) * VEC;
    float v[VEC];
    Loader<In, VEC>::load(src + min(le, n - VEC), v);  // past the end: reread, masked later
#pragma unroll
    for (int c = 0; c < VEC; ++c) x[j * VEC + c] = v[c];
  }
}

// Chunk `chunk` lies entirely inside the slice: no clamping.
template <typename In, int VEC>
__device__ __forceinline__ void wave_load_full(const In *src, int chunk, float (&x)[kWChunkPerLane]) {
  constexpr int ITEMS = kWChunkPerLane / VEC;
  const In *base = src + chunk * kWChunk + wave_lane() * VEC;
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    float v[VEC];
    Loader<In, VEC>::load(base + j * kWaveSize * VEC, v);
#pragma unroll
    for (int c = 0; c < VEC; ++c) x[j * VEC + c] = v[c];
  }
}

// Chunk `chunk` by one code path whatever the chunk: lanes past the slice's end reread its
// last vector, and a chunk past the last (chunk >= nchunks) loads the slice's first vector
// into every lane (one line, never used). Branching between wave_load_full and wave_load
// made the compiler land the loads in temporaries and copy them at once -- waiting for the
// prefetched chunk right after issuing it.
template <typename In, int VEC>
__device__ __forceinline__ void wave_load_any(const In *src, int n, int chunk, int nchunks,
                                              float (&x)[kWChunkPerLane]) {
  constexpr int ITEMS = kWChunkPerLane / VEC;
  const bool live = chunk < nchunks;
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const int le = chunk * kWChunk + (j * kWaveSize + wave_lane()) * VEC;
    float v[VEC];
    Loader<In, VEC>::load(src + (live ? min(le, n - VEC) : 0), v);
#pragma unroll
    for (int c = 0; c < VEC; ++c) x[j * VEC + c] = v[c];
  }
}

template <int VEC>
__device__ __forceinline__ int wave_local(int chunk, int e) {
  return chunk * kWChunk + ((e / VEC) * kWaveSize + wave_lane()) * VEC + e % VEC;
}

// The chunks of one slice (n elements from src) as the one-wave streaming loops read them,
// element e of a lane's 16 being wave_local(chunk, e): 16-byte vectors (VEC > 1) or single
// elements (VEC = 1: an odd length or an unaligned row), through a buffer resource over the
// slice (RowBuffer). Elements past the slice's end, and every element of a chunk index past
// the last, read as zero without touching memory; callers mask them by index. Loads are
// issued unconditionally, so that the wait before a chunk's use leaves the next chunk in
// flight.
template <typename In, int VEC>
struct ChunkReader {
  RowBuffer buf;
  __device__ __forceinline__ ChunkReader(const In *src, int n) : buf(src, (uint32_t)n * (uint32_t)sizeof(In)) {}
  __device__ __forceinline__ void load(int chunk, float (&x)[kWChunkPerLane]) const {
    const uint32_t base = (uint32_t)__builtin_amdgcn_readfirstlane(chunk * (int)(kWChunk * sizeof(In)));
    if constexpr (VEC == 1) {
      const uint32_t lane_off = (uint32_t)wave_lane() * (uint32_t)sizeof(In);
#pragma unroll
      for (int e = 0; e < kWChunkPerLane; ++e)
        x[e] = buf.load_elem((const In *)nullptr, lane_off, base + (uint32_t)(e * kWaveSize * sizeof(In)));
    } else {
      static_assert(VEC * sizeof(In) == 16, "16-byte vectors");
      constexpr int ITEMS = kWChunkPerLane / VEC;
      const uint32_t lane_off = (uint32_t)wave_lane() * 16u;
#pragma unroll
      for (int j = 0; j < ITEMS; ++j) {
        float v[VEC];
        Widen<In, VEC>::from(buf.load16(lane_off, base + (uint32_t)(j * kWaveSize * 16)), v);
#pragma unroll
        for (int c = 0; c < VEC; ++c) x[j * VEC + c] = v[c];
      }
    }
  }
};

// The wave kernel's LDS list holds raw entries, (value bits << 32) | ~index, so that an
// append needs no key transform; a prune or the final sort turns them into composites
// (key_of(value) << 32 | ~index) as it reads them. key_of maps -0 to the key of +0.
__device__ __forceinline__ uint64_t raw_entry(float x, uint32_t index) {
  return ((uint64_t)__float_as_uint(x) << 32) | (uint64_t)(~index);
}
__device__ __forceinline__ uint32_t raw_key(uint64_t raw) { return key_of(__uint_as_float((uint32_t)(raw >> 32))); }
__device__ __forceinline__ uint64_t composite_of_raw(uint64_t raw) {
  return ((uint64_t)raw_key(raw) << 32) | (raw & 0xffffffffull);
}
__device__ __forceinline__ uint64_t raw_of_composite(uint64_t c) {
  return ((uint64_t)__float_as_uint(value_of(composite_key(c))) << 32) | (c & 0xffffffffull);
}

// Sorts the raw list[0..count) descending in registers (count <= 64*R) and leaves its top
// `keep` at list[0..keep), still raw.
template <int R>
__device__ __forceinline__ void wave_sort_list(uint64_t *list, int count, int keep) {
  uint64_t v[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * kWaveSize + wave_lane();
    v[r] = i < count ? composite_of_raw(list[i]) : 0ull;
  }
  wave_sort_desc<R>(v);
  wave_lds_sync();
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * kWaveSize + wave_lane();
    if (i < keep) list[i] = raw_of_composite(v[r]);
  }
  wave_lds_sync();
}

// Sorts the raw list[0..count) descending in registers (count <= 64*R) and writes its top
// `keep`, as composites, to out[0..keep).
template <int R>
__device__ __forceinline__ void store_sorted_top(const uint64_t *list, int count, int keep, uint64_t *out) {
  uint64_t v[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * kWaveSize + wave_lane();
    v[r] = i < count ? composite_of_raw(list[i]) : 0ull;
  }
  wave_sort_desc<R>(v);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * kWaveSize + wave_lane();
    if (i < keep) out[i] = v[r];
  }
}

struct WaveSmem {
  uint64_t list[kWListCap];
  uint32_t hist[kPruneBins];
};

struct Pruned {
  int count;
  uint32_t theta_key;
};

// Drops from the wave's list (count <= 64*R, kk <= count) every entry that cannot be among
// its top kk; returns the new count and the raised theta key. At most kWListCap - 64
// entries are left, so one more element position always fits.
template <int R>
__device__ __noinline__ Pruned wave_prune(WaveSmem &sm, int count, int kk, uint32_t floor_key) {
  const int lane = wave_lane();
  wave_lds_sync();
  uint64_t v[R];
  uint32_t k[R];
  uint32_t kmax = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * kWaveSize + lane;
    v[r] = i < count ? sm.list[i] : 0ull;
    k[r] = i < count ? raw_key(v[r]) : 0u;
    kmax = max(kmax, k[r]);
  }
  kmax = wave_max_u32(kmax);
  const uint32_t range = kmax - min(floor_key, kmax);
  const int bits = range == 0 ? 0 : 32 - __clz((int)range);
  const int shift = bits > 8 ? bits - 8 : 0;  // (kmax - key) >> shift < 256 for key >= floor
#pragma unroll
  for (int i = lane; i < kPruneBins; i += kWaveSize) sm.hist[i] = 0u;
  wave_lds_sync();
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * kWaveSize + lane;
    if (i < count) atomicAdd(&sm.hist[min((kmax - k[r]) >> shift, (uint32_t)(kPruneBins - 1))], 1u);
  }
  wave_lds_sync();
  // The bin holding the kk-th largest: lanes own 4 bins each, in order from the top.
  uint32_t h[4], sum = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    h[q] = sm.hist[lane * 4 + q];
    sum += h[q];
  }
  const uint32_t inc = wave_inclusive_scan_u32(sum);
  const uint64_t reached = __ballot(inc >= (uint32_t)kk);
  const int owner = __ffsll((unsigned long long)reached) - 1;  // kk <= count: some lane reaches it
  int bin = 0;
  if (lane == owner) {
    const uint32_t before = inc - sum;
    bin = lane * 4 + 3;
    if (before + h[0] + h[1] + h[2] >= (uint32_t)kk) bin = lane * 4 + 2;
    if (before + h[0] + h[1] >= (uint32_t)kk) bin = lane * 4 + 1;
    if (before + h[0] >= (uint32_t)kk) bin = lane * 4;
  }
  bin = __builtin_amdgcn_readlane(bin, owner);
  // Smallest key in that bin; everything at or above it is kept.
  const uint32_t drop = ((uint32_t)bin + 1u) << shift;
  uint32_t tk = max(kmax - min(drop, kmax) + 1u, floor_key);
  int kept = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * kWaveSize + lane;
    const bool keep = i < count && k[r] >= tk;
    const uint64_t m = __ballot(keep);
    if (keep) sm.list[kept + (int)lanes_below(m)] = v[r];
    kept += (int)__popcll(m);
  }
  wave_lds_sync();
  if (kept > kWListCap - kWaveSize) {  // massive ties: sort and cut exactly
    wave_sort_list<kWListCap / kWaveSize>(sm.list, kept, kk);
    kept = kk;
    tk = raw_key(sm.list[kk - 1]);
  }
  return {kept, tk};
}

__device__ __forceinline__ Pruned wave_prune_any(WaveSmem &sm, int count, int kk, uint32_t floor_key) {
  if (count <= 128) return wave_prune<2>(sm, count, kk, floor_key);
  if (count <= 256) return wave_prune<4>(sm, count, kk, floor_key);
  return wave_prune<8>(sm, count, kk, floor_key);
}

// Registers per lane (1, 2, 4 or 8) for the union of the row's published lane-maximum keys:
// each of `waves` waves publishes m = min(64, 64 * regs / waves) keys, and the union must hold
// at least kk of them (kk <= 256 here; 8 always suffices for 5 to 16 waves).
__device__ __forceinline__ int bound_regs(int kk, int waves) {
  for (int r = 1; r < 8; r *= 2)
    if (waves * min(kWaveSize, kWaveSize * r / waves) >= kk) return r;
  return 8;
}

// The kk-th largest (1 <= kk <= total <= 64 * R) of keys[0..total), on every lane.
template <int R>
__device__ __forceinline__ uint32_t union_kth(const uint32_t *keys, int total, int kk, uint32_t &largest) {
  uint32_t v[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * kWaveSize + wave_lane();
    v[r] = i < total ? keys[i] : 0u;
  }
  wave_sort_desc<R>(v);
  largest = (uint32_t)__builtin_amdgcn_readlane((int)v[0], 0);
  const int p = kk - 1;
  uint32_t t = 0;
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (r == p / kWaveSize) t = (uint32_t)__builtin_amdgcn_readlane((int)v[r], p % kWaveSize);
  return t;
}

// The row's selection histogram for pools of at most 64 (finish_small_pool): 256 bins of keys
// counted down from `top` (the largest key of the row's first bound's union; larger keys go
// to bin 0) to the row's first bound, below which no list entry lies.
constexpr int kSelBins = 256;
constexpr int kSmallTake = 4 * kWaveSize;  // finish_small_pool: takes of at most 256
// Pools up to this size take finish_small_pool: a take is the pool plus the rest of the bin
// that holds its K-th largest key, and a pool of 256 had no room left for that rest (nearly
// every row fell back to the sorted merge: 47.5 -> 49.3 us at 256 rows with k = 256).
constexpr int kSmallPoolMax = kSmallTake - 32;

struct SelBins {
  uint32_t top;
  int shift;
  __device__ __forceinline__ uint32_t bin(uint32_t key) const {
    return key >= top ? 0u : min((top - key) >> shift, (uint32_t)(kSelBins - 1));
  }
  // The smallest key of bin b (b < kSelBins - 1): keys at or above it lie in bins <= b.
  __device__ __forceinline__ uint32_t lowest(int b) const {
    const uint64_t edge = (uint64_t)(b + 1) << shift;
    return edge > top ? 0u : top - (uint32_t)edge + 1u;
  }
};

__device__ __forceinline__ SelBins sel_bins(uint32_t top, uint32_t bound) {
  const uint32_t range = top - min(bound, top);
  const int bits = range == 0 ? 0 : 32 - __clz((int)range);
  return SelBins{top, bits > 8 ? bits - 8 : 0};
}

// One wave's share of row `row`: slice `slice` of L.slice_len elements or, when `claim` is
// given (CLAIM), chunk `slice` of the whole row and then every chunk the wave claims from the
// LDS counter *claim (shared by the row's waves, starting past their first chunks), so that
// the row's waves end together however the SIMDs schedule them. Every statistic and list of
// the wave is independent of which elements it saw: the max, sum-exp to 1e-5, and a
// superset of the top kk of its elements. With CLAIM the row's `waves` waves (all of the
// workgroup, *claim starting at `waves`) also agree on a first bound through bound_keys (LDS
// room for 8 x 64 keys) and one barrier. The wave's top min(count, kk), sorted descending,
// go to out[0..keep) as composites (out may be sm.list itself: the list is read into
// registers before anything is written), its statistics to *stat.
template <typename In, int VEC, bool CLAIM>
__device__ __forceinline__ void wave_slice(WaveSmem &sm, const Launch &L, const tabby_row_params &P, int row,
                                           int slice, int part, uint64_t *out, SliceStat *stat, int *claim,
                                           uint32_t *bound_keys, int waves, bool sort_end = true,
                                           uint32_t *bound_out = nullptr, uint32_t *sel_hist = nullptr) {
  const int V = L.vocab;
  // CLAIM: the row, or part `part` of it (L.slice_len elements) when the row has several
  // workgroups.
  const int begin = CLAIM ? (L.parts > 1 ? part * L.slice_len : 0) : slice * L.slice_len;
  const int n = CLAIM && L.parts <= 1 ? V : min(L.slice_len, V - begin);
  const int nchunks = (n + kWChunk - 1) / kWChunk;
  const int full_chunks = n / kWChunk;
  const bool valid_params = params_valid(P, L.k_max);
  const int keff = effective_k(P, V);
  const int kk = slice_keep(valid_params, keff, n, L.kcap, L.head_pass, L.topk_cap);
  const In *src = reinterpret_cast<const In *>(L.logits) + (size_t)row * V + begin;
  const ChunkReader<In, VEC> rd(src, n);
  const int prune_at = kWListCap - kWaveSize;

  float lane_max = -INFINITY;
  float lane_ml = 0.0f;   // fl(lane_max * L): the reference of lane_sum's terms
  double lane_sum = 0.0;  // sum of 2^(x*L - lane_ml) over this lane's elements so far
  int count = 0;          // entries in the list; wave-uniform (readfirstlane keeps it scalar)
  uint32_t theta_key = kNegInfKey;
  float theta = -INFINITY;  // == value_of(theta_key)
  uint32_t union_top = kNegInfKey;  // CLAIM: the largest key of the first bound's union

  // Processes chunk c held in `cur` (the next chunk's loads are already in flight). `first`:
  // the wave's first chunk. The loops below issue each load unconditionally on their path,
  // so that the compiler's wait before a chunk's use leaves the next chunk in flight (a load
  // that is only conditionally issued makes it wait for every load).
  auto step = [&](int c, bool first, float (&cur)[kWChunkPerLane]) {
    const bool partial = c >= full_chunks;  // only the slice's last chunk can be partial
    if (partial) {
#pragma unroll
      for (int e = 0; e < kWChunkPerLane; ++e)
        if (wave_local<VEC>(c, e) >= n) cur[e] = -INFINITY;
    }
    float cm = cur[0];
#pragma unroll
    for (int e = 1; e < kWChunkPerLane; ++e) cm = fmaxf(cm, cur[e]);
    const float nm = fmaxf(lane_max, cm);
    if (nm != -INFINITY) {
      // The lane's terms are 2^(x*L - ml) with ml = fl(nm*L) (L = log2 e in f32), the
      // product x*L exact inside the fma; ml itself is the reference the sum is kept
      // against (lane_ml), so that its rounding -- about |nm| * 2^-24 -- does not scale the
      // terms: rescales subtract references, and the end of the slice subtracts the exact
      // product ms*L in f64. Errors then depend on x - max only, not on the max.
      const float ml = nm * kLog2e;
      // Pairwise sum: independent adds interleave with the exps (a running sum made one
      // dependent chain of 16 exp-add pairs per chunk).
      float t[kWChunkPerLane];
#pragma unroll
      for (int e = 0; e < kWChunkPerLane; ++e) t[e] = __builtin_amdgcn_exp2f(fmaf(cur[e], kLog2e, -ml));
#pragma unroll
      for (int h = kWChunkPerLane / 2; h > 0; h >>= 1) {
#pragma unroll
        for (int e = 0; e < h; ++e) t[e] += t[e + h];
      }
      const float part = t[0];
      const double rescale = lane_max == -INFINITY ? 0.0 : (double)__builtin_amdgcn_exp2f(lane_ml - ml);
      lane_sum = lane_sum * rescale + (double)part;
      lane_max = nm;
      lane_ml = ml;
    }
    if (kk == 0) return;
    if (first && kk < n && kk <= kWaveSize) {
      uint32_t k1[1] = {key_of(cm)};
      wave_sort_desc<1>(k1);
      theta_key = min(max((uint32_t)__builtin_amdgcn_readlane((int)k1[0], kk - 1), kNegInfKey), 0xff800000u);
      theta = value_of(theta_key);
    }
    // No lane reaches theta: nothing in this chunk can be a candidate.
    if (!__ballot(cm >= theta) && !partial) return;
    // Padding becomes NaN, which fails x >= theta for every theta, -inf included.
    if (partial) {
#pragma unroll
      for (int e = 0; e < kWChunkPerLane; ++e)
        if (wave_local<VEC>(c, e) >= n) cur[e] = __builtin_nanf("");
    }
    // Elements in groups of four: a group no lane's maximum reaches is skipped with one
    // branch (most chunks hold a candidate, but only in one or two of their groups).
#pragma unroll
    for (int g = 0; g < kWChunkPerLane / 4; ++g) {
      const float gm = fmaxf(fmaxf(cur[4 * g], cur[4 * g + 1]), fmaxf(cur[4 * g + 2], cur[4 * g + 3]));
      if (!__ballot(gm >= theta)) continue;  // NaN padding never reaches theta
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int e = 4 * g + q;
        if (count > prune_at) {
          const Pruned pr = wave_prune_any(sm, count, kk, theta_key);
          count = __builtin_amdgcn_readfirstlane(pr.count);
          theta_key = (uint32_t)__builtin_amdgcn_readfirstlane((int)pr.theta_key);
          theta = value_of(theta_key);
        }
        const bool take = cur[e] >= theta;
        const uint64_t mask = __ballot(take);
        if (mask) {
          if (take) sm.list[count + (int)lanes_below(mask)] = raw_entry(cur[e], (uint32_t)(begin + wave_local<VEC>(c, e)));
          count = __builtin_amdgcn_readfirstlane(count + (int)__popcll(mask));
        }
      }
    }
  };

  float x[kWChunkPerLane], y[kWChunkPerLane];
  if constexpr (CLAIM) {
    auto next = [&]() {
      int c = 0;
      if (wave_lane() == 0) c = atomicAdd(claim, 1);
      return __builtin_amdgcn_readfirstlane(c);
    };
    const int a = slice;
    rd.load(a, x);
    int b = next();
    rd.load(b, y);
    // The row's first bound, shared by its waves. A wave's 64 lane maxima over its first two
    // chunks are 64 distinct elements of the row; each wave publishes its m largest, and the
    // kk-th largest of the union (waves * m >= kk keys) has kk distinct elements at or above
    // it, so it never exceeds the row's kk-th largest. (The union is much tighter than any
    // one wave's offer: the row's top lane maxima are spread over the waves.) Every wave
    // passes the barrier once and computes the same bound.
    if (kk > 0) {
      const int regs = bound_regs(kk, waves);
      const int m = min(kWaveSize, kWaveSize * regs / waves);
      float cm = -INFINITY;
      if (a < nchunks) {
        if (a >= full_chunks) {
#pragma unroll
          for (int e = 0; e < kWChunkPerLane; ++e)
            if (wave_local<VEC>(a, e) >= n) x[e] = -INFINITY;
        }
#pragma unroll
        for (int e = 0; e < kWChunkPerLane; ++e) cm = fmaxf(cm, x[e]);
      }
      if (b < nchunks) {
        if (b >= full_chunks) {
#pragma unroll
          for (int e = 0; e < kWChunkPerLane; ++e)
            if (wave_local<VEC>(b, e) >= n) y[e] = -INFINITY;
        }
#pragma unroll
        for (int e = 0; e < kWChunkPerLane; ++e) cm = fmaxf(cm, y[e]);
      }
      uint32_t k1[1] = {key_of(cm)};
      wave_sort_desc<1>(k1);
      if (wave_lane() < m) bound_keys[slice * m + wave_lane()] = min(max(k1[0], kNegInfKey), 0xff800000u);
      __syncthreads();
      uint32_t t;
      switch (regs) {
        case 1: t = union_kth<1>(bound_keys, waves * m, kk, union_top); break;
        case 2: t = union_kth<2>(bound_keys, waves * m, kk, union_top); break;
        case 4: t = union_kth<4>(bound_keys, waves * m, kk, union_top); break;
        default: t = union_kth<8>(bound_keys, waves * m, kk, union_top); break;
      }
      theta_key = max(theta_key, t);
      theta = value_of(theta_key);
      union_top = max(union_top, theta_key);
      if (slice == 0) TABBY_STAMP(22);
      if (bound_out && slice == 0 && wave_lane() == 0) {
        bound_out[0] = theta_key;
        bound_out[1] = union_top;
      }
    } else {
      __syncthreads();
    }
    if (a < nchunks) step(a, false, x);  // chunk b is already in flight
    // y holds chunk b in flight at the top of each iteration.
    while (b < nchunks) {
      const int c = next();
      if (c >= nchunks) {
        step(b, false, y);
        break;
      }
      rd.load(c, x);
      step(b, false, y);
      b = next();
      if (b >= nchunks) {
        step(c, false, x);
        break;
      }
      rd.load(b, y);
      step(c, false, x);
    }
  } else {
    rd.load(0, x);
    for (int c = 0; c < nchunks; c += 2) {
      if (c + 1 >= nchunks) {
        step(c, c == 0, x);
        break;
      }
      rd.load(c + 1, y);
      step(c, c == 0, x);
      if (c + 2 >= nchunks) {
        step(c + 1, false, y);
        break;
      }
      rd.load(c + 2, x);
      step(c + 1, false, y);
    }
  }

  const float ms = wave_max(lane_max);
  const double ss = wave_sum(rebase_sum(lane_sum, lane_max, lane_ml, ms));
  // The slice's top min(count, kk), sorted descending: the merge only has to merge sorted
  // lists.
  int keep = 0;
  if (kk > 0 && !sort_end) {
    keep = count;  // the raw, unsorted list stays in sm.list for the caller
    if (sel_hist) {
      // Its keys into the row's selection histogram (finish_small_pool), bins counted down
      // from the largest key of the first bound's union.
      const SelBins sb = sel_bins(union_top, bound_out[0]);
      wave_lds_sync();
      for (int i = wave_lane(); i < count; i += kWaveSize) atomicAdd(&sel_hist[sb.bin(raw_key(sm.list[i]))], 1u);
    }
  } else if (kk > 0) {
    // Prune when the list is longer than kk's register class: the sort then stays in the
    // fewest registers (one for kk <= 64).
    if (count > kWaveSize * ((kk + kWaveSize - 1) / kWaveSize)) {
      const Pruned pr = wave_prune_any(sm, count, kk, theta_key);
      count = __builtin_amdgcn_readfirstlane(pr.count);
    }
    keep = min(count, kk);
    wave_lds_sync();
    if (count <= kWaveSize) store_sorted_top<1>(sm.list, count, keep, out);
    else if (count <= 2 * kWaveSize) store_sorted_top<2>(sm.list, count, keep, out);
    else if (count <= 4 * kWaveSize) store_sorted_top<4>(sm.list, count, keep, out);
    else store_sorted_top<8>(sm.list, count, keep, out);
  }
  if (wave_lane() == 0) {
    SliceStat st_out;
    st_out.max = ms;
    st_out.count = (uint32_t)keep;
    st_out.sum = ss;
    *stat = st_out;
  }
}

template <typename In, int VEC>
__global__ __launch_bounds__(kWaveSize) void wave_kernel(Launch L, Workspace W) {
  __shared__ WaveSmem sm;
  int row, slice;
  row_slice_of((int)blockIdx.x, L.rows, L.splits, row, slice);
  const tabby_row_params P = L.params[row];
  wave_slice<In, VEC, false>(sm, L, P, row, slice, 0,
                             W.cands + (size_t)row * W.row_cand_stride + (size_t)slice * L.list_stride,
                             W.stats + (size_t)row * kMaxSplits + slice, nullptr, nullptr, 0);
}

// Smallest key whose scaled logit (l - max)/T in f64 is >= -37.5 (the max's key when T <= 0:
// greedy needs only the row's maxima). Anything below has a weight exp(.) < e^-37.5 < 5.2e-17,
// below 2^-54 = 5.55e-17, and, added in sorted order, is below half an ulp of both sums it
// enters: the scaled total, which is >= 1 (its first term is exp(0)), and a running sum of
// the weights divided by that total, which is >= its first term 1/total while every later
// weight is < 2^-54/total. So it changes neither, and the draw never reaches it.
// The predicate is monotone in the key, so the answer is found from the f32 rounding of
// max - 37.5 T, which lies within a key or two of it, by stepping to the boundary (at most one
// step in 3 million random and edge-case (max, T) pairs checked against a bisection over the
// keys); a bisection of (kNegInfKey, top] stays as the fallback past 64 steps.
__device__ __forceinline__ uint32_t head_threshold(float row_max, double T) {
  const uint32_t top = key_of(row_max);
  if (greedy_temp(T)) return top;
  auto in_head = [&](uint32_t k) { return ((double)value_of(k) - (double)row_max) / T >= -37.5; };
  uint32_t c = min(max(key_of((float)((double)row_max - 37.5 * T)), kNegInfKey + 1u), top);
  int steps = 0;
  while (c < top && !in_head(c) && steps < 64) {
    ++c;
    ++steps;
  }
  while (c > kNegInfKey + 1u && in_head(c - 1u) && steps < 64) {
    --c;
    ++steps;
  }
  if (steps < 64) return c;
  uint32_t lo = kNegInfKey, hi = top;
  while (hi - lo > 1u) {
    const uint32_t mid = lo + (hi - lo) / 2u;
    if (in_head(mid)) hi = mid; else lo = mid;
  }
  return hi;
}

// ---------------------------------------------------------------------------------------
// Kernel 2 (merge): one workgroup per row. Row max and sum-exp from the slice statistics
// (in slice order, so the result does not depend on scheduling), the exact top-keff of the
// slices' candidates, an LDS bitonic sort, and sampleFromTopK.
// ---------------------------------------------------------------------------------------
constexpr int kCandLds = 4096;  // candidate lists up to this size are staged in LDS (two workgroups fit a CU)

template <int KCAP>
struct MergeSmem {
  BlockScratch bs;
  float row_max;
  double sum_exp;
  double pool_mass;
  double scaled_total;
  uint32_t slice_first[kMaxSplits];
  double slice_term[kMaxSplits];
  uint64_t sorted[KCAP];
  uint64_t cand[kCandLds];
  union {
    uint32_t hist[kBins];
    struct {
      double exact[KCAP];
      double w[KCAP];
    } tail;
  } u;
};

template <int KCAP, typename In>
__global__ __launch_bounds__(kBlock) void merge_kernel(Launch L, Workspace W) {
  __shared__ MergeSmem<KCAP> sm;
  const int row = (int)blockIdx.x;
  if (L.pool_rows && W.stats[(size_t)row * kMaxSplits].count == kPoolRowDone) return;
  const int splits = L.splits;
  const int V = L.vocab;
  const tabby_row_params P = L.params[row];
  const bool valid_params = params_valid(P, L.k_max);
  const int keff = effective_k(P, V);
  const bool finite = valid_params && keff <= L.kcap;
  const In *row_src = reinterpret_cast<const In *>(L.logits) + (size_t)row * V;

  // 0. Candidate counts per slice (in the statistics) and their offsets; then the
  //    candidate loads are issued together, ahead of the statistics math.
  const SliceStat *stats = W.stats + (size_t)row * kMaxSplits;
  SliceStat mine;
  mine.max = -INFINITY;
  mine.count = 0u;
  mine.sum = 0.0;
  if ((int)threadIdx.x < splits) mine = stats[threadIdx.x];
  uint32_t total_u;
  const bool collects = valid_params && (finite || L.head_pass);
  const uint32_t first = block_exclusive_scan(collects ? mine.count : 0u, sm.bs, &total_u);
  if ((int)threadIdx.x < splits) sm.slice_first[threadIdx.x] = first;
  __syncthreads();
  const int C = (int)total_u;
  const uint64_t *cands = W.cands + (size_t)row * W.row_cand_stride;
  // Flat candidate i lives in slice s (the last with slice_first[s] <= i), at
  // cands[s*slice_len + i - slice_first[s]].
  auto cand_addr = [&](int i) {
    int lo = 0, hi = splits - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if ((int)sm.slice_first[mid] <= i) lo = mid; else hi = mid - 1;
    }
    return cands + (size_t)lo * L.slice_len + (i - (int)sm.slice_first[lo]);
  };
  const bool staged = C <= kCandLds;
  if (staged) {
    constexpr int B = 8;
    for (int base = 0; base < C; base += B * kBlock) {
      uint64_t v[B];
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const int i = base + u * kBlock + (int)threadIdx.x;
        v[u] = i < C ? *cand_addr(i) : 0ull;
      }
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const int i = base + u * kBlock + (int)threadIdx.x;
        if (i < C) sm.cand[i] = v[u];
      }
    }
  }
  if (threadIdx.x == 0) {
    sm.bs.slot = 0u;
  }

  // 1. Row max and sum-exp, in slice order.
  const float M = block_max(mine.max, sm.bs);
  if ((int)threadIdx.x < splits)
    sm.slice_term[threadIdx.x] =
        mine.max == -INFINITY ? 0.0 : mine.sum * fdlibm_exp((double)mine.max - (double)M);
  __syncthreads();
  if (threadIdx.x == 0) {
    double S = 0.0;
    for (int s = 0; s < splits; ++s) S += sm.slice_term[s];
    sm.sum_exp = S;
  }
  __syncthreads();
  const float row_max = M;
  const double sum_exp = sm.sum_exp;
  const bool in_domain = (row_max > -INFINITY) && (row_max < INFINITY) && (sum_exp > 0.0) &&
                         (sum_exp < INFINITY);

  if (!valid_params || !in_domain) {
    if (threadIdx.x == 0) {
      write_status(L, row, !valid_params ? TABBY_EINVAL : TABBY_EDOMAIN, row_max, sum_exp);
      W.row_state[row].status = !valid_params ? TABBY_EINVAL : TABBY_EDOMAIN;
    }
    return;
  }
  if (!finite && !L.head_pass) {
    if (threadIdx.x == 0) write_status(L, row, TABBY_EINVAL, row_max, sum_exp);
    return;
  }
  // 2. The exact top-keff of the row's candidates, sorted. The candidates include every
  //    element of the row's top-keff (each slice kept all elements >= a lower bound of its
  //    own kk-th largest value).
  const uint32_t floor_key = kNegInfKey;
  auto from_lds = [&](auto &&f) {
    for (int i = threadIdx.x; i < C; i += kBlock) {
      const uint64_t v = sm.cand[i];
      if (composite_key(v) >= floor_key) f(v);
    }
  };
  auto from_global = [&](auto &&f) {
    constexpr int B = 8;  // loads in flight per lane before the first use
    for (int base = 0; base < C; base += B * kBlock) {
      uint64_t v[B];
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const int i = base + u * kBlock + (int)threadIdx.x;
        v[u] = i < C ? *cand_addr(i) : 0ull;
      }
#pragma unroll
      for (int u = 0; u < B; ++u)
        if (base + u * kBlock + (int)threadIdx.x < C && composite_key(v[u]) >= floor_key) f(v[u]);
    }
  };
  if (!finite) {
    // Whole-vocabulary row: hand max / sum-exp / the head threshold to the head kernels. The
    // candidates hold the row's top Nw = max(topk_cap, kHeadList) (slice_keep): when Nw fits a
    // wave's register sort (<= 256) they go on sorted, with the sequential sum of their terms,
    // to head_kernel and head_fast_kernel, as from finish_pool; the head also covers the
    // caller's top-k list, the first topk_cap of them.
    const int Nw = min(max(L.topk_cap, kHeadList), V);
    const int need = min(L.topk_cap, V);
    uint32_t list_key = 0xffffffffu;
    int handed = 0;
    if (Nw <= kWaveKcap && C >= Nw) {
      auto pick = [&](auto &&each) {
        if (threadIdx.x == 0) sm.bs.slot = 0u;
        __syncthreads();
        if (C > Nw) {
          const SelectResult r = radix_select(each, (uint32_t)Nw, sm.u.hist, sm.bs);
          each([&](uint64_t v) {
            const bool take = selected(v, r);
            const uint32_t at = wave_slot(take, &sm.bs.slot);
            if (take && at < (uint32_t)Nw) sm.sorted[at] = v;
          });
        } else {
          each([&](uint64_t v) {
            const uint32_t at = wave_slot(true, &sm.bs.slot);
            if (at < (uint32_t)Nw) sm.sorted[at] = v;
          });
        }
      };
      if (staged) pick(from_lds); else pick(from_global);
      const int npow = next_pow2(Nw);
      for (int i = Nw + (int)threadIdx.x; i < npow; i += kBlock) sm.sorted[i] = 0ull;
      __syncthreads();
      block_sort_desc(sm.sorted, npow);
      uint64_t *list = W.head_sorted + (size_t)row * W.head_stride;
      for (int i = threadIdx.x; i < Nw; i += kBlock) list[i] = sm.sorted[i];
      if (need > 0) list_key = composite_key(sm.sorted[need - 1]);
      handed = Nw;
    } else if (need > 0) {
      if (C >= need) {  // the candidates hold the row's top `need`: select the need-th largest
        const SelectResult r = staged ? radix_select(from_lds, (uint32_t)need, sm.u.hist, sm.bs)
                                      : radix_select(from_global, (uint32_t)need, sm.u.hist, sm.bs);
        // Every selected composite is >= r.prefix, whose low bits below r.shift are zero.
        list_key = (uint32_t)(r.prefix >> 32);
      } else {
        list_key = kNegInfKey;  // fewer candidates than the list: take the whole row
      }
    }
    if (wave_id() != 0) return;
    const double T = P.temperature;
    double list_sum = 0.0;
    if (handed > 0 && !greedy_temp(T)) {
      double *terms = sm.u.tail.w;  // the histogram is no longer needed
      for (int i = lane_id(); i < handed; i += kWaveSize)
        terms[i] = fdlibm_exp(((double)value_of(composite_key(sm.sorted[i])) - (double)row_max) / T);
      wave_lds_sync();
      list_sum = wave_seq_sum(terms, handed, nullptr, INFINITY).total;
    }
    if (lane_id() == 0) {
      RowState rs;
      rs.max = row_max;
      rs.sum_exp = sum_exp;
      rs.status = TABBY_OK;
      rs.handoff = (uint32_t)handed << 16;
      rs.list_sum = list_sum;
      rs.head_key = min(head_threshold(row_max, P.temperature), list_key);
      W.row_state[row] = rs;
    }
    return;
  }
  auto gather = [&](auto &&each) {
    if (C > keff) {
      const SelectResult r = radix_select(each, (uint32_t)keff, sm.u.hist, sm.bs);
      each([&](uint64_t v) {
        const bool take = selected(v, r);
        const uint32_t at = wave_slot(take, &sm.bs.slot);
        if (take && at < (uint32_t)keff) sm.sorted[at] = v;
      });
    } else {
      each([&](uint64_t v) {
        const uint32_t at = wave_slot(true, &sm.bs.slot);
        if (at < (uint32_t)keff) sm.sorted[at] = v;
      });
    }
  };
  if (staged) gather(from_lds); else gather(from_global);
  __syncthreads();

  // 3. Sort and sampleFromTopK: by wave 0 in registers for pools up to 256, else by the
  //    workgroup through LDS.
  if (keff <= kWaveKcap) {
    if (wave_id() != 0) return;
    if (keff <= 64) wave_finish<1, In>(sm.sorted, keff, L, row, row_src, row_max, sum_exp, P);
    else if (keff <= 128) wave_finish<2, In>(sm.sorted, keff, L, row, row_src, row_max, sum_exp, P);
    else wave_finish<4, In>(sm.sorted, keff, L, row, row_src, row_max, sum_exp, P);
    return;
  }
  const int npow = next_pow2(keff);
  for (int i = keff + (int)threadIdx.x; i < npow; i += kBlock) sm.sorted[i] = 0ull;
  __syncthreads();
  block_sort_desc(sm.sorted, npow);
  finish_row<KCAP, In>(sm, L, row, row_src, keff, row_max, sum_exp, P);
}

// ---------------------------------------------------------------------------------------
// Kernel 2 for pools of at most 256 (wave_merge_kernel): one 256-lane workgroup per row.
// Every slice left its top min(kk, count) candidates sorted descending, so the row's top-k is
// a merge of sorted lists: the accumulator (the first list) and each further list, loaded
// reversed, give max(a_i, b_(n-1-i)) -- the top n of their union as a bitonic sequence --
// which a bitonic clean (register strides, then lane strides through DPP / permlane) sorts
// again. Each wave merges a quarter of the lists, then a two-level tree through LDS. The
// slice statistics and the head of every list are loaded in one round trip; the f64 tail of
// sampleFromTopK then runs from LDS: the two independent sums on two waves, the running sums
// on one, each evaluated bit-exactly by the whole wave (seqsum.h).
// ---------------------------------------------------------------------------------------
struct WaveMergeSmem {
  uint64_t sorted[kWaveKcap];
  double a[kWaveKcap];  // exact terms exp(l - max) / sumExp
  double b[kWaveKcap];  // exp((l - max) / T), then the weights
  double c[kWaveKcap];  // running sums of the weights
  uint64_t part[kWaves][kWaveKcap];  // each wave's merged lists
  double pool;                       // poolMass
  int cut, chosen;                   // consideredCount and the drawn position
  float row_max;                     // row statistics, when a separate wave combines them
  double row_sum;
};

// Bitonic clean of 64*R values (index r*64 + lane) into descending order.
template <int R>
__device__ __forceinline__ void bitonic_clean_desc(uint64_t (&a)[R]) {
#pragma unroll
  for (int rs = R / 2; rs > 0; rs >>= 1) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if ((r & rs) == 0) {
        const uint64_t x = a[r], y = a[r | rs];
        a[r] = tmax(x, y);
        a[r | rs] = tmin(x, y);
      }
    }
  }
  const int lane = wave_lane();
#pragma unroll
  for (int stride = kWaveSize / 2; stride > 0; stride >>= 1) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      a[r] = cmpx(a[r], xor_lane_by(a[r], stride), (lane & stride) == 0);
    }
  }
}

// Row statistics from the slice statistics: max, and sum-exp as a fixed butterfly over the
// slices' rescaled sums (deterministic for given inputs). Lane s holds slices s, s + 64, ...
struct RowStats {
  float max;
  double sum_exp;
  uint32_t cnt[kMaxSplits / kWaveSize];  // list lengths, by lane
};

__device__ __forceinline__ RowStats row_stats(const SliceStat *stats, int splits) {
  const int lane = wave_lane();
  SliceStat st[kMaxSplits / kWaveSize];
#pragma unroll
  for (int q = 0; q < kMaxSplits / kWaveSize; ++q) {
    const int s = q * kWaveSize + lane;
    st[q].max = -INFINITY;
    st[q].count = 0u;
    st[q].sum = 0.0;
    if (s < splits) st[q] = stats[s];
  }
  RowStats out;
  float m = -INFINITY;
#pragma unroll
  for (int q = 0; q < kMaxSplits / kWaveSize; ++q) {
    out.cnt[q] = st[q].count;
    m = fmaxf(m, st[q].max);
  }
  out.max = wave_max(m);
  double part = 0.0;
#pragma unroll
  for (int q = 0; q < kMaxSplits / kWaveSize; ++q)
    if (st[q].max != -INFINITY)  // sum-exp is compared within 1e-5: an f32 exp2 rescale will do
      part += st[q].sum * (double)__builtin_amdgcn_exp2f((st[q].max - out.max) * kLog2e);
  out.sum_exp = wave_sum(part);
  return out;
}

// Length of slice s's list (s wave-uniform).
__device__ __forceinline__ int list_count(const RowStats &rs, int s) {
  // One readlane per register and a scalar select (an indexed register array would be
  // placed in scratch memory).
  const int l = s % kWaveSize, q = s / kWaveSize;
  const int c0 = __builtin_amdgcn_readlane((int)rs.cnt[0], l);
  if (q == 0) return c0;
  const int c1 = __builtin_amdgcn_readlane((int)rs.cnt[1], l);
  const int c2 = __builtin_amdgcn_readlane((int)rs.cnt[2], l);
  const int c3 = __builtin_amdgcn_readlane((int)rs.cnt[3], l);
  return q == 1 ? c1 : q == 2 ? c2 : c3;
}

// Merges the sorted slice lists s_begin..s_end-1 of a row into the top 64*R composites,
// sorted descending, in registers (all zero without lists). Slice s's list starts at
// base + s*slice_len and holds count_of(s) entries; reads stay inside the row's row_stride
// entries, and entries past a list's end are masked.
template <int R>
struct ListMerger {
  static constexpr int kBatch = 4;  // lists whose loads are in flight together
  const uint64_t *base;
  int slice_len;
  int64_t row_stride;
  int s_begin, s_end;
  bool tree;  // at most 4 lists: loaded alternately descending and reversed for finish_tree
  uint64_t acc[R];
  uint64_t raw[kBatch][R];

  __device__ __forceinline__ void issue(int s, uint64_t (&dst)[R], bool reversed) const {
    const uint64_t *list = base + (int64_t)s * slice_len;
    const int room = (int)min((int64_t)slice_len, row_stride - (int64_t)s * slice_len);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int p = r * kWaveSize + wave_lane();
      const int j = reversed ? kWaveSize * R - 1 - p : p;
      dst[r] = list[min(j, room - 1)];
    }
  }
  __device__ __forceinline__ static void mask(int n, uint64_t (&v)[R], bool reversed) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int p = r * kWaveSize + wave_lane();
      const int j = reversed ? kWaveSize * R - 1 - p : p;
      if (j >= n) v[r] = 0ull;
    }
  }
  // Issues the first lists' loads (nothing is waited for).
  __device__ __forceinline__ void start() {
    if (s_begin < s_end) issue(s_begin, acc, false);
#pragma unroll
    for (int q = 0; q < kBatch; ++q)
      if (s_begin + 1 + q < s_end) issue(s_begin + 1 + q, raw[q], !tree || (q & 1) == 0);
  }
  // The top 64 of at most four lists (R == 1) by a two-level tree: lists 0 and 1, and 2 and
  // 3, merge side by side (the first pair cleaned descending, the second ascending, so that
  // the two results again form a bitonic sequence), then the pair results merge.
  template <class CountOf>
  __device__ __forceinline__ void finish_tree(CountOf count_of) {
    static_assert(R == 1, "one register per list");
    const int n = s_end - s_begin;
    uint64_t v[4] = {0ull, 0ull, 0ull, 0ull};
    if (n > 0) {
      v[0] = acc[0];
      uint64_t t[1] = {v[0]};
      mask(count_of(s_begin), t, false);
      v[0] = t[0];
    }
#pragma unroll
    for (int j = 1; j < 4; ++j) {
      if (j < n) {
        uint64_t t[1] = {raw[j - 1][0]};
        mask(count_of(s_begin + j), t, (j & 1) != 0);
        v[j] = t[0];
      }
    }
    uint64_t a = tmax(v[0], v[1]), b = tmax(v[2], v[3]);
    const int lane = wave_lane();
    if (n > 2) {
#pragma unroll
      for (int stride = kWaveSize / 2; stride > 0; stride >>= 1) {
        const uint64_t oa = xor_lane_by(a, stride), ob = xor_lane_by(b, stride);
        const bool lower = (lane & stride) == 0;
        a = cmpx(a, oa, lower);   // descending
        b = cmpx(b, ob, !lower);  // ascending
      }
      a = tmax(a, b);
    }
    acc[0] = a;
    if (n > 1) bitonic_clean_desc<1>(acc);
  }
  template <class CountOf>
  __device__ __forceinline__ void finish(CountOf count_of) {
    if (s_begin >= s_end) {
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = 0ull;
      return;
    }
    mask(count_of(s_begin), acc, false);
    for (int s0 = s_begin + 1; s0 < s_end; s0 += kBatch) {
#pragma unroll
      for (int q = 0; q < kBatch; ++q) {
        const int s = s0 + q;
        if (s < s_end) {
          uint64_t b[R];
#pragma unroll
          for (int r = 0; r < R; ++r) b[r] = raw[q][r];
          if (s + kBatch < s_end) issue(s + kBatch, raw[q], true);
          mask(count_of(s), b, true);
#pragma unroll
          for (int r = 0; r < R; ++r) acc[r] = tmax(acc[r], b[r]);
          bitonic_clean_desc<R>(acc);
        }
      }
    }
  }
};

// acc <- the top 64*R of acc and the sorted list `other` (64*R entries, in LDS), sorted.
template <int R>
__device__ __forceinline__ void merge_with(uint64_t (&acc)[R], const uint64_t *other) {
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = tmax(acc[r], other[kWaveSize * R - 1 - (r * kWaveSize + wave_lane())]);
  bitonic_clean_desc<R>(acc);
}

// The draw of sampleFromTopK (src/engine/sampler.ts:170-203) over sm.sorted[0..K), K >= 1,
// by the wave that has just left the weights exp(x/T) in sm.b with their left-to-right sum
// `scaled`: the normalised weights, their running sums (the top-p cumulative sums, evaluated
// bit-exactly by the whole wave: wave_seq_sum) up to the first that reaches top-p -- the
// cut -- and the first running sum above uniform * total. Leaves sm.cut and sm.chosen.
__device__ __forceinline__ void wave_draw(WaveMergeSmem &sm, int K, const tabby_row_params &P, double scaled) {
  const int lane = wave_lane();
  for (int i = lane; i < K; i += kWaveSize) sm.b[i] = sm.b[i] / scaled;
  wave_lds_sync();
  const double top_p = P.top_p;
  const SeqSum run = wave_seq_sum(sm.b, K, sm.c, top_p < 1.0 ? top_p : INFINITY);
  wave_lds_sync();
  const int cut = run.count;
  const double total = run.total;  // the running sum at cut - 1: the reference's total
  const double target = P.uniform * total;
  int chosen = cut - 1;
  for (int base = 0; base < cut; base += kWaveSize) {
    const int i = base + lane;
    const uint64_t hit = __ballot(i < cut && target < sm.c[min(i, cut - 1)]);
    if (hit) {
      chosen = base + __ffsll((unsigned long long)hit) - 1;
      break;
    }
  }
  if (lane == 0) {
    sm.cut = cut;
    sm.chosen = chosen;
  }
}

// The row's result (src/engine/sampler.ts:147-212) once the other passes are done: the exact
// terms exp(x - max)/sum_exp in sm.a with their sum in sm.pool (poolMass) and, for T > 0,
// the draw's sm.cut and sm.chosen (wave_draw); T <= 0 is greedy (sampler.ts:159-167).
template <typename In>
__device__ __forceinline__ void wave_tail(WaveMergeSmem &sm, int K, const Launch &L, int row,
                                          const In *row_src, float max_logit, double sum_exp,
                                          const tabby_row_params &P) {
  const int lane = wave_lane();
  const double T = P.temperature;
  const double pool = sm.pool;
  tabby_row_result res;
  res.max_logit = max_logit;
  res.sum_exp = sum_exp;
  res.pool_mass = pool;
  res.status = TABBY_OK;
  res.topk_count = min(K, L.topk_cap);
  int chosen = 0;
  if (greedy_temp(T)) {  // greedy, the uniform unused
    res.considered = 1;
    res.pool_exhausted = 0;
  } else {
    chosen = sm.chosen;
    res.considered = (uint32_t)sm.cut;
    res.pool_exhausted = (P.top_p < 1.0 && pool < P.top_p) ? 1 : 0;
  }
  const uint64_t cv = sm.sorted[chosen];
  res.id = (int32_t)composite_index(cv);
  res.probability = sm.a[chosen];
  if (lane == 0) L.results[row] = res;
  if (L.topk_cap > 0) {
    const int m = min(K, L.topk_cap);
    for (int i = lane; i < m; i += kWaveSize) {
      const uint32_t idx = composite_index(sm.sorted[i]);
      L.topk_ids[(size_t)row * L.topk_cap + i] = (int32_t)idx;
      L.topk_logits[(size_t)row * L.topk_cap + i] = load_one(row_src + min(idx, (uint32_t)(L.vocab - 1)));
    }
  }
}

// The first four waves of the workgroup each merge a quarter of the row's lists (their
// loads issued by the caller); then a two-level tree through LDS merges the four results
// into sm.sorted[0..K). Further waves only take part in the barriers.
template <int R, class CountOf>
__device__ __forceinline__ void merge_lists_4(WaveMergeSmem &sm, ListMerger<R> &mg, CountOf count_of,
                                              int K) {
  const int w = wave_id(), lane = wave_lane();
  if constexpr (R == 1) {
    if (mg.tree) mg.finish_tree(count_of); else mg.finish(count_of);
  } else {
    mg.finish(count_of);
  }
  if (w < kWaves) {
#pragma unroll
    for (int r = 0; r < R; ++r) sm.part[w][r * kWaveSize + lane] = mg.acc[r];
  }
  __syncthreads();
  if (w == 0 || w == 2) {
    merge_with<R>(mg.acc, sm.part[w + 1]);
    if (w == 2) {
#pragma unroll
      for (int r = 0; r < R; ++r) sm.part[2][r * kWaveSize + lane] = mg.acc[r];
    }
  }
  __syncthreads();
  if (w == 0) {
    merge_with<R>(mg.acc, sm.part[2]);
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (r * kWaveSize + lane < K) sm.sorted[r * kWaveSize + lane] = mg.acc[r];
  }
  __syncthreads();
}

// Where a row's lists lie: list s at base + s * stride, all inside base[0..room).
struct RowLists {
  const uint64_t *base;
  int count;
  int stride;
  int64_t room;
};

template <int R>
__device__ __forceinline__ ListMerger<R> lists_of_wave(const RowLists &rl) {
  const int per = (rl.count + kWaves - 1) / kWaves;
  ListMerger<R> mg;
  mg.base = rl.base;
  mg.slice_len = rl.stride;
  mg.row_stride = rl.room;
  mg.s_begin = min(wave_id() * per, rl.count);  // waves past the fourth get no lists
  mg.s_end = min(mg.s_begin + per, rl.count);
  mg.tree = R == 1 && per <= 4;
  return mg;
}

// The pool a row's merge builds: its top-k, or for a whole-vocabulary row the caller's
// top-k list (finished later by the head kernels).
struct RowPool {
  bool valid;   // parameters valid
  bool finite;  // the pool is the row's top-k (not a whole-vocabulary row)
  int K;        // pool entries to merge
};

__device__ __forceinline__ RowPool row_pool(const Launch &L, const tabby_row_params &P) {
  RowPool rp;
  rp.valid = params_valid(P, L.k_max);
  const int keff = effective_k(P, L.vocab);
  rp.finite = rp.valid && keff <= L.kcap;
  rp.K = !rp.valid ? 0 : rp.finite ? keff : L.head_pass ? min(max(L.topk_cap, kHeadList), L.vocab) : 0;
  return rp;
}

template <typename In, bool REG = false>
__device__ __forceinline__ void finish_pool(WaveMergeSmem &sm, const Launch &L, const Workspace &W, int row,
                                            const tabby_row_params &P, const RowPool &rp, float row_max,
                                            double sum_exp);

template <typename In, class SumExp>
__device__ __forceinline__ void reg_tail(uint64_t v, int K, const Launch &L, int row, const In *row_src,
                                         float M, SumExp sum_exp_of, const tabby_row_params &P);

template <int R, typename In, class SumExp>
__device__ __forceinline__ void reg_tail_wide(const uint64_t (&v)[R], int K, const Launch &L, int row,
                                              const In *row_src, float M, SumExp sum_exp_of,
                                              const tabby_row_params &P, double *scratch);

// The row's top K, sorted, into sm.sorted[0..K) from its sorted lists (merge_lists_4 in the
// register class of K; m1: the first 64 entries' loads, already issued). No barrier when
// K == 0.
template <class CountOf>
__device__ __forceinline__ void merge_pool(WaveMergeSmem &sm, const RowLists &lists, ListMerger<1> &m1,
                                           CountOf count_of, int K) {
  if (K <= 0) return;
  if (K <= kWaveSize) {
    merge_lists_4<1>(sm, m1, count_of, K);
  } else if (K <= 2 * kWaveSize) {
    ListMerger<2> m2 = lists_of_wave<2>(lists);
    m2.start();
    merge_lists_4<2>(sm, m2, count_of, K);
  } else {
    ListMerger<4> m4 = lists_of_wave<4>(lists);
    m4.start();
    merge_lists_4<4>(sm, m4, count_of, K);
  }
}

// Merges row `row`'s sorted slice lists and statistics and finishes the row (at least four
// waves; the lists and statistics are in global memory or in LDS; P is the row's parameters).
template <typename In>
__device__ __forceinline__ void merge_row(WaveMergeSmem &sm, const Launch &L, const Workspace &W, int row,
                                          const tabby_row_params &P, const SliceStat *stats,
                                          const RowLists &lists) {
  // The lists' first 64 entries are loaded before the pool size is known: pools of at most
  // 64 (the common case) then need no second round trip.
  ListMerger<1> m1 = lists_of_wave<1>(lists);
  m1.start();
  const RowStats rs = row_stats(stats, lists.count);
  auto count_of = [&](int s) { return list_count(rs, s); };
  const RowPool rp = row_pool(L, P);
  merge_pool(sm, lists, m1, count_of, rp.K);
  finish_pool<In, true>(sm, L, W, row, P, rp, rs.max, rs.sum_exp);
}

// The rest of a row once its pool, sm.sorted[0..K), and its max and sum-exp are known: the
// f64 tail of sampleFromTopK, the hand-over to the head kernels, or an error status. Wave 0
// and wave 1 work; every wave of the workgroup must call it. REG: finite pools take wave 0's
// register tail (the merge kernels; row_kernel's small pools end in finish_small_pool, and
// its general path keeps the two-wave form).
template <typename In, bool REG>
__device__ __forceinline__ void finish_pool(WaveMergeSmem &sm, const Launch &L, const Workspace &W, int row,
                                            const tabby_row_params &P, const RowPool &rp, float row_max,
                                            double sum_exp) {
  const int lane = wave_lane();
  const int K = rp.K;
  const bool valid_params = rp.valid, finite = rp.finite;
  const In *row_src = reinterpret_cast<const In *>(L.logits) + (size_t)row * L.vocab;
  const bool in_domain = (row_max > -INFINITY) && (row_max < INFINITY) && (sum_exp > 0.0) &&
                         (sum_exp < INFINITY);
  if (REG && valid_params && in_domain && finite) {
    // Wave 0's register tail: one, two or four registers per lane.
    if (wave_id() != 0) return;
    auto S1_of = [&]() { return sum_exp; };
    if (K <= kWaveSize) {
      reg_tail<In>(lane < K ? sm.sorted[lane] : 0ull, K, L, row, row_src, row_max, S1_of, P);
    } else if (K <= 2 * kWaveSize) {
      const uint64_t v[2] = {sm.sorted[lane], kWaveSize + lane < K ? sm.sorted[kWaveSize + lane] : 0ull};
      reg_tail_wide<2, In>(v, K, L, row, row_src, row_max, S1_of, P, sm.b);
    } else {
      uint64_t v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = r * kWaveSize + lane < K ? sm.sorted[r * kWaveSize + lane] : 0ull;
      reg_tail_wide<4, In>(v, K, L, row, row_src, row_max, S1_of, P, sm.b);
    }
    return;
  }
  if (valid_params && in_domain && finite) {
    // sampleFromTopK's two independent passes over the pool (sampler.ts:156-157, 170-172)
    // on two waves: wave 0 the exact terms and poolMass, wave 1 the scaled terms and their
    // total, each a left-to-right sum; wave 1 goes on to the draw.
    const int w = wave_id();
    const double M = (double)row_max, T = P.temperature;
    if (w == 0) {
      for (int i = lane; i < K; i += kWaveSize)
        sm.a[i] = fdlibm_exp_inline((double)value_of(composite_key(sm.sorted[i])) - M) / sum_exp;
      wave_lds_sync();
      const double pool = wave_seq_sum(sm.a, K, nullptr, INFINITY).total;
      if (lane == 0) sm.pool = pool;
    } else if (w == 1) {
      for (int i = lane; i < K; i += kWaveSize)
        sm.b[i] = !greedy_temp(T) ? fdlibm_exp_inline(((double)value_of(composite_key(sm.sorted[i])) - M) / T) : 0.0;
      wave_lds_sync();
      if (!greedy_temp(T)) wave_draw(sm, K, P, wave_seq_sum(sm.b, K, nullptr, INFINITY).total);
    }
    __syncthreads();
  }
  if (wave_id() != 0) return;
  if (!valid_params || !in_domain || (!finite && !L.head_pass)) {
    const int32_t status = !valid_params ? TABBY_EINVAL : !in_domain ? TABBY_EDOMAIN : TABBY_EINVAL;
    if (lane == 0) {
      write_status(L, row, status, row_max, sum_exp);
      W.row_state[row].status = status;
    }
    return;
  }
  if (!finite) {
    // Whole-vocabulary row: hand max / sum-exp / the head threshold to the head kernels, and
    // the row's top K, sorted[0..K), to head_kernel and head_fast_kernel. The head also
    // covers the caller's top-k list, the first topk_cap of them.
    uint64_t *list = W.head_sorted + (size_t)row * W.head_stride;
    const double T = P.temperature;
    for (int i = lane; i < K; i += kWaveSize) {
      list[i] = sm.sorted[i];
      if (!greedy_temp(T)) sm.b[i] = fdlibm_exp_inline(((double)value_of(composite_key(sm.sorted[i])) - (double)row_max) / T);
    }
    wave_lds_sync();
    const double list_sum = !greedy_temp(T) && K > 0 ? wave_seq_sum(sm.b, K, nullptr, INFINITY).total : 0.0;
    if (lane == 0) {
      RowState st;
      st.max = row_max;
      st.sum_exp = sum_exp;
      st.status = TABBY_OK;
      st.handoff = (uint32_t)K << 16;
      st.list_sum = list_sum;
      const int kt = min(L.topk_cap, K);  // the caller's top-k list must lie in the head
      const uint32_t list_key = kt > 0 ? composite_key(sm.sorted[kt - 1]) : 0xffffffffu;
      st.head_key = min(head_threshold(row_max, P.temperature), list_key);
      W.row_state[row] = st;
    }
    return;
  }
  wave_tail<In>(sm, K, L, row, row_src, row_max, sum_exp, P);
}

template <typename In>
__global__ __launch_bounds__(kBlock) void wave_merge_kernel(Launch L, Workspace W) {
  __shared__ WaveMergeSmem sm;
  const int row = (int)blockIdx.x;
  const RowLists lists{W.cands + (size_t)row * W.row_cand_stride, L.splits, L.list_stride, W.row_cand_stride};
  const tabby_row_params P = L.params[row];
  merge_row<In>(sm, L, W, row, P, W.stats + (size_t)row * kMaxSplits, lists);
}

// ---------------------------------------------------------------------------------------
// Batches of at least as many rows as the chip has CUs (pools of at most 256): one
// workgroup per row of max(L.splits, kRowMinWaves) <= kRowWaves waves (the merge below
// uses five), which take the row's chunks from an LDS
// counter (wave_slice with CLAIM) and leave their sorted lists and statistics in LDS; after
// one barrier the first four waves merge the lists as wave_merge_kernel does, reading their
// lengths from LDS, while the fifth combines the statistics. Nothing goes through
// global memory between the two halves, the row finishes as soon as its own chunks are done
// instead of after every row's, and its waves end within about a chunk of each other (with
// fixed slices, the SIMDs' oldest-first issue left the youngest waves ~8 us behind).
// (A tournament -- each finished wave merging with its sibling through an LDS counter, so
// that the lower levels overlap the last waves' streaming -- was measured slower: each level
// is a chain of dependent LDS round trips before its merge.)
// ---------------------------------------------------------------------------------------
constexpr int kRowWaves = 16;
constexpr int kRowMinWaves = kWaves + 1;  // four merge the lists, one the statistics

struct RowSmem {
  WaveSmem wave[kRowWaves];
  SliceStat stats[kRowWaves];
  WaveMergeSmem merge;
  int next_chunk;
  uint32_t bound_keys[8 * kWaveSize];
  // Pools of at most 64 (finish_small_pool): the key histogram over every wave's list, the
  // selected entries and their count, and the row's shared first bound.
  uint32_t sel_hist[kSelBins];
  uint64_t sel[kSmallTake];
  int sel_count;
  uint32_t fin_mask;     // the waves finished streaming (the last one selects the take)
  uint32_t sel_take[2];  // the take's smallest key and its size
  uint32_t part_mask;    // the waves whose statistics the second-to-last one combined ...
  float part_max;        // ... their max
  double part_sum;       // ... and sum-exp against it
  uint32_t bound_key[2];  // the row's first bound and the largest key of its union
};

// The decisions of sampleFromTopK's draw (src/engine/sampler.ts:170-203) from the running sums
// of the weights held one per lane (lane i: the i-th running sum, lanes >= K unused): the cut
// (the first running sum reaching top-p, +1; K without one) and the draw (the first i < cut
// whose running sum exceeds uniform * the running sum at cut - 1; cut - 1 without one).
struct Draw {
  int cut, chosen;
  double total, target;
};

__device__ __forceinline__ Draw draw_of(double running, int K, double top_p, double uniform) {
  const int lane = wave_lane();
  Draw d;
  const uint64_t reach = top_p < 1.0 ? __ballot(lane < K && running >= top_p) : 0ull;
  d.cut = reach ? __ffsll((unsigned long long)reach) : K;
  d.total = lane_f64(running, d.cut - 1);
  d.target = uniform * d.total;
  const uint64_t hit = __ballot(lane < d.cut && d.target < running);
  d.chosen = hit ? __ffsll((unsigned long long)hit) - 1 : d.cut - 1;
  return d;
}

// sampleFromTopK (src/engine/sampler.ts:147-212) over a pool of K <= 64 candidates sorted
// descending one per lane (lane i holds the i-th largest composite), by one wave in registers.
// The reference's sums are sequential left-to-right f64 sums and the cut and the draw depend
// on their last bits. Here the terms s_i come from exp_nonpos (within 8 ulp of exp), their
// prefix sums P_i from one parallel scan (wave_inclusive_scan2: a tree of at most six
// roundings, interleaved with the scan of the exact terms for poolMass), and the running sum
// of the weights is P_i / P_(K-1), within 29 * 2^-53 of the exact ratio. The reference's
// running sums of its weights (V8's exp within an ulp, then K sequential roundings for the
// total, one for each weight, i for the running sum) are within 130 * 2^-53 of the same
// ratio, so the two differ by less than 2^-45.6 of their value: when every comparison that
// decides the cut and the draw clears its threshold by more than 2^-36 relative, the
// reference decides the same way. Each lane checks its own running sum against the
// comparisons it takes part in (the cut's and the chosen entry's, and those just below them)
// and one ballot collects the failures. Otherwise the weights are recomputed with V8's exp
// (fdlibm) and summed bit for bit (reg_seq_sum), and decided again. poolMass and the
// probability (compared within 1e-5) keep the fast terms. T <= 0 is greedy
// (sampler.ts:159-167). S1 is the row's sum-exp (the caller may have computed it already).
template <typename In, class SumExp>
__device__ __forceinline__ void reg_tail(uint64_t v, int K, const Launch &L, int row, const In *row_src,
                                         float M, SumExp sum_exp_of, const tabby_row_params &P) {
  const int lane = wave_lane();
  const bool in = lane < K;
  const double T = P.temperature;
  const double d = (double)value_of(composite_key(v)) - (double)M;
  const double e1 = in ? exp_nonpos(d) : 0.0;
  const double s = (!in || greedy_temp(T)) ? 0.0 : T == 1.0 ? e1 : exp_nonpos(d / T);
  const double S1 = sum_exp_of();
  const double exact = e1 / S1;
  TABBY_STAMP(23);
  double pe = exact, ps = s;
  wave_inclusive_scan2(pe, ps);  // lanes >= K add zeros
  const double pool = lane_f64(pe, K - 1);
  TABBY_STAMP(26);
  tabby_row_result res;
  res.max_logit = M;
  res.sum_exp = S1;
  res.pool_mass = pool;
  res.status = TABBY_OK;
  res.topk_count = min(K, L.topk_cap);
  int chosen = 0;
  if (greedy_temp(T)) {
    res.considered = 1;
    res.pool_exhausted = 0;
  } else {
    const double top_p = P.top_p;
    const double scaled = lane_f64(ps, K - 1);
    const double running = in ? ps / scaled : 0.0;
    Draw dr = draw_of(running, K, top_p, P.uniform);
    TABBY_STAMP(27);
    // Margins of every comparison that fixed the cut and the draw (running sums are
    // non-decreasing, so the neighbours of each boundary are the only ones to check), each
    // lane testing the ones its own running sum decides.
    constexpr double kMargin = 1.0 / 68719476736.0;  // 2^-36
    bool fail = false;
    if (top_p < 1.0) {
      const double m = kMargin * top_p;
      if (dr.cut == K) fail = lane == K - 1 && !(running < top_p - m);
      else fail = (lane == dr.cut - 1 && !(running >= top_p + m)) || (lane == dr.cut - 2 && !(running < top_p - m));
    }
    const double m2 = kMargin * dr.total;
    fail = fail || (lane == dr.chosen && !(running > dr.target + m2)) ||
           (lane == dr.chosen - 1 && !(running < dr.target - m2));
    if (__ballot(fail)) {
      // Bit for bit: V8's exp for the weights, sequential sums (sampler.ts:170-203).
      const double se = in ? fdlibm_exp_inline(d / T) : 0.0;
      double partial;
      const double S = reg_seq_sum(se, K, INFINITY, &partial).total;
      const double w = in ? se / S : 0.0;
      double exact_running;
      const SeqSum run = reg_seq_sum(w, K, top_p < 1.0 ? top_p : INFINITY, &exact_running);
      dr.cut = run.count;
      dr.total = run.total;
      dr.target = P.uniform * dr.total;
      const uint64_t hit = __ballot(lane < dr.cut && dr.target < exact_running);
      dr.chosen = hit ? __ffsll((unsigned long long)hit) - 1 : dr.cut - 1;
    }
    chosen = dr.chosen;
    res.considered = (uint32_t)dr.cut;
    res.pool_exhausted = (top_p < 1.0 && pool < top_p) ? 1 : 0;
    TABBY_STAMP(28);
  }
  const uint64_t cv = (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, chosen) |
                      ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), chosen) << 32);
  res.id = (int32_t)composite_index(cv);
  res.probability = lane_f64(exact, chosen);
  if (lane == 0) L.results[row] = res;
  if (in && lane < L.topk_cap) {
    const uint32_t idx = composite_index(v);
    L.topk_ids[(size_t)row * L.topk_cap + lane] = (int32_t)idx;
    L.topk_logits[(size_t)row * L.topk_cap + lane] = load_one(row_src + min(idx, (uint32_t)(L.vocab - 1)));
  }
}

// reg_tail for pools of 65..64R (R registers per lane; entry i = r * 64 + lane, sorted
// descending over i). The prefix sums are the wave's scans of each register (the exact and
// the scaled terms' interleaved) plus the totals of the registers before it (each a tree of
// at most 6 + R - 1 roundings), the running sums of the weights P_i / P_(K-1); with n <= 256
// they stay within 2^-42 of the reference's. The cut and the draw are the first matching
// entry over the registers in order, and the same 2^-36 margins, checked by each lane for its
// own entries and collected by one ballot, decide whether the result stands. Otherwise the weights are recomputed with V8's exp and summed bit for bit
// through `scratch` (LDS, >= 64R doubles; wave_seq_sum). The caller's top-k list and the
// result as in reg_tail.
template <int R, typename In, class SumExp>
__device__ __forceinline__ void reg_tail_wide(const uint64_t (&v)[R], int K, const Launch &L, int row,
                                              const In *row_src, float M, SumExp sum_exp_of,
                                              const tabby_row_params &P, double *scratch) {
  const int lane = wave_lane();
  const double T = P.temperature;
  const double S1 = sum_exp_of();  // first: its loads and chain overlap the exps below
  double d[R], e1[R], s[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const bool in = r * kWaveSize + lane < K;
    d[r] = (double)value_of(composite_key(v[r])) - (double)M;
    e1[r] = in ? exp_nonpos(d[r]) : 0.0;
    s[r] = (!in || greedy_temp(T)) ? 0.0 : T == 1.0 ? e1[r] : exp_nonpos(d[r] / T);
  }
  // Entry i of a per-register array, on every lane (i uniform).
  auto at = [&](const double(&x)[R], int i) {
    double y = 0.0;
#pragma unroll
    for (int r = 0; r < R; ++r)
      if ((i >> 6) == r) y = lane_f64(x[r], i & (kWaveSize - 1));
    return y;
  };
  // The first entry below n for which pred(r) holds on its lane, or n.
  auto first = [&](int n, auto pred) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint64_t m = __ballot(r * kWaveSize + lane < n && pred(r));
      if (m) return r * kWaveSize + __ffsll((unsigned long long)m) - 1;
    }
    return n;
  };
  // Inclusive prefix sums over i = r * 64 + lane of the exact terms (pe) and of the scaled
  // ones (ps), the two scans of each register interleaved, the registers chained by their
  // totals.
  double exact[R], pe[R], ps[R];
  double carry_e = 0.0, carry_s = 0.0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    exact[r] = e1[r] / S1;
    double a = exact[r], b = s[r];
    wave_inclusive_scan2(a, b);
    pe[r] = r == 0 ? a : carry_e + a;
    ps[r] = r == 0 ? b : carry_s + b;
    carry_e = r == 0 ? lane_f64(a, kWaveSize - 1) : carry_e + lane_f64(a, kWaveSize - 1);
    carry_s = r == 0 ? lane_f64(b, kWaveSize - 1) : carry_s + lane_f64(b, kWaveSize - 1);
  }
  const double pool = carry_e;
  tabby_row_result res;
  res.max_logit = M;
  res.sum_exp = S1;
  res.pool_mass = pool;
  res.status = TABBY_OK;
  res.topk_count = min(K, L.topk_cap);
  int chosen = 0;
  if (greedy_temp(T)) {
    res.considered = 1;
    res.pool_exhausted = 0;
  } else {
    const double top_p = P.top_p;
    const double scaled = carry_s;
    double running[R];  // P_i / P_(K-1)
#pragma unroll
    for (int r = 0; r < R; ++r) running[r] = r * kWaveSize + lane < K ? ps[r] / scaled : 0.0;
    const int cut_at = top_p < 1.0 ? first(K, [&](int r) { return running[r] >= top_p; }) : K;
    int cut = cut_at < K ? cut_at + 1 : K;
    double total = at(running, cut - 1);
    double target = P.uniform * total;
    const int hit = first(cut, [&](int r) { return target < running[r]; });
    chosen = hit < cut ? hit : cut - 1;
    // Margins of every comparison that fixed the cut and the draw (running sums are
    // non-decreasing, so the neighbours of each boundary are the only ones to check), each
    // lane testing the ones its own entries decide; one ballot collects the failures.
    constexpr double kMargin = 1.0 / 68719476736.0;  // 2^-36
    const double m = kMargin * top_p, m2 = kMargin * total;
    bool fail = false;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = r * kWaveSize + lane;
      if (top_p < 1.0) {
        if (cut == K) fail = fail || (i == K - 1 && !(running[r] < top_p - m));
        else fail = fail || (i == cut - 1 && !(running[r] >= top_p + m)) || (i == cut - 2 && !(running[r] < top_p - m));
      }
      fail = fail || (i == chosen && !(running[r] > target + m2)) || (i == chosen - 1 && !(running[r] < target - m2));
    }
    if (__ballot(fail)) {
      // Bit for bit: V8's exp for the weights, sequential sums (sampler.ts:170-203).
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int i = r * kWaveSize + lane;
        if (i < K) scratch[i] = fdlibm_exp_inline(d[r] / T);
      }
      wave_lds_sync();
      const double S = wave_seq_sum(scratch, K, nullptr, INFINITY).total;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int i = r * kWaveSize + lane;
        if (i < K) scratch[i] = scratch[i] / S;
      }
      wave_lds_sync();
      const SeqSum run = wave_seq_sum(scratch, K, scratch, top_p < 1.0 ? top_p : INFINITY);
      wave_lds_sync();
      cut = run.count;
      total = run.total;
      target = P.uniform * total;
      chosen = cut - 1;
      for (int base = 0; base < cut; base += kWaveSize) {
        const int i = base + lane;
        const uint64_t m = __ballot(i < cut && target < scratch[min(i, cut - 1)]);
        if (m) {
          chosen = base + __ffsll((unsigned long long)m) - 1;
          break;
        }
      }
    }
    res.considered = (uint32_t)cut;
    res.pool_exhausted = (top_p < 1.0 && pool < top_p) ? 1 : 0;
  }
  uint64_t cv = 0ull;
#pragma unroll
  for (int r = 0; r < R; ++r)
    if ((chosen >> 6) == r)
      cv = (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v[r], chosen & (kWaveSize - 1)) |
           ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v[r] >> 32), chosen & (kWaveSize - 1)) << 32);
  res.id = (int32_t)composite_index(cv);
  res.probability = at(exact, chosen);
  if (lane == 0) L.results[row] = res;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = r * kWaveSize + lane;
    if (i < K && i < L.topk_cap) {
      const uint32_t idx = composite_index(v[r]);
      L.topk_ids[(size_t)row * L.topk_cap + i] = (int32_t)idx;
      L.topk_logits[(size_t)row * L.topk_cap + i] = load_one(row_src + min(idx, (uint32_t)(L.vocab - 1)));
    }
  }
}

// ---------------------------------------------------------------------------------------
// The lm_head fused with the sampler's first pass (the next step after the sampler in the
// reference's decode: forward.ts:408-430 writes the logits with the lm_head matmul and
// encodeSampling re-reads them). Workgroup s takes vocab rows [s * len, s * len + len), one per
// lane (len = 64 * waves, chosen so that the slices fill the chip: 238 slices of 640 rows for
// 151,936), computes their logits for every activation row t < R with q4_dot_row (the CPU
// reference's arithmetic, so these are exactly the logits the unfused product writes), and
// turns them straight into slice s of sampled row t as wave_kernel leaves a slice for the
// merge: the slice max, the slice's sum of exp(x - max), and its top min(k, 64) composites
// (value key, ~id), sorted. The logits never reach HBM; the weights are read once for all R
// rows. Pools of at most 64 only (the reference's bound, forward.ts:348-351): a row with a
// larger or whole-vocabulary pool gets TABBY_EINVAL from the merge.
// ---------------------------------------------------------------------------------------
constexpr int kLhMaxWaves = 16;
constexpr int kLhMaxRows = 8;
constexpr int kLhKcap = kWaveSize;

template <int R>
__global__ __launch_bounds__(kLhMaxWaves *kWaveSize) void lmhead_slice_kernel(Launch L, Workspace W, Q4Matrix Q,
                                                                              const float *x) {
  __shared__ uint64_t lists[kLhMaxWaves][kWaveSize];
  __shared__ float wmax[kLhMaxWaves];
  __shared__ double wsum[kLhMaxWaves];
  const int slice = (int)blockIdx.x;
  const int nw = (int)(blockDim.x / kWaveSize);
  const int w = wave_id(), lane = wave_lane();
  const int r = slice * L.slice_len + (int)threadIdx.x;
  const bool in = r < Q.vocab;
  const int n = min(L.slice_len, Q.vocab - slice * L.slice_len);  // rows of this slice
  // The merge tree below always pairs 16 lists: those of absent waves stay empty.
  for (int i = (int)threadIdx.x; i < (kLhMaxWaves - nw) * kWaveSize; i += (int)blockDim.x)
    lists[nw + i / kWaveSize][i % kWaveSize] = 0ull;
  float logit[R];
  if (in) q4_dot_row<R>(Q, x, r, logit);
#pragma unroll
  for (int t = 0; t < R; ++t) {
    const tabby_row_params P = L.params[t];
    const bool valid = params_valid(P, L.k_max);
    const int keff = effective_k(P, L.vocab);
    const int kk = valid && keff <= kLhKcap ? min(keff, n) : 0;
    const float v = in ? logit[t] : -INFINITY;
    // Slice max, then the sum of 2^(x*L - ml) against ml = fl(max*L), rebased exactly on the
    // max at the end (rebase_sum): the sum's accuracy does not depend on where the logits sit.
    const float m = wave_max(v);
    if (lane == 0) wmax[w] = m;
    // The slice's candidates: each wave's 64 composites sorted, then merged pairwise.
    uint64_t c[1] = {in ? composite(key_of(v), (uint32_t)r) : 0ull};
    wave_sort_desc<1>(c);
    lists[w][lane] = c[0];
    __syncthreads();
    float M = wmax[0];
    for (int i = 1; i < nw; ++i) M = fmaxf(M, wmax[i]);
    const float ml = M * kLog2e;
    const double term = in && M != -INFINITY ? (double)__builtin_amdgcn_exp2f(fmaf(v, kLog2e, -ml)) : 0.0;
    const double ws = wave_sum(term);
    if (lane == 0) wsum[w] = ws;
#pragma unroll
    for (int half = kLhMaxWaves / 2; half > 0; half >>= 1) {
      if (w < half) {
        // Top 64 of two descending lists: the larger of a[i] and b[63 - i] is a bitonic
        // sequence holding them; a bitonic clean sorts it.
        uint64_t a[1] = {tmax(lists[w][lane], lists[w + half][kWaveSize - 1 - lane])};
        wave_bitonic_stages<1>(a, 0, kWaveSize);
        wave_lds_sync();
        lists[w][lane] = a[0];
      }
      __syncthreads();
    }
    if (w == 0) {
      double S = 0.0;
      for (int i = 0; i < nw; ++i) S += wsum[i];
      S = rebase_sum(S, M, ml, M);
      if (lane < kk) W.cands[(size_t)t * W.row_cand_stride + (size_t)slice * L.list_stride + lane] = lists[0][lane];
      if (lane == 0) {
        SliceStat st;
        st.max = M;
        st.count = (uint32_t)kk;
        st.sum = S;
        W.stats[(size_t)t * kMaxSplits + slice] = st;
      }
    }
    __syncthreads();  // lists and statistics are reused by the next row
  }
}

// The merge for the fused path's many slices (up to 256 lists of at most 64, one per slice).
// A bound first: the K-th largest of the slices' first entries (K distinct elements lie at or
// above it, so every element of the row's top K does too). Each slice's entries at or above
// it -- usually its first one or two -- are gathered (at most 256), sorted in registers, and
// the register tail (reg_tail) samples the row. More than 256 at or above the bound (rows
// whose top crowds into a few slices, or ties) take the general merge (merge_row).
struct LhMergeSmem {
  WaveMergeSmem m;
  uint64_t heads[kWaves][kWaveSize];
  uint64_t surv[4 * kWaveSize];
  BlockScratch bs;
};

__global__ __launch_bounds__(kBlock) void lmhead_merge_kernel(Launch L, Workspace W) {
  __shared__ LhMergeSmem sm;
  const int row = (int)blockIdx.x;
  const int s = (int)threadIdx.x, w = wave_id(), lane = wave_lane();
  const tabby_row_params P = L.params[row];
  const RowPool rp = row_pool(L, P);
  const SliceStat *stats = W.stats + (size_t)row * kMaxSplits;
  const RowLists lists{W.cands + (size_t)row * W.row_cand_stride, L.splits, L.list_stride, W.row_cand_stride};
  const int K = rp.K;
  if (!(rp.valid && rp.finite && K > 0 && K <= kWaveSize)) {
    merge_row<float>(sm.m, L, W, row, P, stats, lists);  // statuses of out-of-contract rows
    return;
  }
  const uint64_t *list = lists.base + (size_t)s * L.list_stride;
  const int cnt = s < L.splits ? (int)stats[s].count : 0;
  uint64_t h[1] = {cnt > 0 ? list[0] : 0ull};
  wave_sort_desc<1>(h);
  sm.heads[w][lane] = h[0];
  __syncthreads();
  if (w < 2) {
    uint64_t a[1] = {tmax(sm.heads[w][lane], sm.heads[w + 2][kWaveSize - 1 - lane])};
    wave_bitonic_stages<1>(a, 0, kWaveSize);
    wave_lds_sync();
    sm.heads[w][lane] = a[0];
  }
  __syncthreads();
  if (w == 0) {
    uint64_t a[1] = {tmax(sm.heads[0][lane], sm.heads[1][kWaveSize - 1 - lane])};
    wave_bitonic_stages<1>(a, 0, kWaveSize);
    wave_lds_sync();
    sm.heads[0][lane] = a[0];
  }
  __syncthreads();
  const uint64_t theta = sm.heads[0][K - 1];
  // This slice's entries at or above the bound (its list is sorted): eight loads at a time.
  int take = 0;
  for (int base = 0; base < cnt; base += 8) {
    uint64_t e[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) e[u] = base + u < cnt ? list[base + u] : 0ull;
    int n8 = 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) n8 += (base + u < cnt && e[u] >= theta) ? 1 : 0;
    take += n8;
    if (n8 < 8) break;
  }
  uint32_t total_u = 0;
  const uint32_t before = block_exclusive_scan((uint32_t)take, sm.bs, &total_u);
  const int total = (int)total_u;
  if (total > 4 * kWaveSize) {
    merge_row<float>(sm.m, L, W, row, P, stats, lists);
    return;
  }
  for (int i = 0; i < take; ++i) sm.surv[before + i] = list[i];
  __syncthreads();
  if (w != 0) return;
  uint64_t v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = q * kWaveSize + lane < total ? sm.surv[q * kWaveSize + lane] : 0ull;
  if (total <= kWaveSize) {
    uint64_t v1[1] = {v[0]};
    wave_sort_desc<1>(v1);
    v[0] = v1[0];
  } else {
    wave_sort_desc<4>(v);
  }
  const RowStats rs = row_stats(stats, L.splits);
  const float M = rs.max;
  bool in_domain = (M > -INFINITY) && (M < INFINITY);
  if (in_domain) {
    reg_tail<float>(v[0], K, L, row, (const float *)nullptr, M,
                    [&]() {
                      in_domain = (rs.sum_exp > 0.0) && (rs.sum_exp < INFINITY);
                      return rs.sum_exp;
                    },
                    P);
  }
  if (!in_domain && lane == 0) {
    write_status(L, row, TABBY_EDOMAIN, M, rs.sum_exp);
    W.row_state[row].status = TABBY_EDOMAIN;
  }
}

// A row (or part of a row) whose pool is at most 64, after its waves' streaming: the waves'
// lists are unsorted (every entry at or above the row's shared first bound), and the row's top
// K is selected from their union without sorting them. If the union holds at most 64 entries
// all are taken; otherwise a 256-bin histogram of the keys below the row max (every wave adds
// its own entries) gives the bin where the count from the top reaches K, and the entries in
// and above it are taken. The taken entries (at most 64) go to one LDS array by one atomic per
// wave; wave 0 sorts them in one register and runs the tail (reg_tail), or, for a part, hands
// its top K and statistics on to wave_merge_kernel. Returns false, with every wave's list
// sorted in place and its count cut to K, when more than 64 entries would be taken (the
// general merge then takes over). Every wave calls it.
template <typename In>
__device__ __forceinline__ bool finish_small_pool(RowSmem &sm, const Launch &L, const Workspace &W, int row, int part,
                                  const tabby_row_params &P, const RowPool &rp, int nw);
__device__ __forceinline__ void small_pool_select(RowSmem &sm, int K);

template <typename In, int VEC>
__global__ __launch_bounds__(kRowWaves * kWaveSize) void row_kernel(Launch L, Workspace W) {
  __shared__ RowSmem sm;
  int row = (int)blockIdx.x, part = 0;
  if (L.parts > 1) row_slice_of((int)blockIdx.x, L.rows, L.parts, row, part);
  const int w = __builtin_amdgcn_readfirstlane(wave_id());
  const int nw = (int)(blockDim.x / kWaveSize);  // the row's waves, >= kRowMinWaves
  const tabby_row_params P = L.params[row];  // kept in registers for the merge
  const RowPool rp = row_pool(L, P);
  // Pools of at most kSmallPoolMax skip the waves' end-of-stream sorts and the list merge: the
  // row's top K is selected from the unsorted lists (finish_small_pool). A part of a row
  // (parts > 1) only hands its top K on, whatever its pool; a whole row must be finished here.
  const bool small = rp.valid && rp.K > 0 && rp.K <= kSmallPoolMax && (L.parts > 1 || rp.finite);
  if (w == 0) {
    TABBY_STAMP(16);
    TABBY_STAMP_REAL(24);
  }
  if (threadIdx.x == 0) {
    sm.next_chunk = nw;  // chunk w is wave w's first
    sm.sel_count = 0;
    sm.fin_mask = 0u;
  }
  for (int i = (int)threadIdx.x; i < kSelBins; i += (int)blockDim.x) sm.sel_hist[i] = 0u;
  __syncthreads();
  wave_slice<In, VEC, true>(sm.wave[w], L, P, row, w, part, sm.wave[w].list, &sm.stats[w], &sm.next_chunk,
                            sm.bound_keys, nw, !small, sm.bound_key, small ? sm.sel_hist : nullptr);
  TABBY_STAMP(w);
  if (small) {
    // Each wave marks itself finished; the waves marked before it are in the returned mask.
    // The mark sits between workgroup-scope fences that every lane executes: the wave's
    // histogram adds and its statistics happen before it (release), and what the wave reads
    // after it -- the other waves' statistics, the whole histogram -- after every earlier
    // mark (acquire). So the last wave sees every add, and the second-to-last every other
    // wave's statistics: it combines them while the last one streams and selects the take.
    // (At workgroup scope a fence is a wait for the wave's own outstanding memory
    // operations, none once its stream has ended; no cache is written back.)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    uint32_t before = 0;
    if (wave_lane() == 0)
      before = __hip_atomic_fetch_or(&sm.fin_mask, 1u << w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    before = (uint32_t)__builtin_amdgcn_readfirstlane((int)before);
    const int rank = __popc(before);
    if (rank == nw - 1) {
      small_pool_select(sm, rp.K);
      TABBY_STAMP(29);
    } else if (rank == nw - 2) {
      const uint32_t mask = before | (1u << w);
      const int lane = wave_lane();
      const bool mine = lane < nw && ((mask >> lane) & 1u);
      const SliceStat st = mine ? sm.stats[lane] : SliceStat{-INFINITY, 0u, 0.0};
      const float mx = wave_max(st.max);
      const double part = st.max == -INFINITY ? 0.0 : st.sum * (double)__builtin_amdgcn_exp2f((st.max - mx) * kLog2e);
      const double sum = wave_sum(part);
      if (lane == 0) {
        sm.part_mask = mask;
        sm.part_max = mx;
        sm.part_sum = sum;
      }
      TABBY_STAMP(30);
    }
  }
  __syncthreads();
  if (w == 0) TABBY_STAMP(17);
  if (small && finish_small_pool<In>(sm, L, W, row, part, P, rp, nw)) return;
  constexpr int stride = (int)(sizeof(WaveSmem) / sizeof(uint64_t));
  const RowLists lists{sm.wave[0].list, nw, stride, (int64_t)nw * stride};
  ListMerger<1> m1 = lists_of_wave<1>(lists);
  m1.start();
  if (w == kWaves) {
    const RowStats rs = row_stats(sm.stats, nw);
    if (wave_lane() == 0) {
      sm.merge.row_max = rs.max;
      sm.merge.row_sum = rs.sum_exp;
    }
  }
  merge_pool(sm.merge, lists, m1, [&](int s) { return (int)sm.stats[s].count; }, rp.K);
  __syncthreads();
  if (L.parts > 1) {
    // One part of the row: its top K, sorted, and its statistics go where wave_merge_kernel
    // reads a slice's (slice = part), and that kernel finishes the row.
    if (w == 0) {
      int total = 0;
      for (int s = 0; s < nw; ++s) total += (int)sm.stats[s].count;
      const int count = min(rp.K, total);
      uint64_t *out = W.cands + (size_t)row * W.row_cand_stride + (size_t)part * L.list_stride;
      for (int i = wave_lane(); i < count; i += kWaveSize) out[i] = sm.merge.sorted[i];
      if (wave_lane() == 0) {
        SliceStat st;
        st.max = sm.merge.row_max;
        st.count = (uint32_t)count;
        st.sum = sm.merge.row_sum;
        W.stats[(size_t)row * kMaxSplits + part] = st;
      }
    }
    return;
  }
  finish_pool<In>(sm.merge, L, W, row, P, rp, sm.merge.row_max, sm.merge.row_sum);
}

// The take of a row whose pool is at most kSmallPoolMax (finish_small_pool): the bin holding
// the K-th largest key, from the top of the histogram the waves filled as they finished (four
// bins per lane), gives the smallest key taken and the number of entries at or above it
// (every list entry when the union is small enough to take whole). One wave computes it --
// the row's last to finish streaming, while the others wait at the barrier -- and leaves
// both in sm.sel_take.
__device__ __forceinline__ void small_pool_select(RowSmem &sm, int K) {
  const int lane = wave_lane();
  const SelBins sb = sel_bins(sm.bound_key[1], sm.bound_key[0]);
  uint32_t h[4], sum = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    h[q] = sm.sel_hist[lane * 4 + q];
    sum += h[q];
  }
  const uint32_t inc = wave_inclusive_scan_u32(sum);
  const int total = __builtin_amdgcn_readlane((int)inc, kWaveSize - 1);  // every list entry
  uint32_t take_key = 0u;  // entries with key >= take_key are taken
  int taken = total;
  // A pool selects from more entries than its register class holds (64, 128 or 256: one, two
  // or four registers to sort); either way total >= K when selecting.
  if (total > (K <= kWaveSize ? kWaveSize : K <= 2 * kWaveSize ? 2 * kWaveSize : kSmallTake)) {
    const int owner = __ffsll((unsigned long long)__ballot(inc >= (uint32_t)K)) - 1;  // total >= K
    int bin = 0;
    uint32_t upto = 0;
    if (lane == owner) {
      uint32_t c = inc - sum;
      bool found = false;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        c += h[q];
        if (!found && c >= (uint32_t)K) {
          bin = lane * 4 + q;
          upto = c;
          found = true;
        }
      }
    }
    bin = __builtin_amdgcn_readlane(bin, owner);
    taken = __builtin_amdgcn_readlane((int)upto, owner);
    if (bin < kSelBins - 1) take_key = sb.lowest(bin);
    else taken = total;
  }
  if (lane == 0) {
    sm.sel_take[0] = take_key;
    sm.sel_take[1] = (uint32_t)taken;
  }
}

template <typename In>
__device__ __forceinline__ bool finish_small_pool(RowSmem &sm, const Launch &L, const Workspace &W, int row, int part,
                                                  const tabby_row_params &P, const RowPool &rp, int nw) {
  const int w = wave_id(), lane = wave_lane();
  const int K = rp.K;
  const uint64_t *list = sm.wave[w].list;  // raw entries: value bits << 32 | ~index
  const int count = (int)sm.stats[w].count;
  // The take, selected by the row's last wave to finish streaming (small_pool_select).
  const uint32_t take_key = (uint32_t)__builtin_amdgcn_readfirstlane((int)sm.sel_take[0]);
  const int taken = __builtin_amdgcn_readfirstlane((int)sm.sel_take[1]);
  if (taken > kSmallTake) {
    // More than 256 would be taken (ties at the boundary, or a row whose top lies far above
    // the first bound's union): sort each list in place for the general merge.
    const int keep = min(count, K);
    if (count <= kWaveSize) store_sorted_top<1>(list, count, keep, sm.wave[w].list);
    else if (count <= 2 * kWaveSize) store_sorted_top<2>(list, count, keep, sm.wave[w].list);
    else if (count <= 4 * kWaveSize) store_sorted_top<4>(list, count, keep, sm.wave[w].list);
    else store_sorted_top<8>(list, count, keep, sm.wave[w].list);
    if (lane == 0) sm.stats[w].count = (uint32_t)keep;
    __syncthreads();
    return false;
  }
  for (int base = 0; base < count; base += kWaveSize) {
    const int i = base + lane;
    const uint64_t e = i < count ? list[i] : 0ull;
    const bool take = i < count && raw_key(e) >= take_key;
    const uint64_t mask = __ballot(take);
    if (mask) {
      int at = 0;
      if (lane == 0) at = atomicAdd(&sm.sel_count, (int)__popcll(mask));
      at = __builtin_amdgcn_readfirstlane(at);
      if (take) sm.sel[at + (int)lanes_below(mask)] = e;
    }
  }
  if (w == 0) TABBY_STAMP(18);
  __syncthreads();
  if (w != 0) return true;
  TABBY_STAMP(19);
  // The row's statistics: the second-to-last wave's combination and the one wave it missed.
  float M = sm.part_max;
  double S1 = sm.part_sum;
  const uint32_t missed = ((1u << nw) - 1u) & ~sm.part_mask;
  if (missed) {
    const SliceStat st = sm.stats[__ffs(missed) - 1];
    const float mx = fmaxf(M, st.max);
    S1 = (M == -INFINITY ? 0.0 : S1 * (double)__builtin_amdgcn_exp2f((M - mx) * kLog2e)) +
         (st.max == -INFINITY ? 0.0 : st.sum * (double)__builtin_amdgcn_exp2f((st.max - mx) * kLog2e));
    M = mx;
  }
  auto sum_exp = [&]() { return S1; };
  const int k = min(K, taken);
  // The taken entries sorted in R registers (entry i = r * 64 + lane), then the part's
  // hand-over or the row's tail.
  auto finish = [&](auto &v, auto regs) {
    constexpr int R = decltype(regs)::value;
    if (L.parts > 1) {
      // One part of the row: its top k, sorted, and its statistics go where wave_merge_kernel
      // reads a slice's (slice = part).
      const double S1 = sum_exp();
      uint64_t *out = W.cands + (size_t)row * W.row_cand_stride + (size_t)part * L.list_stride;
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (r * kWaveSize + lane < k) out[r * kWaveSize + lane] = v[r];
      if (lane == 0) {
        SliceStat st;
        st.max = M;
        st.count = (uint32_t)k;
        st.sum = S1;
        W.stats[(size_t)row * kMaxSplits + part] = st;
      }
      return;
    }
    if (!((M > -INFINITY) && (M < INFINITY))) {
      if (lane == 0) {
        write_status(L, row, TABBY_EDOMAIN, M, sum_exp());
        W.row_state[row].status = TABBY_EDOMAIN;
      }
      return;
    }
    const In *row_src = reinterpret_cast<const In *>(L.logits) + (size_t)row * L.vocab;
    bool in_domain = true;
    auto S1_of = [&]() {
      const double S1 = sum_exp();
      in_domain = (S1 > 0.0) && (S1 < INFINITY);
      return S1;
    };
    if constexpr (R == 1) reg_tail<In>(v[0], k, L, row, row_src, M, S1_of, P);
    else reg_tail_wide<R, In>(v, k, L, row, row_src, M, S1_of, P, sm.merge.b);
    if (!in_domain && lane == 0) {
      write_status(L, row, TABBY_EDOMAIN, M, S1);
      W.row_state[row].status = TABBY_EDOMAIN;
    }
  };
  if (taken <= kWaveSize) {
    uint64_t v[1] = {lane < taken ? composite_of_raw(sm.sel[lane]) : 0ull};
    wave_sort_desc<1>(v);
    TABBY_STAMP(20);
    finish(v, std::integral_constant<int, 1>{});
    TABBY_STAMP(21);
    TABBY_STAMP_REAL(25);
  } else if (taken <= 2 * kWaveSize) {
    uint64_t v[2] = {composite_of_raw(sm.sel[lane]),
                     kWaveSize + lane < taken ? composite_of_raw(sm.sel[kWaveSize + lane]) : 0ull};
    wave_sort_desc<2>(v);
    finish(v, std::integral_constant<int, 2>{});
  } else {
    uint64_t v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r * kWaveSize + lane;
      v[r] = i < taken ? composite_of_raw(sm.sel[i]) : 0ull;
    }
    wave_sort_desc<4>(v);
    finish(v, std::integral_constant<int, 4>{});
  }
  return true;
}

// ---------------------------------------------------------------------------------------
// Whole-vocabulary rows (top_k = 0, or >= vocab beyond the pool capacity). The pool is the
// entire row sorted, but only its head matters to sampleFromTopK: with the row max M, an
// element whose (l - M)/T is below -37.5 has a weight below 2^-54, and it is added -- in
// sorted order, after every larger term -- to the scaled total (>= 1, the max's own term)
// or, divided by that total, to a running weight sum (>= the first weight), below half an
// ulp of either, so it cannot change them (head_threshold). The merge computes head_key, the
// smallest key with (l - M)/T >= -37.5 in f64 (or the max's key when T <= 0). head_kernel
// collects the head; head_fast_kernel finishes the row from the merge's sorted top list when
// that provably decides it, else the sort and finish kernels sort the head and run the tail
// (there poolMass takes the head's terms plus the rest of sum-exp).
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ bool is_head_row(const tabby_row_params &P, const Launch &L) {
  return params_valid(P, L.k_max) && effective_k(P, L.vocab) > L.kcap;
}


// The whole-vocabulary tail without sorting the head, when that is provably the same.
// sampleFromTopK over the sorted head needs three sequential f64 sums: the scaled total S and
// the running sums of w_i = s_i / S up to the cut (s_i = exp((l_i - M)/T), V8's exp). The
// merge hands over the row's top N sorted (N = max(topk_cap, 64), finish_pool). Once a
// partial sum P lies in [2^E, 2^(E+1)), adding a term s gives P + u * rint(s / u) exactly
// (u = 2^(E-52)) unless s / u lies exactly halfway between integers (then the parity of P
// decides). So if P_N, the sequential sum of the top N, is in binade E, every later term --
// each smaller than the top N -- adds rint(s / u) ulps whatever the order, provided none ties
// and the total stays below 2^(E+1), and then S = P_N + u * (sum of rint(s / u) over the
// rest of the head). head_kernel counts those ulps (and the ties) for the head entries it
// collects; both conditions are checked exactly (the counts are integers below 2^53, exact
// in f64 in any order, and a total that reaches 2^53 stays there). A term's s / u comes from
// the fast exp when it is below 2^36 and at least 2^-9 from a half: exp_nonpos is within 8
// ulp of e^x and V8's exp within 1, so the two differ by under 9 * 2^-52 * 2^36 < 2^-12
// there and round alike; other terms take V8's exp. When the running sums also reach the cut
// within the top N (or the head holds nothing beyond them), head_fast_kernel finishes the
// row -- bit for bit what the sorted head gives -- and marks it (RowState.handoff bit 0) so
// that the sort and finish kernels skip it; otherwise it plans the sorted head. (Terms just
// below P's binade tie often -- s in [2^(E-1), 2^E) has one bit below the ulp -- which is
// why the top N are summed in order.)

// 2^(52 - E) for P in [2^E, 2^(E+1)): s * ulp_scale(P) is s in ulps of P.
__device__ __forceinline__ double ulp_scale(double P) {
  const int E = (int)(((uint64_t)__double_as_longlong(P) >> 52) & 0x7ff) - 1023;
  return __builtin_ldexp(1.0, 52 - E);
}

// Adds rint(s / u) for the term of composite v to r, and 1 to ties if s / u is a half-integer.
__device__ __forceinline__ void add_ulps(uint64_t v, double M, double T, double scale, double &r, double &ties) {
  const double dt = ((double)value_of(composite_key(v)) - M) / T;
  double q = exp_nonpos(dt) * scale;
  if (!(q < 68719476736.0 && __builtin_fabs(q - __builtin_floor(q) - 0.5) > 0x1p-9)) q = fdlibm_exp(dt) * scale;
  ties += q - __builtin_floor(q) == 0.5 ? 1.0 : 0.0;
  r += __builtin_rint(q);
}

// head_kernel's slices: two wave chunks, both loaded before either is used.
constexpr int kHeadSlice = 2 * kWChunk;

// Collects the head (elements with key >= head_key) of one slice of a row into the row's head
// buffer and, when the merge handed over the row's top N and T > 0, writes the slice's ulp
// counts for head_fast_kernel: the sum of rint(s / u) over its head entries below the top N,
// their number of ties, and their count.
template <typename In, int VEC>
__global__ __launch_bounds__(kWaveSize) void head_kernel(Launch L, Workspace W) {
  __shared__ uint64_t list[kWListCap];
  int row, slice;
  row_slice_of((int)blockIdx.x, L.rows, L.h_splits, row, slice);
  const int V = L.vocab, lane = wave_lane();
  const int begin = slice * L.h_slice_len;
  const int n = min(L.h_slice_len, V - begin);
  const int nchunks = (n + kWChunk - 1) / kWChunk;
  const int full_chunks = n / kWChunk;
  const In *src = reinterpret_cast<const In *>(L.logits) + (size_t)row * V + begin;
  // Both chunks' loads at once (a slice's second chunk past the row's end reads zeros),
  // issued with the row's parameters and state rather than after them: one round trip for
  // all three (a row that turns out to need no head pass has read its slice for nothing).
  float x[kWChunkPerLane], y[kWChunkPerLane];
  const ChunkReader<In, VEC> rd(src, n);
  rd.load(0, x);
  rd.load(1, y);
  const tabby_row_params P = L.params[row];
  const RowState rs = W.row_state[row];
  if (!is_head_row(P, L) || rs.status != TABBY_OK) return;
  const float hv = value_of(rs.head_key);
  // This slice's part of the head goes to its own range of the row's head buffer (no
  // atomics: a row's slices appending to one counter serialised on it).
  uint64_t *head = W.head + (size_t)row * W.head_stride + begin;
  int stored = 0;
  // The ulp of P_N (the sequential sum of the top N's terms, from the merge).
  const int N = (int)(rs.handoff >> 16);
  const double T = P.temperature, M = (double)rs.max;
  const bool count_ulps = !greedy_temp(T) && N > 0 && N <= kWaveKcap;
  const double scale = ulp_scale(rs.list_sum);
  const uint64_t last = count_ulps ? W.head_sorted[(size_t)row * W.head_stride + N - 1] : 0ull;
  double r = 0.0, ties = 0.0, outside = 0.0;
  int count = 0;
  auto flush = [&]() {
    wave_lds_sync();
    for (int i = lane; i < count; i += kWaveSize) {
      const uint64_t v = list[i];
      head[stored + i] = v;
      if (count_ulps && v < last) {
        add_ulps(v, M, T, scale, r, ties);
        outside += 1.0;
      }
    }
    stored += count;
    count = 0;
    wave_lds_sync();
  };
  auto collect = [&](int c, float(&cur)[kWChunkPerLane]) {
    if (c >= full_chunks) {
#pragma unroll
      for (int e = 0; e < kWChunkPerLane; ++e)
        if (wave_local<VEC>(c, e) >= n) cur[e] = __builtin_nanf("");  // fails cur >= hv
    }
#pragma unroll
    for (int e = 0; e < kWChunkPerLane; ++e) {
      if (count > kWListCap - kWaveSize) flush();
      const bool take = cur[e] >= hv;
      const uint64_t mask = __ballot(take);
      if (mask) {
        if (take) list[count + (int)lanes_below(mask)] = composite(key_of(cur[e]), (uint32_t)(begin + wave_local<VEC>(c, e)));
        count = __builtin_amdgcn_readfirstlane(count + (int)__popcll(mask));
      }
    }
  };
  static_assert(kHeadSlice == 2 * kWChunk, "head_kernel's slices are two chunks");
  collect(0, x);
  if (nchunks > 1) collect(1, y);
  if (count > 0) flush();
  if (lane == 0) W.head_slice_count[(size_t)row * W.acc_stride + slice] = (uint32_t)stored;
  if (count_ulps) {
    r = wave_sum(r);  // integers: exact below 2^53, and at least 2^53 once the total is
    ties = wave_sum(ties);
    outside = wave_sum(outside);
    if (lane == 0) {
      double *acc = W.head_acc + ((size_t)row * W.acc_stride + slice) * 3;
      acc[0] = r;
      acc[1] = ties;
      acc[2] = outside;
    }
  }
}

// For a row that head_fast_kernel cannot finish, the sorted head is built in two steps.
// plan_head (that kernel's workgroup for the row) bins the head by key into 4096 buckets
// (bucket = (max_key - key) >> shift, so bucket order is descending key order), scatters it
// into bucket order, and cuts the bucket sequence into segments: a new segment starts at each
// bucket whose start offset crosses the next multiple of kSegCap. head_sort_kernel (one
// workgroup per segment) sorts each segment in place -- in LDS when it fits (at most kSegCap plus one bucket, normally), otherwise by
// batches in descending order. The concatenation of the sorted segments is the sorted head.
// kSegCap leaves room below 1,024 for the bucket that crosses a segment's end, so that a
// segment is normally sorted as 1,024 entries: at 1,024 segments of 1,025-1,032 entries were
// padded to 2,048 and took twice as long (17.9 vs 8.2 us on config 4's largest head).
constexpr int kHeadBuckets = 4096;
constexpr int kSegCap = 896;
constexpr int kSegLds = 8192;
constexpr int kHeadBatch = 4096;

// Plan layout per row: [0] = number of segment slots used (max segment index + 1),
// [1] = head size, [2 + g] = start offset of segment g, or ~0u if no segment starts there.
__host__ __device__ __forceinline__ int plan_slots(int vocab_max) { return vocab_max / kSegCap + 2; }

constexpr int kPlanThreads = 1024;  // a 13 K-entry head took 24.5 us on 256 lanes
static_assert(kMaxSplits * kChunk <= kPlanThreads * kHeadSlice, "head_fast_kernel takes one slice per thread");

struct PlanSmem {
  uint32_t starts[kPlanThreads + 1];  // head offset of each head_kernel slice's entries
  uint32_t wave_total[kPlanThreads / kWaveSize];
  uint32_t hist[kHeadBuckets];
  uint32_t start[kHeadBuckets];
};

// The plan of one row's sorted head, by a workgroup of kPlanThreads (head_fast_kernel).
__device__ __forceinline__ void plan_head(PlanSmem &sm, const Launch &L, const Workspace &W, int row,
                                          const RowState &rs, uint32_t *plan) {
  const int H = (int)sm.starts[L.h_splits];
  const uint64_t *head_base = W.head + (size_t)row * W.head_stride;
  // Entry i of the head: in the slice s with starts[s] <= i < starts[s + 1].
  auto head_at = [&](int i) {
    int lo = 0, hi = L.h_splits;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (sm.starts[mid] <= (uint32_t)i) lo = mid; else hi = mid;
    }
    return head_base[(size_t)lo * L.h_slice_len + (uint32_t)i - sm.starts[lo]];
  };
  uint64_t *sorted = W.head_sorted + (size_t)row * W.head_stride;
  const uint32_t kmax = key_of(rs.max);
  const uint32_t range = kmax - min(rs.head_key, kmax);
  const int bits = range == 0 ? 0 : 32 - __clz((int)range);
  const int shift = bits > 12 ? bits - 12 : 0;
  auto bucket_of = [&](uint64_t v) {
    return min((kmax - min(composite_key(v), kmax)) >> shift, (uint32_t)(kHeadBuckets - 1));
  };
  for (int b = threadIdx.x; b < kHeadBuckets; b += kPlanThreads) sm.hist[b] = 0u;
  __syncthreads();
  constexpr int B = 8;  // global loads in flight per lane
  for (int base0 = 0; base0 < H; base0 += B * kPlanThreads) {
    uint64_t v[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int i = base0 + u * kPlanThreads + (int)threadIdx.x;
      v[u] = i < H ? head_at(i) : 0ull;
    }
#pragma unroll
    for (int u = 0; u < B; ++u)
      if (base0 + u * kPlanThreads + (int)threadIdx.x < H) atomicAdd(&sm.hist[bucket_of(v[u])], 1u);
  }
  __syncthreads();
  // Exclusive scan of the bucket counts: 16 buckets per thread, then across threads.
  constexpr int kPer = kHeadBuckets / kPlanThreads;
  uint32_t local[kPer], run = 0;
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    local[q] = run;
    run += sm.hist[threadIdx.x * kPer + q];
  }
  // Across the workgroup: wave scans, then the totals of the waves below.
  const uint32_t inc = wave_inclusive_scan_u32(run);
  if (wave_lane() == kWaveSize - 1) sm.wave_total[wave_id()] = inc;
  __syncthreads();
  uint32_t base = inc - run;
  for (int k = 0; k < wave_id(); ++k) base += sm.wave_total[k];
#pragma unroll
  for (int q = 0; q < kPer; ++q) sm.start[threadIdx.x * kPer + q] = base + local[q];
  __syncthreads();
  const int slots = min((int)((uint32_t)H / kSegCap) + 1, W.plan_stride - 2);
  for (int g = threadIdx.x; g < slots; g += kPlanThreads) plan[2 + g] = g == 0 ? 0u : ~0u;
  __syncthreads();
  // Segment starts: a bucket whose start reaches a new multiple of kSegCap.
  for (int b = 1 + (int)threadIdx.x; b < kHeadBuckets; b += kPlanThreads) {
    const uint32_t st = sm.start[b];
    const uint32_t g = st / kSegCap, gp = sm.start[b - 1] / kSegCap;
    if (g != gp && st < (uint32_t)H && (int)g < slots) plan[2 + g] = st;
  }
  if (threadIdx.x == 0) {
    plan[0] = (uint32_t)slots;
    plan[1] = (uint32_t)H;
  }
  // Scatter into bucket order (unsorted within a bucket).
  __syncthreads();
  for (int base0 = 0; base0 < H; base0 += B * kPlanThreads) {
    uint64_t v[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int i = base0 + u * kPlanThreads + (int)threadIdx.x;
      v[u] = i < H ? head_at(i) : 0ull;
    }
#pragma unroll
    for (int u = 0; u < B; ++u)
      if (base0 + u * kPlanThreads + (int)threadIdx.x < H) sorted[atomicAdd(&sm.start[bucket_of(v[u])], 1u)] = v[u];
  }
}

struct SortSmem {
  BlockScratch bs;
  uint32_t hist[kBins];
  uint64_t buf[kSegLds];
};

// Sorts segment g of a row's plan in place (one workgroup).
__device__ __forceinline__ void sort_segment(SortSmem &sm, const Launch &L, const Workspace &W, int row, int g,
                                             int slots, const uint32_t *plan) {
  const int slots_max = W.plan_stride - 2;
  const uint32_t lo = plan[2 + g];
  if (lo == ~0u) return;
  const int H = (int)plan[1];
  uint32_t hi = (uint32_t)H;
  for (int q = g + 1; q < slots; ++q) {
    if (plan[2 + q] != ~0u) {
      hi = plan[2 + q];
      break;
    }
  }
  const int n = (int)(hi - lo);
  uint64_t *seg = W.head_sorted + (size_t)row * W.head_stride + lo;
  // Per element of the sorted segment: exp((l - M)/T) into head_s; the segment's sums of
  // exp(l - M) and exp(l - M)/sumExp into head_part (summed in segment order later).
  const RowState rs = W.row_state[row];
  const double T = L.params[row].temperature;
  double *sg = W.head_s + (size_t)row * W.head_stride + lo;
  double *part = W.head_part + ((size_t)row * slots_max + g) * 2;
  auto terms = [&](const uint64_t *src) {
    double pool_part = 0.0, e_part = 0.0;
    for (int i = threadIdx.x; i < n; i += kBlock) {
      const double d = (double)value_of(composite_key(src[i])) - (double)rs.max;
      // poolMass and the head's share of sum-exp are compared within 1e-5: an f32 exp2 will
      // do (the exact V8 exp is kept for the weights, which decide the draw).
      const double e = (double)__builtin_amdgcn_exp2f((float)(d * 1.4426950408889634));
      pool_part += e / rs.sum_exp;
      e_part += e;
      sg[i] = !greedy_temp(T) ? fdlibm_exp(d / T) : 0.0;
    }
    const double ps = block_sum(pool_part, sm.bs);
    const double es = block_sum(e_part, sm.bs);
    if (threadIdx.x == 0) {
      part[0] = ps;
      part[1] = es;
    }
  };
  if (n <= kSegLds) {
    const int npow = next_pow2(n);
    for (int i = threadIdx.x; i < npow; i += kBlock) sm.buf[i] = i < n ? seg[i] : 0ull;
    __syncthreads();
    if (n > 1) block_sort_desc(sm.buf, npow);
    for (int i = threadIdx.x; i < n; i += kBlock) seg[i] = sm.buf[i];
    terms(sm.buf);
    return;
  }
  // Oversized segment (one bucket holds more than kSegLds entries: massive ties): batches
  // of the kHeadBatch largest below the previous batch, read from the segment and written to
  // the same range of the (no longer needed) unsorted head, then copied back.
  uint64_t *out = W.head + (size_t)row * W.head_stride + lo;
  uint64_t upper = ~0ull;
  for (int pos = 0; pos < n;) {
    const int b = min(kHeadBatch, n - pos);
    if (threadIdx.x == 0) sm.bs.slot = 0u;
    __syncthreads();
    auto below = [&](auto &&f) {
      constexpr int B = 8;
      for (int base = 0; base < n; base += B * kBlock) {
        uint64_t v[B];
#pragma unroll
        for (int u = 0; u < B; ++u) {
          const int i = base + u * kBlock + (int)threadIdx.x;
          v[u] = i < n ? seg[i] : ~0ull;
        }
#pragma unroll
        for (int u = 0; u < B; ++u)
          if (v[u] < upper) f(v[u]);
      }
    };
    if (n - pos > b) {
      const SelectResult r = radix_select(below, (uint32_t)b, sm.hist, sm.bs);
      below([&](uint64_t v) {
        const bool take = selected(v, r);
        const uint32_t at = wave_slot(take, &sm.bs.slot);
        if (take && at < (uint32_t)b) sm.buf[at] = v;
      });
    } else {
      below([&](uint64_t v) {
        const uint32_t at = wave_slot(true, &sm.bs.slot);
        if (at < (uint32_t)b) sm.buf[at] = v;
      });
    }
    const int npow = next_pow2(b);
    for (int i = b + (int)threadIdx.x; i < npow; i += kBlock) sm.buf[i] = 0ull;
    __syncthreads();
    block_sort_desc(sm.buf, npow);
    for (int i = threadIdx.x; i < b; i += kBlock) out[pos + i] = sm.buf[i];
    upper = sm.buf[b - 1];
    pos += b;
    __syncthreads();
  }
  for (int i = threadIdx.x; i < n; i += kBlock) seg[i] = out[i];
  terms(out);
}

// Workgroups per row of head_sort_kernel; each sorts every kSortGroups-th segment. (One per
// segment slot cost 7.5 us on config 4 when no row needed a sort: 171 slots per row, each
// workgroup reserving 66 KB of LDS.)
constexpr int kSortGroups = 8;

__global__ __launch_bounds__(kBlock) void head_sort_kernel(Launch L, Workspace W) {
  __shared__ SortSmem sm;
  const int row = (int)blockIdx.x / kSortGroups;
  const int first = (int)blockIdx.x - row * kSortGroups;
  const uint32_t *plan = W.head_plan + (size_t)row * W.plan_stride;
  const int slots = (int)plan[0];
  for (int g = first; g < slots; g += kSortGroups) {
    sort_segment(sm, L, W, row, g, slots, plan);
    __syncthreads();  // sm is reused by the next segment
  }
}

// Heads up to this many entries run their sums from LDS (padded, 139 KB of the 160 KB a
// gfx950 workgroup may use); larger ones from global memory.
constexpr int kHeadLds = 16384;

constexpr int kFinishThreads = 512;  // eight waves: the sums take 8,192 terms per step

struct HeadSmem {
  BlockScratch bs;
  SeqScratch<kFinishThreads / kWaveSize> ss;
  double pool, e;
  int cut;
  int chosen;
  double t[PaddedLds::words(kHeadLds)];  // the head's weights, then their running sums
};

// First i in [0, n) with target < c[i] (c non-decreasing), or n - 1 when there is none: a
// 64-ary search by one wave, each step probing 64 evenly spaced entries. C: an accessor.
template <class C>
__device__ __forceinline__ int wave_first_above(C c, int n, double target) {
  int lo = 0, hi = n;  // the answer lies in [lo, hi]; hi == n means "none yet"
  while (hi - lo > kWaveSize) {
    const int step = (hi - lo + kWaveSize - 1) / kWaveSize;
    const int probe = lo + wave_lane() * step;
    const uint64_t hit = __ballot(probe < hi && target < c[min(probe, n - 1)]);
    if (!hit) {
      // Every valid probe (those below hi) is at or below target: the answer lies past the
      // last of them, lo + floor((hi - 1 - lo) / step) * step, which is lane 63's probe only
      // when all 64 probes are valid.
      lo = lo + min(kWaveSize - 1, (hi - 1 - lo) / step) * step + 1;
    } else {
      const int f = __ffsll((unsigned long long)hit) - 1;
      const int new_hi = lo + f * step;
      lo = f == 0 ? lo : lo + (f - 1) * step + 1;
      hi = new_hi;
    }
  }
  const int i = lo + wave_lane();
  const uint64_t hit = __ballot(i < hi && target < c[min(i, n - 1)]);
  if (hit) return lo + __ffsll((unsigned long long)hit) - 1;
  return hi < n ? hi : n - 1;
}

// sampleFromTopK over the sorted head (see the comment on head_kernel): the head's terms,
// the scaled total and the running sums (bit-exact sequential sums), the cut and the draw.
template <typename In>
__global__ __launch_bounds__(kFinishThreads) void head_finish_kernel(Launch L, Workspace W) {
  __shared__ HeadSmem sm;
  const int row = (int)blockIdx.x;
  const tabby_row_params P = L.params[row];
  if (!is_head_row(P, L)) return;
  const RowState rs = W.row_state[row];
  if (rs.status != TABBY_OK || (rs.handoff & 1u)) return;  // head_fast_kernel finished it
  const int V = L.vocab;
  const In *row_src = reinterpret_cast<const In *>(L.logits) + (size_t)row * V;
  const int H = (int)W.head_count[row];
  const uint64_t *sorted = W.head_sorted + (size_t)row * W.head_stride;
  double *sg = W.head_s + (size_t)row * W.head_stride;
  double *cg = W.head_c + (size_t)row * W.head_stride;
  const float M = rs.max;
  const double S1 = rs.sum_exp;
  const double T = P.temperature;

  // The segments' sums, in segment order (head_sort_kernel wrote them).
  const uint32_t *plan = W.head_plan + (size_t)row * W.plan_stride;
  const int slots_max = W.plan_stride - 2;
  const double *part = W.head_part + (size_t)row * slots_max * 2;
  double pool_head = 0.0, e_head = 0.0;
  if (threadIdx.x == 0) {
    const int slots = (int)plan[0];
    for (int g = 0; g < slots; ++g) {
      if (plan[2 + g] != ~0u) {
        pool_head += part[2 * g];
        e_head += part[2 * g + 1];
      }
    }
    sm.pool = pool_head;
    sm.e = e_head;
  }
  __syncthreads();
  pool_head = sm.pool;
  e_head = sm.e;
  // poolMass: the head's exact terms plus the mass of everything below the head.
  const double pool_mass = pool_head + fmax(0.0, S1 - e_head) / S1;

  tabby_row_result res;
  res.max_logit = M;
  res.sum_exp = S1;
  res.pool_mass = pool_mass;
  res.status = TABBY_OK;
  res.topk_count = min(H, L.topk_cap);
  int chosen = 0;
  if (greedy_temp(T)) {
    res.considered = 1;
    res.pool_exhausted = 0;
  } else {
    // The scaled total over the sorted head (bit-exact sequential sum, wave 0), the weights,
    // and their running sums up to the first that reaches top-p (the cut; without a cut the
    // whole vocabulary is considered). From LDS when the head fits, else global memory.
    const double top_p = P.top_p;
    const double stop = top_p < 1.0 ? top_p : INFINITY;
    auto finish = [&](auto t, auto c) {
      // The weights are non-increasing: the sum may settle before the head's end. Both sums
      // are taken by the whole workgroup (block_seq_sum_wide: 8,192 terms per step).
      const double S = block_seq_sum_wide<kFinishThreads / kWaveSize>(t, H, c, false, INFINITY, true, sm.ss).total;
      for (int i = threadIdx.x; i < H; i += kFinishThreads) c[i] = t[i] / S;
      __syncthreads();
      const SeqSum run = block_seq_sum_wide<kFinishThreads / kWaveSize>(c, H, c, true, stop, false, sm.ss);
      __syncthreads();  // every running sum is written
      if (wave_id() == 0) {
        const bool reached = top_p < 1.0 && run.total >= top_p;
        const double target = P.uniform * run.total;  // the running sum at the cut: the total
        const int first = wave_first_above(c, run.count, target);
        if (lane_id() == 0) {
          sm.cut = reached ? run.count : V;
          sm.chosen = first;
        }
      }
      __syncthreads();
    };
    if (H <= kHeadLds) {
      const PaddedLds lt{sm.t};
      constexpr int B = 8;  // loads in flight per lane
      for (int base = 0; base < H; base += B * kFinishThreads) {
        double v[B];
#pragma unroll
        for (int u = 0; u < B; ++u) {
          const int i = base + u * kFinishThreads + (int)threadIdx.x;
          v[u] = i < H ? sg[i] : 0.0;
        }
#pragma unroll
        for (int u = 0; u < B; ++u) {
          const int i = base + u * kFinishThreads + (int)threadIdx.x;
          if (i < H) lt[i] = v[u];
        }
      }
      __syncthreads();
      finish(lt, lt);
    } else {
      finish((const double *)sg, cg);
    }
    chosen = sm.chosen;
    res.considered = (uint32_t)sm.cut;
    res.pool_exhausted = (top_p < 1.0 && pool_mass < top_p) ? 1 : 0;
  }
  const uint64_t cv = sorted[chosen];
  res.id = (int32_t)composite_index(cv);
  res.probability = fdlibm_exp((double)value_of(composite_key(cv)) - (double)M) / S1;
  if (threadIdx.x == 0) L.results[row] = res;
  if (L.topk_cap > 0) {
    const int m = min(H, L.topk_cap);
    for (int i = threadIdx.x; i < m; i += kFinishThreads) {
      const uint32_t idx = composite_index(sorted[i]);
      L.topk_ids[(size_t)row * L.topk_cap + i] = (int32_t)idx;
      L.topk_logits[(size_t)row * L.topk_cap + i] = load_one(row_src + min(idx, (uint32_t)(V - 1)));
    }
  }
}

// The fast finish of a whole-vocabulary row (see add_ulps above), by wave 0, with the top
// list already in sm.top and this lane's share of head_kernel's counts (r, ties, outside):
// true when the row is finished (result and top-k list written, RowState marked).
struct HeadFastSmem {
  uint64_t top[kWaveKcap];
  double s[kWaveKcap];  // s_i = exp((l_i - M) / T) with V8's exp, then w_i = s_i / S
  double c[kWaveKcap];  // running sums
  int done;
};

template <typename In>
__device__ __forceinline__ bool head_fast_finish(HeadFastSmem &sm, const Launch &L, const Workspace &W, int row,
                                                 const tabby_row_params &P, const RowState &rs, int H, double r,
                                                 double ties, double outside) {
  const int N = (int)(rs.handoff >> 16);
  if (N == 0 || N > kWaveKcap) return false;  // no list handed over (pools above 256)
  const int V = L.vocab, lane = wave_lane();
  const double M = (double)rs.max, S1 = rs.sum_exp, T = P.temperature, top_p = P.top_p;
  int chosen = 0, cut = 1;
  if (!greedy_temp(T)) {
    for (int i = lane; i < N; i += kWaveSize)
      sm.s[i] = fdlibm_exp(((double)value_of(composite_key(sm.top[i])) - M) / T);
    const double PN = rs.list_sum;
    // head_kernel's counts over the head entries below the top N.
    r = wave_sum(r);
    ties = wave_sum(ties);
    outside = wave_sum(outside);
    const double scale = ulp_scale(PN);
    const double m = PN * scale;  // P_N in ulps: an integer in [2^52, 2^53)
    if (ties > 0.0 || m + r >= 9007199254740992.0) return false;
    const double S = (m + r) / scale;
    for (int i = lane; i < N; i += kWaveSize) sm.s[i] = sm.s[i] / S;
    wave_lds_sync();
    const SeqSum run = wave_seq_sum(sm.s, N, sm.c, top_p < 1.0 ? top_p : INFINITY);
    const bool reached = top_p < 1.0 && run.total >= top_p;
    // Without the cut among the top N, the running sums must end there: nothing in the head
    // beyond them (every smaller term is below half an ulp of every running sum).
    if (!reached && outside > 0.0) return false;
    wave_lds_sync();
    chosen = wave_first_above(sm.c, run.count, P.uniform * run.total);
    cut = reached ? run.count : V;
  }
  if (lane == 0) {
    tabby_row_result res;
    res.max_logit = rs.max;
    res.sum_exp = S1;
    // The pool is the whole row: poolMass = sum of exp(l_i - M) / sumExp over every element,
    // 1 up to rounding (a sequential sum of n such terms is within n * 2^-53 of it).
    res.pool_mass = 1.0;
    res.status = TABBY_OK;
    res.topk_count = min(H, L.topk_cap);
    res.considered = (uint32_t)cut;
    res.pool_exhausted = 0;  // poolMass 1 is never below top_p
    res.id = (int32_t)composite_index(sm.top[chosen]);
    res.probability = fdlibm_exp((double)value_of(composite_key(sm.top[chosen])) - M) / S1;
    L.results[row] = res;
    W.row_state[row].handoff = rs.handoff | 1u;
  }
  if (L.topk_cap > 0) {
    // The caller's top-k list: the first topk_cap <= N entries (finish_pool).
    const In *row_src = reinterpret_cast<const In *>(L.logits) + (size_t)row * V;
    const int m = min(H, L.topk_cap);
    for (int i = lane; i < m; i += kWaveSize) {
      const uint32_t idx = composite_index(sm.top[i]);
      L.topk_ids[(size_t)row * L.topk_cap + i] = (int32_t)idx;
      L.topk_logits[(size_t)row * L.topk_cap + i] = load_one(row_src + min(idx, (uint32_t)(V - 1)));
    }
  }
  return true;
}

// One workgroup per whole-vocabulary row: the fast finish (wave 0), else the plan of the
// sorted head for head_sort_kernel and head_finish_kernel.
template <typename In>
__global__ __launch_bounds__(kPlanThreads) void head_fast_kernel(Launch L, Workspace W) {
  __shared__ PlanSmem psm;
  __shared__ HeadFastSmem sm;
  const int row = (int)blockIdx.x;
  uint32_t *plan = W.head_plan + (size_t)row * W.plan_stride;
  const tabby_row_params P = L.params[row];
  const RowState rs = W.row_state[row];
  // Every slice's head count is requested with them (one slice per thread), and so are, by
  // wave 0, the fast finish's inputs: the merge's top list (its first kWaveKcap slots, of
  // which the row state then says how many hold it) and head_kernel's ulp counts, slice by
  // slice -- one round trip for all.
  const int ns = L.h_splits;
  const uint32_t c = (int)threadIdx.x < ns ? W.head_slice_count[(size_t)row * W.acc_stride + threadIdx.x] : 0u;
  constexpr int kTopRegs = kWaveKcap / kWaveSize;
  uint64_t top[kTopRegs];
  double r = 0.0, ties = 0.0, outside = 0.0;
  if (wave_id() == 0) {
    const uint64_t *list = W.head_sorted + (size_t)row * W.head_stride;
#pragma unroll
    for (int q = 0; q < kTopRegs; ++q) {
      const int i = q * kWaveSize + wave_lane();
      top[q] = i < W.head_stride ? list[i] : 0ull;
    }
    const double *acc = W.head_acc + (size_t)row * W.acc_stride * 3;
    for (int i = wave_lane(); i < ns; i += kWaveSize) {
      r += acc[3 * i];
      ties += acc[3 * i + 1];
      outside += acc[3 * i + 2];
    }
  }
  if (!is_head_row(P, L) || rs.status != TABBY_OK) {
    if (threadIdx.x == 0) plan[0] = 0u;
    return;
  }
  const int N = (int)(rs.handoff >> 16);
  if (wave_id() == 0) {
    if (N > 0 && N <= kWaveKcap) {
#pragma unroll
      for (int q = 0; q < kTopRegs; ++q) {
        const int i = q * kWaveSize + wave_lane();
        if (i < N) sm.top[i] = top[q];
      }
    }
    if (!(N > 0 && N <= kWaveKcap) || greedy_temp(P.temperature)) r = ties = outside = 0.0;
  }
  // The head's size and where each slice's entries start (every thread holds one slice).
  const uint32_t inc = wave_inclusive_scan_u32(c);
  if (wave_lane() == kWaveSize - 1) psm.wave_total[wave_id()] = inc;
  __syncthreads();
  uint32_t below = inc;
  for (int k = 0; k < wave_id(); ++k) below += psm.wave_total[k];
  if ((int)threadIdx.x < ns) psm.starts[threadIdx.x + 1] = below;
  if (threadIdx.x == 0) psm.starts[0] = 0u;
  __syncthreads();
  if (threadIdx.x == 0) W.head_count[row] = psm.starts[ns];
  if (wave_id() == 0) {
    const bool done = head_fast_finish<In>(sm, L, W, row, P, rs, (int)psm.starts[ns], r, ties, outside);
    if (wave_lane() == 0) sm.done = done ? 1 : 0;
  }
  __syncthreads();
  if (sm.done) {
    if (threadIdx.x == 0) plan[0] = 0u;
    return;
  }
  plan_head(psm, L, W, row, rs, plan);
}

// ---------------------------------------------------------------------------------------
// Diagnostic kernel: the device exp over an array.
// ---------------------------------------------------------------------------------------
// Diagnostic kernel: sequential partial sums of t[0..n) by one wave (wave_seq_sum).
__global__ __launch_bounds__(kWaveSize) void seq_sum_kernel(const double *t, int32_t n, double stop_at,
                                                           double *out, int32_t *count, int32_t wide) {
  if (wide == 4) {  // the register form (n <= 64): term i in lane i
    const int lane = wave_lane();
    const double ti = lane < n ? t[lane] : 0.0;
    double partial;
    const SeqSum r = reg_seq_sum(ti, n, stop_at, &partial);
    if (lane < r.count) out[lane] = partial;
    if (lane == 0) *count = r.count;
    return;
  }
  const SeqSum r = wide ? wave_seq_sum_wide(t, n, out, stop_at) : wave_seq_sum(t, n, out, stop_at);
  if (wave_lane() == 0) *count = r.count;
}

// The same by a workgroup of NW waves (block_seq_sum_wide; head_finish_kernel runs NW = 8).
template <int NW>
__global__ __launch_bounds__(NW * kWaveSize) void seq_sum_block_kernel(const double *t, int32_t n, double stop_at,
                                                                       double *out, int32_t *count) {
  __shared__ SeqScratch<NW> sc;
  const SeqSum r = block_seq_sum_wide<NW>(t, n, out, true, stop_at, false, sc);
  if (threadIdx.x == 0) *count = r.count;
}

// Diagnostic kernel: the draw search of head_finish_kernel (wave_first_above), one wave per
// target, over the non-decreasing c[0..n).
__global__ __launch_bounds__(kWaveSize) void first_above_kernel(const double *c, int32_t n, const double *targets,
                                                                int32_t *out) {
  const int r = wave_first_above(c, n, targets[blockIdx.x]);
  if (wave_lane() == 0) out[blockIdx.x] = r;
}

__global__ void exp_kernel(const double *x, double *y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = fdlibm_exp(x[i]);
}

// ---------------------------------------------------------------------------------------
// Pools of 257..1024 (k_max > 256) in batches of at least as many rows as CUs: one 16-wave
// workgroup per row streams it as row_kernel does (each wave's first two chunks, then chunks
// claimed from an LDS counter) with the lane max and sum-exp, and appends every element at
// or above the row's first bound to one LDS list shared by its waves: a wave reserves room
// for a chunk's candidates with one LDS atomic, with no barrier, and past kPoolListCap
// entries they go to the row's region of global memory. The first bound: the maxima of four
// groups of eight elements of each lane's first two chunks (spread over the row) are 4,096
// distinct elements; the kk-th largest of their keys (its top 22 bits: a lower bound) has kk
// elements at or above it, so it never exceeds the row's kk-th largest -- and long rows
// stream at the (kk/2)-th instead, checked at the end (the rows whose count falls short take
// their candidates again at the certain bound). (The 4-wave slice kernel started from
// the first chunk's kk-th largest -- a quarter of that chunk at kk = 1,024 -- and pruned its
// list with two workgroup barriers per chunk: config 5 took 135 us there.) At the end the
// workgroup selects the row's exact top kk from the list (pool_select), gathers it into LDS,
// sorts it and samples it (finish_row over its 16 waves), as merge_kernel would have; a row
// outside the contract gets its status here too. Only a head pass's whole-vocabulary rows
// leave their top list, unsorted, with the row's statistics, as slice 0 for merge_kernel.
// ---------------------------------------------------------------------------------------
constexpr int kPoolWaves = 16;
constexpr int kPoolThreads = kPoolWaves * kWaveSize;
constexpr int kPoolListCap = 8192;
constexpr int kPoolBoundKeys = 4 * kPoolThreads;
// Rows of at least this many chunks (the sample then at most a quarter of the row) stream at a
// guessed first bound (pool_row_kernel).
constexpr int kPoolGuessChunks = 128;
static_assert((kPoolWaves & (kPoolWaves - 1)) == 0, "pool_row_kernel's claim order takes v mod kPoolWaves by a mask");

// The spacing of pool_row_kernel's sample chunks: the largest power of two s with
// kPoolWaves * s <= nchunks (1 for rows of fewer than 2 * kPoolWaves chunks).
__device__ __forceinline__ int pool_sample_stride(int nchunks) {
  int s = 1;
  while (2 * s * kPoolWaves <= nchunks) s *= 2;
  return s;
}

constexpr int kPoolHistPad = kBins + kBins / 8;  // four pad words per 32 bins (pool_pass)

struct PoolSmem {
  union {
    uint64_t list[kPoolListCap];
    uint32_t keys[kPoolBoundKeys];  // the first bound's keys, before anything is appended
    struct {
      double exact[kKcapLarge];
      double w[kKcapLarge];
    } tail;  // finish_row's terms, once the pool is in `sorted`
    uint64_t merge[kKcapLarge];  // the sort's second buffer, before those
  } u;
  union alignas(16) {  // (pool_pass reads and clears the histogram 16 bytes at a time)
    uint32_t hist[kPoolHistPad];
    uint64_t sorted[kKcapLarge];  // the row's pool, gathered after the last selection pass
  };
  SliceStat stats[kPoolWaves];
  BlockScratchT<kPoolWaves> bs;
  double pool_mass;
  double scaled_total;
  uint32_t count;
  int next_chunk;
};
static_assert(sizeof(uint64_t) * kKcapLarge <= sizeof(uint32_t) * kPoolHistPad, "the pool fits the histogram's words");
static_assert(kKcapLarge <= kPoolThreads, "block_merge_sort_desc sorts one entry per thread");

// One histogram pass of the pool kernel's selections, by the whole workgroup: the entries
// that bin_of admits (bin >= 0; bin 0 holds the largest) are counted, and wave 0 finds the
// bin where the count from the top reaches `need` (each lane reads its 32 consecutive bins as
// eight 16-byte words, stored four pad words per 32 so that every lane's bins start 16-byte
// aligned and eight lanes' reads cover the 32 banks). Returns the bin, the entries in the bins
// above it and the entries in it.
struct PoolBin {
  uint32_t bin, above, count;
};

__device__ __forceinline__ int pool_hist_at(int b) { return b + ((b >> 5) << 2); }

// The selection visits the candidate list in batches: `batches(g)` loads kPoolBatch entries
// per lane (all in flight before the first is used) and calls g(v, ok) with them; each_of
// hands the valid ones to f one by one.
constexpr int kPoolBatch = 4;
template <class Batches, class F>
__device__ __forceinline__ void each_of(Batches &batches, F &&f) {
  batches([&](const uint64_t (&v)[kPoolBatch], const bool (&ok)[kPoolBatch]) {
#pragma unroll
    for (int u = 0; u < kPoolBatch; ++u)
      if (ok[u]) f(v[u]);
  });
}

// wave_slot for a batch: slots for every taken entry of the lanes' B entries, with one LDS
// atomic for the wave (pos[u] is set where take[u]).
template <int B>
__device__ __forceinline__ void wave_slots(const bool (&take)[B], uint32_t *slot, uint32_t (&pos)[B]) {
  uint64_t m[B], any = 0ull;
  uint32_t total = 0u;
#pragma unroll
  for (int u = 0; u < B; ++u) {
    m[u] = __ballot(take[u]);
    any |= m[u];
    total += (uint32_t)__popcll(m[u]);
  }
  if (!any) return;
  const int leader = __ffsll((unsigned long long)any) - 1;  // a lane that takes: active
  uint32_t base = 0u;
  if ((int)lane_id() == leader) base = atomicAdd(slot, total);
  base = (uint32_t)__builtin_amdgcn_readlane((int)base, leader);
#pragma unroll
  for (int u = 0; u < B; ++u) {
    pos[u] = base + lanes_below(m[u]);
    base += (uint32_t)__popcll(m[u]);
  }
}

// Zeroes the pool histogram (no barrier).
__device__ __forceinline__ void pool_hist_clear(PoolSmem &sm) {
  static_assert(kPoolHistPad % 4 == 0 && kPoolHistPad <= 4 * kPoolThreads, "one 16-byte store per thread");
  if ((int)threadIdx.x < kPoolHistPad / 4) reinterpret_cast<u32x4 *>(sm.hist)[threadIdx.x] = u32x4{0u, 0u, 0u, 0u};
}

// The histogram is zero on entry (cleared after the first bound's select) and again on return:
// wave 0 zeroes the bins as it searches them, so a pass takes two barriers.
template <class Batches, class BinOf>
__device__ __forceinline__ PoolBin pool_pass(PoolSmem &sm, Batches &batches, BinOf bin_of, uint32_t need) {
  each_of(batches, [&](uint64_t v) {
    const int b = bin_of(v);
    // Lanes whose entries all fall in one bin (a tied key's entries do) add their count
    // with one atomic: 64 atomics on one LDS address serialise.
    // (Both masks are ballots of real predicates over the active lanes: a ballot of `true`
    // may be folded to the whole wave, which the loop's last, partial step is not.)
    const int b0 = __builtin_amdgcn_readfirstlane(b);
    const uint64_t same = __ballot(b == b0);
    if (!__ballot(b != b0)) {
      if (b0 >= 0 && wave_lane() == __ffsll((unsigned long long)same) - 1)
        atomicAdd(&sm.hist[pool_hist_at(b0)], (uint32_t)__popcll(same));
    } else if (b >= 0) {
      atomicAdd(&sm.hist[pool_hist_at(b)], 1u);
    }
  });
  __syncthreads();
  if (wave_id() == 0) {
    // Lane sums and their scan find the lane that owns the bin; then lanes 0..31 take one of
    // that lane's 32 bins each and a second scan finds the bin (a walk of the owner's bins by
    // the owner alone was a chain of up to 31 dependent LDS reads).
    constexpr int PER = kBins / kWaveSize;
    constexpr int kStride = PER + 4;  // a lane's bins and their pad, in words
    const int lane = wave_lane();
    uint32_t sum = 0u;
    static_assert(PER == 32 && kStride % 4 == 0, "pool_hist_at: a lane's bins are lane * 36 + q, 16-byte aligned");
    u32x4 *mine = reinterpret_cast<u32x4 *>(sm.hist + lane * kStride);
    u32x4 h[PER / 4];
#pragma unroll
    for (int q = 0; q < PER / 4; ++q) h[q] = mine[q];
#pragma unroll
    for (int q = 0; q < PER / 4; ++q) sum += h[q].x + h[q].y + h[q].z + h[q].w;
    const uint32_t inc = wave_inclusive_scan_u32(sum);
    // need <= the total: some lane's running sum reaches it (else the last lane, whose
    // reads stay inside the histogram).
    const uint64_t got = __ballot(inc >= need);
    const int owner = got ? __ffsll((unsigned long long)got) - 1 : kWaveSize - 1;
    const uint32_t before = (uint32_t)__builtin_amdgcn_readlane((int)(inc - sum), owner);
    const uint32_t c = lane < PER ? sm.hist[owner * kStride + lane] : 0u;
    // Zero for the next pass (after the reads above: a wave's LDS operations complete in order).
#pragma unroll
    for (int q = 0; q < PER / 4; ++q) mine[q] = u32x4{0u, 0u, 0u, 0u};
    const uint32_t cum = before + wave_inclusive_scan_u32(c);
    // The owner's last bin holds it if none before does.
    const uint64_t reach = __ballot(lane < PER - 1 && cum >= need);
    const int q = reach ? __ffsll((unsigned long long)reach) - 1 : PER - 1;
    if (lane == q) {
      sm.bs.bin = (uint32_t)(owner * PER + q);
      sm.bs.above = cum - c;
      sm.bs.count = c;
    }
  }
  __syncthreads();
  // (No barrier after the read: the next pass's search writes sm.bs only after its visit's
  // barrier, and the histogram is already zero.)
  return PoolBin{sm.bs.bin, sm.bs.above, sm.bs.count};
}

// The composite T with exactly `need` entries >= T (1 <= need <= entries), given that every
// entry's key lies in [lo, hi]: key passes over the live key range, 2,048 bins each, until one
// key remains (a quantized row resolves in one), then the ~index digits of that key's
// entries, from bit index_bits - 1 down (every index is below 2^index_bits, so the ~index
// bits above are ones). A pass that leaves its bin exactly taken ends early.
// The rest of pool_select from a key range [lo, hi] that holds the `need`-th entry: narrower
// key passes until one key remains, then that key's ties by their indices' digits.
template <class Batches>
__device__ __forceinline__ uint64_t pool_select_from(PoolSmem &sm, Batches &batches, uint32_t need, uint32_t lo,
                                                     uint32_t hi, int key_passes, int index_bits) {
  while (lo != hi) {
    ++key_passes;
    const uint32_t range = hi - lo;
    const int bits = 32 - __builtin_clz(range);
    const int shift = bits > 11 ? bits - 11 : 0;
    const uint32_t top_key = hi, low_key = lo;
    const PoolBin r = pool_pass(sm, batches, [&](uint64_t v) {
      const uint32_t k = composite_key(v);
      return (k >= low_key && k <= top_key) ? (int)((top_key - k) >> shift) : -1;
    }, need);
    need -= r.above;
    const uint32_t bin_top = hi - (r.bin << shift);
    const uint32_t bin_low = bin_top - min((1u << shift) - 1u, bin_top - lo);
    if (r.count == need) {  // the whole bin is taken
      if (wave_id() == 0) {
        TABBY_RECORD(26, key_passes);
        TABBY_STAMP(23);
      }
      return (uint64_t)bin_low << 32;
    }
    hi = bin_top;
    lo = bin_low;
    if (shift == 0) break;
  }
  if (wave_id() == 0) {
    TABBY_RECORD(26, key_passes);
    TABBY_STAMP(23);
  }
  // The index digits from the top of the row's index width (11 bits, then the rest): above it
  // every ~index bit is one. (At vocab 151,936 the first pass bins 128 indices each, so the few
  // hundred entries of a tied key rarely share the chosen bin and one pass usually ends it.)
  int done = index_bits;
  uint64_t prefix = ((uint64_t)lo << 32) | (uint64_t)(done >= 32 ? 0u : ~0u << done);
  while (done > 0) {
    const int width = min(done, 11);
    const int sh = done - width;
    const uint32_t mask = (1u << width) - 1u;
    const uint64_t want = prefix >> done;
    const int d = done;
    const PoolBin r = pool_pass(sm, batches, [&](uint64_t v) {
      return (v >> d) == want ? (int)(mask - ((uint32_t)(v >> sh) & mask)) : -1;
    }, need);
    need -= r.above;
    prefix |= (uint64_t)(mask - r.bin) << sh;
    done = sh;
    if (r.count == need) return prefix;
  }
  return prefix;
}

// The row's kk-th largest candidate composite (need = kk entries at or above it), among the
// candidates that `batches` visits -- entries [sel_begin, sel_end) of the list (list[i] in LDS
// for i < kPoolListCap, else region[i]), at first the C candidates -- all with keys in
// [lo, hi]: histogram passes over the keys (2,048 bins of the candidates' own range, narrowed
// until one key remains -- a quantized row resolves in one), then over the tied key's index
// digits. After the first pass only the chosen bin's entries matter: they are copied behind
// the candidates (B entries at list[C ..), when C + B fits the LDS list) and `batches` is moved
// onto them, so the later passes visit those B alone instead of all C (config 5: ~2,800
// candidates, a tied bin of a few hundred; the later passes had re-read every candidate).
// Indices are below 2^index_bits.
// The caller has set sm.bs.slot2 = 0, sm.bs.u[0] = ~0 and sm.bs.u[1] = 0 (the compaction's
// counters) before the call; the passes' barriers publish them.
template <class Batches>
__device__ __forceinline__ uint64_t pool_select(PoolSmem &sm, Batches &batches, uint32_t need, uint32_t lo, uint32_t hi,
                                                uint32_t C, uint32_t &sel_begin, uint32_t &sel_end, int index_bits) {
  if (lo == hi) return pool_select_from(sm, batches, need, lo, hi, 0, index_bits);
  const uint32_t range = hi - lo;
  const int bits = 32 - __builtin_clz(range);
  const int shift = bits > 11 ? bits - 11 : 0;
  const PoolBin r = pool_pass(sm, batches, [&](uint64_t v) {
    const uint32_t k = composite_key(v);
    return (k >= lo && k <= hi) ? (int)((hi - k) >> shift) : -1;
  }, need);
  need -= r.above;
  const uint32_t bin_top = hi - (r.bin << shift);
  const uint32_t bin_low = bin_top - min((1u << shift) - 1u, bin_top - lo);
  if (r.count == need) {  // the whole bin is taken
    if (wave_id() == 0) {
      TABBY_RECORD(26, 1);
      TABBY_STAMP(23);
    }
    return (uint64_t)bin_low << 32;
  }
  if (shift == 0 || C + r.count > (uint32_t)kPoolListCap)
    return pool_select_from(sm, batches, need, bin_low, bin_top, 1, index_bits);
  // The chosen bin's entries, copied to list[C, C + B), and their smallest and largest key
  // (the later passes bin [smallest, largest]; one key -- a tie -- goes straight to the index
  // digits). Their counters were set before the first pass.
  uint32_t kmin = ~0u, kmax = 0u;
  batches([&](const uint64_t (&v)[kPoolBatch], const bool (&ok)[kPoolBatch]) {
    bool in[kPoolBatch];
    uint32_t at[kPoolBatch];
#pragma unroll
    for (int u = 0; u < kPoolBatch; ++u) {
      const uint32_t k = composite_key(v[u]);
      in[u] = ok[u] && k >= bin_low && k <= bin_top;
    }
    wave_slots(in, &sm.bs.slot2, at);
#pragma unroll
    for (int u = 0; u < kPoolBatch; ++u) {
      if (in[u]) {
        const uint32_t k = composite_key(v[u]);
        sm.u.list[C + at[u]] = v[u];
        kmin = min(kmin, k);
        kmax = max(kmax, k);
      }
    }
  });
  kmin = ~wave_max_u32(~kmin);
  kmax = wave_max_u32(kmax);
  if (wave_lane() == 0) {
    atomicMin(&sm.bs.u[0], kmin);
    atomicMax(&sm.bs.u[1], kmax);
  }
  __syncthreads();
  sel_begin = C;
  sel_end = C + sm.bs.slot2;  // the bin's r.count entries
  const uint32_t lo2 = sm.bs.u[0], hi2 = sm.bs.u[1];  // (nothing writes them again)
  return pool_select_from(sm, batches, need, lo2, hi2, 1, index_bits);
}

// Two workgroups per CU (74 KB of LDS and at most 64 VGPRs each): 512 rows run in one round,
// and one row's bound and tail overlap the other's streaming (the SIMDs issue the older
// workgroup's waves first, so the first-dispatched row ends its stream well before the
// other, whose tail alone then runs with nothing streaming beside it).
template <typename In, int VEC>
__global__ __launch_bounds__(kPoolThreads, 8) void pool_row_kernel(Launch L, Workspace W) {
  __shared__ PoolSmem sm;
  const int row = (int)blockIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(wave_id()), lane = wave_lane();  // w: scalar
  const tabby_row_params P = L.params[row];
  const int n = L.vocab;
  const int nchunks = (n + kWChunk - 1) / kWChunk;
  const int full_chunks = n / kWChunk;
  const bool valid_params = params_valid(P, L.k_max);
  const int keff = effective_k(P, n);
  const int kk = slice_keep(valid_params, keff, n, L.kcap, L.head_pass, L.topk_cap);
  const In *src = reinterpret_cast<const In *>(L.logits) + (size_t)row * n;
  uint64_t *region = W.cands + (size_t)row * W.row_cand_stride;
  if (w == 0) {
    TABBY_STAMP(16);
    TABBY_STAMP_REAL(24);
    // Where the workgroup runs: XCC_ID, and HW_ID's CU, shader-array and engine fields.
    TABBY_RECORD(30, ((__builtin_amdgcn_s_getreg((31 << 11) | 20) & 0xfu) << 16) |
                         ((__builtin_amdgcn_s_getreg((31 << 11) | 4) >> 8) & 0xffu));
  }
  // Claim order: claim v takes chunk (v mod 16) s + v / 16 while v < 16 s (s the largest power
  // of two with 16 s <= the row's chunks), then chunk v. Claims w and 16 + w, wave w's first
  // two chunks (s w and s w + 1 when s >= 2), are the first bound's sample, spread over the row
  // so that it stands for the whole row; each chunk is still 4 KB of consecutive elements.
  const int s_log = __builtin_ctz(pool_sample_stride(nchunks));
  auto chunk_of = [&](int v) {
    return v < (kPoolWaves << s_log) ? ((v & (kPoolWaves - 1)) << s_log) + v / kPoolWaves : v;
  };
  if (threadIdx.x == 0) {
    sm.next_chunk = 2 * kPoolWaves;
    sm.count = 0u;
  }
  __syncthreads();
  const ChunkReader<In, VEC> rd(src, n);
  auto load = [&](int c, float(&v)[kWChunkPerLane]) { rd.load(c, v); };
  auto claim = [&]() {
    int c = 0;
    if (lane == 0) c = atomicAdd(&sm.next_chunk, 1);
    return chunk_of(__builtin_amdgcn_readfirstlane(c));
  };
  // Elements past the row's end (or a chunk past its last) become -inf for the statistics.
  auto mask_tail = [&](int c, float(&v)[kWChunkPerLane]) {
    if (c >= full_chunks) {
#pragma unroll
      for (int e = 0; e < kWChunkPerLane; ++e)
        if (wave_local<VEC>(c, e) >= n) v[e] = -INFINITY;
    }
  };
  float x[kWChunkPerLane], y[kWChunkPerLane];
  const int a = chunk_of(w);
  int b = chunk_of(kPoolWaves + w);
  load(a, x);
  load(b, y);
  mask_tail(a, x);
  mask_tail(b, y);
  // A bound from the sample: the top 22 key bits of the need-th largest of its 4,096 group
  // maxima (four elements of a lane's first chunk and the same four of its second), so that
  // `need` distinct elements of the row lie at or above it.
  // The select leaves the histogram zeroed for the selection's passes (pool_pass).
  auto sample_bound = [&](uint32_t need) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float gm = -INFINITY;
#pragma unroll
      for (int q = 0; q < 4; ++q) gm = fmaxf(gm, fmaxf(x[4 * g + q], y[4 * g + q]));
      sm.u.keys[threadIdx.x * 4 + g] = min(max(key_of(gm), kNegInfKey), 0xff800000u);
    }
    __syncthreads();
    auto keys = [&](auto &&f) {
      for (int i = threadIdx.x; i < kPoolBoundKeys; i += kPoolThreads) f((uint64_t)sm.u.keys[i] << 32);
    };
    const float t = theta_of(radix_select(keys, need, sm.hist, sm.bs, 2).prefix);
    pool_hist_clear(sm);
    __syncthreads();  // the keys are read before the list overwrites them
    return t;
  };
  // The first bound. At kk the bound is certain to leave kk candidates, but the sample is a
  // fifth of a 151,936 row, so it leaves ~6 kk there; rows of at least kPoolGuessChunks
  // chunks (a sample of at most a quarter) stream at the (kk/2)-th largest group maximum
  // instead -- ~2.5 kk candidates when the sample stands for the row -- and take their
  // candidates again at the certain bound if the guess leaves fewer than kk.
  const bool guess = kk > 1 && kk < n && nchunks >= kPoolGuessChunks;
  float theta = -INFINITY;
  if (kk > 0 && kk < n) {
    theta = sample_bound(guess ? (uint32_t)kk / 2u : (uint32_t)kk);
    if (w == 0) TABBY_STAMP(22);
  }

  float lane_max = -INFINITY;
  float lane_ml = 0.0f;   // the reference of lane_sum's terms (as in wave_slice)
  double lane_sum = 0.0;
  // Appends chunk c's elements at or above theta to the list.
  auto append = [&](int c, float(&cur)[kWChunkPerLane]) __attribute__((always_inline)) {
    // Past the row's end the elements become NaN, which fails x >= theta for every theta
    // (-inf included), so that one compare decides each element below.
    if (c >= full_chunks) {
#pragma unroll
      for (int e = 0; e < kWChunkPerLane; ++e)
        if (wave_local<VEC>(c, e) >= n) cur[e] = __builtin_nanf("");
    }
    // The chunk's candidates: each lane counts its own, a wave scan places the lanes' runs
    // one after another behind one reservation for the wave, and each lane writes its
    // candidates to its run in element order (a compare, the entry and its store per
    // element; placing every element's takers by a ballot and a lane count cost four
    // instructions more per element).
    uint32_t mine = 0u;
#pragma unroll
    for (int e = 0; e < kWChunkPerLane; ++e) mine += cur[e] >= theta ? 1u : 0u;
    const uint32_t inc = wave_inclusive_scan_u32(mine);
    const uint32_t total = (uint32_t)__builtin_amdgcn_readlane((int)inc, kWaveSize - 1);
    if (total == 0u) return;
    uint32_t at = 0u;
    if (lane == 0) at = atomicAdd(&sm.count, total);
    at = (uint32_t)__builtin_amdgcn_readfirstlane((int)at);
    uint32_t pos = at + inc - mine;
    // A reservation inside the LDS list (all but the rarest) stores through a pointer that
    // steps by one entry, with no per-element test of where the entry goes.
    if (at + total <= (uint32_t)kPoolListCap) {
      uint64_t *dst = sm.u.list + pos;
#pragma unroll
      for (int e = 0; e < kWChunkPerLane; ++e) {
        if (cur[e] >= theta) *dst++ = composite(key_of(cur[e]), (uint32_t)wave_local<VEC>(c, e));
      }
    } else {
#pragma unroll
      for (int e = 0; e < kWChunkPerLane; ++e) {
        if (cur[e] >= theta) {
          const uint64_t v = composite(key_of(cur[e]), (uint32_t)wave_local<VEC>(c, e));
          if (pos < (uint32_t)kPoolListCap) sm.u.list[pos] = v; else region[pos] = v;
          ++pos;
        }
      }
    }
  };
  auto step = [&](int c, float(&cur)[kWChunkPerLane]) __attribute__((always_inline)) {
    mask_tail(c, cur);
    float cm = cur[0];
#pragma unroll
    for (int e = 1; e < kWChunkPerLane; ++e) cm = fmaxf(cm, cur[e]);
    const float nm = fmaxf(lane_max, cm);
    if (nm != -INFINITY) {
      const float ml = nm * kLog2e;
      float t[kWChunkPerLane];
#pragma unroll
      for (int e = 0; e < kWChunkPerLane; ++e) t[e] = __builtin_amdgcn_exp2f(fmaf(cur[e], kLog2e, -ml));
#pragma unroll
      for (int h = kWChunkPerLane / 2; h > 0; h >>= 1) {
#pragma unroll
        for (int e = 0; e < h; ++e) t[e] += t[e + h];
      }
      const double rescale = lane_max == -INFINITY ? 0.0 : (double)__builtin_amdgcn_exp2f(lane_ml - ml);
      lane_sum = lane_sum * rescale + (double)t[0];
      lane_max = nm;
      lane_ml = ml;
    }
    if (kk == 0 || !__ballot(cm >= theta)) return;
    append(c, cur);
  };
  if (a < nchunks) step(a, x);  // chunk b is already in flight
  while (b < nchunks) {
    const int c = claim();
    load(c, x);
    step(b, y);
    if (c >= nchunks) break;
    b = claim();
    load(b, y);
    step(c, x);
  }
  TABBY_STAMP(w);
  const float ms = wave_max(lane_max);
  const double ss = wave_sum(rebase_sum(lane_sum, lane_max, lane_ml, ms));
  if (lane == 0) {
    SliceStat st;
    st.max = ms;
    st.count = 0u;
    st.sum = ss;
    sm.stats[w] = st;
  }
  __syncthreads();
  uint32_t C = sm.count;
  // A guessed bound that left fewer than kk candidates (a sample unlike the rest of its row):
  // the certain bound from the sample, read again, and the row's candidates at it, an
  // element per lane and step (a rare path, kept apart from the stream's code).
  const bool rescan = guess && C < (uint32_t)kk;
  if (rescan) {
    __syncthreads();  // every wave has read the count (the sample's keys overwrite the list)
    load(chunk_of(w), x);
    load(chunk_of(kPoolWaves + w), y);
    mask_tail(chunk_of(w), x);
    mask_tail(chunk_of(kPoolWaves + w), y);
    theta = sample_bound((uint32_t)kk);
    if (threadIdx.x == 0) sm.count = 0u;
    __syncthreads();
    constexpr int kAhead = 8;  // loads in flight per lane
    for (int base = 0; base < n; base += kAhead * kPoolThreads) {
      float v[kAhead];
#pragma unroll
      for (int u = 0; u < kAhead; ++u) {
        const int i = base + u * kPoolThreads + (int)threadIdx.x;
        v[u] = i < n ? load_one(src + i) : __builtin_nanf("");
      }
#pragma unroll
      for (int u = 0; u < kAhead; ++u) {
        const bool take = v[u] >= theta;
        const uint64_t m = __ballot(take);
        if (m) {
          uint32_t at = 0u;
          if (lane == 0) at = atomicAdd(&sm.count, (uint32_t)__popcll(m));
          at = (uint32_t)__builtin_amdgcn_readfirstlane((int)at);
          if (take) {
            const uint32_t pos = at + (uint32_t)lanes_below(m);
            const uint64_t e = composite(key_of(v[u]), (uint32_t)(base + u * kPoolThreads + (int)threadIdx.x));
            if (pos < (uint32_t)kPoolListCap) sm.u.list[pos] = e; else region[pos] = e;
          }
        }
      }
    }
    __syncthreads();
    C = sm.count;
  }
  // The row's exact top kk of the candidates, unsorted: to `sorted` in LDS for a row this
  // workgroup samples itself (valid parameters, a pool of at most kcap, finite statistics:
  // every row that merge_kernel would sample from the pool), else to region[0 .. kept) for
  // merge_kernel (statuses and whole-vocabulary rows).
  if (w == 0) {
    TABBY_STAMP(17);
    TABBY_RECORD(31, C);
    TABBY_RECORD(29, rescan ? 1 : 0);
  }
  const RowStats rs = row_stats(sm.stats, kPoolWaves);
  // The row's outcome, as merge_kernel decides it: a status (parameters outside the contract,
  // statistics outside the domain, a whole-vocabulary row with no head pass), a pool this
  // workgroup samples (`here`), or a whole-vocabulary row for merge_kernel and the head
  // kernels. (C >= kk >= 1 for a pool in the domain: theta has kk elements at or above it --
  // the floor always, a guessed bound once the count above has shown it.)
  const bool in_domain = rs.max > -INFINITY && rs.max < INFINITY && rs.sum_exp > 0.0 && rs.sum_exp < INFINITY;
  const bool pool = keff <= L.kcap;
  int32_t status = TABBY_OK;
  if (!valid_params || !in_domain) status = !valid_params ? TABBY_EINVAL : TABBY_EDOMAIN;
  else if (!pool && !L.head_pass) status = TABBY_EINVAL;
  else if (pool && C == 0u) status = TABBY_EDOMAIN;
  const bool here = status == TABBY_OK && pool;
  auto put = [&](uint32_t at, uint64_t v) {
    if (here) sm.sorted[at] = v; else region[at] = v;
  };
  uint32_t kept = 0u;
  const bool selects = status == TABBY_OK && kk > 0;
  if (selects && C > (uint32_t)kk) {
    uint32_t sel_begin = 0u, sel_end = C;  // the entries `batches` visits (pool_select narrows them)
    auto batches = [&](auto &&g) {
      for (uint32_t base = sel_begin; base < sel_end; base += kPoolBatch * kPoolThreads) {
        uint64_t v[kPoolBatch];
        bool ok[kPoolBatch];
#pragma unroll
        for (int u = 0; u < kPoolBatch; ++u) {
          const uint32_t i = base + u * kPoolThreads + threadIdx.x;
          ok[u] = i < sel_end;
          v[u] = !ok[u] ? 0ull : i < (uint32_t)kPoolListCap ? sm.u.list[i] : region[i];
        }
        g(v, ok);
      }
    };
    // Every candidate's key lies between theta's and the row max's.
    // The compaction's and the gather's slot counters, published by the passes' barriers.
    if (threadIdx.x == 0) {
      sm.bs.slot = 0u;
      sm.bs.slot2 = 0u;
      sm.bs.u[0] = ~0u;
      sm.bs.u[1] = 0u;
    }
    const uint64_t thr = pool_select(sm, batches, (uint32_t)kk, key_of(theta), key_of(rs.max), C, sel_begin, sel_end,
                                     n > 1 ? 32 - __builtin_clz((unsigned)(n - 1)) : 1);
    sel_begin = 0u;  // the gather below visits every candidate
    sel_end = C;
    // (No barrier: the last pass's search, which read the histogram that `sorted` overlays,
    // ended with one.)
    // region[0 .. kk) lies below the overflow entries (kk <= 1,024 < kPoolListCap).
    if (w == 0) TABBY_STAMP(18);
    batches([&](const uint64_t (&v)[kPoolBatch], const bool (&ok)[kPoolBatch]) {
      bool take[kPoolBatch];
      uint32_t at[kPoolBatch];
#pragma unroll
      for (int u = 0; u < kPoolBatch; ++u) take[u] = ok[u] && v[u] >= thr;
      wave_slots(take, &sm.bs.slot, at);
#pragma unroll
      for (int u = 0; u < kPoolBatch; ++u)
        if (take[u] && at[u] < (uint32_t)kk) put(at[u], v[u]);
    });
    kept = (uint32_t)kk;
  } else if (selects) {
    for (uint32_t i = threadIdx.x; i < C; i += kPoolThreads) put(i, sm.u.list[i]);  // C <= kk: in LDS
    kept = C;
  }
  if (here) {
    // sampleFromTopK over the pool, as merge_kernel would: the statistics are this row's one
    // slice's (the merge's sum in slice order is that slice's sum), the pool sorted descending.
    const int count = (int)kept;
    const int npow = next_pow2(count);
    for (int i = count + (int)threadIdx.x; i < npow; i += kPoolThreads) sm.sorted[i] = 0ull;
    __syncthreads();  // the gather's reads of the list are done: finish_row reuses it
    if (w == 0) TABBY_STAMP(19);
    block_merge_sort_desc<kPoolWaves>(sm.sorted, sm.u.merge, npow);
    if (w == 0) TABBY_STAMP(20);
    finish_row<kKcapLarge, In, PoolSmem, kPoolWaves>(sm, L, row, src, count, rs.max, rs.sum_exp, P);
  }
  if (w == 0) {
    if (lane == 0) {
      SliceStat st;
      st.max = rs.max;
      st.count = here || status != TABBY_OK ? kPoolRowDone : kept;
      st.sum = rs.sum_exp;
      W.stats[(size_t)row * kMaxSplits] = st;
      if (status != TABBY_OK) {
        write_status(L, row, status, rs.max, rs.sum_exp);
        W.row_state[row].status = status;
      }
    }
    TABBY_STAMP(21);
    TABBY_STAMP_REAL(25);
  }
}

}  // namespace tabby

// Scratch of the allocation-free entry (tabby_sampler_sample_device_noalloc), per GPU.
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

// =========================================================================================
// Host side.
// =========================================================================================
using namespace tabby;

struct tabby_sampler {
  int device = 0;
  int cus = 0;  // compute units of the device
  int32_t vocab_max = 0, rows_max = 0, k_max = 0;
  Workspace ws{};
  void *ws_base = nullptr;
  size_t head_rows_cap = 0;  // rows the head buffers are sized for (0: not allocated)
  void *head_base = nullptr;
  tabby_row_params *params_dev = nullptr;
  tabby_row_result *results_dev = nullptr;
  tabby_row_params *params_pinned = nullptr;
  tabby_row_result *results_pinned = nullptr;
  int32_t *topk_ids_dev = nullptr;
  float *topk_logits_dev = nullptr;
  size_t topk_elems_cap = 0;
};

namespace tabby {

thread_local std::string g_last_error;

int record_failure(int status, const std::string &msg) {
  g_last_error = msg;
  return status;
}

int device_cus(int device, int *cus) {
  static std::mutex mu;
  static int cached[64] = {0};
  if (device < 0 || device >= 64) return record_failure(TABBY_EINVAL, "device ordinal out of range");
  std::lock_guard<std::mutex> lock(mu);
  if (cached[device] == 0) {
    int n = 0;
    const hipError_t e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device);
    if (e != hipSuccess) return record_hip_failure(e, "hipDeviceGetAttribute(multiprocessor count)");
    cached[device] = n;
  }
  *cus = cached[device];
  return TABBY_OK;
}

int handle_view(const tabby_sampler *h, HandleView *out) {
  if (!h) return record_failure(TABBY_EINVAL, "sampler handle is null");
  out->device = h->device;
  out->cus = h->cus;
  out->vocab_max = h->vocab_max;
  out->rows_max = h->rows_max;
  out->k_max = h->k_max;
  out->scratch = h->ws.cands;
  out->scratch_bytes = (size_t)h->rows_max * (size_t)h->ws.row_cand_stride * sizeof(uint64_t);
  return TABBY_OK;
}

}  // namespace tabby

namespace {

int fail(int status, const std::string &msg) { return record_failure(status, msg); }

int hip_fail(hipError_t e, const char *what) {
  return fail(TABBY_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define HIP_TRY(expr)                                  \
  do {                                                 \
    hipError_t e_ = (expr);                            \
    if (e_ != hipSuccess) return hip_fail(e_, #expr);  \
  } while (0)

struct Plan {
  int slice_len;
  int splits;
  int vec;
};

// Enough slices per row that the batch fills the chip about once: 256 CUs x 3 resident
// 256-lane workgroups of the slice kernel (its 41.5 KB of LDS leaves room for three; a
// larger grid ran in two rounds -- config 5, 512 rows: 3 slices per row took 225 us, one
// 200 us), rounded down, or 256 CUs x 4 SIMDs x 4 one-wave workgroups for the wave kernel
// (measured at 256 rows: 16 slices per row, 39.9 us per call, beat 12 per row, 41.4 us --
// the SIMDs issue their oldest wave first and a fourth wave hides more of the others'
// waits -- and 18 or 20 per row, which no longer fit at once, ~50 us). Each
// slice is at least one chunk long (two for the wave kernel) and aligned to the vector
// loads. A row's wave slices are capped at kMaxWaveSplits: with few rows the chip is idle
// anyway and the latency is one slice's chain plus the merge, whose cost grows with the
// number of lists (measured on one row: 24 slices of 2048 beat 12 of 4096 and 48 of 1024
// at vocab 49152; 37 slices of 4096 beat 46 and 74 at vocab 151936).
constexpr int kTargetGroups = 768;
constexpr int kTargetWaves = 4096;
constexpr int kMaxWaveSplits = 36;

Plan make_plan(int rows, int vocab, int dtype, const void *logits, bool wave) {
  Plan p;
  const int vec_elems = dtype == TABBY_F32 ? 4 : 8;
  const bool aligned = ((uintptr_t)logits % 16u) == 0 && vocab % vec_elems == 0;
  p.vec = aligned ? vec_elems : 1;
  const int chunk = wave ? 2 * kWChunk : kChunk;
  const int target = wave ? kTargetWaves : kTargetGroups;
  const int most = std::min(wave ? kMaxWaveSplits : kMaxSplits, (vocab + chunk - 1) / chunk);
  const int want = std::max(1, std::min(most, wave ? (target + rows - 1) / rows : target / rows));
  const int granule = (wave ? kWaveSize : kBlock) * p.vec;
  const int per = (vocab + want - 1) / want;
  p.slice_len = (per + granule - 1) / granule * granule;
  p.splits = (vocab + p.slice_len - 1) / p.slice_len;
  return p;
}

// One workgroup per row (row_kernel) once the rows alone fill the CUs and a row's slices
// fit one workgroup.
bool per_row_launch(const Launch &L, int cus) { return L.kcap <= kWaveKcap && L.rows >= cus && L.splits <= kRowWaves; }

// Up to half as many rows as CUs (pools <= 256): each row is cut into parts of at least
// kMinPart elements, one 16-wave row_kernel workgroup each, about one workgroup per CU in all;
// wave_merge_kernel then merges the parts' sorted lists (one row of 151,936: 14.8 us in ten
// parts against 18.8 us in 37 one-wave slices; 32 rows: 17.2 against 22.9 us). Returns the
// number of parts (< 2: not used) and sets part_len (a multiple of a wave chunk, so parts
// start on vector boundaries).
constexpr int kMinPart = kRowWaves * kWChunk;
constexpr int kMaxParts = 16;
int row_parts(int rows, int vocab, int cus, int &part_len) {
  const int by_cus = cus / std::max(rows, 1);
  const int by_len = (vocab + kMinPart - 1) / kMinPart;
  int parts = std::min(std::min(by_cus, by_len), kMaxParts);
  if (parts < 2) return 0;
  const int per = (vocab + parts - 1) / parts;
  part_len = (per + kWChunk - 1) / kWChunk * kWChunk;
  return (vocab + part_len - 1) / part_len;
}

template <typename In, int VEC>
hipError_t launch_pair(const Launch &L, const Workspace &W, int cus, hipStream_t stream) {
  const dim3 slices((unsigned)(L.rows * L.splits)), rows((unsigned)L.rows);
  if (L.parts == 1) {
    hipLaunchKernelGGL((row_kernel<In, VEC>), rows, dim3((unsigned)(L.row_waves * kWaveSize)), 0, stream, L, W);
  } else if (L.parts > 1) {
    hipLaunchKernelGGL((row_kernel<In, VEC>), slices, dim3((unsigned)(L.row_waves * kWaveSize)), 0, stream, L, W);
    hipLaunchKernelGGL((wave_merge_kernel<In>), rows, dim3(kBlock), 0, stream, L, W);
  } else if (L.kcap <= kWaveKcap) {
    hipLaunchKernelGGL((wave_kernel<In, VEC>), slices, dim3(kWaveSize), 0, stream, L, W);
    hipLaunchKernelGGL((wave_merge_kernel<In>), rows, dim3(kBlock), 0, stream, L, W);
  } else if (L.pool_rows) {
    // pool_row_kernel ends every row but a head pass's whole-vocabulary ones, which
    // merge_kernel hands to the head kernels.
    hipLaunchKernelGGL((pool_row_kernel<In, VEC>), rows, dim3(kPoolThreads), 0, stream, L, W);
    if (L.head_pass)
      hipLaunchKernelGGL((merge_kernel<kKcapLarge, In>), rows, dim3(kBlock), 0, stream, L, W);
  } else {
    hipLaunchKernelGGL((slice_kernel<In, VEC>), slices, dim3(kBlock), 0, stream, L, W);
    hipLaunchKernelGGL((merge_kernel<kKcapLarge, In>), rows, dim3(kBlock), 0, stream, L, W);
  }
  return hipGetLastError();
}

template <typename In, int VEC>
hipError_t launch_head(const Launch &L, const Workspace &W, hipStream_t stream) {
  hipLaunchKernelGGL((head_kernel<In, VEC>), dim3((unsigned)(L.rows * L.h_splits)), dim3(kWaveSize), 0,
                     stream, L, W);
  hipLaunchKernelGGL((head_fast_kernel<In>), dim3((unsigned)L.rows), dim3(kPlanThreads), 0, stream, L, W);
  hipLaunchKernelGGL(head_sort_kernel, dim3((unsigned)(L.rows * kSortGroups)), dim3(kBlock), 0, stream, L, W);
  hipLaunchKernelGGL((head_finish_kernel<In>), dim3((unsigned)L.rows), dim3(kFinishThreads), 0, stream, L, W);
  return hipGetLastError();
}

hipError_t dispatch(int dtype, const Plan &p, const Launch &L, const Workspace &W, int cus, hipStream_t s) {
  hipError_t e;
  if (dtype == TABBY_F32) {
    e = p.vec == 4 ? launch_pair<float, 4>(L, W, cus, s) : launch_pair<float, 1>(L, W, cus, s);
    if (e == hipSuccess && L.head_pass) e = p.vec == 4 ? launch_head<float, 4>(L, W, s) : launch_head<float, 1>(L, W, s);
    return e;
  }
  e = p.vec == 8 ? launch_pair<uint16_t, 8>(L, W, cus, s) : launch_pair<uint16_t, 1>(L, W, cus, s);
  if (e == hipSuccess && L.head_pass) e = p.vec == 8 ? launch_head<uint16_t, 8>(L, W, s) : launch_head<uint16_t, 1>(L, W, s);
  return e;
}

// The launch shape of one call: which kernels run and how each row is cut (everything in L
// except the parameter, result and top-k pointers). Sorted lists of consecutive slices sit
// slice_len entries apart (the handle's candidate region has room for a whole row).
Plan plan_launch(int rows, int vocab, int dtype, const void *logits, int k_max, int topk_cap, int cus,
                 bool head_pass, Launch &L) {
  const int kcap = k_max <= kKcapSmall ? kKcapSmall : kKcapLarge;
  const Plan p = make_plan(rows, vocab, dtype, logits, kcap <= kWaveKcap);
  L = Launch{};
  L.logits = logits;
  L.rows = rows;
  L.vocab = vocab;
  L.splits = p.splits;
  L.slice_len = p.slice_len;
  L.topk_cap = topk_cap;
  L.k_max = k_max;
  L.kcap = kcap;
  L.head_pass = head_pass ? 1 : 0;
  L.h_slice_len = kHeadSlice;
  L.h_splits = (vocab + kHeadSlice - 1) / kHeadSlice;
  L.parts = 0;
  L.row_waves = 0;
  L.pool_rows = 0;
  if (kcap > kWaveKcap && rows >= cus) {
    // One pool_row_kernel workgroup per row (merge_kernel, for a head pass, reads a
    // whole-vocabulary row's list as slice 0).
    L.pool_rows = 1;
    L.splits = 1;
    L.slice_len = vocab;
  } else if (L.kcap <= kWaveKcap && rows * 2 > cus && rows < cus) {
    // Between half the CUs and all of them: one 16-wave workgroup per row all the same (the
    // idle CUs leave the others more of the HBM bandwidth). Against the one-wave slices and
    // their merge kernel: 130 rows 32.5 -> 22.6 us, 200 rows 39.5 -> 26.5 us, 255 rows 43.9 ->
    // 31.2 us (151,936 f32, k = 50), 200 rows at k = 100 50.6 -> 29.4 us.
    L.parts = 1;
    L.row_waves = kRowWaves;
  } else if (per_row_launch(L, cus)) {
    L.parts = 1;
    L.row_waves = std::max(L.splits, kRowMinWaves);  // at least the five the merge uses
  } else if (kcap <= kWaveKcap) {
    int part_len = 0;
    const int parts = row_parts(rows, vocab, cus, part_len);
    if (parts >= 2 && parts <= 3) {
      // Two or three parts' worth of row: one workgroup streams it all and finishes it, with
      // no second launch (config 1, one row of 49,152: 14.2 us, against 14.9 us in three
      // parts).
      L.parts = 1;
      L.row_waves = kRowWaves;
    } else if (parts >= 2) {
      L.parts = parts;
      L.splits = parts;  // wave_merge_kernel merges one list per part
      L.slice_len = part_len;
      L.row_waves = kRowWaves;
    }
  }
  L.list_stride = L.slice_len;
  return p;
}

// The allocation-free entry's scratch: its row statuses, slice statistics and packed
// sorted lists live in `scratch`, one copy per GPU, held until the process ends. In host
// code the array's name stands for a host-side placeholder, not a device address: each
// device's address is taken once with hipGetSymbolAddress (with that device current) and
// only that pointer reaches kernels.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices];
int g_scratch_cus[kMaxDevices];

int scratch_of_current_device(int &device, void *&base, int &cus) {
  HIP_TRY(hipGetDevice(&device));
  if (device < 0 || device >= kMaxDevices)
    return fail(TABBY_EINVAL, "device ordinal " + std::to_string(device) + " is beyond " + std::to_string(kMaxDevices));
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[device]) {
    void *p = nullptr;
    HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    int n = 0;
    HIP_TRY(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device));
    g_scratch_cus[device] = n;
    g_scratch_ptr[device] = p;
  }
  base = g_scratch_ptr[device];
  cus = g_scratch_cus[device];
  return TABBY_OK;
}

int check_common(tabby_sampler *h, const void *logits, int32_t dtype, int32_t rows, int32_t vocab,
                 int32_t topk_cap) {
  if (!h) return fail(TABBY_EINVAL, "sampler handle is null");
  if (!logits) return fail(TABBY_EINVAL, "logits pointer is null");
  if (dtype != TABBY_F32 && dtype != TABBY_F16) return fail(TABBY_EINVAL, "dtype must be TABBY_F32 or TABBY_F16");
  if (rows < 1 || rows > h->rows_max)
    return fail(TABBY_EINVAL, "rows must be between 1 and " + std::to_string(h->rows_max) + ", got " + std::to_string(rows));
  if (vocab < 1 || vocab > h->vocab_max)
    return fail(TABBY_EINVAL, "vocab must be between 1 and " + std::to_string(h->vocab_max) + ", got " + std::to_string(vocab));
  if (topk_cap < 0) return fail(TABBY_EINVAL, "topk_cap must be >= 0");
  return TABBY_OK;
}

}  // namespace

extern "C" {

#ifdef TABBY_TIMELINE
// The timeline library only (not part of the drop-in boundary): copies the row kernel's phase
// stamps (kTimelineGroups x kTimelineSlots uint64, see TABBY_STAMP) to host memory.
TABBY_API int tabby_debug_timeline(void *host, size_t bytes) {
  if (bytes > sizeof(unsigned long long) * tabby::kTimelineGroups * tabby::kTimelineSlots) return TABBY_EINVAL;
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(tabby::g_timeline), bytes, 0, hipMemcpyDeviceToHost) == hipSuccess
             ? TABBY_OK
             : TABBY_EHIP;
}
#endif

const char *tabby_last_error(void) { return g_last_error.c_str(); }

const char *tabby_version(void) { return "tabby_sampler 0.1.0 (gfx950)"; }

int tabby_sampler_create(int device, int32_t vocab_max, int32_t rows_max, int32_t k_max,
                         tabby_sampler **out) {
  if (!out) return fail(TABBY_EINVAL, "out pointer is null");
  *out = nullptr;
  if (vocab_max < 1 || vocab_max > kMaxSplits * kChunk)
    return fail(TABBY_EINVAL, "vocab_max must be between 1 and " + std::to_string(kMaxSplits * kChunk));
  if (rows_max < 1 || rows_max > (1 << 20)) return fail(TABBY_EINVAL, "rows_max must be between 1 and 1048576");
  if (k_max < 1 || k_max > kKcapLarge)
    return fail(TABBY_ECAPACITY, "k_max must be between 1 and " + std::to_string(kKcapLarge));
  HIP_TRY(hipSetDevice(device));
  int cus = 0;
  HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));

  tabby_sampler *h = new tabby_sampler();
  h->device = device;
  h->cus = cus;
  h->vocab_max = vocab_max;
  h->rows_max = rows_max;
  h->k_max = k_max;
  h->ws.row_cand_stride = vocab_max;  // each slice may flush up to its own length

  const size_t rows = (size_t)rows_max;
  size_t off = 0;
  auto carve = [&](size_t bytes) {
    const size_t at = off;
    off += (bytes + 255) & ~(size_t)255;
    return at;
  };
  const size_t o_hcnt = carve(rows * 4);
  const size_t o_stats = carve(rows * kMaxSplits * sizeof(SliceStat));
  const size_t o_cands = carve(rows * (size_t)h->ws.row_cand_stride * 8);
  const size_t o_rs = carve(rows * sizeof(RowState));
  const size_t o_par = carve(rows * sizeof(tabby_row_params));
  const size_t o_res = carve(rows * sizeof(tabby_row_result));
  hipError_t e = hipMalloc(&h->ws_base, off);
  if (e != hipSuccess) {
    delete h;
    return hip_fail(e, "hipMalloc(workspace)");
  }
  char *b = (char *)h->ws_base;
  h->ws.head_count = (uint32_t *)(b + o_hcnt);
  h->ws.stats = (SliceStat *)(b + o_stats);
  h->ws.cands = (uint64_t *)(b + o_cands);
  h->ws.row_state = (RowState *)(b + o_rs);
  h->params_dev = (tabby_row_params *)(b + o_par);
  h->results_dev = (tabby_row_result *)(b + o_res);
  e = hipMemset(h->ws_base, 0, off);
  if (e == hipSuccess) e = hipHostMalloc((void **)&h->params_pinned, rows * sizeof(tabby_row_params), hipHostMallocDefault);
  if (e == hipSuccess) e = hipHostMalloc((void **)&h->results_pinned, rows * sizeof(tabby_row_result), hipHostMallocDefault);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    tabby_sampler_destroy(h);
    return hip_fail(e, "tabby_sampler_create");
  }
  *out = h;
  return TABBY_OK;
}

int tabby_sampler_destroy(tabby_sampler *h) {
  if (!h) return TABBY_OK;
  (void)hipSetDevice(h->device);
  (void)hipDeviceSynchronize();
  if (h->ws_base) (void)hipFree(h->ws_base);
  if (h->head_base) (void)hipFree(h->head_base);
  if (h->topk_ids_dev) (void)hipFree(h->topk_ids_dev);
  if (h->topk_logits_dev) (void)hipFree(h->topk_logits_dev);
  if (h->params_pinned) (void)hipHostFree(h->params_pinned);
  if (h->results_pinned) (void)hipHostFree(h->results_pinned);
  delete h;
  return TABBY_OK;
}

int tabby_sampler_sample_device(tabby_sampler *h, const void *logits_dev, int32_t dtype,
                                int32_t rows, int32_t vocab, const tabby_row_params *params_dev,
                                tabby_row_result *results_dev, int32_t *topk_ids_dev,
                                float *topk_logits_dev, int32_t topk_cap, uint32_t flags,
                                void *stream) {
  int rc = check_common(h, logits_dev, dtype, rows, vocab, topk_cap);
  if (rc) return rc;
  if (!params_dev || !results_dev) return fail(TABBY_EINVAL, "params and results pointers must be non-null");
  if (topk_cap > 0 && (!topk_ids_dev || !topk_logits_dev))
    return fail(TABBY_EINVAL, "topk_cap > 0 needs both top-k output pointers");
  if ((flags & TABBY_FLAG_FULL_VOCAB) && topk_cap > h->k_max)
    return fail(TABBY_EINVAL, "topk_cap must be <= k_max (" + std::to_string(h->k_max) +
                                  ") when whole-vocabulary rows are sampled, got " + std::to_string(topk_cap));
  if (flags & TABBY_FLAG_FULL_VOCAB) {
    // Head buffers for whole-vocabulary rows: four arrays of vocab_max 8-byte entries per
    // row, allocated on first use and grown to the largest batch seen.
    if ((size_t)rows > h->head_rows_cap) {
      HIP_TRY(hipSetDevice(h->device));
      if (h->head_base) {
        HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
        HIP_TRY(hipFree(h->head_base));
        h->head_base = nullptr;
        h->head_rows_cap = 0;
      }
      const size_t per = (size_t)rows * (size_t)h->vocab_max;
      const int plan_stride = plan_slots(h->vocab_max) + 2;
      const size_t plan_bytes = ((size_t)rows * plan_stride * 4 + 255) & ~(size_t)255;
      const size_t part_bytes = ((size_t)rows * (plan_stride - 2) * 16 + 255) & ~(size_t)255;
      const int acc_stride = (h->vocab_max + kHeadSlice - 1) / kHeadSlice;
      const size_t acc_bytes = (size_t)rows * acc_stride * 24;
      HIP_TRY(hipMalloc(&h->head_base, per * 32 + plan_bytes + part_bytes + acc_bytes + (size_t)rows * acc_stride * 4));
      char *b = (char *)h->head_base;
      h->ws.head_plan = (uint32_t *)(b + per * 32);
      h->ws.head_part = (double *)(b + per * 32 + plan_bytes);
      h->ws.head_acc = (double *)(b + per * 32 + plan_bytes + part_bytes);
      h->ws.head_slice_count = (uint32_t *)(b + per * 32 + plan_bytes + part_bytes + acc_bytes);
      h->ws.plan_stride = plan_stride;
      h->ws.acc_stride = acc_stride;
      h->ws.head = (uint64_t *)b;
      h->ws.head_sorted = (uint64_t *)(b + per * 8);
      h->ws.head_s = (double *)(b + per * 16);
      h->ws.head_c = (double *)(b + per * 24);
      h->ws.head_stride = h->vocab_max;
      h->head_rows_cap = (size_t)rows;
    }
  }

  Launch L;
  const Plan p = plan_launch(rows, vocab, dtype, logits_dev, h->k_max, topk_cap, h->cus,
                             (flags & TABBY_FLAG_FULL_VOCAB) != 0, L);
  L.params = params_dev;
  L.results = results_dev;
  L.topk_ids = topk_ids_dev;
  L.topk_logits = topk_logits_dev;
  HIP_TRY(hipSetDevice(h->device));
  HIP_TRY(dispatch(dtype, p, L, h->ws, h->cus, (hipStream_t)stream));
  return TABBY_OK;
}

int tabby_sampler_sample_lmhead_q4_device(tabby_sampler *h, const uint32_t *packed_dev,
                                          const uint16_t *packed_scales_dev, const float *bias_dev,
                                          const float *hidden_dev, int32_t rows, int32_t vocab, int32_t hidden,
                                          int32_t block_size, const tabby_row_params *params_dev,
                                          tabby_row_result *results_dev, void *stream) {
  if (!h) return fail(TABBY_EINVAL, "sampler handle is null");
  if (!packed_dev || !packed_scales_dev || !hidden_dev || !params_dev || !results_dev)
    return fail(TABBY_EINVAL, "null pointer");
  int rc = check_q4_shape(vocab, hidden, block_size);
  if (rc) return rc;
  if ((uintptr_t)packed_dev % 16 != 0) return fail(TABBY_EINVAL, "packed weights must be 16-byte aligned");
  if (rows < 1 || rows > std::min(h->rows_max, kLhMaxRows))
    return fail(TABBY_EINVAL, "rows must be between 1 and " + std::to_string(std::min(h->rows_max, kLhMaxRows)) +
                                  ", got " + std::to_string(rows));
  if (vocab > h->vocab_max)
    return fail(TABBY_EINVAL, "vocab must be at most " + std::to_string(h->vocab_max) + ", got " + std::to_string(vocab));
  // At most kMaxSplits slices of at most kLhMaxWaves waves of rows (lmhead_slice_kernel's
  // launch bound): 262,144 rows.
  if (vocab > kMaxSplits * kLhMaxWaves * kWaveSize)
    return fail(TABBY_ECAPACITY, "the fused lm_head takes at most " + std::to_string(kMaxSplits * kLhMaxWaves * kWaveSize) +
                                     " vocabulary rows, got " + std::to_string(vocab));
  // Slices of 64 * waves rows: one slice for vocabularies up to 1,024; otherwise enough
  // waves per slice (at least four) that at most 256 slices cover the vocabulary -- about one
  // per CU (238 slices of 640 rows for 151,936).
  const int waves = vocab <= kLhMaxWaves * kWaveSize
                        ? (vocab + kWaveSize - 1) / kWaveSize
                        : std::max(4, ((vocab + kMaxSplits - 1) / kMaxSplits + kWaveSize - 1) / kWaveSize);
  const int slice_len = waves * kWaveSize;
  const int slices = (vocab + slice_len - 1) / slice_len;
  if ((int64_t)slices * kLhKcap > h->ws.row_cand_stride)
    return fail(TABBY_ECAPACITY, "the handle's candidate region is too small for this vocab (create it with "
                                 "vocab_max >= 64)");
  Launch L{};
  L.logits = nullptr;  // no logits: top-k lists are not written on this path
  L.params = params_dev;
  L.results = results_dev;
  L.rows = rows;
  L.vocab = vocab;
  L.splits = slices;
  L.slice_len = slice_len;
  L.list_stride = kLhKcap;
  L.topk_cap = 0;
  L.k_max = h->k_max;
  L.kcap = kLhKcap;
  L.head_pass = 0;
  const Q4Matrix Q{packed_dev, packed_scales_dev, bias_dev, vocab, hidden, block_size};
  const hipStream_t s = (hipStream_t)stream;
  HIP_TRY(hipSetDevice(h->device));
  switch (rows) {
    case 1: hipLaunchKernelGGL(lmhead_slice_kernel<1>, dim3(slices), dim3(slice_len), 0, s, L, h->ws, Q, hidden_dev); break;
    case 2: hipLaunchKernelGGL(lmhead_slice_kernel<2>, dim3(slices), dim3(slice_len), 0, s, L, h->ws, Q, hidden_dev); break;
    case 3: hipLaunchKernelGGL(lmhead_slice_kernel<3>, dim3(slices), dim3(slice_len), 0, s, L, h->ws, Q, hidden_dev); break;
    case 4: hipLaunchKernelGGL(lmhead_slice_kernel<4>, dim3(slices), dim3(slice_len), 0, s, L, h->ws, Q, hidden_dev); break;
    case 5: hipLaunchKernelGGL(lmhead_slice_kernel<5>, dim3(slices), dim3(slice_len), 0, s, L, h->ws, Q, hidden_dev); break;
    case 6: hipLaunchKernelGGL(lmhead_slice_kernel<6>, dim3(slices), dim3(slice_len), 0, s, L, h->ws, Q, hidden_dev); break;
    case 7: hipLaunchKernelGGL(lmhead_slice_kernel<7>, dim3(slices), dim3(slice_len), 0, s, L, h->ws, Q, hidden_dev); break;
    default: hipLaunchKernelGGL(lmhead_slice_kernel<8>, dim3(slices), dim3(slice_len), 0, s, L, h->ws, Q, hidden_dev); break;
  }
  HIP_TRY(hipGetLastError());
  hipLaunchKernelGGL(lmhead_merge_kernel, dim3(rows), dim3(kBlock), 0, s, L, h->ws);
  HIP_TRY(hipGetLastError());
  return TABBY_OK;
}

int tabby_sampler_sample(tabby_sampler *h, const void *logits_dev, int32_t dtype, int32_t rows,
                         int32_t vocab, const tabby_row_params *params_host,
                         tabby_row_result *results_host, int32_t *topk_ids_host,
                         float *topk_logits_host, int32_t topk_cap, void *stream) {
  int rc = check_common(h, logits_dev, dtype, rows, vocab, topk_cap);
  if (rc) return rc;
  if (!params_host || !results_host) return fail(TABBY_EINVAL, "params and results pointers must be non-null");
  if (topk_cap > 0 && (!topk_ids_host || !topk_logits_host))
    return fail(TABBY_EINVAL, "topk_cap > 0 needs both top-k output pointers");
  uint32_t flags = 0;
  for (int32_t r = 0; r < rows; ++r) {
    const tabby_row_params &p = params_host[r];
    if (p.top_k < 0 || p.top_k > h->k_max)  // forward.ts:348-351
      return fail(TABBY_EINVAL, "topK must be between 0 and " + std::to_string(h->k_max) + ", got " + std::to_string(p.top_k));
    if (p.reserved != 0) return fail(TABBY_EINVAL, "tabby_row_params.reserved must be 0");
    if (!(p.uniform >= 0.0 && p.uniform < 1.0))
      return fail(TABBY_EINVAL, "uniform must be in [0, 1), row " + std::to_string(r));
    if (!(p.temperature < INFINITY))
      return fail(TABBY_EINVAL, "temperature must not be NaN or +Infinity, row " + std::to_string(r));
    if (p.top_k == 0 || p.top_k >= vocab) {
      if (vocab > (h->k_max <= kKcapSmall ? kKcapSmall : kKcapLarge)) flags |= TABBY_FLAG_FULL_VOCAB;
    }
  }
  hipStream_t s = (hipStream_t)stream;
  HIP_TRY(hipSetDevice(h->device));
  if (topk_cap > 0) {
    const size_t need = (size_t)rows * topk_cap;
    if (need > h->topk_elems_cap) {
      if (h->topk_ids_dev) (void)hipFree(h->topk_ids_dev);
      if (h->topk_logits_dev) (void)hipFree(h->topk_logits_dev);
      h->topk_ids_dev = nullptr;
      h->topk_logits_dev = nullptr;
      h->topk_elems_cap = 0;
      HIP_TRY(hipMalloc(&h->topk_ids_dev, need * sizeof(int32_t)));
      HIP_TRY(hipMalloc(&h->topk_logits_dev, need * sizeof(float)));
      h->topk_elems_cap = need;
    }
  }
  memcpy(h->params_pinned, params_host, (size_t)rows * sizeof(tabby_row_params));
  HIP_TRY(hipMemcpyAsync(h->params_dev, h->params_pinned, (size_t)rows * sizeof(tabby_row_params), hipMemcpyHostToDevice, s));
  rc = tabby_sampler_sample_device(h, logits_dev, dtype, rows, vocab, h->params_dev, h->results_dev,
                                   topk_cap > 0 ? h->topk_ids_dev : nullptr,
                                   topk_cap > 0 ? h->topk_logits_dev : nullptr, topk_cap, flags, stream);
  if (rc) return rc;
  HIP_TRY(hipMemcpyAsync(h->results_pinned, h->results_dev, (size_t)rows * sizeof(tabby_row_result), hipMemcpyDeviceToHost, s));
  if (topk_cap > 0) {
    HIP_TRY(hipMemcpyAsync(topk_ids_host, h->topk_ids_dev, (size_t)rows * topk_cap * sizeof(int32_t), hipMemcpyDeviceToHost, s));
    HIP_TRY(hipMemcpyAsync(topk_logits_host, h->topk_logits_dev, (size_t)rows * topk_cap * sizeof(float), hipMemcpyDeviceToHost, s));
  }
  HIP_TRY(hipStreamSynchronize(s));
  memcpy(results_host, h->results_pinned, (size_t)rows * sizeof(tabby_row_result));
  for (int32_t r = 0; r < rows; ++r) {
    const int st = results_host[r].status;
    if (st == TABBY_OK) continue;
    if (st == TABBY_EDOMAIN) return fail(st, "row " + std::to_string(r) + " is outside the contract (NaN, +inf, or all -inf logits)");
    if (st == TABBY_EEMPTY) return fail(st, "sampleFromTopK: empty candidate set");
    return fail(st, "row " + std::to_string(r) + " failed with status " + std::to_string(st));
  }
  return TABBY_OK;
}

int tabby_sampler_sample_device_noalloc(const void *logits_dev, int32_t dtype, int32_t rows, int32_t vocab,
                                        int32_t k_max, const tabby_row_params *params_dev,
                                        tabby_row_result *results_dev, int32_t *topk_ids_dev,
                                        float *topk_logits_dev, int32_t topk_cap, void *stream) {
  if (!logits_dev) return fail(TABBY_EINVAL, "logits pointer is null");
  if (dtype != TABBY_F32 && dtype != TABBY_F16) return fail(TABBY_EINVAL, "dtype must be TABBY_F32 or TABBY_F16");
  if (rows < 1 || rows > (1 << 20)) return fail(TABBY_EINVAL, "rows must be between 1 and 1048576, got " + std::to_string(rows));
  if (vocab < 1 || vocab > kMaxSplits * kChunk)
    return fail(TABBY_EINVAL, "vocab must be between 1 and " + std::to_string(kMaxSplits * kChunk) + ", got " + std::to_string(vocab));
  if (k_max < 1 || k_max > kWaveKcap)
    return fail(TABBY_ECAPACITY, "k_max must be between 1 and " + std::to_string(kWaveKcap) +
                                     " for the allocation-free entry, got " + std::to_string(k_max));
  if (topk_cap < 0) return fail(TABBY_EINVAL, "topk_cap must be >= 0");
  if (!params_dev || !results_dev) return fail(TABBY_EINVAL, "params and results pointers must be non-null");
  if (topk_cap > 0 && (!topk_ids_dev || !topk_logits_dev))
    return fail(TABBY_EINVAL, "topk_cap > 0 needs both top-k output pointers");
  int device = 0, cus = 0;
  void *base = nullptr;
  const int rc = scratch_of_current_device(device, base, cus);
  if (rc) return rc;

  Launch L;
  const Plan p = plan_launch(rows, vocab, dtype, logits_dev, k_max, topk_cap, cus, false, L);
  L.params = params_dev;
  L.results = results_dev;
  L.topk_ids = topk_ids_dev;
  L.topk_logits = topk_logits_dev;
  // Row statuses always; when rows are cut into slices or parts, their statistics and their
  // sorted lists, packed kWaveKcap entries apart (a list never holds more than the pool).
  // Everything is written before it is read within the call, so nothing needs clearing.
  Workspace W{};
  size_t off = 0;
  auto carve = [&](size_t bytes) {
    const size_t at = off;
    off += (bytes + 255) & ~(size_t)255;
    return (char *)base + at;
  };
  W.row_state = (RowState *)carve((size_t)rows * sizeof(RowState));
  L.list_stride = kWaveKcap;
  if (L.parts != 1) {
    W.stats = (SliceStat *)carve((size_t)rows * kMaxSplits * sizeof(SliceStat));
    W.row_cand_stride = (int64_t)L.splits * kWaveKcap;
    W.cands = (uint64_t *)carve((size_t)rows * (size_t)W.row_cand_stride * sizeof(uint64_t));
  }
  if (off > kNoAllocScratchBytes)
    return fail(TABBY_ECAPACITY, std::to_string(rows) + " rows of " + std::to_string(vocab) + " need " +
                                     std::to_string(off) + " bytes of scratch; the allocation-free entry has " +
                                     std::to_string(kNoAllocScratchBytes));
  HIP_TRY(dispatch(dtype, p, L, W, cus, (hipStream_t)stream));
  return TABBY_OK;
}

int tabby_debug_seq_sum(const double *terms_dev, int32_t n, double stop_at, double *prefix_dev,
                        int32_t *count_dev, int32_t wide, void *stream) {
  if (!terms_dev || !prefix_dev || !count_dev) return fail(TABBY_EINVAL, "null pointer");
  if (n < 1) return fail(TABBY_EINVAL, "n must be >= 1");
  if (wide == 4 && n > kWaveSize) return fail(TABBY_EINVAL, "the register form takes at most 64 terms");
  if (wide == 2)
    hipLaunchKernelGGL(seq_sum_block_kernel<kWaves>, dim3(1), dim3(kWaves * kWaveSize), 0, (hipStream_t)stream,
                       terms_dev, n, stop_at, prefix_dev, count_dev);
  else if (wide == 3)
    hipLaunchKernelGGL(seq_sum_block_kernel<kFinishThreads / kWaveSize>, dim3(1), dim3(kFinishThreads), 0,
                       (hipStream_t)stream, terms_dev, n, stop_at, prefix_dev, count_dev);
  else
    hipLaunchKernelGGL(seq_sum_kernel, dim3(1), dim3(kWaveSize), 0, (hipStream_t)stream, terms_dev, n,
                       stop_at, prefix_dev, count_dev, wide);
  HIP_TRY(hipGetLastError());
  return TABBY_OK;
}

int tabby_debug_first_above(const double *c_dev, int32_t n, const double *targets_dev, int32_t m,
                            int32_t *out_dev, void *stream) {
  if (!c_dev || !targets_dev || !out_dev) return fail(TABBY_EINVAL, "null pointer");
  if (n < 1 || m < 1 || m > (1 << 24)) return fail(TABBY_EINVAL, "n must be >= 1 and m in [1, 2^24]");
  hipLaunchKernelGGL(first_above_kernel, dim3((unsigned)m), dim3(kWaveSize), 0, (hipStream_t)stream, c_dev, n,
                     targets_dev, out_dev);
  HIP_TRY(hipGetLastError());
  return TABBY_OK;
}

int tabby_debug_exp(const double *x_dev, double *y_dev, int64_t n, void *stream) {
  if (n < 0 || (n > 0 && (!x_dev || !y_dev))) return fail(TABBY_EINVAL, "bad arguments");
  if (n == 0) return TABBY_OK;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(exp_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, x_dev, y_dev, n);
  HIP_TRY(hipGetLastError());
  return TABBY_OK;
}

}  // extern "C"
