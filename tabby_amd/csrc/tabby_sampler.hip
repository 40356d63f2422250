// MI355X (gfx950) token sampler: kernels and the C ABI declared in include/tabby_sampler.h.
//
// The reference (xOAviOx/tabby) computes, for one row, max and sum-exp with two two-stage
// tree reductions (src/shaders/reduce_max.wgsl, reduce_sumexp.wgsl) and the top-k with k
// rounds of a full argmax pass plus a single-workgroup select-and-mask
// (src/shaders/topk_partial.wgsl, topk_select.wgsl), orchestrated by encodeSampling
// (src/engine/forward.ts:522-601); the f64 tail runs on the CPU (src/engine/sampler.ts:147-212).
//
// Here one launch samples a whole batch:
//   * grid = rows x splits; each 256-lane workgroup owns one slice of one row and reads it
//     from HBM exactly once, 16 bytes per lane per load, into registers;
//   * from registers it computes the slice max, the slice sum of exp(x - max) (f32 terms,
//     f64 accumulation), and the exact top-k of the slice by radix select on 64-bit
//     (value key, ~index) composites -- the lower index wins ties, as in sampler.ts:28;
//   * the last workgroup of a row to finish (an atomic arrival counter, reset by that same
//     workgroup) merges the slices: max, sum-exp, a radix select over the slices'
//     candidates, an LDS bitonic sort, and then sampleFromTopK's f64 tail in the reference's
//     exact order of operations (sequential sums; V8's exp via the fdlibm method).
// Rows whose pool is the whole vocabulary (top_k = 0) are finished by a second kernel that
// re-reads the row's head (see head_kernel).

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>

#include "block_ops.h"
#include "device_math.h"
#include "tabby_sampler.h"

namespace tabby {

constexpr float kLog2e = 1.44269504088896340736f;
constexpr int kMaxSplits = kBlock;  // one merge lane per slice
constexpr int kSliceElemsSmall = 16;
constexpr int kSliceElemsLarge = 64;
constexpr int kMinSliceLen = kSliceElemsSmall * kBlock;
constexpr int kMaxSliceLen = kSliceElemsLarge * kBlock;
constexpr int kKcapSmall = 256;
constexpr int kKcapLarge = 1024;

struct SliceStat {
  float max;      // slice max (f32, exact)
  uint32_t count; // candidates written
  double sum;     // sum over the slice of exp(x - max)
};

// Per-row hand-over from the sampling kernel to the head kernel (whole-vocabulary rows).
struct RowState {
  float max;
  uint32_t head_key;  // elements with key >= head_key form the row's head
  double sum_exp;
  int32_t status;
  uint32_t pad;
};

struct Workspace {
  uint32_t *arrivals;       // [rows_cap] arrival counters of the sampling kernel
  uint32_t *head_arrivals;  // [rows_cap] arrival counters of the head kernel
  uint32_t *head_count;     // [rows_cap] head sizes
  SliceStat *stats;         // [rows_cap * kMaxSplits]
  uint64_t *cands;          // [rows_cap * kMaxSplits * cand_stride]
  RowState *row_state;      // [rows_cap]
  uint64_t *head;           // [head_rows * head_stride] (whole-vocabulary rows only)
  uint64_t *head_sorted;    // [head_rows * head_stride]
  double *head_exact;       // [head_rows * head_stride]
  double *head_w;           // [head_rows * head_stride]
  int32_t cand_stride;
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
  int32_t head_pass; // 1 when head_kernel runs after this launch
};

// ---------------------------------------------------------------------------------------
// Loads: VEC consecutive elements (16 bytes for the vector forms) widened to f32. f16
// widening is exact (tests/support.ts:61-74 states the same property for its reference).
// ---------------------------------------------------------------------------------------
template <typename In, int VEC>
struct Loader;

template <>
struct Loader<float, 4> {
  __device__ static void load(const float *p, float (&v)[4]) {
    const float4 f = *reinterpret_cast<const float4 *>(p);
    v[0] = f.x;
    v[1] = f.y;
    v[2] = f.z;
    v[3] = f.w;
  }
};

template <>
struct Loader<float, 1> {
  __device__ static void load(const float *p, float (&v)[1]) { v[0] = *p; }
};

__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

template <>
struct Loader<uint16_t, 8> {
  __device__ static void load(const uint16_t *p, float (&v)[8]) {
    const uint4 u = *reinterpret_cast<const uint4 *>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = half_bits_to_float(w[i] & 0xffffu);
      v[2 * i + 1] = half_bits_to_float(w[i] >> 16);
    }
  }
};

template <>
struct Loader<uint16_t, 1> {
  __device__ static void load(const uint16_t *p, float (&v)[1]) { v[0] = half_bits_to_float(*p); }
};

__device__ __forceinline__ float load_one(const float *p) { return *p; }
__device__ __forceinline__ float load_one(const uint16_t *p) { return half_bits_to_float(*p); }

__device__ __forceinline__ int32_t effective_k(const tabby_row_params &p, int vocab) {
  return (p.top_k <= 0 || p.top_k >= vocab) ? vocab : p.top_k;
}

__device__ __forceinline__ bool params_valid(const tabby_row_params &p, int k_max) {
  return p.top_k >= 0 && p.top_k <= k_max && p.reserved == 0 && !(p.uniform < 0.0) &&
         !(p.uniform >= 1.0) && p.uniform == p.uniform;
}

// ---------------------------------------------------------------------------------------
// Slice stage, shared by both kernels: load ELEMS elements per lane, return them as keys.
// ---------------------------------------------------------------------------------------
template <typename In, int VEC, int ELEMS>
__device__ __forceinline__ void load_slice(const In *src, int n, float (&x)[ELEMS]) {
  constexpr int ITEMS = ELEMS / VEC;
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const int le = (j * kBlock + (int)threadIdx.x) * VEC;
    const bool valid = le < n;
    // Lanes past the end read the slice's last vector (always in bounds) and discard it.
    float v[VEC];
    Loader<In, VEC>::load(src + (valid ? le : n - VEC), v);
#pragma unroll
    for (int c = 0; c < VEC; ++c) x[j * VEC + c] = valid ? v[c] : -INFINITY;
  }
}

template <int VEC>
__device__ __forceinline__ uint32_t elem_index(int begin, int e) {
  // Element e of this lane's registers sits at row index begin + (j*kBlock + lane)*VEC + c.
  const int j = e / VEC, c = e % VEC;
  return (uint32_t)(begin + (j * kBlock + (int)threadIdx.x) * VEC + c);
}

// ---------------------------------------------------------------------------------------
// LDS layout of the sampling kernel. The histogram and the tail arrays are never live at
// the same time, so they share storage.
// ---------------------------------------------------------------------------------------
template <int KCAP>
struct SampleSmem {
  BlockScratch bs;
  int32_t is_last;
  float row_max;
  double sum_exp;
  double pool_mass;
  double scaled_total;
  double slice_term[kMaxSplits];
  uint64_t sorted[KCAP];
  union {
    uint32_t hist[kBins];
    struct {
      double exact[KCAP];
      double w[KCAP];
    } tail;
  } u;
};

// sampleFromTopK (src/engine/sampler.ts:147-212) over the `count` sorted candidates in
// sm.sorted, f64 throughout, with the reference's order of operations: the per-element
// terms are independent and computed by all lanes; every sum is a sequential left-to-right
// f64 sum on lane 0. The running sums of the draw (sampler.ts:195-203) are the same
// numbers as the top-p cumulative sums (sampler.ts:178-185), and `total` (:191-192) is the
// last of them, so lane 0 computes that sequence once and keeps it.
template <int KCAP, typename In>
__device__ void finish_row(SampleSmem<KCAP> &sm, const Launch &L, int row, const In *row_src,
                           int count, float max_logit, double sum_exp,
                           const tabby_row_params &P) {
  const double T = P.temperature;
  for (int i = threadIdx.x; i < count; i += kBlock) {
    const float l = value_of(composite_key(sm.sorted[i]));
    const double d = (double)l - (double)max_logit;
    sm.u.tail.exact[i] = fdlibm_exp(d) / sum_exp;
    sm.u.tail.w[i] = T > 0.0 ? fdlibm_exp(d / T) : 0.0;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double pool = 0.0, scaled = 0.0;
    for (int i = 0; i < count; ++i) {
      pool += sm.u.tail.exact[i];
      scaled += sm.u.tail.w[i];
    }
    sm.pool_mass = pool;
    sm.scaled_total = scaled;
  }
  __syncthreads();
  const double pool_mass = sm.pool_mass;
  const double scaled_total = sm.scaled_total;
  if (T > 0.0) {
    for (int i = threadIdx.x; i < count; i += kBlock) sm.u.tail.w[i] = sm.u.tail.w[i] / scaled_total;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    tabby_row_result r;
    r.max_logit = max_logit;
    r.sum_exp = sum_exp;
    r.pool_mass = pool_mass;
    r.status = TABBY_OK;
    r.topk_count = min(count, L.topk_cap);
    if (T <= 0.0) {
      r.id = (int32_t)composite_index(sm.sorted[0]);
      r.probability = sm.u.tail.exact[0];
      r.considered = 1;
      r.pool_exhausted = 0;
    } else {
      double *c = sm.u.tail.w;  // becomes the running sums in place
      const double top_p = P.top_p;
      int cut = count;
      double acc = 0.0;
      for (int i = 0; i < count; ++i) {
        acc += c[i];
        c[i] = acc;
        if (top_p < 1.0 && acc >= top_p) {
          cut = i + 1;
          break;
        }
      }
      const double target = P.uniform * c[cut - 1];
      int chosen = cut - 1;
      for (int i = 0; i < cut; ++i) {
        if (target < c[i]) {
          chosen = i;
          break;
        }
      }
      r.id = (int32_t)composite_index(sm.sorted[chosen]);
      r.probability = sm.u.tail.exact[chosen];
      r.considered = (uint32_t)cut;
      r.pool_exhausted = (top_p < 1.0 && pool_mass < top_p) ? 1 : 0;
    }
    L.results[row] = r;
  }
  if (L.topk_cap > 0) {
    const int m = min(count, L.topk_cap);
    for (int i = threadIdx.x; i < m; i += kBlock) {
      const uint32_t idx = composite_index(sm.sorted[i]);
      L.topk_ids[(size_t)row * L.topk_cap + i] = (int32_t)idx;
      L.topk_logits[(size_t)row * L.topk_cap + i] = load_one(row_src + min(idx, (uint32_t)(L.vocab - 1)));
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
// The sampling kernel.
// ---------------------------------------------------------------------------------------
template <typename In, int VEC, int ELEMS, int KCAP>
__global__ __launch_bounds__(kBlock) void sample_kernel(Launch L, Workspace W) {
  __shared__ SampleSmem<KCAP> sm;

  const int splits = L.splits;
  const int row = (int)blockIdx.x / splits;
  const int slice = (int)blockIdx.x - row * splits;
  const int V = L.vocab;
  const int begin = slice * L.slice_len;
  const int n = min(L.slice_len, V - begin);
  const tabby_row_params P = L.params[row];
  const bool valid_params = params_valid(P, L.k_max);
  const int keff = effective_k(P, V);
  const bool finite = valid_params && keff <= L.kcap;
  const int kk = finite ? min(keff, n) : 0;
  const In *row_src = reinterpret_cast<const In *>(L.logits) + (size_t)row * V;

  // 1. One pass over HBM into registers.
  float x[ELEMS];
  load_slice<In, VEC, ELEMS>(row_src + begin, n, x);

  // 2. Lane max and lane sum of exp(x - lane max); then the slice's.
  float mt = x[0];
#pragma unroll
  for (int e = 1; e < ELEMS; ++e) mt = fmaxf(mt, x[e]);
  float st = 0.0f;
  if (mt != -INFINITY) {
    const float ml = mt * kLog2e;
#pragma unroll
    for (int e = 0; e < ELEMS; ++e) st += __builtin_amdgcn_exp2f(fmaf(x[e], kLog2e, -ml));
  }
  const float ms = block_max(mt, sm.bs);
  const double term = (mt == -INFINITY) ? 0.0
                                        : (double)st * (double)__builtin_amdgcn_exp2f((mt - ms) * kLog2e);
  const double ss = block_sum(term, sm.bs);

  // 3. Keys in place of the values.
  uint32_t key[ELEMS];
#pragma unroll
  for (int e = 0; e < ELEMS; ++e) key[e] = key_of(x[e]);

  // 4. This slice's top-kk composites, unordered, into the row's candidate area.
  uint64_t *out = W.cands + ((size_t)row * kMaxSplits + slice) * W.cand_stride;
  if (kk > 0) {
    if (kk >= n) {
#pragma unroll
      for (int e = 0; e < ELEMS; ++e) {
        const uint32_t idx = elem_index<VEC>(begin, e);
        const int local = (int)idx - begin;
        if (local < n) out[local] = composite(key[e], idx);
      }
    } else {
      auto regs = [&](auto &&f) {
#pragma unroll
        for (int e = 0; e < ELEMS; ++e) f(composite(key[e], elem_index<VEC>(begin, e)));
      };
      const SelectResult r = radix_select(regs, (uint32_t)kk, sm.u.hist, sm.bs);
      if (threadIdx.x == 0) sm.bs.slot = 0;
      __syncthreads();
#pragma unroll
      for (int e = 0; e < ELEMS; ++e) {
        const uint64_t v = composite(key[e], elem_index<VEC>(begin, e));
        if (selected(v, r)) {
          const uint32_t at = atomicAdd(&sm.bs.slot, 1u);
          if (at < (uint32_t)kk) out[at] = v;  // exactly kk are selected; the bound is a guard
        }
      }
    }
  }
  if (threadIdx.x == 0) {
    SliceStat st_out;
    st_out.max = ms;
    st_out.count = (uint32_t)kk;
    st_out.sum = ss;
    W.stats[(size_t)row * kMaxSplits + slice] = st_out;
  }

  // 5. Arrival: the last workgroup of the row merges.
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = atomicAdd(&W.arrivals[row], 1u);
    sm.is_last = prev == (uint32_t)(splits - 1);
  }
  __syncthreads();
  if (!sm.is_last) return;
  __threadfence();

  // 6. Row max and sum-exp from the slice statistics, in slice order.
  const SliceStat *stats = W.stats + (size_t)row * kMaxSplits;
  float M = -INFINITY;
  for (int s = 0; s < splits; ++s) M = fmaxf(M, stats[s].max);
  if ((int)threadIdx.x < splits) {
    const SliceStat st_s = stats[threadIdx.x];
    sm.slice_term[threadIdx.x] =
        st_s.max == -INFINITY ? 0.0 : st_s.sum * fdlibm_exp((double)st_s.max - (double)M);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double S = 0.0;
    for (int s = 0; s < splits; ++s) S += sm.slice_term[s];
    sm.row_max = M;
    sm.sum_exp = S;
  }
  __syncthreads();
  const float row_max = sm.row_max;
  const double sum_exp = sm.sum_exp;
  const bool in_domain = (row_max > -INFINITY) && (row_max < INFINITY) && (sum_exp > 0.0) &&
                         (sum_exp < INFINITY);
  if (threadIdx.x == 0) W.arrivals[row] = 0u;  // ready for the next launch

  if (!valid_params || !in_domain) {
    if (threadIdx.x == 0) {
      write_status(L, row, !valid_params ? TABBY_EINVAL : TABBY_EDOMAIN, row_max, sum_exp);
      if (!finite) W.row_state[row].status = !valid_params ? TABBY_EINVAL : TABBY_EDOMAIN;
    }
    return;
  }
  if (!finite && !L.head_pass) {
    if (threadIdx.x == 0) write_status(L, row, TABBY_EINVAL, row_max, sum_exp);
    return;
  }
  if (!finite) {
    // Whole-vocabulary row: hand max / sum-exp / the head threshold to head_kernel.
    if (threadIdx.x == 0) {
      RowState rs;
      rs.max = row_max;
      rs.sum_exp = sum_exp;
      rs.status = TABBY_OK;
      rs.pad = 0;
      const uint32_t top = key_of(row_max);
      if (P.temperature <= 0.0) {
        rs.head_key = top;  // greedy needs only the row's maxima
      } else {
        // Smallest key whose scaled logit (l - max)/T in f64 is >= -40. Anything below has
        // exp(.) < 2^-54 and can change neither the scaled total nor a running sum, both of
        // which are >= their first term when it is added (see finish_head).
        uint32_t lo = kNegInfKey, hi = top;
        while (hi - lo > 1u) {
          const uint32_t mid = lo + (hi - lo) / 2u;
          const double q = ((double)value_of(mid) - (double)row_max) / P.temperature;
          if (q >= -40.0) hi = mid; else lo = mid;
        }
        rs.head_key = hi;
      }
      W.row_state[row] = rs;
      W.head_count[row] = 0u;
    }
    return;
  }

  // 7. Merge the slices' candidates: exact top-keff by radix select, then sort.
  auto cands = [&](auto &&f) {
    for (int s = 0; s < splits; ++s) {
      const int ns = min(L.slice_len, V - s * L.slice_len);
      const int cs = min(keff, ns);
      const uint64_t *src = W.cands + ((size_t)row * kMaxSplits + s) * W.cand_stride;
      for (int i = threadIdx.x; i < cs; i += kBlock) f(src[i]);
    }
  };
  int total_cands = 0;
  for (int s = 0; s < splits; ++s) total_cands += min(keff, min(L.slice_len, V - s * L.slice_len));
  if (threadIdx.x == 0) sm.bs.slot = 0;
  __syncthreads();
  if (total_cands > keff) {
    const SelectResult r = radix_select(cands, (uint32_t)keff, sm.u.hist, sm.bs);
    cands([&](uint64_t v) {
      if (selected(v, r)) {
        const uint32_t at = atomicAdd(&sm.bs.slot, 1u);
        if (at < (uint32_t)keff) sm.sorted[at] = v;
      }
    });
  } else {
    cands([&](uint64_t v) {
      const uint32_t at = atomicAdd(&sm.bs.slot, 1u);
      if (at < (uint32_t)keff) sm.sorted[at] = v;
    });
  }
  const int npow = next_pow2(keff);
  for (int i = keff + (int)threadIdx.x; i < npow; i += kBlock) sm.sorted[i] = 0ull;
  __syncthreads();
  bitonic_sort_desc(sm.sorted, npow);

  // 8. sampleFromTopK.
  finish_row<KCAP, In>(sm, L, row, row_src, keff, row_max, sum_exp, P);
}

// ---------------------------------------------------------------------------------------
// Diagnostic kernel: the device exp over an array.
// ---------------------------------------------------------------------------------------
__global__ void exp_kernel(const double *x, double *y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = fdlibm_exp(x[i]);
}

}  // namespace tabby

// =========================================================================================
// Host side.
// =========================================================================================
using namespace tabby;

struct tabby_sampler {
  int device = 0;
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

namespace {

thread_local std::string g_last_error;

int fail(int status, const std::string &msg) {
  g_last_error = msg;
  return status;
}

int hip_fail(hipError_t e, const char *what) {
  return fail(TABBY_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define HIP_TRY(expr)                                  \
  do {                                                 \
    hipError_t e_ = (expr);                            \
    if (e_ != hipSuccess) return hip_fail(e_, #expr);  \
  } while (0)

struct Plan {
  int elems;
  int slice_len;
  int splits;
  int vec;
};

// Large slices (64 elements per lane) when the batch alone fills the chip; small ones
// (16 per lane) for a few rows, to spread a row over more CUs.
Plan make_plan(int rows, int vocab, int dtype, const void *logits) {
  Plan p;
  const int large_splits = (vocab + kMaxSliceLen - 1) / kMaxSliceLen;
  p.elems = ((int64_t)rows * large_splits >= 512) ? kSliceElemsLarge : kSliceElemsSmall;
  p.slice_len = p.elems * kBlock;
  p.splits = (vocab + p.slice_len - 1) / p.slice_len;
  const int vec_elems = dtype == TABBY_F32 ? 4 : 8;
  const bool aligned = ((uintptr_t)logits % 16u) == 0 && vocab % vec_elems == 0;
  p.vec = aligned ? vec_elems : 1;
  return p;
}

template <typename In, int VEC, int ELEMS>
hipError_t launch_sample(const Launch &L, const Workspace &W, hipStream_t stream) {
  const dim3 grid((unsigned)(L.rows * L.splits));
  if (L.kcap <= kKcapSmall) {
    hipLaunchKernelGGL((sample_kernel<In, VEC, ELEMS, kKcapSmall>), grid, dim3(kBlock), 0, stream, L, W);
  } else {
    hipLaunchKernelGGL((sample_kernel<In, VEC, ELEMS, kKcapLarge>), grid, dim3(kBlock), 0, stream, L, W);
  }
  return hipGetLastError();
}

template <typename In, int VEC>
hipError_t dispatch_elems(const Plan &p, const Launch &L, const Workspace &W, hipStream_t s) {
  if (p.elems == kSliceElemsLarge) return launch_sample<In, VEC, kSliceElemsLarge>(L, W, s);
  return launch_sample<In, VEC, kSliceElemsSmall>(L, W, s);
}

hipError_t dispatch(int dtype, const Plan &p, const Launch &L, const Workspace &W, hipStream_t s) {
  if (dtype == TABBY_F32) {
    if (p.vec == 4) return dispatch_elems<float, 4>(p, L, W, s);
    return dispatch_elems<float, 1>(p, L, W, s);
  }
  if (p.vec == 8) return dispatch_elems<uint16_t, 8>(p, L, W, s);
  return dispatch_elems<uint16_t, 1>(p, L, W, s);
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

const char *tabby_last_error(void) { return g_last_error.c_str(); }

const char *tabby_version(void) { return "tabby_sampler 0.1.0 (gfx950)"; }

int tabby_sampler_create(int device, int32_t vocab_max, int32_t rows_max, int32_t k_max,
                         tabby_sampler **out) {
  if (!out) return fail(TABBY_EINVAL, "out pointer is null");
  *out = nullptr;
  if (vocab_max < 1 || vocab_max > kMaxSplits * kMinSliceLen)
    return fail(TABBY_EINVAL, "vocab_max must be between 1 and " + std::to_string(kMaxSplits * kMinSliceLen));
  if (rows_max < 1 || rows_max > (1 << 20)) return fail(TABBY_EINVAL, "rows_max must be between 1 and 1048576");
  if (k_max < 1 || k_max > kKcapLarge)
    return fail(TABBY_ECAPACITY, "k_max must be between 1 and " + std::to_string(kKcapLarge));
  HIP_TRY(hipSetDevice(device));

  tabby_sampler *h = new tabby_sampler();
  h->device = device;
  h->vocab_max = vocab_max;
  h->rows_max = rows_max;
  h->k_max = k_max;
  // A slice emits min(keff, n) candidates and keff can reach the kernel's pool capacity
  // (top_k >= vocab with vocab <= capacity), so the stride is the capacity, not k_max.
  h->ws.cand_stride = std::min(k_max <= kKcapSmall ? kKcapSmall : kKcapLarge, kMaxSliceLen);

  const size_t rows = (size_t)rows_max;
  size_t off = 0;
  auto carve = [&](size_t bytes) {
    const size_t at = off;
    off += (bytes + 255) & ~(size_t)255;
    return at;
  };
  const size_t o_arr = carve(rows * 4), o_harr = carve(rows * 4), o_hcnt = carve(rows * 4);
  const size_t o_stats = carve(rows * kMaxSplits * sizeof(SliceStat));
  const size_t o_cands = carve(rows * kMaxSplits * (size_t)h->ws.cand_stride * 8);
  const size_t o_rs = carve(rows * sizeof(RowState));
  const size_t o_par = carve(rows * sizeof(tabby_row_params));
  const size_t o_res = carve(rows * sizeof(tabby_row_result));
  hipError_t e = hipMalloc(&h->ws_base, off);
  if (e != hipSuccess) {
    delete h;
    return hip_fail(e, "hipMalloc(workspace)");
  }
  char *b = (char *)h->ws_base;
  h->ws.arrivals = (uint32_t *)(b + o_arr);
  h->ws.head_arrivals = (uint32_t *)(b + o_harr);
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
  if (flags & TABBY_FLAG_FULL_VOCAB)
    return fail(TABBY_ECAPACITY, "whole-vocabulary pools (top_k = 0) are not available in this build");

  const Plan p = make_plan(rows, vocab, dtype, logits_dev);
  Launch L;
  L.logits = logits_dev;
  L.params = params_dev;
  L.results = results_dev;
  L.topk_ids = topk_ids_dev;
  L.topk_logits = topk_logits_dev;
  L.rows = rows;
  L.vocab = vocab;
  L.splits = p.splits;
  L.slice_len = p.slice_len;
  L.topk_cap = topk_cap;
  L.k_max = h->k_max;
  L.kcap = h->k_max <= kKcapSmall ? kKcapSmall : kKcapLarge;
  L.head_pass = 0;
  HIP_TRY(hipSetDevice(h->device));
  HIP_TRY(dispatch(dtype, p, L, h->ws, (hipStream_t)stream));
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

int tabby_debug_exp(const double *x_dev, double *y_dev, int64_t n, void *stream) {
  if (n < 0 || (n > 0 && (!x_dev || !y_dev))) return fail(TABBY_EINVAL, "bad arguments");
  if (n == 0) return TABBY_OK;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(exp_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, x_dev, y_dev, n);
  HIP_TRY(hipGetLastError());
  return TABBY_OK;
}

}  // extern "C"
