// Row softmax of attention scores, bit for bit the reference's.
//
// The reference softmaxes each row of scores in place (src/shaders/softmax_rows.wgsl:1-55,
// one invocation per row; dispatched at src/engine/forward.ts:912-926) and checks it against
// softmaxRows (src/reference/cpu.ts:238-264), whose arithmetic is f32 throughout:
//   valid = causal_period ? causal_offset + (row % causal_period) + 1 : row_len
//   M     = Math.max over the row's first `valid` entries (a NaN makes it NaN)
//   e_i   = f32(Math.exp(f32(x_i - M)));  S = f32(S + e_i) left to right from 0
//   out_i = f32(e_i * f32(1 / S)) for i < valid, 0 for the masked rest.
// Here each row is one wave. x_i - M is one f32 subtraction (the reference rounds the f64
// difference of two f32 values to f32, which is the same number); Math.exp rounded to f32 is
// exp_to_f32 (a fast f64 exp, V8's fdlibm method where the f32 rounding is close); 1 / S is an
// f64 division rounded
// to f32, as JS evaluates it; e_i * inv is one f32 multiplication (the f64 product of two f32
// values is exact, so JS's rounding of it to f32 is the f32 product).
//
// The sequential f32 sum is computed by the whole wave without changing a bit (the f32 form
// of the method in seqsum.h): while the running sum P = m * u lies in one binade, with ulp
// u = 2^(E-23) and integer m < 2^24, fl(P + t) = (m + rint(t / u)) * u exactly, with an exact
// half-ulp tie going to the even result (a parity automaton scanned over the lanes); so the
// partial sums are m plus an integer prefix sum, and only a term that takes m to 2^24 or
// beyond (the sum leaves the binade) is added on its own, after which the scan resumes.
// A row of n terms has about log2(n) such events.
//
// Rows of up to 4,096 entries (16-byte aligned) are read once into registers and written once:
// HBM traffic 2 * row_len * 4 bytes. Longer or unaligned rows take three passes (max; exp,
// sum and the exps written to `out`; the scaling), as the reference's kernel does.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "abi_internal.h"
#include "device_math.h"
#include "seqsum.h"
#include "wave_ops.h"

namespace tabby {
namespace {

constexpr int kSmWaves = 4;  // rows per workgroup, one wave each
// Rows per workgroup of softmax_rows_block_kernel: one per wave. Measured on 14 x 512 causal
// rows of 512 (the prefill shape): 16 rows 17.8 us, 8 rows 15.5 us, 4 rows 13.1 us -- the
// batch is small for the chip, and smaller blocks overlap more of their loads, exps and sums.
constexpr int kBlockRows = 4;
constexpr int kBlockMinRows = 256;  // batches with fewer rows keep one wave per row
constexpr double kTwo24 = 16777216.0;
constexpr double kTwo25 = 33554432.0;

typedef float sm_f32x4 __attribute__((ext_vector_type(4)));

// Parity (0/1) of an integer-valued double; values that large only occur at event
// positions, whose parity is never used.
__device__ __forceinline__ uint32_t parity_of(double integral) {
  return (uint32_t)(int64_t)fmin(integral, 1.0e15) & 1u;
}

// P + t_0 + t_1 + ... in f32, one rounding per addition, left to right, over one step of the
// row: lane l holds the step's terms l*V .. l*V + V - 1 in t[]. P is wave-uniform; terms are
// >= 0 and finite (a NaN term makes the sum NaN, as it would sequentially). Returns the sum.
template <int V>
__device__ float seq_sum_f32_step(float P, const float (&t)[V]) {
  const int lane = wave_lane();
  bool nan = false;
#pragma unroll
  for (int j = 0; j < V; ++j) nan |= t[j] != t[j];
  if (P != P || __ballot(nan)) return __builtin_nanf("");
  int start = 0;  // positions of the step below this one are in P already
  while (true) {
    // P = m * 2^sh with m an integer below 2^24 (sh = -149 for zero and subnormal P).
    const int ef = (int)(__float_as_uint(P) >> 23);
    const int sh = (ef == 0 ? 1 : ef) - 150;
    const double m = __builtin_ldexp((double)P, -sh);
    double inc[V], fl[V];
    bool tie[V];
    bool any_tie = false;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const bool active = lane * V + j >= start;
      const double x = active ? __builtin_ldexp((double)t[j], -sh) : 0.0;  // t / u, exact
      fl[j] = __builtin_floor(x);
      tie[j] = x - fl[j] == 0.5;
      inc[j] = tie[j] ? fl[j] : __builtin_rint(x);
      any_tie |= tie[j];
    }
    if (__ballot(any_tie)) {
      // A tie adds fl or fl + 1, whichever leaves m even: the parity of m before every term,
      // from the maps x -> (x & k) ^ c (a non-tie XORs its increment's parity, a tie resets
      // to 0) composed over the lanes below and this lane's earlier terms.
      uint32_t f[V];
      uint32_t lane_map = kParityId;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        f[j] = tie[j] ? 0u : (1u | (parity_of(inc[j]) << 1));
        lane_map = parity_then(lane_map, f[j]);
      }
      uint32_t p = parity_apply(parity_exclusive_scan(lane_map), parity_of(m));
#pragma unroll
      for (int j = 0; j < V; ++j) {
        if (tie[j]) inc[j] = fl[j] + (double)((p + parity_of(fl[j])) & 1u);
        p = parity_apply(f[j], p);
      }
    }
    // An increment of 2^24 or more is an event whatever its size: capped at 2^25, every
    // prefix below stays an exact integer (64 * V * 2^25 < 2^53).
#pragma unroll
    for (int j = 0; j < V; ++j) inc[j] = fmin(inc[j], kTwo25);
    double c[V];
    c[0] = inc[0];
#pragma unroll
    for (int j = 1; j < V; ++j) c[j] = c[j - 1] + inc[j];
    const double below = wave_inclusive_scan(c[V - 1]) - c[V - 1];
    int first = V;
#pragma unroll
    for (int j = V - 1; j >= 0; --j)
      if (m + (below + c[j]) >= kTwo24) first = j;
    const uint64_t ev = __ballot(first < V);
    if (!ev) return (float)__builtin_ldexp(m + lane_f64(below + c[V - 1], kWaveSize - 1), sh);
    // The first event: every term before it is exact in the integer sum; it is added alone.
    const int L = __ffsll((unsigned long long)ev) - 1;
    const int j = __builtin_amdgcn_readlane(first, L);
    double before = below;
    float tj = t[0];
#pragma unroll
    for (int i = 0; i < V; ++i)
      if (i == j) {
        before = i == 0 ? below : below + c[i > 0 ? i - 1 : 0];
        tj = t[i];
      }
    const float p_before = (float)__builtin_ldexp(m + lane_f64(before, L), sh);
    P = p_before + __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(tj), L));
    start = L * V + j + 1;
    if (start >= kWaveSize * V) return P;
  }
}

// fround(Math.exp(d)), d = x_i - M <= 0 or NaN (exp_to_f32).
__device__ __forceinline__ float exp_f32_of(float d) { return exp_to_f32(d); }

struct RowDims {
  int n_rows;
  int row_len;
  int causal_period;
  int causal_offset;
};

__device__ __forceinline__ int valid_of(const RowDims &d, int row) {
  return d.causal_period != 0 ? d.causal_offset + (row % d.causal_period) + 1 : d.row_len;
}

// Rows of at most NSTEP * 256 entries, 16-byte aligned: one read into registers, one write.
template <int NSTEP>
__global__ __launch_bounds__(kSmWaves *kWaveSize) void softmax_rows_reg_kernel(const float *x, float *out, RowDims d) {
  const int row = (int)blockIdx.x * kSmWaves + (int)threadIdx.x / kWaveSize;
  if (row >= d.n_rows) return;
  const int lane = wave_lane();
  const int valid = valid_of(d, row);
  const float *src = x + (size_t)row * d.row_len;
  float *dst = out + (size_t)row * d.row_len;
  float v[NSTEP][4];
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) {
    const int i = s * 256 + lane * 4;
    if (i < d.row_len) {
      const sm_f32x4 q = __builtin_nontemporal_load(reinterpret_cast<const sm_f32x4 *>(src + i));
      v[s][0] = q.x;
      v[s][1] = q.y;
      v[s][2] = q.z;
      v[s][3] = q.w;
    } else {
      v[s][0] = v[s][1] = v[s][2] = v[s][3] = -INFINITY;
    }
  }
  // Math.max: the largest valid entry, NaN if any valid entry is NaN.
  float mx = -INFINITY;
  bool nan = false;
#pragma unroll
  for (int s = 0; s < NSTEP; ++s)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (s * 256 + lane * 4 + e < valid) {
        mx = fmaxf(mx, v[s][e]);
        nan |= v[s][e] != v[s][e];
      }
  mx = wave_max(mx);
  if (__ballot(nan)) mx = __builtin_nanf("");
  float P = 0.0f;
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[s][e] = s * 256 + lane * 4 + e < valid ? exp_f32_of(v[s][e] - mx) : 0.0f;
    if (s * 256 < valid) P = seq_sum_f32_step<4>(P, v[s]);
  }
  const float inv = (float)(1.0 / (double)P);
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) {
    const int i = s * 256 + lane * 4;
    if (i < d.row_len) {
      sm_f32x4 q;
      q.x = i + 0 < valid ? v[s][0] * inv : 0.0f;
      q.y = i + 1 < valid ? v[s][1] * inv : 0.0f;
      q.z = i + 2 < valid ? v[s][2] * inv : 0.0f;
      q.w = i + 3 < valid ? v[s][3] * inv : 0.0f;
      __builtin_nontemporal_store(q, reinterpret_cast<sm_f32x4 *>(dst + i));
    }
  }
}

// Many short rows (row_len <= kBlockCols): BR rows per workgroup of four waves, one lane per
// row for the sum (BR a multiple of 4). The waves take the block's rows one at a time (coalesced loads into
// registers, the row max by DPP, the exps of their own entries) and leave the exps in LDS;
// then lane r of wave 0 adds row r's exps left to right -- the reference's own sequential f32
// sum, one row per lane -- and the waves scale the exps in LDS and write the rows out.
// HBM traffic 2 * row_len * 4 bytes per row. The sum is a chain of row_len dependent adds
// per lane, shared by BR rows: for many rows this beats the wave-wide exact scan, whose
// restart per binade crossing costs a whole step.
constexpr int kBlockCols = 512;

template <int BR>
__global__ __launch_bounds__(kSmWaves *kWaveSize) void softmax_rows_block_kernel(const float *x, float *out,
                                                                                 RowDims d) {
  // Row pitch: eight pad words keep each row's start 16-byte aligned (the sum reads 16 bytes
  // at a time), put rows r and r + 1 on different banks, and hold the sum's read-ahead of
  // eight entries past a full row.
  constexpr int kPitch = kBlockCols + 8;
  constexpr int kPer = kBlockCols / kWaveSize;
  constexpr int kRowsPerWave = BR / kSmWaves;
  __shared__ float tile[BR * kPitch];
  __shared__ float inv[BR];
  const int lane = wave_lane();
  const int wave = (int)threadIdx.x / kWaveSize;
  const int row0 = (int)blockIdx.x * BR;
  const int rows = min(BR, d.n_rows - row0);
  // Wave w takes rows w, w + 4, ...: every load of all of them is issued before any is used.
  float v[kRowsPerWave][kPer];
  int valid[kRowsPerWave];
#pragma unroll
  for (int j = 0; j < kRowsPerWave; ++j) {
    const int r = wave + j * kSmWaves;
    valid[j] = r < rows ? valid_of(d, row0 + r) : 0;
    const float *src = x + (size_t)(row0 + r) * d.row_len;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = k * kWaveSize + lane;
      v[j][k] = i < valid[j] ? __builtin_nontemporal_load(src + i) : -INFINITY;
    }
  }
#pragma unroll
  for (int j = 0; j < kRowsPerWave; ++j) {
    const int r = wave + j * kSmWaves;
    float mx = -INFINITY;
    bool nan = false;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      mx = fmaxf(mx, v[j][k]);
      nan |= v[j][k] != v[j][k];
    }
    mx = wave_max(mx);
    if (__ballot(nan)) mx = __builtin_nanf("");
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = k * kWaveSize + lane;
      if (i < valid[j]) tile[r * kPitch + i] = exp_f32_of(v[j][k] - mx);
    }
  }
  __syncthreads();
  if (wave == 0 && lane < rows) {
    // The row's exps left to right; the next eight are read while these eight are added.
    const int n = valid_of(d, row0 + lane);
    const sm_f32x4 *t4 = reinterpret_cast<const sm_f32x4 *>(tile + lane * kPitch);
    float sum = 0.0f;
    const int n8 = n / 8;
    sm_f32x4 a = t4[0], b = t4[1];
    for (int g = 0; g < n8; ++g) {
      const sm_f32x4 na = t4[2 * g + 2], nb = t4[2 * g + 3];  // at most the row's padding
      sum = sum + a.x;
      sum = sum + a.y;
      sum = sum + a.z;
      sum = sum + a.w;
      sum = sum + b.x;
      sum = sum + b.y;
      sum = sum + b.z;
      sum = sum + b.w;
      a = na;
      b = nb;
    }
    const float *t = tile + lane * kPitch;
    for (int i = n8 * 8; i < n; ++i) sum = sum + t[i];
    inv[lane] = (float)(1.0 / (double)sum);
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kRowsPerWave; ++j) {
    const int r = wave + j * kSmWaves;
    if (r >= rows) break;
    const float q = inv[r];
    float *dst = out + (size_t)(row0 + r) * d.row_len;
    for (int i = lane; i < d.row_len; i += kWaveSize)
      __builtin_nontemporal_store(i < valid[j] ? tile[r * kPitch + i] * q : 0.0f, dst + i);
  }
}

// Any row: three passes of one element per lane per step (64 entries), as the reference's
// kernel makes them -- max; exp, sum and e_i written to out; out_i = e_i * inv and the
// masked tail zeroed. In place (out == x) each lane rewrites only entries it has read.
__global__ __launch_bounds__(kSmWaves *kWaveSize) void softmax_rows_stream_kernel(const float *x, float *out,
                                                                                  RowDims d) {
  const int row = (int)blockIdx.x * kSmWaves + (int)threadIdx.x / kWaveSize;
  if (row >= d.n_rows) return;
  const int lane = wave_lane();
  const int valid = valid_of(d, row);
  const float *src = x + (size_t)row * d.row_len;
  float *dst = out + (size_t)row * d.row_len;
  float mx = -INFINITY;
  bool nan = false;
  for (int i = lane; i < valid; i += kWaveSize) {
    const float v = src[i];
    mx = fmaxf(mx, v);
    nan |= v != v;
  }
  mx = wave_max(mx);
  if (__ballot(nan)) mx = __builtin_nanf("");
  float P = 0.0f;
  for (int base = 0; base < valid; base += kWaveSize) {
    const int i = base + lane;
    float e[1];
    e[0] = i < valid ? exp_f32_of(src[i] - mx) : 0.0f;
    if (i < valid) dst[i] = e[0];
    P = seq_sum_f32_step<1>(P, e);
  }
  const float inv = (float)(1.0 / (double)P);
  for (int i = lane; i < d.row_len; i += kWaveSize) dst[i] = i < valid ? dst[i] * inv : 0.0f;
}

__global__ void exp_f32_kernel(const float *x, float *y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = exp_f32_of(x[i]);
}

}  // namespace
}  // namespace tabby

using namespace tabby;

extern "C" int tabby_debug_exp_f32(const float *x_dev, float *y_dev, int64_t n, void *stream) {
  if (!x_dev || !y_dev) return record_failure(TABBY_EINVAL, "null pointer");
  if (n < 1 || n > ((int64_t)1 << 31)) return record_failure(TABBY_EINVAL, "n must be in [1, 2^31]");
  hipLaunchKernelGGL(exp_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, x_dev,
                     y_dev, n);
  TABBY_HIP_CHECK(hipGetLastError());
  return TABBY_OK;
}

extern "C" int tabby_softmax_rows_device(const float *x_dev, float *out_dev, int32_t n_rows, int32_t row_len,
                                         int32_t causal_period, int32_t causal_offset, void *stream) {
  if (!x_dev || !out_dev) return record_failure(TABBY_EINVAL, "null pointer");
  if (n_rows < 1 || row_len < 1) return record_failure(TABBY_EINVAL, "n_rows and row_len must be >= 1");
  if (causal_period < 0 || causal_offset < 0)
    return record_failure(TABBY_EINVAL, "causal_period and causal_offset must be >= 0");
  if (causal_period > 0 && (int64_t)causal_offset + causal_period > row_len)
    return record_failure(TABBY_EINVAL, "causal_offset + causal_period (" +
                                            std::to_string((int64_t)causal_offset + causal_period) +
                                            ") exceeds row_len (" + std::to_string(row_len) + ")");
  if ((int64_t)n_rows * row_len > ((int64_t)1 << 40)) return record_failure(TABBY_EINVAL, "tensor too large");
  // In place or disjoint: a partial overlap would let one row's writes reach another's reads.
  const char *xb = (const char *)x_dev, *ob = (const char *)out_dev;
  const size_t bytes = (size_t)n_rows * row_len * sizeof(float);
  if (xb != ob && xb < ob + bytes && ob < xb + bytes)
    return record_failure(TABBY_EINVAL, "out must be x itself or not overlap it");
  const RowDims d{n_rows, row_len, causal_period, causal_offset};
  const hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)((n_rows + kSmWaves - 1) / kSmWaves)), block(kSmWaves * kWaveSize);
  const bool aligned = (uintptr_t)x_dev % 16 == 0 && (uintptr_t)out_dev % 16 == 0 && row_len % 4 == 0;
  if (row_len <= kBlockCols && n_rows >= kBlockMinRows) {
    hipLaunchKernelGGL(softmax_rows_block_kernel<kBlockRows>, dim3((unsigned)((n_rows + kBlockRows - 1) / kBlockRows)),
                       block, 0, s, x_dev, out_dev, d);
  } else if (aligned && row_len <= 256) {
    hipLaunchKernelGGL(softmax_rows_reg_kernel<1>, grid, block, 0, s, x_dev, out_dev, d);
  } else if (aligned && row_len <= 512) {
    hipLaunchKernelGGL(softmax_rows_reg_kernel<2>, grid, block, 0, s, x_dev, out_dev, d);
  } else if (aligned && row_len <= 1024) {
    hipLaunchKernelGGL(softmax_rows_reg_kernel<4>, grid, block, 0, s, x_dev, out_dev, d);
  } else if (aligned && row_len <= 2048) {
    hipLaunchKernelGGL(softmax_rows_reg_kernel<8>, grid, block, 0, s, x_dev, out_dev, d);
  } else if (aligned && row_len <= 4096) {
    hipLaunchKernelGGL(softmax_rows_reg_kernel<16>, grid, block, 0, s, x_dev, out_dev, d);
  } else {
    hipLaunchKernelGGL(softmax_rows_stream_kernel, grid, block, 0, s, x_dev, out_dev, d);
  }
  TABBY_HIP_CHECK(hipGetLastError());
  return TABBY_OK;
}
