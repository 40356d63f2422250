// Greedy decoding's fast path: the argmax of each row of logits, on the GPU.
//
// The reference picks greedy tokens with argmax (src/engine/sampler.ts:13-23): a strict `>`
// scan from index 0, so the lowest index wins ties, +0 and -0 are equal, a NaN never wins,
// and a row whose first entry is NaN, or whose entries are all -inf or NaN, yields 0. Its
// decode loop gets the same id from a one-candidate pool (forward.runSegment with
// {topK: 1}, inference.worker.ts:216-229; generateGreedy, sampler.ts:54-76). Here that is one
// read of the row with no pool, no sum and no tail: each thread keeps the first maximum of
// its own elements (it scans them in index order), and threads, waves and workgroups combine
// by 64-bit composites (value key, ~index), the larger value or, for equal values, the lower
// index winning -- exactly the reference's order. HBM-bound: vocab * sizeof(In) per row.
//
// Grid: one 1,024-lane workgroup per row when there are at least as many rows as CUs, which
// writes its row's answer; otherwise rows x splits workgroups of 256 lanes, each writing a
// composite to the handle's scratch, and argmax_finish_kernel combines a row's splits.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "abi_internal.h"
#include "device_math.h"
#include "loads.h"
#include "wave_ops.h"

namespace tabby {
namespace {

constexpr int kArgBlock = 256;       // lanes per workgroup when rows are split
constexpr int kArgRowBlock = 1024;   // lanes per workgroup when a workgroup takes a whole row
constexpr int kArgUnroll = 4;        // 16-byte loads in flight per lane
constexpr int kArgMaxSplits = 64;

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = tmax(v, xor_lane<1>(v));
  v = tmax(v, xor_lane<2>(v));
  v = tmax(v, xor_lane<4>(v));
  v = tmax(v, xor_lane<8>(v));
  v = tmax(v, xor_lane<16>(v));
  v = tmax(v, xor_lane<32>(v));
  return v;
}

// The composite of the first maximum among this lane's elements, scanned in index order with
// the reference's strict `>`: a NaN never compares greater, so it is skipped. A lane whose
// elements are all -inf or NaN offers -inf at an arbitrary index; the row's answer is then
// decided without it (see row_answer).
template <typename In, int VEC, int BLOCK>
__device__ __forceinline__ uint64_t lane_first_max(const In *row, int begin, int end) {
  const int lane = (int)threadIdx.x;
  float best = -INFINITY;
  int at = 0;
  constexpr int kStep = BLOCK * VEC;
  // Whole 16-byte groups: kArgUnroll loads in flight per lane.
  const int vend = begin + ((end - begin) / VEC) * VEC;
  int i = begin + lane * VEC;
  for (; i + (kArgUnroll - 1) * kStep < vend; i += kArgUnroll * kStep) {
    float v[kArgUnroll][VEC];
#pragma unroll
    for (int u = 0; u < kArgUnroll; ++u) Loader<In, VEC>::load(row + i + u * kStep, v[u]);
#pragma unroll
    for (int u = 0; u < kArgUnroll; ++u)
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        if (v[u][e] > best) {
          best = v[u][e];
          at = i + u * kStep + e;
        }
  }
  for (; i < vend; i += kStep) {
    float v[VEC];
    Loader<In, VEC>::load(row + i, v);
#pragma unroll
    for (int e = 0; e < VEC; ++e)
      if (v[e] > best) {
        best = v[e];
        at = i + e;
      }
  }
  // The ragged end (fewer than VEC elements), one element per lane, after the lane's others.
  const int j = vend + lane;
  if (j < end) {
    const float v = load_one(row + j);
    if (v > best) {
      best = v;
      at = j;
    }
  }
  return composite(key_of(best), (uint32_t)at);
}

// The reference's answer from the row's largest composite: the composite's index, unless the
// first entry is NaN (nothing compares greater than it, sampler.ts:14-18) or nothing in the
// row lies above -inf (nothing compares greater than the first entry, -inf or NaN): then 0.
template <typename In>
__device__ __forceinline__ int row_answer(const In *src, uint64_t best) {
  const float first = load_one(src);
  if (first != first || composite_key(best) <= kNegInfKey) return 0;
  return (int)composite_index(best);
}

template <typename In, int VEC, int BLOCK>
__global__ __launch_bounds__(BLOCK) void argmax_kernel(const In *logits, int vocab, int splits, int split_len,
                                                       uint64_t *partial, int32_t *ids, float *max_logits) {
  __shared__ uint64_t wave_best[BLOCK / kWaveSize];
  const int row = (int)blockIdx.x / splits;
  const int split = (int)blockIdx.x - row * splits;
  const In *src = logits + (size_t)row * (size_t)vocab;
  const int begin = split * split_len;
  const int end = min(vocab, begin + split_len);
  uint64_t c = lane_first_max<In, VEC, BLOCK>(src, begin, end);
  c = wave_max_u64(c);
  const int w = (int)threadIdx.x / kWaveSize;
  if (wave_lane() == 0) wave_best[w] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = wave_best[0];
#pragma unroll
    for (int i = 1; i < BLOCK / kWaveSize; ++i) b = tmax(b, wave_best[i]);
    if (splits == 1) {
      const int id = row_answer(src, b);
      ids[row] = id;
      if (max_logits) max_logits[row] = load_one(src + id);
    } else {
      partial[(size_t)row * splits + split] = b;
    }
  }
}

// One lane per row: the row's splits combined (largest composite), then the answer.
template <typename In>
__global__ __launch_bounds__(kArgBlock) void argmax_finish_kernel(const In *logits, int rows, int vocab, int splits,
                                                                  const uint64_t *partial, int32_t *ids,
                                                                  float *max_logits) {
  const int row = (int)(blockIdx.x * kArgBlock + threadIdx.x);
  if (row >= rows) return;
  const uint64_t *p = partial + (size_t)row * splits;
  uint64_t b = p[0];
  for (int s = 1; s < splits; ++s) b = tmax(b, p[s]);
  const In *src = logits + (size_t)row * (size_t)vocab;
  const int id = row_answer(src, b);
  ids[row] = id;
  if (max_logits) max_logits[row] = load_one(src + id);
}

template <typename In, int VEC>
int launch_argmax(const HandleView &hv, const In *logits, int rows, int vocab, int32_t *ids, float *max_logits,
                  hipStream_t stream) {
  if (rows >= hv.cus) {
    // A 16-wave workgroup per row writes the row's answer itself: no second launch (a split
    // batch's finishing kernel cost ~4 us on 256 rows, the read itself ~24.7 us).
    hipLaunchKernelGGL((argmax_kernel<In, VEC, kArgRowBlock>), dim3((unsigned)rows), dim3(kArgRowBlock), 0, stream,
                       logits, vocab, 1, vocab, (uint64_t *)nullptr, ids, max_logits);
    TABBY_HIP_CHECK(hipGetLastError());
    return TABBY_OK;
  }
  // Fewer rows: workgroups enough for about four 4-wave workgroups per CU, each split at
  // least 16 KB of logits, at most kArgMaxSplits.
  const int min_split = (16384 / (int)sizeof(In) + kArgBlock * VEC - 1) / (kArgBlock * VEC) * (kArgBlock * VEC);
  const int want = (4 * hv.cus + rows - 1) / rows;
  const int by_len = (vocab + min_split - 1) / min_split;
  int splits = std::max(1, std::min({want, by_len, kArgMaxSplits}));
  // Splits start on 16-byte boundaries of the row (vocab * sizeof(In) is 16-byte aligned
  // when VEC > 1 is chosen).
  int split_len = (vocab + splits - 1) / splits;
  split_len = (split_len + VEC - 1) / VEC * VEC;
  splits = (vocab + split_len - 1) / split_len;
  uint64_t *partial = (uint64_t *)hv.scratch;
  if (splits > 1 && (size_t)rows * splits * sizeof(uint64_t) > hv.scratch_bytes)
    return record_failure(TABBY_ECAPACITY, "argmax: the handle's scratch is too small for this batch");
  hipLaunchKernelGGL((argmax_kernel<In, VEC, kArgBlock>), dim3((unsigned)(rows * splits)), dim3(kArgBlock), 0,
                     stream, logits, vocab, splits, split_len, partial, ids, max_logits);
  TABBY_HIP_CHECK(hipGetLastError());
  if (splits > 1) {
    hipLaunchKernelGGL((argmax_finish_kernel<In>), dim3((unsigned)((rows + kArgBlock - 1) / kArgBlock)),
                       dim3(kArgBlock), 0, stream, logits, rows, vocab, splits, partial, ids, max_logits);
    TABBY_HIP_CHECK(hipGetLastError());
  }
  return TABBY_OK;
}

}  // namespace
}  // namespace tabby

using namespace tabby;

extern "C" int tabby_argmax_device(tabby_sampler *sampler, const void *logits_dev, int32_t dtype, int32_t rows,
                                   int32_t vocab, int32_t *ids_dev, float *max_logits_dev, void *stream) {
  HandleView hv;
  int rc = handle_view(sampler, &hv);
  if (rc) return rc;
  if (!logits_dev || !ids_dev) return record_failure(TABBY_EINVAL, "null pointer");
  if (dtype != TABBY_F32 && dtype != TABBY_F16) return record_failure(TABBY_EINVAL, "dtype must be TABBY_F32 or TABBY_F16");
  if (rows < 1 || vocab < 1) return record_failure(TABBY_EINVAL, "rows and vocab must be >= 1");
  if (rows > hv.rows_max || vocab > hv.vocab_max)
    return record_failure(TABBY_ECAPACITY, "rows " + std::to_string(rows) + " x vocab " + std::to_string(vocab) +
                                               " exceeds the handle's " + std::to_string(hv.rows_max) + " x " +
                                               std::to_string(hv.vocab_max));
  TABBY_HIP_CHECK(hipSetDevice(hv.device));
  const hipStream_t s = (hipStream_t)stream;
  const size_t esize = dtype == TABBY_F32 ? 4 : 2;
  // 16-byte loads need every row to start on a 16-byte boundary.
  const bool vec = ((uintptr_t)logits_dev % 16 == 0) && ((size_t)vocab * esize % 16 == 0);
  if (dtype == TABBY_F32)
    return vec ? launch_argmax<float, 4>(hv, (const float *)logits_dev, rows, vocab, ids_dev, max_logits_dev, s)
               : launch_argmax<float, 1>(hv, (const float *)logits_dev, rows, vocab, ids_dev, max_logits_dev, s);
  return vec ? launch_argmax<uint16_t, 8>(hv, (const uint16_t *)logits_dev, rows, vocab, ids_dev, max_logits_dev, s)
             : launch_argmax<uint16_t, 1>(hv, (const uint16_t *)logits_dev, rows, vocab, ids_dev, max_logits_dev, s);
}
