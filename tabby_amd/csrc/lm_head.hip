// The lm_head on its own: repacking the reference's int4 weights into this library's layout,
// and the int4 matrix-vector product that writes logits (bit for bit matmulQuantized,
// src/reference/cpu.ts:352-393; see q4_gemv.h). The fused form -- the product feeding the
// sampler's first pass directly, so the logits never reach HBM -- is
// tabby_sampler_sample_lmhead_q4_device in tabby_sampler.hip.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <string>

#include "abi_internal.h"
#include "q4_gemv.h"

namespace tabby {
namespace {

constexpr int kGemvBlock = 256;   // output rows per workgroup, one per lane
constexpr int kGemvMaxRows = 8;   // activation rows per launch (their accumulators are registers)

// The reference's layout (tools/convert.py, matvec_q4.wgsl): row r's words at [r][hidden / 8],
// its f16 scales at [r][hidden / block]. Thread i moves one u32x4 group (or one scale).
__global__ void q4_pack_kernel(const uint32_t *words, const uint16_t *scales, int vocab, int hidden, int block,
                               uint32_t *packed, uint16_t *scales_out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int groups = hidden / kQ4Group;
  const int blocks = hidden / block;
  if (i < (int64_t)vocab * groups) {
    const int r = (int)(i / groups), g = (int)(i % groups);
    const u32x4 v = *reinterpret_cast<const u32x4 *>(words + (size_t)r * (hidden / 8) + (size_t)g * 4);
    *reinterpret_cast<u32x4 *>(packed + ((size_t)g * vocab + r) * 4) = v;
  }
  if (i < (int64_t)vocab * blocks) {
    const int r = (int)(i / blocks), b = (int)(i % blocks);
    scales_out[(size_t)b * vocab + r] = scales[(size_t)r * blocks + b];
  }
}

template <int R>
__global__ __launch_bounds__(kGemvBlock) void q4_gemv_kernel(Q4Matrix W, const float *x, float *y) {
  const int r = (int)(blockIdx.x * kGemvBlock + threadIdx.x);
  if (r >= W.vocab) return;
  float acc[R];
  if constexpr (R >= 4) q4_dot_row_serial<R>(W, x, r, acc);
  else q4_dot_row<R>(W, x, r, acc);
#pragma unroll
  for (int t = 0; t < R; ++t) y[(size_t)t * W.vocab + r] = acc[t];
}

template <int R>
int launch_gemv(const Q4Matrix &W, const float *x, float *y, hipStream_t s) {
  hipLaunchKernelGGL(q4_gemv_kernel<R>, dim3((unsigned)((W.vocab + kGemvBlock - 1) / kGemvBlock)), dim3(kGemvBlock), 0,
                     s, W, x, y);
  TABBY_HIP_CHECK(hipGetLastError());
  return TABBY_OK;
}

}  // namespace

// Shape checks shared with the fused entry point.
int check_q4_shape(int32_t vocab, int32_t hidden, int32_t block) {
  if (vocab < 1 || hidden < kQ4Group || hidden % kQ4Group != 0)
    return record_failure(TABBY_EINVAL, "vocab must be >= 1 and hidden a positive multiple of 32");
  if (block < kQ4Group || block % kQ4Group != 0 || hidden % block != 0)
    return record_failure(TABBY_EINVAL, "block_size must be a multiple of 32 that divides hidden");
  return TABBY_OK;
}

}  // namespace tabby

using namespace tabby;

extern "C" int tabby_lmhead_q4_pack_device(const uint32_t *words_dev, const uint16_t *scales_dev, int32_t vocab,
                                           int32_t hidden, int32_t block_size, uint32_t *packed_dev,
                                           uint16_t *packed_scales_dev, void *stream) {
  if (!words_dev || !scales_dev || !packed_dev || !packed_scales_dev) return record_failure(TABBY_EINVAL, "null pointer");
  int rc = check_q4_shape(vocab, hidden, block_size);
  if (rc) return rc;
  if ((uintptr_t)words_dev % 16 != 0 || (uintptr_t)packed_dev % 16 != 0)
    return record_failure(TABBY_EINVAL, "word arrays must be 16-byte aligned");
  const int64_t n = (int64_t)vocab * (hidden / kQ4Group);  // >= vocab * blocks
  hipLaunchKernelGGL(q4_pack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, words_dev,
                     scales_dev, vocab, hidden, block_size, packed_dev, packed_scales_dev);
  TABBY_HIP_CHECK(hipGetLastError());
  return TABBY_OK;
}

extern "C" int tabby_lmhead_q4_device(const uint32_t *packed_dev, const uint16_t *packed_scales_dev,
                                      const float *bias_dev, const float *hidden_dev, int32_t rows, int32_t vocab,
                                      int32_t hidden, int32_t block_size, float *logits_dev, void *stream) {
  if (!packed_dev || !packed_scales_dev || !hidden_dev || !logits_dev) return record_failure(TABBY_EINVAL, "null pointer");
  int rc = check_q4_shape(vocab, hidden, block_size);
  if (rc) return rc;
  if (rows < 1) return record_failure(TABBY_EINVAL, "rows must be >= 1");
  if ((uintptr_t)packed_dev % 16 != 0) return record_failure(TABBY_EINVAL, "packed weights must be 16-byte aligned");
  const Q4Matrix W{packed_dev, packed_scales_dev, bias_dev, vocab, hidden, block_size};
  const hipStream_t s = (hipStream_t)stream;
  // Up to eight activation rows per pass over the weights.
  for (int t0 = 0; t0 < rows; t0 += kGemvMaxRows) {
    const int n = std::min(kGemvMaxRows, rows - t0);
    const float *x = hidden_dev + (size_t)t0 * hidden;
    float *y = logits_dev + (size_t)t0 * vocab;
    switch (n) {
      case 1: rc = launch_gemv<1>(W, x, y, s); break;
      case 2: rc = launch_gemv<2>(W, x, y, s); break;
      case 3: rc = launch_gemv<3>(W, x, y, s); break;
      case 4: rc = launch_gemv<4>(W, x, y, s); break;
      case 5: rc = launch_gemv<5>(W, x, y, s); break;
      case 6: rc = launch_gemv<6>(W, x, y, s); break;
      case 7: rc = launch_gemv<7>(W, x, y, s); break;
      default: rc = launch_gemv<8>(W, x, y, s); break;
    }
    if (rc) return rc;
  }
  return TABBY_OK;
}
