// The lm_head's int4 matrix-vector product, one output row per lane, in the reference's order.
//
// The reference's lm_head (src/engine/forward.ts:408-428 -> encodeQuantMatmul, :732-770;
// src/shaders/matvec_q4.wgsl) multiplies block-quantized int4 weights by the last hidden
// state, and its CPU reference matmulQuantized (src/reference/cpu.ts:352-393) fixes the
// arithmetic: for output row m, word by word (eight 4-bit values, value j at bits 4j,
// dequant(q) = q - 8 times the block's scale), partial = the f32 sum, in order, of
// f32((q_j - 8) * x_j); acc = f32(acc + f32(partial * scale)); then + bias[m]. One lane per
// output row follows that order exactly, so the logits here are the CPU reference's bit for
// bit (the build uses -ffp-contract=off: no product is fused into its sum).
//
// Layout in HBM (this library's, made from the reference's by tabby_lmhead_q4_pack_device):
//   packed  u32 [hidden / 32][vocab][4]: the four words of a 32-weight group of row r are
//           16 consecutive bytes, and consecutive rows' groups are adjacent, so a wave's
//           64 lanes read 1 KB contiguous per load;
//   scales  f16 bits [hidden / block][vocab]: a wave reads 128 contiguous bytes per block.
// The activations x [R][hidden] are the same for every lane: their loads are scalar.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "loads.h"

namespace tabby {

constexpr int kQ4Group = 32;  // weights per 16-byte load: four u32 words

struct Q4Matrix {
  const uint32_t *packed;  // [hidden / 32][vocab][4]
  const uint16_t *scales;  // [hidden / block][vocab], f16 bits
  const float *bias;       // [vocab] or null
  int vocab, hidden, block;
};

// acc[t] = row `r` of W times x[t] (+ bias[r]) for t < R, in matmulQuantized's order.
// AHEAD: groups in flight per lane. A row's groups are a chain of dependent accumulations,
// and at one row per lane the grid holds only ~2.3 waves per SIMD, so the lane keeps the codes
// and scales of the next AHEAD groups loading while it works on the current one (one row: the
// product 23.4 -> 21.0 us). Many activation rows hide the loads behind their arithmetic:
// q4_dot_row_serial below serves them.
template <int R, int AHEAD = 4>
__device__ __forceinline__ void q4_dot_row(const Q4Matrix &W, const float *__restrict__ x, int r, float (&acc)[R]) {
#pragma unroll
  for (int t = 0; t < R; ++t) acc[t] = 0.0f;
  const int groups = W.hidden / kQ4Group;
  const u32x4 *p = reinterpret_cast<const u32x4 *>(W.packed) + r;
  const size_t stride = (size_t)W.vocab;  // u32x4 entries between consecutive groups of one row
  const uint16_t *sp = W.scales + r;
  const int per_block = W.block / kQ4Group;  // groups per scale
  // Loads are unconditional (past the last group they reread it), so that no register holding
  // a load in flight is ever copied, which would wait for it.
  auto load_group = [&](int g, u32x4 &q, uint32_t &sc) {
    const int gg = min(g, groups - 1);
    q = __builtin_nontemporal_load(p + (size_t)gg * stride);
    sc = sp[(size_t)(gg / per_block) * stride];
  };
  u32x4 q[AHEAD];
  uint32_t sc[AHEAD];
#pragma unroll
  for (int d = 0; d < AHEAD; ++d) load_group(d, q[d], sc[d]);
  for (int g0 = 0; g0 < groups; g0 += AHEAD) {
#pragma unroll
    for (int d = 0; d < AHEAD; ++d) {
      const int g = g0 + d;
      if (g >= groups) break;  // uniform
      const u32x4 cur = q[d];
      const float scale = half_bits_to_float(sc[d]);
      load_group(g + AHEAD, q[d], sc[d]);
      // q - 8 is the signed 4-bit reading of q ^ 8: one XOR per word, then one signed
      // bit-field extract and one conversion per value.
      const uint32_t word[4] = {cur.x ^ 0x88888888u, cur.y ^ 0x88888888u, cur.z ^ 0x88888888u, cur.w ^ 0x88888888u};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k0 = g * kQ4Group + i * 8;
        float c[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) c[j] = (float)((int32_t)(word[i] << (28 - 4 * j)) >> 28);
#pragma unroll
        for (int t = 0; t < R; ++t) {
          const float *xt = x + (size_t)t * W.hidden + k0;
          float partial = 0.0f;
#pragma unroll
          for (int j = 0; j < 8; ++j) partial = partial + c[j] * xt[j];
          acc[t] = acc[t] + partial * scale;
        }
      }
    }
  }
  if (W.bias) {
    const float b = W.bias[r];
#pragma unroll
    for (int t = 0; t < R; ++t) acc[t] = acc[t] + b;
  }
}

// The same product with one group's codes in flight and each scale loaded where it is used:
// the smaller loop the standalone product keeps for four or more activation rows (eight rows:
// 82 us, against 95 us in the form above).
template <int R>
__device__ __forceinline__ void q4_dot_row_serial(const Q4Matrix &W, const float *__restrict__ x, int r,
                                                  float (&acc)[R]) {
#pragma unroll
  for (int t = 0; t < R; ++t) acc[t] = 0.0f;
  const int groups = W.hidden / kQ4Group;
  const u32x4 *p = reinterpret_cast<const u32x4 *>(W.packed) + r;
  const size_t stride = (size_t)W.vocab;
  u32x4 q = __builtin_nontemporal_load(p);
  for (int g = 0; g < groups; ++g) {
    const u32x4 cur = q;
    if (g + 1 < groups) q = __builtin_nontemporal_load(p + (size_t)(g + 1) * stride);  // next group in flight
    const float scale = half_bits_to_float(W.scales[(size_t)(g * kQ4Group / W.block) * stride + r]);
    const uint32_t word[4] = {cur.x ^ 0x88888888u, cur.y ^ 0x88888888u, cur.z ^ 0x88888888u, cur.w ^ 0x88888888u};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k0 = g * kQ4Group + i * 8;
      float c[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) c[j] = (float)((int32_t)(word[i] << (28 - 4 * j)) >> 28);
#pragma unroll
      for (int t = 0; t < R; ++t) {
        const float *xt = x + (size_t)t * W.hidden + k0;
        float partial = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) partial = partial + c[j] * xt[j];
        acc[t] = acc[t] + partial * scale;
      }
    }
  }
  if (W.bias) {
    const float b = W.bias[r];
#pragma unroll
    for (int t = 0; t < R; ++t) acc[t] = acc[t] + b;
  }
}

}  // namespace tabby
