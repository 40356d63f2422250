// Wave-level (64-lane) building blocks: reductions, and a bitonic sort of 64*R values held
// in registers (index r*64 + lane), which needs no LDS and no barrier -- the strides below
// 64 are lane exchanges (__shfl_xor), the larger ones swaps between a lane's registers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tabby {

constexpr int kWaveSize = 64;

__device__ __forceinline__ int wave_lane() { return (int)(threadIdx.x & 63); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Makes this wave's LDS writes visible to its other lanes (LDS operations of one wave
// complete in order; waiting for them is all that is needed).
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

template <typename T>
__device__ __forceinline__ T tmax(T a, T b) { return a > b ? a : b; }
template <typename T>
__device__ __forceinline__ T tmin(T a, T b) { return a < b ? a : b; }

// Descending bitonic sort of the 64*R values v[r] (element index r*64 + lane).
template <int R, typename T>
__device__ __forceinline__ void wave_sort_desc(T (&v)[R]) {
  const int lane = wave_lane();
#pragma unroll
  for (int size = 2; size <= kWaveSize * R; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (stride >= kWaveSize) {
        const int rs = stride / kWaveSize;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if ((r & rs) == 0) {
            const int r2 = r | rs;
            const bool desc = (((r * kWaveSize) | lane) & size) == 0;
            const T a = v[r], b = v[r2];
            const bool swap = desc ? (a < b) : (a > b);
            v[r] = swap ? b : a;
            v[r2] = swap ? a : b;
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const T o = __shfl_xor(v[r], stride);
          const bool lower = (lane & stride) == 0;
          const bool desc = (((r * kWaveSize) | lane) & size) == 0;
          v[r] = (lower == desc) ? tmax(v[r], o) : tmin(v[r], o);
        }
      }
    }
  }
}


}  // namespace tabby
