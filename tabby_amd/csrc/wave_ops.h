// Wave-level (64-lane) building blocks: lane exchanges, reductions, and a bitonic sort of
// 64*R values held in registers (index r*64 + lane), which needs no LDS and no barrier -- the
// strides below 64 are lane exchanges (xor_lane), the larger ones swaps between a lane's
// registers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tabby {

constexpr int kWaveSize = 64;

__device__ __forceinline__ int wave_lane() { return (int)(threadIdx.x & 63); }

// The value held by lane (lane ^ S), S a power of two below 64, without going through LDS:
// DPP quad permutes for 1 and 2, row shifts for 4, a row rotation for 8 (i + 8 mod 16 is
// i ^ 8 within a 16-lane row), and gfx950's permlane swaps for 16 and 32, which exchange
// alternate 16-lane rows and the two 32-lane halves of a pair of registers.
template <int S>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
  static_assert(S == 1 || S == 2 || S == 4 || S == 8 || S == 16 || S == 32, "lane stride");
  if constexpr (S == 1) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);  // quad_perm 1,0,3,2
  } else if constexpr (S == 2) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);  // quad_perm 2,3,0,1
  } else if constexpr (S == 4) {
    const uint32_t up = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x104, 0xF, 0xF, false);  // row_shl:4
    const uint32_t dn = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x114, 0xF, 0xF, false);  // row_shr:4
    return (wave_lane() & 4) ? dn : up;
  } else if constexpr (S == 8) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, false);  // row_ror:8
  } else if constexpr (S == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (wave_lane() & 16) ? r[0] : r[1];
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (wave_lane() & 32) ? r[0] : r[1];
  }
}

template <int S>
__device__ __forceinline__ uint64_t xor_lane(uint64_t v) {
  return (uint64_t)xor_lane<S>((uint32_t)v) | ((uint64_t)xor_lane<S>((uint32_t)(v >> 32)) << 32);
}

template <int S>
__device__ __forceinline__ float xor_lane(float v) {
  return __uint_as_float(xor_lane<S>(__float_as_uint(v)));
}

template <int S>
__device__ __forceinline__ double xor_lane(double v) {
  return __longlong_as_double((long long)xor_lane<S>((uint64_t)__double_as_longlong(v)));
}

// xor_lane with a stride known only after unrolling.
template <typename T>
__device__ __forceinline__ T xor_lane_by(T v, int stride) {
  switch (stride) {
    case 1: return xor_lane<1>(v);
    case 2: return xor_lane<2>(v);
    case 4: return xor_lane<4>(v);
    case 8: return xor_lane<8>(v);
    case 16: return xor_lane<16>(v);
    default: return xor_lane<32>(v);
  }
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, xor_lane<32>(v));
  v = fmaxf(v, xor_lane<16>(v));
  v = fmaxf(v, xor_lane<8>(v));
  v = fmaxf(v, xor_lane<4>(v));
  v = fmaxf(v, xor_lane<2>(v));
  return fmaxf(v, xor_lane<1>(v));
}

// A fixed butterfly: the same inputs give the same bits on every lane and every run.
__device__ __forceinline__ double wave_sum(double v) {
  v += xor_lane<32>(v);
  v += xor_lane<16>(v);
  v += xor_lane<8>(v);
  v += xor_lane<4>(v);
  v += xor_lane<2>(v);
  return v + xor_lane<1>(v);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, xor_lane<32>(v));
  v = max(v, xor_lane<16>(v));
  v = max(v, xor_lane<8>(v));
  v = max(v, xor_lane<4>(v));
  v = max(v, xor_lane<2>(v));
  return max(v, xor_lane<1>(v));
}

// Inclusive prefix sum over the wave's lanes in lane order: DPP row shifts (0 shifted in)
// within each 16-lane row, then row_bcast:15 (lane 15 of each row added to the next row: rows
// 1 and 3) and row_bcast:31 (lane 31 added to rows 2 and 3).
__device__ __forceinline__ uint32_t wave_inclusive_scan_u32(uint32_t x) {
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xF, 0xF, true);  // row_shr:1
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xF, 0xF, true);  // row_shr:2
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xF, 0xF, true);  // row_shr:4
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xF, 0xF, true);  // row_shr:8
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xA, 0xF, false);  // row_bcast:15
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return x;
}

// Makes this wave's LDS writes visible to its other lanes (LDS operations of one wave
// complete in order; waiting for them is all that is needed).
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

template <typename T>
__device__ __forceinline__ T tmax(T a, T b) { return a > b ? a : b; }
template <typename T>
__device__ __forceinline__ T tmin(T a, T b) { return a < b ? a : b; }

// One compare-exchange of a lane exchange: the larger of v and its partner's o where
// keep_max, else the smaller. One compare and one select: for the lanes keeping the smaller
// value the compare's lane mask is inverted (a scalar XOR; o == v needs no swap either way).
template <typename T>
__device__ __forceinline__ T cmpx(T v, T o, bool keep_max) { return ((o > v) == keep_max) ? o : v; }

// The bitonic network's stages for one `size` over strides below 64*R, on the 64*R values
// v[r] at global indices base + r*64 + lane (base a multiple of 64*R); the direction of each
// pair is descending where (index & size) == 0, as in a descending sort of the whole array.
template <int R, typename T>
__device__ __forceinline__ void wave_bitonic_stages(T (&v)[R], int base, int size) {
  const int lane = wave_lane();
  const int top = min(size >> 1, kWaveSize * R / 2);
#pragma unroll
  for (int stride = kWaveSize * R / 2; stride > 0; stride >>= 1) {
    if (stride > top) continue;
    if (stride >= kWaveSize) {
      const int rs = stride / kWaveSize;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if ((r & rs) == 0) {
          const int r2 = r | rs;
          const bool desc = ((base + r * kWaveSize + lane) & size) == 0;
          const T a = v[r], b = v[r2];
          const bool swap = desc ? (a < b) : (a > b);
          v[r] = swap ? b : a;
          v[r2] = swap ? a : b;
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const T o = xor_lane_by(v[r], stride);
        const bool lower = (lane & stride) == 0;
        const bool desc = ((base + r * kWaveSize + lane) & size) == 0;
        v[r] = cmpx(v[r], o, lower == desc);
      }
    }
  }
}

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
          const T o = xor_lane_by(v[r], stride);
          const bool lower = (lane & stride) == 0;
          const bool desc = (((r * kWaveSize) | lane) & size) == 0;
          v[r] = cmpx(v[r], o, lower == desc);
        }
      }
    }
  }
}


}  // namespace tabby
