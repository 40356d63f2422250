// Loads of logits from HBM, shared by the library's kernels: VEC consecutive elements (16
// bytes for the vector forms) widened to f32. f16 widening is exact (tests/support.ts:61-74
// states the same property for its reference). f16 logits are passed as their uint16_t bits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tabby {

template <typename In, int VEC>
struct Loader;

// Streaming loads are nontemporal: every logit is read once, so they should not displace
// other lines in the caches (measured ~12% more HBM bandwidth on MI355X for this pattern).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <>
struct Loader<float, 4> {
  __device__ static void load(const float *p, float (&v)[4]) {
    const f32x4 f = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
    v[0] = f.x;
    v[1] = f.y;
    v[2] = f.z;
    v[3] = f.w;
  }
};

template <>
struct Loader<float, 1> {
  __device__ static void load(const float *p, float (&v)[1]) { v[0] = __builtin_nontemporal_load(p); }
};

__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

template <>
struct Loader<uint16_t, 8> {
  __device__ static void load(const uint16_t *p, float (&v)[8]) {
    const u32x4 u = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
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
  __device__ static void load(const uint16_t *p, float (&v)[1]) {
    v[0] = half_bits_to_float(__builtin_nontemporal_load(p));
  }
};

// Streaming reads through a buffer resource over one row (or slice) of logits: the address
// is a per-lane offset plus a scalar offset (the chunk's, in an SGPR), so a chunk costs no
// per-lane 64-bit address arithmetic (sixteen element loads would otherwise hold sixteen
// 64-bit addresses), and the resource's range check returns zeros without touching memory
// for bytes at or past its end, so a chunk that runs past the row's end, or a chunk index
// past the last, needs no clamping (the callers mask such elements by index). Nontemporal,
// like the global loads above.
constexpr int kBufNontemporal = 2;     // the instruction's nt bit
constexpr int kBufWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format, no swizzle

struct RowBuffer {
  __amdgpu_buffer_rsrc_t rsrc;
  __device__ __forceinline__ RowBuffer(const void *base, uint32_t bytes)
      : rsrc(__builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, kBufWord3)) {}
  __device__ __forceinline__ u32x4 load16(uint32_t lane_offset, uint32_t scalar_offset) const {
    return __builtin_amdgcn_raw_buffer_load_b128(rsrc, lane_offset, scalar_offset, kBufNontemporal);
  }
  __device__ __forceinline__ float load_elem(const float *, uint32_t lane_offset, uint32_t scalar_offset) const {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsrc, lane_offset, scalar_offset, kBufNontemporal));
  }
  __device__ __forceinline__ float load_elem(const uint16_t *, uint32_t lane_offset, uint32_t scalar_offset) const {
    return half_bits_to_float(__builtin_amdgcn_raw_buffer_load_b16(rsrc, lane_offset, scalar_offset, kBufNontemporal));
  }
};

// The VEC values of one 16-byte load, widened to f32.
template <typename In, int VEC>
struct Widen;
template <>
struct Widen<float, 4> {
  __device__ static void from(u32x4 u, float (&v)[4]) {
    v[0] = __uint_as_float(u.x);
    v[1] = __uint_as_float(u.y);
    v[2] = __uint_as_float(u.z);
    v[3] = __uint_as_float(u.w);
  }
};
template <>
struct Widen<uint16_t, 8> {
  __device__ static void from(u32x4 u, float (&v)[8]) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = half_bits_to_float(w[i] & 0xffffu);
      v[2 * i + 1] = half_bits_to_float(w[i] >> 16);
    }
  }
};

__device__ __forceinline__ float load_one(const float *p) { return *p; }
__device__ __forceinline__ float load_one(const uint16_t *p) { return half_bits_to_float(*p); }

}  // namespace tabby
