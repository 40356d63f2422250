// Workgroup-level building blocks for the sampler kernels: reductions, scans, the
// radix select over 64-bit composites, and an LDS bitonic sort.
//
// Workgroups are kBlock = 256 lanes = 4 wave64s. Cross-lane steps inside a wave use DPP and
// permlane exchanges (wave_ops.h); the cross-wave step goes through a few words of LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wave_ops.h"

namespace tabby {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;
constexpr int kBins = 2048;  // 11-bit radix digits

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// LDS words the helpers below communicate through. One per workgroup of NW waves; the
// helpers take the workgroup's size from it (kBlock lanes unless stated).
template <int NW>
struct BlockScratchT {
  float f[NW];
  double d[NW];
  double d2[NW];
  uint32_t u[NW];
  uint32_t bin, above, count, slot, slot2;
};
using BlockScratch = BlockScratchT<kWaves>;

template <int NW>
__device__ __forceinline__ float block_max(float v, BlockScratchT<NW> &s) {
  v = wave_max(v);
  __syncthreads();
  if (lane_id() == 0) s.f[wave_id()] = v;
  __syncthreads();
  float r = s.f[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r = fmaxf(r, s.f[i]);
  return r;
}

// Fixed reduction tree, so the result is bit-identical from run to run.
template <int NW>
__device__ __forceinline__ double block_sum(double v, BlockScratchT<NW> &s) {
  v = wave_sum(v);
  __syncthreads();
  if (lane_id() == 0) s.d[wave_id()] = v;
  __syncthreads();
  double r = s.d[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r += s.d[i];
  return r;
}

// Exclusive prefix sum in thread order; *total receives the workgroup sum.
template <int NW>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, BlockScratchT<NW> &s,
                                                         uint32_t *total) {
  const int lane = lane_id();
  const uint32_t inc = wave_inclusive_scan_u32(v);
  __syncthreads();
  if (lane == 63) s.u[wave_id()] = inc;
  __syncthreads();
  uint32_t base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const uint32_t w = s.u[i];
    base += (i < wave_id()) ? w : 0u;
    tot += w;
  }
  *total = tot;
  return base + inc - v;
}

// Given a filled histogram, find the bin b holding the need-th largest element counted
// from the top: above(b) < need <= above(b) + hist[b]. Thread t owns the PER bins just
// below kBins - t*PER, so thread order is descending bin order. Publishes b, above(b) and
// hist[b] in s.bin / s.above / s.count.
template <int NW>
__device__ __forceinline__ void find_bin(const uint32_t *hist, uint32_t need, BlockScratchT<NW> &s) {
  constexpr int PER = kBins / (NW * 64);
  const int top = kBins - 1 - (int)threadIdx.x * PER;
  uint32_t c[PER];
  uint32_t sum = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    c[i] = hist[top - i];
    sum += c[i];
  }
  uint32_t total;
  const uint32_t before = block_exclusive_scan(sum, s, &total);
  if (before < need && need <= before + sum) {
    uint32_t acc = before;
    bool found = false;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if (!found && need <= acc + c[i]) {
        s.bin = (uint32_t)(top - i);
        s.above = acc;
        s.count = c[i];
        found = true;
      }
      acc += c[i];
    }
  }
  __syncthreads();
}

// Radix select on 64-bit composites: finds the threshold such that exactly `need` of the
// elements visited by for_each satisfy (v >> shift) >= (prefix >> shift). Digits are
// 11/11/10 bits of the value key, then 11/11/10 bits of the ~index word; a pass that leaves
// the threshold bin exactly full ends the search early, so index digits are only visited
// when values tie across the threshold. Requires 1 <= need <= number of elements.
struct SelectResult {
  uint64_t prefix;
  int shift;
};

__device__ __forceinline__ int digit_shift(int pass) {
  return pass == 0 ? 53 : pass == 1 ? 42 : pass == 2 ? 32 : pass == 3 ? 21 : pass == 4 ? 10 : 0;
}

// max_passes < 6 stops early: the result then only bounds the need-th largest from below
// (every selected element is still >= prefix, and at least `need` elements are selected).
template <int NW, class ForEach>
__device__ __forceinline__ SelectResult radix_select(ForEach for_each, uint32_t need, uint32_t *hist,
                                     BlockScratchT<NW> &s, int max_passes = 6) {
  uint64_t prefix = 0;
  int done = 64;
  for (int pass = 0; pass < max_passes; ++pass) {
    const int shift = digit_shift(pass);
    const uint32_t dmask = (pass == 2 || pass == 5) ? 0x3ffu : 0x7ffu;
    for (int i = threadIdx.x; i < kBins; i += NW * 64) hist[i] = 0u;
    __syncthreads();
    const bool first = pass == 0;
    const int cmp_shift = first ? 0 : done;
    const uint64_t want = first ? 0 : (prefix >> cmp_shift);
    for_each([&](uint64_t v) {
      if (first || (v >> cmp_shift) == want) atomicAdd(&hist[(uint32_t)(v >> shift) & dmask], 1u);
    });
    __syncthreads();
    find_bin(hist, need, s);
    const uint32_t b = s.bin, above = s.above, count = s.count;
    __syncthreads();
    prefix |= (uint64_t)b << shift;
    need -= above;
    done = shift;
    if (count == need) break;
  }
  return {prefix, done};
}

__device__ __forceinline__ bool selected(uint64_t v, SelectResult r) {
  return (v >> r.shift) >= (r.prefix >> r.shift);
}

// In-place descending bitonic sort of a[0..n), n a power of two, by the whole workgroup of
// NW waves.
template <int NW = kWaves>
__device__ __forceinline__ void bitonic_sort_desc(uint64_t *a, int n) {
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < (n >> 1); i += NW * 64) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const uint64_t x = a[lo], y = a[hi];
        if ((x < y) == desc) {
          a[lo] = y;
          a[hi] = x;
        }
      }
      __syncthreads();
    }
  }
}

// In-place descending sort of a[0..n) in LDS, n a power of two, by the whole workgroup:
// each wave sorts chunks of 64 * R entries in registers (the network's stages below the
// chunk need no barrier), and only the strides of a chunk and above go through LDS with a
// barrier each. R = 4 (256-entry chunks) suits four waves; with sixteen, R = 1 keeps every
// wave busy in the register stages at the cost of two more LDS strides per merge level.
template <int NW = kWaves, int R = 4>
__device__ __forceinline__ void block_sort_desc(uint64_t *a, int n) {
  constexpr int kChunkN = kWaveSize * R;  // entries per wave pass
  if (n < kChunkN) {
    bitonic_sort_desc<NW>(a, n);
    return;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  auto chunk_pass = [&](int size, bool full) {
    for (int base = wave * kChunkN; base < n; base += NW * kChunkN) {
      uint64_t v[R];
#pragma unroll
      for (int r = 0; r < R; ++r) v[r] = a[base + r * kWaveSize + lane];
      if (full) {
        for (int sz = 2; sz <= kChunkN; sz <<= 1) wave_bitonic_stages<R>(v, base, sz);
      } else {
        wave_bitonic_stages<R>(v, base, size);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) a[base + r * kWaveSize + lane] = v[r];
    }
    __syncthreads();
  };
  chunk_pass(0, true);
  for (int size = 2 * kChunkN; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride >= kChunkN; stride >>= 1) {
      for (int i = threadIdx.x; i < (n >> 1); i += NW * 64) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const uint64_t x = a[lo], y = a[hi];
        if ((x < y) == desc) {
          a[lo] = y;
          a[hi] = x;
        }
      }
      __syncthreads();
    }
    chunk_pass(size, false);
  }
}

// One merge round of block_merge_sort_desc: runs of L = 32 R sorted descending are merged in
// pairs by wave w, which writes register r = w mod R (sorted places 64 r .. 64 r + 63) of pair
// p = w / R. The pair's first run followed by its second reversed is a bitonic sequence X of
// 2L; the bitonic merge's stages of stride 64 and above compare X[i] with X[i + stride] at the
// same lane, and of each of them the wave keeps only the half its register falls in: the
// maxima above, the minima below, one compare and select per pair, R - 1 in all. What is left
// is the bitonic 64 of register r, sorted by the stages below 64 through lane exchanges. The
// loads and the store are 64 consecutive entries each.
template <int R>
__device__ __forceinline__ void bitonic_merge_round(const uint64_t *src, uint64_t *dst, int w) {
  constexpr int L = 32 * R;
  const int lane = lane_id(), p = w / R, r = w - p * R;
  const uint64_t *A = src + 2 * p * L, *B = A + L;
  uint64_t v[R];
#pragma unroll
  for (int q = 0; q < R; ++q) v[q] = q < R / 2 ? A[64 * q + lane] : B[2 * L - 1 - 64 * q - lane];
#pragma unroll
  for (int half = R / 2; half >= 1; half >>= 1) {
    const bool low = (r & half) != 0;  // the minima's half
#pragma unroll
    for (int k = 0; k < half; ++k) v[k] = cmpx(v[k], v[k + half], !low);
  }
#pragma unroll
  for (int stride = 32; stride > 0; stride >>= 1) v[0] = cmpx(v[0], xor_lane_by(v[0], stride), (lane & stride) == 0);
  dst[2 * p * L + 64 * r + lane] = v[0];
}

// In-place descending sort of a[0..n), n a power of two and at most NW * 64 <= 1,024, by the
// whole workgroup of NW waves, through tmp[0..n) in LDS: each wave sorts 64 entries in
// registers, then log2(n / 64) merge rounds, one barrier each. Up to runs of 256 a round is
// bitonic_merge_round: each of the n / 64 waves computes 64 entries of the merged runs from 2,
// 4 or 8 loads (0.9, 0.7 and 0.8 us of config 5's tail against 1.05, 0.97 and 1.08 for the
// binary search below). The round of runs of 512 places each entry by binary search in the
// other run -- an equal entry of the left run counts as ahead of the right run's, so that
// equal entries, the zero padding among them, take distinct places -- which beat the bitonic
// form's 16 loads and 15 selects per lane there (1.17 against 1.25 us).
template <int NW>
__device__ __forceinline__ void block_merge_sort_desc(uint64_t *a, uint64_t *tmp, int n) {
  static_assert(NW <= 16, "n <= 1,024: the last round is the binary search's");
  const int t = (int)threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  if (n <= 64) {
    if (t < 64) {
      uint64_t v[1] = {lane < n ? a[lane] : 0ull};
      wave_sort_desc<1>(v);
      if (lane < n) a[lane] = v[0];
    }
    __syncthreads();
    return;
  }
  if (t < n) {
    uint64_t v[1] = {a[t]};
    wave_sort_desc<1>(v);
    a[t] = v[0];
  }
  __syncthreads();
  uint64_t *src = a, *dst = tmp;
  for (int len = 64; len < n; len <<= 1) {
    if (len == 512) {
      // The last round by binary search: each entry's place in the other run (16 loads per
      // lane and 15 selects made the bitonic form slower here).
      if (t < n) {
        const uint64_t x = src[t];
        const int run = t / len, i = t - run * len;
        const bool left = (run & 1) == 0;
        const uint64_t *other = src + (run ^ 1) * len;
        auto ahead = [&](uint64_t y) { return left ? y > x : y >= x; };
        int pos = 0;  // entries of `other` ahead of x: a prefix of it
        for (int step = len >> 1; step > 0; step >>= 1)
          if (ahead(other[pos + step - 1])) pos += step;
        pos += ahead(other[pos]) ? 1 : 0;  // only at pos == len - 1 can other[pos] be ahead
        dst[(run & ~1) * len + i + pos] = x;
      }
    } else if (w < n / 64) {
      switch (len) {
        case 64: bitonic_merge_round<2>(src, dst, w); break;
        case 128: bitonic_merge_round<4>(src, dst, w); break;
        default: bitonic_merge_round<8>(src, dst, w); break;
      }
    }
    __syncthreads();
    uint64_t *const s2 = src;
    src = dst;
    dst = s2;
  }
  if (src != a) {
    if (t < n) a[t] = src[t];
    __syncthreads();
  }
}

__host__ __device__ __forceinline__ int next_pow2(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

}  // namespace tabby
