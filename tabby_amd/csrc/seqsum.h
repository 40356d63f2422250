// Sequential f64 sums, bit for bit, computed by a whole wave.
//
// The reference adds its terms one at a time, left to right (src/engine/sampler.ts:156-203:
// poolMass, the scaled total, the running sums of the draw), so each partial sum is
// P_j = fl(P_(j-1) + t_j) with IEEE round-to-nearest-even. For non-negative terms this
// chain can be evaluated in parallel without changing a single bit:
//
//   While P lies in one binade [2^E, 2^(E+1)) its ulp is u = 2^(E-52) and P = m*u with an
//   integer m < 2^53. The exact sum P + t rounds to the nearest multiple of u as long as the
//   result stays below 2^(E+1), so fl(P + t) = P + u * rint(t / u) -- except when t / u has
//   a fractional part of exactly 1/2, where the tie goes to the even multiple and so depends
//   on m. t / u is an exact power-of-two scaling of t. Hence, between "events", the partial
//   sums are m*u + u * (an integer prefix sum of rint(t_j / u)), and an integer prefix sum
//   has no order dependence.
//
//   A tie (t / u = f + 1/2) rounds to the even one of m + f and m + f + 1, so it adds
//   f + ((m + f) mod 2) and leaves an even sum. Only the parity of the running m matters, and
//   it follows a two-state automaton: a non-tie step XORs it with the parity of its increment,
//   a tie step resets it to 0. Steps compose as maps x -> (x AND k) XOR c, an associative
//   monoid, so the parity before every term comes from a wave scan too, and ties cost
//   nothing extra (terms drawn from few distinct values, as with quantised logits, can tie
//   on most steps).
//
//   An event is a term that takes the integer sum to 2^53 or beyond (the sum leaves the
//   binade and is rounded with a coarser ulp), or the first partial sum that reaches the
//   stop value. An event term is added with an ordinary f64 add from the exact P before it;
//   then the binade is recomputed and the scan resumes after it. P only grows (terms are
//   >= 0), so there are at most a few dozen binade changes.
//
// Integers below 2^53 are exact in f64, so the prefix sums are done in f64: every partial
// sum of non-negative integers is exact while it is below 2^53, and once the true value
// reaches 2^53 the rounded value is >= 2^53 too (2^53 is representable and rounding is
// monotone), which is exactly the event test.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wave_ops.h"

namespace tabby {

constexpr double kTwo52 = 4503599627370496.0;
constexpr double kTwo53 = 9007199254740992.0;
constexpr int kSeqShort = 256;  // sums up to this length run on one lane

// Lane i receives lane i - S of its 16-lane row, or +0 for the first S lanes of the row.
template <int S>
__device__ __forceinline__ double row_shift_up(double v) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, 0x110 + S, 0xF, 0xF, true);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), 0x110 + S, 0xF, 0xF, true);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

__device__ __forceinline__ double lane_f64(double v, int lane) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), lane);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// The DPP move of control `ctrl` applied to both halves of v; rows outside row_mask get 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, ROW_MASK, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, ROW_MASK, 0xF, false);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Inclusive prefix sum over the wave's lanes of non-negative integer-valued v (see above:
// exact below 2^53, >= 2^53 otherwise; for other terms lane i's sum is a tree of at most six
// roundings over lanes 0..i): within rows of 16 by DPP shifts, then row_bcast:15 (lane 15 of
// each row added to the next row: rows 1 and 3) and row_bcast:31 (lane 31 added to rows 2
// and 3).
__device__ __forceinline__ double wave_inclusive_scan(double x) {
  x += row_shift_up<1>(x);
  x += row_shift_up<2>(x);
  x += row_shift_up<4>(x);
  x += row_shift_up<8>(x);
  x += dpp_f64<0x142, 0xA>(x);  // row_bcast:15
  x += dpp_f64<0x143, 0xC>(x);  // row_bcast:31
  return x;
}

// Two independent inclusive prefix sums over the wave's lanes, interleaved stage by stage so
// that each one's DPP moves fill the other's latency: within rows of 16 by row shifts, then
// row_bcast:15 (lane 15 of each row added to the next row: rows 1 and 3) and row_bcast:31
// (lane 31 added to rows 2 and 3). Lane i's sum is a tree of at most six roundings over lanes
// 0..i (for integer-valued terms below 2^53 it is exact).
__device__ __forceinline__ void wave_inclusive_scan2(double &a, double &b) {
  a += row_shift_up<1>(a);
  b += row_shift_up<1>(b);
  a += row_shift_up<2>(a);
  b += row_shift_up<2>(b);
  a += row_shift_up<4>(a);
  b += row_shift_up<4>(b);
  a += row_shift_up<8>(a);
  b += row_shift_up<8>(b);
  a += dpp_f64<0x142, 0xA>(a);  // row_bcast:15
  b += dpp_f64<0x142, 0xA>(b);
  a += dpp_f64<0x143, 0xC>(a);  // row_bcast:31
  b += dpp_f64<0x143, 0xC>(b);
}

// Parity maps x -> (x & k) ^ c on {0, 1}, encoded k | c << 1; kParityId is the identity.
constexpr uint32_t kParityId = 1u;

// The map "apply lo, then hi".
__device__ __forceinline__ uint32_t parity_then(uint32_t lo, uint32_t hi) {
  const uint32_t k = lo & hi & 1u;
  const uint32_t c = (((lo >> 1) & hi) ^ (hi >> 1)) & 1u;
  return k | (c << 1);
}

__device__ __forceinline__ uint32_t parity_apply(uint32_t f, uint32_t x) { return (x & f & 1u) ^ ((f >> 1) & 1u); }

// The composition of the maps of the lanes below this one (exclusive scan in lane order).
__device__ __forceinline__ uint32_t parity_exclusive_scan(uint32_t f) {
  uint32_t x = f;
  x = parity_then((uint32_t)__builtin_amdgcn_update_dpp((int)kParityId, (int)x, 0x111, 0xF, 0xF, false), x);
  x = parity_then((uint32_t)__builtin_amdgcn_update_dpp((int)kParityId, (int)x, 0x112, 0xF, 0xF, false), x);
  x = parity_then((uint32_t)__builtin_amdgcn_update_dpp((int)kParityId, (int)x, 0x114, 0xF, 0xF, false), x);
  x = parity_then((uint32_t)__builtin_amdgcn_update_dpp((int)kParityId, (int)x, 0x118, 0xF, 0xF, false), x);
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)x, 15);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)x, 31);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)x, 47);
  const uint32_t b1 = r0, b2 = parity_then(r0, r1), b3 = parity_then(b2, r2);
  const int lane = wave_lane(), row = lane >> 4;
  const uint32_t below_row = row == 0 ? kParityId : row == 1 ? b1 : row == 2 ? b2 : b3;
  const uint32_t incl = parity_then(below_row, x);
  // Exclusive: the inclusive map of the lane below; a row's first lane takes the rows below.
  uint32_t e = (uint32_t)__builtin_amdgcn_update_dpp((int)kParityId, (int)incl, 0x111, 0xF, 0xF, false);
  if ((lane & 15) == 0) e = below_row;
  return e;
}

__device__ __forceinline__ uint32_t low_bit(double integral) { return (uint32_t)((uint64_t)integral & 1u); }

// Term arrays are read and written through accessors: a plain pointer (LDS or global), or
// PaddedLds, an LDS array with one pad word after every 16 entries, so that the wide form's
// 16 consecutive entries per lane fall on nearly distinct banks (2-way instead of 32-way).
struct PaddedLds {
  double *p;
  __device__ __forceinline__ double &operator[](int j) const { return p[j + (j >> 4)]; }
  __host__ __device__ static constexpr int words(int n) { return n + (n >> 4) + 1; }
};

struct SeqSum {
  double total;  // the last partial sum computed
  int count;     // terms added (the sum stopped early if count < n)
};

// Short sums: every lane adds the same terms left to right (broadcast LDS reads, eight ahead
// of the adds), so the loop is uniform scalar control flow with no per-lane branching; lane
// 0 alone writes the partial sums. kStop: stop at the first partial sum >= stop_at.
template <bool kOut, bool kStop, class In, class Out>
__device__ __forceinline__ SeqSum uniform_seq_sum(In t, int n, Out out, double stop_at) {
  const bool writer = wave_lane() == 0;
  double P = t[0];
  if (kOut && writer) out[0] = P;
  if (kStop && __ballot(P >= stop_at)) return {P, 1};
  int i = 1;
  for (; i + 8 <= n; i += 8) {
    double v[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = t[i + q];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      P += v[q];
      if (kOut && writer) out[i + q] = P;
      if (kStop && __ballot(P >= stop_at)) return {P, i + q + 1};
    }
  }
  for (; i < n; ++i) {
    P += t[i];
    if (kOut && writer) out[i] = P;
    if (kStop && __ballot(P >= stop_at)) return {P, i + 1};
  }
  return {P, n};
}

template <class In, class Out>
__device__ __forceinline__ SeqSum lane_seq_sum(In t, int n, Out out, bool has_out, double stop_at) {
  const bool stop = stop_at < INFINITY;
  if (has_out) return stop ? uniform_seq_sum<true, true>(t, n, out, stop_at) : uniform_seq_sum<true, false>(t, n, out, stop_at);
  return stop ? uniform_seq_sum<false, true>(t, n, out, stop_at) : uniform_seq_sum<false, false>(t, n, out, stop_at);
}

__device__ __forceinline__ SeqSum lane_seq_sum(const double *t, int n, double *out, double stop_at) {
  return lane_seq_sum(t, n, out, out != nullptr, stop_at);
}

// Adds t[0..n) left to right (n >= 1, every t_j >= 0, t[0] > 0, and every partial sum at
// least 2^-960 so that its ulp is a normal number) exactly as a sequential f64 loop would.
// If out is non-null, out[j] receives the j-th partial sum (out may be t itself). The sum
// stops at the first j whose partial sum is >= stop_at (INFINITY: none); count is then
// j + 1. t and out live in LDS or global memory; all 64 lanes call this together.
// A short sum with a stop (top-p's running sums) takes its first kSeqStopSerial terms one by
// one -- peaked rows stop among them -- and the rest by the scan below: one by one, each term
// waits on the previous add, its compare and a branch (config 1's flat rows run all 40).
constexpr int kSeqStopSerial = 8;

__device__ __forceinline__ SeqSum wave_seq_sum(const double *t, int n, double *out, double stop_at) {
  const bool stop = stop_at < INFINITY;
  if (n <= kSeqShort && (!stop || n <= kSeqStopSerial)) return lane_seq_sum(t, n, out, stop_at);
  const int lane = wave_lane();
  double P;
  int a;
  if (n <= kSeqShort) {
    const SeqSum head = lane_seq_sum(t, kSeqStopSerial, out, stop_at);
    if (head.count < kSeqStopSerial || head.total >= stop_at) return head;
    P = head.total;
    a = kSeqStopSerial;
  } else {
    P = t[0];
    if (out && lane == 0) out[0] = P;
    if (P >= stop_at) return {P, 1};
    a = 1;
  }
  while (a < n) {
    // The binade of P: P = m * u with m in [2^52, 2^53).
    const int E = ((int)((uint64_t)__double_as_longlong(P) >> 52) & 0x7ff) - 1023;
    const double u = __longlong_as_double((long long)((uint64_t)(E - 52 + 1023) << 52));
    const double scale = __longlong_as_double((long long)((uint64_t)(52 - E + 1023) << 52));
    const double m = P * scale;
    // Lane L takes term a + L: its rounded increment, a tie rounding to the even sum.
    const int j = a + lane;
    const double q = j < n ? t[j] * scale : 0.0;
    const double fl = __builtin_floor(q);
    const bool tie = q < kTwo52 && q - fl == 0.5;
    double r = __builtin_rint(q);
    if (__ballot(tie)) {  // the parity scan only when some term of this step ties
      const uint32_t parity_before = parity_apply(parity_exclusive_scan(tie ? 0u : 1u | (low_bit(r) << 1)), low_bit(m));
      if (tie) r = fl + (double)(parity_before ^ low_bit(fl));
    }
    const double cum = m + wave_inclusive_scan(r);
    const bool crosses = cum >= kTwo53;
    const bool stops = cum * u >= stop_at;
    const uint64_t flagged = __ballot(j < n && (crosses || stops));
    const int Lf = flagged ? __ffsll((unsigned long long)flagged) - 1 : kWaveSize;
    // Partial sums before the first flagged term are exact: cum * u.
    if (out && j < n && lane < Lf) out[j] = cum * u;
    if (Lf == kWaveSize) {
      const int last = min(n, a + kWaveSize) - 1;
      P = lane_f64(cum, last - a) * u;
      a = last + 1;
      continue;
    }
    const int jf = a + Lf;
    const bool plain_stop = (__builtin_amdgcn_readlane((int)(stops && !crosses), Lf)) != 0;
    if (plain_stop) {  // exact partial sum that reaches stop_at
      const double at = lane_f64(cum, Lf) * u;
      if (out && lane == 0) out[jf] = at;
      return {at, jf + 1};
    }
    // A binade change: one ordinary f64 add from the exact partial sum before it.
    const double before = (Lf == 0 ? m : lane_f64(cum, Lf - 1)) * u;
    P = before + t[jf];
    if (out && lane == 0) out[jf] = P;
    if (P >= stop_at) return {P, jf + 1};
    a = jf + 1;
  }
  return {P, n};
}

// The same sum for at most 64 terms held in registers, lane i holding t_i (lanes >= n hold
// 0), with no memory traffic: a step masks the lanes before its first term instead of moving
// the terms between lanes. Same contract as wave_seq_sum (n >= 1, t >= 0, t_0 > 0); *partial
// receives in lane i < count the i-th partial sum (other lanes: 0).
__device__ __forceinline__ SeqSum reg_seq_sum(double t, int n, double stop_at, double *partial) {
  const int lane = wave_lane();
  double P = lane_f64(t, 0);
  double mine = lane == 0 ? P : 0.0;
  if (P >= stop_at) {
    *partial = mine;
    return {P, 1};
  }
  int a = 1;
  while (a < n) {
    const int E = ((int)((uint64_t)__double_as_longlong(P) >> 52) & 0x7ff) - 1023;
    const double u = __longlong_as_double((long long)((uint64_t)(E - 52 + 1023) << 52));
    const double scale = __longlong_as_double((long long)((uint64_t)(52 - E + 1023) << 52));
    const double m = P * scale;
    const bool live = lane >= a && lane < n;
    const double q = live ? t * scale : 0.0;
    const double fl = __builtin_floor(q);
    const bool tie = live && q < kTwo52 && q - fl == 0.5;
    double r = __builtin_rint(q);
    if (__ballot(tie)) {  // lanes outside the step add 0 and pass the parity through
      const uint32_t parity_before = parity_apply(parity_exclusive_scan(tie ? 0u : 1u | (low_bit(r) << 1)), low_bit(m));
      if (tie) r = fl + (double)(parity_before ^ low_bit(fl));
    }
    const double cum = m + wave_inclusive_scan(r);
    const bool crosses = cum >= kTwo53;
    const bool stops = cum * u >= stop_at;
    const uint64_t flagged = __ballot(live && (crosses || stops));
    const int Lf = flagged ? __ffsll((unsigned long long)flagged) - 1 : kWaveSize;
    if (live && lane < Lf) mine = cum * u;  // exact partial sums before the first event
    if (Lf == kWaveSize) {
      P = lane_f64(cum, n - 1) * u;
      break;
    }
    if (__builtin_amdgcn_readlane((int)(stops && !crosses), Lf) != 0) {  // a plain stop
      const double at = lane_f64(cum, Lf) * u;
      if (lane == Lf) mine = at;
      *partial = mine;
      return {at, Lf + 1};
    }
    // A binade change: one ordinary f64 add from the exact partial sum before it.
    const double before = (Lf == a ? m : lane_f64(cum, Lf - 1)) * u;
    P = before + lane_f64(t, Lf);
    if (lane == Lf) mine = P;
    if (P >= stop_at) {
      *partial = mine;
      return {P, Lf + 1};
    }
    a = Lf + 1;
  }
  *partial = mine;
  return {P, n};
}

// The same sum for long sequences in global memory or padded LDS: each lane takes 16
// consecutive terms (one 128-byte line) per step, so a step covers 1024 terms; an event
// restarts the step after the event term. Same contract as wave_seq_sum; out is written
// only if has_out. settle: the terms are non-increasing, so once a whole step has added
// only terms below half an ulp of the sum (no event), every later term is too and the sum
// cannot change again: it returns there (only when nothing is written).
template <class In, class Out>
__device__ __forceinline__ SeqSum wave_seq_sum_wide(In t, int n, Out out, bool has_out, double stop_at,
                                                    bool settle = false) {
  constexpr int kPer = 16, kStep = kWaveSize * kPer;
  if (n <= kSeqShort) return lane_seq_sum(t, n, out, has_out, stop_at);
  const int lane = wave_lane();
  double P = t[0];
  if (has_out && lane == 0) out[0] = P;
  if (P >= stop_at) return {P, 1};
  int a = 1;
  while (a < n) {
    const int E = ((int)((uint64_t)__double_as_longlong(P) >> 52) & 0x7ff) - 1023;
    const double u = __longlong_as_double((long long)((uint64_t)(E - 52 + 1023) << 52));
    const double scale = __longlong_as_double((long long)((uint64_t)(52 - E + 1023) << 52));
    const double m = P * scale;
    const int first = a + lane * kPer;
    double q[kPer], r[kPer];
    uint32_t tie_bits = 0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      q[i] = (first + i < n ? t[first + i] : 0.0) * scale;
      r[i] = __builtin_rint(q[i]);
      // r - q is exact (the two are within 1/2 of each other), so a tie is |r - q| == 1/2.
      if (q[i] < kTwo52 && __builtin_fabs(r[i] - q[i]) == 0.5) tie_bits |= 1u << i;
    }
    if (__ballot(tie_bits != 0u)) {
      // Each term's parity map (a tie resets, any other term XORs its increment's parity),
      // composed along the lane, then scanned across lanes for the parity at the lane's
      // start; a tie then adds its floor plus the bit that makes the sum even.
      uint32_t lane_map = kParityId;
#pragma unroll
      for (int i = 0; i < kPer; ++i)
        lane_map = parity_then(lane_map, ((tie_bits >> i) & 1u) ? 0u : 1u | (low_bit(r[i]) << 1));
      uint32_t parity = parity_apply(parity_exclusive_scan(lane_map), low_bit(m));
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        if ((tie_bits >> i) & 1u) {
          const double fl = q[i] - 0.5;
          r[i] = fl + (double)(parity ^ low_bit(fl));
          parity = 0u;
        } else {
          parity ^= low_bit(r[i]);
        }
      }
    }
    double pre[kPer];
    double run = 0.0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      run += r[i];
      pre[i] = run;
    }
    const double incl = wave_inclusive_scan(run);
    // Exclusive prefix: the inclusive scan of the lane below (exact while below 2^53, and
    // >= 2^53 otherwise, which only matters past an event) -- a one-lane shift within each
    // 16-lane row, with the row starts filled from the last lane of the row below.
    double below = row_shift_up<1>(incl);
    const double i15 = lane_f64(incl, 15), i31 = lane_f64(incl, 31), i47 = lane_f64(incl, 47);
    if (lane == 16) below = i15;
    if (lane == 32) below = i31;
    if (lane == 48) below = i47;
    const double base = m + below;
    // Partial sums only grow: a lane whose last one neither crosses 2^53 nor reaches the stop
    // has no event; the others look for their first. (Terms past n are 0, so the lane's
    // last partial sum is base + run.)
    const int last_i = min(kPer, n - first) - 1;  // this lane's last term (negative: none)
    const double cum_end = base + run;
    int my_first = kPer;
    bool my_stop = false;
    if (last_i >= 0 && (cum_end >= kTwo53 || cum_end * u >= stop_at)) {
#pragma unroll
      for (int i = kPer - 1; i >= 0; --i) {
        const double cum = base + pre[i];
        if (i <= last_i && (cum >= kTwo53 || cum * u >= stop_at)) {
          my_first = i;
          my_stop = cum < kTwo53;
        }
      }
    }
    const uint64_t has = __ballot(my_first < kPer);
    const int Lf = has ? __ffsll((unsigned long long)has) - 1 : kWaveSize;
    const int fi = Lf < kWaveSize ? __builtin_amdgcn_readlane(my_first, Lf) : 0;
    const int flagged = Lf < kWaveSize ? a + Lf * kPer + fi : n;
    if (has_out) {
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int j = first + i;
        if (j < n && j < flagged) out[j] = (base + pre[i]) * u;
      }
    }
    if (flagged >= n) {
      const int last = min(n, a + kStep) - 1;
      const int ll = (last - a) / kPer;
      P = lane_f64(cum_end, ll) * u;  // lane ll holds the step's last term
      if (settle && !has_out && t[last] * scale < 0.5) return {P, n};
      a = last + 1;
      continue;
    }
    const bool is_stop = __builtin_amdgcn_readlane((int)my_stop, Lf) != 0;
    double before_mine = 0.0, at_mine = 0.0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      if (i == fi) {
        before_mine = i == 0 ? base : base + pre[i - 1];
        at_mine = base + pre[i];
      }
    }
    if (is_stop) {
      const double at = lane_f64(at_mine, Lf) * u;
      if (has_out && lane == 0) out[flagged] = at;
      return {at, flagged + 1};
    }
    P = lane_f64(before_mine, Lf) * u + t[flagged];
    if (has_out && lane == 0) out[flagged] = P;
    if (P >= stop_at) return {P, flagged + 1};
    a = flagged + 1;
  }
  return {P, n};
}

__device__ __forceinline__ SeqSum wave_seq_sum_wide(const double *t, int n, double *out, double stop_at) {
  return wave_seq_sum_wide(t, n, out, out != nullptr, stop_at);
}

// LDS words through which the NW waves of block_seq_sum_wide combine a step.
template <int NW>
struct SeqScratch {
  uint32_t map[NW];    // each wave's parity map over its terms
  uint32_t tie[NW];    // whether the wave holds a tie
  double total[NW];    // each wave's integer increment
  int flag[NW];        // each wave's first event (n: none)
  uint32_t stop[NW];   // that event is a plain stop
  double before[NW];   // the integer partial sum before it, and at it
  double at[NW];
  double last[NW];     // the integer partial sum at the wave's last term
  SeqSum result;
};

// wave_seq_sum_wide by a whole workgroup of NW waves: a step covers NW * 1024 terms, wave w
// the w-th 1024. The waves' integer increments are added in wave order (exact, as in one
// wave); a tie needs the parity of the running sum before it, so when a step holds a tie the
// waves' parity maps are composed in wave order (a wave without ties just XORs its terms'
// low bits: one ballot). The step's first event, from the first wave that has one, decides
// as in one wave. Three barriers per step, four with a tie. Same contract as
// wave_seq_sum_wide; every thread of the workgroup calls it and gets the result.
template <int NW, class In, class Out>
__device__ __forceinline__ SeqSum block_seq_sum_wide(In t, int n, Out out, bool has_out, double stop_at,
                                                     bool settle, SeqScratch<NW> &sc) {
  constexpr int kPer = 16, kStep = kWaveSize * kPer, kBlockStep = NW * kStep;
  const int lane = wave_lane(), w = (int)(threadIdx.x >> 6);
  if (n <= kSeqShort) {
    if (w == 0) {
      const SeqSum r = lane_seq_sum(t, n, out, has_out, stop_at);
      if (lane == 0) sc.result = r;
    }
    __syncthreads();
    const SeqSum r = sc.result;
    __syncthreads();  // sc is free again when the call returns
    return r;
  }
  double P = t[0];
  if (has_out && threadIdx.x == 0) out[0] = P;
  if (P >= stop_at) return {P, 1};
  int a = 1;
  while (a < n) {
    const int E = ((int)((uint64_t)__double_as_longlong(P) >> 52) & 0x7ff) - 1023;
    const double u = __longlong_as_double((long long)((uint64_t)(E - 52 + 1023) << 52));
    const double scale = __longlong_as_double((long long)((uint64_t)(52 - E + 1023) << 52));
    const double m = P * scale;
    const int wfirst = a + w * kStep;
    const int first = wfirst + lane * kPer;
    double q[kPer], r[kPer];
    uint32_t tie_bits = 0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      q[i] = (first + i < n ? t[first + i] : 0.0) * scale;
      r[i] = __builtin_rint(q[i]);
      if (q[i] < kTwo52 && __builtin_fabs(r[i] - q[i]) == 0.5) tie_bits |= 1u << i;
    }
    const bool wtie = __ballot(tie_bits != 0u) != 0ull;
    uint32_t lane_map = kParityId, excl = kParityId, wave_map;
    if (wtie) {
#pragma unroll
      for (int i = 0; i < kPer; ++i)
        lane_map = parity_then(lane_map, ((tie_bits >> i) & 1u) ? 0u : 1u | (low_bit(r[i]) << 1));
      excl = parity_exclusive_scan(lane_map);
      wave_map = (uint32_t)__builtin_amdgcn_readlane((int)parity_then(excl, lane_map), kWaveSize - 1);
    } else {
      uint32_t par = 0u;
#pragma unroll
      for (int i = 0; i < kPer; ++i) par ^= low_bit(r[i]);
      wave_map = 1u | ((uint32_t)(__popcll(__ballot(par != 0u)) & 1) << 1);  // x -> x ^ parity
    }
    auto totals = [&](double (&pre)[kPer], double &run, double &incl) {
      run = 0.0;
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        run += r[i];
        pre[i] = run;
      }
      incl = wave_inclusive_scan(run);
    };
    double pre[kPer], run, incl;
    totals(pre, run, incl);
    if (lane == 0) {
      sc.map[w] = wave_map;
      sc.tie[w] = wtie ? 1u : 0u;
    }
    if (lane == kWaveSize - 1) sc.total[w] = incl;
    __syncthreads();
    bool any_tie = false;
#pragma unroll
    for (int k = 0; k < NW; ++k) any_tie |= sc.tie[k] != 0u;
    if (any_tie) {
      if (wtie) {
        uint32_t prefix = kParityId;
        for (int k = 0; k < w; ++k) prefix = parity_then(prefix, sc.map[k]);
        uint32_t parity = parity_apply(parity_then(prefix, excl), low_bit(m));
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
          if ((tie_bits >> i) & 1u) {
            const double fl = q[i] - 0.5;
            r[i] = fl + (double)(parity ^ low_bit(fl));
            parity = 0u;
          } else {
            parity ^= low_bit(r[i]);
          }
        }
        totals(pre, run, incl);
      }
      __syncthreads();  // every wave has read the first totals
      if (lane == kWaveSize - 1) sc.total[w] = incl;
      __syncthreads();
    }
    double wave_prefix = 0.0;
    for (int k = 0; k < w; ++k) wave_prefix += sc.total[k];
    double below = row_shift_up<1>(incl);
    const double i15 = lane_f64(incl, 15), i31 = lane_f64(incl, 31), i47 = lane_f64(incl, 47);
    if (lane == 16) below = i15;
    if (lane == 32) below = i31;
    if (lane == 48) below = i47;
    const double base = m + wave_prefix + below;
    const int last_i = min(kPer, n - first) - 1;
    const double cum_end = base + run;
    int my_first = kPer;
    bool my_stop = false;
    if (last_i >= 0 && (cum_end >= kTwo53 || cum_end * u >= stop_at)) {
#pragma unroll
      for (int i = kPer - 1; i >= 0; --i) {
        const double cum = base + pre[i];
        if (i <= last_i && (cum >= kTwo53 || cum * u >= stop_at)) {
          my_first = i;
          my_stop = cum < kTwo53;
        }
      }
    }
    const uint64_t has = __ballot(my_first < kPer);
    const int Lf = has ? __ffsll((unsigned long long)has) - 1 : kWaveSize;
    const int fi = Lf < kWaveSize ? __builtin_amdgcn_readlane(my_first, Lf) : 0;
    double before_mine = 0.0, at_mine = 0.0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      if (i == fi) {
        before_mine = i == 0 ? base : base + pre[i - 1];
        at_mine = base + pre[i];
      }
    }
    const int wlast = min(n, wfirst + kStep) - 1;  // the wave's last term (< wfirst: none)
    const int ll = wlast >= wfirst ? (wlast - wfirst) / kPer : 0;
    const double last_cum = lane_f64(cum_end, ll);
    if (Lf < kWaveSize) {
      const double bf = lane_f64(before_mine, Lf), at = lane_f64(at_mine, Lf);
      const int st = __builtin_amdgcn_readlane((int)my_stop, Lf);
      if (lane == 0) {
        sc.flag[w] = wfirst + Lf * kPer + fi;
        sc.stop[w] = (uint32_t)st;
        sc.before[w] = bf;
        sc.at[w] = at;
      }
    } else if (lane == 0) {
      sc.flag[w] = n;
    }
    if (lane == 0) sc.last[w] = last_cum;
    __syncthreads();
    int flagged = n, fw = 0;
    for (int k = NW - 1; k >= 0; --k) {
      if (sc.flag[k] < n) {
        flagged = sc.flag[k];
        fw = k;
      }
    }
    if (has_out) {
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int j = first + i;
        if (j < n && j < flagged) out[j] = (base + pre[i]) * u;
      }
    }
    if (flagged >= n) {
      const int last = min(n, a + kBlockStep) - 1;
      P = sc.last[(last - a) / kStep] * u;  // the wave holding the step's last term
      const bool settled = settle && !has_out && t[last] * scale < 0.5;
      a = last + 1;
      __syncthreads();  // sc is reused by the next step
      if (settled) return {P, n};
      continue;
    }
    const bool is_stop = sc.stop[fw] != 0u;
    const double before = sc.before[fw], at = sc.at[fw];
    // The event term is read by every wave before the barrier: with out == t, thread 0
    // overwrites it with the partial sum right after.
    const double t_flagged = is_stop ? 0.0 : t[flagged];
    __syncthreads();  // sc is reused by the next step; every wave holds t[flagged]
    if (is_stop) {
      const double v = at * u;
      if (has_out && threadIdx.x == 0) out[flagged] = v;
      return {v, flagged + 1};
    }
    P = before * u + t_flagged;
    if (has_out && threadIdx.x == 0) out[flagged] = P;
    if (P >= stop_at) return {P, flagged + 1};
    a = flagged + 1;
  }
  return {P, n};
}

}  // namespace tabby
