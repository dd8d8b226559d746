// Wavefront (64-lane) reductions for CDNA: DPP moves inside each row of 16
// lanes (a few cycles each, no LDS traffic), then v_readlane of the four row
// results.  Each step adds a lane's value to its partner's, so every lane of
// a row ends with the bitwise same result.  Call with the whole wave active.
#pragma once

#include <hip/hip_runtime.h>

namespace llmhip {

// The wave's index in the workgroup, as a wave-uniform (scalar) value, so that
// per-wave indices and loop bounds derived from it live in SGPRs.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// state[0] (the first position of the pass) through the scalar cache.  The
// state is written only by the sampling and advance kernels, never while a
// kernel that reads it runs, so a constant-memory load is exact; the wait for
// it is then off the vector-load counter, whose waits are in issue order.
__device__ __forceinline__ uint32_t state_pos(const uint32_t* state) {
  return *(const __attribute__((address_space(4))) uint32_t*)state;
}

// n / d by a multiply and a shift, for n < 2^31 and d >= 1 (Granlund and
// Montgomery's round-up method, "Division by invariant integers using
// multiplication", 1994): with l = ceil(log2 d) and
// m = floor(2^32 (2^l - d) / d) + 1, n / d = (umulhi(n, m) + n) >> l.
// A runtime division costs a long instruction sequence at a kernel's start.
struct FastDiv {
  uint32_t d, mul, sh;
};
inline FastDiv fast_div(uint32_t d) {
  if (d == 0) return FastDiv{0, 0, 0};  // no divisor: callers check their divisors first
  uint32_t l = 0;
  while ((1ull << l) < d) l++;
  return FastDiv{d, (uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1), l};
}
__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) { return (__umulhi(n, f.mul) + n) >> f.sh; }

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

constexpr int DPP_XOR1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141; // lane i <- 7-i within 8
constexpr int DPP_MIRROR = 0x140;      // lane i <- 15-i within 16

// sum over the 16 lanes of each row, in every lane of the row
__device__ __forceinline__ float row_sum16(float x) {
  x += dpp_mov<DPP_XOR1>(x);
  x += dpp_mov<DPP_XOR2>(x);
  x += dpp_mov<DPP_HALF_MIRROR>(x);
  x += dpp_mov<DPP_MIRROR>(x);
  return x;
}

__device__ __forceinline__ float row_max16(float x) {
  x = fmaxf(x, dpp_mov<DPP_XOR1>(x));
  x = fmaxf(x, dpp_mov<DPP_XOR2>(x));
  x = fmaxf(x, dpp_mov<DPP_HALF_MIRROR>(x));
  x = fmaxf(x, dpp_mov<DPP_MIRROR>(x));
  return x;
}

// x from lane ^ 16 and lane ^ 32, by gfx950's row swaps (VALU) instead of
// LDS permutes: v_permlane16_swap(x, x) leaves row r's partner row in the
// second result for even rows and in the first for odd rows;
// v_permlane32_swap likewise for the two halves of the wave.
__device__ __forceinline__ float xor16(float x, int lane) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __uint_as_float(((lane >> 4) & 1) ? r[0] : r[1]);
}
__device__ __forceinline__ float xor32(float x, int lane) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(lane < 32 ? r[1] : r[0]);
}

__device__ __forceinline__ float lane_value(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

// x equal across each row of 16 lanes -> the sum / max of the four rows (wave-uniform)
__device__ __forceinline__ float rows_sum4(float x) {
  return (lane_value(x, 0) + lane_value(x, 16)) + (lane_value(x, 32) + lane_value(x, 48));
}

__device__ __forceinline__ float rows_max4(float x) {
  return fmaxf(fmaxf(lane_value(x, 0), lane_value(x, 16)), fmaxf(lane_value(x, 32), lane_value(x, 48)));
}

}  // namespace llmhip
