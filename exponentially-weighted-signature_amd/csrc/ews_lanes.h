// Lane sums within aligned groups of a 64-lane wavefront by DPP (data-parallel primitives: the VALU reads another
// lane of its own row of 16 in the same instruction), instead of LDS permutes, whose round trip through the LDS
// unit puts a memory wait between every two steps of a reduction.
//   quad_perm [1,0,3,2] = lane ^ 1, quad_perm [2,3,0,1] = lane ^ 2 (within each quad);
//   row_half_mirror: lane l of each 8 reads lane 7 - l (the other quad of the 8), so after the quad sums it
//   completes an 8-lane sum; row_mirror: lane l of each 16 reads lane 15 - l (the other 8);
//   row_ror:8 = lane ^ 8 within each row of 16.
// Lanes 16 and 32 apart are in other DPP rows: v_permlane16_swap / v_permlane32_swap (VALU ops) exchange the odd
// 16-lane rows of one copy with the even rows of another (the wavefront's halves), so that a copy swapped with
// itself yields each lane's value and its partner's.
#pragma once

#include <hip/hip_runtime.h>

namespace ews {
namespace lanes {

// v[l] + v[l ^ 16], v[l] + v[l ^ 32] in every lane
__device__ __forceinline__ float add_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
constexpr int kXor1 = 0xB1, kXor2 = 0x4E, kHalfMirror = 0x141, kMirror = 0x140, kXor8 = 0x128;

// sum over each aligned group of 2, 4, 8, 16 lanes; every lane returns its group's sum
__device__ __forceinline__ float sum2(float v) { return v + dpp<kXor1>(v); }
__device__ __forceinline__ float sum4(float v) {
  v += dpp<kXor1>(v);
  return v + dpp<kXor2>(v);
}
__device__ __forceinline__ float sum8(float v) {
  v = sum4(v);
  return v + dpp<kHalfMirror>(v);
}
__device__ __forceinline__ float sum16(float v) {
  v = sum8(v);
  return v + dpp<kMirror>(v);
}
__device__ __forceinline__ float sum64(float v) { return add_xor32(add_xor16(sum16(v))); }
// float64: the two 32-bit halves moved by the same DPP control
template <int CTRL>
__device__ __forceinline__ double dpp(double v) {
  const unsigned long long x = (unsigned long long)__double_as_longlong(v);
  const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)x, CTRL, 0xf, 0xf, false);
  const unsigned hi = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)(x >> 32), CTRL, 0xf, 0xf, false);
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
__device__ __forceinline__ double sum8(double v) {
  v += dpp<kXor1>(v);
  v += dpp<kXor2>(v);
  return v + dpp<kHalfMirror>(v);
}
// float64 lane exchanges 16 and 32 apart: both halves swapped
__device__ __forceinline__ double add_xor16(double v) {
  const unsigned long long x = (unsigned long long)__double_as_longlong(v);
  const auto lo = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
  const auto hi = __builtin_amdgcn_permlane16_swap((unsigned)(x >> 32), (unsigned)(x >> 32), false, false);
  return __longlong_as_double((long long)(((unsigned long long)hi[0] << 32) | lo[0])) +
         __longlong_as_double((long long)(((unsigned long long)hi[1] << 32) | lo[1]));
}
__device__ __forceinline__ double add_xor32(double v) {
  const unsigned long long x = (unsigned long long)__double_as_longlong(v);
  const auto lo = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
  const auto hi = __builtin_amdgcn_permlane32_swap((unsigned)(x >> 32), (unsigned)(x >> 32), false, false);
  return __longlong_as_double((long long)(((unsigned long long)hi[0] << 32) | lo[0])) +
         __longlong_as_double((long long)(((unsigned long long)hi[1] << 32) | lo[1]));
}
// sum over the 64 lanes (every lane returns it)
__device__ __forceinline__ double sum64(double v) {
  v = sum8(v);
  v += dpp<kMirror>(v);
  v = add_xor16(v);
  return add_xor32(v);
}

// sum over lanes l, l ^ 8, l ^ 16, l ^ 32 (the same lane of each group of 8)
__device__ __forceinline__ float colsum8(float v) {
  v += dpp<kXor8>(v);
  v = add_xor16(v);
  return add_xor32(v);
}
// sum over each aligned group of n lanes, n a power of two up to 64
__device__ __forceinline__ float sum_n(float v, int n) {
  if (n >= 2) v += dpp<kXor1>(v);
  if (n >= 4) v += dpp<kXor2>(v);
  if (n >= 8) v += dpp<kHalfMirror>(v);
  if (n >= 16) v += dpp<kMirror>(v);
  if (n >= 32) v = add_xor16(v);
  if (n >= 64) v = add_xor32(v);
  return v;
}

}  // namespace lanes
}  // namespace ews
