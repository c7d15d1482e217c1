// Lane sums within aligned groups of a 64-lane wavefront by DPP (data-parallel primitives: the VALU reads another
// lane of its own row of 16 in the same instruction), instead of LDS permutes, whose round trip through the LDS
// unit puts a memory wait between every two steps of a reduction.
//   quad_perm [1,0,3,2] = lane ^ 1, quad_perm [2,3,0,1] = lane ^ 2 (within each quad);
//   row_half_mirror: lane l of each 8 reads lane 7 - l (the other quad of the 8), so after the quad sums it
//   completes an 8-lane sum; row_mirror: lane l of each 16 reads lane 15 - l (the other 8);
//   row_ror:8 = lane ^ 8 within each row of 16.
// Lanes 16 and 32 apart are in other DPP rows and still go through __shfl_xor.
#pragma once

#include <hip/hip_runtime.h>

namespace ews {
namespace lanes {

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
// sum over the 64 lanes (every lane returns it)
__device__ __forceinline__ double sum64(double v) {
  v = sum8(v);
  v += dpp<kMirror>(v);
  v += __shfl_xor(v, 16, 64);
  return v + __shfl_xor(v, 32, 64);
}

// sum over lanes l, l ^ 8, l ^ 16, l ^ 32 (the same lane of each group of 8)
__device__ __forceinline__ float colsum8(float v) {
  v += dpp<kXor8>(v);
  v += __shfl_xor(v, 16, 64);
  return v + __shfl_xor(v, 32, 64);
}
// sum over each aligned group of n lanes, n a power of two up to 64
__device__ __forceinline__ float sum_n(float v, int n) {
  if (n >= 2) v += dpp<kXor1>(v);
  if (n >= 4) v += dpp<kXor2>(v);
  if (n >= 8) v += dpp<kHalfMirror>(v);
  if (n >= 16) v += dpp<kMirror>(v);
  if (n >= 32) v += __shfl_xor(v, 16, 64);
  if (n >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

}  // namespace lanes
}  // namespace ews
