// common.h — device helpers and error plumbing shared by the library's
// HIP sources (the selective scan and the causal conv).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "../../include/selectssm.h"

namespace ssm {

constexpr float kLog2e = 1.4426950408889634f;

// Error state of the calling thread (ssm_last_error) and helpers that set it.
extern thread_local std::string g_last_error;
int fail(int code, const std::string& msg);
int hip_check(hipError_t e, const char* what);

// ---------------------------------------------------------------- element I/O

struct bf16 {
  uint16_t bits;
};

template <typename T>
__device__ __forceinline__ float ld(const T* p, int64_t i);
template <>
__device__ __forceinline__ float ld<float>(const float* p, int64_t i) {
  return p[i];
}
template <>
__device__ __forceinline__ float ld<bf16>(const bf16* p, int64_t i) {
  return __uint_as_float(static_cast<uint32_t>(p[i].bits) << 16);
}

// Element `off` of a (wave-uniform) base pointer, addressed with a 32-bit byte
// offset so the load is one SGPR-base + VGPR-offset instruction (the host
// keeps every per-batch-row byte offset below 2^32).
template <typename T>
__device__ __forceinline__ float ld32(const T* base, uint32_t off) {
  const uint32_t byte = off * (uint32_t)sizeof(T);
  return ld(reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + byte), 0);
}

template <typename T>
__device__ __forceinline__ void st(T* p, int64_t i, float v);
template <>
__device__ __forceinline__ void st<float>(float* p, int64_t i, float v) {
  p[i] = v;
}
template <>
__device__ __forceinline__ void st<bf16>(bf16* p, int64_t i, float v) {
  // round to nearest even; NaN stays a quiet NaN
  uint32_t x = __float_as_uint(v);
  uint16_t r;
  if ((x & 0x7fffffffu) > 0x7f800000u) {
    r = static_cast<uint16_t>((x >> 16) | 0x40u);
  } else {
    x += 0x7fffu + ((x >> 16) & 1u);
    r = static_cast<uint16_t>(x >> 16);
  }
  p[i].bits = r;
}

// store counterpart of ld32
template <typename T>
__device__ __forceinline__ void st32(T* base, uint32_t off, float v) {
  const uint32_t byte = off * (uint32_t)sizeof(T);
  st(reinterpret_cast<T*>(reinterpret_cast<char*>(base) + byte), 0, v);
}

// Runs f() on the lanes whose channel exists.  A workgroup whose 64 channels
// all exist (every one when D % 64 == 0) takes a wave-uniform branch and needs
// no per-lane exec masking.
template <typename F>
__device__ __forceinline__ void on_valid_lanes(bool full_block, bool valid, F&& f) {
  if (full_block) {
    f();
  } else if (valid) {
    f();
  }
}

// Whether v holds on any lane of a workgroup of NW waves, with the barrier
// included: each wave's vote goes to its slot of flags (NW ints of LDS), then
// every lane reads all slots.  A caller that votes again before the next
// barrier passes the other half of a double buffer.
template <int NW>
__device__ __forceinline__ bool barrier_any(bool v, int* flags) {
  const bool w = __ballot(v) != 0;
  if ((threadIdx.x & 63) == 0) flags[threadIdx.x >> 6] = w;
  __syncthreads();
  int any = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) any |= flags[i];
  return any != 0;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// 1 / (1 + e^-x): one v_exp_f32 and one v_rcp_f32 (both about 1 ulp)
__device__ __forceinline__ float sigmoid(float x) {
  return fast_rcp(1.0f + fast_exp2(-x * kLog2e));
}

// log(1 + y) for y >= 0 as log(u) * y / (u - 1) with u = fl(1 + y): the
// rounding of 1 + y cancels in the ratio (Goldberg, "What every computer
// scientist should know about floating-point arithmetic", 1991, Theorem 4);
// log(u) is v_log_f32 (log2) times ln 2
__device__ __forceinline__ float log1p_nonneg(float y) {
  constexpr float kLn2 = 0.6931471805599453f;
  const float u = 1.0f + y;
  const float d = u - 1.0f;
  return d == 0.0f ? y : __builtin_amdgcn_logf(u) * kLn2 * (y * fast_rcp(d));
}

// softplus(x) = log(1 + e^x) = max(x, 0) + log1p(e^-|x|), as jax.nn.softplus
// (logaddexp(x, 0)) defines it
__device__ __forceinline__ float softplus(float x) {
  return fmaxf(x, 0.0f) + log1p_nonneg(fast_exp2(-fabsf(x) * kLog2e));
}

// ------------------------------------------------------ cross-lane reductions

template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum of v over the 16 lanes of each row; every lane of the row gets it.
__device__ __forceinline__ float row_sum16(float v) {
  v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_move<0x141>(v);  // row_half_mirror
  v += dpp_move<0x140>(v);  // row_mirror
  return v;
}

// Sum of v over the 32 lanes of each wave half; every lane of the half gets it.
__device__ __forceinline__ float half_sum32(float v) {
  v = row_sum16(v);
  auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

// Lanes l and l^32 hold the two halves of one channel's sum: the result is a
// summed over the halves in lanes < 32 and b summed over the halves in lanes >= 32.
__device__ __forceinline__ float half_pair(float a, float b) {
  auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

// Eight per-lane values, each summed over the 32 lanes of its wave half: 16
// totals per wave.  Lane l ends with the total of x[reduce32x8_value(l)] over
// half reduce32x8_half(l); the 4 lanes of each aligned quad hold the same one.
__device__ __forceinline__ float reduce32x8(const float (&x)[8]) {
  float p[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {  // rows 0..3 keep x[2m], x[2m+1] of half 0, x[2m], x[2m+1] of half 1
    auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(x[2 * m]), __float_as_uint(x[2 * m + 1]), false, false);
    p[m] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  const int lid = __lane_id();
  const bool b3 = (lid & 8) != 0;
  const bool b2 = (lid & 4) != 0;
  float q[2];
#pragma unroll
  for (int m = 0; m < 2; ++m) {  // lanes with bit 3 clear keep p[2m], set keep p[2m+1]
    const float keep = b3 ? p[2 * m + 1] : p[2 * m];
    const float give = b3 ? p[2 * m] : p[2 * m + 1];
    q[m] = keep + dpp_move<0x128>(give);  // row_ror:8
  }
  const float keep = b2 ? q[1] : q[0];    // bit 2 clear keeps q[0], set keeps q[1]
  const float give = b2 ? q[0] : q[1];
  float r = keep + dpp_move<0x141>(give);  // row_half_mirror
  r += dpp_move<0xB1>(r);                  // quad_perm [1,0,3,2]
  r += dpp_move<0x4E>(r);                  // quad_perm [2,3,0,1]
  return r;
}
__device__ __forceinline__ int reduce32x8_value(int lane) {
  return 4 * ((lane >> 2) & 1) + 2 * ((lane >> 3) & 1) + ((lane >> 4) & 1);
}
__device__ __forceinline__ int reduce32x8_half(int lane) { return lane >> 5; }

}  // namespace ssm
