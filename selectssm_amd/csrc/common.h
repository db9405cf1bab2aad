// common.h — device helpers and error plumbing shared by the library's
// HIP sources (the selective scan and the causal conv).
#pragma once

#include <hip/hip_runtime.h>
#include <rocprofiler-sdk-roctx/roctx.h>

#include <cstdint>
#include <string>

#include "../../include/selectssm.h"

namespace ssm {

constexpr float kLog2e = 1.4426950408889634f;

// A roctx range over one C-ABI call (named after the entry point), so a
// rocprofv3 --marker-trace run attributes every kernel to the call that
// launched it.  Without a profiler attached the push and pop do nothing.
struct ApiRange {
  explicit ApiRange(const char* name) { roctxRangePushA(name); }
  ~ApiRange() { roctxRangePop(); }
  ApiRange(const ApiRange&) = delete;
  ApiRange& operator=(const ApiRange&) = delete;
};

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

template <typename T>
__device__ __forceinline__ void st(T* p, int64_t i, float v);
template <>
__device__ __forceinline__ void st<float>(float* p, int64_t i, float v) {
  p[i] = v;
}
template <>
__device__ __forceinline__ void st<bf16>(bf16* p, int64_t i, float v) {
  // one v_cvt_pk_bf16_f32: round to nearest even, denormals kept, NaN stays a
  // quiet NaN.  Checked on gfx950 against the integer form of that rounding
  // (x + 0x7fff + bit 16, NaN -> x >> 16 | 0x40) for all 2^32 inputs: equal
  // apart from NaN payloads.
  p[i].bits = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
}

// Element `off` of a (wave-uniform) base pointer, addressed with a 32-bit
// byte offset so the store is one SGPR-base + VGPR-offset instruction (the
// host keeps every per-batch-row byte offset below 2^32).
template <typename T>
__device__ __forceinline__ void st32(T* base, uint32_t off, float v) {
  const uint32_t byte = off * (uint32_t)sizeof(T);
  st(reinterpret_cast<T*>(reinterpret_cast<char*>(base) + byte), 0, v);
}

// A tensor base (one batch row) addressed with two 32-bit byte offsets: a
// per-lane one fixed for the kernel and a wave-uniform one (row arithmetic
// on scalars).  Their sum is one vector add, and the access is one
// global_load/store with the base in SGPRs and the sum as its unsigned
// 32-bit offset, so no per-access 64-bit address math; the host keeps every
// per-batch-row extent at or below 4 GiB.
struct buf_t {
  const char* p;
};
__device__ __forceinline__ buf_t make_buf(const void* p) { return buf_t{static_cast<const char*>(p)}; }
template <typename T>
__device__ __forceinline__ float bld(buf_t r, uint32_t voff, uint32_t soff) {
  return ld(reinterpret_cast<const T*>(r.p + (voff + soff)), 0);
}
// A staged element: what a tile's fetch loads and the later commit converts
// (val).  bf16 keeps its raw 16 bits in the register until then: widening
// them next to the load would put the load's wait there, in front of the
// tile's compute, instead of at the commit after it.
template <typename T>
struct stg;
template <>
struct stg<float> {
  float v;
};
template <>
struct stg<bf16> {
  uint16_t v;
};
template <typename T>
__device__ __forceinline__ stg<T> bldr(buf_t r, uint32_t voff, uint32_t soff);
template <>
__device__ __forceinline__ stg<float> bldr<float>(buf_t r, uint32_t voff, uint32_t soff) {
  return stg<float>{*reinterpret_cast<const float*>(r.p + (voff + soff))};
}
template <>
__device__ __forceinline__ stg<bf16> bldr<bf16>(buf_t r, uint32_t voff, uint32_t soff) {
  return stg<bf16>{*reinterpret_cast<const uint16_t*>(r.p + (voff + soff))};
}
// element `off` of a (wave-uniform) base pointer, staged
template <typename T>
__device__ __forceinline__ stg<T> ld32r(const T* base, uint32_t off) {
  return bldr<T>(make_buf(base), off * (uint32_t)sizeof(T), 0);
}
__device__ __forceinline__ float val(stg<float> s) { return s.v; }
__device__ __forceinline__ float val(stg<bf16> s) { return __uint_as_float(static_cast<uint32_t>(s.v) << 16); }
// four consecutive elements, staged (16-byte aligned for f32, 8-byte for bf16)
template <typename T>
struct stg4;
template <>
struct stg4<float> {
  float4 v;
};
template <>
struct stg4<bf16> {
  uint2 v;
};
template <typename T>
__device__ __forceinline__ stg4<T> bld4r(buf_t r, uint32_t voff, uint32_t soff) {
  if constexpr (sizeof(T) == 4) {
    return stg4<T>{*reinterpret_cast<const float4*>(r.p + (voff + soff))};
  } else {
    return stg4<T>{*reinterpret_cast<const uint2*>(r.p + (voff + soff))};
  }
}
__device__ __forceinline__ float4 val(stg4<float> s) { return s.v; }
__device__ __forceinline__ float4 val(stg4<bf16> s) {
  return make_float4(__uint_as_float(s.v.x << 16), __uint_as_float(s.v.x & 0xffff0000u), __uint_as_float(s.v.y << 16),
                     __uint_as_float(s.v.y & 0xffff0000u));
}

template <typename T>
__device__ __forceinline__ void bst(buf_t r, uint32_t voff, uint32_t soff, float v) {
  st(reinterpret_cast<T*>(const_cast<char*>(r.p) + (voff + soff)), 0, v);
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

// The bitwise OR over the NW waves of a workgroup of a wave-uniform int v,
// barrier and slots as in barrier_any.
template <int NW>
__device__ __forceinline__ int barrier_or(int v, int* flags) {
  if ((threadIdx.x & 63) == 0) flags[threadIdx.x >> 6] = v;
  __syncthreads();
  int any = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) any |= flags[i];
  return any;
}

// Keeps v computed at this point of the program: an empty asm statement that
// reads and writes v in a VGPR and emits no instruction.  Arithmetic feeding
// it cannot be moved past it, so a walk whose results are used only after a
// long unrolled loop stays step by step, next to its LDS reads, instead of
// being gathered after the loop (which held every step's operands in
// registers at once).
__device__ __forceinline__ void pin(float& v) { asm volatile("" : "+v"(v)); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// 1 / (1 + e^-x): one v_exp_f32 and one v_rcp_f32 (both about 1 ulp)
__device__ __forceinline__ float sigmoid(float x) {
  return fast_rcp(1.0f + fast_exp2(-x * kLog2e));
}

// softplus(x) = log(1 + e^x) = max(x, 0) + log1p(e), e = e^-|x|, as
// jax.nn.softplus (logaddexp(x, 0)) defines it.  With u = fl(1 + e),
// log1p(e) = log(u) + log(1 + d / u) for d = e - (u - 1), which is exact
// (u - 1 is exact for u in [1, 2]; then e and u - 1 are within a factor 2 of
// each other, or u = 1 and d = e).  |d| <= 2^-24 u, so log(1 + d / u) is d / u
// to within 2^-48; softplus takes d itself for d / u (an error of at most
// |d| e / u, under 1.5 ulp of log1p(e)), softplus_sigmoid multiplies by the
// 1 / u it needs anyway.  log(u) is v_log_f32 (log2) times ln 2.
constexpr float kLn2 = 0.6931471805599453f;
__device__ __forceinline__ float softplus(float x) {
  const float e = fast_exp2(-fabsf(x) * kLog2e);
  const float u = 1.0f + e;
  return fmaxf(x, 0.0f) + fmaf(__builtin_amdgcn_logf(u), kLn2, e - (u - 1.0f));
}

// softplus(x) and its derivative sigmoid(x) (into *sg) from one exp and one
// rcp: sigmoid(x) = 1 / u for x >= 0 and e / u below
__device__ __forceinline__ float softplus_sigmoid(float x, float* sg) {
  const float e = fast_exp2(-fabsf(x) * kLog2e);
  const float u = 1.0f + e;
  const float r = fast_rcp(u);
  *sg = x >= 0.0f ? r : e * r;
  return fmaxf(x, 0.0f) + fmaf(__builtin_amdgcn_logf(u), kLn2, (e - (u - 1.0f)) * r);
}

// ------------------------------------------------------ cross-lane reductions
//
// DPP patterns used below (all within a row of 16 lanes, every lane has a source):
//   row_newbcast:k (0x150+k) lane k of the row
//   row_ror:8 (0x128)        lane ^ 8
//   row_half_mirror (0x141)  lane ^ 7 within each group of 8
//   quad_perm [2,3,0,1]      lane ^ 2
//   quad_perm [1,0,3,2]      lane ^ 1

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, true));
}

// Lane k of each row of 16 lanes, broadcast to its row (DPP row_newbcast:k,
// 0x150 + k, gfx90a and later).  k must be a constant after unrolling; the
// switch then folds to one case.  A broadcast feeding a multiply becomes the
// multiply's DPP operand (v_mul_f32_dpp), so it costs no instruction.
__device__ __forceinline__ float row_bcast(float v, int k) {
  switch (k & 15) {
    case 0: return dpp_mov<0x150>(v);
    case 1: return dpp_mov<0x151>(v);
    case 2: return dpp_mov<0x152>(v);
    case 3: return dpp_mov<0x153>(v);
    case 4: return dpp_mov<0x154>(v);
    case 5: return dpp_mov<0x155>(v);
    case 6: return dpp_mov<0x156>(v);
    case 7: return dpp_mov<0x157>(v);
    case 8: return dpp_mov<0x158>(v);
    case 9: return dpp_mov<0x159>(v);
    case 10: return dpp_mov<0x15A>(v);
    case 11: return dpp_mov<0x15B>(v);
    case 12: return dpp_mov<0x15C>(v);
    case 13: return dpp_mov<0x15D>(v);
    case 14: return dpp_mov<0x15E>(v);
    default: return dpp_mov<0x15F>(v);
  }
}
constexpr int kDppRor8 = 0x128;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppXor2 = 0x4E;
constexpr int kDppXor1 = 0xB1;

// Lanes l and l ^ 32 hold parts of the same sums: the result is a summed over
// both in lanes < 32 and b summed over both in lanes >= 32.
__device__ __forceinline__ float half_pair(float a, float b) {
  auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

// Rows r and r ^ 1 (16 lanes each) hold parts of the same sums: rows 0 and 2
// get a summed over their row pair, rows 1 and 3 get b summed over theirs.
__device__ __forceinline__ float row_pair(float a, float b) {
  auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

// Four per-lane values (consecutive steps 0..3), each summed over the 4 rows
// of the wave: row r ends with step yrow_step(r) (rows hold 0, 2, 1, 3).
__device__ __forceinline__ float rows_transpose_sum4(float y0, float y1, float y2, float y3) {
  return row_pair(half_pair(y0, y1), half_pair(y2, y3));
}
__device__ __forceinline__ int yrow_step(int row) { return ((row & 1) << 1) | (row >> 1); }

// Sum over the 8 lanes c = lane & 7 of each half-row, of S per-lane values
// whose state order is permuted by the lane: x[j] holds state j ^ sig with
// sig = chan_sig<S>(c).  Pairing lanes whose sig differ lets one DPP add
// combine two states (each lane keeps the state its partner sends), so the S
// values cost S - 1 adds before the remaining channel bits are summed plainly.
// The result in lane c is state chan_sig<S>(c) summed over the 8 channels.
//   S = 2: sig = c2.  lane ^ 7 flips sig: x0 + x1'; then plain lane ^ 2, ^ 1.
//   S = 4: sig = (c0 ^ c1 ^ c2) | c2 << 1.  lane ^ 7 flips both bits of sig:
//          x0 + x3', x1 + x2'; lane ^ 1 flips bit 0: r0 + r1'; then plain
//          lane ^ 3, which keeps sig.  The pairings ^7, ^1, ^3 reach all 8.
template <int S>
__device__ __forceinline__ int chan_sig(int c) {
  if constexpr (S == 1) return 0;
  else if constexpr (S == 2) return (c >> 2) & 1;
  else return ((c ^ (c >> 1) ^ (c >> 2)) & 1) | (((c >> 2) & 1) << 1);
}
constexpr int kDppXor3 = 0x1B;  // quad_perm [3,2,1,0]: lane ^ 3
template <int S>
__device__ __forceinline__ float chan_reduce8(const float (&x)[S]) {
  static_assert(S == 1 || S == 2 || S == 4, "1, 2 or 4 states per lane");
  if constexpr (S == 1) {
    float r = x[0] + dpp_mov<kDppHalfMirror>(x[0]);
    r += dpp_mov<kDppXor2>(r);
    return r + dpp_mov<kDppXor1>(r);
  } else if constexpr (S == 2) {
    float r = x[0] + dpp_mov<kDppHalfMirror>(x[1]);
    r += dpp_mov<kDppXor2>(r);
    return r + dpp_mov<kDppXor1>(r);
  } else {
    const float r0 = x[0] + dpp_mov<kDppHalfMirror>(x[3]);
    const float r1 = x[1] + dpp_mov<kDppHalfMirror>(x[2]);
    const float r = r0 + dpp_mov<kDppXor1>(r1);
    return r + dpp_mov<kDppXor3>(r);
  }
}

}  // namespace ssm
