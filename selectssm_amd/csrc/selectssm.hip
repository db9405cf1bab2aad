// selectssm.hip — selective-scan forward/backward for MI355X (gfx950, CDNA4).
//
// Work decomposition (both kernels)
//   * lane = channel d: the 64 lanes of a wave hold 64 consecutive channels,
//     so u / delta / dy / y rows ((B,L,D) row-major) are read and written as
//     coalesced 256-byte wave accesses and the sum over N (y, du, ddelta)
//     never crosses lanes;
//   * wave = NPW of the N states: the NG = ceil(N/NPW) waves of a workgroup
//     hold all states of a 64-channel block, and partial sums over states are
//     combined through LDS;
//   * workgroup = (channel block, batch row); time runs sequentially inside
//     the workgroup, so there is no carry exchange between workgroups.
//   B_t,n and C_t,n are wave-uniform (scalar loads); A[d,n] lives in VGPRs
//   pre-scaled by log2(e) so the decay is one v_exp_f32 of one product.
//
// Backward = the custom-VJP adjoint of ssmrecscan.py:150-160 with the
// recursive storage of ssmrecscan.py:111-148 replaced by checkpoints: the
// forward stores h entering every CK-step block; the backward walks blocks in
// reverse, recomputes a_t and h_{t-1} of the block into registers, then runs
// the adjoint f_t = C_t dy_t + a_{t+1} f_{t+1} backwards through the block.
// Sums over channels (dB, dC) are reduced across the wave with v_permlane32/16
// swaps + DPP, then across workgroups in fixed order (deterministic).

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>
#include <type_traits>

#include "../../include/selectssm.h"

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWave = 64;
// checkpoint interval = backward block length (8 only where 16 would not fit in LDS)
__host__ __device__ constexpr int ck_for(int ng, bool epi) { return (ng >= 8 && epi) ? 8 : 16; }
#ifndef SSM_PLAIN_NPW
#define SSM_PLAIN_NPW 2
#endif
constexpr int kPlainNPW = SSM_PLAIN_NPW;  // states per wave of the plain scan
constexpr int kPF = 4;    // steps of LDS read-ahead for B, C
constexpr int kTT = 32;   // forward time tile staged in LDS (a multiple of kCK)

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

// element at a 32-bit unsigned offset from a (wave-uniform) base pointer
template <typename T>
__device__ __forceinline__ float ld32(const T* base, uint32_t off) {
  return ld(reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + (size_t)off * sizeof(T)), 0);
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

// store at a 32-bit unsigned offset from a (wave-uniform) base pointer
template <typename T>
__device__ __forceinline__ void st32(T* base, uint32_t off, float v) {
  st(reinterpret_cast<T*>(reinterpret_cast<char*>(base) + (size_t)off * sizeof(T)), 0, v);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float sigmoid(float x) {
  return 1.0f / (1.0f + fast_exp2(-x * kLog2e));
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

// Transpose-reduce of four per-lane values over all 64 lanes.  Row k of the
// result holds the total of x[kRowState[k]] in every lane of that row.
__device__ __forceinline__ float wave_reduce4(float x0, float x1, float x2, float x3) {
  auto s01 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x0), __float_as_uint(x1), false, false);
  auto s23 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x2), __float_as_uint(x3), false, false);
  float p0 = __uint_as_float(s01[0]) + __uint_as_float(s01[1]);  // rows 0,1: x0; rows 2,3: x1
  float p1 = __uint_as_float(s23[0]) + __uint_as_float(s23[1]);  // rows 0,1: x2; rows 2,3: x3
  auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(p0), __float_as_uint(p1), false, false);
  float q = __uint_as_float(s[0]) + __uint_as_float(s[1]);  // row0 x0, row1 x2, row2 x1, row3 x3
  return row_sum16(q);
}

// Two per-lane values over all 64 lanes: rows 0,1 hold the total of x0, rows 2,3 of x1.
__device__ __forceinline__ float wave_reduce2(float x0, float x1) {
  auto s01 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x0), __float_as_uint(x1), false, false);
  const float p = __uint_as_float(s01[0]) + __uint_as_float(s01[1]);  // lanes < 32: x0; >= 32: x1
  auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(p), __float_as_uint(p), false, false);
  return row_sum16(__uint_as_float(s[0]) + __uint_as_float(s[1]));
}

// Full sum of one value over the wave (every lane gets it).
__device__ __forceinline__ float wave_sum(float v) {
  v = row_sum16(v);
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// Eight per-lane values over all 64 lanes.  Lane l ends with the total of
// x[wave_reduce8_index(l)]; the 8 lanes of each group of 8 hold the same one.
__device__ __forceinline__ float wave_reduce8(const float (&x)[8]) {
  float p[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {  // lanes < 32 keep x[2m], lanes >= 32 keep x[2m+1]
    auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x[2 * m]), __float_as_uint(x[2 * m + 1]), false, false);
    p[m] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  float q[2];
#pragma unroll
  for (int m = 0; m < 2; ++m) {  // rows 0..3 keep p[2m](r0+r1), p[2m+1](r0+r1), p[2m](r2+r3), p[2m+1](r2+r3)
    auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(p[2 * m]), __float_as_uint(p[2 * m + 1]), false, false);
    q[m] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  // lanes with bit 3 clear keep q[0], set keep q[1]; the partner 8 lanes away adds its copy
  const bool hi = (__lane_id() & 8) != 0;
  const float keep = hi ? q[1] : q[0];
  const float give = hi ? q[0] : q[1];
  float r = keep + dpp_move<0x128>(give);  // row_ror:8
  r += dpp_move<0xB1>(r);                  // quad_perm [1,0,3,2]
  r += dpp_move<0x4E>(r);                  // quad_perm [2,3,0,1]
  r += dpp_move<0x141>(r);                 // row_half_mirror
  return r;
}
__device__ __forceinline__ int wave_reduce8_index(int lane) {
  return 4 * ((lane >> 3) & 1) + ((0x3120 >> (4 * (lane >> 4))) & 0xf);
}

// Sum over the wave of each of the NPW per-lane values.  The totals land in a
// few lanes; wave_reduce_state(lane) names the value a lane holds (-1: none).
template <int NPW>
__device__ __forceinline__ float wave_reduce(const float (&x)[NPW]) {
  if constexpr (NPW == 4) return wave_reduce4(x[0], x[1], x[2], x[3]);
  else if constexpr (NPW == 2) return wave_reduce2(x[0], x[1]);
  else return wave_sum(x[0]);
}
template <int NPW>
__device__ __forceinline__ int wave_reduce_state(int lane) {
  if constexpr (NPW == 4) return (lane & 15) == 0 ? (0x3120 >> (4 * (lane >> 4))) & 0xf : -1;  // rows hold x0,x2,x1,x3
  else if constexpr (NPW == 2) return (lane & 31) == 0 ? lane >> 5 : -1;
  else return lane == 0 ? 0 : -1;
}

// NPW consecutive floats from (16-byte aligned) LDS in one read
template <int NPW>
__device__ __forceinline__ void lds_vec(const float* p, float (&o)[NPW]) {
  if constexpr (NPW == 4) {
    const float4 v = *reinterpret_cast<const float4*>(p);
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
  } else if constexpr (NPW == 2) {
    const float2 v = *reinterpret_cast<const float2*>(p);
    o[0] = v.x; o[1] = v.y;
  } else {
    o[0] = *p;
  }
}

// ------------------------------------------------------------- staged tiles
//
// Each kernel walks time in tiles.  While a tile is being computed from LDS,
// the next tile's inputs are already in flight into registers (fetch), and
// are written to the other LDS buffer after the tile (commit).  Thread
// (wave w, lane c) stages rows i = w, w+NG, ... of a [rows][64] tile, column c,
// so every global access of a wave is one contiguous 64-element row.

// element (scan step t, lane channel d) of a (B,L,D) array, optionally read at
// the mirrored output position (L-1-t, D-1-d); 0 outside the tensor
template <typename T>
__device__ __forceinline__ float ld_at(const T* X, int64_t bLD, int L, int D, int t, int d, bool rev, bool comp) {
  if (t >= L || d >= D) return 0.0f;
  const int r = rev ? L - 1 - t : t;
  const int c = comp ? D - 1 - d : d;
  return ld(X, bLD + (int64_t)r * D + c);
}

// ------------------------------------------------------------------ forward

template <typename T>
struct FwdArgs {
  const T* u;
  const T* delta;
  const float* A;
  const T* Bc;
  const T* Cc;
  const float* Dskip;
  const T* z;
  T* y;
  float* ckpt;
  int L, D, N, nblk;
  int dstride;  // 1, or 0 for a (B,L,1) delta
  uint32_t flags;
};

// NPW states per wave, NG waves per workgroup (NPW*NG >= N), EPI: the skip /
// gate epilogue is fused (its extra staging only exists in EPI builds).
template <int NPW, int NG, bool EPI, typename T>
__global__ void __launch_bounds__(kWave* NG, 1) ssm_fwd_kernel(FwdArgs<T> p) {
  constexpr int kCK = ck_for(NG, EPI);
  static_assert(kTT % kCK == 0, "time tile must hold whole checkpoint blocks");
  constexpr int NS = NG * NPW;                                     // padded state count
  constexpr int RPT = kTT / NG;                                    // staged rows per thread
  constexpr int BCE = (kTT * NS + kWave * NG - 1) / (kWave * NG);  // staged B/C elements per thread
  constexpr int EB = EPI ? 2 : 1;                                  // epilogue staging buffers
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = blockIdx.y;
  const int L = p.L, D = p.D, N = p.N;
  const int d = blockIdx.x * kWave + lane;
  const bool valid = d < D;
  const int dc = valid ? d : 0;
  const int n0 = wave * NPW;
  const bool rev = p.flags & SSM_REVERSE;
  const bool comp = rev && (p.flags & SSM_COMPLEMENT);
  const bool skip = EPI && (p.flags & SSM_SKIP);
  const bool gate = EPI && (p.flags & SSM_GATE);
  const bool stage_eu = skip && rev;  // u at the output position is another element
  const int q = comp ? D - 1 - dc : dc;
  const float Dq = (skip && valid) ? p.Dskip[q] : 0.0f;

  float A2[NPW], h[NPW];
#pragma unroll
  for (int j = 0; j < NPW; ++j) {
    const int n = n0 + j;
    A2[j] = (valid && n < N) ? p.A[(int64_t)dc * N + n] * kLog2e : 0.0f;
    h[j] = 0.0f;
  }

  __shared__ float s_u[2][kTT][kWave], s_dt[2][kTT][kWave];
  __shared__ float s_eu[EB][EPI ? kTT : 1][kWave], s_ez[EB][EPI ? kTT : 1][kWave];
  __shared__ __attribute__((aligned(16))) float s_B[2][kTT][NS];
  __shared__ __attribute__((aligned(16))) float s_C[2][kTT][NS];
  __shared__ float s_y[NG][kTT][kWave];

  const int64_t bLD = (int64_t)b * L * D;
  const int64_t bLN = (int64_t)b * L * N;
  const int dtD = p.dstride ? D : 1;
  const int64_t bLDt = (int64_t)b * L * dtD;
  const int dd_lane = p.dstride ? dc : 0;

  // uniform (b,0,0) bases; rows are added in scalar registers, the lane's
  // channel is the only per-lane offset
  const T* __restrict__ u_b = p.u + bLD;
  const T* __restrict__ dt_b = p.delta + bLDt;
  const T* __restrict__ z_b = EPI ? p.z + bLD : nullptr;
  const T* __restrict__ B_b = p.Bc + bLN;
  const T* __restrict__ C_b = p.Cc + bLN;
  T* __restrict__ y_b = p.y + bLD;
  float* __restrict__ ck_b = p.ckpt != nullptr ? p.ckpt + (int64_t)b * p.nblk * N * D : nullptr;
  const int LN = L * N;
  const int ND = N * D;

  // fetch() only issues loads (clamped addresses, raw values); commit(), run
  // after the tile's compute, zeroes what lies outside the tensor and writes
  // LDS, so the loads' latency is covered by a whole tile.
  float r_u[RPT], r_dt[RPT], r_eu[RPT], r_ez[RPT], r_B[BCE], r_C[BCE];
  auto fetch = [&](int t0) {
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int tc = min(t0 + wave + k * NG, L - 1);
      r_u[k] = ld32(u_b, (uint32_t)(tc * D + dc));
      r_dt[k] = ld32(dt_b, (uint32_t)(tc * dtD + dd_lane));
      if (stage_eu || gate) {
        const int pr = rev ? L - 1 - tc : tc;
        if (stage_eu) r_eu[k] = ld32(u_b, (uint32_t)(pr * D + q));
        if (gate) r_ez[k] = ld32(z_b, (uint32_t)(pr * D + q));
      }
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = threadIdx.x + k * kWave * NG;
      int gi;
      if (NS == N) {
        gi = t0 * N + e;
      } else {
        const int i = e / NS, n = e - i * NS;
        gi = (t0 + i) * N + min(n, N - 1);
      }
      const int gc = min(gi, LN - 1);
      r_B[k] = ld32(B_b, (uint32_t)gc);
      r_C[k] = ld32(C_b, (uint32_t)gc);
    }
  };
  auto commit = [&](int buf, int t0) {
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int i = wave + k * NG;
      const bool in = valid && t0 + i < L;
      s_u[buf][i][lane] = in ? r_u[k] : 0.0f;
      s_dt[buf][i][lane] = in ? r_dt[k] : 0.0f;
      if (stage_eu) s_eu[buf][i][lane] = in ? r_eu[k] : 0.0f;
      if (gate) s_ez[buf][i][lane] = in ? r_ez[k] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = threadIdx.x + k * kWave * NG;
      if (e < kTT * NS) {
        const int i = e / NS, n = e - i * NS;
        const bool in = t0 + i < L && n < N;
        (&s_B[buf][0][0])[e] = in ? r_B[k] : 0.0f;
        (&s_C[buf][0][0])[e] = in ? r_C[k] : 0.0f;
      }
    }
  };

  fetch(0);
  commit(0, 0);
  __syncthreads();
  int buf = 0;
  for (int t0 = 0; t0 < L; t0 += kTT, buf ^= 1) {
    const bool more = t0 + kTT < L;
    if (more) fetch(t0 + kTT);
    const int tn = min(kTT, L - t0);
    auto tile = [&](auto full_tag) {
      constexpr bool kFull = decltype(full_tag)::value;
      // operands of the whole tile in registers first, so no step waits on LDS
      float uu[kTT], dd[kTT], ys[kTT];
#pragma unroll
      for (int i = 0; i < kTT; ++i) {
        if (kFull || i < tn) {
          uu[i] = s_u[buf][i][lane];
          dd[i] = s_dt[buf][i][lane];
        }
      }
      // B, C of step i+kPF are read while step i computes (ring of kPF+1)
      float Br[kPF + 1][NPW], Cr[kPF + 1][NPW];
#pragma unroll
      for (int i = 0; i < kPF; ++i) {
        if (kFull || i < tn) {
          lds_vec<NPW>(&s_B[buf][i][n0], Br[i]);
          lds_vec<NPW>(&s_C[buf][i][n0], Cr[i]);
        }
      }
#pragma unroll
      for (int i = 0; i < kTT; ++i) {
        if (kFull || i < tn) {
          if (i + kPF < kTT && (kFull || i + kPF < tn)) {
            lds_vec<NPW>(&s_B[buf][i + kPF][n0], Br[(i + kPF) % (kPF + 1)]);
            lds_vec<NPW>(&s_C[buf][i + kPF][n0], Cr[(i + kPF) % (kPF + 1)]);
          }
          __builtin_amdgcn_sched_barrier(0);
          const float* Bn = Br[i % (kPF + 1)];
          const float* Cn = Cr[i % (kPF + 1)];
          if (ck_b != nullptr && (i % kCK) == 0) {
            const int blk = (t0 + i) / kCK;
#pragma unroll
            for (int j = 0; j < NPW; ++j) {
              const int n = n0 + j;
              if (n < N && valid) st32(ck_b, (uint32_t)(blk * ND + n * D + d), h[j]);
            }
          }
          const float w = dd[i] * uu[i];
          float yp = 0.0f;
#pragma unroll
          for (int j = 0; j < NPW; ++j) {
            const float a = fast_exp2(A2[j] * dd[i]);
            h[j] = fmaf(a, h[j], Bn[j] * w);
            yp = fmaf(Cn[j], h[j], yp);
          }
          ys[i] = yp;
        }
      }
#pragma unroll
      for (int i = 0; i < kTT; ++i)
        if (kFull || i < tn) s_y[wave][i][lane] = ys[i];
    };
    if (tn == kTT) tile(std::true_type{}); else tile(std::false_type{});
    __syncthreads();
    auto yreduce = [&](auto full_tag) {
      constexpr bool kFull = decltype(full_tag)::value;
#pragma unroll
      for (int k = 0; k < kTT / NG; ++k) {
        const int i = wave + k * NG;
        if (kFull || i < tn) {
          float ys = 0.0f;
#pragma unroll
          for (int w = 0; w < NG; ++w) ys += s_y[w][i][lane];
          const int t = t0 + i;
          const int pt = rev ? L - 1 - t : t;
          if (skip) ys = fmaf(stage_eu ? s_eu[buf][i][lane] : s_u[buf][i][lane], Dq, ys);
          if (gate) {
            const float zz = s_ez[buf][i][lane];
            ys *= zz * sigmoid(zz);
          }
          if (valid) st32(y_b, (uint32_t)(pt * D + q), ys);
        }
      }
    };
    if (tn == kTT) yreduce(std::true_type{}); else yreduce(std::false_type{});
    if (more) commit(buf ^ 1, t0 + kTT);
    __syncthreads();
  }
}

// ----------------------------------------------------------------- backward

template <typename T>
struct BwdArgs {
  const T* u;
  const T* delta;
  const float* A;
  const T* Bc;
  const T* Cc;
  const float* Dskip;
  const T* z;
  const float* ckpt;
  const T* dy;
  T* du;
  T* ddelta;
  T* dz;
  float* ws_dB;   // [ncb][B][L][N]
  float* ws_dC;   // [ncb][B][L][N]
  float* ws_dA;   // [B][D][N]
  float* ws_dD;   // [B][D]
  float* ws_ddt;  // [ncb][B][L] (broadcast delta only)
  int Bt, L, D, N, nblk, ncb;
  int dstride;
  uint32_t flags;
};

template <int NPW, int NG, bool EPI, typename T>
__global__ void __launch_bounds__(kWave* NG, 1) ssm_bwd_kernel(BwdArgs<T> p) {
  constexpr int kCK = ck_for(NG, EPI);
  constexpr int NS = NG * NPW;
  constexpr int RPT = kCK / NG;
  constexpr int kRB = 8 / NPW;  // steps per batched dB / dC reduction
  static_assert(kCK % kRB == 0, "reduction batches must tile the block");
  constexpr int BCE = (kCK * NS + kWave * NG - 1) / (kWave * NG);
  constexpr int EB = EPI ? 2 : 1;
  constexpr int ER = EPI ? kCK : 1;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = blockIdx.y;
  const int cb = blockIdx.x;
  const int L = p.L, D = p.D, N = p.N;
  const int d = cb * kWave + lane;
  const bool valid = d < D;
  const int dc = valid ? d : 0;
  const int n0 = wave * NPW;
  const bool rev = p.flags & SSM_REVERSE;
  const bool comp = rev && (p.flags & SSM_COMPLEMENT);
  const bool gate = EPI && (p.flags & SSM_GATE);
  const bool skip = EPI && (p.flags & SSM_SKIP);
  const bool stage_dyo = skip && rev;         // gated dy at the unmirrored (t,d) for the skip term
  const bool stage_eu = gate && skip && rev;  // u at the output position for y_pre
  const int q = comp ? D - 1 - dc : dc;
  const float Dd = (skip && valid) ? p.Dskip[dc] : 0.0f;
  const float Dq = (skip && valid) ? p.Dskip[q] : 0.0f;

  float Av[NPW], A2[NPW], g[NPW], dAacc[NPW];
#pragma unroll
  for (int j = 0; j < NPW; ++j) {
    const int n = n0 + j;
    Av[j] = (valid && n < N) ? p.A[(int64_t)dc * N + n] : 0.0f;
    A2[j] = Av[j] * kLog2e;
    g[j] = 0.0f;
    dAacc[j] = 0.0f;
  }
  float dDacc = 0.0f;

  __shared__ float s_u[2][kCK][kWave], s_dt[2][kCK][kWave], s_dy[2][kCK][kWave];
  __shared__ float s_go[EB][ER][kWave], s_gz[EB][ER][kWave];  // gate: raw dy and z at the output position
  __shared__ float s_eu[EB][ER][kWave], s_dyo[EB][ER][kWave];
  __shared__ __attribute__((aligned(16))) float s_B[2][kCK][NS];
  __shared__ __attribute__((aligned(16))) float s_C[2][kCK][NS];
  __shared__ float sbuf[EPI ? 3 : 2][NG][kCK][kWave];  // per-wave partials: du, ddelta, (y)
  __shared__ float bcbuf[2][kCK][NS];                  // dB, dC wave partials
  __shared__ float bdummy[2][kWave];                   // sink for lanes without a total

  const int64_t bLD = (int64_t)b * L * D;
  const int64_t bLN = (int64_t)b * L * N;
  const int dtD = p.dstride ? D : 1;
  const int64_t bLDt = (int64_t)b * L * dtD;
  const int dd_lane = p.dstride ? dc : 0;

  const T* __restrict__ u_b = p.u + bLD;
  const T* __restrict__ dt_b = p.delta + bLDt;
  const T* __restrict__ dy_b = p.dy + bLD;
  const T* __restrict__ z_b = EPI ? p.z + bLD : nullptr;
  const T* __restrict__ B_b = p.Bc + bLN;
  const T* __restrict__ C_b = p.Cc + bLN;
  const float* __restrict__ ck_b = p.ckpt + (int64_t)b * p.nblk * N * D;
  T* __restrict__ du_b = p.du + bLD;
  T* __restrict__ ddt_b = p.ddelta + bLD;  // only used when delta is (B,L,D)
  T* __restrict__ dz_b = EPI ? p.dz + bLD : nullptr;
  const int LN = L * N;

  // fetch() only issues loads; commit() (after the block's compute) masks,
  // applies the gate and writes LDS
  float r_u[RPT], r_dt[RPT], r_dy[RPT], r_gz[RPT], r_eu[RPT], r_dyo[RPT], r_zo[RPT];
  float r_B[BCE], r_C[BCE], r_h[NPW];
  auto fetch = [&](int blk) {
    const int t0 = blk * kCK;
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int tc = min(t0 + wave + k * NG, L - 1);
      const int pr = rev ? L - 1 - tc : tc;  // output row of scan step tc
      r_u[k] = ld32(u_b, (uint32_t)(tc * D + dc));
      r_dt[k] = ld32(dt_b, (uint32_t)(tc * dtD + dd_lane));
      r_dy[k] = ld32(dy_b, (uint32_t)(pr * D + q));
      if (gate) r_gz[k] = ld32(z_b, (uint32_t)(pr * D + q));
      if (stage_eu) r_eu[k] = ld32(u_b, (uint32_t)(pr * D + q));
      if (stage_dyo) {
        r_dyo[k] = ld32(dy_b, (uint32_t)(tc * D + dc));
        if (gate) r_zo[k] = ld32(z_b, (uint32_t)(tc * D + dc));
      }
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = threadIdx.x + k * kWave * NG;
      int gi;
      if (NS == N) {
        gi = t0 * N + e;
      } else {
        const int i = e / NS, n = e - i * NS;
        gi = (t0 + i) * N + min(n, N - 1);
      }
      const int gc = min(gi, LN - 1);
      r_B[k] = ld32(B_b, (uint32_t)gc);
      r_C[k] = ld32(C_b, (uint32_t)gc);
    }
#pragma unroll
    for (int j = 0; j < NPW; ++j) r_h[j] = ld32(ck_b, (uint32_t)((blk * N + min(n0 + j, N - 1)) * D + dc));
  };
  auto commit = [&](int buf, int blk) {
    const int t0 = blk * kCK;
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int i = wave + k * NG;
      const bool in = valid && t0 + i < L;
      s_u[buf][i][lane] = in ? r_u[k] : 0.0f;
      s_dt[buf][i][lane] = in ? r_dt[k] : 0.0f;
      const float go = in ? r_dy[k] : 0.0f;
      if (gate) {
        const float gz = in ? r_gz[k] : 0.0f;
        s_go[buf][i][lane] = go;
        s_gz[buf][i][lane] = gz;
        s_dy[buf][i][lane] = go * gz * sigmoid(gz);
      } else {
        s_dy[buf][i][lane] = go;
      }
      if (stage_eu) s_eu[buf][i][lane] = in ? r_eu[k] : 0.0f;
      if (stage_dyo) {
        float v = in ? r_dyo[k] : 0.0f;
        if (gate) {
          const float zz = r_zo[k];
          v *= zz * sigmoid(zz);
        }
        s_dyo[buf][i][lane] = v;
      }
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = threadIdx.x + k * kWave * NG;
      if (e < kCK * NS) {
        const int i = e / NS, n = e - i * NS;
        const bool in = t0 + i < L && n < N;
        (&s_B[buf][0][0])[e] = in ? r_B[k] : 0.0f;
        (&s_C[buf][0][0])[e] = in ? r_C[k] : 0.0f;
      }
    }
  };

  fetch(p.nblk - 1);
  commit(0, p.nblk - 1);
  __syncthreads();
  int buf = 0;
  float h[NPW];
  for (int blk = p.nblk - 1; blk >= 0; --blk, buf ^= 1) {
    const int t0 = blk * kCK;
    const int tn = min(kCK, L - t0);
#pragma unroll
    for (int j = 0; j < NPW; ++j) h[j] = (valid && n0 + j < N) ? r_h[j] : 0.0f;
    const bool more = blk > 0;
    if (more) fetch(blk - 1);

    auto sweeps = [&](auto full_tag) {
      constexpr bool kFull = decltype(full_tag)::value;
      float a_s[kCK][NPW], hp_s[kCK][NPW];
      float uu[kCK], dd[kCK], dyv[kCK];
#pragma unroll
      for (int i = 0; i < kCK; ++i) {
        if (kFull || i < tn) {
          uu[i] = s_u[buf][i][lane];
          dd[i] = s_dt[buf][i][lane];
          dyv[i] = s_dy[buf][i][lane];
        }
      }
      // dB / dC values of kRB consecutive steps are reduced over the wave
      // together (8 values per wave_reduce8); the 8 lanes holding each total's
      // first copy write it, the others write a per-lane dummy slot
      float xb[kRB][NPW];
      auto flush = [&](int i0, int qsel) {
        float x8[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) x8[m] = xb[m / NPW][m % NPW];
        const float r = wave_reduce8(x8);
        const int v = wave_reduce8_index(lane);
        float* dst = (lane & 7) == 0 ? &bcbuf[qsel][i0 + v / NPW][n0 + v % NPW] : &bdummy[qsel][lane];
        *dst = r;
      };
      // forward recompute of the block: a_t, h_{t-1}; dC_t = sum_d dy_t h_t
#pragma unroll
      for (int i = 0; i < kCK; ++i) {
        if (i % kRB == 0) {
#pragma unroll
          for (int bi = 0; bi < kRB; ++bi)
#pragma unroll
            for (int j = 0; j < NPW; ++j) xb[bi][j] = 0.0f;
        }
        if (kFull || i < tn) {
          float Bn[NPW], Cn[NPW];
          lds_vec<NPW>(&s_B[buf][i][n0], Bn);
          if (gate) lds_vec<NPW>(&s_C[buf][i][n0], Cn);
          const float w = dd[i] * uu[i];
          float yp = 0.0f;
#pragma unroll
          for (int j = 0; j < NPW; ++j) {
            const float a = fast_exp2(A2[j] * dd[i]);
            a_s[i][j] = a;
            hp_s[i][j] = h[j];
            h[j] = fmaf(a, h[j], Bn[j] * w);
            xb[i % kRB][j] = dyv[i] * h[j];
            if (gate) yp = fmaf(Cn[j], h[j], yp);
          }
          if (gate) sbuf[EPI ? 2 : 0][wave][i][lane] = yp;
        }
        if (i % kRB == kRB - 1 && (kFull || i - (kRB - 1) < tn)) flush(i - (kRB - 1), 1);
      }
      // adjoint, backwards through the block
#pragma unroll
      for (int i = kCK - 1; i >= 0; --i) {
        if (i % kRB == kRB - 1) {
#pragma unroll
          for (int bi = 0; bi < kRB; ++bi)
#pragma unroll
            for (int j = 0; j < NPW; ++j) xb[bi][j] = 0.0f;
        }
        if (kFull || i < tn) {
          float Bn[NPW], Cn[NPW];
          lds_vec<NPW>(&s_B[buf][i][n0], Bn);
          lds_vec<NPW>(&s_C[buf][i][n0], Cn);
          const float w = dd[i] * uu[i];
          float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
          for (int j = 0; j < NPW; ++j) {
            const float f = fmaf(Cn[j], dyv[i], g[j]);
            const float gg = a_s[i][j] * f;
            const float qv = gg * hp_s[i][j];
            s2 = fmaf(Av[j], qv, s2);
            dAacc[j] = fmaf(dd[i], qv, dAacc[j]);
            s1 = fmaf(Bn[j], f, s1);
            xb[i % kRB][j] = f * w;
            g[j] = gg;
          }
          sbuf[0][wave][i][lane] = dd[i] * s1;
          sbuf[1][wave][i][lane] = fmaf(uu[i], s1, s2);
        }
        if (i % kRB == 0 && (kFull || i < tn)) flush(i, 0);
      }
    };
    if (tn == kCK) sweeps(std::true_type{}); else sweeps(std::false_type{});
    __syncthreads();

    // combine the per-wave partials; write du, ddelta (and dz)
    auto combine = [&](auto full_tag) {
      constexpr bool kFull = decltype(full_tag)::value;
#pragma unroll
      for (int k = 0; k < kCK / NG; ++k) {
        const int i = wave + k * NG;
        if (kFull || i < tn) {
          float du = 0.0f, ddt = 0.0f;
#pragma unroll
          for (int w = 0; w < NG; ++w) {
            du += sbuf[0][w][i][lane];
            ddt += sbuf[1][w][i][lane];
          }
          const int t = t0 + i;
          const float uu = s_u[buf][i][lane];
          if (skip) {
            // y_out[t,d] holds u[t,d]*D[d] (selectssm.py:238): its gradient lands on u[t,d]
            const float dyo = stage_dyo ? s_dyo[buf][i][lane] : s_dy[buf][i][lane];
            du = fmaf(Dd, dyo, du);
            dDacc = fmaf(dyo, uu, dDacc);
          }
          if (valid) {
            st32(du_b, (uint32_t)(t * D + dc), du);
            if (p.dstride) st32(ddt_b, (uint32_t)(t * D + dc), ddt);
          }
          if (!p.dstride) {
            const float tot = wave_sum(valid ? ddt : 0.0f);
            if (lane == 0) p.ws_ddt[((int64_t)cb * p.Bt + b) * L + t] = tot;
          }
          if (gate && valid) {
            float ys = 0.0f;
#pragma unroll
            for (int w = 0; w < NG; ++w) ys += sbuf[EPI ? 2 : 0][w][i][lane];
            if (skip) ys = fmaf(stage_eu ? s_eu[buf][i][lane] : uu, Dq, ys);
            const float zz = s_gz[buf][i][lane];
            const float sg = sigmoid(zz);
            const int pt = rev ? L - 1 - t : t;
            st32(dz_b, (uint32_t)(pt * D + q), s_go[buf][i][lane] * ys * sg * (1.0f + zz * (1.0f - sg)));
          }
        }
      }
    };
    if (tn == kCK) combine(std::true_type{}); else combine(std::false_type{});
    // dB, dC partials of this channel block, coalesced
    {
      float* __restrict__ wB = p.ws_dB + (((int64_t)cb * p.Bt + b) * L + t0) * N;
      float* __restrict__ wC = p.ws_dC + (((int64_t)cb * p.Bt + b) * L + t0) * N;
      for (int idx = threadIdx.x; idx < tn * N; idx += kWave * NG) {
        int i, n;
        if (NS == N) {
          i = idx / NS;
          n = idx - i * NS;
        } else {
          i = idx / N;
          n = idx - i * N;
        }
        wB[idx] = bcbuf[0][i][n];
        wC[idx] = bcbuf[1][i][n];
      }
    }
    if (more) commit(buf ^ 1, blk - 1);
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < NPW; ++j) {
    const int n = n0 + j;
    if (valid && n < N) p.ws_dA[((int64_t)b * D + d) * N + n] = dAacc[j];
  }
  if (skip) {
    // dD partial: every wave accumulated a disjoint subset of timesteps
    __shared__ float dred[NG][kWave];
    dred[wave][lane] = dDacc;
    __syncthreads();
    if (wave == 0 && valid) {
      float s = 0.0f;
#pragma unroll
      for (int w = 0; w < NG; ++w) s += dred[w][lane];
      p.ws_dD[(int64_t)b * D + d] = s;
    }
  }
}

// out[i] = sum_k ws[k*count + i], k = 0..nparts-1 in order
template <typename TO>
__global__ void reduce_parts_kernel(const float* __restrict__ ws, TO* __restrict__ out, int nparts,
                                    int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  float s = 0.0f;
  for (int k = 0; k < nparts; ++k) s += ws[(int64_t)k * count + i];
  st(out, i, s);
}

// ------------------------------------------------------------------- host side

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(SSM_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
  return SSM_OK;
}

struct Shape {
  int B, L, D, N, nblk, ncb;
  int NPW, NG;  // states per wave, waves per workgroup
  bool epi;     // skip / gate epilogue fused
};

// Kernel variant for a shape: fewer states per wave give more waves per SIMD
// (the plain scan); the fused epilogue stages more per block and keeps 4.
void pick_variant(Shape* s, uint32_t flags) {
  s->epi = (flags & (SSM_SKIP | SSM_GATE)) != 0;
  s->NPW = (!s->epi && s->N <= 16) ? kPlainNPW : 4;
  const int ng = (s->N + s->NPW - 1) / s->NPW;
  s->NG = 1;
  while (s->NG < ng) s->NG *= 2;  // instantiated state-group counts: 1, 2, 4, 8
  const int ck = ck_for(s->NG, s->epi);
  s->nblk = (s->L + ck - 1) / ck;
}

int validate(const ssm_desc_t* desc, Shape* s) {
  if (desc == nullptr) return fail(SSM_ERR_INVALID, "desc is NULL");
  if (desc->batch < 1 || desc->seqlen < 1 || desc->dim < 1)
    return fail(SSM_ERR_INVALID, "batch, seqlen and dim must be >= 1");
  if (desc->dstate < 1 || desc->dstate > 32) return fail(SSM_ERR_INVALID, "dstate must be in 1..32");
  if (desc->batch > 65535) return fail(SSM_ERR_INVALID, "batch must be <= 65535");
  // per-batch-row element offsets are 32-bit inside the kernels
  if (desc->seqlen * desc->dim > (int64_t(1) << 31) - 1 || desc->seqlen * desc->dstate > (int64_t(1) << 31) - 1)
    return fail(SSM_ERR_INVALID, "seqlen*dim must fit in int32");
  if ((desc->seqlen / 8 + 1) * desc->dstate * desc->dim > (int64_t(1) << 31) - 1)
    return fail(SSM_ERR_INVALID, "checkpoint rows of one batch row must fit in int32");
  if (desc->dtype != SSM_F32 && desc->dtype != SSM_BF16) return fail(SSM_ERR_INVALID, "dtype must be SSM_F32 or SSM_BF16");
  if (desc->flags & ~(SSM_REVERSE | SSM_COMPLEMENT | SSM_SKIP | SSM_GATE))
    return fail(SSM_ERR_INVALID, "unknown flag bits");
  if ((desc->flags & SSM_COMPLEMENT) && !(desc->flags & SSM_REVERSE))
    return fail(SSM_ERR_INVALID, "SSM_COMPLEMENT requires SSM_REVERSE (selectssm.py:116)");
  if (desc->delta_broadcast != 0 && desc->delta_broadcast != 1)
    return fail(SSM_ERR_INVALID, "delta_broadcast must be 0 or 1");
  if (desc->reserved != 0) return fail(SSM_ERR_INVALID, "reserved must be 0");
  s->B = (int)desc->batch;
  s->L = (int)desc->seqlen;
  s->D = (int)desc->dim;
  s->N = (int)desc->dstate;
  s->ncb = (s->D + kWave - 1) / kWave;
  pick_variant(s, desc->flags);
  return SSM_OK;
}

template <int P, int G, bool E, typename F>
bool dispatch_one(const Shape& s, F&& f) {
  if (s.NPW != P || s.NG != G || s.epi != E) return false;
  f(std::integral_constant<int, P>{}, std::integral_constant<int, G>{}, std::integral_constant<bool, E>{});
  return true;
}

// Calls f(npw, ng, epi) with the compile-time variant matching s.
template <typename F>
bool dispatch_variant(const Shape& s, F&& f) {
  return dispatch_one<kPlainNPW, 1, false>(s, f) || dispatch_one<kPlainNPW, 2, false>(s, f) ||
         dispatch_one<kPlainNPW, 4, false>(s, f) || dispatch_one<kPlainNPW, 8, false>(s, f) ||
         (kPlainNPW != 4 && dispatch_one<4, 8, false>(s, f)) || dispatch_one<4, 1, true>(s, f) ||
         dispatch_one<4, 2, true>(s, f) || dispatch_one<4, 4, true>(s, f) || dispatch_one<4, 8, true>(s, f);
}

size_t ckpt_floats(const Shape& s) { return (size_t)s.B * s.nblk * s.N * s.D; }

struct WsLayout {
  size_t dB, dC, dA, dD, ddt, total;  // float offsets
};

WsLayout ws_layout(const Shape& s, bool bcast) {
  WsLayout w{};
  const size_t bc = (size_t)s.ncb * s.B * s.L * s.N;
  w.dB = 0;
  w.dC = w.dB + bc;
  w.dA = w.dC + bc;
  w.dD = w.dA + (size_t)s.B * s.D * s.N;
  w.ddt = w.dD + (size_t)s.B * s.D;
  w.total = w.ddt + (bcast ? (size_t)s.ncb * s.B * s.L : 0);
  return w;
}

template <typename T>
int launch_fwd(hipStream_t st, const ssm_desc_t* desc, const Shape& s, const void* u, const void* delta,
               const float* A, const void* Bc, const void* Cc, const float* Dskip, const void* z, void* y,
               float* ckpt) {
  FwdArgs<T> a;
  a.u = static_cast<const T*>(u);
  a.delta = static_cast<const T*>(delta);
  a.A = A;
  a.Bc = static_cast<const T*>(Bc);
  a.Cc = static_cast<const T*>(Cc);
  a.Dskip = Dskip;
  a.z = static_cast<const T*>(z);
  a.y = static_cast<T*>(y);
  a.ckpt = ckpt;
  a.L = s.L;
  a.D = s.D;
  a.N = s.N;
  a.nblk = s.nblk;
  a.dstride = desc->delta_broadcast ? 0 : 1;
  a.flags = desc->flags;
  dim3 grid(s.ncb, s.B);
  if (!dispatch_variant(s, [&](auto npw, auto ng, auto epi) {
        constexpr int P = decltype(npw)::value, G = decltype(ng)::value;
        constexpr bool E = decltype(epi)::value;
        hipLaunchKernelGGL((ssm_fwd_kernel<P, G, E, T>), grid, dim3(kWave * G), 0, st, a);
      }))
    return fail(SSM_ERR_UNSUPPORTED, "no kernel variant for this shape");
  return hip_check(hipGetLastError(), "ssm_fwd launch");
}

template <typename T>
int launch_bwd(hipStream_t st, const ssm_desc_t* desc, const Shape& s, const void* u, const void* delta,
               const float* A, const void* Bc, const void* Cc, const float* Dskip, const void* z,
               const float* ckpt, const void* dy, void* du, void* ddelta, float* dA, void* dB, void* dC,
               float* dD, void* dz, void* workspace) {
  const bool bcast = desc->delta_broadcast != 0;
  const WsLayout wl = ws_layout(s, bcast);
  float* ws = static_cast<float*>(workspace);
  BwdArgs<T> a;
  a.u = static_cast<const T*>(u);
  a.delta = static_cast<const T*>(delta);
  a.A = A;
  a.Bc = static_cast<const T*>(Bc);
  a.Cc = static_cast<const T*>(Cc);
  a.Dskip = Dskip;
  a.z = static_cast<const T*>(z);
  a.ckpt = ckpt;
  a.dy = static_cast<const T*>(dy);
  a.du = static_cast<T*>(du);
  a.ddelta = static_cast<T*>(ddelta);
  a.dz = static_cast<T*>(dz);
  a.ws_dB = ws + wl.dB;
  a.ws_dC = ws + wl.dC;
  a.ws_dA = ws + wl.dA;
  a.ws_dD = ws + wl.dD;
  a.ws_ddt = ws + wl.ddt;
  a.Bt = s.B;
  a.L = s.L;
  a.D = s.D;
  a.N = s.N;
  a.nblk = s.nblk;
  a.ncb = s.ncb;
  a.dstride = bcast ? 0 : 1;
  a.flags = desc->flags;
  dim3 grid(s.ncb, s.B);
  if (!dispatch_variant(s, [&](auto npw, auto ng, auto epi) {
        constexpr int P = decltype(npw)::value, G = decltype(ng)::value;
        constexpr bool E = decltype(epi)::value;
        hipLaunchKernelGGL((ssm_bwd_kernel<P, G, E, T>), grid, dim3(kWave * G), 0, st, a);
      }))
    return fail(SSM_ERR_UNSUPPORTED, "no kernel variant for this shape");
  int rc = hip_check(hipGetLastError(), "ssm_bwd launch");
  if (rc) return rc;
  auto reduce = [&](const float* part, auto* out, int nparts, int64_t count) {
    using TO = std::remove_pointer_t<decltype(out)>;
    const int threads = 256;
    const int64_t blocks = (count + threads - 1) / threads;
    hipLaunchKernelGGL((reduce_parts_kernel<TO>), dim3((unsigned)blocks), dim3(threads), 0, st, part, out,
                       nparts, count);
  };
  const int64_t bln = (int64_t)s.B * s.L * s.N;
  reduce(ws + wl.dB, static_cast<T*>(dB), s.ncb, bln);
  reduce(ws + wl.dC, static_cast<T*>(dC), s.ncb, bln);
  reduce(ws + wl.dA, dA, s.B, (int64_t)s.D * s.N);
  if (desc->flags & SSM_SKIP) reduce(ws + wl.dD, dD, s.B, (int64_t)s.D);
  if (bcast) reduce(ws + wl.ddt, static_cast<T*>(ddelta), s.ncb, (int64_t)s.B * s.L);
  return hip_check(hipGetLastError(), "ssm_bwd reduce launch");
}

}  // namespace

// ------------------------------------------------------------------- C ABI

extern "C" {

int ssm_abi_version(void) { return SSM_ABI_VERSION; }

const char* ssm_last_error(void) { return g_last_error.c_str(); }

size_t ssm_ckpt_bytes(const ssm_desc_t* desc) {
  Shape s;
  if (validate(desc, &s)) return 0;
  return ckpt_floats(s) * sizeof(float);
}

size_t ssm_bwd_workspace_bytes(const ssm_desc_t* desc) {
  Shape s;
  if (validate(desc, &s)) return 0;
  return ws_layout(s, desc->delta_broadcast != 0).total * sizeof(float);
}

int ssm_fwd(void* stream, const ssm_desc_t* desc, const void* u, const void* delta, const float* A,
            const void* Bc, const void* Cc, const float* Dskip, const void* z, void* y, float* ckpt) {
  g_last_error.clear();
  Shape s;
  if (int rc = validate(desc, &s)) return rc;
  if (!u || !delta || !A || !Bc || !Cc || !y) return fail(SSM_ERR_INVALID, "ssm_fwd: required pointer is NULL");
  if ((desc->flags & SSM_SKIP) && !Dskip) return fail(SSM_ERR_INVALID, "SSM_SKIP needs Dskip");
  if ((desc->flags & SSM_GATE) && !z) return fail(SSM_ERR_INVALID, "SSM_GATE needs z");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (desc->dtype == SSM_F32)
    return launch_fwd<float>(st, desc, s, u, delta, A, Bc, Cc, Dskip, z, y, ckpt);
  return launch_fwd<bf16>(st, desc, s, u, delta, A, Bc, Cc, Dskip, z, y, ckpt);
}

int ssm_bwd(void* stream, const ssm_desc_t* desc, const void* u, const void* delta, const float* A,
            const void* Bc, const void* Cc, const float* Dskip, const void* z, const float* ckpt, const void* dy,
            void* du, void* ddelta, float* dA, void* dB, void* dC, float* dD, void* dz, void* workspace) {
  g_last_error.clear();
  Shape s;
  if (int rc = validate(desc, &s)) return rc;
  if (!u || !delta || !A || !Bc || !Cc || !ckpt || !dy || !du || !ddelta || !dA || !dB || !dC || !workspace)
    return fail(SSM_ERR_INVALID, "ssm_bwd: required pointer is NULL");
  if ((desc->flags & SSM_SKIP) && (!Dskip || !dD)) return fail(SSM_ERR_INVALID, "SSM_SKIP needs Dskip and dD");
  if ((desc->flags & SSM_GATE) && (!z || !dz)) return fail(SSM_ERR_INVALID, "SSM_GATE needs z and dz");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (desc->dtype == SSM_F32)
    return launch_bwd<float>(st, desc, s, u, delta, A, Bc, Cc, Dskip, z, ckpt, dy, du, ddelta, dA, dB, dC, dD,
                             dz, workspace);
  return launch_bwd<bf16>(st, desc, s, u, delta, A, Bc, Cc, Dskip, z, ckpt, dy, du, ddelta, dA, dB, dC, dD, dz,
                          workspace);
}

}  // extern "C"
