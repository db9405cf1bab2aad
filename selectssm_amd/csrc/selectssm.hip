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
constexpr int kNPW = 4;   // states per wave
constexpr int kCK = 16;   // checkpoint interval = backward block length
constexpr int kTB = 16;   // forward staging block for the cross-wave y sum

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
__device__ constexpr int kRowState[4] = {0, 2, 1, 3};

// Full sum of one value over the wave (every lane gets it).
__device__ __forceinline__ float wave_sum(float v) {
  v = row_sum16(v);
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
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

template <int NG, typename T>
__global__ void __launch_bounds__(kWave* NG, 1) ssm_fwd_kernel(FwdArgs<T> p) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = blockIdx.y;
  const int L = p.L, D = p.D, N = p.N;
  const int d = blockIdx.x * kWave + lane;
  const bool valid = d < D;
  const int dc = valid ? d : 0;
  const int n0 = wave * kNPW;

  float A2[kNPW], h[kNPW];
#pragma unroll
  for (int j = 0; j < kNPW; ++j) {
    const int n = n0 + j;
    A2[j] = (valid && n < N) ? p.A[(int64_t)dc * N + n] * kLog2e : 0.0f;
    h[j] = 0.0f;
  }

  __shared__ float ybuf[NG][kTB][kWave];

  const int64_t rowD = (int64_t)b * L * D;  // (b,0,0) in (B,L,D)
  const int64_t rowN = (int64_t)b * L * N;  // (b,0,0) in (B,L,N)
  const int64_t rowDt = (int64_t)b * L * (p.dstride ? D : 1);
  const int dtD = p.dstride ? D : 1;
  const int dd_lane = p.dstride ? dc : 0;
  const bool rev = p.flags & SSM_REVERSE;
  const bool comp = rev && (p.flags & SSM_COMPLEMENT);

  for (int t0 = 0; t0 < L; t0 += kTB) {
    const int tn = min(kTB, L - t0);
#pragma unroll 4
    for (int i = 0; i < tn; ++i) {
      const int t = t0 + i;
      if (p.ckpt != nullptr && (t % kCK) == 0) {
        const int blk = t / kCK;
#pragma unroll
        for (int j = 0; j < kNPW; ++j) {
          const int n = n0 + j;
          if (valid && n < N) p.ckpt[(((int64_t)b * p.nblk + blk) * N + n) * D + d] = h[j];
        }
      }
      const float uu = valid ? ld(p.u, rowD + (int64_t)t * D + dc) : 0.0f;
      const float dd = valid ? ld(p.delta, rowDt + (int64_t)t * dtD + dd_lane) : 0.0f;
      const float w = dd * uu;
      float yp = 0.0f;
#pragma unroll
      for (int j = 0; j < kNPW; ++j) {
        const int n = n0 + j;
        const float Bn = n < N ? ld(p.Bc, rowN + (int64_t)t * N + n) : 0.0f;
        const float Cn = n < N ? ld(p.Cc, rowN + (int64_t)t * N + n) : 0.0f;
        const float a = fast_exp2(A2[j] * dd);
        h[j] = fmaf(a, h[j], Bn * w);
        yp = fmaf(Cn, h[j], yp);
      }
      ybuf[wave][i][lane] = yp;
    }
    __syncthreads();
    for (int i = wave; i < tn; i += NG) {
      float ys = 0.0f;
#pragma unroll
      for (int w = 0; w < NG; ++w) ys += ybuf[w][i][lane];
      if (valid) {
        const int t = t0 + i;
        const int pt = rev ? L - 1 - t : t;
        const int q = comp ? D - 1 - d : d;
        const int64_t o = rowD + (int64_t)pt * D + q;
        if (p.flags & SSM_SKIP) ys += ld(p.u, o) * p.Dskip[q];
        if (p.flags & SSM_GATE) {
          const float zz = ld(p.z, o);
          ys *= zz * sigmoid(zz);
        }
        st(p.y, o, ys);
      }
    }
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

template <typename T>
__device__ __forceinline__ float gated_dy(const BwdArgs<T>& p, int64_t o) {
  float g = ld(p.dy, o);
  if (p.flags & SSM_GATE) {
    const float zz = ld(p.z, o);
    g *= zz * sigmoid(zz);
  }
  return g;
}

template <int NG, typename T>
__global__ void __launch_bounds__(kWave* NG, 1) ssm_bwd_kernel(BwdArgs<T> p) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = blockIdx.y;
  const int cb = blockIdx.x;
  const int L = p.L, D = p.D, N = p.N;
  const int d = cb * kWave + lane;
  const bool valid = d < D;
  const int dc = valid ? d : 0;
  const int n0 = wave * kNPW;
  const bool rev = p.flags & SSM_REVERSE;
  const bool comp = rev && (p.flags & SSM_COMPLEMENT);
  const bool gate = p.flags & SSM_GATE;
  const bool skip = p.flags & SSM_SKIP;
  const int q = comp ? D - 1 - dc : dc;  // output channel of this lane

  float Av[kNPW], A2[kNPW], g[kNPW], dAacc[kNPW];
#pragma unroll
  for (int j = 0; j < kNPW; ++j) {
    const int n = n0 + j;
    Av[j] = (valid && n < N) ? p.A[(int64_t)dc * N + n] : 0.0f;
    A2[j] = Av[j] * kLog2e;
    g[j] = 0.0f;
    dAacc[j] = 0.0f;
  }
  float dDacc = 0.0f;

  __shared__ float sbuf[3][NG][kCK][kWave];   // per-wave partials: du, ddelta, y
  __shared__ float bcbuf[2][kCK][NG * kNPW];  // dB, dC wave partials

  const int64_t rowD = (int64_t)b * L * D;
  const int64_t rowN = (int64_t)b * L * N;
  const int dtD = p.dstride ? D : 1;
  const int64_t rowDt = (int64_t)b * L * dtD;
  const int dd_lane = p.dstride ? dc : 0;

  for (int blk = p.nblk - 1; blk >= 0; --blk) {
    const int t0 = blk * kCK;
    const int tn = min(kCK, L - t0);
    float h[kNPW];
#pragma unroll
    for (int j = 0; j < kNPW; ++j) {
      const int n = n0 + j;
      h[j] = (valid && n < N) ? p.ckpt[(((int64_t)b * p.nblk + blk) * N + n) * D + d] : 0.0f;
    }
    float a_s[kCK][kNPW], hp_s[kCK][kNPW];
    float dt_s[kCK], u_s[kCK], dy_s[kCK];

    // forward recompute of the block: a_t, h_{t-1}; dC_t = sum_d dy_t h_t
#pragma unroll
    for (int i = 0; i < kCK; ++i) {
      if (i < tn) {
        const int t = t0 + i;
        const int pt = rev ? L - 1 - t : t;
        const float uu = valid ? ld(p.u, rowD + (int64_t)t * D + dc) : 0.0f;
        const float dd = valid ? ld(p.delta, rowDt + (int64_t)t * dtD + dd_lane) : 0.0f;
        const float dyv = valid ? gated_dy(p, rowD + (int64_t)pt * D + q) : 0.0f;
        const float w = dd * uu;
        float c[kNPW];
        float yp = 0.0f;
#pragma unroll
        for (int j = 0; j < kNPW; ++j) {
          const int n = n0 + j;
          const float Bn = n < N ? ld(p.Bc, rowN + (int64_t)t * N + n) : 0.0f;
          const float a = fast_exp2(A2[j] * dd);
          a_s[i][j] = a;
          hp_s[i][j] = h[j];
          h[j] = fmaf(a, h[j], Bn * w);
          c[j] = dyv * h[j];
          if (gate) {
            const float Cn = n < N ? ld(p.Cc, rowN + (int64_t)t * N + n) : 0.0f;
            yp = fmaf(Cn, h[j], yp);
          }
        }
        if (gate) sbuf[2][wave][i][lane] = yp;
        const float r = wave_reduce4(c[0], c[1], c[2], c[3]);
        if ((lane & 15) == 0) {
          const int n = n0 + kRowState[lane >> 4];
          if (n < NG * kNPW) bcbuf[1][i][n] = r;
        }
        dt_s[i] = dd;
        u_s[i] = uu;
        dy_s[i] = dyv;
      }
    }

    // adjoint, backwards through the block
#pragma unroll
    for (int i = kCK - 1; i >= 0; --i) {
      if (i < tn) {
        const int t = t0 + i;
        const float w = dt_s[i] * u_s[i];
        float s1 = 0.0f, s2 = 0.0f;
        float e[kNPW];
#pragma unroll
        for (int j = 0; j < kNPW; ++j) {
          const int n = n0 + j;
          const float Bn = n < N ? ld(p.Bc, rowN + (int64_t)t * N + n) : 0.0f;
          const float Cn = n < N ? ld(p.Cc, rowN + (int64_t)t * N + n) : 0.0f;
          const float f = fmaf(Cn, dy_s[i], g[j]);
          const float gg = a_s[i][j] * f;
          const float qv = gg * hp_s[i][j];
          s2 = fmaf(Av[j], qv, s2);
          dAacc[j] = fmaf(dt_s[i], qv, dAacc[j]);
          s1 = fmaf(Bn, f, s1);
          e[j] = f * w;
          g[j] = gg;
        }
        const float r = wave_reduce4(e[0], e[1], e[2], e[3]);
        if ((lane & 15) == 0) {
          const int n = n0 + kRowState[lane >> 4];
          if (n < NG * kNPW) bcbuf[0][i][n] = r;
        }
        sbuf[0][wave][i][lane] = dt_s[i] * s1;
        sbuf[1][wave][i][lane] = fmaf(u_s[i], s1, s2);
      }
    }
    __syncthreads();

    // combine the per-wave partials; write du, ddelta (and dz)
    for (int i = wave; i < tn; i += NG) {
      float du = 0.0f, ddt = 0.0f;
#pragma unroll
      for (int w = 0; w < NG; ++w) {
        du += sbuf[0][w][i][lane];
        ddt += sbuf[1][w][i][lane];
      }
      const int t = t0 + i;
      const int64_t o = rowD + (int64_t)t * D + dc;  // scan-domain (t, d)
      if (skip && valid) {
        // y_out[t,d] holds u[t,d]*D[d] (selectssm.py:238): its gradient lands on u[t,d]
        const float dyo = gated_dy(p, o);
        du = fmaf(p.Dskip[dc], dyo, du);
        dDacc = fmaf(dyo, ld(p.u, o), dDacc);
      }
      if (valid) {
        st(p.du, o, du);
        if (p.dstride) st(p.ddelta, rowDt + (int64_t)t * dtD + dc, ddt);
      }
      if (!p.dstride) {
        const float tot = wave_sum(valid ? ddt : 0.0f);
        if (lane == 0) p.ws_ddt[((int64_t)cb * p.Bt + b) * L + t] = tot;
      }
      if (gate && valid) {
        float ys = 0.0f;
#pragma unroll
        for (int w = 0; w < NG; ++w) ys += sbuf[2][w][i][lane];
        const int pt = rev ? L - 1 - t : t;
        const int64_t oo = rowD + (int64_t)pt * D + q;  // output position of scan step (t,d)
        if (skip) ys = fmaf(ld(p.u, oo), p.Dskip[q], ys);
        const float zz = ld(p.z, oo);
        const float sg = sigmoid(zz);
        st(p.dz, oo, ld(p.dy, oo) * ys * sg * (1.0f + zz * (1.0f - sg)));
      }
    }
    // dB, dC partials of this channel block, coalesced
    for (int idx = threadIdx.x; idx < tn * N; idx += kWave * NG) {
      const int i = idx / N, n = idx - i * N;
      const int64_t o = (((int64_t)cb * p.Bt + b) * L + t0 + i) * N + n;
      p.ws_dB[o] = bcbuf[0][i][n];
      p.ws_dC[o] = bcbuf[1][i][n];
    }
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < kNPW; ++j) {
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
  int B, L, D, N, nblk, ncb, NG;
};

int validate(const ssm_desc_t* desc, Shape* s) {
  if (desc == nullptr) return fail(SSM_ERR_INVALID, "desc is NULL");
  if (desc->batch < 1 || desc->seqlen < 1 || desc->dim < 1)
    return fail(SSM_ERR_INVALID, "batch, seqlen and dim must be >= 1");
  if (desc->dstate < 1 || desc->dstate > 32) return fail(SSM_ERR_INVALID, "dstate must be in 1..32");
  if (desc->batch > 65535) return fail(SSM_ERR_INVALID, "batch must be <= 65535");
  if (desc->seqlen * desc->dim > (int64_t(1) << 31) - 1 || desc->seqlen * desc->dstate > (int64_t(1) << 31) - 1)
    return fail(SSM_ERR_INVALID, "seqlen*dim must fit in int32");
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
  s->nblk = (s->L + kCK - 1) / kCK;
  s->ncb = (s->D + kWave - 1) / kWave;
  const int ng = (s->N + kNPW - 1) / kNPW;
  s->NG = 1;
  while (s->NG < ng) s->NG *= 2;  // instantiated state-group counts: 1, 2, 4, 8
  return SSM_OK;
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
  switch (s.NG) {
    case 1: hipLaunchKernelGGL((ssm_fwd_kernel<1, T>), grid, dim3(kWave * 1), 0, st, a); break;
    case 2: hipLaunchKernelGGL((ssm_fwd_kernel<2, T>), grid, dim3(kWave * 2), 0, st, a); break;
    case 4: hipLaunchKernelGGL((ssm_fwd_kernel<4, T>), grid, dim3(kWave * 4), 0, st, a); break;
    case 8: hipLaunchKernelGGL((ssm_fwd_kernel<8, T>), grid, dim3(kWave * 8), 0, st, a); break;
    default: return fail(SSM_ERR_UNSUPPORTED, "unsupported state-group count");
  }
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
  switch (s.NG) {
    case 1: hipLaunchKernelGGL((ssm_bwd_kernel<1, T>), grid, dim3(kWave * 1), 0, st, a); break;
    case 2: hipLaunchKernelGGL((ssm_bwd_kernel<2, T>), grid, dim3(kWave * 2), 0, st, a); break;
    case 4: hipLaunchKernelGGL((ssm_bwd_kernel<4, T>), grid, dim3(kWave * 4), 0, st, a); break;
    case 8: hipLaunchKernelGGL((ssm_bwd_kernel<8, T>), grid, dim3(kWave * 8), 0, st, a); break;
    default: return fail(SSM_ERR_UNSUPPORTED, "unsupported state-group count");
  }
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
