// conv.hip — causal depthwise conv1d + activation for MI355X (gfx950): the
// step before the scan in SelectiveSSM.__call__ (selectssm.py:167-185).
//
//   u[b,t,d] = act(v[b,t,d]),  v[b,t,d] = sum_k w[k,d] * x_s[b, t-(K-1)+k, d]
//
// x_s is x in the scan domain (time-reversed, and with the complement also
// channel-reversed, when the SSM runs in reverse): the flip is an index map
// on the loads of x and the stores of dx, never a materialised copy.
//
// Work decomposition: lane = scan-domain channel (a wave moves 64 consecutive
// channels of one time row: 256 contiguous bytes in f32, also under the
// complement map, which only reverses the order of the lanes' addresses);
// each thread walks kCT consecutive steps with the K-1 steps before them held
// in registers; a workgroup is kCW waves on consecutive time chunks of the
// same channels.  Pure HBM streaming: one read of x (plus a K-1 step halo per
// chunk) and one write of u; the backward reads x and du once and writes dx.
// dw partial sums are added over the workgroup's waves in LDS and then over
// workgroups in fixed order, so dw is deterministic.  dw is a sum over every
// (batch, step) of the tensor (2^14 terms at BASELINE config 1's width, 2^20 at
// config 3): its partial sums are accumulated in float64 (each tile's partial
// rounded once to float32), so its error is a few float32 roundings of the
// result rather than one per tile; the conv is HBM-bound and the float64 FMAs
// cost no time there.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <type_traits>

#include "../../include/selectssm.h"
#include "common.h"

namespace {

using namespace ssm;

constexpr int kLanes = 64;  // channels per wave
constexpr int kCT = 32;     // time steps per thread
constexpr int kCW = 4;      // waves per workgroup (consecutive time chunks)
constexpr int kMaxK = 8;

template <typename T>
struct ConvArgs {
  const T* x;
  const float* w;
  T* u;
  const T* du;
  T* dx;
  float* ws_dw;  // [B][ntile][K][D] (backward, when dw is wanted)
  int L, D, ntile;
  int ldx;  // row stride of x (dx is always (B,L,D))
  bool rev, comp;
  bool acc;  // backward: dx += (SSM_ACCUMULATE)
  int act;
};

__device__ __forceinline__ float act_fwd(int act, float v) {
  if (act == SSM_ACT_SILU) return v * sigmoid(v);
  if (act == SSM_ACT_RELU) return fmaxf(v, 0.0f);
  return v;
}

// d act / dv; relu'(0) = 0 as jax.nn.relu's gradient
__device__ __forceinline__ float act_grad(int act, float v) {
  if (act == SSM_ACT_SILU) {
    const float s = sigmoid(v);
    return s * (1.0f + v * (1.0f - s));
  }
  if (act == SSM_ACT_RELU) return v > 0.0f ? 1.0f : 0.0f;
  return 1.0f;
}

// M consecutive scan-domain steps t_lo .. t_lo + M - 1 of one column: `col`
// points at the column's element of row 0, rows are `ld` elements apart, and
// with `rev` step t is row L - 1 - t.  Steps outside [0, L) read as 0 (the
// conv's causal left padding and the end of the row), and so does every step
// when !live.  All M loads are issued at clamped, in-bounds rows before any
// value is used, with bf16 kept as its raw 16 bits until then, so they are in
// flight together.  (A load under a branch, or one widened next to it, gets
// its wait on the spot: one HBM round trip per step.  The compiler sinks a
// load whose value only a masked select uses into a branch of its own, so
// each raw value passes an empty asm first, which makes the load
// unconditional.)
template <int M, typename T>
__device__ __forceinline__ void load_rows(float (&out)[M], const T* col, int t_lo, int L, int ld, bool rev,
                                          bool live) {
  uint32_t raw[M];
#pragma unroll
  for (int j = 0; j < M; ++j) {
    const int t = min(max(t_lo + j, 0), L - 1);
    const int r = rev ? L - 1 - t : t;
    const T* e = col + (int64_t)r * ld;
    if constexpr (sizeof(T) == 4) {
      raw[j] = *reinterpret_cast<const uint32_t*>(e);
    } else {
      raw[j] = *reinterpret_cast<const uint16_t*>(e);
    }
  }
#pragma unroll
  for (int j = 0; j < M; ++j) {
    const int t = t_lo + j;
    uint32_t v = raw[j];
    asm volatile("" : "+v"(v));
    const float f = sizeof(T) == 4 ? __uint_as_float(v) : __uint_as_float(v << 16);
    out[j] = (live && t >= 0 && t < L) ? f : 0.0f;
  }
}

template <int K, typename T>
__global__ void __launch_bounds__(kLanes* kCW) conv_fwd_kernel(ConvArgs<T> p) {
  const int lane = threadIdx.x & (kLanes - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kLanes);
  const int L = p.L, D = p.D;
  const int d = blockIdx.x * kLanes + lane;                 // scan-domain channel
  const int t0 = (blockIdx.y * kCW + wave) * kCT;           // scan-domain time
  if (d >= D || t0 >= L) return;
  const int q = p.comp ? D - 1 - d : d;                     // channel of x
  const int ldx = p.ldx;
  const T* __restrict__ xb = p.x + (int64_t)blockIdx.z * L * ldx;
  T* __restrict__ ub = p.u + (int64_t)blockIdx.z * L * D;
  float wk[K];
#pragma unroll
  for (int k = 0; k < K; ++k) wk[k] = p.w[(int64_t)k * D + d];
  // x_s[t0 - (K-1) .. t0 + kCT - 1]
  float xs[kCT + K - 1];
  load_rows<kCT + K - 1>(xs, xb + q, t0 - (K - 1), L, ldx, p.rev, true);
#pragma unroll
  for (int i = 0; i < kCT; ++i) {
    const int t = t0 + i;
    if (t < L) {
      float v = 0.0f;
#pragma unroll
      for (int k = 0; k < K; ++k) v = fmaf(wk[k], xs[i + k], v);
      st(ub, (int64_t)t * D + d, act_fwd(p.act, v));
    }
  }
}

// ACC: dx += (SSM_ACCUMULATE), a separate build so that the plain backward's
// loads and registers are those of a kernel without the extra dx read
template <int K, bool ACC, typename T>
__global__ void __launch_bounds__(kLanes* kCW) conv_bwd_kernel(ConvArgs<T> p) {
  const int lane = threadIdx.x & (kLanes - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kLanes);
  const int L = p.L, D = p.D;
  const int d = blockIdx.x * kLanes + lane;
  const int t0 = (blockIdx.y * kCW + wave) * kCT;
  const bool live = d < D && t0 < L;
  const int dc = d < D ? d : D - 1;
  const int q = p.comp ? D - 1 - dc : dc;
  const int ldx = p.ldx;
  const int64_t base = (int64_t)blockIdx.z * L * D;
  const T* __restrict__ xb = p.x + (int64_t)blockIdx.z * L * ldx;
  const T* __restrict__ dub = p.du + base;
  float wk[K];
#pragma unroll
  for (int k = 0; k < K; ++k) wk[k] = p.w[(int64_t)k * D + dc];
  // x_s[t0 - (K-1) .. t0 + kCT + K - 2] and du[t0 .. t0 + kCT + K - 2]:
  // dx_s[t] needs dv at t .. t + K - 1, and dv[t] needs v[t]
  float xs[kCT + 2 * K - 2], dv[kCT + K - 1];
  load_rows<kCT + 2 * K - 2>(xs, xb + q, t0 - (K - 1), L, ldx, p.rev, live);
  load_rows<kCT + K - 1>(dv, dub + dc, t0, L, D, false, live);
#pragma unroll
  for (int j = 0; j < kCT + K - 1; ++j) {
    float v = 0.0f;
#pragma unroll
    for (int k = 0; k < K; ++k) v = fmaf(wk[k], xs[j + k], v);
    dv[j] *= act_grad(p.act, v);
  }
  if (p.dx != nullptr && live) {
    T* __restrict__ dxb = p.dx + base;
    // SSM_ACCUMULATE: the dx already there, loaded (like x and du) before any use
    float dxo[ACC ? kCT : 1];
    if constexpr (ACC) load_rows<kCT>(dxo, dxb + q, t0, L, D, p.rev, true);
#pragma unroll
    for (int i = 0; i < kCT; ++i) {
      const int t = t0 + i;
      if (t < L) {
        float g = 0.0f;
#pragma unroll
        for (int k = 0; k < K; ++k) g = fmaf(wk[k], dv[i + K - 1 - k], g);
        if constexpr (ACC) {
          pin(g);  // rounded on its own (with K = 1 the sum would fuse into the product)
          g = dxo[i] + g;  // one rounding, as adding two dx arrays would
        }
        const int r = p.rev ? L - 1 - t : t;
        st(dxb, (int64_t)r * D + q, g);
      }
    }
  }
  if (p.ws_dw == nullptr) return;  // uniform over the workgroup
  // dw[k,d] over this thread's steps (dv beyond L is 0), then over the waves,
  // in float64
  __shared__ double sdw[kCW][K][kLanes];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < kCT; ++i) s = fma((double)dv[i], (double)xs[i + k], s);
    sdw[wave][k][lane] = s;
  }
  __syncthreads();
  if (wave == 0 && d < D) {
    float* __restrict__ out = p.ws_dw + ((int64_t)blockIdx.z * p.ntile + blockIdx.y) * K * D;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      double s = 0.0;
#pragma unroll
      for (int w = 0; w < kCW; ++w) s += sdw[w][k][lane];
      out[(int64_t)k * D + d] = (float)s;
    }
  }
}

// out[y*count + i] = sum over parts k in [y*per, min(nparts, (y+1)*per)) of
// ws[k*count + i], y = blockIdx.y: a workgroup takes 64 consecutive columns;
// its 16 lane groups sum the parts k0 + g, k0 + g + 16, ... in order, and the
// 16 group sums are added in order through LDS (a fixed order overall, so dw
// is deterministic), all in float64.  Many parts (long rows) go through two
// launches: slices of kRedSlice parts into a staging area, then the slices.
constexpr int kRedCols = 64, kRedGroups = 16, kRedSlice = 64;
__global__ void __launch_bounds__(kRedCols* kRedGroups) conv_reduce_kernel(const float* __restrict__ ws,
                                                                          float* __restrict__ out, int nparts,
                                                                          int per, int64_t count) {
  const int col = threadIdx.x % kRedCols;
  const int grp = threadIdx.x / kRedCols;
  const int64_t i = (int64_t)blockIdx.x * kRedCols + col;
  const int k0 = blockIdx.y * per;
  const int k1 = min(nparts, k0 + per);
  out += (int64_t)blockIdx.y * count;
  double s = 0.0;
  if (i < count)
    for (int k = k0 + grp; k < k1; k += kRedGroups) s += (double)ws[(int64_t)k * count + i];
  __shared__ double part[kRedGroups][kRedCols];
  part[grp][col] = s;
  __syncthreads();
  if (grp == 0 && i < count) {
    double t = 0.0;
#pragma unroll
    for (int g = 0; g < kRedGroups; ++g) t += part[g][col];
    out[i] = (float)t;
  }
}

struct ConvShape {
  int B, L, D, K, ntile, ldx;
};

// slices of the first reduction launch (0: one launch over all parts; also
// when the slices would not fit a grid's y dimension)
int red_slices(int64_t nparts) {
  const int64_t S = (nparts + kRedSlice - 1) / kRedSlice;
  return nparts > kRedSlice && S <= 65535 ? (int)S : 0;
}

int validate_conv(const ssm_conv_desc_t* desc, ConvShape* s) {
  if (desc == nullptr) return fail(SSM_ERR_INVALID, "desc is NULL");
  if (desc->batch < 1 || desc->seqlen < 1 || desc->dim < 1)
    return fail(SSM_ERR_INVALID, "batch, seqlen and dim must be >= 1");
  if (desc->batch > 65535) return fail(SSM_ERR_INVALID, "batch must be <= 65535");
  // each extent bounded first, so that the products below cannot overflow
  constexpr int64_t kMaxExtent = (int64_t(1) << 31) - 1;
  if (desc->seqlen > kMaxExtent || desc->dim > kMaxExtent || desc->ld_x < 0 || desc->ld_x > kMaxExtent)
    return fail(SSM_ERR_INVALID, "seqlen, dim and ld_x must be < 2^31");
  if (desc->seqlen * desc->dim > (int64_t(1) << 31) - 1) return fail(SSM_ERR_INVALID, "seqlen*dim must be < 2^31");
  if (desc->ksize < 1 || desc->ksize > kMaxK) return fail(SSM_ERR_INVALID, "ksize must be in 1..8");
  if (desc->dtype != SSM_F32 && desc->dtype != SSM_BF16) return fail(SSM_ERR_INVALID, "dtype must be SSM_F32 or SSM_BF16");
  if (desc->flags & ~(SSM_REVERSE | SSM_COMPLEMENT | SSM_ACCUMULATE))
    return fail(SSM_ERR_INVALID, "conv flags: only SSM_REVERSE, SSM_COMPLEMENT, SSM_ACCUMULATE");
  if (desc->activation != SSM_ACT_NONE && desc->activation != SSM_ACT_SILU && desc->activation != SSM_ACT_RELU)
    return fail(SSM_ERR_INVALID, "activation must be SSM_ACT_NONE, SSM_ACT_SILU or SSM_ACT_RELU");
  s->B = (int)desc->batch;
  s->L = (int)desc->seqlen;
  s->D = (int)desc->dim;
  s->K = desc->ksize;
  if (desc->ld_x != 0 && desc->ld_x < desc->dim) return fail(SSM_ERR_INVALID, "ld_x must be 0 or >= dim");
  if (desc->seqlen * (desc->ld_x ? desc->ld_x : desc->dim) > (int64_t(1) << 31) - 1)
    return fail(SSM_ERR_INVALID, "seqlen*ld_x must be < 2^31");
  s->ldx = desc->ld_x ? (int)desc->ld_x : s->D;
  s->ntile = (s->L + kCT * kCW - 1) / (kCT * kCW);
  if (s->ntile > 65535) return fail(SSM_ERR_INVALID, "seqlen must be <= 65535*128");
  return SSM_OK;
}

template <typename F>
bool dispatch_k(int K, F&& f) {
  switch (K) {
    case 1: f(std::integral_constant<int, 1>{}); return true;
    case 2: f(std::integral_constant<int, 2>{}); return true;
    case 3: f(std::integral_constant<int, 3>{}); return true;
    case 4: f(std::integral_constant<int, 4>{}); return true;
    case 5: f(std::integral_constant<int, 5>{}); return true;
    case 6: f(std::integral_constant<int, 6>{}); return true;
    case 7: f(std::integral_constant<int, 7>{}); return true;
    case 8: f(std::integral_constant<int, 8>{}); return true;
    default: return false;
  }
}

template <typename T>
ConvArgs<T> conv_args(const ssm_conv_desc_t* desc, const ConvShape& s) {
  ConvArgs<T> a{};
  a.L = s.L;
  a.D = s.D;
  a.ntile = s.ntile;
  a.ldx = s.ldx;
  a.rev = (desc->flags & SSM_REVERSE) != 0;
  a.comp = (desc->flags & SSM_COMPLEMENT) != 0;
  a.acc = (desc->flags & SSM_ACCUMULATE) != 0;
  a.act = desc->activation;
  return a;
}

template <typename T>
int launch_conv_fwd(hipStream_t st, const ssm_conv_desc_t* desc, const ConvShape& s, const void* x,
                    const float* w, void* u) {
  ConvArgs<T> a = conv_args<T>(desc, s);
  a.x = static_cast<const T*>(x);
  a.w = w;
  a.u = static_cast<T*>(u);
  const dim3 grid((s.D + kLanes - 1) / kLanes, s.ntile, s.B);
  dispatch_k(s.K, [&](auto kc) {
    constexpr int K = decltype(kc)::value;
    hipLaunchKernelGGL((conv_fwd_kernel<K, T>), grid, dim3(kLanes * kCW), 0, st, a);
  });
  return hip_check(hipGetLastError(), "ssm_conv_fwd launch");
}

template <typename T>
int launch_conv_bwd(hipStream_t st, const ssm_conv_desc_t* desc, const ConvShape& s, const void* x,
                    const float* w, const void* du, void* dx, float* dw, void* workspace) {
  ConvArgs<T> a = conv_args<T>(desc, s);
  a.x = static_cast<const T*>(x);
  a.w = w;
  a.du = static_cast<const T*>(du);
  a.dx = static_cast<T*>(dx);
  a.ws_dw = dw != nullptr ? static_cast<float*>(workspace) : nullptr;
  const dim3 grid((s.D + kLanes - 1) / kLanes, s.ntile, s.B);
  dispatch_k(s.K, [&](auto kc) {
    constexpr int K = decltype(kc)::value;
    if (a.acc)
      hipLaunchKernelGGL((conv_bwd_kernel<K, true, T>), grid, dim3(kLanes * kCW), 0, st, a);
    else
      hipLaunchKernelGGL((conv_bwd_kernel<K, false, T>), grid, dim3(kLanes * kCW), 0, st, a);
  });
  if (int rc = hip_check(hipGetLastError(), "ssm_conv_bwd launch")) return rc;
  if (dw != nullptr) {
    const int64_t count = (int64_t)s.K * s.D;
    const int nparts = s.B * s.ntile;
    const int S = red_slices(nparts);
    const unsigned gx = (unsigned)((count + kRedCols - 1) / kRedCols);
    const float* parts = static_cast<const float*>(workspace);
    if (S > 0) {
      // slices of kRedSlice parts into the staging area after the parts
      float* stage = static_cast<float*>(workspace) + (int64_t)nparts * count;
      hipLaunchKernelGGL(conv_reduce_kernel, dim3(gx, (unsigned)S), dim3(kRedCols * kRedGroups), 0, st, parts, stage,
                         nparts, kRedSlice, count);
      if (int rc = hip_check(hipGetLastError(), "ssm_conv_bwd reduce launch")) return rc;
      hipLaunchKernelGGL(conv_reduce_kernel, dim3(gx, 1u), dim3(kRedCols * kRedGroups), 0, st,
                         static_cast<const float*>(stage), dw, S, S, count);
    } else {
      hipLaunchKernelGGL(conv_reduce_kernel, dim3(gx, 1u), dim3(kRedCols * kRedGroups), 0, st, parts, dw, nparts,
                         nparts, count);
    }
    return hip_check(hipGetLastError(), "ssm_conv_bwd reduce launch");
  }
  return SSM_OK;
}

}  // namespace

extern "C" {

size_t ssm_conv_bwd_workspace_bytes(const ssm_conv_desc_t* desc) {
  g_last_error.clear();
  ConvShape s;
  if (validate_conv(desc, &s)) return 0;
  const int64_t nparts = (int64_t)s.B * s.ntile;
  return (size_t)(nparts + red_slices(nparts)) * s.K * s.D * sizeof(float);
}

int ssm_conv_fwd(void* stream, const ssm_conv_desc_t* desc, const void* x, const float* w, void* u) {
  const ApiRange range("ssm_conv_fwd");
  g_last_error.clear();
  ConvShape s;
  if (int rc = validate_conv(desc, &s)) return rc;
  if (!x || !w || !u) return fail(SSM_ERR_INVALID, "ssm_conv_fwd: required pointer is NULL");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (desc->dtype == SSM_F32) return launch_conv_fwd<float>(st, desc, s, x, w, u);
  return launch_conv_fwd<bf16>(st, desc, s, x, w, u);
}

int ssm_conv_bwd(void* stream, const ssm_conv_desc_t* desc, const void* x, const float* w, const void* du,
                 void* dx, float* dw, void* workspace) {
  const ApiRange range("ssm_conv_bwd");
  g_last_error.clear();
  ConvShape s;
  if (int rc = validate_conv(desc, &s)) return rc;
  if (!x || !w || !du) return fail(SSM_ERR_INVALID, "ssm_conv_bwd: required pointer is NULL");
  if (dw != nullptr && workspace == nullptr) return fail(SSM_ERR_INVALID, "ssm_conv_bwd: dw needs workspace");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (desc->dtype == SSM_F32) return launch_conv_bwd<float>(st, desc, s, x, w, du, dx, dw, workspace);
  return launch_conv_bwd<bf16>(st, desc, s, x, w, du, dx, dw, workspace);
}

}  // extern "C"
