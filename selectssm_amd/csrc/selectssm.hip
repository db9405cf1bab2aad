// selectssm.hip — selective-scan forward/backward for MI355X (gfx950, CDNA4).
//
// Work decomposition (both kernels)
//   * workgroup = (block of 32 channels, batch row, time segment); time runs
//     sequentially inside the workgroup.  With 32 channels per workgroup a CU
//     holds two workgroups whose barriers are independent.
//   * rows too few to fill the chip (B * ceil(D/32) small: long-sequence
//     shapes) are split in time into segments joined by carries: an aggregate
//     pass gives each segment's (decay product P, end state H from a zero
//     start), and each segment of the main pass folds the earlier segments'
//     aggregates into its starting state, h = P h + H (the combine of
//     selectssm.py:81-85 applied to whole segments).  The backward does the
//     same for the adjoint carry, right to left.  The aggregate walks flush
//     products below 2^-126 to zero and stop where every P of the workgroup
//     is 0, since all further terms are then exact zeros.
//   * lane = channel: lane l holds channel l & 31, and the two 32-lane halves
//     of a wave hold different states of the same 32 channels.  Each lane keeps
//     2 states, a wave 4, and the NG = ceil(N/4) waves of a workgroup all N.
//     u / delta / dy / y rows ((B,L,D) row-major) move as 128-byte rows; the
//     sum over states (y, du, ddelta) is one cross-half add plus an LDS sum
//     over the NG waves.
//   * A[d,n] lives in VGPRs pre-scaled by log2(e), so the decay is one
//     v_exp_f32 of one product; B_t,n / C_t,n are read from LDS as broadcasts.
//   * time is walked in tiles staged in LDS: the next tile's loads are issued
//     before the current tile computes and written to the other buffer after.
//
// Backward = the custom-VJP adjoint of ssmrecscan.py:150-160 with the
// recursive storage of ssmrecscan.py:111-148 replaced by checkpoints: the
// forward stores h entering every 16-step block; the backward walks blocks in
// reverse, recomputes a_t and h_{t-1} of the block into registers, then runs
// the adjoint f_t = C_t dy_t + a_{t+1} f_{t+1} backwards through the block.
// Sums over channels (dB, dC) are reduced within each 32-lane half with
// v_permlane16_swap + DPP, 4 steps at a time, then across channel blocks in
// fixed order, so every gradient is deterministic.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <algorithm>
#include <cstdio>
#include <string>
#include <type_traits>

#include "../../include/selectssm.h"
#include "common.h"

namespace {

using namespace ssm;

constexpr int kWave = 64;
constexpr int kCh = 32;   // channels per workgroup (lane & 31)
constexpr int kSPW = 4;   // states per wave: 2 per lane, the two lane halves differ
constexpr int kTT = 32;   // forward time tile
constexpr int kCK = 16;   // checkpoint interval = backward block length
#ifndef SSM_BWD_RB
#define SSM_BWD_RB 16
#endif
#ifndef SSM_BWD_PF
#define SSM_BWD_PF 2
#endif
#ifndef SSM_FWD_PF
#define SSM_FWD_PF 2
#endif
#ifndef SSM_LDS_DB
#define SSM_LDS_DB 1
#endif
#ifndef SSM_LDS_DC
#define SSM_LDS_DC 0
#endif
constexpr int kRS = 36;   // padded row (floats) of the dB / dC transpose tile: 16-lane float4 reads hit distinct banks

// --------------------------------------------------------------- forward

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
  float* agg_H;  // [B][nseg][N][D]: state at the end of each segment from a zero start
  float* agg_P;  // [B][nseg][N][D]: product of the segment's decays a_t
  int L, D, N, nblk;
  int ldy, ldz;       // row strides (elements) of y and z
  int seg_len, nseg;  // time segments per row (seg_len a multiple of kTT)
  int dstride;        // 1, or 0 for a (B,L,1) delta
  uint32_t flags;
};

// NG waves (4 states each) per workgroup; EPI: the extra staging of the
// reverse skip and the gate.  Workgroup (cb, b, seg) scans time segment seg of
// its rows, starting from the state the earlier segments hand over (folded
// from their aggregates, ssm_fwd_agg_kernel), and writes y and the
// checkpoints.
// SP: delta arrives before softplus (SSM_DELTA_SOFTPLUS); a separate build,
// because carrying the unused softplus code in the time loop slows it down.
template <int NG, bool EPI, bool SP, typename T>
__global__ void __launch_bounds__(kWave* NG, NG <= 4 ? 8 / NG : 1) ssm_fwd_kernel(FwdArgs<T> p) {
  constexpr int NS = NG * kSPW;         // padded state count
  constexpr int NT = kWave * NG;        // threads
  constexpr int RPT = kTT * kCh / NT;   // staged (step, channel) elements per thread
  constexpr int RSTEP = NT / kCh;       // staged rows between a thread's elements
  constexpr int BCE = kTT * NS / NT;    // staged B / C elements per thread
  static_assert(BCE * NT == kTT * NS && RPT * NT == kTT * kCh, "staging must tile exactly");
  static_assert(kTT % kCK == 0, "time tile must hold whole checkpoint blocks");
  constexpr int EB = EPI ? 2 : 1;
  constexpr int ER = EPI ? kTT : 1;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & (kCh - 1);
  const int hf = lane >> 5;
  const int b = blockIdx.y;
  const int cb = blockIdx.x;
  const int seg = blockIdx.z;
  const int L = p.L, D = p.D, N = p.N;
  const int t_lo = seg * p.seg_len;
  const int t_hi = min(L, t_lo + p.seg_len);
  const int d = cb * kCh + c;
  const bool valid = d < D;
  const int dc = valid ? d : 0;
  const int n0 = wave * kSPW + 2 * hf;  // this lane's states n0, n0 + 1
  const bool rev = p.flags & SSM_REVERSE;
  const bool comp = rev && (p.flags & SSM_COMPLEMENT);
  // the skip of a forward scan uses the staged u itself; the reverse skip and
  // the gate need the extra staging of EPI builds
  const bool skip = (p.flags & SSM_SKIP) != 0;
  const bool gate = EPI && (p.flags & SSM_GATE);
  const bool stage_eu = EPI && skip && rev;  // u at the output position is another element
  // staging / output mapping: thread -> column scol, rows srow0 + k * RSTEP
  const int scol = tid & (kCh - 1);
  const int srow0 = tid / kCh;
  const int sd = cb * kCh + scol;
  const bool svalid = sd < D;
  const bool full_cb = (cb + 1) * kCh <= D;
  const int sdc = svalid ? sd : 0;
  const int sq = comp ? D - 1 - sdc : sdc;  // output channel of the staged column
  const float Dq = (skip && svalid) ? p.Dskip[sq] : 0.0f;

  float A2[2], h[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + j;
    A2[j] = (valid && n < N) ? p.A[(int64_t)dc * N + n] * kLog2e : 0.0f;
    h[j] = 0.0f;
  }
  if (seg > 0) {
    // state entering this segment: h = P h + H over the earlier segments in
    // order (the combine of selectssm.py:81-85 applied to whole segments)
    const int64_t base = (int64_t)b * p.nseg * N * D + dc;
    const int nc0 = min(n0, N - 1), nc1 = min(n0 + 1, N - 1);
#pragma unroll 4
    for (int s = 0; s < seg; ++s) {
      const int64_t o0 = base + ((int64_t)s * N + nc0) * D, o1 = base + ((int64_t)s * N + nc1) * D;
      h[0] = fmaf(p.agg_P[o0], h[0], p.agg_H[o0]);
      h[1] = fmaf(p.agg_P[o1], h[1], p.agg_H[o1]);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
      if (!(valid && n0 + j < N)) h[j] = 0.0f;
  }

  __shared__ float s_u[2][kTT][kCh], s_dt[2][kTT][kCh];
  __shared__ float s_eu[EB][ER][kCh], s_ez[EB][ER][kCh];
  __shared__ __attribute__((aligned(16))) float s_B[2][kTT][NS];
  __shared__ __attribute__((aligned(16))) float s_C[2][kTT][NS];
  __shared__ float s_y[NG][kTT][kCh];

  const int64_t bLD = (int64_t)b * L * D;
  const int64_t bLN = (int64_t)b * L * N;
  const int dtD = p.dstride ? D : 1;
  const int64_t bLDt = (int64_t)b * L * dtD;
  const int scol_dt = p.dstride ? sdc : 0;
  const T* __restrict__ u_b = p.u + bLD;
  const T* __restrict__ dt_b = p.delta + bLDt;
  const int ldy = p.ldy, ldz = p.ldz;
  const T* __restrict__ z_b = EPI ? p.z + (int64_t)b * L * ldz : nullptr;
  const T* __restrict__ B_b = p.Bc + bLN;
  const T* __restrict__ C_b = p.Cc + bLN;
  T* __restrict__ y_b = p.y + (int64_t)b * L * ldy;
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
      const int tc = min(t0 + srow0 + k * RSTEP, L - 1);
      r_u[k] = ld32(u_b, (uint32_t)(tc * D + sdc));
      r_dt[k] = ld32(dt_b, (uint32_t)(tc * dtD + scol_dt));
      if (stage_eu || gate) {
        const int pr = rev ? L - 1 - tc : tc;
        if (stage_eu) r_eu[k] = ld32(u_b, (uint32_t)(pr * D + sq));
        if (gate) r_ez[k] = ld32(z_b, (uint32_t)(pr * ldz + sq));
      }
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = tid + k * NT;
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
      const int i = srow0 + k * RSTEP;
      const bool in = svalid && t0 + i < L;
      s_dt[buf][i][scol] = in ? (SP ? softplus(r_dt[k]) : r_dt[k]) : 0.0f;
      s_u[buf][i][scol] = in ? r_u[k] : 0.0f;
      if (stage_eu) s_eu[buf][i][scol] = in ? r_eu[k] : 0.0f;
      if (gate) s_ez[buf][i][scol] = in ? r_ez[k] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = tid + k * NT;
      const int i = e / NS, n = e - (e / NS) * NS;
      const bool in = t0 + i < L && n < N;
      (&s_B[buf][0][0])[e] = in ? r_B[k] : 0.0f;
      (&s_C[buf][0][0])[e] = in ? r_C[k] : 0.0f;
    }
  };

  // segments start on tile boundaries (seg_len is a multiple of kTT), so
  // only the tile at L can be partial
  fetch(t_lo);
  commit(0, t_lo);
  __syncthreads();
  int buf = 0;
  for (int t0 = t_lo; t0 < t_hi; t0 += kTT, buf ^= 1) {
    const bool more = t0 + kTT < t_hi;
    if (more) fetch(t0 + kTT);
    const int tn = min(kTT, L - t0);
    auto tile = [&](auto full_tag) {
      constexpr bool kFull = decltype(full_tag)::value;
      // operands of the whole tile in registers first, so no step waits on LDS
      float uu[kTT], dd[kTT], ys[kTT];
#pragma unroll
      for (int i = 0; i < kTT; ++i) {
        if (kFull || i < tn) {
          uu[i] = s_u[buf][i][c];
          dd[i] = s_dt[buf][i][c];
        }
      }
      {
        // B_t, C_t read FPF steps ahead of use, before the y writes in between
        constexpr int FPF = SSM_FWD_PF;
        float2 Bl[kTT], Cl[kTT];
#pragma unroll
        for (int i = 0; i < FPF; ++i) {
          Bl[i] = *reinterpret_cast<const float2*>(&s_B[buf][i][n0]);
          Cl[i] = *reinterpret_cast<const float2*>(&s_C[buf][i][n0]);
        }
#pragma unroll
        for (int i = 0; i < kTT; ++i) {
          if (FPF > 0 && i + FPF < kTT) {
            Bl[i + FPF] = *reinterpret_cast<const float2*>(&s_B[buf][i + FPF][n0]);
            Cl[i + FPF] = *reinterpret_cast<const float2*>(&s_C[buf][i + FPF][n0]);
          }
          ys[i] = 0.0f;
          if (kFull || i < tn) {
            const float2 Bv = FPF > 0 ? Bl[i] : *reinterpret_cast<const float2*>(&s_B[buf][i][n0]);
            const float2 Cv = FPF > 0 ? Cl[i] : *reinterpret_cast<const float2*>(&s_C[buf][i][n0]);
            if (ck_b != nullptr && (i % kCK) == 0) {
              const int blk = (t0 + i) / kCK;
#pragma unroll
              for (int j = 0; j < 2; ++j)
                if (valid && n0 + j < N) st32(ck_b, (uint32_t)(blk * ND + (n0 + j) * D + d), h[j]);
            }
            const float w = dd[i] * uu[i];
            const float a0 = fast_exp2(A2[0] * dd[i]);
            const float a1 = fast_exp2(A2[1] * dd[i]);
            h[0] = fmaf(a0, h[0], Bv.x * w);
            h[1] = fmaf(a1, h[1], Bv.y * w);
            ys[i] = fmaf(Cv.y, h[1], Cv.x * h[0]);
          }
        }
        // add the two halves of each step's sum: even steps land in lanes < 32,
        // odd steps in lanes >= 32
#pragma unroll
        for (int i = 0; i < kTT; i += 2)
          if (kFull || i < tn) s_y[wave][i + hf][c] = half_pair(ys[i], ys[i + 1]);
      }
    };
    if (tn == kTT) tile(std::true_type{}); else tile(std::false_type{});
    {
      __syncthreads();
      auto yreduce = [&](auto full_tag) {
        constexpr bool kFull = decltype(full_tag)::value;
#pragma unroll
        for (int k = 0; k < RPT; ++k) {
          const int i = srow0 + k * RSTEP;
          if (kFull || i < tn) {
            float ys = 0.0f;
#pragma unroll
            for (int w = 0; w < NG; ++w) ys += s_y[w][i][scol];
            const int t = t0 + i;
            const int pt = rev ? L - 1 - t : t;
            if (skip) {
              float uo = s_u[buf][i][scol];
              if constexpr (EPI) {
                if (stage_eu) uo = s_eu[buf][i][scol];
              }
              ys = fmaf(uo, Dq, ys);
            }
            if (gate) {
              const float zz = s_ez[buf][i][scol];
              ys *= zz * sigmoid(zz);
            }
            on_valid_lanes(full_cb, svalid, [&] { st32(y_b, (uint32_t)(pt * ldy + sq), ys); });
          }
        }
      };
      if (tn == kTT) yreduce(std::true_type{}); else yreduce(std::false_type{});
    }
    if (more) commit(buf ^ 1, t0 + kTT);
    __syncthreads();
  }
}

// A segment's running decay product is flushed to zero once it falls below
// the smallest normal float (2^-126), as in flush-to-zero arithmetic: with
// subnormals kept, a product whose step factors exceed 1/2 stalls at the
// smallest subnormal instead of reaching 0.  What the flush drops is below
// 2^-126 times the later terms; it would matter only if the remaining decays
// grew by some 2^100 within the segment, which A <= 0, delta >= 0 rule out.
__device__ __forceinline__ void flush_tiny(float (&P)[2]) {
#pragma unroll
  for (int j = 0; j < 2; ++j) P[j] = P[j] < 0x1p-126f ? 0.0f : P[j];
}

// Forward aggregate pass of a time-split scan.  Workgroup (cb, b, seg), for
// segments seg < nseg - 1, writes the segment's state at its end from a zero
// start, H = sum_t P_t B_t delta_t u_t with P_t the product of the decays
// after step t, and the whole segment's decay product P.  It walks the segment
// from its end (H += P B delta u, then P *= a), so once every P of the
// workgroup is 0 (flushed at tile ends, flush_tiny) all earlier steps add
// exact zeros and the walk stops there: with decaying states only the last
// few thousand steps of a long segment are read.
template <int NG, bool SP, typename T>
__global__ void __launch_bounds__(kWave* NG, NG <= 4 ? 8 / NG : 1) ssm_fwd_agg_kernel(FwdArgs<T> p) {
  constexpr int NS = NG * kSPW;
  constexpr int NT = kWave * NG;
  constexpr int RPT = kTT * kCh / NT;
  constexpr int RSTEP = NT / kCh;
  constexpr int BCE = kTT * NS / NT;
  static_assert(BCE * NT == kTT * NS && RPT * NT == kTT * kCh, "staging must tile exactly");
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & (kCh - 1);
  const int hf = lane >> 5;
  const int b = blockIdx.y;
  const int cb = blockIdx.x;
  const int seg = blockIdx.z;
  const int L = p.L, D = p.D, N = p.N;
  const int t_lo = seg * p.seg_len;
  const int t_hi = min(L, t_lo + p.seg_len);
  const int d = cb * kCh + c;
  const bool valid = d < D;
  const int dc = valid ? d : 0;
  const int n0 = wave * kSPW + 2 * hf;
  const int scol = tid & (kCh - 1);
  const int srow0 = tid / kCh;
  const int sd = cb * kCh + scol;
  const bool svalid = sd < D;
  const int sdc = svalid ? sd : 0;

  float A2[2], H[2] = {0.0f, 0.0f}, P[2] = {1.0f, 1.0f};
  bool live[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    live[j] = valid && n0 + j < N;
    A2[j] = live[j] ? p.A[(int64_t)dc * N + n0 + j] * kLog2e : 0.0f;
  }

  __shared__ float s_u[2][kTT][kCh], s_dt[2][kTT][kCh];
  __shared__ __attribute__((aligned(16))) float s_B[2][kTT][NS];
  __shared__ int s_alive[2][NG];

  const int dtD = p.dstride ? D : 1;
  const int scol_dt = p.dstride ? sdc : 0;
  const T* __restrict__ u_b = p.u + (int64_t)b * L * D;
  const T* __restrict__ dt_b = p.delta + (int64_t)b * L * dtD;
  const T* __restrict__ B_b = p.Bc + (int64_t)b * L * N;
  const int LN = L * N;

  float r_u[RPT], r_dt[RPT], r_B[BCE];
  auto fetch = [&](int t0) {
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int tc = min(t0 + srow0 + k * RSTEP, L - 1);
      r_u[k] = ld32(u_b, (uint32_t)(tc * D + sdc));
      r_dt[k] = ld32(dt_b, (uint32_t)(tc * dtD + scol_dt));
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = tid + k * NT;
      int gi;
      if (NS == N) {
        gi = t0 * N + e;
      } else {
        const int i = e / NS, n = e - i * NS;
        gi = (t0 + i) * N + min(n, N - 1);
      }
      r_B[k] = ld32(B_b, (uint32_t)min(gi, LN - 1));
    }
  };
  auto commit = [&](int buf, int t0) {
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int i = srow0 + k * RSTEP;
      const bool in = svalid && t0 + i < L;
      s_u[buf][i][scol] = in ? r_u[k] : 0.0f;
      s_dt[buf][i][scol] = in ? (SP ? softplus(r_dt[k]) : r_dt[k]) : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = tid + k * NT;
      const int i = e / NS, n = e - (e / NS) * NS;
      (&s_B[buf][0][0])[e] = (t0 + i < L && n < N) ? r_B[k] : 0.0f;
    }
  };

  const int t_last = t_lo + (t_hi - 1 - t_lo) / kTT * kTT;
  fetch(t_last);
  commit(0, t_last);
  __syncthreads();
  int buf = 0;
  for (int t0 = t_last;; t0 -= kTT, buf ^= 1) {
    const bool more = t0 > t_lo;
    if (more) fetch(t0 - kTT);
    const int tn = min(kTT, L - t0);
    auto tile = [&](auto full_tag) {
      constexpr bool kFull = decltype(full_tag)::value;
      float uu[kTT], dd[kTT];
#pragma unroll
      for (int i = 0; i < kTT; ++i) {
        if (kFull || i < tn) {
          uu[i] = s_u[buf][i][c];
          dd[i] = s_dt[buf][i][c];
        }
      }
#pragma unroll
      for (int i = kTT - 1; i >= 0; --i) {
        if (kFull || i < tn) {
          const float2 Bv = *reinterpret_cast<const float2*>(&s_B[buf][i][n0]);
          const float w = dd[i] * uu[i];
          H[0] = fmaf(P[0], Bv.x * w, H[0]);
          H[1] = fmaf(P[1], Bv.y * w, H[1]);
          P[0] *= fast_exp2(A2[0] * dd[i]);
          P[1] *= fast_exp2(A2[1] * dd[i]);
        }
      }
    };
    if (tn == kTT) tile(std::true_type{}); else tile(std::false_type{});
    if (more) commit(buf ^ 1, t0 - kTT);
    // products below the smallest normal float are flushed to zero; every
    // earlier step then adds an exact zero, so the walk ends once all are 0
    flush_tiny(P);
    const bool alive = (live[0] && P[0] != 0.0f) || (live[1] && P[1] != 0.0f);
    if (!barrier_any<NG>(alive, s_alive[buf]) || !more) break;
  }
  const int64_t o = (int64_t)b * p.nseg + seg;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    if (live[j]) {
      p.agg_H[(o * N + n0 + j) * D + d] = H[j];
      p.agg_P[(o * N + n0 + j) * D + d] = P[j];
    }
  }
}

// -------------------------------------------------------------- backward

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
  float* ws_dA;   // [B][nseg][D][N]
  float* ws_dD;   // [B][nseg][D]
  float* ws_ddt;  // [ncb][B][L] (broadcast delta only)
  float* agg_G;   // [B][nseg][N][D]: adjoint carry leaving each segment (leftwards) from a zero start
  float* agg_P;   // [B][nseg][N][D]: product of the segment's decays a_t
  int Bt, L, D, N, nblk, ncb;
  int ldy, ldz;   // row strides (elements) of dy and of z
  int seg_len, nseg;
  int dstride;
  uint32_t flags;
};

template <int NG, bool EPI, typename T>
__global__ void __launch_bounds__(kWave* NG, NG <= 4 ? 8 / NG : 1) ssm_bwd_kernel(BwdArgs<T> p) {
  constexpr int NS = NG * kSPW;
  constexpr int NT = kWave * NG;
  constexpr int RPT = kCK * kCh / NT;
  constexpr int RSTEP = NT / kCh;
  constexpr int BCE = kCK * NS / NT;
  static_assert(BCE * NT == kCK * NS && RPT * NT == kCK * kCh, "staging must tile exactly");
  // dB and dC sums over the 32 channels of a wave half: through an LDS
  // transpose tile (LDS_DB / LDS_DC) or in registers with cross-lane moves
  constexpr bool kDbLds = SSM_LDS_DB != 0;
  constexpr bool kDcLds = SSM_LDS_DC != 0;
  // steps per batched dB / dC reduction (the fused-epilogue build stages more
  // operands in LDS and keeps a smaller tile, to stay at 2 workgroups per CU)
  constexpr int kRB = EPI ? 4 : SSM_BWD_RB;
  static_assert(kCK % kRB == 0, "reduction batches must tile the block");
  constexpr int EB = EPI ? 2 : 1;
  constexpr int ER = EPI ? kCK : 1;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & (kCh - 1);
  const int hf = lane >> 5;
  const int b = blockIdx.y;
  const int cb = blockIdx.x;
  const int seg = blockIdx.z;
  const int L = p.L, D = p.D, N = p.N;
  const int blk_lo = seg * (p.seg_len / kCK);
  const int blk_hi = min(p.nblk, blk_lo + p.seg_len / kCK);
  const int d = cb * kCh + c;
  const bool valid = d < D;
  const int dc = valid ? d : 0;
  const int n0 = wave * kSPW + 2 * hf;
  const bool rev = p.flags & SSM_REVERSE;
  const bool comp = rev && (p.flags & SSM_COMPLEMENT);
  const bool gate = EPI && (p.flags & SSM_GATE);
  const bool skip = (p.flags & SSM_SKIP) != 0;  // non-EPI builds run only the forward-scan skip
  const bool stage_dyo = EPI && skip && rev;  // gated dy at the unmirrored (t,d) for the skip term
  const bool stage_eu = gate && skip && rev;  // u at the output position for y_pre
  const bool dsp = p.flags & SSM_DELTA_SOFTPLUS;
  const int scol = tid & (kCh - 1);
  const int srow0 = tid / kCh;
  const int sd = cb * kCh + scol;
  const bool svalid = sd < D;
  const bool full_cb = (cb + 1) * kCh <= D;
  const int sdc = svalid ? sd : 0;
  const int sq = comp ? D - 1 - sdc : sdc;
  const float Dd = (skip && svalid) ? p.Dskip[sdc] : 0.0f;
  const float Dq = (skip && svalid) ? p.Dskip[sq] : 0.0f;

  float Av[2], A2[2], g[2], dAacc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + j;
    Av[j] = (valid && n < N) ? p.A[(int64_t)dc * N + n] : 0.0f;
    A2[j] = Av[j] * kLog2e;
    g[j] = 0.0f;
    dAacc[j] = 0.0f;
  }
  if (seg < p.nseg - 1) {
    // adjoint carry entering this segment from the right: g = P g + G over the
    // later segments, last segment first (g = a_t f_t at each segment's first
    // step is linear in the carry it receives)
    const int64_t base = (int64_t)b * p.nseg * N * D + dc;
    const int nc0 = min(n0, N - 1), nc1 = min(n0 + 1, N - 1);
#pragma unroll 4
    for (int s = p.nseg - 1; s > seg; --s) {
      const int64_t o0 = base + ((int64_t)s * N + nc0) * D, o1 = base + ((int64_t)s * N + nc1) * D;
      g[0] = fmaf(p.agg_P[o0], g[0], p.agg_G[o0]);
      g[1] = fmaf(p.agg_P[o1], g[1], p.agg_G[o1]);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
      if (!(valid && n0 + j < N)) g[j] = 0.0f;
  }
  // dA and dD are sums over every step of the row: per block (16 steps), per
  // group of 16 blocks, then the total, so a 2^20-step row's total sees 4096
  // fp32 adds instead of 2^20
  float dAmid[2] = {0.0f, 0.0f};
  float dDacc = 0.0f;  // for column scol, over this thread's rows
  float dDmid = 0.0f;

  __shared__ float s_u[2][kCK][kCh], s_dt[2][kCK][kCh], s_dy[2][kCK][kCh];
  __shared__ float s_go[EB][ER][kCh], s_gz[EB][ER][kCh];  // gate: raw dy and z at the output position
  __shared__ float s_eu[EB][ER][kCh], s_dyo[EB][ER][kCh];
  __shared__ __attribute__((aligned(16))) float s_B[2][kCK][NS];
  __shared__ __attribute__((aligned(16))) float s_C[2][kCK][NS];
  __shared__ float s_sig[2][kCK][kCh];                 // softplus'(delta) = sigmoid(delta) (SSM_DELTA_SOFTPLUS)
  __shared__ float sbuf[NG][kCK][kWave];               // [du | ddelta] per wave
  __shared__ float ybuf[EPI ? NG : 1][EPI ? kCK : 1][kCh];  // (gate) y of each wave's states, per channel
  __shared__ float bcbuf[2][kCK][NS];                  // dB, dC totals of this channel block
  __shared__ float bdummy[2][kWave];                   // sink for lanes without a total
  // per wave: the dB (or dC) values of kRB steps, one row of 32 channels per
  // (step, state slot, half), summed row-wise every kRB steps
  __shared__ __attribute__((aligned(16))) float rbuf[NG][kRB * 4][kRS];

  const int64_t bLD = (int64_t)b * L * D;
  const int64_t bLN = (int64_t)b * L * N;
  const int dtD = p.dstride ? D : 1;
  const int64_t bLDt = (int64_t)b * L * dtD;
  const int scol_dt = p.dstride ? sdc : 0;
  const T* __restrict__ u_b = p.u + bLD;
  const T* __restrict__ dt_b = p.delta + bLDt;
  const int ldy = p.ldy, ldz = p.ldz;
  const T* __restrict__ dy_b = p.dy + (int64_t)b * L * ldy;
  const T* __restrict__ z_b = EPI ? p.z + (int64_t)b * L * ldz : nullptr;
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
  float r_B[BCE], r_C[BCE], r_h[2];
  auto fetch = [&](int blk) {
    const int t0 = blk * kCK;
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int tc = min(t0 + srow0 + k * RSTEP, L - 1);
      const int pr = rev ? L - 1 - tc : tc;  // output row of scan step tc
      r_u[k] = ld32(u_b, (uint32_t)(tc * D + sdc));
      r_dt[k] = ld32(dt_b, (uint32_t)(tc * dtD + scol_dt));
      r_dy[k] = ld32(dy_b, (uint32_t)(pr * ldy + sq));
      if (gate) r_gz[k] = ld32(z_b, (uint32_t)(pr * ldz + sq));
      if (stage_eu) r_eu[k] = ld32(u_b, (uint32_t)(pr * D + sq));
      if (stage_dyo) {
        r_dyo[k] = ld32(dy_b, (uint32_t)(tc * ldy + sdc));
        if (gate) r_zo[k] = ld32(z_b, (uint32_t)(tc * ldz + sdc));
      }
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = tid + k * NT;
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
    for (int j = 0; j < 2; ++j) r_h[j] = ld32(ck_b, (uint32_t)((blk * N + min(n0 + j, N - 1)) * D + dc));
  };
  // softplus(delta) and its derivative: a separate copy of the staging loop
  auto stage_dt = [&](int buf, int t0, auto sp_tag) {
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int i = srow0 + k * RSTEP;
      const bool in = svalid && t0 + i < L;
      if constexpr (decltype(sp_tag)::value) {
        s_dt[buf][i][scol] = in ? softplus(r_dt[k]) : 0.0f;
        s_sig[buf][i][scol] = in ? sigmoid(r_dt[k]) : 0.0f;
      } else {
        s_dt[buf][i][scol] = in ? r_dt[k] : 0.0f;
      }
    }
  };
  auto commit = [&](int buf, int blk) {
    const int t0 = blk * kCK;
    if (dsp) stage_dt(buf, t0, std::true_type{}); else stage_dt(buf, t0, std::false_type{});
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int i = srow0 + k * RSTEP;
      const bool in = svalid && t0 + i < L;
      s_u[buf][i][scol] = in ? r_u[k] : 0.0f;
      const float go = in ? r_dy[k] : 0.0f;
      if (gate) {
        const float gz = in ? r_gz[k] : 0.0f;
        s_go[buf][i][scol] = go;
        s_gz[buf][i][scol] = gz;
        s_dy[buf][i][scol] = go * gz * sigmoid(gz);
      } else {
        s_dy[buf][i][scol] = go;
      }
      if (stage_eu) s_eu[buf][i][scol] = in ? r_eu[k] : 0.0f;
      if (stage_dyo) {
        float v = in ? r_dyo[k] : 0.0f;
        if (gate) {
          const float zz = r_zo[k];
          v *= zz * sigmoid(zz);
        }
        s_dyo[buf][i][scol] = v;
      }
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = tid + k * NT;
      const int i = e / NS, n = e - (e / NS) * NS;
      const bool in = t0 + i < L && n < N;
      (&s_B[buf][0][0])[e] = in ? r_B[k] : 0.0f;
      (&s_C[buf][0][0])[e] = in ? r_C[k] : 0.0f;
    }
  };

  fetch(blk_hi - 1);
  commit(0, blk_hi - 1);
  __syncthreads();
  int buf = 0;
  float h[2];
  for (int blk = blk_hi - 1; blk >= blk_lo; --blk, buf ^= 1) {
    const int t0 = blk * kCK;
    const int tn = min(kCK, L - t0);
#pragma unroll
    for (int j = 0; j < 2; ++j) h[j] = (valid && n0 + j < N) ? r_h[j] : 0.0f;
    const bool more = blk > blk_lo;
    if (more) fetch(blk - 1);

    auto sweeps = [&](auto full_tag) {
      constexpr bool kFull = decltype(full_tag)::value;
      float a_s[kCK][2], hp_s[kCK][2];
      float uu[kCK], dd[kCK], dyv[kCK];
#pragma unroll
      for (int i = 0; i < kCK; ++i) {
        if (kFull || i < tn) {
          uu[i] = s_u[buf][i][c];
          dd[i] = s_dt[buf][i][c];
          dyv[i] = s_dy[buf][i][c];
        }
      }
      // dB / dC: lane (c, hf) writes its two values of step i into rows
      // ((i % kRB) * 2 + slot) * 2 + hf of its wave's tile.  When a batch of
      // kRB steps is written, lane l reads its part of row l % kRows with
      // float4 loads; two steps later it sums them, the parts are added across
      // lanes, and lanes < kRows write the totals (the others a per-lane dummy
      // slot).  LDS operations of one wave execute in order and the compiler
      // keeps the tile's (possibly aliasing) writes and reads in program
      // order, so no barrier or wait is needed between them.
      // B_t and C_t are read kPF steps ahead of use, before the tile writes
      // of the steps in between, so their latency is covered as well.
      float(*tile)[kRS] = rbuf[wave];
      auto put = [&](int i, float v0, float v1) {
        tile[((i % kRB) * 2 + 0) * 2 + hf][c] = v0;
        tile[((i % kRB) * 2 + 1) * 2 + hf][c] = v1;
      };
      constexpr int kRows = kRB * 4;            // 64, 32 or 16 rows
      constexpr int kPer = 32 * kRows / kWave;  // values of a row per lane: 32, 16 or 8
      float4 pq[kPer / 4];
      auto flush_issue = [&]() {
        const float4* src = reinterpret_cast<const float4*>(&tile[lane % kRows][kPer * (lane / kRows)]);
#pragma unroll
        for (int k = 0; k < kPer / 4; ++k) pq[k] = src[k];
      };
      auto flush_finish = [&](int i0, int qsel) {
        float v = 0.0f;
#pragma unroll
        for (int k = 0; k < kPer / 4; ++k) v += (pq[k].x + pq[k].y) + (pq[k].z + pq[k].w);
        if constexpr (kRows == 16) {  // lanes l, l ^ 16 hold parts of one row
          auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
          v = __uint_as_float(s16[0]) + __uint_as_float(s16[1]);
        }
        if constexpr (kRows < kWave) {  // lanes l, l ^ 32 hold parts of one row
          auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
          v = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        }
        const int r = lane % kRows;
        const int n = wave * kSPW + 2 * (r & 1) + ((r >> 1) & 1);
        float* dst = lane < kRows ? &bcbuf[qsel][i0 + (r >> 2)][n] : &bdummy[qsel][lane];
        *dst = v;
      };
      // register path: 4 steps x 2 states summed together with cross-lane moves
      float xb[4][2];
      auto xflush = [&](int i0, int qsel) {
        float x8[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) x8[m] = xb[m >> 1][m & 1];
        const float r = reduce32x8(x8);
        const int v = reduce32x8_value(lane);
        const int n = wave * kSPW + 2 * reduce32x8_half(lane) + (v & 1);
        float* dst = (lane & 3) == 0 ? &bcbuf[qsel][i0 + (v >> 1)][n] : &bdummy[qsel][lane];
        *dst = r;
      };
      // steps ahead that B / C are read (the fused-epilogue build has fewer
      // registers to spare)
      constexpr int kPF = EPI ? 1 : SSM_BWD_PF;
      float2 Bl[kCK], Cl[kCK];
      auto ldB = [&](int i) { Bl[i] = *reinterpret_cast<const float2*>(&s_B[buf][i][n0]); };
      auto ldC = [&](int i) { Cl[i] = *reinterpret_cast<const float2*>(&s_C[buf][i][n0]); };
      float yp[kCK];  // (gate) this lane's part of y, per step
      // forward recompute of the block: a_t, h_{t-1}; dC_t = sum_d dy_t h_t
#pragma unroll
      for (int i = 0; i < kPF; ++i) {
        ldB(i);
        if (gate) ldC(i);
      }
#pragma unroll
      for (int i = 0; i < kCK; ++i) {
        if (i + kPF < kCK) {
          ldB(i + kPF);
          if (gate) ldC(i + kPF);
        }
        if (kFull || i < tn) {
          const float w = dd[i] * uu[i];
          const float Bn[2] = {Bl[i].x, Bl[i].y};
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const float a = fast_exp2(A2[j] * dd[i]);
            a_s[i][j] = a;
            hp_s[i][j] = h[j];
            h[j] = fmaf(a, h[j], Bn[j] * w);
          }
          if constexpr (kDcLds) {
            put(i, dyv[i] * h[0], dyv[i] * h[1]);
          } else {
            xb[i % 4][0] = dyv[i] * h[0];
            xb[i % 4][1] = dyv[i] * h[1];
          }
          if (gate) {
            yp[i] = fmaf(Cl[i].y, h[1], Cl[i].x * h[0]);
            // steps i-1, i: the halves' sums land in lanes < 32 (even step) and >= 32 (odd);
            // a partial block's last step, if even, is paired with nothing
            if (i & 1) {
              ybuf[EPI ? wave : 0][EPI ? i - 1 + hf : 0][c] = half_pair(yp[i - 1], yp[i]);
            } else if (!kFull && i == tn - 1) {
              ybuf[EPI ? wave : 0][EPI ? i + hf : 0][c] = half_pair(yp[i], 0.0f);
            }
          }
        }
        // batches are flushed whole: a partial block's rows beyond tn give totals nobody reads
        if constexpr (kDcLds) {
          if (i % kRB == kRB - 1) flush_issue();
          if (i % kRB == 1 && i > kRB) flush_finish(i - 1 - kRB, 1);
        } else {
          if (!kFull && i >= tn) xb[i % 4][0] = xb[i % 4][1] = 0.0f;
          if (i % 4 == 3) xflush(i - 3, 1);
        }
      }
      // adjoint, backwards through the block
      float dAblk[2] = {0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < kPF; ++i) {
        ldB(kCK - 1 - i);
        ldC(kCK - 1 - i);
      }
#pragma unroll
      for (int i = kCK - 1; i >= 0; --i) {
        if (i >= kPF) {
          ldB(i - kPF);
          ldC(i - kPF);
        }
        if (kFull || i < tn) {
          const float Bn[2] = {Bl[i].x, Bl[i].y};
          const float Cn[2] = {Cl[i].x, Cl[i].y};
          const float w = dd[i] * uu[i];
          float s1 = 0.0f, s2 = 0.0f, fw[2];
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const float f = fmaf(Cn[j], dyv[i], g[j]);
            const float gg = a_s[i][j] * f;
            const float qv = gg * hp_s[i][j];
            s2 = fmaf(Av[j], qv, s2);
            dAblk[j] = fmaf(dd[i], qv, dAblk[j]);
            s1 = fmaf(Bn[j], f, s1);
            fw[j] = f * w;
            g[j] = gg;
          }
          if constexpr (kDbLds) {
            put(i, fw[0], fw[1]);
          } else {
            xb[i % 4][0] = fw[0];
            xb[i % 4][1] = fw[1];
          }
          // du partial in lanes < 32, ddelta partial in lanes >= 32
          sbuf[wave][i][lane] = half_pair(dd[i] * s1, fmaf(uu[i], s1, s2));
        }
        if constexpr (kDcLds) {
          if (i == kCK - 3) flush_finish(kCK - kRB, 1);  // the forward sweep's last dC batch
        }
        if constexpr (kDbLds) {
          if (i % kRB == 0) flush_issue();
          if (i % kRB == kRB - 2 && i < kCK - kRB) flush_finish(i + 2, 0);
        } else {
          if (!kFull && i >= tn) xb[i % 4][0] = xb[i % 4][1] = 0.0f;
          if (i % 4 == 0) xflush(i, 0);
        }
      }
      if constexpr (kDbLds) flush_finish(0, 0);
      dAmid[0] += dAblk[0];
      dAmid[1] += dAblk[1];
    };
    if (tn == kCK) sweeps(std::true_type{}); else sweeps(std::false_type{});
    __syncthreads();

    // combine the per-wave partials; write du, ddelta (and dz)
    auto combine = [&](auto full_tag) {
      constexpr bool kFull = decltype(full_tag)::value;
      float dDblk = 0.0f;  // per block, like dA
#pragma unroll
      for (int k = 0; k < RPT; ++k) {
        const int i = srow0 + k * RSTEP;
        if (kFull || i < tn) {
          float du = 0.0f, ddt = 0.0f;
#pragma unroll
          for (int w = 0; w < NG; ++w) {
            du += sbuf[w][i][scol];
            ddt += sbuf[w][i][kCh + scol];
          }
          const int t = t0 + i;
          const float uu = s_u[buf][i][scol];
          if (dsp) ddt *= s_sig[buf][i][scol];  // through softplus (the same factor for every channel when broadcast)
          if (skip) {
            // y_out[t,d] holds u[t,d]*D[d] (selectssm.py:238): its gradient lands on u[t,d]
            float dyo = s_dy[buf][i][scol];
            if constexpr (EPI) {
              if (stage_dyo) dyo = s_dyo[buf][i][scol];
            }
            du = fmaf(Dd, dyo, du);
            dDblk = fmaf(dyo, uu, dDblk);
          }
          on_valid_lanes(full_cb, svalid, [&] {
            st32(du_b, (uint32_t)(t * D + sdc), du);
            if (p.dstride) st32(ddt_b, (uint32_t)(t * D + sdc), ddt);
          });
          if (!p.dstride) {
            // the 32 threads of this half-wave hold the 32 channels of row i
            const float tot = half_sum32(svalid ? ddt : 0.0f);
            if (scol == 0) p.ws_ddt[((int64_t)cb * p.Bt + b) * L + t] = tot;
          }
          if (gate && svalid) {
            float ys = 0.0f;
#pragma unroll
            for (int w = 0; w < NG; ++w) ys += ybuf[EPI ? w : 0][EPI ? i : 0][scol];
            if (skip) ys = fmaf(stage_eu ? s_eu[buf][i][scol] : uu, Dq, ys);
            const float zz = s_gz[buf][i][scol];
            const float sg = sigmoid(zz);
            const int pt = rev ? L - 1 - t : t;
            st32(dz_b, (uint32_t)(pt * D + sq), s_go[buf][i][scol] * ys * sg * (1.0f + zz * (1.0f - sg)));
          }
        }
      }
      dDmid += dDblk;
    };
    if (tn == kCK) combine(std::true_type{}); else combine(std::false_type{});
    if (((blk - blk_lo) & 15) == 0) {  // close a group of 16 blocks (and the row's last group)
      dAacc[0] += dAmid[0];
      dAacc[1] += dAmid[1];
      dDacc += dDmid;
      dAmid[0] = dAmid[1] = dDmid = 0.0f;
    }
    // dB, dC totals of this channel block, coalesced
    {
      float* __restrict__ wB = p.ws_dB + (((int64_t)cb * p.Bt + b) * L + t0) * N;
      float* __restrict__ wC = p.ws_dC + (((int64_t)cb * p.Bt + b) * L + t0) * N;
      for (int idx = tid; idx < tn * N; idx += NT) {
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
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + j;
    if (valid && n < N) p.ws_dA[(((int64_t)b * p.nseg + seg) * D + d) * N + n] = dAacc[j];
  }
  if (skip) {
    // dD partial: the threads of one column accumulated disjoint rows
    __shared__ float dred[RSTEP][kCh];
    dred[srow0][scol] = dDacc;
    __syncthreads();
    if (tid < kCh && svalid) {
      float sacc = 0.0f;
#pragma unroll
      for (int r = 0; r < RSTEP; ++r) sacc += dred[r][tid];
      p.ws_dD[((int64_t)b * p.nseg + seg) * D + sd] = sacc;
    }
  }
}

// Aggregate pass of a time-split backward.  Workgroup (cb, b, seg - 1), for
// segments seg >= 1, writes the carry the segment hands to the segment on its
// left with no carry from the right, G = a_t f_t at the segment's first step t
// (f_t = C_t dy_t + a_{t+1} f_{t+1}, ssmrecscan.py:96-100, 150-153), i.e.
// G = sum_t P_t C_t dy_t with P_t the product of the decays up to and including
// step t, and the whole segment's decay product P, through which a carry from
// the right enters G.  It walks the segment forwards (P *= a, then G += P C dy),
// so once every P of the workgroup is 0 (flushed at tile ends, flush_tiny) all
// later steps add exact zeros and the walk stops there.
template <int NG, bool EPI, typename T>
__global__ void __launch_bounds__(kWave* NG, NG <= 4 ? 8 / NG : 1) ssm_bwd_agg_kernel(BwdArgs<T> p) {
  constexpr int NS = NG * kSPW;
  constexpr int NT = kWave * NG;
  constexpr int RPT = kTT * kCh / NT;
  constexpr int RSTEP = NT / kCh;
  constexpr int BCE = kTT * NS / NT;
  static_assert(BCE * NT == kTT * NS && RPT * NT == kTT * kCh, "staging must tile exactly");
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & (kCh - 1);
  const int hf = lane >> 5;
  const int b = blockIdx.y;
  const int cb = blockIdx.x;
  const int seg = blockIdx.z + 1;
  const int L = p.L, D = p.D, N = p.N;
  const int t_lo = seg * p.seg_len;
  const int t_hi = min(L, t_lo + p.seg_len);
  const int d = cb * kCh + c;
  const bool valid = d < D;
  const int dc = valid ? d : 0;
  const int n0 = wave * kSPW + 2 * hf;
  const bool rev = p.flags & SSM_REVERSE;
  const bool comp = rev && (p.flags & SSM_COMPLEMENT);
  const bool gate = EPI && (p.flags & SSM_GATE);
  const bool dsp = p.flags & SSM_DELTA_SOFTPLUS;
  const int scol = tid & (kCh - 1);
  const int srow0 = tid / kCh;
  const int sd = cb * kCh + scol;
  const bool svalid = sd < D;
  const int sdc = svalid ? sd : 0;
  const int sq = comp ? D - 1 - sdc : sdc;

  float A2[2], G[2] = {0.0f, 0.0f}, P[2] = {1.0f, 1.0f};
  bool live[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    live[j] = valid && n0 + j < N;
    A2[j] = live[j] ? p.A[(int64_t)dc * N + n0 + j] * kLog2e : 0.0f;
  }

  __shared__ float s_dt[2][kTT][kCh], s_dy[2][kTT][kCh];
  __shared__ __attribute__((aligned(16))) float s_C[2][kTT][NS];
  __shared__ int s_alive[2][NG];

  const int64_t bLD = (int64_t)b * L * D;
  const int64_t bLN = (int64_t)b * L * N;
  const int dtD = p.dstride ? D : 1;
  const int scol_dt = p.dstride ? sdc : 0;
  const T* __restrict__ dt_b = p.delta + (int64_t)b * L * dtD;
  const int ldy = p.ldy, ldz = p.ldz;
  const T* __restrict__ dy_b = p.dy + (int64_t)b * L * ldy;
  const T* __restrict__ z_b = EPI ? p.z + (int64_t)b * L * ldz : nullptr;
  const T* __restrict__ C_b = p.Cc + bLN;
  const int LN = L * N;

  float r_dt[RPT], r_dy[RPT], r_gz[RPT], r_C[BCE];
  auto fetch = [&](int t0) {
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int tc = min(t0 + srow0 + k * RSTEP, L - 1);
      const int pr = rev ? L - 1 - tc : tc;
      r_dt[k] = ld32(dt_b, (uint32_t)(tc * dtD + scol_dt));
      r_dy[k] = ld32(dy_b, (uint32_t)(pr * ldy + sq));
      if (gate) r_gz[k] = ld32(z_b, (uint32_t)(pr * ldz + sq));
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = tid + k * NT;
      int gi;
      if (NS == N) {
        gi = t0 * N + e;
      } else {
        const int i = e / NS, n = e - i * NS;
        gi = (t0 + i) * N + min(n, N - 1);
      }
      r_C[k] = ld32(C_b, (uint32_t)min(gi, LN - 1));
    }
  };
  auto stage_dt = [&](int buf, int t0, auto sp_tag) {
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int i = srow0 + k * RSTEP;
      const bool in = svalid && t0 + i < L;
      const float v = decltype(sp_tag)::value ? softplus(r_dt[k]) : r_dt[k];
      s_dt[buf][i][scol] = in ? v : 0.0f;
    }
  };
  auto commit = [&](int buf, int t0) {
    if (dsp) stage_dt(buf, t0, std::true_type{}); else stage_dt(buf, t0, std::false_type{});
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int i = srow0 + k * RSTEP;
      const bool in = svalid && t0 + i < L;
      const float go = in ? r_dy[k] : 0.0f;
      if (gate) {
        const float gz = in ? r_gz[k] : 0.0f;
        s_dy[buf][i][scol] = go * gz * sigmoid(gz);  // as the main backward pass stages it
      } else {
        s_dy[buf][i][scol] = go;
      }
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = tid + k * NT;
      const int i = e / NS, n = e - (e / NS) * NS;
      (&s_C[buf][0][0])[e] = (t0 + i < L && n < N) ? r_C[k] : 0.0f;
    }
  };

  fetch(t_lo);
  commit(0, t_lo);
  __syncthreads();
  int buf = 0;
  for (int t0 = t_lo;; t0 += kTT, buf ^= 1) {
    const bool more = t0 + kTT < t_hi;
    if (more) fetch(t0 + kTT);
    const int tn = min(kTT, L - t0);
    auto tile = [&](auto full_tag) {
      constexpr bool kFull = decltype(full_tag)::value;
      float dd[kTT], dyv[kTT];
#pragma unroll
      for (int i = 0; i < kTT; ++i) {
        if (kFull || i < tn) {
          dd[i] = s_dt[buf][i][c];
          dyv[i] = s_dy[buf][i][c];
        }
      }
#pragma unroll
      for (int i = 0; i < kTT; ++i) {
        if (kFull || i < tn) {
          const float2 Cv = *reinterpret_cast<const float2*>(&s_C[buf][i][n0]);
          P[0] *= fast_exp2(A2[0] * dd[i]);
          P[1] *= fast_exp2(A2[1] * dd[i]);
          G[0] = fmaf(P[0], Cv.x * dyv[i], G[0]);
          G[1] = fmaf(P[1], Cv.y * dyv[i], G[1]);
        }
      }
    };
    if (tn == kTT) tile(std::true_type{}); else tile(std::false_type{});
    if (more) commit(buf ^ 1, t0 + kTT);
    // as in the forward aggregate: flushed products end the walk
    flush_tiny(P);
    const bool alive = (live[0] && P[0] != 0.0f) || (live[1] && P[1] != 0.0f);
    if (!barrier_any<NG>(alive, s_alive[buf]) || !more) break;
  }
  const int64_t o = (int64_t)b * p.nseg + seg;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    if (live[j]) {
      p.agg_G[(o * N + n0 + j) * D + d] = G[j];
      p.agg_P[(o * N + n0 + j) * D + d] = P[j];
    }
  }
}

// out[i] = sum_k ws[k*count + i], k = 0..nparts-1 in order.  Each thread sums
// 4 consecutive outputs with 8 parts' loads in flight; V4 (count a multiple of
// 4, ws 16-byte aligned) loads them as float4.
template <typename TO, bool V4>
__global__ void reduce_parts_kernel(const float* __restrict__ ws, TO* __restrict__ out, int nparts,
                                    int64_t count) {
  const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i0 >= count) return;
  constexpr int kIn = 8;
  if constexpr (V4) {
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto add = [&](const float4 v) {
      s[0] += v.x;
      s[1] += v.y;
      s[2] += v.z;
      s[3] += v.w;
    };
    int k = 0;
    for (; k + kIn <= nparts; k += kIn) {
      float4 v[kIn];
#pragma unroll
      for (int j = 0; j < kIn; ++j) v[j] = *reinterpret_cast<const float4*>(ws + (int64_t)(k + j) * count + i0);
#pragma unroll
      for (int j = 0; j < kIn; ++j) add(v[j]);
    }
    for (; k < nparts; ++k) add(*reinterpret_cast<const float4*>(ws + (int64_t)k * count + i0));
#pragma unroll
    for (int e = 0; e < 4; ++e) st(out, i0 + e, s[e]);
  } else {
    const int m = (int)(count - i0 < 4 ? count - i0 : 4);
    for (int e = 0; e < m; ++e) {
      float sum = 0.0f;
      for (int k = 0; k < nparts; ++k) sum += ws[(int64_t)k * count + i0 + e];
      st(out, i0 + e, sum);
    }
  }
}

// ------------------------------------------------------------------- host side

struct Shape {
  int B, L, D, N, nblk, ncb;
  int NG;    // waves per workgroup (4 states each)
  bool epi;  // skip / gate epilogue fused
  int seg_len, nseg;  // time segments per row
  int ldy, ldz;       // row strides of y / dy and of z
};

// Automatic time split: a row is split only when the unsplit grid would leave
// more than half of the resident-wave slots empty (256 CUs x 4 SIMDs x 2 waves
// of these kernels on MI355X), into enough segments to fill them, each at
// least kMinAutoSeg steps long.  The choice depends on the desc alone, so a
// given desc always computes in the same order.
constexpr int kFillWaves = 2048;
constexpr int kMinAutoSeg = 512;
constexpr int kMaxSeg = 1024;

void choose_segments(const ssm_desc_t* desc, Shape* s) {
  int64_t want = desc->segments;
  if (want == 0) {
    const int64_t waves = (int64_t)s->B * s->ncb * s->NG;
    want = 2 * waves >= kFillWaves ? 1 : (kFillWaves + waves - 1) / waves;
    want = std::min<int64_t>(want, std::max(1, s->L / kMinAutoSeg));
  }
  int64_t len = (s->L + want - 1) / want;
  len = (len + kTT - 1) / kTT * kTT;  // segments start on forward tiles
  s->seg_len = (int)len;
  s->nseg = (int)((s->L + len - 1) / len);
}

int validate(const ssm_desc_t* desc, Shape* s) {
  if (desc == nullptr) return fail(SSM_ERR_INVALID, "desc is NULL");
  if (desc->batch < 1 || desc->seqlen < 1 || desc->dim < 1)
    return fail(SSM_ERR_INVALID, "batch, seqlen and dim must be >= 1");
  if (desc->dstate < 1 || desc->dstate > 32) return fail(SSM_ERR_INVALID, "dstate must be in 1..32");
  if (desc->batch > 65535) return fail(SSM_ERR_INVALID, "batch must be <= 65535");
  // per-batch-row byte offsets are 32-bit inside the kernels
  if (desc->seqlen * desc->dim > (int64_t(1) << 30) || desc->seqlen * desc->dstate > (int64_t(1) << 30))
    return fail(SSM_ERR_INVALID, "seqlen*dim and seqlen*dstate must be <= 2^30");
  if ((desc->seqlen + kCK - 1) / kCK * desc->dstate * desc->dim > (int64_t(1) << 30))
    return fail(SSM_ERR_INVALID, "checkpoints of one batch row must hold <= 2^30 floats");
  if (desc->dtype != SSM_F32 && desc->dtype != SSM_BF16) return fail(SSM_ERR_INVALID, "dtype must be SSM_F32 or SSM_BF16");
  if (desc->flags & ~(SSM_REVERSE | SSM_COMPLEMENT | SSM_SKIP | SSM_GATE | SSM_DELTA_SOFTPLUS))
    return fail(SSM_ERR_INVALID, "unknown flag bits");
  if ((desc->flags & SSM_COMPLEMENT) && !(desc->flags & SSM_REVERSE))
    return fail(SSM_ERR_INVALID, "SSM_COMPLEMENT requires SSM_REVERSE (selectssm.py:116)");
  if (desc->delta_broadcast != 0 && desc->delta_broadcast != 1)
    return fail(SSM_ERR_INVALID, "delta_broadcast must be 0 or 1");
  if (desc->segments < 0 || desc->segments > kMaxSeg) return fail(SSM_ERR_INVALID, "segments must be in 0..1024");
  if ((desc->ld_y != 0 && desc->ld_y < desc->dim) || (desc->ld_z != 0 && desc->ld_z < desc->dim))
    return fail(SSM_ERR_INVALID, "ld_y and ld_z must be 0 or >= dim");
  if ((desc->ld_y != 0 && desc->seqlen * desc->ld_y > (int64_t(1) << 30)) ||
      (desc->ld_z != 0 && desc->seqlen * desc->ld_z > (int64_t(1) << 30)))
    return fail(SSM_ERR_INVALID, "seqlen*ld_y and seqlen*ld_z must be <= 2^30");
  s->B = (int)desc->batch;
  s->L = (int)desc->seqlen;
  s->D = (int)desc->dim;
  s->N = (int)desc->dstate;
  s->ncb = (s->D + kCh - 1) / kCh;
  s->ldy = desc->ld_y ? (int)desc->ld_y : s->D;
  s->ldz = desc->ld_z ? (int)desc->ld_z : s->D;
  s->nblk = (s->L + kCK - 1) / kCK;
  // extra epilogue staging: the gate, and the reverse skip's u at the mirrored position
  s->epi = (desc->flags & SSM_GATE) || ((desc->flags & SSM_SKIP) && (desc->flags & SSM_REVERSE));
  const int ng = (s->N + kSPW - 1) / kSPW;
  s->NG = 1;
  while (s->NG < ng) s->NG *= 2;  // instantiated wave counts: 1, 2, 4, 8
  choose_segments(desc, s);
  return SSM_OK;
}

template <int G, bool E, typename F>
bool dispatch_one(const Shape& s, F&& f) {
  if (s.NG != G || s.epi != E) return false;
  f(std::integral_constant<int, G>{}, std::integral_constant<bool, E>{});
  return true;
}

// Calls f(ng, epi) with the compile-time variant matching s.
template <typename F>
bool dispatch_variant(const Shape& s, F&& f) {
  return dispatch_one<1, false>(s, f) || dispatch_one<2, false>(s, f) || dispatch_one<4, false>(s, f) ||
         dispatch_one<8, false>(s, f) || dispatch_one<1, true>(s, f) || dispatch_one<2, true>(s, f) ||
         dispatch_one<4, true>(s, f) || dispatch_one<8, true>(s, f);
}

size_t ckpt_floats(const Shape& s) { return (size_t)s.B * s.nblk * s.N * s.D; }

// Per-segment aggregates of a time-split scan: [B][nseg][N][D] states (or
// adjoint carries) then [B][nseg][N][D] decay products.  None for one segment.
size_t agg_floats(const Shape& s) { return s.nseg > 1 ? (size_t)2 * s.B * s.nseg * s.N * s.D : 0; }

struct WsLayout {
  size_t dB, dC, dA, dD, ddt, aggG, aggP, total;  // float offsets
};

WsLayout ws_layout(const Shape& s, bool bcast) {
  WsLayout w{};
  const size_t bc = (size_t)s.ncb * s.B * s.L * s.N;
  const size_t parts = (size_t)s.B * s.nseg;  // dA, dD partials: one per (batch row, segment)
  w.dB = 0;
  w.dC = w.dB + bc;
  w.dA = w.dC + bc;
  w.dD = w.dA + parts * s.D * s.N;
  w.ddt = w.dD + parts * s.D;
  w.aggG = w.ddt + (bcast ? (size_t)s.ncb * s.B * s.L : 0);
  w.aggP = w.aggG + (s.nseg > 1 ? parts * s.N * s.D : 0);
  w.total = w.aggG + agg_floats(s);
  return w;
}

template <typename T>
int launch_fwd(hipStream_t st, const ssm_desc_t* desc, const Shape& s, const void* u, const void* delta,
               const float* A, const void* Bc, const void* Cc, const float* Dskip, const void* z, void* y,
               float* ckpt, void* workspace) {
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
  a.agg_H = static_cast<float*>(workspace);
  a.agg_P = a.agg_H + (s.nseg > 1 ? (size_t)s.B * s.nseg * s.N * s.D : 0);
  a.L = s.L;
  a.D = s.D;
  a.N = s.N;
  a.nblk = s.nblk;
  a.seg_len = s.seg_len;
  a.nseg = s.nseg;
  a.ldy = s.ldy;
  a.ldz = s.ldz;
  a.dstride = desc->delta_broadcast ? 0 : 1;
  a.flags = desc->flags;
  if (!dispatch_variant(s, [&](auto ng, auto epi) {
        constexpr int G = decltype(ng)::value;
        constexpr bool E = decltype(epi)::value;
        auto go = [&](auto sp) {
          constexpr bool SP = decltype(sp)::value;
          if (s.nseg > 1)  // aggregates of every segment but the last
            hipLaunchKernelGGL((ssm_fwd_agg_kernel<G, SP, T>), dim3(s.ncb, s.B, s.nseg - 1), dim3(kWave * G), 0,
                               st, a);
          hipLaunchKernelGGL((ssm_fwd_kernel<G, E, SP, T>), dim3(s.ncb, s.B, s.nseg), dim3(kWave * G), 0,
                             st, a);
        };
        if (desc->flags & SSM_DELTA_SOFTPLUS) go(std::true_type{}); else go(std::false_type{});
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
  a.agg_G = ws + wl.aggG;
  a.agg_P = ws + wl.aggP;
  a.Bt = s.B;
  a.L = s.L;
  a.D = s.D;
  a.N = s.N;
  a.nblk = s.nblk;
  a.ncb = s.ncb;
  a.seg_len = s.seg_len;
  a.nseg = s.nseg;
  a.ldy = s.ldy;
  a.ldz = s.ldz;
  a.dstride = bcast ? 0 : 1;
  a.flags = desc->flags;
  if (!dispatch_variant(s, [&](auto ng, auto epi) {
        constexpr int G = decltype(ng)::value;
        constexpr bool E = decltype(epi)::value;
        if (s.nseg > 1)  // adjoint aggregates of every segment but the first
          hipLaunchKernelGGL((ssm_bwd_agg_kernel<G, E, T>), dim3(s.ncb, s.B, s.nseg - 1), dim3(kWave * G), 0, st, a);
        hipLaunchKernelGGL((ssm_bwd_kernel<G, E, T>), dim3(s.ncb, s.B, s.nseg), dim3(kWave * G), 0, st, a);
      }))
    return fail(SSM_ERR_UNSUPPORTED, "no kernel variant for this shape");
  int rc = hip_check(hipGetLastError(), "ssm_bwd launch");
  if (rc) return rc;
  auto reduce = [&](const float* part, auto* out, int nparts, int64_t count) {
    using TO = std::remove_pointer_t<decltype(out)>;
    const int threads = 256;
    const int64_t blocks = ((count + 3) / 4 + threads - 1) / threads;
    if (count % 4 == 0 && reinterpret_cast<uintptr_t>(part) % 16 == 0)
      hipLaunchKernelGGL((reduce_parts_kernel<TO, true>), dim3((unsigned)blocks), dim3(threads), 0, st, part,
                         out, nparts, count);
    else
      hipLaunchKernelGGL((reduce_parts_kernel<TO, false>), dim3((unsigned)blocks), dim3(threads), 0, st, part,
                         out, nparts, count);
  };
  const int64_t bln = (int64_t)s.B * s.L * s.N;
  reduce(ws + wl.dB, static_cast<T*>(dB), s.ncb, bln);
  reduce(ws + wl.dC, static_cast<T*>(dC), s.ncb, bln);
  reduce(ws + wl.dA, dA, s.B * s.nseg, (int64_t)s.D * s.N);
  if (desc->flags & SSM_SKIP) reduce(ws + wl.dD, dD, s.B * s.nseg, (int64_t)s.D);
  if (bcast) reduce(ws + wl.ddt, static_cast<T*>(ddelta), s.ncb, (int64_t)s.B * s.L);
  return hip_check(hipGetLastError(), "ssm_bwd reduce launch");
}

}  // namespace

// ------------------------------------------------------------------- C ABI

namespace ssm {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(SSM_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
  return SSM_OK;
}

}  // namespace ssm

extern "C" {

int ssm_abi_version(void) { return SSM_ABI_VERSION; }

const char* ssm_last_error(void) { return g_last_error.c_str(); }

size_t ssm_ckpt_bytes(const ssm_desc_t* desc) {
  g_last_error.clear();
  Shape s;
  if (validate(desc, &s)) return 0;
  return ckpt_floats(s) * sizeof(float);
}

size_t ssm_fwd_workspace_bytes(const ssm_desc_t* desc) {
  g_last_error.clear();
  Shape s;
  if (validate(desc, &s)) return 0;
  return agg_floats(s) * sizeof(float);
}

size_t ssm_bwd_workspace_bytes(const ssm_desc_t* desc) {
  g_last_error.clear();
  Shape s;
  if (validate(desc, &s)) return 0;
  return ws_layout(s, desc->delta_broadcast != 0).total * sizeof(float);
}

int ssm_fwd(void* stream, const ssm_desc_t* desc, const void* u, const void* delta, const float* A,
            const void* Bc, const void* Cc, const float* Dskip, const void* z, void* y, float* ckpt,
            void* workspace) {
  g_last_error.clear();
  Shape s;
  if (int rc = validate(desc, &s)) return rc;
  if (!u || !delta || !A || !Bc || !Cc || !y) return fail(SSM_ERR_INVALID, "ssm_fwd: required pointer is NULL");
  if (s.nseg > 1 && !workspace) return fail(SSM_ERR_INVALID, "ssm_fwd: workspace is NULL but ssm_fwd_workspace_bytes > 0");
  if ((desc->flags & SSM_SKIP) && !Dskip) return fail(SSM_ERR_INVALID, "SSM_SKIP needs Dskip");
  if ((desc->flags & SSM_GATE) && !z) return fail(SSM_ERR_INVALID, "SSM_GATE needs z");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (desc->dtype == SSM_F32)
    return launch_fwd<float>(st, desc, s, u, delta, A, Bc, Cc, Dskip, z, y, ckpt, workspace);
  return launch_fwd<bf16>(st, desc, s, u, delta, A, Bc, Cc, Dskip, z, y, ckpt, workspace);
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
