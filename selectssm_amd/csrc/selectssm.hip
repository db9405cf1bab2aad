// selectssm.hip — selective-scan forward/backward for MI355X (gfx950, CDNA4).
//
// Both kernels give each workgroup 64 channels of one batch row and one time
// segment; time runs sequentially inside the workgroup, and all states of a
// channel live in one wave, so every sum over states stays inside the wave.
//
// Forward (ssm_fwd_kernel): 4 waves.  lane = c + 16 g holds channel c of the
// wave's 16 and the SPL states SPL*g .. SPL*g + SPL - 1 (state row g), so a
// lane carries SPL = 4 states for N <= 16.  Per step and state: one v_exp_f32
// of A*log2(e)*delta, h = a h + B (delta u), y += C h.  The sum over the 4
// state rows of 4 consecutive steps is one transposed exchange (2 x
// v_permlane32_swap + v_permlane16_swap and 3 adds): row r ends with step
// yrow_step(r), and every lane stores one (step, channel) of y.
//
// Backward (ssm_bwd_kernel): 8 waves.  lane = c + 8 g holds channel c of the
// wave's 8 and SPL states of state group g (SPL = 2 for N <= 16), in an order
// permuted by the lane (state SPL*g + (j ^ sig(c)) in slot j) so that the sums
// over channels for dB and dC take one DPP add per pair of states
// (chan_reduce8).  The sums over states (du, ddelta) of 2 steps are one
// transposed exchange over the 8 groups.  The custom-VJP adjoint of
// ssmrecscan.py:150-160 with the recursive storage of ssmrecscan.py:111-148
// replaced by checkpoints: the forward stores h entering every block of 16
// steps; the backward walks blocks in reverse, recomputes a_t and h_{t-1} of
// the block into registers, then runs the adjoint f_t = C_t dy_t + a_{t+1}
// f_{t+1} backwards through the block.
//
// Rows too few to fill the chip (long-sequence shapes) are split in time into
// segments joined by carries: an aggregate pass gives each segment's (decay
// product P, end state H from a zero start), and each segment of the main pass
// folds the earlier segments' aggregates into its starting state, h = P h + H
// (the combine of selectssm.py:81-85 applied to whole segments); the backward
// does the same for the adjoint carry, right to left.  The aggregate walks
// flush products below 2^-126 to zero and stop where every P of the workgroup
// is 0, since all further terms are then exact zeros.
//
// Time is walked in tiles staged in LDS: the next tile's global loads are
// issued before the current tile computes and written to the other buffer
// after it (the backward: between the block's two sweeps, when none of the
// block's stores is in flight yet); inside a tile the LDS operands of step
// i + PF are read while step i computes (sched_barrier keeps the reads where
// they are written).  Staged bf16 values stay raw 16-bit registers until they
// are written to LDS (a widening next to the load would wait for it there).
// With 2 states per lane the backward keeps the block's (u, delta, dy) and
// (without the gate) B in registers from its recompute sweep, so the adjoint
// sweep reads only C from LDS.  Sums
// over channel blocks (dB, dC, broadcast ddelta) and over rows / segments
// (dA, dD) go through partial buffers reduced in a fixed order, so every
// gradient is deterministic.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <algorithm>
#include <cstdio>
#include <mutex>
#include <string>
#include <type_traits>

#include "../../include/selectssm.h"
#include "common.h"

namespace {

using namespace ssm;

constexpr int kWave = 64;
constexpr int kBlkCh = 64;    // channels per workgroup
constexpr int kFwdWaves = 4;  // forward: 16 channels x 4 state rows per wave
constexpr int kBwdWaves = 8;  // backward: 8 channels x 8 state groups per wave
#ifndef SSM_FWD_TT
#define SSM_FWD_TT 32
#endif
constexpr int kTT = SSM_FWD_TT;  // forward time tile
#ifndef SSM_CK
#define SSM_CK 16
#endif
constexpr int kCK = SSM_CK;   // checkpoint interval = backward block length
// ssm_bwd_pair: 1 runs both calls' main passes as one launch when they allow it;
// 0 (default) one launch per call.  The backward already has two waves per SIMD
// with one call: the joint launch measured equal at op level (config 2) and
// 0.2 ms slower per BidirectionalMamba step (config-2 module, gated build).
// The aggregate passes of a pair always share a launch.
#ifndef SSM_PAIR_JOINT_BWD_MAIN
#define SSM_PAIR_JOINT_BWD_MAIN 0
#endif
#ifndef SSM_FWD_PF
#define SSM_FWD_PF 2
#endif
#ifndef SSM_FWD_APIPE
#define SSM_FWD_APIPE 1  // forward: decays of step i + 1 computed during step i
#endif
#ifndef SSM_BWD_PF
#define SSM_BWD_PF 1
#endif
// backward: the channel sums of step i are issued with step i + 1's compute,
// so their dependent DPP chains interleave with independent work
#ifndef SSM_BWD_PIPE
#define SSM_BWD_PIPE 1
#endif

// S consecutive floats of LDS (16-byte aligned when S >= 4) into registers
template <int S>
__device__ __forceinline__ void lds_vec(const float* p, float (&v)[S]) {
  if constexpr (S == 1) {
    v[0] = p[0];
  } else if constexpr (S == 2) {
    const float2 t = *reinterpret_cast<const float2*>(p);
    v[0] = t.x;
    v[1] = t.y;
  } else {
    static_assert(S % 4 == 0, "vector of 1, 2 or a multiple of 4 floats");
#pragma unroll
    for (int k = 0; k < S / 4; ++k) {
      const float4 t = reinterpret_cast<const float4*>(p)[k];
      v[4 * k] = t.x;
      v[4 * k + 1] = t.y;
      v[4 * k + 2] = t.z;
      v[4 * k + 3] = t.w;
    }
  }
}

// A segment's running decay product is flushed to zero once it falls below
// the smallest normal float (2^-126), as in flush-to-zero arithmetic: with
// subnormals kept, a product whose step factors exceed 1/2 stalls at the
// smallest subnormal instead of reaching 0.  What the flush drops is below
// 2^-126 times the later terms; it would matter only if the remaining decays
// grew by some 2^100 within the segment, which A <= 0, delta >= 0 rule out.
template <int S>
__device__ __forceinline__ void flush_tiny(float (&P)[S]) {
#pragma unroll
  for (int j = 0; j < S; ++j) P[j] = P[j] < 0x1p-126f ? 0.0f : P[j];
}

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
  T* ypre;       // gated residual: y before the gate, (B,L,D) in the output map (or null)
  float* agg_H;  // [B][nseg][N][D]: state at the end of each segment from a zero start
  float* agg_P;  // [B][nseg][N][D]: product of the segment's decays a_t
  int L, D, N, nblk;
  int ldy, ldz;       // row strides (elements) of y and z
  int ldbc;           // row stride (elements) of B and C
  int seg_len, nseg;  // time segments per row (seg_len a multiple of kTT)
  int asub;           // aggregate walks per segment (agg_H / agg_P: [B][nseg * asub][N][D])
  int* aflag;         // [B][nseg * asub][ncb] with asub > 1 (else null): 1 once a piece's products are all 0
  int dstride;        // 1, or 0 for a (B,L,1) delta
  uint32_t flags;
};

// The arguments of the call a workgroup belongs to, picked field by field from
// the two calls of a launch (a select of the structs' addresses would copy
// both to scratch memory; per-field selects of uniform values stay in SGPRs).
#define SSM_FWD_FIELDS(X)                                                                                     \
  X(u) X(delta) X(A) X(Bc) X(Cc) X(Dskip) X(z) X(y) X(ckpt) X(ypre) X(agg_H) X(agg_P) X(L) X(D) X(N) X(nblk)  \
  X(ldy) X(ldz) X(ldbc) X(seg_len) X(nseg) X(asub) X(aflag) X(dstride) X(flags)
template <typename T>
__device__ __forceinline__ FwdArgs<T> pick_args(const FwdArgs<T>& a0, const FwdArgs<T>& a1, bool second) {
  FwdArgs<T> r;
#define SSM_PICK(f) r.f = second ? a1.f : a0.f;
  SSM_FWD_FIELDS(SSM_PICK)
  return r;
}

// Staging of a forward tile (kTT steps x 64 channels) by the 256 threads:
// thread -> column scol (channel cb*64 + scol), rows srow0 + k*4, k < 8.  A
// wave loads whole 64-channel rows, so each load instruction is 256
// contiguous bytes (fp32).
struct FwdStage {
  static constexpr int NT = kWave * kFwdWaves;
  static constexpr int RPT = kTT * kBlkCh / NT;
  static constexpr int RSTEP = NT / kBlkCh;
};

// Workgroup (cb, b, seg) scans time segment seg of its 64 channels, starting
// from the state the earlier segments hand over (folded from their
// aggregates, ssm_fwd_agg_kernel), and writes y and the checkpoints.
// SPL: states per lane (N <= 4 * SPL).  EPI: the extra staging of the reverse
// skip and the gate.  SP: delta arrives before softplus (SSM_DELTA_SOFTPLUS).
// VEC: u and delta rows are read as aligned 4-element vectors (D % 4 == 0,
// per-channel delta); chosen per launch, so every tile stages the same way.
// Workgroups with blockIdx.y < rows0 scan rows of p0, the others rows of p1
// (blockIdx.y - rows0): both directions of a BidirectionalMamba pass in one
// launch.  A single call passes its arguments twice.
template <int SPL, bool EPI, bool SP, bool VEC, typename T>
__global__ void __launch_bounds__(kWave* kFwdWaves, 1) ssm_fwd_kernel(FwdArgs<T> p0, FwdArgs<T> p1, int rows0) {
  const bool second = (int)blockIdx.y >= rows0;
  const FwdArgs<T> p = pick_args<T>(p0, p1, second);
  constexpr int NS = 4 * SPL;  // padded state count
  constexpr int NT = FwdStage::NT, RPT = FwdStage::RPT, RSTEP = FwdStage::RSTEP;
  constexpr int BCN = kTT * NS;                 // staged B (or C) elements per tile
  constexpr int BCE = (BCN + NT - 1) / NT;      // per thread
  constexpr int PF = SSM_FWD_PF;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;
  const int g = lane >> 4;
  const int b = second ? (int)blockIdx.y - rows0 : (int)blockIdx.y;
  const int cb = blockIdx.x;
  const int seg = blockIdx.z;
  const int L = p.L, D = p.D, N = p.N;
  const int t_lo = seg * p.seg_len;
  const int t_hi = min(L, t_lo + p.seg_len);
  const int cw = wave * 16 + c;  // channel within the block
  const int d = cb * kBlkCh + cw;
  const bool valid = d < D;
  const int dc = valid ? d : 0;
  // output map: time (rev) and channel (comp) reversal of the scan position
  const bool rev = p.flags & SSM_REVERSE;
  const bool comp = (p.flags & SSM_COMPLEMENT) != 0;
  // skip source map: the skip adds u at this map of the scan position (and D of
  // its channel); by default the output position itself, the reference's quirk
  const bool smap = (p.flags & SSM_SKIP_MAP) != 0;
  const bool srev = smap ? (p.flags & SSM_SKIP_REVERSE) != 0 : rev;
  const bool scomp = smap ? (p.flags & SSM_SKIP_COMPLEMENT) != 0 : comp;
  // the skip from the scan position uses the staged u itself; any other skip
  // source and the gate need the extra per-lane loads of EPI builds
  const bool skip = (p.flags & SSM_SKIP) != 0;
  const bool gate = EPI && (p.flags & SSM_GATE);
  const bool stage_eu = EPI && skip && (srev || scomp);  // the skip's u is another element
  const int q = comp ? D - 1 - dc : dc;                  // output channel of this lane
  const float Dq = (skip && valid) ? p.Dskip[scomp ? D - 1 - dc : dc] : 0.0f;
  const int scol = tid & (kBlkCh - 1);
  const int srow0 = wave;  // = tid / kBlkCh: the staged rows of a wave are uniform
  const int sd = cb * kBlkCh + scol;
  const bool svalid = sd < D;
  const int sdc = svalid ? sd : 0;
  const bool full_cb = (cb + 1) * kBlkCh <= D;

  float A2[SPL], h[SPL];
#pragma unroll
  for (int j = 0; j < SPL; ++j) {
    const int n = SPL * g + j;
    A2[j] = (valid && n < N) ? p.A[dc * N + n] * kLog2e : 0.0f;
    h[j] = 0.0f;
  }
  if (seg > 0) {
    // state entering this segment: h = P h + H over the earlier segments'
    // aggregate pieces in order (the combine of selectssm.py:81-85 applied to
    // whole pieces)
    const int64_t base = (int64_t)b * p.nseg * p.asub * N * D + dc;
#pragma unroll 2
    for (int s = 0; s < seg * p.asub; ++s) {
#pragma unroll
      for (int j = 0; j < SPL; ++j) {
        const int64_t o = base + ((int64_t)s * N + min(SPL * g + j, N - 1)) * D;
        h[j] = fmaf(p.agg_P[o], h[j], p.agg_H[o]);
      }
    }
#pragma unroll
    for (int j = 0; j < SPL; ++j)
      if (!(valid && SPL * g + j < N)) h[j] = 0.0f;
  }

  __shared__ float2 s_ud[2][kTT][kBlkCh];  // (u, delta)
  __shared__ __attribute__((aligned(16))) float s_B[2][kTT][NS];
  __shared__ __attribute__((aligned(16))) float s_C[2][kTT][NS];

  const int dtD = p.dstride ? D : 1;
  const int scol_dt = p.dstride ? sdc : 0;
  const T* __restrict__ u_b = p.u + (int64_t)b * L * D;
  const T* __restrict__ dt_b = p.delta + (int64_t)b * L * dtD;
  const int ldy = p.ldy, ldz = p.ldz;
  const T* __restrict__ z_b = EPI ? p.z + (int64_t)b * L * ldz : nullptr;
  const int ldbc = p.ldbc;
  const T* __restrict__ B_b = p.Bc + (int64_t)b * L * ldbc;
  const T* __restrict__ C_b = p.Cc + (int64_t)b * L * ldbc;
  T* __restrict__ y_b = p.y + (int64_t)b * L * ldy;
  float* __restrict__ ck_b = p.ckpt != nullptr ? p.ckpt + (int64_t)b * p.nblk * N * D : nullptr;
  const int ND = N * D;
  const buf_t ru = make_buf(u_b), rdt = make_buf(dt_b), rB = make_buf(B_b), rC = make_buf(C_b);
  const buf_t rz = make_buf(EPI ? z_b : u_b), ry = make_buf(y_b), rck = make_buf(ck_b != nullptr ? ck_b : p.A);
  const uint32_t cb_c = (uint32_t)(sdc * sizeof(T));
  const uint32_t cb_dt = (uint32_t)(scol_dt * sizeof(T));

  // fetch() only issues loads (clamped addresses, raw values); commit(), run
  // after the tile's compute, zeroes what lies outside the tensor and writes
  // LDS, so the loads' latency is covered by a whole tile.  VEC launches read
  // u and delta as 4-element vectors: thread -> rows vr, vr + 16, channels
  // vc .. vc + 3 (D % 4 == 0, so a vector is wholly inside or outside D).
  stg<T> r_u[RPT], r_dt[RPT], r_B[BCE], r_C[BCE];
  // EPI builds: z (gate) and the skip's u at another element (skip maps) at
  // this lane's own output steps of the tile, one per 4-step group, loaded by
  // the fetch straight into registers (no LDS staging: the gated forward keeps
  // the plain forward's LDS size, and so its waves per SIMD) and converted by
  // the commit
  constexpr int KG = EPI ? kTT / 4 : 1;
  const int yoff = yrow_step(g);  // step of each 4-step group this lane's row ends with
  const uint32_t lq = (uint32_t)(q * sizeof(T)), lqs = (uint32_t)((scomp ? D - 1 - dc : dc) * sizeof(T));
  stg<T> zn[KG], en[KG];
  float zc[KG], ec[KG];
  constexpr int VK = kTT / 16;  // vector rows per thread
  stg4<T> v_u[VK], v_dt[VK];
  static_assert(NT == 256 && kTT % 16 == 0, "vector staging: 16 threads per row, 16 rows per pass");
  const int vr = tid >> 4, vc = (tid & 15) * 4;
  const bool vin = cb * kBlkCh + vc < D;
  const uint32_t vcb = (uint32_t)((vin ? cb * kBlkCh + vc : 0) * sizeof(T));
  const uint32_t rowb = (uint32_t)(D * sizeof(T));  // bytes per (B,L,D) row
  auto fetch = [&](int t0) {
    if constexpr (VEC) {
#pragma unroll
      for (int k = 0; k < VK; ++k) {
        const uint32_t o = (uint32_t)min(t0 + vr + 16 * k, L - 1) * rowb + vcb;
        v_u[k] = bld4r<T>(ru, o, 0);
        v_dt[k] = bld4r<T>(rdt, o, 0);
      }
    } else {
#pragma unroll
      for (int k = 0; k < RPT; ++k) {
        const int tc = min(t0 + srow0 + k * RSTEP, L - 1);  // wave-uniform
        r_u[k] = bldr<T>(ru, cb_c, (uint32_t)tc * rowb);
        r_dt[k] = bldr<T>(rdt, cb_dt, (uint32_t)(tc * dtD * sizeof(T)));
      }
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = tid + k * NT;
      if (BCN % NT == 0 || e < BCN) {
        const int i = e / NS, n = e - (e / NS) * NS;
        const uint32_t o = (uint32_t)((min(t0 + i, L - 1) * ldbc + min(n, N - 1)) * sizeof(T));
        r_B[k] = bldr<T>(rB, o, 0);
        r_C[k] = bldr<T>(rC, o, 0);
      }
    }
    if constexpr (EPI) {
      if (stage_eu || gate) {
#pragma unroll
        for (int k = 0; k < KG; ++k) {
          const int tc = min(t0 + 4 * k + yoff, L - 1);  // this lane's output step of group k
          const int pr = rev ? L - 1 - tc : tc;    // output row (z)
          const int prs = srev ? L - 1 - tc : tc;  // skip-source row (u)
          if (stage_eu) en[k] = bldr<T>(ru, lqs, (uint32_t)prs * rowb);
          if (gate) zn[k] = bldr<T>(rz, lq, (uint32_t)(pr * ldz * sizeof(T)));
        }
      }
    }
  };
  auto commit = [&](int buf, int t0) {
    if constexpr (VEC) {
#pragma unroll
      for (int k = 0; k < VK; ++k) {
        const bool in = vin && t0 + vr + 16 * k < L;
        const float4 uv = val(v_u[k]), dr = val(v_dt[k]);
        const float4 dv = SP ? make_float4(softplus(dr.x), softplus(dr.y), softplus(dr.z), softplus(dr.w)) : dr;
        float4* dst = reinterpret_cast<float4*>(&s_ud[buf][vr + 16 * k][vc]);
        dst[0] = in ? make_float4(uv.x, dv.x, uv.y, dv.y) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        dst[1] = in ? make_float4(uv.z, dv.z, uv.w, dv.w) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    } else {
#pragma unroll
      for (int k = 0; k < RPT; ++k) {
        const int i = srow0 + k * RSTEP;
        const bool in = svalid && t0 + i < L;
        const float dv = SP ? softplus(val(r_dt[k])) : val(r_dt[k]);
        s_ud[buf][i][scol] = in ? make_float2(val(r_u[k]), dv) : make_float2(0.0f, 0.0f);
      }
    }
    if constexpr (EPI) {
#pragma unroll
      for (int k = 0; k < KG; ++k) {
        zc[k] = gate ? val(zn[k]) : 0.0f;
        ec[k] = stage_eu ? val(en[k]) : 0.0f;
      }
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = tid + k * NT;
      if (BCN % NT == 0 || e < BCN) {
        const int i = e / NS, n = e - (e / NS) * NS;
        const bool in = t0 + i < L && n < N;
        (&s_B[buf][0][0])[e] = in ? val(r_B[k]) : 0.0f;
        (&s_C[buf][0][0])[e] = in ? val(r_C[k]) : 0.0f;
      }
    }
  };

  // y of step t0 + i - 3 + yoff is stored at row t0 + i - 3 + yoff, or with
  // the reverse map at L-1-(t0+i) + (3 - yoff): a uniform row plus this offset
  const uint32_t yo = (uint32_t)(((rev ? 3 - yoff : yoff) * ldy + q) * sizeof(T));
  const uint32_t yrowb = (uint32_t)(ldy * sizeof(T));
  // the gated residual, y before the gate: dense (B,L,D) rows in the output map
  T* __restrict__ yp_b = EPI && p.ypre != nullptr ? p.ypre + (int64_t)b * L * D : nullptr;
  const buf_t ryp = make_buf(yp_b != nullptr ? yp_b : y_b);
  const uint32_t ypo = (uint32_t)(((rev ? 3 - yoff : yoff) * D + q) * sizeof(T));
  uint32_t cko[SPL];  // checkpoint offsets of this lane's states within a block
#pragma unroll
  for (int j = 0; j < SPL; ++j) cko[j] = (uint32_t)(((SPL * g + j) * D + d) * sizeof(float));
  const uint32_t ckrowb = (uint32_t)(ND * sizeof(float));  // bytes per checkpoint block
  // segments start on tile boundaries (seg_len is a multiple of kTT), so
  // only the tile at L can be partial; its steps beyond L are zeros, which
  // leave h unchanged, and are not stored
  fetch(t_lo);
  commit(0, t_lo);
  __syncthreads();
  int buf = 0;
  for (int t0 = t_lo; t0 < t_hi; t0 += kTT, buf ^= 1) {
    const bool more = t0 + kTT < t_hi;
    if (more) fetch(t0 + kTT);
    // a full tile (every channel and state exists, no step beyond L) runs
    // without per-lane predicates; tiles of a launch without checkpoints
    // (inference) skip their stores
    const bool full = full_cb && N == NS && t0 + kTT <= L;
    auto tile = [&](auto full_tag, auto ck_tag, auto yp_tag) {
      constexpr bool kFull = decltype(full_tag)::value;
      constexpr bool kCkpt = decltype(ck_tag)::value;
      constexpr bool kYp = EPI && decltype(yp_tag)::value;  // store the gated residual
      // operands of steps i .. i + PF + 1 in a ring of PF + 2 register sets;
      // (u, delta) of two steps are read by one LDS instruction
      static_assert(PF % 2 == 0, "operands are prefetched in step pairs");
      constexpr int R = PF + 2;
      float2 ud[R];
      float Cq[R][SPL];
      // B of the tile in registers: lane c of state row g holds B of step
      // 16 hh + c for the row's states; step i broadcasts lane i % 16 of its
      // row (row_bcast) straight into the B * (delta u) multiply, so B costs
      // one LDS read per 16 steps instead of one per step
      static_assert(kTT % 16 == 0, "B is held in 16-step register tiles");
      float Bt[kTT / 16][SPL];
#pragma unroll
      for (int hh = 0; hh < kTT / 16; ++hh) lds_vec<SPL>(&s_B[buf][16 * hh + c][SPL * g], Bt[hh]);
      auto pre = [&](int i) {  // steps i, i + 1 (i even)
        ud[i % R] = s_ud[buf][i][cw];
        ud[(i + 1) % R] = s_ud[buf][i + 1][cw];
#pragma unroll
        for (int k = 0; k < 2; ++k) lds_vec<SPL>(&s_C[buf][i + k][SPL * g], Cq[(i + k) % R]);
      };
#pragma unroll
      for (int i = 0; i < PF; i += 2) pre(i);
      float yp[4];
      float an[SPL];  // decays of the next step
      // epilogue operands of the current 4-step group at this lane's output
      // step, read at the group's first step so their LDS latency is covered
      float uo = 0.0f, zo = 0.0f;
      // running row offsets of the y and checkpoint stores (scalars)
      uint32_t yro = (uint32_t)(rev ? L - 4 - t0 : t0) * yrowb;
      const uint32_t ystep = rev ? 0u - 4u * yrowb : 4u * yrowb;
      uint32_t ypro = (uint32_t)(rev ? L - 4 - t0 : t0) * rowb;
      const uint32_t ypstep = rev ? 0u - 4u * rowb : 4u * rowb;
      uint32_t cro = (uint32_t)(t0 / kCK) * ckrowb;
#pragma unroll
      for (int i = 0; i < kTT; ++i) {
        if (i % 2 == 0 && i + PF < kTT) pre(i + PF);
        if ((i & 3) == 0) {
          // skip (Dq is 0 without it): u at the output position, which the
          // reverse map makes another element (staged in EPI builds)
          const int ti = i + yoff;
          if constexpr (EPI) {
            // z and the skip's u at another element come from registers; z is
            // taken (and discarded below) without the gate as well
            const float us = s_ud[buf][ti][cw].x;
            uo = stage_eu ? ec[i >> 2] : us;
            zo = zc[i >> 2];
          } else {
            uo = s_ud[buf][ti][cw].x;
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (kCkpt && (i % kCK) == 0 && (kFull || t0 + i < L)) {
#pragma unroll
          for (int j = 0; j < SPL; ++j) {
            const int n = SPL * g + j;
            if (kFull || (valid && n < N)) bst<float>(rck, cko[j], cro, h[j]);
          }
          cro += ckrowb;
        }
        const float uu = ud[i % R].x, dd = ud[i % R].y;
        const float w = dd * uu;
        float a[SPL];
#pragma unroll
        for (int j = 0; j < SPL; ++j) a[j] = SSM_FWD_APIPE && i > 0 ? an[j] : fast_exp2(A2[j] * dd);
        if (SSM_FWD_APIPE && i + 1 < kTT) {
          // the next step's decays, a step ahead of their use
          const float dn = ud[(i + 1) % R].y;
#pragma unroll
          for (int j = 0; j < SPL; ++j) an[j] = fast_exp2(A2[j] * dn);
        }
        float ys = 0.0f;
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
          h[j] = fmaf(a[j], h[j], row_bcast(Bt[i / 16][j], i) * w);
          ys = j == 0 ? Cq[i % R][0] * h[0] : fmaf(Cq[i % R][j], h[j], ys);
        }
        yp[i & 3] = ys;
        if constexpr (EPI) {
          // the gate factor z sigmoid(z) (1 without the gate), two steps
          // after its read and ahead of its use
          if ((i & 3) == 2) zo = gate ? zo * sigmoid(zo) : 1.0f;
        }
        if ((i & 3) == 3) {
          // y of steps i-3..i summed over the state rows: this lane's row holds step ti
          float yv = rows_transpose_sum4(yp[0], yp[1], yp[2], yp[3]);
          const int ti = i - 3 + yoff;
          const int t = t0 + ti;
          yv = fmaf(uo, Dq, yv);
          if constexpr (kYp) {
            if constexpr (kFull) {
              bst<T>(ryp, ypo, ypro, yv);
              ypro += ypstep;
            } else if (valid && t < L) {
              bst<T>(ryp, (uint32_t)(rev ? L - 1 - t : t) * rowb + (uint32_t)(q * sizeof(T)), 0, yv);
            }
          }
          if constexpr (EPI) yv *= zo;
          if constexpr (kFull) {
            // row t0+i-3 (or L-1-(t0+i) >= 0 with the reverse map) plus the lane's yo
            bst<T>(ry, yo, yro, yv);
            yro += ystep;
          } else if (valid && t < L) {
            bst<T>(ry, (uint32_t)(rev ? L - 1 - t : t) * yrowb + (uint32_t)(q * sizeof(T)), 0, yv);
          }
        }
      }
    };
    constexpr std::true_type yes{};
    constexpr std::false_type no{};
    if (ck_b == nullptr) {
      if (full) tile(yes, no, no); else tile(no, no, no);
    } else if constexpr (EPI) {
      if (yp_b != nullptr) {
        if (full) tile(yes, yes, yes); else tile(no, yes, yes);
      } else {
        if (full) tile(yes, yes, no); else tile(no, yes, no);
      }
    } else {
      if (full) tile(yes, yes, no); else tile(no, yes, no);
    }
    if (more) commit(buf ^ 1, t0 + kTT);
    __syncthreads();
  }
}

// Forward aggregate pass of a time-split scan.  Workgroup (cb, b, seg), for
// segments seg < nseg - 1, writes the segment's state at its end from a zero
// start, H = sum_t P_t B_t delta_t u_t with P_t the product of the decays
// after step t, and the whole segment's decay product P.  It walks the segment
// from its end a tile at a time (P: the product of the decays after the tile;
// H += P times the tile's own sum, then P *= the tile's decay), so once every
// P of the workgroup is 0 (flushed at tile ends, flush_tiny) all earlier
// steps add exact zeros and the walk stops there: with decaying states only
// the last few thousand steps of a long segment are read.
//
// With asub > 1 the segment is walked in asub pieces (workgroup z selects the
// piece), each into its own (H, P); the main pass folds them in order.  When
// a piece's products all end at 0 it raises its flag, and the piece before
// it in the segment, whose contributions reach the segment's end only through
// those products (an exact 0 times a finite value), stops and writes H = P = 0:
// the fold then gives the same floats.  The pieces at the segments' ends are
// dispatched first; with fast decays an earlier piece, polling once per tile,
// then stops as soon as the piece after it has flushed instead of walking
// until its own products flush.
template <int SPL, bool SP, typename T>
__device__ __forceinline__ void fwd_agg_body(const FwdArgs<T>& p, const int b) {
  constexpr int NS = 4 * SPL;
  constexpr int NT = FwdStage::NT, RPT = FwdStage::RPT, RSTEP = FwdStage::RSTEP;
  constexpr int BCN = kTT * NS;
  constexpr int BCE = (BCN + NT - 1) / NT;
  constexpr int PF = SSM_FWD_PF;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;
  const int g = lane >> 4;
  // b: the batch row (blockIdx.y of a single launch)
  const int cb = blockIdx.x;
  // blockIdx.z = (asub - 1 - part) * (nseg - 1) + segment, for segments
  // 0 .. nseg - 2: every segment's last piece first
  const int nsg = p.nseg - 1;
  const int zq = blockIdx.z / nsg;
  const int part = p.asub - 1 - zq;
  const int seg = (blockIdx.z - zq * nsg) * p.asub + part;  // aggregate piece of the row
  const int L = p.L, D = p.D, N = p.N;
  const int alen = p.seg_len / p.asub;
  const int t_lo = seg * alen;
  const int t_hi = min(L, t_lo + alen);
  int* const fl = p.aflag ? p.aflag + ((int64_t)b * p.nseg * p.asub + seg) * gridDim.x + cb : nullptr;
  const int* const fnext = fl && part < p.asub - 1 ? fl + gridDim.x : nullptr;  // the next piece's flag
  const int cw = wave * 16 + c;
  const int d = cb * kBlkCh + cw;
  const bool valid = d < D;
  const int dc = valid ? d : 0;
  const int scol = tid & (kBlkCh - 1);
  const int srow0 = wave;  // = tid / kBlkCh: the staged rows of a wave are uniform
  const int sd = cb * kBlkCh + scol;
  const bool svalid = sd < D;
  const int sdc = svalid ? sd : 0;

  float A2[SPL], H[SPL], P[SPL];
  bool live[SPL];
#pragma unroll
  for (int j = 0; j < SPL; ++j) {
    live[j] = valid && SPL * g + j < N;
    A2[j] = live[j] ? p.A[dc * N + SPL * g + j] * kLog2e : 0.0f;
    H[j] = 0.0f;
    P[j] = 1.0f;
  }

  __shared__ float2 s_ud[2][kTT][kBlkCh];
  __shared__ __attribute__((aligned(16))) float s_B[2][kTT][NS];
  __shared__ int s_alive[2][kFwdWaves];

  const int dtD = p.dstride ? D : 1;
  const int scol_dt = p.dstride ? sdc : 0;
  const T* __restrict__ u_b = p.u + (int64_t)b * L * D;
  const T* __restrict__ dt_b = p.delta + (int64_t)b * L * dtD;
  const int ldbc = p.ldbc;
  const T* __restrict__ B_b = p.Bc + (int64_t)b * L * ldbc;
  const buf_t ru = make_buf(u_b), rdt = make_buf(dt_b), rB = make_buf(B_b);
  const uint32_t so_c = (uint32_t)(sdc * sizeof(T)), so_dt = (uint32_t)(scol_dt * sizeof(T));
  const uint32_t rowb = (uint32_t)(D * sizeof(T)), dtrowb = (uint32_t)(dtD * sizeof(T));

  stg<T> r_u[RPT], r_dt[RPT], r_B[BCE];
  auto fetch = [&](int t0) {
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int tc = min(t0 + srow0 + k * RSTEP, L - 1);  // wave-uniform
      r_u[k] = bldr<T>(ru, so_c, (uint32_t)tc * rowb);
      r_dt[k] = bldr<T>(rdt, so_dt, (uint32_t)tc * dtrowb);
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = tid + k * NT;
      if (BCN % NT == 0 || e < BCN) {
        const int i = e / NS, n = e - (e / NS) * NS;
        r_B[k] = bldr<T>(rB, (uint32_t)((min(t0 + i, L - 1) * ldbc + min(n, N - 1)) * sizeof(T)), 0);
      }
    }
  };
  auto commit = [&](int buf, int t0) {
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int i = srow0 + k * RSTEP;
      const bool in = svalid && t0 + i < L;
      const float dv = SP ? softplus(val(r_dt[k])) : val(r_dt[k]);
      s_ud[buf][i][scol] = in ? make_float2(val(r_u[k]), dv) : make_float2(0.0f, 0.0f);
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = tid + k * NT;
      if (BCN % NT == 0 || e < BCN) {
        const int i = e / NS, n = e - (e / NS) * NS;
        (&s_B[buf][0][0])[e] = (t0 + i < L && n < N) ? val(r_B[k]) : 0.0f;
      }
    }
  };

  const int t_last = t_lo + (t_hi - 1 - t_lo) / kTT * kTT;
  fetch(t_last);
  commit(0, t_last);
  __syncthreads();
  int buf = 0, vote = 0;
  for (int t0 = t_last;; t0 -= kTT, buf ^= 1) {
    const bool more = t0 > t_lo;
    // read now, used at the tile's end: the load's latency hides behind the tile
    const bool nflush = fnext && __hip_atomic_load(fnext, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
    if (more) fetch(t0 - kTT);
    constexpr int R = PF + 1;
    float2 ud[R];
    float Bq[R][SPL];
    auto pre = [&](int i) {
      ud[i % R] = s_ud[buf][i][cw];
      lds_vec<SPL>(&s_B[buf][i][SPL * g], Bq[i % R]);
    };
#pragma unroll
    for (int k = 0; k < PF; ++k) pre(kTT - 1 - k);
    // the tile's terms relative to its end: Ht = sum_i e_i B_i delta_i u_i
    // with e_i = exp2(A log2(e) s_i), s_i the sum of the tile's deltas after
    // step i; then H += P Ht and P *= exp2(A log2(e) s) once per tile.  One
    // exponential per state and step as before, and no running product.
    float Ht[SPL], s = 0.0f;
#pragma unroll
    for (int j = 0; j < SPL; ++j) Ht[j] = 0.0f;
#pragma unroll
    for (int i = kTT - 1; i >= 0; --i) {
      if (i - PF >= 0) pre(i - PF);
      __builtin_amdgcn_sched_barrier(0);
      const float uu = ud[i % R].x, dd = ud[i % R].y;
      const float w = dd * uu;
#pragma unroll
      for (int j = 0; j < SPL; ++j) Ht[j] = fmaf(fast_exp2(A2[j] * s), Bq[i % R][j] * w, Ht[j]);
      s += dd;
#pragma unroll
      for (int j = 0; j < SPL; ++j) pin(Ht[j]);
    }
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
      H[j] = fmaf(P[j], Ht[j], H[j]);
      P[j] *= fast_exp2(A2[j] * s);
    }
    if (more) commit(buf ^ 1, t0 - kTT);
    // products below the smallest normal float are flushed to zero; every
    // earlier step then adds an exact zero, so the walk ends once all are 0
    flush_tiny(P);
    bool alive = false;
#pragma unroll
    for (int j = 0; j < SPL; ++j) alive = alive || (live[j] && P[j] != 0.0f);
    // bit 0: a product of the workgroup is still live; bit 1: the next piece's are all 0
    vote = barrier_or<kFwdWaves>((__ballot(alive) != 0 ? 1 : 0) | (nflush ? 2 : 0), s_alive[buf]);
    if (vote != 1 || !more) break;
  }
  const bool stop = (vote & 2) != 0;
  const int64_t o = (int64_t)b * p.nseg * p.asub + seg;
#pragma unroll
  for (int j = 0; j < SPL; ++j) {
    if (live[j]) {
      p.agg_H[(o * N + SPL * g + j) * D + d] = stop ? 0.0f : H[j];
      p.agg_P[(o * N + SPL * g + j) * D + d] = stop ? 0.0f : P[j];
    }
  }
  if (fl && (stop || (vote & 1) == 0) && tid == 0)
    __hip_atomic_store(fl, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroups with blockIdx.y < rows0 aggregate rows of p0, the others rows of
// p1 (blockIdx.y - rows0): both directions of a BidirectionalMamba pass run
// their aggregate walks in one launch.  A single launch passes p0 twice.
template <int SPL, bool SP, typename T>
__global__ void __launch_bounds__(kWave* kFwdWaves, 1) ssm_fwd_agg_kernel(FwdArgs<T> p0, FwdArgs<T> p1,
                                                                         int rows0) {
  const int y = blockIdx.y;
  if (y < rows0) fwd_agg_body<SPL, SP, T>(p0, y);
  else fwd_agg_body<SPL, SP, T>(p1, y - rows0);
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
  const T* ypre;  // gated residual: y before the gate, written by the forward (or null)
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
  int ldbc;       // row stride (elements) of B and C
  int seg_len, nseg;
  int asub;    // aggregate walks per segment (agg_G / agg_P: [B][nseg * asub][N][D])
  int* aflag;  // [B][nseg * asub][ncb] with asub > 1 (else null): 1 once a piece's products are all 0
  int dstride;
  uint32_t flags;
};

#define SSM_BWD_FIELDS(X)                                                                                     \
  X(u) X(delta) X(A) X(Bc) X(Cc) X(Dskip) X(z) X(ckpt) X(ypre) X(dy) X(du) X(ddelta) X(dz) X(ws_dB) X(ws_dC)  \
  X(ws_dA) X(ws_dD) X(ws_ddt) X(agg_G) X(agg_P) X(Bt) X(L) X(D) X(N) X(nblk) X(ncb) X(ldy) X(ldz) X(ldbc)     \
  X(seg_len) X(nseg) X(asub) X(aflag) X(dstride) X(flags)
template <typename T>
__device__ __forceinline__ BwdArgs<T> pick_args(const BwdArgs<T>& a0, const BwdArgs<T>& a1, bool second) {
  BwdArgs<T> r;
  SSM_BWD_FIELDS(SSM_PICK)
  return r;
}
#undef SSM_PICK

// Staging of a backward block (kCK steps x 64 channels) by the 512 threads:
// thread -> column scol, rows srow0 + k*8, k < 2.
struct BwdStage {
  static constexpr int NT = kWave * kBwdWaves;
  static constexpr int RPT = kCK * kBlkCh / NT;
  static constexpr int RSTEP = NT / kBlkCh;
};

// Workgroup (cb, b, seg) walks the blocks of time segment seg of its 64
// channels in reverse, starting from the adjoint carry the later segments
// hand over (ssm_bwd_agg_kernel), and writes du, ddelta, dz and the partial
// sums of dB, dC, dA, dD (and of a broadcast ddelta).
// SPL: states per lane (N <= 8 * SPL).  EPI: the gate (dz formed in the
// staging pass from the forward's residual y before the gate) and skip source
// maps.  BC: delta is (B,L,1), shared by the channels.  ACC (with EPI): dz +=
// the gate's gradient (SSM_ACCUMULATE), a build of its own.
// Rows of p0 below rows0, rows of p1 above, as ssm_fwd_kernel.
template <int SPL, bool EPI, bool BC, bool ACC, typename T>
__global__ void __launch_bounds__(kWave* kBwdWaves, 1) ssm_bwd_kernel(BwdArgs<T> p0, BwdArgs<T> p1, int rows0) {
  static_assert(EPI || !ACC, "dz is accumulated only by the gated (EPI) builds");
  const bool second = (int)blockIdx.y >= rows0;
  const BwdArgs<T> p = pick_args<T>(p0, p1, second);
  constexpr int NS = 8 * SPL;
  constexpr int NT = BwdStage::NT, RPT = BwdStage::RPT, RSTEP = BwdStage::RSTEP;
  constexpr int BCN = kCK * NS;
  constexpr int BCE = (BCN + NT - 1) / NT;
  constexpr int EB = EPI ? 2 : 1;
  constexpr int ER = EPI ? kCK : 1;
  constexpr int PF = SSM_BWD_PF;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 7;
  const int g = lane >> 3;
  const int b = second ? (int)blockIdx.y - rows0 : (int)blockIdx.y;
  const int cb = blockIdx.x;
  const int seg = blockIdx.z;
  const int L = p.L, D = p.D, N = p.N;
  const int blk_lo = seg * (p.seg_len / kCK);
  const int blk_hi = min(p.nblk, blk_lo + p.seg_len / kCK);
  const int cw = wave * 8 + c;
  const int d = cb * kBlkCh + cw;
  const bool valid = d < D;
  const int dc = valid ? d : 0;
  const int sig = chan_sig<SPL>(c);
  int nj[SPL];  // state of slot j
#pragma unroll
  for (int j = 0; j < SPL; ++j) nj[j] = SPL * g + (j ^ sig);
  // output map (rev, comp) and skip source map (srev, scomp), as in the forward
  const bool rev = p.flags & SSM_REVERSE;
  const bool comp = (p.flags & SSM_COMPLEMENT) != 0;
  const bool smap = (p.flags & SSM_SKIP_MAP) != 0;
  const bool srev = smap ? (p.flags & SSM_SKIP_REVERSE) != 0 : rev;
  const bool scomp = smap ? (p.flags & SSM_SKIP_COMPLEMENT) != 0 : comp;
  const bool gate = EPI && (p.flags & SSM_GATE);
  // dz += the gate's gradient: the old dz at the output position is staged like z
  const bool acc_dz = ACC && gate;
  const bool skip = (p.flags & SSM_SKIP) != 0;  // non-EPI builds run only the skip from the scan position
  // u[t,d] is added (times D[d]) at the output position O(S(t,d)) with S the
  // skip source map: its gradient reads the gated dy there, which is the lane's
  // own staged dy when S is the identity and another element otherwise
  const bool stage_dyo = EPI && skip && (srev || scomp);
  const bool mrev = rev != srev, mcomp = comp != scomp;   // O(S(t,d)) relative to (t,d)
  const bool dsp = p.flags & SSM_DELTA_SOFTPLUS;
  const float Dd = (skip && valid) ? p.Dskip[dc] : 0.0f;  // u[t,d] carries D[d] (selectssm.py:238)
  const int scol = tid & (kBlkCh - 1);
  const int srow0 = wave;  // = tid / kBlkCh: the staged rows of a wave are uniform
  const int sd = cb * kBlkCh + scol;
  const bool svalid = sd < D;
  const int sdc = svalid ? sd : 0;
  const int sq = comp ? D - 1 - sdc : sdc;     // output channel of the staged column
  const int sqm = mcomp ? D - 1 - sdc : sdc;   // channel of O(S(.)) for the skip's gradient
  const bool full_cb = (cb + 1) * kBlkCh <= D;
  // after the exchange over state groups, row g >> 1 of the wave holds
  // du (rows 0, 1) or ddelta (rows 2, 3) of one of 2 steps, twice (both halves)
  const int orow = g >> 1;
  const bool is_du = orow < 2;
  const bool lead = (g & 1) == 0;
  const float Ddu = is_du ? Dd : 0.0f;                  // the skip's du term, on du rows
  const float dmask = (is_du && lead) ? 1.0f : 0.0f;    // one lane per (step, channel) adds to dD
  // du / ddelta of step t0 + i + (1 - (orow & 1)) go to row t0 + i plus this offset
  const uint32_t oo = (uint32_t)((1 - (orow & 1)) * D + d);  // elements

  float Av[SPL], A2[SPL], gc[SPL], dAacc[SPL], dAmid[SPL];
#pragma unroll
  for (int j = 0; j < SPL; ++j) {
    Av[j] = (valid && nj[j] < N) ? p.A[dc * N + nj[j]] : 0.0f;
    A2[j] = Av[j] * kLog2e;
    gc[j] = 0.0f;
    dAacc[j] = 0.0f;
    dAmid[j] = 0.0f;
  }
  if (seg < p.nseg - 1) {
    // adjoint carry entering this segment from the right: g = P g + G over the
    // later segments' aggregate pieces, last first (g = a_t f_t at each piece's first
    // step is linear in the carry it receives)
    const int64_t base = (int64_t)b * p.nseg * p.asub * N * D + dc;
#pragma unroll 2
    for (int s = p.nseg * p.asub - 1; s >= (seg + 1) * p.asub; --s) {
#pragma unroll
      for (int j = 0; j < SPL; ++j) {
        const int64_t o = base + ((int64_t)s * N + min(nj[j], N - 1)) * D;
        gc[j] = fmaf(p.agg_P[o], gc[j], p.agg_G[o]);
      }
    }
#pragma unroll
    for (int j = 0; j < SPL; ++j)
      if (!(valid && nj[j] < N)) gc[j] = 0.0f;
  }
  // dA and dD are sums over every step of the row: per block (16 steps), per
  // group of 16 blocks, then the total, so a 2^20-step row's total sees 4096
  // fp32 adds instead of 2^20
  float dDacc = 0.0f, dDmid = 0.0f;

  __shared__ float4 s_x[2][kCK][kBlkCh];  // (u, delta, dy of the scan, softplus'(delta) or 1)
  // (B, C) of each step in the state order of each lane class: [t][group][sig][B slots, C slots]
  __shared__ __attribute__((aligned(16))) float s_bc[2][kCK][8][SPL][2 * SPL];
  // per-wave channel sums, in two sets where LDS allows (all but N > 16 with
  // the gate): a block's totals are then added after the one barrier that
  // also publishes the next block's staged operands (in the next block, with
  // kLateTotals), while the next block's sweeps write the other set
  constexpr int kSB = (SPL == 4 && EPI) ? 1 : 2;
  int sb = 0;
  // the next block's staging commit runs between the block's two sweeps,
  // except in the gated N > 16 builds (registers already spilled, one LDS set
  // of channel sums), where it follows them
  constexpr bool kMidCommit = !(SPL == 4 && EPI);
  // with two sets and the commit between the sweeps, a block's dB / dC totals
  // are added in the next block, after its commit, instead of right after the
  // block-end barrier, where every wave waited on the same LDS reads at once
  constexpr bool kLateTotals = kSB == 2 && kMidCommit;
  __shared__ float s_dB[kSB][kBwdWaves][kCK][NS], s_dC[kSB][kBwdWaves][kCK][NS];
  __shared__ float s_dyo[EB][ER][kBlkCh];  // skip map: the gated dy at O(S(t,d))
  __shared__ float s_ddt[kSB][kBwdWaves][kCK];  // broadcast delta: per-wave channel sums of ddelta

  const int dtD = p.dstride ? D : 1;
  const int scol_dt = p.dstride ? sdc : 0;
  const T* __restrict__ u_b = p.u + (int64_t)b * L * D;
  const T* __restrict__ dt_b = p.delta + (int64_t)b * L * dtD;
  const int ldy = p.ldy, ldz = p.ldz;
  const T* __restrict__ dy_b = p.dy + (int64_t)b * L * ldy;
  const T* __restrict__ z_b = EPI ? p.z + (int64_t)b * L * ldz : nullptr;
  const int ldbc = p.ldbc;
  const T* __restrict__ B_b = p.Bc + (int64_t)b * L * ldbc;
  const T* __restrict__ C_b = p.Cc + (int64_t)b * L * ldbc;
  const float* __restrict__ ck_b = p.ckpt + (int64_t)b * p.nblk * N * D;
  T* __restrict__ out_b = (is_du ? p.du : p.ddelta) + (int64_t)b * L * D;  // ddelta only when (B,L,D)
  T* __restrict__ dz_b = EPI ? p.dz + (int64_t)b * L * D : nullptr;
  const T* __restrict__ yp_b = EPI && p.ypre != nullptr ? p.ypre + (int64_t)b * L * D : nullptr;  // gated residual

  // fetch() only issues loads; commit() (between the block's sweeps, or after
  // them, kMidCommit) masks, applies softplus and the gate and writes LDS
  stg<T> r_u[RPT], r_dt[RPT], r_dy[RPT], r_gz[RPT], r_yp[RPT], r_dyo[RPT], r_zo[RPT], r_dza[RPT];
  stg<T> r_B[BCE], r_C[BCE];
  float r_h[SPL];
  float h_next[SPL];  // checkpoint of the block staged by the last commit
  // byte offsets of this thread's staged column in a u row and an output row
  const uint32_t so_c = (uint32_t)(sdc * sizeof(T));
  const uint32_t so_q = (uint32_t)(sq * sizeof(T));
  const uint32_t so_dt = (uint32_t)(scol_dt * sizeof(T));
  const buf_t ru = make_buf(u_b), rdt = make_buf(dt_b), rdy = make_buf(dy_b), rB = make_buf(B_b), rC = make_buf(C_b);
  const buf_t rck = make_buf(ck_b);
  const uint32_t rowb = (uint32_t)(D * sizeof(T));      // bytes per (B,L,D) row
  const uint32_t dyrowb = (uint32_t)(ldy * sizeof(T));  // bytes per dy row
  const uint32_t ckrowb = (uint32_t)(N * D * sizeof(float));
  uint32_t cko[SPL];  // checkpoint offsets of this lane's states within a block
#pragma unroll
  for (int j = 0; j < SPL; ++j) cko[j] = (uint32_t)((min(nj[j], N - 1) * D + dc) * sizeof(float));
  auto fetch = [&](int blk) {
    const int t0 = blk * kCK;
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int tc = min(t0 + srow0 + k * RSTEP, L - 1);  // wave-uniform
      const int pr = rev ? L - 1 - tc : tc;              // output row of scan step tc
      r_u[k] = bldr<T>(ru, so_c, (uint32_t)tc * rowb);
      r_dt[k] = bldr<T>(rdt, so_dt, (uint32_t)(tc * dtD * sizeof(T)));
      r_dy[k] = bldr<T>(rdy, so_q, (uint32_t)pr * dyrowb);
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = tid + k * NT;
      if (BCN % NT == 0 || e < BCN) {
        const int i = e / NS, n = e - (e / NS) * NS;
        const uint32_t o = (uint32_t)((min(t0 + i, L - 1) * ldbc + min(n, N - 1)) * sizeof(T));
        r_B[k] = bldr<T>(rB, o, 0);
        r_C[k] = bldr<T>(rC, o, 0);
      }
    }
    if (gate || stage_dyo) {
#pragma unroll
      for (int k = 0; k < RPT; ++k) {
        const int tc = min(t0 + srow0 + k * RSTEP, L - 1);
        const int pr = rev ? L - 1 - tc : tc;     // output row
        const int prm = mrev ? L - 1 - tc : tc;   // row of O(S(.))
        if (gate) {
          r_gz[k] = ld32r(z_b, (uint32_t)(pr * ldz + sq));
          r_yp[k] = ld32r(yp_b, (uint32_t)(pr * D + sq));
        }
        if (acc_dz) r_dza[k] = ld32r(dz_b, (uint32_t)(pr * D + sq));
        if (stage_dyo) {
          r_dyo[k] = ld32r(dy_b, (uint32_t)(prm * ldy + sqm));
          if (gate) r_zo[k] = ld32r(z_b, (uint32_t)(prm * ldz + sqm));
        }
      }
    }
#pragma unroll
    for (int j = 0; j < SPL; ++j) r_h[j] = bld<float>(rck, cko[j], (uint32_t)blk * ckrowb);
  };
  // softplus(delta) and its derivative: a separate copy of the staging loop
  auto stage_x = [&](int buf, int t0, auto sp_tag) {
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int i = srow0 + k * RSTEP;
      const bool in = svalid && t0 + i < L;
      float dtv = val(r_dt[k]), sg = 1.0f;
      if constexpr (decltype(sp_tag)::value) dtv = softplus_sigmoid(dtv, &sg);
      const float go = in ? val(r_dy[k]) : 0.0f;
      float dyg = go;
      if (gate) {
        const float gz = in ? val(r_gz[k]) : 0.0f;
        const float sgz = sigmoid(gz);
        dyg = go * gz * sgz;
        // dz = dy y_pre silu'(z), elementwise: y_pre is the forward's gated
        // residual, at the output position of scan step t0 + i like dy and z
        if (in) {
          const int pr = rev ? L - 1 - (t0 + i) : t0 + i;
          float dzv = go * val(r_yp[k]) * sgz * (1.0f + gz * (1.0f - sgz));
          if (acc_dz) {
            pin(dzv);  // rounded on its own, as a separate dz would be (no fused multiply-add)
            dzv = val(r_dza[k]) + dzv;
          }
          st32(dz_b, (uint32_t)(pr * D + sq), dzv);
        }
      }
      s_x[buf][i][scol] = in ? make_float4(val(r_u[k]), dtv, dyg, sg) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  };
  auto commit = [&](int buf, int blk) {
    const int t0 = blk * kCK;
#pragma unroll
    for (int j = 0; j < SPL; ++j) h_next[j] = (valid && nj[j] < N) ? r_h[j] : 0.0f;
    if (dsp) stage_x(buf, t0, std::true_type{}); else stage_x(buf, t0, std::false_type{});
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int i = srow0 + k * RSTEP;
      const bool in = svalid && t0 + i < L;
      if (stage_dyo) {
        float v = in ? val(r_dyo[k]) : 0.0f;
        if (gate) {
          const float zz = val(r_zo[k]);
          v *= zz * sigmoid(zz);
        }
        s_dyo[buf][i][scol] = v;
      }
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = tid + k * NT;
      if (BCN % NT == 0 || e < BCN) {
        const int i = e / NS, n = e - (e / NS) * NS;
        const bool in = t0 + i < L && n < N;
        const float vb = in ? val(r_B[k]) : 0.0f, vc = in ? val(r_C[k]) : 0.0f;
        const int gg = n / SPL, jj = n % SPL;
#pragma unroll
        for (int s = 0; s < SPL; ++s) {
          s_bc[buf][i][gg][s][jj ^ s] = vb;
          s_bc[buf][i][gg][s][SPL + (jj ^ s)] = vc;
        }
      }
    }
  };

  // dB, dC totals of the block at t0x of this channel block, from LDS set sbx:
  // the 8 waves' sums added in order
  auto totals = [&](int t0x, int sbx) {
    for (int e = tid; e < 2 * kCK * NS; e += NT) {
      const int which = e / (kCK * NS);
      const int r = e - which * (kCK * NS);
      const int i = r / NS, n = r - (r / NS) * NS;
      if (n < N && t0x + i < L) {
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < kBwdWaves; ++w) s += which ? s_dC[sbx][w][i][n] : s_dB[sbx][w][i][n];
        float* dst = which ? p.ws_dC : p.ws_dB;
        dst[(((int64_t)cb * p.Bt + b) * L + t0x + i) * N + n] = s;
      }
    }
    if (BC && tid < kCK && t0x + tid < L) {
      float s = 0.0f;
#pragma unroll
      for (int w = 0; w < kBwdWaves; ++w) s += s_ddt[sbx][w][tid];
      p.ws_ddt[((int64_t)cb * p.Bt + b) * L + t0x + tid] = s;
    }
  };

  fetch(blk_hi - 1);
  commit(0, blk_hi - 1);
  __syncthreads();
  int buf = 0;
  float h[SPL];
  for (int blk = blk_hi - 1; blk >= blk_lo; --blk, buf ^= 1) {
    const int t0 = blk * kCK;
#pragma unroll
    for (int j = 0; j < SPL; ++j) h[j] = h_next[j];
    const bool more = blk > blk_lo;
    if (more) fetch(blk - 1);
    // a full block (every channel exists, no step beyond L) runs without
    // per-lane predicates
    const bool full = full_cb && t0 + kCK <= L;
    float dAblk[SPL];
#pragma unroll
    for (int j = 0; j < SPL; ++j) dAblk[j] = 0.0f;
    float dDblk = 0.0f;
    // the skip / softplus terms are a compile-time property of each instance
    // of the sweeps (branches in the unrolled step loop would split it into
    // many small scheduling regions); the gate is no longer in the sweeps: dz
    // is formed elementwise in the staging, from the forward's residual
    auto sweeps = [&](auto full_tag, auto sd_tag) {
      constexpr bool kFull = decltype(full_tag)::value;
      constexpr bool kSD = decltype(sd_tag)::value;  // skip || dsp
      float a_s[kCK][SPL], hp_s[kCK][SPL];
      // (u, delta, dy) and B of the block kept in registers from the
      // recompute for the adjoint where they fit (2 states per lane): the
      // adjoint then reads only C from LDS, which is the tighter resource
      // with 8 waves reading their operands every step
      constexpr bool kKeepX = SPL == 2;
      constexpr bool kKeepB = SPL == 2 && !EPI;
      float3 x_s[kKeepX ? kCK : 1];
      float b_s[kKeepB ? kCK : 1][SPL];
      constexpr int R = PF + 1;  // ring of operand sets, steps i .. i +- PF
      float4 xr[R];
      float bc[R][2 * SPL];
      auto pre = [&](int i, auto adj_tag) {
        constexpr bool kAdj = decltype(adj_tag)::value;
        if (!(kAdj && kKeepX)) xr[i % R] = s_x[buf][i][cw];
        if (kAdj && kKeepB) {
          float cv[SPL];
          lds_vec<SPL>(&s_bc[buf][i][g][sig][SPL], cv);
#pragma unroll
          for (int j = 0; j < SPL; ++j) bc[i % R][SPL + j] = cv[j];
        } else {
          lds_vec<2 * SPL>(&s_bc[buf][i][g][sig][0], bc[i % R]);
        }
      };
      // forward recompute of the block: a_t, h_{t-1}; dC_t = sum_d dy_t h_t
#pragma unroll
      for (int i = 0; i < PF; ++i) pre(i, std::false_type{});
      float vCp[SPL], vBp[SPL];  // (SSM_BWD_PIPE) the previous step's products
#pragma unroll
      for (int i = 0; i < kCK; ++i) {
        if (i + PF < kCK) pre(i + PF, std::false_type{});
        __builtin_amdgcn_sched_barrier(0);
        const float uu = xr[i % R].x, dd = xr[i % R].y, dyv = xr[i % R].z;
        if constexpr (kKeepX) x_s[i] = make_float3(uu, dd, dyv);
        if constexpr (kKeepB) {
#pragma unroll
          for (int j = 0; j < SPL; ++j) b_s[i][j] = bc[i % R][j];
        }
        const float w = dd * uu;
        float vC[SPL];
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
          const float a = fast_exp2(A2[j] * dd);
          a_s[i][j] = a;
          hp_s[i][j] = h[j];
          h[j] = fmaf(a, h[j], bc[i % R][j] * w);
          vC[j] = dyv * h[j];
        }
        if constexpr (SSM_BWD_PIPE) {
          if (i > 0) s_dC[sb][wave][i - 1][SPL * g + sig] = chan_reduce8<SPL>(vCp);
#pragma unroll
          for (int j = 0; j < SPL; ++j) vCp[j] = vC[j];
          if (i == kCK - 1) s_dC[sb][wave][i][SPL * g + sig] = chan_reduce8<SPL>(vCp);
        } else {
          s_dC[sb][wave][i][SPL * g + sig] = chan_reduce8<SPL>(vC);
        }
      }
      // The next block's operands go to LDS here, between the sweeps (that
      // buffer was last read before the previous block-end barrier).  One
      // counter (vmcnt) covers both loads and stores, and the wait for this
      // block's fetch loads is vmcnt(0): after the adjoint it also waited for
      // the adjoint's last du / ddelta stores, here none is in flight.
      if constexpr (kMidCommit) {
        if (more) commit(buf ^ 1, blk - 1);
      }
      // the previous block's dB / dC totals (its sums are in the other set,
      // complete since the last barrier; that set is written again only after
      // the next one)
      if constexpr (kLateTotals) {
        if (blk < blk_hi - 1) totals(t0 + kCK, sb ^ 1);
      }
      // adjoint, backwards through the block
      float v1p = 0.0f, v2p = 0.0f;
#pragma unroll
      for (int k = 0; k < PF; ++k) pre(kCK - 1 - k, std::true_type{});
#pragma unroll
      for (int i = kCK - 1; i >= 0; --i) {
        if (i - PF >= 0) pre(i - PF, std::true_type{});
        __builtin_amdgcn_sched_barrier(0);
        const float uu = kKeepX ? x_s[i].x : xr[i % R].x;
        const float dd = kKeepX ? x_s[i].y : xr[i % R].y;
        const float dyv = kKeepX ? x_s[i].z : xr[i % R].z;
        const float w = dd * uu;
        float s1 = 0.0f, s2 = 0.0f, vB[SPL];
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
          const float f = fmaf(bc[i % R][SPL + j], dyv, gc[j]);
          const float gg = a_s[i][j] * f;
          const float qv = gg * hp_s[i][j];
          s2 = j == 0 ? Av[0] * qv : fmaf(Av[j], qv, s2);
          dAblk[j] = fmaf(dd, qv, dAblk[j]);
          const float Bv = kKeepB ? b_s[i][j] : bc[i % R][j];
          s1 = j == 0 ? Bv * f : fmaf(Bv, f, s1);
          vB[j] = f * w;
          gc[j] = gg;
        }
        if constexpr (SSM_BWD_PIPE) {
          if (i < kCK - 1) s_dB[sb][wave][i + 1][SPL * g + sig] = chan_reduce8<SPL>(vBp);
#pragma unroll
          for (int j = 0; j < SPL; ++j) vBp[j] = vB[j];
          if (i == 0) s_dB[sb][wave][0][SPL * g + sig] = chan_reduce8<SPL>(vBp);
        } else {
          s_dB[sb][wave][i][SPL * g + sig] = chan_reduce8<SPL>(vB);
        }
        // du = delta sum_n f B; ddelta = sum_n f (A a h_{t-1} + B u)
        const float v1 = dd * s1, v2 = fmaf(uu, s1, s2);
        if (i & 1) {
          v1p = v1;
          v2p = v2;
        } else {
          // steps i+1, i summed over the state groups: rows 0, 1 hold du of
          // steps i+1, i and rows 2, 3 ddelta of steps i+1, i (both halves)
          float val = row_pair(half_pair(v1p, v2p), half_pair(v1, v2));
          val += dpp_mov<kDppRor8>(val);
          const int ti = i + ((orow & 1) ? 0 : 1);
          const int t = t0 + ti;
          if constexpr (kSD) {
            // du[t,d] += D[d] dy_out[t,d] and dD[d] += dy_out[t,d] u[t,d] on
            // du rows (Ddu is 0 without the skip); ddelta through softplus
            // (x.w is softplus'(delta), or 1)
            const float4 xo = s_x[buf][ti][cw];
            float dyo = xo.z;
            if constexpr (EPI) {
              if (stage_dyo) dyo = s_dyo[buf][ti][cw];
            }
            val = fmaf(Ddu, dyo, val);
            dDblk = fmaf(dmask * dyo, xo.x, dDblk);
            val *= is_du ? 1.0f : xo.w;
          }
          // du and ddelta rows of the wave store to different tensors: a
          // per-lane pointer (out_b)
          const uint32_t ro = (uint32_t)((t0 + i) * D);
          if constexpr (!BC) {
            if (kFull || (valid && t < L)) st32(out_b, ro + oo, val);
          } else {
            if (is_du && valid && t < L) st32(out_b, ro + oo, val);
            // one ddelta shared by the channels: sum the wave's 8 channels
            float sv = val + dpp_mov<kDppHalfMirror>(val);
            sv += dpp_mov<kDppXor2>(sv);
            sv += dpp_mov<kDppXor1>(sv);
            if (!is_du && lead && c == 0) s_ddt[sb][wave][ti] = sv;
          }
        }
      }
    };
    auto run_sweeps = [&](auto sd_tag) {
      if (full) sweeps(std::true_type{}, sd_tag); else sweeps(std::false_type{}, sd_tag);
    };
    if (skip || dsp) run_sweeps(std::true_type{}); else run_sweeps(std::false_type{});
#pragma unroll
    for (int j = 0; j < SPL; ++j) dAmid[j] += dAblk[j];
    dDmid += dDblk;
    if (((blk - blk_lo) & 15) == 0) {  // close a group of 16 blocks (and the row's last group)
#pragma unroll
      for (int j = 0; j < SPL; ++j) {
        dAacc[j] += dAmid[j];
        dAmid[j] = 0.0f;
      }
      dDacc += dDmid;
      dDmid = 0.0f;
    }
    if constexpr (kLateTotals) {
      __syncthreads();
      sb ^= 1;
    } else if constexpr (kSB == 2) {
      if constexpr (!kMidCommit) {
        if (more) commit(buf ^ 1, blk - 1);
      }
      __syncthreads();
      totals(t0, sb);
      sb ^= 1;
    } else {
      __syncthreads();
      totals(t0, sb);
      if constexpr (!kMidCommit) {
        if (more) commit(buf ^ 1, blk - 1);
      }
      __syncthreads();
    }
  }
  if constexpr (kLateTotals) totals(blk_lo * kCK, sb ^ 1);  // the last block's, after its barrier

#pragma unroll
  for (int j = 0; j < SPL; ++j)
    if (valid && nj[j] < N) p.ws_dA[(((int64_t)b * p.nseg + seg) * D + d) * N + nj[j]] = dAacc[j];
  if (skip) {
    // dD partial: the lanes of one channel accumulated disjoint steps
    __shared__ float s_red[kBwdWaves * kWave];
    s_red[tid] = dDacc;
    __syncthreads();
    if (tid < kBlkCh && cb * kBlkCh + tid < D) {
      const int w = tid >> 3, cc = tid & 7;
      float s = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) s += s_red[w * kWave + cc + 8 * k];
      p.ws_dD[((int64_t)b * p.nseg + seg) * D + cb * kBlkCh + tid] = s;
    }
  }
}

// Aggregate pass of a time-split backward.  Workgroup (cb, b, seg - 1), for
// segments seg >= 1, writes the carry the segment hands to the segment on its
// left with no carry from the right, G = a_t f_t at the segment's first step t
// (f_t = C_t dy_t + a_{t+1} f_{t+1}, ssmrecscan.py:96-100, 150-153), i.e.
// G = sum_t P_t C_t dy_t with P_t the product of the decays up to and including
// step t, and the whole segment's decay product P, through which a carry from
// the right enters G.  It walks the segment forwards a tile at a time (P: the
// product of the decays before the tile; G += P times the tile's own sum, then
// P *= the tile's decay), so once every P of the workgroup is 0 (flushed at
// tile ends, flush_tiny) all later steps add exact zeros and the walk stops
// there.  Pieces (asub > 1) as in the forward aggregate pass, mirrored: a
// piece whose products all end at 0 lets the piece after it stop, and the
// segments' first pieces are dispatched first.
template <int SPL, bool EPI, typename T>
__device__ __forceinline__ void bwd_agg_body(const BwdArgs<T>& p, const int b) {
  constexpr int NS = 8 * SPL;
  constexpr int NT = kWave * kBwdWaves;
  constexpr int RPT = kTT * kBlkCh / NT;
  constexpr int RSTEP = NT / kBlkCh;
  constexpr int BCN = kTT * NS;
  constexpr int BCE = (BCN + NT - 1) / NT;
  constexpr int PF = SSM_BWD_PF;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 7;
  const int g = lane >> 3;
  // b: the batch row (blockIdx.y of a single launch)
  const int cb = blockIdx.x;
  // blockIdx.z = part * (nseg - 1) + segment - 1, for segments 1 .. nseg - 1:
  // every segment's first piece first
  const int nsg = p.nseg - 1;
  const int part = blockIdx.z / nsg;
  const int seg = (1 + blockIdx.z - part * nsg) * p.asub + part;  // aggregate piece of the row
  const int L = p.L, D = p.D, N = p.N;
  const int alen = p.seg_len / p.asub;
  const int t_lo = seg * alen;
  const int t_hi = min(L, t_lo + alen);
  int* const fl = p.aflag ? p.aflag + ((int64_t)b * p.nseg * p.asub + seg) * gridDim.x + cb : nullptr;
  const int* const fprev = fl && part > 0 ? fl - gridDim.x : nullptr;  // the previous piece's flag
  const int cw = wave * 8 + c;
  const int d = cb * kBlkCh + cw;
  const bool valid = d < D;
  const int dc = valid ? d : 0;
  const bool rev = p.flags & SSM_REVERSE;
  const bool comp = (p.flags & SSM_COMPLEMENT) != 0;
  const bool gate = EPI && (p.flags & SSM_GATE);
  const bool dsp = p.flags & SSM_DELTA_SOFTPLUS;
  const int scol = tid & (kBlkCh - 1);
  const int srow0 = wave;  // = tid / kBlkCh: the staged rows of a wave are uniform
  const int sd = cb * kBlkCh + scol;
  const bool svalid = sd < D;
  const int sdc = svalid ? sd : 0;
  const int sq = comp ? D - 1 - sdc : sdc;

  float A2[SPL], G[SPL], P[SPL];
  bool live[SPL];
#pragma unroll
  for (int j = 0; j < SPL; ++j) {
    live[j] = valid && SPL * g + j < N;
    A2[j] = live[j] ? p.A[dc * N + SPL * g + j] * kLog2e : 0.0f;
    G[j] = 0.0f;
    P[j] = 1.0f;
  }

  __shared__ float2 s_dy[2][kTT][kBlkCh];  // (delta, dy of the scan)
  __shared__ __attribute__((aligned(16))) float s_C[2][kTT][NS];
  __shared__ int s_alive[2][kBwdWaves];

  const int dtD = p.dstride ? D : 1;
  const int scol_dt = p.dstride ? sdc : 0;
  const T* __restrict__ dt_b = p.delta + (int64_t)b * L * dtD;
  const int ldy = p.ldy, ldz = p.ldz;
  const T* __restrict__ dy_b = p.dy + (int64_t)b * L * ldy;
  const T* __restrict__ z_b = EPI ? p.z + (int64_t)b * L * ldz : nullptr;
  const int ldbc = p.ldbc;
  const T* __restrict__ C_b = p.Cc + (int64_t)b * L * ldbc;

  const buf_t rdt = make_buf(dt_b), rdy = make_buf(dy_b), rz = make_buf(EPI ? z_b : dy_b), rC = make_buf(C_b);
  const uint32_t so_dt = (uint32_t)(scol_dt * sizeof(T)), so_q = (uint32_t)(sq * sizeof(T));
  const uint32_t dtrowb = (uint32_t)(dtD * sizeof(T)), dyrowb = (uint32_t)(ldy * sizeof(T));
  const uint32_t zrowb = (uint32_t)(ldz * sizeof(T));
  stg<T> r_dt[RPT], r_dy[RPT], r_gz[RPT], r_C[BCE];
  auto fetch = [&](int t0) {
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int tc = min(t0 + srow0 + k * RSTEP, L - 1);  // wave-uniform
      const int pr = rev ? L - 1 - tc : tc;
      r_dt[k] = bldr<T>(rdt, so_dt, (uint32_t)tc * dtrowb);
      r_dy[k] = bldr<T>(rdy, so_q, (uint32_t)pr * dyrowb);
      if (gate) r_gz[k] = bldr<T>(rz, so_q, (uint32_t)pr * zrowb);
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = tid + k * NT;
      if (BCN % NT == 0 || e < BCN) {
        const int i = e / NS, n = e - (e / NS) * NS;
        r_C[k] = bldr<T>(rC, (uint32_t)((min(t0 + i, L - 1) * ldbc + min(n, N - 1)) * sizeof(T)), 0);
      }
    }
  };
  auto commit = [&](int buf, int t0) {
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int i = srow0 + k * RSTEP;
      const bool in = svalid && t0 + i < L;
      const float dtv = dsp ? softplus(val(r_dt[k])) : val(r_dt[k]);
      float go = in ? val(r_dy[k]) : 0.0f;
      if (gate) {
        const float gz = in ? val(r_gz[k]) : 0.0f;
        go *= gz * sigmoid(gz);  // as the main backward pass stages it
      }
      s_dy[buf][i][scol] = in ? make_float2(dtv, go) : make_float2(0.0f, 0.0f);
    }
#pragma unroll
    for (int k = 0; k < BCE; ++k) {
      const int e = tid + k * NT;
      if (BCN % NT == 0 || e < BCN) {
        const int i = e / NS, n = e - (e / NS) * NS;
        (&s_C[buf][0][0])[e] = (t0 + i < L && n < N) ? val(r_C[k]) : 0.0f;
      }
    }
  };

  fetch(t_lo);
  commit(0, t_lo);
  __syncthreads();
  int buf = 0, vote = 0;
  for (int t0 = t_lo;; t0 += kTT, buf ^= 1) {
    const bool more = t0 + kTT < t_hi;
    const bool pflush = fprev && __hip_atomic_load(fprev, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
    if (more) fetch(t0 + kTT);
    constexpr int R = PF + 1;
    float2 xd[R];
    float Cq[R][SPL];
    auto pre = [&](int i) {
      xd[i % R] = s_dy[buf][i][cw];
      lds_vec<SPL>(&s_C[buf][i][SPL * g], Cq[i % R]);
    };
#pragma unroll
    for (int i = 0; i < PF; ++i) pre(i);
    // the tile's terms relative to its start: Gt = sum_i e_i C_i dy_i with
    // e_i = exp2(A log2(e) s_i), s_i the sum of the tile's deltas up to and
    // including step i; then G += P Gt and P *= exp2(A log2(e) s) once per tile
    float Gt[SPL], s = 0.0f;
#pragma unroll
    for (int j = 0; j < SPL; ++j) Gt[j] = 0.0f;
#pragma unroll
    for (int i = 0; i < kTT; ++i) {
      if (i + PF < kTT) pre(i + PF);
      __builtin_amdgcn_sched_barrier(0);
      const float dd = xd[i % R].x, dyv = xd[i % R].y;
      s += dd;
#pragma unroll
      for (int j = 0; j < SPL; ++j) Gt[j] = fmaf(fast_exp2(A2[j] * s), Cq[i % R][j] * dyv, Gt[j]);
#pragma unroll
      for (int j = 0; j < SPL; ++j) pin(Gt[j]);
    }
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
      G[j] = fmaf(P[j], Gt[j], G[j]);
      P[j] *= fast_exp2(A2[j] * s);
    }
    if (more) commit(buf ^ 1, t0 + kTT);
    // as in the forward aggregate: flushed products end the walk
    flush_tiny(P);
    bool alive = false;
#pragma unroll
    for (int j = 0; j < SPL; ++j) alive = alive || (live[j] && P[j] != 0.0f);
    vote = barrier_or<kBwdWaves>((__ballot(alive) != 0 ? 1 : 0) | (pflush ? 2 : 0), s_alive[buf]);
    if (vote != 1 || !more) break;
  }
  const bool stop = (vote & 2) != 0;
  const int64_t o = (int64_t)b * p.nseg * p.asub + seg;
#pragma unroll
  for (int j = 0; j < SPL; ++j) {
    if (live[j]) {
      p.agg_G[(o * N + SPL * g + j) * D + d] = stop ? 0.0f : G[j];
      p.agg_P[(o * N + SPL * g + j) * D + d] = stop ? 0.0f : P[j];
    }
  }
  if (fl && (stop || (vote & 1) == 0) && tid == 0)
    __hip_atomic_store(fl, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// As ssm_fwd_agg_kernel: rows of p0 below rows0, rows of p1 above.
template <int SPL, bool EPI, typename T>
__global__ void __launch_bounds__(kWave* kBwdWaves, 1) ssm_bwd_agg_kernel(BwdArgs<T> p0, BwdArgs<T> p1,
                                                                         int rows0) {
  const int y = blockIdx.y;
  if (y < rows0) bwd_agg_body<SPL, EPI, T>(p0, y);
  else bwd_agg_body<SPL, EPI, T>(p1, y - rows0);
}

// One reduction of the backward's partial sums: out[i] = sum_k part[k*count + i],
// k = 0..nparts-1 in order, with element i of the dense sums stored at row
// i / w, column i % w of an output whose rows are ld elements apart (w = ld:
// dense).  v4: count and w multiples of 4 and part 16-byte aligned (float4
// loads).  bf16: the output elements are bf16 (else float).
struct RedJob {
  const float* part;
  void* out;
  int64_t count, w, ld;
  int nparts, v4, bf16;
};
constexpr int kMaxRedJobs = 5;  // dB, dC, dA, dD, broadcast ddelta
struct RedJobs {
  RedJob j0, j1, j2, j3, j4;
};
// field-wise selects (a dynamically indexed argument struct would be copied
// to scratch)
__device__ __forceinline__ RedJob pick_job(const RedJobs& J, int y) {
  RedJob r;
#define SSM_JOB(f) r.f = y == 0 ? J.j0.f : y == 1 ? J.j1.f : y == 2 ? J.j2.f : y == 3 ? J.j3.f : J.j4.f;
  SSM_JOB(part) SSM_JOB(out) SSM_JOB(count) SSM_JOB(w) SSM_JOB(ld) SSM_JOB(nparts) SSM_JOB(v4) SSM_JOB(bf16)
#undef SSM_JOB
  return r;
}

// Every reduction of one backward call in one launch: blockIdx.y selects the
// job.  Each thread sums 4 consecutive outputs, with kIn parts' loads in
// flight.
__global__ void reduce_parts_kernel(RedJobs jobs) {
  const RedJob jb = pick_job(jobs, blockIdx.y);
  const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i0 >= jb.count) return;
  const int64_t w = jb.w, ld = jb.ld, count = jb.count;
  const float* __restrict__ ws = jb.part;
  auto oidx = [&](int64_t i) { return w == ld ? i : (i / w) * ld + i % w; };
  auto put = [&](int64_t o, float v) {
    if (jb.bf16) st(static_cast<bf16*>(jb.out), o, v);
    else st(static_cast<float*>(jb.out), o, v);
  };
  constexpr int kIn = 8;
  if (jb.v4) {
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto add = [&](const float4 v) {
      s[0] += v.x;
      s[1] += v.y;
      s[2] += v.z;
      s[3] += v.w;
    };
    int k = 0;
    for (; k + kIn <= jb.nparts; k += kIn) {
      float4 v[kIn];
#pragma unroll
      for (int j = 0; j < kIn; ++j) v[j] = *reinterpret_cast<const float4*>(ws + (int64_t)(k + j) * count + i0);
#pragma unroll
      for (int j = 0; j < kIn; ++j) add(v[j]);
    }
    for (; k < jb.nparts; ++k) add(*reinterpret_cast<const float4*>(ws + (int64_t)k * count + i0));
    const int64_t o = oidx(i0);  // the 4 stay in one row (w % 4 == 0)
#pragma unroll
    for (int e = 0; e < 4; ++e) put(o + e, s[e]);
  } else {
    const int m = (int)(count - i0 < 4 ? count - i0 : 4);
    for (int e = 0; e < m; ++e) {
      float sum = 0.0f;
      for (int k = 0; k < jb.nparts; ++k) sum += ws[(int64_t)k * count + i0 + e];
      put(oidx(i0 + e), sum);
    }
  }
}

// ------------------------------------------------------------------- host side

struct Shape {
  int B, L, D, N, nblk, ncb;  // ncb: 64-channel blocks
  int spl_f, spl_b;           // states per lane of the forward and backward kernels
  bool epi;                   // skip / gate epilogue fused
  int seg_len, nseg;          // time segments per row
  int asub, nagg;             // aggregate walks per segment, and in a row (nseg * asub)
  int ldy, ldz;               // row strides of y / dy and of z
  int ldbc;                   // row stride of B, C, dB, dC
};

// Automatic time split: a row is split only when the unsplit backward grid
// would leave more than half of the resident-wave slots empty (256 CUs x 4
// SIMDs x 2 waves on MI355X), into enough segments to fill them, each at least
// kMinAutoSeg steps long.  The choice depends on the desc alone, so a given
// desc always computes in the same order.
constexpr int kFillWaves = 2048;
constexpr int kMaxGridY = 65535;  // grid.y limit: batch rows (or both calls' rows of a pair) per launch
constexpr int kMinAutoSeg = 512;
constexpr int kMaxSeg = 1024;
constexpr int kMinPiece = 16384;  // steps of an aggregate piece

void choose_segments(const ssm_desc_t* desc, Shape* s) {
  int64_t want = desc->segments;
  if (want == 0) {
    const int64_t waves = (int64_t)s->B * s->ncb * kBwdWaves;
    want = 2 * waves >= kFillWaves ? 1 : (kFillWaves + waves - 1) / waves;
    want = std::min<int64_t>(want, std::max(1, s->L / kMinAutoSeg));
  }
  int64_t len = (s->L + want - 1) / want;
  len = (len + kTT - 1) / kTT * kTT;  // segments start on forward tiles
  s->seg_len = (int)len;
  s->nseg = (int)((s->L + len - 1) / len);
  // The aggregate passes walk every segment but one, with 4 forward waves per
  // 64 channels: for long rows of few channels that is under one wave per
  // SIMD, and a walk that does not decay to 0 crosses the whole segment.  Each
  // segment's walk is then split in 2, 4 or 8 pieces of at least kMinPiece
  // steps; the main passes fold the pieces' carries in order, a few FMAs each.
  // A piece walks until its own decay product flushes (or a flag stops it), so
  // for walks a little longer than a piece the pieces only add reads: pieces
  // pay where walks can run far beyond kMinPiece steps.
  s->asub = 1;
  if (s->nseg > 1) {
    const int64_t awaves = (int64_t)s->B * s->ncb * (s->nseg - 1) * kFwdWaves;
    while (s->asub < 8 && awaves * s->asub < kFillWaves && s->seg_len % (2 * s->asub * kTT) == 0 &&
           s->seg_len / (2 * s->asub) >= kMinPiece)
      s->asub *= 2;
  }
  s->nagg = s->nseg * s->asub;
}

int validate(const ssm_desc_t* desc, Shape* s) {
  if (desc == nullptr) return fail(SSM_ERR_INVALID, "desc is NULL");
  if (desc->batch < 1 || desc->seqlen < 1 || desc->dim < 1)
    return fail(SSM_ERR_INVALID, "batch, seqlen and dim must be >= 1");
  if (desc->dstate < 1 || desc->dstate > 32) return fail(SSM_ERR_INVALID, "dstate must be in 1..32");
  if (desc->batch > kMaxGridY) return fail(SSM_ERR_INVALID, "batch must be <= 65535");
  // per-batch-row byte offsets are 32-bit inside the kernels; each extent is
  // bounded first so that the products below cannot overflow
  constexpr int64_t kMaxExtent = int64_t(1) << 30;
  if (desc->seqlen > kMaxExtent || desc->dim > kMaxExtent || desc->ld_y < 0 || desc->ld_y > kMaxExtent ||
      desc->ld_z < 0 || desc->ld_z > kMaxExtent || desc->ld_bc < 0 || desc->ld_bc > kMaxExtent)
    return fail(SSM_ERR_INVALID, "seqlen, dim, ld_y, ld_z and ld_bc must be <= 2^30 (ld_*: 0 or >= the row width)");
  if (desc->seqlen * desc->dim > (int64_t(1) << 30) || desc->seqlen * desc->dstate > (int64_t(1) << 30))
    return fail(SSM_ERR_INVALID, "seqlen*dim and seqlen*dstate must be <= 2^30");
  if ((desc->seqlen + kCK - 1) / kCK * desc->dstate * desc->dim > (int64_t(1) << 30))
    return fail(SSM_ERR_INVALID, "checkpoints of one batch row must hold <= 2^30 floats");
  if (desc->dtype != SSM_F32 && desc->dtype != SSM_BF16) return fail(SSM_ERR_INVALID, "dtype must be SSM_F32 or SSM_BF16");
  if (desc->flags & ~(SSM_REVERSE | SSM_COMPLEMENT | SSM_SKIP | SSM_GATE | SSM_DELTA_SOFTPLUS | SSM_SKIP_MAP |
                      SSM_SKIP_REVERSE | SSM_SKIP_COMPLEMENT | SSM_ACCUMULATE))
    return fail(SSM_ERR_INVALID, "unknown flag bits");
  if ((desc->flags & SSM_ACCUMULATE) && !(desc->flags & SSM_GATE))
    return fail(SSM_ERR_INVALID, "SSM_ACCUMULATE (dz += ...) needs SSM_GATE");
  if ((desc->flags & (SSM_SKIP_REVERSE | SSM_SKIP_COMPLEMENT)) && !(desc->flags & SSM_SKIP_MAP))
    return fail(SSM_ERR_INVALID, "SSM_SKIP_REVERSE / SSM_SKIP_COMPLEMENT need SSM_SKIP_MAP");
  if (desc->delta_broadcast != 0 && desc->delta_broadcast != 1)
    return fail(SSM_ERR_INVALID, "delta_broadcast must be 0 or 1");
  if (desc->segments < 0 || desc->segments > kMaxSeg) return fail(SSM_ERR_INVALID, "segments must be in 0..1024");
  if ((desc->ld_y != 0 && desc->ld_y < desc->dim) || (desc->ld_z != 0 && desc->ld_z < desc->dim))
    return fail(SSM_ERR_INVALID, "ld_y and ld_z must be 0 or >= dim");
  if ((desc->ld_y != 0 && desc->seqlen * desc->ld_y > (int64_t(1) << 30)) ||
      (desc->ld_z != 0 && desc->seqlen * desc->ld_z > (int64_t(1) << 30)))
    return fail(SSM_ERR_INVALID, "seqlen*ld_y and seqlen*ld_z must be <= 2^30");
  if (desc->ld_bc != 0 && (desc->ld_bc < desc->dstate || desc->seqlen * desc->ld_bc > (int64_t(1) << 30)))
    return fail(SSM_ERR_INVALID, "ld_bc must be 0 or >= dstate, with seqlen*ld_bc <= 2^30");
  // the backward's partial-sum reduction runs one thread per 4 sums of its
  // largest job (B*L*N for dB and dC, D*N for dA) in a 1-D grid
  if (std::max(desc->batch * desc->seqlen * desc->dstate, desc->dim * desc->dstate) > (int64_t(1) << 33))
    return fail(SSM_ERR_INVALID, "batch*seqlen*dstate and dim*dstate must be <= 2^33");
  s->B = (int)desc->batch;
  s->L = (int)desc->seqlen;
  s->D = (int)desc->dim;
  s->N = (int)desc->dstate;
  s->ncb = (s->D + kBlkCh - 1) / kBlkCh;
  s->ldy = desc->ld_y ? (int)desc->ld_y : s->D;
  s->ldz = desc->ld_z ? (int)desc->ld_z : s->D;
  s->ldbc = desc->ld_bc ? (int)desc->ld_bc : s->N;
  s->nblk = (s->L + kCK - 1) / kCK;
  // extra epilogue staging: the gate, and a skip whose u is not at the scan position
  // (by default the skip source is the output position: the reverse skip's quirk)
  const uint32_t f = desc->flags;
  const bool skip_moved = (f & SSM_SKIP_MAP) ? (f & (SSM_SKIP_REVERSE | SSM_SKIP_COMPLEMENT)) != 0
                                             : (f & (SSM_REVERSE | SSM_COMPLEMENT)) != 0;
  s->epi = (f & SSM_GATE) || ((f & SSM_SKIP) && skip_moved);
  s->spl_f = s->N <= 16 ? 4 : 8;  // 4 state rows per forward wave
  s->spl_b = s->N <= 16 ? 2 : 4;  // 8 state groups per backward wave
  choose_segments(desc, s);
  return SSM_OK;
}

// Calls f(spl, epi) with the compile-time variant matching s (spl = s.spl_f
// for the forward kernels, s.spl_b for the backward ones).
template <int S0, int S1, typename F>
bool dispatch_spl(int spl, bool epi, F&& f) {
  auto one = [&](auto sv, auto ev) {
    if (spl != decltype(sv)::value || epi != decltype(ev)::value) return false;
    f(sv, ev);
    return true;
  };
  return one(std::integral_constant<int, S0>{}, std::false_type{}) ||
         one(std::integral_constant<int, S1>{}, std::false_type{}) ||
         one(std::integral_constant<int, S0>{}, std::true_type{}) ||
         one(std::integral_constant<int, S1>{}, std::true_type{});
}

size_t ckpt_floats(const Shape& s) { return (size_t)s.B * s.nblk * s.N * s.D; }
// The forward's residuals are its checkpoints, then (with SSM_GATE) y before
// the gate: (B,L,D) of the I/O type in the output map, from which the backward
// forms dz elementwise instead of recomputing y = C h
size_t ypre_bytes(const ssm_desc_t* desc, const Shape& s) {
  if (!(desc->flags & SSM_GATE)) return 0;
  const size_t n = (size_t)s.B * s.L * s.D * (desc->dtype == SSM_F32 ? sizeof(float) : sizeof(uint16_t));
  return (n + 15) / 16 * 16;  // the buffer stays a whole number of floats (and 16-byte granules)
}

// Aggregates of a time-split scan, per piece (asub per segment):
// [B][nseg * asub][N][D] states (or adjoint carries) then [B][nseg * asub][N][D]
// decay products.  None for one segment.
size_t agg_floats(const Shape& s) { return s.nseg > 1 ? (size_t)2 * s.B * s.nagg * s.N * s.D : 0; }
// The pieces' end flags, [B][nseg * asub][ncb] ints after the aggregates (asub > 1)
size_t flag_ints(const Shape& s) { return s.asub > 1 ? (size_t)s.B * s.nagg * s.ncb : 0; }

struct WsLayout {
  size_t dB, dC, dA, dD, ddt, aggG, aggP, flg, total;  // float offsets
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
  w.aggP = w.aggG + (s.nseg > 1 ? (size_t)s.B * s.nagg * s.N * s.D : 0);
  w.flg = w.aggG + agg_floats(s);
  w.total = w.flg + flag_ints(s);
  return w;
}

template <typename T>
FwdArgs<T> fwd_args(const ssm_desc_t* desc, const Shape& s, const void* u, const void* delta, const float* A,
                    const void* Bc, const void* Cc, const float* Dskip, const void* z, void* y, float* ckpt,
                    void* workspace) {
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
  a.ypre = ckpt != nullptr && (desc->flags & SSM_GATE) ? reinterpret_cast<T*>(ckpt + ckpt_floats(s)) : nullptr;
  a.agg_H = static_cast<float*>(workspace);
  a.agg_P = a.agg_H + (s.nseg > 1 ? (size_t)s.B * s.nagg * s.N * s.D : 0);
  a.aflag = s.asub > 1 ? reinterpret_cast<int*>(a.agg_H + agg_floats(s)) : nullptr;
  a.L = s.L;
  a.D = s.D;
  a.N = s.N;
  a.nblk = s.nblk;
  a.seg_len = s.seg_len;
  a.nseg = s.nseg;
  a.asub = s.asub;
  a.ldy = s.ldy;
  a.ldz = s.ldz;
  a.ldbc = s.ldbc;
  a.dstride = desc->delta_broadcast ? 0 : 1;
  a.flags = desc->flags;
  return a;
}

// u and delta rows read as aligned 4-element vectors (the forward's VEC variant)
template <typename T>
bool fwd_vec(const ssm_desc_t* desc, const Shape& s, const FwdArgs<T>& a) {
  return s.D % 4 == 0 && !desc->delta_broadcast && reinterpret_cast<uintptr_t>(a.u) % (4 * sizeof(T)) == 0 &&
         reinterpret_cast<uintptr_t>(a.delta) % (4 * sizeof(T)) == 0;
}

// Zeroes n ints at f0 and, when it differs, at f1: the pieces' end flags of
// one or two calls, before their aggregate pass (a kernel, not a memset, so
// the sequence can be captured in a graph).
__global__ void clear_flags_kernel(int* f0, int* f1, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    f0[i] = 0;
    if (f1 != f0) f1[i] = 0;
  }
}

int launch_clear_flags(hipStream_t st, const Shape& s, int* f0, int* f1) {
  if (s.asub <= 1) return SSM_OK;
  const int64_t n = (int64_t)flag_ints(s);
  hipLaunchKernelGGL(clear_flags_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, f0, f1, n);
  return hip_check(hipGetLastError(), "aggregate flag clear launch");
}

// Aggregates of every segment but the last (s.nseg > 1): rows of a0, and with
// a pair (rows = 2 * s.B) the rows of a1 in the same launch.
template <typename T>
int launch_fwd_agg(hipStream_t st, const Shape& s, const FwdArgs<T>& a0, const FwdArgs<T>& a1, int rows) {
  if (int rc = launch_clear_flags(st, s, a0.aflag, a1.aflag)) return rc;
  if (!dispatch_spl<4, 8>(s.spl_f, false, [&](auto spl, auto) {
        constexpr int S = decltype(spl)::value;
        auto go = [&](auto sp) {
          constexpr bool SP = decltype(sp)::value;
          hipLaunchKernelGGL((ssm_fwd_agg_kernel<S, SP, T>), dim3(s.ncb, rows, (s.nseg - 1) * s.asub), dim3(kWave * kFwdWaves),
                             0, st, a0, a1, s.B);
        };
        if (a0.flags & SSM_DELTA_SOFTPLUS) go(std::true_type{}); else go(std::false_type{});
      }))
    return fail(SSM_ERR_UNSUPPORTED, "no kernel variant for this shape");
  return hip_check(hipGetLastError(), "ssm_fwd aggregate launch");
}

// The main forward pass over rows of a0, and with a pair (rows = 2 * s.B) the
// rows of a1 in the same launch (same shape and kernel variant).
template <typename T>
int launch_fwd_main(hipStream_t st, const Shape& s, const FwdArgs<T>& a0, const FwdArgs<T>& a1, int rows,
                    bool vec) {
  if (!dispatch_spl<4, 8>(s.spl_f, s.epi, [&](auto spl, auto epi) {
        constexpr int S = decltype(spl)::value;
        constexpr bool E = decltype(epi)::value;
        auto go = [&](auto sp) {
          constexpr bool SP = decltype(sp)::value;
          if (vec)
            hipLaunchKernelGGL((ssm_fwd_kernel<S, E, SP, true, T>), dim3(s.ncb, rows, s.nseg),
                               dim3(kWave * kFwdWaves), 0, st, a0, a1, s.B);
          else
            hipLaunchKernelGGL((ssm_fwd_kernel<S, E, SP, false, T>), dim3(s.ncb, rows, s.nseg),
                               dim3(kWave * kFwdWaves), 0, st, a0, a1, s.B);
        };
        if (a0.flags & SSM_DELTA_SOFTPLUS) go(std::true_type{}); else go(std::false_type{});
      }))
    return fail(SSM_ERR_UNSUPPORTED, "no kernel variant for this shape");
  return hip_check(hipGetLastError(), "ssm_fwd launch");
}

template <typename T>
int launch_fwd(hipStream_t st, const ssm_desc_t* desc, const Shape& s, const FwdArgs<T>& a) {
  if (s.nseg > 1)
    if (int rc = launch_fwd_agg<T>(st, s, a, a, s.B)) return rc;
  return launch_fwd_main<T>(st, s, a, a, s.B, fwd_vec<T>(desc, s, a));
}

template <typename T>
BwdArgs<T> bwd_args(const ssm_desc_t* desc, const Shape& s, const void* u, const void* delta, const float* A,
                    const void* Bc, const void* Cc, const float* Dskip, const void* z, const float* ckpt,
                    const void* dy, void* du, void* ddelta, void* dz, void* workspace) {
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
  a.ypre = (desc->flags & SSM_GATE) ? reinterpret_cast<const T*>(ckpt + ckpt_floats(s)) : nullptr;
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
  a.aflag = s.asub > 1 ? reinterpret_cast<int*>(ws + wl.flg) : nullptr;
  a.Bt = s.B;
  a.L = s.L;
  a.D = s.D;
  a.N = s.N;
  a.nblk = s.nblk;
  a.ncb = s.ncb;
  a.seg_len = s.seg_len;
  a.nseg = s.nseg;
  a.asub = s.asub;
  a.ldy = s.ldy;
  a.ldz = s.ldz;
  a.ldbc = s.ldbc;
  a.dstride = bcast ? 0 : 1;
  a.flags = desc->flags;
  return a;
}

// Adjoint aggregates of every segment but the first (s.nseg > 1): rows of a0,
// and with a pair (rows = 2 * s.B) the rows of a1 in the same launch.
template <typename T>
int launch_bwd_agg(hipStream_t st, const Shape& s, const BwdArgs<T>& a0, const BwdArgs<T>& a1, int rows) {
  if (int rc = launch_clear_flags(st, s, a0.aflag, a1.aflag)) return rc;
  if (!dispatch_spl<2, 4>(s.spl_b, s.epi, [&](auto spl, auto epi) {
        constexpr int S = decltype(spl)::value;
        constexpr bool E = decltype(epi)::value;
        hipLaunchKernelGGL((ssm_bwd_agg_kernel<S, E, T>), dim3(s.ncb, rows, (s.nseg - 1) * s.asub), dim3(kWave * kBwdWaves), 0,
                           st, a0, a1, s.B);
      }))
    return fail(SSM_ERR_UNSUPPORTED, "no kernel variant for this shape");
  return hip_check(hipGetLastError(), "ssm_bwd aggregate launch");
}

// The main backward pass over rows of a0, and with a pair (rows = 2 * s.B) the
// rows of a1 in the same launch (same shape and kernel variant).
template <typename T>
int launch_bwd_main(hipStream_t st, const ssm_desc_t* desc, const Shape& s, const BwdArgs<T>& a0,
                    const BwdArgs<T>& a1, int rows) {
  if (!dispatch_spl<2, 4>(s.spl_b, s.epi, [&](auto spl, auto epi) {
        constexpr int S = decltype(spl)::value;
        constexpr bool E = decltype(epi)::value;
        auto go = [&](auto bc, auto acc) {
          constexpr bool kBC = decltype(bc)::value, kAcc = E && decltype(acc)::value;
          hipLaunchKernelGGL((ssm_bwd_kernel<S, E, kBC, kAcc, T>), dim3(s.ncb, rows, s.nseg),
                             dim3(kWave * kBwdWaves), 0, st, a0, a1, s.B);
        };
        const bool acc = (desc->flags & SSM_ACCUMULATE) != 0;  // validated: only with the gate (EPI)
        if (desc->delta_broadcast) {
          if (acc) go(std::true_type{}, std::true_type{}); else go(std::true_type{}, std::false_type{});
        } else {
          if (acc) go(std::false_type{}, std::true_type{}); else go(std::false_type{}, std::false_type{});
        }
      }))
    return fail(SSM_ERR_UNSUPPORTED, "no kernel variant for this shape");
  return hip_check(hipGetLastError(), "ssm_bwd launch");
}

// The fixed-order reductions of a backward's partial sums into dB, dC, dA, dD
// (and a broadcast delta's gradient).
template <typename T>
int launch_bwd_reduce(hipStream_t st, const ssm_desc_t* desc, const Shape& s, float* dA, void* dB, void* dC,
                      float* dD, void* ddelta, void* workspace) {
  const bool bcast = desc->delta_broadcast != 0;
  const WsLayout wl = ws_layout(s, bcast);
  float* ws = static_cast<float*>(workspace);
  RedJob job[kMaxRedJobs] = {};
  int njobs = 0;
  int64_t maxcount = 0;
  auto reduce = [&](const float* part, void* out, bool out_bf16, int nparts, int64_t count, int64_t w, int64_t ld) {
    const bool v4 = count % 4 == 0 && w % 4 == 0 && reinterpret_cast<uintptr_t>(part) % 16 == 0;
    job[njobs++] = RedJob{part, out, count, w, ld, nparts, v4 ? 1 : 0, out_bf16 ? 1 : 0};
    maxcount = std::max(maxcount, count);
  };
  constexpr bool kBf16 = std::is_same_v<T, bf16>;
  const int64_t bln = (int64_t)s.B * s.L * s.N;
  const int64_t dn = (int64_t)s.D * s.N;
  const int64_t bl = (int64_t)s.B * s.L;
  reduce(ws + wl.dB, dB, kBf16, s.ncb, bln, s.N, s.ldbc);
  reduce(ws + wl.dC, dC, kBf16, s.ncb, bln, s.N, s.ldbc);
  reduce(ws + wl.dA, dA, false, s.B * s.nseg, dn, dn, dn);
  if (desc->flags & SSM_SKIP) reduce(ws + wl.dD, dD, false, s.B * s.nseg, (int64_t)s.D, s.D, s.D);
  if (bcast) reduce(ws + wl.ddt, ddelta, kBf16, s.ncb, bl, bl, bl);
  const RedJobs jobs{job[0], job[1], job[2], job[3], job[4]};
  const int threads = 256;
  const int64_t blocks = ((maxcount + 3) / 4 + threads - 1) / threads;
  hipLaunchKernelGGL(reduce_parts_kernel, dim3((unsigned)blocks, (unsigned)njobs), dim3(threads), 0, st, jobs);
  return hip_check(hipGetLastError(), "ssm_bwd reduce launch");
}

template <typename T>
int launch_bwd(hipStream_t st, const ssm_desc_t* desc, const Shape& s, const BwdArgs<T>& a, float* dA, void* dB,
               void* dC, float* dD, void* ddelta, void* workspace) {
  if (s.nseg > 1)
    if (int rc = launch_bwd_agg<T>(st, s, a, a, s.B)) return rc;
  if (int rc = launch_bwd_main<T>(st, desc, s, a, a, s.B)) return rc;
  return launch_bwd_reduce<T>(st, desc, s, dA, dB, dC, dD, ddelta, workspace);
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

// ------------------------------------------- static scratch (ssm_bwd_static)
//
// The workspace of ssm_bwd_static: a file-scope device array of fixed size.
// Every GPU the library runs on holds its own copy until the process ends.  In
// host code `scratch` only names the symbol; its device address on the
// current device comes from hipGetSymbolAddress, looked up once per device and
// kept.  Calls on one GPU share the array (overlapping calls race); no kernel
// needs it cleared, since every partial the reductions read is written first
// by the same call.
static __device__ __align__(256) float scratch[SSM_STATIC_SCRATCH_BYTES / sizeof(float)];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The address of `scratch` on the current device (looked up on the first call there).
int scratch_on_current_device(void** out) {
  int dev = -1;
  if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (dev < 0 || dev >= kMaxDevices) return fail(SSM_ERR_UNSUPPORTED, "device ordinal beyond 63");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    if (int rc = hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)")) return rc;
    if (ptr == nullptr) return fail(SSM_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return SSM_OK;
}

}  // namespace

extern "C" {

int ssm_abi_version(void) { return SSM_ABI_VERSION; }

const char* ssm_last_error(void) { return g_last_error.c_str(); }

size_t ssm_ckpt_bytes(const ssm_desc_t* desc) {
  g_last_error.clear();
  Shape s;
  if (validate(desc, &s)) return 0;
  return ckpt_floats(s) * sizeof(float) + ypre_bytes(desc, s);
}

size_t ssm_fwd_workspace_bytes(const ssm_desc_t* desc) {
  g_last_error.clear();
  Shape s;
  if (validate(desc, &s)) return 0;
  return agg_floats(s) * sizeof(float) + flag_ints(s) * sizeof(int);
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
  const ApiRange range("ssm_fwd");
  g_last_error.clear();
  Shape s;
  if (int rc = validate(desc, &s)) return rc;
  if (!u || !delta || !A || !Bc || !Cc || !y) return fail(SSM_ERR_INVALID, "ssm_fwd: required pointer is NULL");
  if (s.nseg > 1 && !workspace) return fail(SSM_ERR_INVALID, "ssm_fwd: workspace is NULL but ssm_fwd_workspace_bytes > 0");
  if ((desc->flags & SSM_SKIP) && !Dskip) return fail(SSM_ERR_INVALID, "SSM_SKIP needs Dskip");
  if ((desc->flags & SSM_GATE) && !z) return fail(SSM_ERR_INVALID, "SSM_GATE needs z");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (desc->dtype == SSM_F32)
    return launch_fwd<float>(st, desc, s, fwd_args<float>(desc, s, u, delta, A, Bc, Cc, Dskip, z, y, ckpt, workspace));
  return launch_fwd<bf16>(st, desc, s, fwd_args<bf16>(desc, s, u, delta, A, Bc, Cc, Dskip, z, y, ckpt, workspace));
}

int ssm_bwd(void* stream, const ssm_desc_t* desc, const void* u, const void* delta, const float* A,
            const void* Bc, const void* Cc, const float* Dskip, const void* z, const float* ckpt, const void* dy,
            void* du, void* ddelta, float* dA, void* dB, void* dC, float* dD, void* dz, void* workspace) {
  const ApiRange range("ssm_bwd");
  g_last_error.clear();
  Shape s;
  if (int rc = validate(desc, &s)) return rc;
  if (!u || !delta || !A || !Bc || !Cc || !ckpt || !dy || !du || !ddelta || !dA || !dB || !dC || !workspace)
    return fail(SSM_ERR_INVALID, "ssm_bwd: required pointer is NULL");
  if ((desc->flags & SSM_SKIP) && (!Dskip || !dD)) return fail(SSM_ERR_INVALID, "SSM_SKIP needs Dskip and dD");
  if ((desc->flags & SSM_GATE) && (!z || !dz)) return fail(SSM_ERR_INVALID, "SSM_GATE needs z and dz");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (desc->dtype == SSM_F32)
    return launch_bwd<float>(st, desc, s,
                             bwd_args<float>(desc, s, u, delta, A, Bc, Cc, Dskip, z, ckpt, dy, du, ddelta, dz, workspace),
                             dA, dB, dC, dD, ddelta, workspace);
  return launch_bwd<bf16>(st, desc, s,
                          bwd_args<bf16>(desc, s, u, delta, A, Bc, Cc, Dskip, z, ckpt, dy, du, ddelta, dz, workspace),
                          dA, dB, dC, dD, ddelta, workspace);
}

int ssm_bwd_static(void* stream, const ssm_desc_t* desc, const void* u, const void* delta, const float* A,
                   const void* Bc, const void* Cc, const float* Dskip, const void* z, const float* ckpt,
                   const void* dy, void* du, void* ddelta, float* dA, void* dB, void* dC, float* dD, void* dz) {
  const ApiRange range("ssm_bwd_static");
  g_last_error.clear();
  Shape s;
  if (int rc = validate(desc, &s)) return rc;
  const size_t need = ws_layout(s, desc->delta_broadcast != 0).total * sizeof(float);
  if (need > SSM_STATIC_SCRATCH_BYTES)
    return fail(SSM_ERR_INVALID, "ssm_bwd_static: this desc needs " + std::to_string(need) +
                                     " bytes of workspace, more than the static scratch's " +
                                     std::to_string((size_t)SSM_STATIC_SCRATCH_BYTES) + " (use ssm_bwd)");
  // the stream must belong to the current device, whose copy of the scratch is used
  if (stream != nullptr) {
    int sdev = -1, dev = -1;
    if (int rc = hip_check(hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev), "hipStreamGetDevice"))
      return rc;
    if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
    if (sdev != dev) return fail(SSM_ERR_INVALID, "ssm_bwd_static: the stream belongs to another device than the current one");
  }
  void* ws = nullptr;
  if (int rc = scratch_on_current_device(&ws)) return rc;
  return ssm_bwd(stream, desc, u, delta, A, Bc, Cc, Dskip, z, ckpt, dy, du, ddelta, dA, dB, dC, dD, dz, ws);
}

// The two calls of a pair as ssm_fwd / ssm_bwd would make them.  When the two
// descs have the same shape, their time-split aggregate passes share one
// launch, and so do their main passes when they also need the same kernel
// variant (epilogue staging, vector staging).  Each call keeps its own time
// segments, so the results equal two separate calls bit for bit.
static bool same_shape(const ssm_desc_t& a, const ssm_desc_t& b) {
  return a.batch == b.batch && a.seqlen == b.seqlen && a.dim == b.dim && a.dstate == b.dstate &&
         a.dtype == b.dtype && a.delta_broadcast == b.delta_broadcast && a.segments == b.segments &&
         ((a.flags ^ b.flags) & SSM_DELTA_SOFTPLUS) == 0;
}

int ssm_fwd_pair(void* stream, const ssm_desc_t* desc, const ssm_fwd_io_t* io) {
  const ApiRange range("ssm_fwd_pair");
  g_last_error.clear();
  if (desc == nullptr || io == nullptr) return fail(SSM_ERR_INVALID, "ssm_fwd_pair: desc or io is NULL");
  Shape s[2];
  for (int k = 0; k < 2; ++k) {
    if (int rc = validate(&desc[k], &s[k])) return rc;
    const ssm_fwd_io_t& q = io[k];
    if (!q.u || !q.delta || !q.A || !q.B || !q.C || !q.y)
      return fail(SSM_ERR_INVALID, "ssm_fwd_pair: required pointer is NULL");
    if (s[k].nseg > 1 && !q.workspace)
      return fail(SSM_ERR_INVALID, "ssm_fwd_pair: workspace is NULL but ssm_fwd_workspace_bytes > 0");
    if ((desc[k].flags & SSM_SKIP) && !q.D) return fail(SSM_ERR_INVALID, "SSM_SKIP needs D");
    if ((desc[k].flags & SSM_GATE) && !q.z) return fail(SSM_ERR_INVALID, "SSM_GATE needs z");
  }
  // one element type for both calls: the kernels of a pair are chosen once
  if (desc[0].dtype != desc[1].dtype) return fail(SSM_ERR_INVALID, "ssm_fwd_pair: the two descs must have the same dtype");
  const bool same = same_shape(desc[0], desc[1]) && 2 * s[0].B <= kMaxGridY;
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto run = [&](auto tag) -> int {
    using T = decltype(tag);
    FwdArgs<T> a[2];
    bool vec[2];
    for (int k = 0; k < 2; ++k) {
      a[k] = fwd_args<T>(&desc[k], s[k], io[k].u, io[k].delta, io[k].A, io[k].B, io[k].C, io[k].D, io[k].z,
                         io[k].y, io[k].ckpt, io[k].workspace);
      vec[k] = fwd_vec<T>(&desc[k], s[k], a[k]);
    }
    if (same && s[0].nseg > 1) {
      if (int rc = launch_fwd_agg<T>(st, s[0], a[0], a[1], 2 * s[0].B)) return rc;
    } else {
      for (int k = 0; k < 2; ++k)
        if (s[k].nseg > 1)
          if (int rc = launch_fwd_agg<T>(st, s[k], a[k], a[k], s[k].B)) return rc;
    }
    if (same && s[0].epi == s[1].epi && vec[0] == vec[1])
      return launch_fwd_main<T>(st, s[0], a[0], a[1], 2 * s[0].B, vec[0]);
    for (int k = 0; k < 2; ++k)
      if (int rc = launch_fwd_main<T>(st, s[k], a[k], a[k], s[k].B, vec[k])) return rc;
    return SSM_OK;
  };
  return desc[0].dtype == SSM_F32 ? run(float{}) : run(bf16{});
}

int ssm_bwd_pair(void* stream, const ssm_desc_t* desc, const ssm_bwd_io_t* io) {
  const ApiRange range("ssm_bwd_pair");
  g_last_error.clear();
  if (desc == nullptr || io == nullptr) return fail(SSM_ERR_INVALID, "ssm_bwd_pair: desc or io is NULL");
  Shape s[2];
  for (int k = 0; k < 2; ++k) {
    if (int rc = validate(&desc[k], &s[k])) return rc;
    const ssm_bwd_io_t& q = io[k];
    if (!q.u || !q.delta || !q.A || !q.B || !q.C || !q.ckpt || !q.dy || !q.du || !q.ddelta || !q.dA || !q.dB ||
        !q.dC || !q.workspace)
      return fail(SSM_ERR_INVALID, "ssm_bwd_pair: required pointer is NULL");
    if ((desc[k].flags & SSM_SKIP) && (!q.D || !q.dD)) return fail(SSM_ERR_INVALID, "SSM_SKIP needs D and dD");
    if ((desc[k].flags & SSM_GATE) && (!q.z || !q.dz)) return fail(SSM_ERR_INVALID, "SSM_GATE needs z and dz");
  }
  if (desc[0].dtype != desc[1].dtype) return fail(SSM_ERR_INVALID, "ssm_bwd_pair: the two descs must have the same dtype");
  // the backward kernels' variant: the epilogue staging (and delta broadcast, part of the shape)
  const bool same = same_shape(desc[0], desc[1]) && s[0].epi == s[1].epi && 2 * s[0].B <= kMaxGridY;
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto run = [&](auto tag) -> int {
    using T = decltype(tag);
    BwdArgs<T> a[2];
    for (int k = 0; k < 2; ++k)
      a[k] = bwd_args<T>(&desc[k], s[k], io[k].u, io[k].delta, io[k].A, io[k].B, io[k].C, io[k].D, io[k].z,
                         io[k].ckpt, io[k].dy, io[k].du, io[k].ddelta, io[k].dz, io[k].workspace);
    if (same) {
      if (s[0].nseg > 1)
        if (int rc = launch_bwd_agg<T>(st, s[0], a[0], a[1], 2 * s[0].B)) return rc;
      // a call accumulating into dz may share it with the other: run them in order
      if (SSM_PAIR_JOINT_BWD_MAIN && !((desc[0].flags | desc[1].flags) & SSM_ACCUMULATE)) {
        if (int rc = launch_bwd_main<T>(st, &desc[0], s[0], a[0], a[1], 2 * s[0].B)) return rc;
      } else {
        for (int k = 0; k < 2; ++k)
          if (int rc = launch_bwd_main<T>(st, &desc[k], s[k], a[k], a[k], s[k].B)) return rc;
      }
    } else {
      for (int k = 0; k < 2; ++k) {
        if (s[k].nseg > 1)
          if (int rc = launch_bwd_agg<T>(st, s[k], a[k], a[k], s[k].B)) return rc;
        if (int rc = launch_bwd_main<T>(st, &desc[k], s[k], a[k], a[k], s[k].B)) return rc;
      }
    }
    for (int k = 0; k < 2; ++k)
      if (int rc = launch_bwd_reduce<T>(st, &desc[k], s[k], io[k].dA, io[k].dB, io[k].dC, io[k].dD, io[k].ddelta,
                                        io[k].workspace))
        return rc;
    return SSM_OK;
  };
  return desc[0].dtype == SSM_F32 ? run(float{}) : run(bf16{});
}

}  // extern "C"
