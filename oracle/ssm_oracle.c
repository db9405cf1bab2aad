/*
 * ssm_oracle.c — CPU restatement of the reference's custom-VJP selective scan.
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/ (checked against oracle/ssm_oracle.py)
 * and as bench.py's cpu_baseline ("port").  The product never links it.
 *
 * It follows the reference's algorithm structure, per (batch, channel) row
 * (paths relative to the reference's src/selectssm/):
 *   forward   ssm_recursive_scan (ssmrecscan.py:36-77): split the time range
 *             while len > min_recursion_length and len % recursive_split == 0
 *             (56), scan the pieces in order threading (g, h) (63); leaves
 *             run the odd/even associative scan of jax.lax.associative_scan
 *             on (alpha, beta) pairs (67-68), hs = gs*h_init + hs (69),
 *             y = C.hs (72).
 *   backward  ssm_scan_backward_recursive (ssmrecscan.py:111-161): in the
 *             recursive case a reverse pass over the pieces computes the
 *             adjoint entering each piece from its right, recomputing alpha
 *             per step (121-133); then a forward pass recurses into every piece
 *             with (h_left, f_alpha_right), summing dA (134-143).  Leaves
 *             (149-161): forward scan keeping h_{t-1}, reverse scan keeping
 *             f_t, then the closed forms of 154-160.
 * Rows are independent except for the sums over channels (dB, dC) and over
 * (batch, time) (dA); those are accumulated per thread and summed at the end.
 * OpenMP parallelises over rows.  All arithmetic is float32 like the
 * reference; the associative-scan leaf keeps the reference's combine order.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define MAXN 64

typedef struct {
  int L, N, min_len, split;
  const float *u, *dt, *Bc, *Cc, *dy; /* row views: u[t*ustride] etc. */
  int64_t ustride, bstride;           /* D for (B,L,D) rows, N for (B,L,N) rows */
  const float* A;                     /* A[d, 0..N) */
  float* y;                           /* forward output row */
  float *du, *ddt;                    /* backward output rows */
  float *dB, *dC;                     /* (L,N) thread-private accumulators */
  float* dA;                          /* (N) thread-private accumulator */
  float* scratch;                     /* leaf workspace */
} Row;

/* inclusive scan of (g,h) pairs with the odd/even recursion of
 * jax.lax.associative_scan; combine(l, r) = (g_l g_r, g_r h_l + h_r). */
static void assoc_scan(float* g, float* h, int n, float* tmp) {
  if (n < 2) return;
  int m = n / 2; /* number of pairs */
  float* rg = tmp;
  float* rh = tmp + m;
  for (int i = 0; i < m; ++i) {
    float gl = g[2 * i], hl = h[2 * i], gr = g[2 * i + 1], hr = h[2 * i + 1];
    rg[i] = gl * gr;
    rh[i] = gr * hl + hr;
  }
  assoc_scan(rg, rh, m, tmp + 2 * m);
  /* odd positions 1,3,.. take the reduced prefixes; even positions 2,4,.. combine
   * the previous odd prefix with the original element */
  for (int i = 1; 2 * i < n; ++i) {
    float gl = rg[i - 1], hl = rh[i - 1], gr = g[2 * i], hr = h[2 * i];
    g[2 * i] = gl * gr;
    h[2 * i] = gr * hl + hr;
  }
  for (int i = 0; i < m; ++i) {
    g[2 * i + 1] = rg[i];
    h[2 * i + 1] = rh[i];
  }
}

/* ---------------------------------------------------------------- forward */

static void fwd_rec(Row* r, int t0, int len, float* g, float* h) {
  if (len > r->min_len && len % r->split == 0) {
    int m = len / r->split;
    for (int i = 0; i < r->split; ++i) fwd_rec(r, t0 + i * m, m, g, h);
    return;
  }
  const int N = r->N;
  for (int n = 0; n < N; ++n) {
    float* ga = r->scratch;
    float* ha = ga + len;
    float* tmp = ha + len;
    for (int i = 0; i < len; ++i) {
      const int t = t0 + i;
      const float d = r->dt[t * r->ustride];
      ga[i] = expf(r->A[n] * d);
      ha[i] = r->Bc[t * r->bstride + n] * r->u[t * r->ustride] * d;
    }
    assoc_scan(ga, ha, len, tmp);
    for (int i = 0; i < len; ++i) {
      const int t = t0 + i;
      const float hs = ga[i] * h[n] + ha[i];
      r->y[t * r->ustride] += r->Cc[t * r->bstride + n] * hs;
      if (i == len - 1) {
        g[n] = ga[i] * g[n];
        h[n] = hs;
      }
    }
  }
}

/* --------------------------------------------------------------- backward */

static void bwd_rec(Row* r, int t0, int len, float* h_left, const float* fa_right) {
  const int N = r->N;
  if (len > r->min_len && len % r->split == 0) {
    const int m = len / r->split;
    float* fas = (float*)malloc(sizeof(float) * r->split * N);
    float fa[MAXN];
    memcpy(fa, fa_right, sizeof(float) * N);
    for (int i = r->split - 1; i >= 0; --i) {
      memcpy(fas + i * N, fa, sizeof(float) * N);
      for (int t = t0 + i * m + m - 1; t >= t0 + i * m; --t) {
        const float d = r->dt[t * r->ustride];
        const float dyv = r->dy[t * r->ustride];
        for (int n = 0; n < N; ++n) {
          const float alpha = expf(r->A[n] * d);
          const float f = fa[n] + r->Cc[t * r->bstride + n] * dyv;
          fa[n] = f * alpha;
        }
      }
    }
    for (int i = 0; i < r->split; ++i) bwd_rec(r, t0 + i * m, m, h_left, fas + i * N);
    free(fas);
    return;
  }
  float* hs = r->scratch;   /* len*N: h_{t-1} */
  float* al = hs + len * N; /* len*N: alpha_t */
  float* fs = al + len * N; /* len*N: f_t */
  for (int i = 0; i < len; ++i) {
    const int t = t0 + i;
    const float d = r->dt[t * r->ustride], uu = r->u[t * r->ustride];
    for (int n = 0; n < N; ++n) {
      const float a = expf(r->A[n] * d);
      al[i * N + n] = a;
      hs[i * N + n] = h_left[n];
      h_left[n] = h_left[n] * a + r->Bc[t * r->bstride + n] * uu * d;
    }
  }
  float fa[MAXN];
  memcpy(fa, fa_right, sizeof(float) * N);
  for (int i = len - 1; i >= 0; --i) {
    const int t = t0 + i;
    const float dyv = r->dy[t * r->ustride];
    for (int n = 0; n < N; ++n) {
      const float f = fa[n] + r->Cc[t * r->bstride + n] * dyv;
      fs[i * N + n] = f;
      fa[n] = f * al[i * N + n];
    }
  }
  for (int i = 0; i < len; ++i) {
    const int t = t0 + i;
    const float d = r->dt[t * r->ustride], uu = r->u[t * r->ustride], dyv = r->dy[t * r->ustride];
    float dx = 0.0f, ddt = 0.0f;
    for (int n = 0; n < N; ++n) {
      const float f = fs[i * N + n];
      const float Bn = r->Bc[t * r->bstride + n];
      const float ah = al[i * N + n] * hs[i * N + n];
      const float df = d * f;
      const float hnext = (i + 1 < len) ? hs[(i + 1) * N + n] : h_left[n];
      dx += df * Bn;
      r->dA[n] += df * ah;
      r->dB[t * N + n] += df * uu;
      r->dC[t * N + n] += dyv * hnext;
      ddt += f * (r->A[n] * ah + Bn * uu);
    }
    r->du[t * r->ustride] = dx;
    r->ddt[t * r->ustride] = ddt;
  }
}

static size_t leaf_scratch_floats(int L, int N, int min_len, int split) {
  /* the largest leaf: shrink L while it splits */
  int len = L;
  while (len > min_len && split > 1 && len % split == 0) len /= split;
  size_t f = (size_t)3 * len + 2 * (size_t)len; /* forward leaf + scan temporaries */
  size_t b = (size_t)3 * len * N;
  return (f > b ? f : b) + 64;
}

/*
 * Forward: y (B,L,D) from u, dt (B,L,D), A (D,N), Bc, Cc (B,L,N).
 * Returns 0, or -1 when N > 64 or recursive_split < 2.
 */
int oracle_scan_fwd(int B, int L, int D, int N, const float* u, const float* dt, const float* A, const float* Bc,
                    const float* Cc, float* y, int min_len, int split, int nthreads) {
  if (N > MAXN || split < 2) return -1;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
  const size_t sf = leaf_scratch_floats(L, N, min_len, split);
  memset(y, 0, sizeof(float) * (size_t)B * L * D);
#pragma omp parallel
  {
    float* scratch = (float*)malloc(sizeof(float) * sf);
#pragma omp for schedule(dynamic, 4)
    for (int64_t row = 0; row < (int64_t)B * D; ++row) {
      const int b = (int)(row / D), d = (int)(row % D);
      Row r;
      memset(&r, 0, sizeof(r));
      r.L = L;
      r.N = N;
      r.min_len = min_len;
      r.split = split;
      r.ustride = D;
      r.bstride = N;
      r.u = u + (int64_t)b * L * D + d;
      r.dt = dt + (int64_t)b * L * D + d;
      r.Bc = Bc + (int64_t)b * L * N;
      r.Cc = Cc + (int64_t)b * L * N;
      r.A = A + (int64_t)d * N;
      r.y = y + (int64_t)b * L * D + d;
      r.scratch = scratch;
      float g[MAXN], h[MAXN];
      for (int n = 0; n < N; ++n) {
        g[n] = 1.0f;
        h[n] = 0.0f;
      }
      fwd_rec(&r, 0, L, g, h);
    }
    free(scratch);
  }
  return 0;
}

/* add one thread's channel sums for batch row b into dB, dC and clear them */
static void flush_bc(float* dB, float* dC, float* pB, float* pC, int b, int L, int N) {
#pragma omp critical
  {
    float* oB = dB + (int64_t)b * L * N;
    float* oC = dC + (int64_t)b * L * N;
    for (int64_t i = 0; i < (int64_t)L * N; ++i) {
      oB[i] += pB[i];
      oC[i] += pC[i];
    }
  }
  memset(pB, 0, sizeof(float) * (size_t)L * N);
  memset(pC, 0, sizeof(float) * (size_t)L * N);
}

/*
 * Backward (custom VJP): du, ddt (B,L,D), dA (D,N), dB, dC (B,L,N) for dy.
 */
int oracle_scan_bwd(int B, int L, int D, int N, const float* u, const float* dt, const float* A, const float* Bc,
                    const float* Cc, const float* dy, float* du, float* ddt, float* dA, float* dB, float* dC,
                    int min_len, int split, int nthreads) {
  if (N > MAXN || split < 2) return -1;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
  const size_t sf = leaf_scratch_floats(L, N, min_len, split);
  memset(dA, 0, sizeof(float) * (size_t)D * N);
  memset(dB, 0, sizeof(float) * (size_t)B * L * N);
  memset(dC, 0, sizeof(float) * (size_t)B * L * N);
#pragma omp parallel
  {
    float* scratch = (float*)malloc(sizeof(float) * sf);
    float* pB = (float*)calloc((size_t)L * N, sizeof(float));
    float* pC = (float*)calloc((size_t)L * N, sizeof(float));
    float* pA = (float*)calloc((size_t)D * N, sizeof(float));
    int cur_b = -1;
#pragma omp for schedule(static)
    for (int64_t row = 0; row < (int64_t)B * D; ++row) {
      const int b = (int)(row / D), d = (int)(row % D);
      if (b != cur_b) {
        if (cur_b >= 0) flush_bc(dB, dC, pB, pC, cur_b, L, N);
        cur_b = b;
      }
      Row r;
      memset(&r, 0, sizeof(r));
      r.L = L;
      r.N = N;
      r.min_len = min_len;
      r.split = split;
      r.ustride = D;
      r.bstride = N;
      r.u = u + (int64_t)b * L * D + d;
      r.dt = dt + (int64_t)b * L * D + d;
      r.dy = dy + (int64_t)b * L * D + d;
      r.Bc = Bc + (int64_t)b * L * N;
      r.Cc = Cc + (int64_t)b * L * N;
      r.A = A + (int64_t)d * N;
      r.du = du + (int64_t)b * L * D + d;
      r.ddt = ddt + (int64_t)b * L * D + d;
      r.dB = pB;
      r.dC = pC;
      r.dA = pA + (int64_t)d * N;
      r.scratch = scratch;
      float h[MAXN] = {0}, fa[MAXN] = {0};
      bwd_rec(&r, 0, L, h, fa);
    }
    if (cur_b >= 0) flush_bc(dB, dC, pB, pC, cur_b, L, N);
#pragma omp critical
    for (int64_t i = 0; i < (int64_t)D * N; ++i) dA[i] += pA[i];
    free(pA);
    free(pB);
    free(pC);
    free(scratch);
  }
  return 0;
}
