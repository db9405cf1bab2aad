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
 * OpenMP parallelises over rows.  The arithmetic is float32 like the
 * reference; the associative-scan leaf keeps the reference's combine order.
 * Compiled a second time with -DORACLE_F64, the same algorithm runs in
 * float64 and exports its entry points with an _f64 suffix: an fp64 oracle
 * for sizes the numpy restatement cannot reach (long sums such as dA over
 * 2^20 steps).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#ifdef ORACLE_F64
typedef double real;
#define EXP exp
#define SUFFIX(name) name##_f64
#else
typedef float real;
#define EXP expf
#define SUFFIX(name) name
#endif

#define MAXN 64

typedef struct {
  int L, N, min_len, split;
  const real *u, *dt, *Bc, *Cc, *dy; /* row views: u[t*ustride] etc. */
  int64_t ustride, bstride;           /* D for (B,L,D) rows, N for (B,L,N) rows */
  const real* A;                     /* A[d, 0..N) */
  real* y;                           /* forward output row */
  real *du, *ddt;                    /* backward output rows */
  real *dB, *dC;                     /* (L,N) thread-private accumulators */
  real* dA;                          /* (N) thread-private accumulator */
  real* scratch;                     /* leaf workspace */
} Row;

/* inclusive scan of (g,h) pairs with the odd/even recursion of
 * jax.lax.associative_scan; combine(l, r) = (g_l g_r, g_r h_l + h_r). */
static void assoc_scan(real* g, real* h, int n, real* tmp) {
  if (n < 2) return;
  int m = n / 2; /* number of pairs */
  real* rg = tmp;
  real* rh = tmp + m;
  for (int i = 0; i < m; ++i) {
    real gl = g[2 * i], hl = h[2 * i], gr = g[2 * i + 1], hr = h[2 * i + 1];
    rg[i] = gl * gr;
    rh[i] = gr * hl + hr;
  }
  assoc_scan(rg, rh, m, tmp + 2 * m);
  /* odd positions 1,3,.. take the reduced prefixes; even positions 2,4,.. combine
   * the previous odd prefix with the original element */
  for (int i = 1; 2 * i < n; ++i) {
    real gl = rg[i - 1], hl = rh[i - 1], gr = g[2 * i], hr = h[2 * i];
    g[2 * i] = gl * gr;
    h[2 * i] = gr * hl + hr;
  }
  for (int i = 0; i < m; ++i) {
    g[2 * i + 1] = rg[i];
    h[2 * i + 1] = rh[i];
  }
}

/* ---------------------------------------------------------------- forward */

static void fwd_rec(Row* r, int t0, int len, real* g, real* h) {
  if (len > r->min_len && len % r->split == 0) {
    int m = len / r->split;
    for (int i = 0; i < r->split; ++i) fwd_rec(r, t0 + i * m, m, g, h);
    return;
  }
  const int N = r->N;
  for (int n = 0; n < N; ++n) {
    real* ga = r->scratch;
    real* ha = ga + len;
    real* tmp = ha + len;
    for (int i = 0; i < len; ++i) {
      const int t = t0 + i;
      const real d = r->dt[t * r->ustride];
      ga[i] = EXP(r->A[n] * d);
      ha[i] = r->Bc[t * r->bstride + n] * r->u[t * r->ustride] * d;
    }
    assoc_scan(ga, ha, len, tmp);
    for (int i = 0; i < len; ++i) {
      const int t = t0 + i;
      const real hs = ga[i] * h[n] + ha[i];
      r->y[t * r->ustride] += r->Cc[t * r->bstride + n] * hs;
      if (i == len - 1) {
        g[n] = ga[i] * g[n];
        h[n] = hs;
      }
    }
  }
}

/* --------------------------------------------------------------- backward */

static void bwd_rec(Row* r, int t0, int len, real* h_left, const real* fa_right) {
  const int N = r->N;
  if (len > r->min_len && len % r->split == 0) {
    const int m = len / r->split;
    real* fas = (real*)malloc(sizeof(real) * r->split * N);
    real fa[MAXN];
    memcpy(fa, fa_right, sizeof(real) * N);
    for (int i = r->split - 1; i >= 0; --i) {
      memcpy(fas + i * N, fa, sizeof(real) * N);
      for (int t = t0 + i * m + m - 1; t >= t0 + i * m; --t) {
        const real d = r->dt[t * r->ustride];
        const real dyv = r->dy[t * r->ustride];
        for (int n = 0; n < N; ++n) {
          const real alpha = EXP(r->A[n] * d);
          const real f = fa[n] + r->Cc[t * r->bstride + n] * dyv;
          fa[n] = f * alpha;
        }
      }
    }
    for (int i = 0; i < r->split; ++i) bwd_rec(r, t0 + i * m, m, h_left, fas + i * N);
    free(fas);
    return;
  }
  real* hs = r->scratch;   /* len*N: h_{t-1} */
  real* al = hs + len * N; /* len*N: alpha_t */
  real* fs = al + len * N; /* len*N: f_t */
  for (int i = 0; i < len; ++i) {
    const int t = t0 + i;
    const real d = r->dt[t * r->ustride], uu = r->u[t * r->ustride];
    for (int n = 0; n < N; ++n) {
      const real a = EXP(r->A[n] * d);
      al[i * N + n] = a;
      hs[i * N + n] = h_left[n];
      h_left[n] = h_left[n] * a + r->Bc[t * r->bstride + n] * uu * d;
    }
  }
  real fa[MAXN];
  memcpy(fa, fa_right, sizeof(real) * N);
  for (int i = len - 1; i >= 0; --i) {
    const int t = t0 + i;
    const real dyv = r->dy[t * r->ustride];
    for (int n = 0; n < N; ++n) {
      const real f = fa[n] + r->Cc[t * r->bstride + n] * dyv;
      fs[i * N + n] = f;
      fa[n] = f * al[i * N + n];
    }
  }
  for (int i = 0; i < len; ++i) {
    const int t = t0 + i;
    const real d = r->dt[t * r->ustride], uu = r->u[t * r->ustride], dyv = r->dy[t * r->ustride];
    real dx = (real)0, ddt = (real)0;
    for (int n = 0; n < N; ++n) {
      const real f = fs[i * N + n];
      const real Bn = r->Bc[t * r->bstride + n];
      const real ah = al[i * N + n] * hs[i * N + n];
      const real df = d * f;
      const real hnext = (i + 1 < len) ? hs[(i + 1) * N + n] : h_left[n];
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
int SUFFIX(oracle_scan_fwd)(int B, int L, int D, int N, const real* u, const real* dt, const real* A, const real* Bc,
                    const real* Cc, real* y, int min_len, int split, int nthreads) {
  if (N > MAXN || split < 2) return -1;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
  const size_t sf = leaf_scratch_floats(L, N, min_len, split);
  memset(y, 0, sizeof(real) * (size_t)B * L * D);
#pragma omp parallel
  {
    real* scratch = (real*)malloc(sizeof(real) * sf);
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
      real g[MAXN], h[MAXN];
      for (int n = 0; n < N; ++n) {
        g[n] = (real)1;
        h[n] = (real)0;
      }
      fwd_rec(&r, 0, L, g, h);
    }
    free(scratch);
  }
  return 0;
}

/* add one thread's channel sums for batch row b into dB, dC and clear them */
static void flush_bc(real* dB, real* dC, real* pB, real* pC, int b, int L, int N) {
#pragma omp critical
  {
    real* oB = dB + (int64_t)b * L * N;
    real* oC = dC + (int64_t)b * L * N;
    for (int64_t i = 0; i < (int64_t)L * N; ++i) {
      oB[i] += pB[i];
      oC[i] += pC[i];
    }
  }
  memset(pB, 0, sizeof(real) * (size_t)L * N);
  memset(pC, 0, sizeof(real) * (size_t)L * N);
}

/*
 * Backward (custom VJP): du, ddt (B,L,D), dA (D,N), dB, dC (B,L,N) for dy.
 */
int SUFFIX(oracle_scan_bwd)(int B, int L, int D, int N, const real* u, const real* dt, const real* A, const real* Bc,
                    const real* Cc, const real* dy, real* du, real* ddt, real* dA, real* dB, real* dC,
                    int min_len, int split, int nthreads) {
  if (N > MAXN || split < 2) return -1;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
  const size_t sf = leaf_scratch_floats(L, N, min_len, split);
  memset(dA, 0, sizeof(real) * (size_t)D * N);
  memset(dB, 0, sizeof(real) * (size_t)B * L * N);
  memset(dC, 0, sizeof(real) * (size_t)B * L * N);
#pragma omp parallel
  {
    real* scratch = (real*)malloc(sizeof(real) * sf);
    real* pB = (real*)calloc((size_t)L * N, sizeof(real));
    real* pC = (real*)calloc((size_t)L * N, sizeof(real));
    real* pA = (real*)calloc((size_t)D * N, sizeof(real));
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
      real h[MAXN] = {0}, fa[MAXN] = {0};
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
