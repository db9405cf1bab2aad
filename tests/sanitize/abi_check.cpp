// abi_check.cpp — the library's host-side validation and size-query paths and
// the C oracle, run under AddressSanitizer and UndefinedBehaviorSanitizer (host
// code only; see Makefile).  No GPU is needed: every library call here is
// refused by validation before it would touch the device, and the oracle is
// plain C.  Exits 0 when every check holds; a sanitizer report aborts.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "selectssm.h"

extern "C" {
int oracle_scan_fwd(int B, int L, int D, int N, const float* u, const float* dt, const float* A, const float* Bc,
                    const float* Cc, float* y, int min_len, int split, int nthreads);
int oracle_scan_bwd(int B, int L, int D, int N, const float* u, const float* dt, const float* A, const float* Bc,
                    const float* Cc, const float* dy, float* du, float* ddt, float* dA, float* dB, float* dC,
                    int min_len, int split, int nthreads);
int oracle_scan_fwd_f64(int B, int L, int D, int N, const double* u, const double* dt, const double* A,
                        const double* Bc, const double* Cc, double* y, int min_len, int split, int nthreads);
int oracle_scan_bwd_f64(int B, int L, int D, int N, const double* u, const double* dt, const double* A,
                        const double* Bc, const double* Cc, const double* dy, double* du, double* ddt, double* dA,
                        double* dB, double* dC, int min_len, int split, int nthreads);
}

static int g_fail = 0;

static void check(bool ok, const std::string& what) {
  if (!ok) {
    std::printf("FAIL: %s (last error: \"%s\")\n", what.c_str(), ssm_last_error());
    ++g_fail;
  }
}

static ssm_desc_t desc(int64_t B, int64_t L, int64_t D, int64_t N) {
  ssm_desc_t d;
  std::memset(&d, 0, sizeof d);
  d.batch = B;
  d.seqlen = L;
  d.dim = D;
  d.dstate = N;
  d.dtype = SSM_F32;
  return d;
}

// an address that is never dereferenced: every call below fails validation first
static void* const P = reinterpret_cast<void*>(uintptr_t(256));

static void size_queries() {
  std::mt19937 rng(1);
  for (int i = 0; i < 400; ++i) {
    ssm_desc_t d = desc(1 + rng() % 64, 1 + rng() % 50000, 1 + rng() % 3000, 1 + rng() % 32);
    d.segments = rng() % 3 == 0 ? int32_t(rng() % 1025) : 0;
    d.delta_broadcast = int32_t(rng() % 2);
    d.dtype = int32_t(rng() % 2);
    const size_t ck = ssm_ckpt_bytes(&d);
    const size_t fw = ssm_fwd_workspace_bytes(&d);
    const size_t bw = ssm_bwd_workspace_bytes(&d);
    check(ck == size_t(d.batch) * ((d.seqlen + 15) / 16) * d.dstate * d.dim * 4, "checkpoint size formula");
    check(bw > 0 && std::strlen(ssm_last_error()) == 0, "valid desc: workspace size, no error");
    // whole aggregates (end state and decay product per state and channel), and with
    // pieces an int flag per 64-channel block each
    const size_t per = 2 * size_t(d.batch) * d.dstate * d.dim * 4;
    const size_t per_flagged = per + size_t(d.batch) * ((d.dim + 63) / 64) * 4;
    check(fw % per == 0 || fw % per_flagged == 0, "forward workspace holds whole segments");
  }
}

static void invalid_descs() {
  struct Case {
    const char* field;
    void (*set)(ssm_desc_t&);
  };
  const Case cases[] = {
      {"batch 0", [](ssm_desc_t& d) { d.batch = 0; }},
      {"batch 65536", [](ssm_desc_t& d) { d.batch = 65536; }},
      {"seqlen -1", [](ssm_desc_t& d) { d.seqlen = -1; }},
      {"dstate 33", [](ssm_desc_t& d) { d.dstate = 33; }},
      {"dtype 9", [](ssm_desc_t& d) { d.dtype = 9; }},
      {"skip-map bits without SSM_SKIP_MAP", [](ssm_desc_t& d) { d.flags = SSM_SKIP_REVERSE; }},
      {"flags 512", [](ssm_desc_t& d) { d.flags = 512; }},
      {"SSM_ACCUMULATE without SSM_GATE", [](ssm_desc_t& d) { d.flags = SSM_ACCUMULATE; }},
      {"delta_broadcast 2", [](ssm_desc_t& d) { d.delta_broadcast = 2; }},
      {"segments 1025", [](ssm_desc_t& d) { d.segments = 1025; }},
      {"ld_y < dim", [](ssm_desc_t& d) { d.ld_y = 3; }},
      {"ld_z huge", [](ssm_desc_t& d) { d.ld_z = int64_t(1) << 40; }},
      {"ld_bc < dstate", [](ssm_desc_t& d) { d.ld_bc = 2; }},
      {"seqlen*dim > 2^30", [](ssm_desc_t& d) { d.seqlen = int64_t(1) << 21; d.dim = 1024; }},
      {"seqlen overflow", [](ssm_desc_t& d) { d.seqlen = int64_t(1) << 62; }},
      {"dim overflow", [](ssm_desc_t& d) { d.dim = int64_t(1) << 62; }},
      {"ld_y overflow", [](ssm_desc_t& d) { d.ld_y = int64_t(1) << 62; }},
      {"ld_bc overflow", [](ssm_desc_t& d) { d.ld_bc = int64_t(1) << 62; }},
      {"ld_bc negative", [](ssm_desc_t& d) { d.ld_bc = -64; }},
  };
  for (const Case& c : cases) {
    ssm_desc_t d = desc(2, 64, 64, 16);
    c.set(d);
    check(ssm_ckpt_bytes(&d) == 0 && std::strlen(ssm_last_error()) > 0, std::string("size query rejects ") + c.field);
    check(ssm_fwd(nullptr, &d, P, P, (const float*)P, P, P, nullptr, nullptr, P, nullptr, nullptr) ==
              SSM_ERR_INVALID,
          std::string("ssm_fwd rejects ") + c.field);
    check(ssm_bwd(nullptr, &d, P, P, (const float*)P, P, P, nullptr, nullptr, (const float*)P, P, P, P,
                  (float*)P, P, P, nullptr, nullptr, P) == SSM_ERR_INVALID,
          std::string("ssm_bwd rejects ") + c.field);
    check(ssm_bwd_static(nullptr, &d, P, P, (const float*)P, P, P, nullptr, nullptr, (const float*)P, P, P, P,
                         (float*)P, P, P, nullptr, nullptr) == SSM_ERR_INVALID,
          std::string("ssm_bwd_static rejects ") + c.field);
  }
  check(ssm_fwd(nullptr, nullptr, P, P, (const float*)P, P, P, nullptr, nullptr, P, nullptr, nullptr) ==
            SSM_ERR_INVALID,
        "NULL desc");
}

static void missing_operands() {
  ssm_desc_t d = desc(2, 64, 64, 16);
  check(ssm_fwd(nullptr, &d, nullptr, P, (const float*)P, P, P, nullptr, nullptr, P, nullptr, nullptr) ==
            SSM_ERR_INVALID,
        "ssm_fwd: NULL u");
  d.flags = SSM_SKIP;
  check(ssm_fwd(nullptr, &d, P, P, (const float*)P, P, P, nullptr, nullptr, P, nullptr, nullptr) ==
            SSM_ERR_INVALID,
        "SSM_SKIP without Dskip");
  d.flags = SSM_GATE;
  check(ssm_bwd(nullptr, &d, P, P, (const float*)P, P, P, nullptr, P, (const float*)P, P, P, P, (float*)P, P, P,
                nullptr, nullptr, P) == SSM_ERR_INVALID,
        "SSM_GATE without dz");
  ssm_desc_t split = desc(2, 100, 8, 4);
  split.segments = 3;
  check(ssm_fwd(nullptr, &split, P, P, (const float*)P, P, P, nullptr, nullptr, P, nullptr, nullptr) ==
            SSM_ERR_INVALID,
        "time-split forward without workspace");
  ssm_desc_t big = desc(8, 8192, 2048, 16);
  check(ssm_bwd_static(nullptr, &big, P, P, (const float*)P, P, P, nullptr, nullptr, (const float*)P, P, P, P,
                       (float*)P, P, P, nullptr, nullptr) == SSM_ERR_INVALID &&
            std::strstr(ssm_last_error(), "static scratch") != nullptr,
        "ssm_bwd_static refuses a workspace beyond its scratch");
}

static void pairs() {
  ssm_desc_t d[2] = {desc(2, 64, 64, 16), desc(2, 64, 64, 16)};
  ssm_fwd_io_t fio[2];
  ssm_bwd_io_t bio[2];
  for (int k = 0; k < 2; ++k) {
    fio[k] = ssm_fwd_io_t{P, P, (const float*)P, P, P, nullptr, nullptr, P, nullptr, nullptr};
    bio[k] = ssm_bwd_io_t{P, P, (const float*)P, P, P, nullptr, nullptr, (const float*)P, P,
                          P, P, (float*)P, P, P, nullptr, nullptr, P};
  }
  for (int32_t t : {SSM_F32, SSM_BF16}) {
    d[0].dtype = t;
    d[1].dtype = t == SSM_F32 ? SSM_BF16 : SSM_F32;
    check(ssm_fwd_pair(nullptr, d, fio) == SSM_ERR_INVALID && std::strstr(ssm_last_error(), "same dtype"),
          "ssm_fwd_pair refuses mixed dtypes");
    check(ssm_bwd_pair(nullptr, d, bio) == SSM_ERR_INVALID && std::strstr(ssm_last_error(), "same dtype"),
          "ssm_bwd_pair refuses mixed dtypes");
  }
  d[0].dtype = d[1].dtype = SSM_F32;
  d[1].dstate = 40;
  check(ssm_fwd_pair(nullptr, d, fio) == SSM_ERR_INVALID, "ssm_fwd_pair validates both descs");
  d[1].dstate = 16;
  fio[1].y = nullptr;
  check(ssm_fwd_pair(nullptr, d, fio) == SSM_ERR_INVALID, "ssm_fwd_pair: NULL y of the second call");
  check(ssm_fwd_pair(nullptr, nullptr, fio) == SSM_ERR_INVALID, "ssm_fwd_pair: NULL desc");
  check(ssm_bwd_pair(nullptr, d, nullptr) == SSM_ERR_INVALID, "ssm_bwd_pair: NULL io");
}

static void conv() {
  ssm_conv_desc_t c;
  std::memset(&c, 0, sizeof c);
  c.batch = 2;
  c.seqlen = 128 * 100;
  c.dim = 64;
  c.ksize = 4;
  c.dtype = SSM_F32;
  c.activation = SSM_ACT_SILU;
  check(ssm_conv_bwd_workspace_bytes(&c) == size_t(200 + 4) * 4 * 64 * 4, "conv workspace formula");
  c.ksize = 9;
  check(ssm_conv_fwd(nullptr, &c, P, (const float*)P, P) == SSM_ERR_INVALID, "conv rejects ksize 9");
  c.ksize = 4;
  c.flags = SSM_SKIP;
  check(ssm_conv_fwd(nullptr, &c, P, (const float*)P, P) == SSM_ERR_INVALID, "conv rejects scan-only flags");
  c.flags = 0;
  check(ssm_conv_bwd(nullptr, &c, P, (const float*)P, P, P, (float*)P, nullptr) == SSM_ERR_INVALID,
        "conv backward needs its workspace for dw");
  for (int64_t big : {int64_t(1) << 40, int64_t(1) << 62}) {
    ssm_conv_desc_t b = c;
    b.seqlen = big;
    check(ssm_conv_fwd(nullptr, &b, P, (const float*)P, P) == SSM_ERR_INVALID, "conv rejects a huge seqlen");
    b = c;
    b.ld_x = big;
    check(ssm_conv_bwd_workspace_bytes(&b) == 0, "conv rejects a huge ld_x");
    b = c;
    b.dim = big;
    check(ssm_conv_fwd(nullptr, &b, P, (const float*)P, P) == SSM_ERR_INVALID, "conv rejects a huge dim");
  }
}

template <typename R, typename Fwd, typename Bwd>
static void oracle_case(int B, int L, int D, int N, int min_len, int split, Fwd fwd, Bwd bwd, std::vector<double>* y_out) {
  std::mt19937 rng(B * 1000 + L + D + N);
  std::normal_distribution<double> nd;
  std::uniform_real_distribution<double> ud(0.0, std::log(16.0));
  const size_t bld = size_t(B) * L * D, bln = size_t(B) * L * N;
  std::vector<R> u(bld), dt(bld), A(size_t(D) * N), Bc(bln), Cc(bln), dy(bld), y(bld), du(bld), ddt(bld),
      dA(size_t(D) * N), dB(bln), dC(bln);
  for (size_t i = 0; i < bld; ++i) {
    u[i] = R(nd(rng));
    dt[i] = R(std::log1p(std::exp(0.5 * nd(rng) - 4.0)));
    dy[i] = R(nd(rng));
  }
  for (auto& a : A) a = R(-std::exp(ud(rng)));
  for (size_t i = 0; i < bln; ++i) {
    Bc[i] = R(0.25 * nd(rng));
    Cc[i] = R(0.25 * nd(rng));
  }
  check(fwd(B, L, D, N, u.data(), dt.data(), A.data(), Bc.data(), Cc.data(), y.data(), min_len, split, 1) == 0,
        "oracle forward runs");
  check(bwd(B, L, D, N, u.data(), dt.data(), A.data(), Bc.data(), Cc.data(), dy.data(), du.data(), ddt.data(),
            dA.data(), dB.data(), dC.data(), min_len, split, 1) == 0,
        "oracle backward runs");
  bool finite = true;
  for (size_t i = 0; i < bld; ++i) finite = finite && std::isfinite(double(y[i])) && std::isfinite(double(du[i]));
  for (auto v : dA) finite = finite && std::isfinite(double(v));
  check(finite, "oracle outputs are finite");
  y_out->assign(y.begin(), y.end());
}

static void oracle() {
  // odd leaves (L = 1000 -> 125, 81 with split 3, L = 7, L = 1), split 4, N up to 32
  const int shapes[][6] = {{2, 96, 8, 4, 2, 2}, {1, 1000, 5, 16, 2, 2}, {2, 81, 3, 3, 2, 3},
                           {1, 64, 5, 32, 3, 4}, {3, 7, 4, 2, 2, 2},   {2, 1, 9, 16, 2, 2}};
  for (const auto& s : shapes) {
    std::vector<double> y32, y64;
    oracle_case<float>(s[0], s[1], s[2], s[3], s[4], s[5], oracle_scan_fwd, oracle_scan_bwd, &y32);
    oracle_case<double>(s[0], s[1], s[2], s[3], s[4], s[5], oracle_scan_fwd_f64, oracle_scan_bwd_f64, &y64);
    double err = 0.0;
    for (size_t i = 0; i < y32.size(); ++i) err = std::fmax(err, std::fabs(y32[i] - y64[i]) / (1e-5 + std::fabs(y64[i])));
    check(err < 1e-2, "float32 and float64 oracle forwards agree");
  }
  std::vector<float> x(4, 0.0f);
  check(oracle_scan_fwd(1, 1, 1, 65, x.data(), x.data(), x.data(), x.data(), x.data(), x.data(), 2, 2, 1) == -1,
        "oracle refuses N > 64");
  check(oracle_scan_fwd(1, 1, 1, 1, x.data(), x.data(), x.data(), x.data(), x.data(), x.data(), 2, 1, 1) == -1,
        "oracle refuses split 1");
}

int main() {
  check(ssm_abi_version() == SSM_ABI_VERSION, "ABI version");
  size_queries();
  invalid_descs();
  missing_operands();
  pairs();
  conv();
  oracle();
  if (g_fail) {
    std::printf("%d check(s) failed\n", g_fail);
    return 1;
  }
  std::printf("abi_check: all checks passed\n");
  return 0;
}
