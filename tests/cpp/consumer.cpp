// A C++ consumer of the drop-in boundary: compiled against ltx25_ops.h (the
// ltx25::Ops facade with MetalOps' member names, src/ltx25-metal-ops.h:
// 64-105) and linked against libltx25_qlinear.so, as a plugin build would
// link it. Checked against the oracle (oracle/liboracle.so, test
// infrastructure).
//
// Runs: Ops::init, Ops::linear(QWeight) with a bf16 bias, Ops::linear_gelu,
// the dense Ops::linear, then wait_ok; then a malformed call whose failure
// the facade holds until wait_ok, as the reference's callers learn of
// failures at wait_ok (src/ltx25-dit.cc:1922-1933).
//
// Exit codes: 0 all checks passed; 1 a check failed; 3 init failed (no
// gfx950 device: the expected outcome on a host without one).
#include "ltx25_ops.h"
#include "oracle.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace {

int g_failed = 0;

void expect(bool ok, const char* what)
{
  if (!ok) {
    std::printf("FAIL: %s\n", what);
    g_failed = 1;
  }
}

double max_rel(const std::vector<float>& got, const std::vector<float>& ref)
{
  double num = 0.0;
  double den = 0.0;
  for (size_t i = 0; i < got.size(); ++i) {
    num = std::fmax(num, std::fabs((double)got[i] - ref[i]));
    den = std::fmax(den, std::fabs((double)ref[i]));
  }
  return num / (den > 0 ? den : 1e-30);
}

template <typename T>
T* upload(const std::vector<T>& h)
{
  void* d = nullptr;
  if (hipMalloc(&d, h.size() * sizeof(T)) != hipSuccess) { return nullptr; }
  if (hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess) {
    return nullptr;
  }
  return (T*)d;
}

std::vector<float> download_bf16(const void* d, size_t n)
{
  std::vector<uint16_t> h(n);
  (void)hipMemcpy(h.data(), d, n * 2, hipMemcpyDeviceToHost);
  std::vector<float> f(n);
  orc_bf16_to_f32_n(h.data(), f.data(), n);
  return f;
}

}  // namespace

int main()
{
  ltx25::Ops ops;
  std::string err;
  if (!ops.init(&err)) {
    std::printf("NODEV: %s\n", err.c_str());
    return 3;
  }
  if (!ops.quant_available()) {
    std::printf("FAIL: quant_available is false after a successful init\n");
    return 1;
  }
  const int M = 200, K = 512, N = 384;
  std::vector<float> x(M * K), w(N * K), bias(N);
  orc_fill_normal(x.data(), x.size(), 101, 0.0f, 1.0f);
  orc_fill_normal(w.data(), w.size(), 102, 0.0f, 0.02f);
  orc_fill_normal(bias.data(), bias.size(), 103, 0.0f, 0.5f);
  std::vector<uint16_t> xb(M * K), bb(N);
  orc_f32_to_bf16_n(x.data(), xb.data(), xb.size());
  orc_f32_to_bf16_n(bias.data(), bb.data(), bb.size());
  orc_bf16_to_f32_n(xb.data(), x.data(), x.size());       // the bf16 values the GPU sees
  orc_bf16_to_f32_n(bb.data(), bias.data(), bias.size());
  std::vector<uint32_t> codes(N * K / 4);
  std::vector<uint16_t> sc(N * K / 64), qb(N * K / 64), wdb(N * K);
  std::vector<float> wdf(N * K);
  orc_quantize_affine(w.data(), N, K, 8, 64, codes.data(), sc.data(), qb.data(), nullptr);
  orc_dequant(codes.data(), sc.data(), qb.data(), N, K, 8, 64, wdf.data(), wdb.data());

  hipStream_t st = nullptr;
  if (hipStreamCreate(&st) != hipSuccess) { std::printf("FAIL: stream\n"); return 1; }
  void* dx = upload(xb);
  void* dcodes = upload(codes);
  void* dsc = upload(sc);
  void* dqb = upload(qb);
  void* dbias = upload(bb);
  void* dwd = upload(wdb);
  void *dy = nullptr, *dg = nullptr, *dd = nullptr;
  if (!dx || !dcodes || !dsc || !dqb || !dbias || !dwd || hipMalloc(&dy, M * N * 2) != hipSuccess ||
      hipMalloc(&dg, M * N * 2) != hipSuccess || hipMalloc(&dd, M * N * 2) != hipSuccess) {
    std::printf("FAIL: device allocation\n");
    return 1;
  }
  ltx25::QWeight qw;
  qw.codes = dcodes;
  qw.scales = dsc;
  qw.qbias = dqb;
  qw.bits = 8;
  qw.group = 64;
  qw.quantized = true;
  expect(!qw.empty(), "QWeight::empty on a bound weight");

  ops.linear(st, dx, qw, dbias, dy, M, K, N);
  ops.linear_gelu(st, dx, qw, dbias, dg, M, K, N);
  ops.linear(st, dx, dwd, dbias, dd, M, K, N);
  expect(ops.wait_ok(st, &err), "wait_ok after three good dispatches");

  std::vector<float> ref(M * N), ref_g(M * N);
  orc_linear_f64(x.data(), wdf.data(), bias.data(), M, K, N, ref.data());
  orc_gelu_tanh(ref.data(), ref_g.data(), ref.size());
  const std::vector<float> y = download_bf16(dy, M * N);
  const std::vector<float> g = download_bf16(dg, M * N);
  const std::vector<float> d = download_bf16(dd, M * N);
  const double e_lin = max_rel(y, ref), e_gelu = max_rel(g, ref_g);
  std::printf("linear max-rel %.3e, linear_gelu max-rel %.3e\n", e_lin, e_gelu);
  expect(e_lin <= 1e-2, "linear(QWeight) within 1e-2 of the oracle");
  expect(e_gelu <= 1e-2, "linear_gelu within 1e-2 of the oracle");
  expect(std::memcmp(y.data(), d.data(), y.size() * sizeof(float)) == 0,
         "quantized and dense-over-the-dequantized-weight linears are bit-identical");

  // a malformed dispatch: K not a multiple of the group. It returns void, the
  // failure is held and reported by the next wait_ok, then cleared.
  ops.linear(st, dx, qw, dbias, dy, M, K - 8, N);
  const bool ok_bad = ops.wait_ok(st, &err);
  expect(!ok_bad, "wait_ok reports the held dispatch failure");
  expect(err.find("group") != std::string::npos, "the held message names the cause");
  std::printf("held failure: %s\n", err.c_str());
  expect(ops.wait_ok(st, &err), "the failure is cleared after it is reported");

  for (void* p : {dx, dcodes, dsc, dqb, dbias, dwd, dy, dg, dd}) { (void)hipFree(p); }
  (void)hipStreamDestroy(st);
  if (g_failed == 0) { std::printf("OK\n"); }
  return g_failed;
}
