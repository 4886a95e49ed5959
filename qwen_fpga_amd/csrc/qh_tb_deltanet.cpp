// Delta-rule testbench on the MI355X op-level ABI, a drop-in for the
// reference's tb_deltanet (hls/tb/tb_deltanet.cpp:54-93).
//
//   qh_tb_deltanet [<tv_deltanet.bin>]        (default artifacts/tv_deltanet.bin)
//
// The file is scripts/export_testvectors.py:55-60's layout, float32 little
// endian, one tensor after another: q [16][128] (after l2norm and the 1/sqrt(128)
// scale), k [16][128], v [16][128], g [16], beta [16], S_in [16][128][128],
// o_core [16][128], S_out [16][128][128] -- 2,130,048 bytes.  S_in is updated
// by qh_delta_rule_layer; the run passes when the output and the new state are
// within 2e-5 (max |d|) of o_core and S_out, the reference testbench's
// tolerance.  Exit code 0 on PASS, 1 on FAIL or a device error, 2 on an input
// error.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdio>
#include <fstream>
#include <vector>

#include "qh_decode.h"

namespace {
constexpr int H = 16, K = 128, V = 128;
struct Stat {
  double max_abs = 0.0, max_rel = 0.0;
};
Stat compare(const float* a, const float* b, size_t n) {
  Stat s;
  for (size_t i = 0; i < n; ++i) {
    const double d = std::fabs((double)a[i] - (double)b[i]);
    s.max_abs = d > s.max_abs ? d : s.max_abs;
    const double den = std::fabs((double)b[i]);
    if (den > 1e-6) s.max_rel = d / den > s.max_rel ? d / den : s.max_rel;
  }
  return s;
}
}  // namespace

int main(int argc, char** argv) {
  const char* path = argc > 1 ? argv[1] : "artifacts/tv_deltanet.bin";
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  if (!f) {
    std::fprintf(stderr, "open %s failed -- run scripts/export_testvectors.py first\n", path);
    return 2;
  }
  const size_t want = (size_t)(3 * H * K + 2 * H + H * K * V + H * V + H * K * V);
  const size_t bytes = (size_t)f.tellg();
  if (bytes != want * 4) {
    std::fprintf(stderr, "test vector size mismatch: %zu bytes, layout needs %zu\n", bytes, want * 4);
    return 2;
  }
  std::vector<float> tv(want);
  f.seekg(0);
  f.read(reinterpret_cast<char*>(tv.data()), (std::streamsize)(want * 4));
  // q, k, v, g, beta (nin floats, copied to the device as they lie), then S_in, o_core, S_out
  const size_t nin = 3 * H * K + 2 * H, nS = (size_t)H * K * V;
  const float* S_in = &tv[nin];
  const float* o_ref = S_in + nS;
  const float* S_ref = o_ref + H * V;

  // device copies: q k v g beta | S | out
  float* d = nullptr;
  if (hipMalloc(&d, (nin + nS + H * V) * sizeof(float)) != hipSuccess) {
    std::fprintf(stderr, "hipMalloc failed\n");
    return 1;
  }
  float* dS = d + nin;
  float* dout = dS + nS;
  int st = hipMemcpy(d, tv.data(), nin * sizeof(float), hipMemcpyHostToDevice) == hipSuccess &&
                   hipMemcpy(dS, S_in, nS * sizeof(float), hipMemcpyHostToDevice) == hipSuccess
               ? QH_OK
               : QH_EDEVICE;
  if (st == QH_OK)
    st = qh_delta_rule_layer(d, d + H * K, d + 2 * H * K, d + 3 * H * K, d + 3 * H * K + H, dS, dout, nullptr);
  std::vector<float> S(nS), out(H * V);
  if (st == QH_OK &&
      (hipMemcpy(S.data(), dS, nS * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess ||
       hipMemcpy(out.data(), dout, H * V * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess))
    st = QH_EDEVICE;
  (void)hipFree(d);
  if (st != QH_OK) {
    std::fprintf(stderr, "delta_rule_layer: %s\n", qh_strerror(st));
    return 1;
  }
  const Stat so = compare(out.data(), o_ref, (size_t)H * V);
  const Stat ss = compare(S.data(), S_ref, nS);
  std::printf("delta_rule_layer  H=%d K=%d V=%d  (MI355X)\n", H, K, V);
  std::printf("  out  max|d| %.3e   max rel %.3e   (%d elems)\n", so.max_abs, so.max_rel, H * V);
  std::printf("  S'   max|d| %.3e   max rel %.3e   (%d elems)\n", ss.max_abs, ss.max_rel, H * K * V);
  const double TOL = 2e-5;   // fp32 reassociation only (tb_deltanet.cpp:89)
  const bool ok = so.max_abs < TOL && ss.max_abs < TOL;
  std::printf("%s (tol %.0e)\n", ok ? "PASS" : "FAIL", TOL);
  return ok ? 0 : 1;
}
