// The RTL's int8 GEMV and matvec checks on the MI355X: a drop-in for the
// reference's Verilator benches rtl/tb/sim_gemv.cpp (exact int32 accumulators)
// and rtl/tb/sim_matvec.cpp (fixed-point output within 4 LSB of the fp32 model).
//
//   qh_sim_matvec [<tv_gemv.bin>] [--outw N]   (default artifacts/tv_gemv.bin, OUTW 16)
//
// The file is scripts/export_gemv_tv.py:62-72's layout: int8 x[IN], int8
// w[OUT][IN], int32 acc[OUT], float32 sx, float32 sw[OUT], float32 y[OUT],
// little endian; IN and OUT come from the tv_gemv.json beside it ({"IN": 1024,
// "OUT": 512} when there is none, the reference benches' constants).  The
// multipliers are formed on the host as sim_matvec.cpp:36-41 forms them
// (qh_dequant_mult, SHIFT 16, OUTQ 14), qh_matvec_i8 runs the GEMV and the
// dequant on the device, and both reference criteria are applied.  --outw
// widens the output register as matvec_i8.sv's OUTW parameter does (16 in the
// reference bench; paths whose outputs leave the Q14 int16 range need more).  Exit code 0
// when both pass, 1 on a failure or a device error, 2 on an input error.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include "qh_decode.h"

namespace {
// {"IN": a, "OUT": b}: the two integers after the two keys
bool read_dims(const std::string& json_path, int* n_in, int* n_out) {
  std::ifstream f(json_path);
  if (!f) return false;
  std::stringstream ss;
  ss << f.rdbuf();
  const std::string t = ss.str();
  const size_t i = t.find("\"IN\""), o = t.find("\"OUT\"");
  if (i == std::string::npos || o == std::string::npos) return false;
  *n_in = std::atoi(t.c_str() + t.find(':', i) + 1);
  *n_out = std::atoi(t.c_str() + t.find(':', o) + 1);
  return true;
}
}  // namespace

int main(int argc, char** argv) {
  std::string path = "artifacts/tv_gemv.bin";
  int OUTW = 16;
  for (int i = 1; i < argc; ++i) {
    if (std::string(argv[i]) == "--outw" && i + 1 < argc) {
      OUTW = std::atoi(argv[++i]);
    } else if (argv[i][0] == '-') {
      std::fprintf(stderr, "usage: qh_sim_matvec [<tv_gemv.bin>] [--outw N]\n");
      return 2;
    } else {
      path = argv[i];
    }
  }
  const int SHIFT = 16, OUTQ = 14;
  if (OUTW < 1 || OUTW > 32) {
    std::fprintf(stderr, "--outw must be 1..32\n");
    return 2;
  }
  int IN = 1024, OUT = 512;
  const size_t dot = path.find_last_of('.');
  read_dims((dot == std::string::npos ? path : path.substr(0, dot)) + ".json", &IN, &OUT);
  if (IN <= 0 || OUT <= 0 || IN % 16 != 0 || IN > 4096) {
    std::fprintf(stderr, "unsupported dimensions IN=%d OUT=%d\n", IN, OUT);
    return 2;
  }
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  if (!f) {
    std::fprintf(stderr, "run scripts/export_gemv_tv.py first\n");
    return 2;
  }
  const size_t need = (size_t)IN + (size_t)OUT * IN + 4u * OUT + 4u + 8u * OUT;
  if ((size_t)f.tellg() != need) {
    std::fprintf(stderr, "%s: %lld bytes, IN=%d OUT=%d needs %zu\n", path.c_str(), (long long)f.tellg(), IN, OUT,
                 need);
    return 2;
  }
  f.seekg(0);
  std::vector<int8_t> x(IN), w((size_t)OUT * IN);
  std::vector<int32_t> acc_ref(OUT);
  float sx = 0.0f;
  std::vector<float> sw(OUT), y_ref(OUT);
  f.read(reinterpret_cast<char*>(x.data()), IN);
  f.read(reinterpret_cast<char*>(w.data()), (std::streamsize)w.size());
  f.read(reinterpret_cast<char*>(acc_ref.data()), 4L * OUT);
  f.read(reinterpret_cast<char*>(&sx), 4);
  f.read(reinterpret_cast<char*>(sw.data()), 4L * OUT);
  f.read(reinterpret_cast<char*>(y_ref.data()), 4L * OUT);

  std::vector<int32_t> mult(OUT);
  int st = qh_dequant_mult(mult.data(), sx, sw.data(), OUT, OUTQ, SHIFT);
  if (st != QH_OK) {
    std::fprintf(stderr, "dequant multipliers: %s\n", qh_strerror(st));
    return 2;
  }
  // device buffers: x (16-byte aligned) | w | mult | acc | y_q
  const size_t xb = ((size_t)IN + 255) & ~(size_t)255, wb = ((w.size() + 255) & ~(size_t)255);
  char* d = nullptr;
  if (hipMalloc(&d, xb + wb + 12u * OUT) != hipSuccess) {
    std::fprintf(stderr, "hipMalloc failed\n");
    return 1;
  }
  int8_t* dx = reinterpret_cast<int8_t*>(d);
  int8_t* dw = reinterpret_cast<int8_t*>(d + xb);
  int32_t* dmult = reinterpret_cast<int32_t*>(d + xb + wb);
  int32_t* dacc = dmult + OUT;
  int32_t* dyq = dacc + OUT;
  std::vector<int32_t> acc(OUT), yq(OUT);
  st = hipMemcpy(dx, x.data(), IN, hipMemcpyHostToDevice) == hipSuccess &&
               hipMemcpy(dw, w.data(), w.size(), hipMemcpyHostToDevice) == hipSuccess &&
               hipMemcpy(dmult, mult.data(), 4u * OUT, hipMemcpyHostToDevice) == hipSuccess
           ? QH_OK
           : QH_EDEVICE;
  if (st == QH_OK) st = qh_matvec_i8(dyq, dacc, dw, dmult, dx, OUT, IN, SHIFT, OUTW, nullptr);
  if (st == QH_OK && (hipMemcpy(acc.data(), dacc, 4u * OUT, hipMemcpyDeviceToHost) != hipSuccess ||
                      hipMemcpy(yq.data(), dyq, 4u * OUT, hipMemcpyDeviceToHost) != hipSuccess))
    st = QH_EDEVICE;
  (void)hipFree(d);
  if (st != QH_OK) {
    std::fprintf(stderr, "matvec_i8: %s\n", qh_strerror(st));
    return 1;
  }

  // sim_gemv.cpp: exact int32 accumulators
  int mism = 0;
  for (int o = 0; o < OUT; ++o)
    if (acc[o] != acc_ref[o]) {
      if (mism < 5) std::printf("  mismatch row %d: got %d exp %d\n", o, acc[o], acc_ref[o]);
      ++mism;
    }
  std::printf("gemv_i8 (MI355X): %d of %d accumulators exact\n", OUT - mism, OUT);
  const bool gemv_ok = mism == 0;
  std::printf("%s\n", gemv_ok ? "PASS  gemv_i8 == numpy int32 (bit-exact)" : "FAIL");

  // sim_matvec.cpp: Q14 output against round(y_fp32 * 2^14), within 4 LSB
  int bad = 0, worst = 0;
  for (int o = 0; o < OUT; ++o) {
    const int ref = (int)std::lround((double)y_ref[o] * (1 << OUTQ));
    const int dd = std::abs(yq[o] - ref);
    worst = dd > worst ? dd : worst;
    if (dd > 4) {
      if (bad < 5) std::printf("  row %d: got %d exp %d (d=%d)\n", o, yq[o], ref, dd);
      ++bad;
    }
  }
  std::printf("matvec_i8 (MI355X): %d rows, worst |diff| = %d LSB (Q%d, %d-bit output)\n", OUT, worst, OUTQ, OUTW);
  const bool mv_ok = bad == 0;
  std::printf("%s\n", mv_ok ? "PASS  matvec_i8 == model fp32 (within fixed-point rounding)" : "FAIL");
  return gemv_ok && mv_ok ? 0 : 1;
}
