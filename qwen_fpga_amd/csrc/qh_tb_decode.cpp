// End-to-end decode testbench on the MI355X engine, a drop-in for the
// reference's tb_decode (hls/tb/tb_decode.cpp:67-112).
//
//   qh_tb_decode [<blob> [<weights.idx|-> [<decode_ref.bin>]]] [--w8a8] [--persistent]
//
// Defaults are the reference's paths: artifacts/qwen35_int8.bin,
// artifacts/weights.idx and artifacts/decode_ref.bin.  decode_ref.bin is the
// flat file of scripts/export_decode_ref.py:47-53: int32 n, int32 fed[n],
// int32 argmax[n], float32 logits0[QH_VOCAB] (step-0 logits), little endian.
// Every fed token is decoded in order from a reset state; the run passes when
// the argmax matches at every step and the step-0 logits are within 5e-2
// (max |d|) of the file's, the reference testbench's criteria.  Exit code 0
// on PASS, 1 on FAIL or an engine error, 2 on a usage / input error.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <string>
#include <vector>

#include "qh_decode.h"

int main(int argc, char** argv) {
  std::vector<const char*> pos;
  int mode = QH_MODE_W8A16;
  bool persistent = false;
  for (int i = 1; i < argc; ++i) {
    if (std::strcmp(argv[i], "--w8a8") == 0)
      mode = QH_MODE_W8A8;
    else if (std::strcmp(argv[i], "--persistent") == 0)
      persistent = true;
    else if (argv[i][0] == '-' && argv[i][1] == '-') {
      std::fprintf(stderr, "usage: qh_tb_decode [<blob> [<weights.idx|-> [<decode_ref.bin>]]] [--w8a8] [--persistent]\n");
      return 2;
    } else
      pos.push_back(argv[i]);
  }
  const char* blob = pos.size() > 0 ? pos[0] : "artifacts/qwen35_int8.bin";
  const char* idx = pos.size() > 1 ? pos[1] : "artifacts/weights.idx";
  if (std::strcmp(idx, "-") == 0) idx = nullptr;
  const char* refp = pos.size() > 2 ? pos[2] : "artifacts/decode_ref.bin";

  std::ifstream rf(refp, std::ios::binary);
  if (!rf) {
    std::fprintf(stderr, "open %s failed -- run scripts/export_decode_ref.py first\n", refp);
    return 2;
  }
  int32_t n = 0;
  rf.read(reinterpret_cast<char*>(&n), 4);
  if (!rf || n <= 0 || n > (1 << 24)) {
    std::fprintf(stderr, "%s: bad step count\n", refp);
    return 2;
  }
  std::vector<int32_t> fed(n), am_ref(n);
  std::vector<float> logits0_ref(QH_VOCAB);
  rf.read(reinterpret_cast<char*>(fed.data()), 4L * n);
  rf.read(reinterpret_cast<char*>(am_ref.data()), 4L * n);
  rf.read(reinterpret_cast<char*>(logits0_ref.data()), 4L * QH_VOCAB);
  if (!rf) {
    std::fprintf(stderr, "%s: truncated (need 4 + 8 n + 4 * %d bytes)\n", refp, QH_VOCAB);
    return 2;
  }
  rf.peek();
  if (!rf.eof()) {
    std::fprintf(stderr, "%s: trailing bytes after the step-0 logits\n", refp);
    return 2;
  }

  qh_engine* e = nullptr;
  int st = qh_engine_create(blob, idx, n, &e);
  if (st != QH_OK) {
    std::fprintf(stderr, "engine: %s\n", qh_strerror(st));
    return st == QH_EIO || st == QH_EFORMAT ? 2 : 1;
  }
  qh_engine_set_mode(e, mode);
  if (persistent && qh_engine_set_exec(e, QH_EXEC_PERSISTENT) != QH_OK)
    std::fprintf(stderr, "persistent executor unavailable; using the graph executor\n");
  std::printf("blob %s, %d steps, %s\n", blob, n, mode == QH_MODE_W8A8 ? "W8A8" : "W8A16");

  std::vector<float> logits0(QH_VOCAB);
  std::printf("\n%4s %8s %9s %9s %s\n", "step", "tok", "mi355x", "golden", "");
  std::printf("---------------------------------------------\n");
  int mism = 0;
  for (int i = 0; i < n; ++i) {
    int am = -1;
    st = qh_decode_token(e, fed[i], i == 0 ? logits0.data() : nullptr, &am);
    if (st != QH_OK) {
      std::fprintf(stderr, "decode step %d: %s\n", i, qh_strerror(st));
      qh_engine_destroy(e);
      return 1;
    }
    const bool ok = am == am_ref[i];
    if (!ok) ++mism;
    std::printf("%4d %8d %9d %9d %s\n", i, fed[i], am, am_ref[i], ok ? "ok" : "MISMATCH");
  }
  std::printf("---------------------------------------------\n");
  double maxabs = 0.0, sabs = 0.0;
  for (int v = 0; v < QH_VOCAB; ++v) {
    const double d = std::fabs((double)logits0[v] - (double)logits0_ref[v]);
    maxabs = d > maxabs ? d : maxabs;
    sabs += d;
  }
  std::printf("step-0 logits: max|d| %.3e  mean|d| %.3e  (vs decode_ref)\n", maxabs, sabs / QH_VOCAB);
  const bool pass = mism == 0 && maxabs < 5e-2;
  std::printf("\n%s  (%d/%d steps match)\n", pass ? "PASS - MI355X decode == golden" : "FAIL", n - mism, n);
  qh_engine_destroy(e);
  return pass ? 0 : 1;
}
