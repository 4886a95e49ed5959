// run_hls drop-in on the MI355X engine (reference CLI: hls/tb/run_hls.cpp:37-79).
//
//   qh_run_hls <bin> <ids.txt> <n_new> [eos] [--w8a8] [--graph] [--idx weights.idx]
//
// Tokens run in the persistent kernel (one launch for the prompt, one for the
// generation) unless --graph asks for a graph launch per token or the device
// refuses cooperative launches; both give the same ids.
// Greedy generation from the packed int8 blob: the prompt ids are fed through
// the recurrent path, then up to n_new ids are generated, stopping before eos.
// Generated ids go to stdout (space separated), timing to stderr.  Exit code 2
// on a usage / input error, 1 on an engine error.
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <vector>

#include "qh_decode.h"

int main(int argc, char** argv) {
  std::vector<const char*> pos;
  const char* idx = nullptr;
  int mode = QH_MODE_W8A16;
  bool graph = false;
  for (int i = 1; i < argc; ++i) {
    if (std::strcmp(argv[i], "--w8a8") == 0) {
      mode = QH_MODE_W8A8;
    } else if (std::strcmp(argv[i], "--graph") == 0) {
      graph = true;
    } else if (std::strcmp(argv[i], "--idx") == 0 && i + 1 < argc) {
      idx = argv[++i];
    } else {
      pos.push_back(argv[i]);
    }
  }
  if (pos.size() < 3) {
    std::fprintf(stderr, "usage: qh_run_hls <bin> <ids.txt> <n_new> [eos] [--w8a8] [--graph] [--idx weights.idx]\n");
    return 2;
  }
  const int n_new = std::atoi(pos[2]);
  const int eos = pos.size() > 3 ? std::atoi(pos[3]) : -1;
  std::vector<int> prompt;
  {
    std::ifstream f(pos[1]);
    int t;
    while (f >> t) prompt.push_back(t);
  }
  if (prompt.empty()) {
    std::fprintf(stderr, "no prompt ids\n");
    return 2;
  }
  if (n_new < 0) {
    std::fprintf(stderr, "n_new must be >= 0\n");
    return 2;
  }
  qh_engine* e = nullptr;
  int st = qh_engine_create(pos[0], idx, (int)prompt.size() + n_new + 1, &e);
  if (st != QH_OK) {
    std::fprintf(stderr, "engine: %s\n", qh_strerror(st));
    return st == QH_EIO || st == QH_EFORMAT ? 2 : 1;
  }
  qh_engine_set_mode(e, mode);
  if (!graph) (void)qh_engine_set_exec(e, QH_EXEC_PERSISTENT);   // QH_ESTATE: no cooperative launch
  using clk = std::chrono::steady_clock;
  auto ms = [](clk::time_point a, clk::time_point b) {
    return std::chrono::duration<double, std::milli>(b - a).count();
  };
  int n_out = 0;
  std::vector<int> gen;
  const auto t0 = clk::now();
  st = qh_generate(e, prompt.data(), (int)prompt.size(), 0, eos, nullptr, &n_out);   // prefill
  const auto t1 = clk::now();
  if (st == QH_OK && n_new > 0) {
    const int cur = qh_engine_last_argmax(e);
    if (cur != eos) {   // run_hls.cpp:61-65: push cur, feed it, repeat
      gen.push_back(cur);
      std::vector<int> rest(n_new);
      st = qh_generate(e, &cur, 1, n_new - 1, eos, rest.data(), &n_out);
      for (int i = 0; i < n_out; ++i) gen.push_back(rest[i]);
    }
  }
  const auto t2 = clk::now();
  if (st != QH_OK) {
    std::fprintf(stderr, "engine: %s\n", qh_strerror(st));
    qh_engine_destroy(e);
    return 1;
  }
  for (size_t i = 0; i < gen.size(); ++i) std::printf("%d%s", gen[i], i + 1 < gen.size() ? " " : "\n");
  const double pf = ms(t0, t1), dc = ms(t1, t2);
  std::fprintf(stderr,
               "[mi355x] prefill %zu tok %.1f ms (%.1f tok/s) | decode %zu tok %.1f ms (%.1f tok/s) | %s\n",
               prompt.size(), pf, prompt.size() / (pf / 1000.0), gen.size(), dc,
               gen.empty() ? 0.0 : gen.size() / (dc / 1000.0),
               qh_engine_get_exec(e) == QH_EXEC_PERSISTENT ? "persistent kernel" : "graph per token");
  qh_engine_destroy(e);
  return 0;
}
