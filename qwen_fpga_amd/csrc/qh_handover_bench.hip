// qh_handover_bench: the cost of the persistent kernel's hand-over between
// workgroups on this GPU, measured in isolation (no weights, no arithmetic).
//
//   qwen_fpga_amd/bin/qh_handover_bench [rounds]
//
// 1. ping-pong: two workgroups alternately store a 32-bit tag with a
//    device-coherent store (sc1) and poll the other's with device-coherent loads
//    -- the one-way latency of a hand-over between two workgroups, on one XCD
//    and across XCDs (workgroup b runs on XCD b % 8; checked with HW_REG_XCC_ID).
// 2. all-to-all: G workgroups each publish 1024 / G of a 1024-value vector as
//    8-byte {value, tag} pairs (the TagIO layout of qh_stages.hpp: one 64-bit
//    store per pair) and every workgroup waits until it holds all 1024 current
//    pairs, its W waves polling a share each; then a workgroup barrier, and the
//    next round uses the next tag.  Reports microseconds per round, the
//    hand-over floor of one decode stage (126 such exchanges per token).
//
// Every wait has a poll limit; a run that hits it prints ABORT and exits.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

namespace {

typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
constexpr int kSc1 = 16;   // device-coherent: bypasses the non-coherent L1 (sc1)
constexpr unsigned kLimit = 1u << 22;

#define CHECK(x)                                                                      \
  do {                                                                                \
    hipError_t e_ = (x);                                                              \
    if (e_ != hipSuccess) {                                                           \
      std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
      std::exit(1);                                                                   \
    }                                                                                 \
  } while (0)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7ffffff0, 0x00020000);
}
__device__ __forceinline__ unsigned xcc_id() {
  unsigned v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xf;
}

__global__ void xcc_map(unsigned* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

// Workgroups 0 and `peer`, one lane each; every other workgroup exits at once.
__global__ void pingpong(uint32_t* flags, int iters, int peer, unsigned long long* ticks, int* abort_flag) {
  const int b = blockIdx.x;
  if (threadIdx.x != 0 || (b != 0 && b != peer)) return;
  const auto rs = rsrc(flags);
  const int mine = b == 0 ? 0 : 64, theirs = b == 0 ? 64 : 0;   // separate 256-byte lines
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  for (int i = 1; i <= iters; ++i) {
    if (b == 0) __builtin_amdgcn_raw_buffer_store_b32((uint32_t)i, rs, mine * 4, 0, kSc1);
    unsigned p = 0;
    while (true) {
      asm volatile("" ::: "memory");   // a new load every iteration
      if (__builtin_amdgcn_raw_buffer_load_b32(rs, theirs * 4, 0, kSc1) == (uint32_t)i) break;
      if (++p > kLimit) {
        *abort_flag = 1;
        return;
      }
    }
    if (b != 0) __builtin_amdgcn_raw_buffer_store_b32((uint32_t)i, rs, mine * 4, 0, kSc1);
  }
  if (b == 0) ticks[0] = __builtin_amdgcn_s_memrealtime() - t0;
}

// All-to-all of N pairs (N a multiple of 128 and of G) among the workgroups
// with member[b] >= 0 (G of them).
__global__ void all_to_all(u32x2* vec, const int* member, int G, int N, int rounds, int* abort_flag,
                           unsigned long long* ticks) {
  const int b = blockIdx.x, t = threadIdx.x, lane = t & 63, W = blockDim.x >> 6;
  const int m = member[b];
  if (m < 0) return;
  const int per = N / G;   // pairs published by each member
  const auto rs = rsrc(vec);
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  for (int r = 1; r <= rounds; ++r) {
    const int buf = (r & 1) * N;   // two buffers: a round's pairs are not overwritten while read
    for (int e = t; e < per; e += blockDim.x) {
      u32x2 p;
      p[0] = (uint32_t)(m * per + e);
      p[1] = (uint32_t)r;
      __builtin_amdgcn_raw_buffer_store_b64(p, rs, (buf + m * per + e) * 8, 0, kSc1);
    }
    // wave w polls pairs [w * N / W, (w + 1) * N / W), 16 bytes (two pairs) per lane per load
    const int lo = (t >> 6) * (N / W), n = N / W;
    unsigned p = 0;
    while (true) {
      asm volatile("" ::: "memory");   // a new load every iteration
      bool ok = true;
      for (int i = 2 * lane; i < n; i += 128) {
        const u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(rs, (buf + lo + i) * 8, 0, kSc1);
        ok = ok & (u[1] == (uint32_t)r) & (u[3] == (uint32_t)r);
      }
      if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
      if (++p > kLimit) {
        __hip_atomic_store(abort_flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      if ((p & 255u) == 0 && __hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
    }
    __syncthreads();
    if (__hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return;
  }
  if (t == 0) ticks[b] = __builtin_amdgcn_s_memrealtime() - t0;
}


// Two-level all-to-all of 1024 pairs over all 256 workgroups, grouped into 8
// groups of 32 (group of workgroup b: b % 8, its XCD, when `by_xcd`; else
// b / 32, a group spread over every XCD).  Level 1: the first F members of a
// group each fetch 1024 / F pairs from the global vector with wave 0 and
// republish them into the group's own copy; level 2: every member's W waves
// poll the group's copy, as in all_to_all.
__global__ void two_level(u32x2* vec, u32x2* grp, int F, int by_xcd, int rounds, int* abort_flag,
                          unsigned long long* ticks) {
  const int b = blockIdx.x, t = threadIdx.x, lane = t & 63, W = blockDim.x >> 6;
  const int g = by_xcd ? (b & 7) : (b >> 5), j = by_xcd ? (b >> 3) : (b & 31);   // group, rank in it
  const auto rs = rsrc(vec), rg = rsrc(grp);
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  bool stop = false;
  for (int r = 1; r <= rounds && !stop; ++r) {
    const int buf = (r & 1) * 1024;
    if (t < 4) {   // publish pairs 4b .. 4b + 3
      u32x2 p;
      p[0] = (uint32_t)(4 * b + t);
      p[1] = (uint32_t)r;
      __builtin_amdgcn_raw_buffer_store_b64(p, rs, (buf + 4 * b + t) * 8, 0, kSc1);
    }
    const int gbase = ((r & 1) * 8 + g) * 1024;
    if (j < F && t < 64) {   // level 1: pairs [j * n1, (j + 1) * n1), two per lane
      const int n1 = 1024 / F;
      const int i = j * n1 + 2 * lane;
      const bool mine = 2 * lane < n1;
      unsigned p = 0;
      u32x4 u;
      while (true) {
        asm volatile("" ::: "memory");
        u = __builtin_amdgcn_raw_buffer_load_b128(rs, (buf + (mine ? i : j * n1)) * 8, 0, kSc1);
        if (__builtin_amdgcn_ballot_w64(mine && (u[1] != (uint32_t)r || u[3] != (uint32_t)r)) == 0) break;
        if (++p > kLimit) {
          __hip_atomic_store(abort_flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        if ((p & 255u) == 0 && __hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
      }
      if (mine) __builtin_amdgcn_raw_buffer_store_b128(u, rg, (gbase + i) * 8, 0, kSc1);
    }
    {   // level 2: wave w polls the group copy's pairs [w * 1024 / W, (w + 1) * 1024 / W)
      const int lo = (t >> 6) * (1024 / W), n = 1024 / W;
      unsigned p = 0;
      while (true) {
        asm volatile("" ::: "memory");
        bool ok = true;
        for (int i = 2 * lane; i < n; i += 128) {
          const u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(rg, (gbase + lo + i) * 8, 0, kSc1);
          ok = ok & (u[1] == (uint32_t)r) & (u[3] == (uint32_t)r);
        }
        if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
        if (++p > kLimit) {
          __hip_atomic_store(abort_flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        if ((p & 255u) == 0 && __hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
      }
    }
    __syncthreads();
    stop = __hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
  }
  if (t == 0) ticks[b] = __builtin_amdgcn_s_memrealtime() - t0;
}


// The all-to-all of 1024 pairs among 256 workgroups of 4 waves (as all_to_all)
// while the waves also stream weights, as a decode GEMV stage does: mode 0 no
// weights; 1: each wave issues 8 KiB of weight loads (8 x 16 bytes per lane),
// then its first poll; 2: its first poll, then the weight loads (the decode
// kernel's order; repolls queue behind the weights); 3: waves 0-1 poll half the
// vector each and waves 2-3 load 16 KiB of weights each (the weight stream kept
// off the polling waves).  The weights are folded into one value per lane once
// the vector is complete (where the dot products would use them); they rotate
// through a buffer larger than the Infinity Cache, so every round reads HBM.
__global__ void a2a_weights(u32x2* vec, const u32x4* wbuf, unsigned wunits, int mode, int rounds, int* abort_flag,
                            unsigned long long* ticks, uint32_t* sink) {
  const int b = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6, nblk = gridDim.x;
  const auto rs = rsrc(vec);
  const bool polls = mode != 3 || wave < 2;
  const int nw = mode == 0 ? 0 : mode == 3 ? (wave < 2 ? 0 : 16) : 8;   // weight loads per lane
  const int np = mode == 3 ? 4 : 2;                                     // poll loads per lane
  const int lo = mode == 3 ? wave * 512 : wave * 256;
  uint32_t acc = 0;
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  bool stop = false;
  for (int r = 1; r <= rounds && !stop; ++r) {
    const int buf = (r & 1) * 1024;
    if (t < 4) {
      u32x2 p;
      p[0] = (uint32_t)(4 * b + t);
      p[1] = (uint32_t)r;
      __builtin_amdgcn_raw_buffer_store_b64(p, rs, (buf + 4 * b + t) * 8, 0, kSc1);
    }
    const unsigned wbase = (unsigned)(((size_t)r * nblk * 4 + b * 4 + wave) * 16 * 64 % wunits);
    u32x4 wv[16];
    u32x4 u[4];
    auto issue_weights = [&]() {
#pragma unroll
      for (int k = 0; k < 16; ++k)
        if (k < nw) wv[k] = wbuf[(wbase + k * 64 + lane) % wunits];
      asm volatile("" ::: "memory");
    };
    auto issue_poll = [&]() {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (k < np) u[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, (buf + lo + 2 * lane + 128 * k) * 8, 0, kSc1);
      asm volatile("" ::: "memory");
    };
    if (mode == 1) issue_weights();
    if (polls) issue_poll();
    if (mode == 2 || mode == 3) issue_weights();
    if (polls) {
      unsigned p = 0;
      while (true) {
        bool ok = true;
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (k < np) ok = ok & (u[k][1] == (uint32_t)r) & (u[k][3] == (uint32_t)r);
        if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
        if (++p > kLimit) {
          __hip_atomic_store(abort_flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        if ((p & 255u) == 0 && __hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
        issue_poll();
      }
    }
#pragma unroll
    for (int k = 0; k < 16; ++k)
      if (k < nw) acc ^= wv[k][0] ^ wv[k][1] ^ wv[k][2] ^ wv[k][3];
    __syncthreads();
    stop = __hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
  }
  if (t == 0) ticks[b] = __builtin_amdgcn_s_memrealtime() - t0;
  sink[b * blockDim.x + t] = acc;
}

}  // namespace

int main(int argc, char** argv) {
  const int rounds = argc > 1 ? std::atoi(argv[1]) : 2000;
  if (rounds < 1 || rounds > 1000000) {
    std::fprintf(stderr, "rounds must be 1 .. 1000000\n");
    return 2;
  }
  int dev = 0, ncu = 0;
  CHECK(hipGetDevice(&dev));
  CHECK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
  const int nblk = ncu < 256 ? ncu : 256;
  unsigned* map;
  CHECK(hipMalloc(&map, sizeof(unsigned) * nblk));
  hipLaunchKernelGGL(xcc_map, dim3(nblk), dim3(64), 0, 0, map);
  CHECK(hipDeviceSynchronize());
  std::vector<unsigned> xcc(nblk);
  CHECK(hipMemcpy(xcc.data(), map, sizeof(unsigned) * nblk, hipMemcpyDeviceToHost));
  int off = 0;
  for (int i = 0; i < nblk; ++i) off += xcc[i] != (unsigned)(i % 8);
  std::printf("workgroups: %d; workgroups not on XCD b %% 8: %d\n", nblk, off);

  uint32_t* flags;
  int* abort_flag;
  unsigned long long* ticks;
  u32x2* vec;
  int* member;
  CHECK(hipMalloc(&flags, 1024));
  CHECK(hipMalloc(&abort_flag, sizeof(int)));
  CHECK(hipMalloc(&ticks, sizeof(unsigned long long) * 256));
  CHECK(hipMalloc(&vec, sizeof(u32x2) * 2 * 4096));
  CHECK(hipMalloc(&member, sizeof(int) * 256));
  auto reset = [&]() {
    CHECK(hipMemset(flags, 0, 1024));
    CHECK(hipMemset(abort_flag, 0, sizeof(int)));
    CHECK(hipMemset(ticks, 0, sizeof(unsigned long long) * 256));
    CHECK(hipMemset(vec, 0, sizeof(u32x2) * 2 * 4096));
    CHECK(hipDeviceSynchronize());
  };
  auto aborted = [&]() {
    int a = 0;
    CHECK(hipMemcpy(&a, abort_flag, sizeof(int), hipMemcpyDeviceToHost));
    return a != 0;
  };
  // s_memrealtime counts at 100 MHz
  const double tick_ns = 10.0;

  for (int peer : {8, 1, 128}) {   // same XCD, neighbouring XCD, far workgroup
    if (peer >= nblk) continue;
    reset();
    hipLaunchKernelGGL(pingpong, dim3(nblk), dim3(64), 0, 0, flags, rounds, peer, ticks, abort_flag);
    CHECK(hipDeviceSynchronize());
    unsigned long long tk = 0;
    CHECK(hipMemcpy(&tk, ticks, sizeof tk, hipMemcpyDeviceToHost));
    std::printf("ping-pong workgroup 0 <-> %d (%s XCD): %.1f ns one way%s\n", peer,
                xcc[peer] == xcc[0] ? "same" : "other", tk * tick_ns / (2.0 * rounds), aborted() ? " ABORT" : "");
  }

  struct Case {
    int G, W;
    bool same_xcd;
    int N;
  };
  const Case cases[] = {{256, 1, false, 1024}, {256, 2, false, 1024}, {256, 4, false, 1024}, {256, 8, false, 1024},
                        {64, 4, false, 1024},  {32, 4, false, 1024},  {32, 4, true, 1024},   {8, 4, true, 1024},
                        {2, 4, false, 1024},   {256, 4, false, 512},  {256, 4, false, 2048}, {256, 4, false, 3584},
                        {256, 8, false, 3584}};
  for (const Case& c : cases) {
    if (c.G > nblk) continue;
    std::vector<int> mem(nblk, -1);
    int k = 0;
    for (int b = 0; b < nblk && k < c.G; ++b)
      if (!c.same_xcd || xcc[b] == xcc[0]) mem[b] = k++;
    if (k < c.G) continue;
    CHECK(hipMemcpy(member, mem.data(), sizeof(int) * nblk, hipMemcpyHostToDevice));
    reset();
    hipLaunchKernelGGL(all_to_all, dim3(nblk), dim3(64 * c.W), 0, 0, vec, member, c.G, c.N, rounds, abort_flag,
                       ticks);
    CHECK(hipDeviceSynchronize());
    std::vector<unsigned long long> tk(nblk);
    CHECK(hipMemcpy(tk.data(), ticks, sizeof(unsigned long long) * nblk, hipMemcpyDeviceToHost));
    const unsigned long long mx = *std::max_element(tk.begin(), tk.end());
    std::printf("all-to-all of %4d tagged pairs, G = %3d workgroups (%s), %d poll waves each: %.3f us per round%s\n",
                c.N, c.G, c.same_xcd ? "one XCD" : "all XCDs", c.W, mx * tick_ns / 1000.0 / rounds,
                aborted() ? " ABORT" : "");
    if (aborted()) return 1;
  }
  if (nblk == 256) {
    // the all-to-all with a weight stream beside it
    const unsigned wunits = 32u << 20;   // 512 MiB of 16-byte units
    u32x4* wbuf;
    uint32_t* sink;
    CHECK(hipMalloc(&wbuf, sizeof(u32x4) * (size_t)wunits));
    CHECK(hipMemset(wbuf, 1, sizeof(u32x4) * (size_t)wunits));
    CHECK(hipMalloc(&sink, sizeof(uint32_t) * 256 * 256));
    const char* what[] = {"no weights", "8 KiB of weights per wave before the first poll",
                          "8 KiB of weights per wave after the first poll",
                          "waves 0-1 poll, waves 2-3 load 16 KiB of weights each"};
    for (int mode = 0; mode < 4; ++mode) {
      reset();
      hipLaunchKernelGGL(a2a_weights, dim3(nblk), dim3(256), 0, 0, vec, wbuf, wunits, mode, rounds, abort_flag, ticks,
                         sink);
      CHECK(hipDeviceSynchronize());
      std::vector<unsigned long long> tk(nblk);
      CHECK(hipMemcpy(tk.data(), ticks, sizeof(unsigned long long) * nblk, hipMemcpyDeviceToHost));
      const unsigned long long mx = *std::max_element(tk.begin(), tk.end());
      std::printf("all-to-all of 1024 pairs, 256 workgroups, 4 waves, %s: %.3f us per round%s\n", what[mode],
                  mx * tick_ns / 1000.0 / rounds, aborted() ? " ABORT" : "");
      if (aborted()) return 1;
    }
    u32x2* grp;
    CHECK(hipMalloc(&grp, sizeof(u32x2) * 2 * 8 * 1024));
    struct Case2 {
      int F, by_xcd;
    };
    for (const Case2& c : {Case2{32, 1}, Case2{8, 1}, Case2{32, 0}, Case2{8, 0}}) {
      // A level-1 fetcher is one wave with one 16-byte load (two pairs) per lane, so it
      // covers at most 128 pairs: 1024 / F must not exceed that (and F must divide 1024
      // and fit in a group of 32), or the group copy would never be complete.
      if (c.F < 1 || c.F > 32 || 1024 % c.F != 0 || 1024 / c.F > 128) {
        std::fprintf(stderr, "two-level case with %d fetchers per group is not supported (1024 / F > 128)\n", c.F);
        return 2;
      }
      reset();
      CHECK(hipMemset(grp, 0, sizeof(u32x2) * 2 * 8 * 1024));
      hipLaunchKernelGGL(two_level, dim3(nblk), dim3(256), 0, 0, vec, grp, c.F, c.by_xcd, rounds, abort_flag, ticks);
      CHECK(hipDeviceSynchronize());
      std::vector<unsigned long long> tk(nblk);
      CHECK(hipMemcpy(tk.data(), ticks, sizeof(unsigned long long) * nblk, hipMemcpyDeviceToHost));
      const unsigned long long mx = *std::max_element(tk.begin(), tk.end());
      std::printf("two-level all-to-all, 256 workgroups in 8 groups of 32 (%s), %2d fetchers per group, "
                  "4 poll waves: %.3f us per round%s\n",
                  c.by_xcd ? "one XCD each" : "spread over XCDs", c.F, mx * tick_ns / 1000.0 / rounds,
                  aborted() ? " ABORT" : "");
      if (aborted()) return 1;
    }
  }
  return 0;
}
