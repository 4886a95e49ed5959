// Device bodies of the decode stages, shared by the per-stage kernels
// (qh_kernels.hip: op-level C ABI and the graph engine) and the persistent
// decode kernel (qh_persist.hip).  Each body runs as
//
//   io.arrive()     the per-stage kernels issue the load of the engine's stop flag
//   prefetch        input vector, weights / own state of the first work item in flight
//   io.wait()       the per-stage kernels check the stop flag here
//
// A wave's loads return in issue order, so every load whose value is needed
// first (stop flag, then input vector) is issued before the weights: waiting
// for it then does not wait for the weights.
//   compute         vectors produced by other workgroups are read through the
//                   I/O policy, results are written through it
//
// Two I/O policies:
//   PlainIO  fp32 vectors with device-coherent loads and stores (sc1).  The
//            per-stage kernels use it: kernel boundaries order producers and
//            consumers.
//   TagIO    a vector element i is the 8-byte pair {value bits, tag} at byte
//            8 i, written by one 64-bit store.  A consumer polls the pairs it
//            needs until every tag equals the tag of the producing stage of
//            the current token, so a consumer waits for exactly its inputs and
//            there is no grid-wide barrier.  The persistent kernel uses it.
//
// Work items (row batches, heads, attention splits) are assigned to
// (workgroup, wave) by the same formulas under both policies, and every value
// is produced by the same code, so the two paths are bit-identical.
#pragma once
#include "qh_device.hpp"
#include "qh_kernels.hpp"

namespace qh {

typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

template <int OFF, typename T>
__device__ __forceinline__ T xperm(T v) {
  if constexpr (sizeof(T) == 4 && __is_same(T, float))
    return xor_perm<OFF>(v);
  else
    return xor_perm_i<OFF>(v);
}
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;

// A value loaded before it is needed (epilogue residual): raw bits and tag.
struct Raw {
  uint32_t v = 0, t = 0;
};

__device__ __forceinline__ bool wave_all(bool ok) { return __builtin_amdgcn_ballot_w64(!ok) == 0; }

// Buffer descriptor over n bytes at base; n = 0 makes every access a no-op
// that reads 0, so optional loads can be issued without a branch.  base and n
// must be wave-uniform (scalar registers; see wave_uniform).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_n(const void* base, int n) {
  return __builtin_amdgcn_make_buffer_rsrc(wave_uniform(base), (short)0, __builtin_amdgcn_readfirstlane(n),
                                           0x00020000);
}

// Workgroup copies of handed-over vectors (GEMV inputs, the LM head's h): a
// ring of four 4096-float slots.  A workgroup takes the slots in order, one or
// two per stage, and each copy ends with a workgroup barrier, so a slot is
// rewritten only after every wave has passed two later barriers -- long after
// its last read of the slot's previous contents.
// The per-stage kernels take slots of 4096 floats (op-level K up to 4096); the
// persistent kernel, whose largest staged vector is the 3584-element MLP
// activation, takes slots of 3584 so that the DeltaNet state tiles it keeps in
// LDS fit beside them.  Each kernel allocates only the ring it uses.
constexpr int kLdsSlot = 4096;
constexpr int kTagSlot = 3584;
template <int SLOT>
__device__ __forceinline__ float* lds_ring() {
  __shared__ float ring[4 * SLOT];
  return ring;
}

// Per-wave areas for region polls (pollr_finish): 768 floats (six regions) per wave.
constexpr int kWaveArea = 768;
__device__ __forceinline__ float* wave_area() {
  __shared__ __attribute__((aligned(16))) float a[4 * kWaveArea];
  return a + kWaveArea * (threadIdx.x >> 6);
}

struct PlainIO {
  static constexpr bool kTagged = false;
  const int* done = nullptr;   // engine stop flag (graph engine); null: never stopped
  int ring = 0;                // next LDS slot
  int dv = 0;                  // the stop flag, loaded by arrive()
  __device__ __forceinline__ float* slot() { return lds_ring<kLdsSlot>() + kLdsSlot * (ring++ & 3); }
  __device__ __forceinline__ void mark(int) {}
  // Issued before any weight load of the stage: a wave's loads return in
  // issue order, so waiting for the flag in wait() then waits for this load
  // only.  Without a flag the load goes through an empty descriptor (reads 0).
  __device__ __forceinline__ void arrive() {
    dv = (int)__builtin_amdgcn_raw_buffer_load_b32(rsrc_n(done, done != nullptr ? 4 : 0), 0, 0, kSc1);
  }
  __device__ __forceinline__ bool wait() { return dv == 0; }
  // N chunks of 16 consecutive elements starting at idx[j] (a multiple of 4)
  template <int N>
  __device__ __forceinline__ bool ld16(const float* base, int, const int (&idx)[N], float (&v)[N][16]) {
#pragma unroll
    for (int j = 0; j < N; ++j) ldc16(base, idx[j], v[j]);
    return true;
  }
  template <int N>
  __device__ __forceinline__ bool ldn(const float* base, int, const int (&idx)[N], float (&v)[N]) {
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] = ldcb(base, idx[j]);
    return true;
  }
  __device__ __forceinline__ bool ld1(const float* base, int, int idx, float& v) {
    v = ldcb(base, idx);
    return true;
  }
  __device__ __forceinline__ bool ld1i(const int* base, int, int idx, int& v) {
    v = __float_as_int(ldcb(reinterpret_cast<const float*>(base), idx));
    return true;
  }
  __device__ __forceinline__ Raw issue1(const float* base, int idx, bool valid = true) {
    Raw r;
    r.v = __builtin_amdgcn_raw_buffer_load_b32(rsrc_n(base, valid ? 0x7ffffff0 : 0), idx * 4, 0, kSc1);
    return r;
  }
  __device__ __forceinline__ bool resolve1(const Raw& r, const float*, int, int, float& v) {
    v = __uint_as_float(r.v);
    return true;
  }
  __device__ __forceinline__ void st1(float* base, int, int idx, float v) { stcb(base, idx, v); }
  __device__ __forceinline__ void st1i(int* base, int, int idx, int v) {
    stcb(reinterpret_cast<float*>(base), idx, __int_as_float(v));
  }
  __device__ __forceinline__ void st16(float* base, int, int idx, const float* v) { stc16(base, idx, v); }
  __device__ __forceinline__ void st4(float* base, int, int idx, const float* v) { stc4(base, idx, v); }
  // N 16-element chunks and M single elements, all from one vector
  template <int N, int M>
  __device__ __forceinline__ bool ld16vn(const float* base, int st, const int (&idx)[N], float (&v)[N][16],
                                         const int (&idx1)[M], float (&v1)[M]) {
    ld16<N>(base, st, idx, v);
#pragma unroll
    for (int m = 0; m < M; ++m) v1[m] = ldcb(base, idx1[m]);
    return true;
  }
  template <int N>
  __device__ __forceinline__ bool ld16v(const float* base, int st, const int (&idx)[N], float (&v)[N][16], int idx1,
                                        float& v1) {
    const int i1[1] = {idx1};
    float o1[1];
    const bool ok = ld16vn<N, 1>(base, st, idx, v, i1, o1);
    v1 = o1[0];
    return ok;
  }
  // ld16vn in two steps, so that loads issued in between queue behind it.
  template <int N, int M>
  struct Poll16 {
    float v[N][16];
    float v1[M];
  };
  template <int N, int M>
  __device__ __forceinline__ void poll_issue(const float* base, const int (&idx)[N], const int (&idx1)[M],
                                             Poll16<N, M>& P) {
    ld16vn<N, M>(base, 0, idx, P.v, idx1, P.v1);
  }
  template <int N, int M>
  __device__ __forceinline__ bool poll_finish(const float*, int, const int (&)[N], const int (&)[M], Poll16<N, M>& P,
                                              float (&v)[N][16], float (&v1)[M]) {
#pragma unroll
    for (int j = 0; j < N; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) v[j][e] = P.v[j][e];
#pragma unroll
    for (int m = 0; m < M; ++m) v1[m] = P.v1[m];
    return true;
  }
  // Region poll (see TagIO): lane l reads elements 2l, 2l + 1 of each 128-element region and writes
  // them to dst + 128 r + 2l (LDS, this wave's own area); plus M single elements.
  template <int R, int M>
  struct PollR {
    float v[R][2];
    float v1[M];
  };
  template <int R, int M>
  __device__ __forceinline__ void pollr_issue(const float* base, const int (&rb)[R], const int (&idx1)[M],
                                              PollR<R, M>& P) {
    const int lane = threadIdx.x & 63;
    const __amdgpu_buffer_rsrc_t rs = coh_rsrc(base);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const u32x2 t = __builtin_amdgcn_raw_buffer_load_b64(rs, (rb[r] + 2 * lane) * 4, 0, kSc1);
      P.v[r][0] = __uint_as_float(t[0]);
      P.v[r][1] = __uint_as_float(t[1]);
    }
#pragma unroll
    for (int m = 0; m < M; ++m) P.v1[m] = ldcb(base, idx1[m]);
  }
  template <int R, int M>
  __device__ __forceinline__ bool pollr_finish(const float*, int, const int (&)[R], const int (&)[M], PollR<R, M>& P,
                                               float* dst, float (&v1)[M]) {
    const int lane = threadIdx.x & 63;
    __attribute__((address_space(3))) float* d = (__attribute__((address_space(3))) float*)dst;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      d[128 * r + 2 * lane] = P.v[r][0];
      d[128 * r + 2 * lane + 1] = P.v[r][1];
    }
#pragma unroll
    for (int m = 0; m < M; ++m) v1[m] = P.v1[m];
    return true;
  }
  // A vector the workgroup copied to LDS earlier in this stage program (none here).
  __device__ __forceinline__ const float* cached(const float*, int) const { return nullptr; }
  // Workgroup copy of a vector, in two steps around the stage's weight loads:
  // stage_issue loads elements 4 (t + i blockDim) .. +3 for i < kPL (through a
  // descriptor over exactly K floats, so loads past the end read 0 and K = 0
  // loads nothing); stage_finish writes them to LDS, copies whatever a small
  // workgroup did not cover, and ends with a workgroup barrier.
  static constexpr int kPL = 4;   // 4 x 16 B per thread: K <= 4096 with 256 threads
  struct VecPoll {
    u32x4 u[kPL];
  };
  __device__ __forceinline__ void stage_issue(const float* base, int K, VecPoll& vp) {
    const __amdgpu_buffer_rsrc_t rs = rsrc_n(base, 4 * K);
#pragma unroll
    for (int i = 0; i < kPL; ++i)
      vp.u[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, 16 * ((int)threadIdx.x + i * (int)blockDim.x), 0, kSc1);
  }
  __device__ __forceinline__ bool stage_finish(const float*  base, int, int K, float* lds, VecPoll& vp) {
#pragma unroll
    for (int i = 0; i < kPL; ++i) {
      const int p = 4 * ((int)threadIdx.x + i * (int)blockDim.x);
      if (p < K)
        *reinterpret_cast<float4*>(lds + p) = make_float4(__uint_as_float(vp.u[i][0]), __uint_as_float(vp.u[i][1]),
                                                          __uint_as_float(vp.u[i][2]), __uint_as_float(vp.u[i][3]));
    }
    for (int p = 4 * ((int)threadIdx.x + kPL * (int)blockDim.x); p < K; p += 4 * (int)blockDim.x) {
      float v[4];
      ldc4(base, p, v);
      *reinterpret_cast<float4*>(lds + p) = make_float4(v[0], v[1], v[2], v[3]);
    }
    __syncthreads();
    return true;
  }
  // The whole workgroup copies elements [0, K) (K a multiple of 4) into lds;
  // every thread must call it (it ends with a workgroup barrier).
  __device__ __forceinline__ bool stage_vec(const float* base, int st, int K, float* lds) {
    VecPoll vp;
    stage_issue(base, K, vp);
    return stage_finish(base, st, K, lds, vp);
  }
};

// Polls before a hand-over wait gives up (one poll is a memory round trip,
// roughly a microsecond): about a second, then the launch aborts.
constexpr unsigned kPollLimit = 1u << 20;

// Giving up: a wave whose wait reaches the poll limit (or that sees the abort
// flag another wave set) marks itself failed and FINISHES the wait with the
// stale values it holds, so it still passes every workgroup barrier of the
// stage and takes part in the next stage's descriptor copy.  The persistent
// kernel ORs the failure of all waves of a workgroup through LDS at the next
// stage boundary, and the whole workgroup leaves together.  Stale values can
// reach other workgroups as data but never as an address (the token fed back
// is clamped to the vocabulary); those workgroups give up at their next miss.
struct TagIO {
  static constexpr bool kTagged = true;
  uint32_t tag0 = 0;          // tag of stage 0 of the current token
  int* abort_flag = nullptr;  // global: set by the first wave that gives up
  unsigned poll_limit = kPollLimit;
  bool failed = false;        // this wave gave up a wait (sticky for the launch)
  int ring = 0;               // next LDS slot
  __device__ __forceinline__ float* slot() { return lds_ring<kTagSlot>() + kTagSlot * (ring++ & 3); }
  uint64_t* tr = nullptr;     // optional timing trace of the current stage (points 0..2)
  __device__ __forceinline__ void mark(int p) {
    if (tr != nullptr && tid_here() == 0) tr[p] = __builtin_amdgcn_s_memrealtime();
  }
  __device__ __forceinline__ uint32_t tag(int st) const { return tag0 + (uint32_t)st; }
  __device__ __forceinline__ void arrive() {}
  __device__ __forceinline__ bool wait() { return true; }
  // The persistent kernel's next stage descriptor: each thread's word of it is
  // loaded at the start of a stage (desc_next) and written to its LDS slot at
  // the stage's first tag check (desc_put).  The poll being checked was issued
  // after the descriptor load and a wave's loads return in order, so the write
  // waits for nothing more.  Written at the stage boundary instead, it would
  // wait for every load and store of the stage (the compiler cannot count
  // them across the stage bodies), the stores' acknowledgements included.
  uint32_t dword = 0;
  __attribute__((address_space(3))) uint32_t* ddst = nullptr;   // nullptr: no word for this thread
  bool dpend = false;
  __device__ __forceinline__ void desc_next(const uint32_t* src, uint32_t* slot, int nwords) {
    const int t = threadIdx.x;
    ddst = t < nwords ? as_lds_w(slot + t) : nullptr;
    if (t < nwords) dword = src[t];
    dpend = true;
  }
  __device__ __forceinline__ void desc_put() {
    if (dpend) {
      if (ddst != nullptr) *ddst = dword;
      dpend = false;
    }
  }
  // After a failed poll: false (and the wave marked failed) once the limit is
  // reached or another wave gave up.  A failed wave polls no more.
  __device__ __forceinline__ bool again(unsigned& polls) {
    ++polls;
    if (failed) return false;
    if (polls > poll_limit) {
      stc_i(abort_flag, 1);
      failed = true;
      return false;
    }
    if ((polls & 63u) == 0 && ldc_i(abort_flag) != 0) {
      failed = true;
      return false;
    }
    return true;
  }
  // Phase 1 of every wait: while the producers are still at work a wave polls
  // one pair per lane (512 bytes), so waiting consumers put almost no load on
  // the memory fabric that the producers' weight streams use.
  __device__ __forceinline__ bool sample(const __amdgpu_buffer_rsrc_t& rs, int idx, uint32_t tg, unsigned& polls) {
    while (true) {
      asm volatile("" ::: "memory");
      const u32x2 u = __builtin_amdgcn_raw_buffer_load_b64(rs, idx * 8, 0, kSc1);
      if (wave_all(u[1] == tg)) return true;
      if (!again(polls)) return false;
    }
  }
  // The first load of every wait is checked outside the retry loop, so the
  // compiler can wait for exactly that load (and not for loads issued after it).
  template <int N>
  __device__ __forceinline__ static void issue16(const __amdgpu_buffer_rsrc_t& rs, const int (&idx)[N], u32x4 (&u)[N][8]) {
    asm volatile("" ::: "memory");   // re-issue the loads on every poll
#pragma unroll
    for (int j = 0; j < N; ++j)
#pragma unroll
      for (int k = 0; k < 8; ++k) u[j][k] = __builtin_amdgcn_raw_buffer_load_b128(rs, (idx[j] + 2 * k) * 8, 0, kSc1);
  }
  template <int N>
  __device__ __forceinline__ static bool tags16(const u32x4 (&u)[N][8], uint32_t tg) {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < N; ++j)
#pragma unroll
      for (int k = 0; k < 8; ++k) ok = ok & (u[j][k][1] == tg) & (u[j][k][3] == tg);
    return wave_all(ok);
  }
  template <int N>
  __device__ __forceinline__ bool ld16(const float* base, int st, const int (&idx)[N], float (&v)[N][16]) {
    const uint32_t tg = tag(st);
    const __amdgpu_buffer_rsrc_t rs = coh_rsrc(base);
    u32x4 u[N][8];
    issue16<N>(rs, idx, u);
    const bool hit = tags16<N>(u, tg);
    desc_put();
    if (!hit) {
      unsigned polls = 0;
      do {   // after a miss, wait on one pair per lane before loading everything again
        if (!again(polls) || !sample(rs, idx[N - 1] + 15, tg, polls)) break;   // gave up: stale values
        issue16<N>(rs, idx, u);
      } while (!tags16<N>(u, tg));
    }
#pragma unroll
    for (int j = 0; j < N; ++j)
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        v[j][2 * k] = __uint_as_float(u[j][k][0]);
        v[j][2 * k + 1] = __uint_as_float(u[j][k][2]);
      }
    return true;
  }
  template <int N>
  __device__ __forceinline__ bool ldn(const float* base, int st, const int (&idx)[N], float (&v)[N]) {
    const uint32_t tg = tag(st);
    const __amdgpu_buffer_rsrc_t rs = coh_rsrc(base);
    u32x2 u[N];
    auto issue = [&]() {
      asm volatile("" ::: "memory");
#pragma unroll
      for (int j = 0; j < N; ++j) u[j] = __builtin_amdgcn_raw_buffer_load_b64(rs, idx[j] * 8, 0, kSc1);
    };
    auto tags = [&]() {
      bool ok = true;
#pragma unroll
      for (int j = 0; j < N; ++j) ok = ok & (u[j][1] == tg);
      return wave_all(ok);
    };
    issue();
    const bool hit = tags();
    desc_put();
    if (!hit) {
      unsigned polls = 0;
      do {
        if (!again(polls)) break;   // gave up: stale values
        if (N > 1 && !sample(rs, idx[N - 1], tg, polls)) break;
        issue();
      } while (!tags());
    }
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] = __uint_as_float(u[j][0]);
    return true;
  }
  __device__ __forceinline__ bool ld1(const float* base, int st, int idx, float& v) {
    int i1[1] = {idx};
    float v1[1];
    const bool ok = ldn<1>(base, st, i1, v1);
    v = v1[0];
    return ok;
  }
  __device__ __forceinline__ bool ld1i(const int* base, int st, int idx, int& v) {
    float f;
    const bool ok = ld1(reinterpret_cast<const float*>(base), st, idx, f);
    v = __float_as_int(f);
    return ok;
  }
  __device__ __forceinline__ Raw issue1(const float* base, int idx, bool valid = true) {
    const u32x2 u = __builtin_amdgcn_raw_buffer_load_b64(rsrc_n(base, valid ? 0x7ffffff0 : 0), idx * 8, 0, kSc1);
    Raw r;
    r.v = u[0];
    r.t = u[1];
    return r;
  }
  __device__ __forceinline__ bool resolve1(const Raw& r, const float* base, int st, int idx, float& v) {
    const bool hit = wave_all(r.t == tag(st));
    desc_put();
    if (hit) {
      v = __uint_as_float(r.v);
      return true;
    }
    return ld1(base, st, idx, v);
  }
  __device__ __forceinline__ void st1(float* base, int st, int idx, float v) {
    u32x2 u;
    u[0] = __float_as_uint(v);
    u[1] = tag(st);
    __builtin_amdgcn_raw_buffer_store_b64(u, coh_rsrc(base), idx * 8, 0, kSc1);
  }
  __device__ __forceinline__ void st1i(int* base, int st, int idx, int v) {
    st1(reinterpret_cast<float*>(base), st, idx, __int_as_float(v));
  }
  // N 16-element chunks and M single elements of one vector, polled together.
  // poll_issue makes the first attempt; loads issued after it return after it,
  // so work placed between the two steps overlaps the hand-over wait.
  template <int N, int M>
  struct Poll16 {
    u32x4 u[N][8];
    u32x2 u1[M];
  };
  template <int N, int M>
  __device__ __forceinline__ void poll_issue(const float* base, const int (&idx)[N], const int (&idx1)[M],
                                             Poll16<N, M>& P) {
    const __amdgpu_buffer_rsrc_t rs = coh_rsrc(base);
    issue16<N>(rs, idx, P.u);
#pragma unroll
    for (int m = 0; m < M; ++m) P.u1[m] = __builtin_amdgcn_raw_buffer_load_b64(rs, idx1[m] * 8, 0, kSc1);
    asm volatile("" ::: "memory");   // nothing issued later may move ahead of these loads
  }
  template <int N, int M>
  __device__ __forceinline__ bool poll_finish(const float* base, int st, const int (&idx)[N], const int (&idx1)[M],
                                              Poll16<N, M>& P, float (&v)[N][16], float (&v1)[M]) {
    const uint32_t tg = tag(st);
    auto tags = [&]() {
      bool ok = true;
#pragma unroll
      for (int m = 0; m < M; ++m) ok = ok & (P.u1[m][1] == tg);
      return tags16<N>(P.u, tg) && wave_all(ok);
    };
    const bool hit = tags();
    desc_put();
    mark(3);   // trace: first poll returned
    if (!hit) {
      const __amdgpu_buffer_rsrc_t rs = coh_rsrc(base);
      unsigned polls = 0;
      do {
        if (!again(polls) || !sample(rs, idx1[M - 1], tg, polls)) break;   // gave up: stale values
        poll_issue<N, M>(base, idx, idx1, P);
      } while (!tags());
      mark(4);   // trace: complete after a repoll
    }
#pragma unroll
    for (int j = 0; j < N; ++j)
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        v[j][2 * k] = __uint_as_float(P.u[j][k][0]);
        v[j][2 * k + 1] = __uint_as_float(P.u[j][k][2]);
      }
#pragma unroll
    for (int m = 0; m < M; ++m) v1[m] = __uint_as_float(P.u1[m][0]);
    return true;
  }
  // Region poll: R regions of 128 consecutive pairs (1 KiB each, first pair rb[r]) and M single
  // pairs.  Lane l loads pairs 2l, 2l + 1 of every region with one 16-byte load, so a load
  // instruction covers eight whole lines -- a wave fetches each freshly written line once (the
  // 16-element form touches eight lines per instruction, 16 bytes of each, again and again).  The
  // values go to dst + 128 r + 2l, this wave's own LDS area, for any lane to read back.
  template <int R, int M>
  struct PollR {
    u32x4 u[R];
    u32x2 u1[M];
  };
  template <int R, int M>
  __device__ __forceinline__ void pollr_issue(const float* base, const int (&rb)[R], const int (&idx1)[M],
                                              PollR<R, M>& P) {
    const int lane = threadIdx.x & 63;
    const __amdgpu_buffer_rsrc_t rs = coh_rsrc(base);
    asm volatile("" ::: "memory");
#pragma unroll
    for (int r = 0; r < R; ++r) P.u[r] = __builtin_amdgcn_raw_buffer_load_b128(rs, (rb[r] + 2 * lane) * 8, 0, kSc1);
#pragma unroll
    for (int m = 0; m < M; ++m) P.u1[m] = __builtin_amdgcn_raw_buffer_load_b64(rs, idx1[m] * 8, 0, kSc1);
    asm volatile("" ::: "memory");   // nothing issued later may move ahead of these loads
  }
  template <int R, int M>
  __device__ __forceinline__ bool pollr_finish(const float* base, int st, const int (&rb)[R], const int (&idx1)[M],
                                               PollR<R, M>& P, float* dst, float (&v1)[M]) {
    const uint32_t tg = tag(st);
    auto tags = [&]() {
      bool ok = true;
#pragma unroll
      for (int r = 0; r < R; ++r) ok = ok & (P.u[r][1] == tg) & (P.u[r][3] == tg);
#pragma unroll
      for (int m = 0; m < M; ++m) ok = ok & (P.u1[m][1] == tg);
      return wave_all(ok);
    };
    const bool hit = tags();
    desc_put();
    mark(3);   // trace: first poll returned
    if (!hit) {
      const __amdgpu_buffer_rsrc_t rs = coh_rsrc(base);
      unsigned polls = 0;
      do {
        if (!again(polls) || !sample(rs, idx1[M - 1], tg, polls)) break;   // gave up: stale values
        pollr_issue<R, M>(base, rb, idx1, P);
      } while (!tags());
      mark(4);   // trace: complete after a repoll
    }
    const int lane = threadIdx.x & 63;
    __attribute__((address_space(3))) float* d = (__attribute__((address_space(3))) float*)dst;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      d[128 * r + 2 * lane] = __uint_as_float(P.u[r][0]);
      d[128 * r + 2 * lane + 1] = __uint_as_float(P.u[r][2]);
    }
#pragma unroll
    for (int m = 0; m < M; ++m) v1[m] = __uint_as_float(P.u1[m][0]);
    return true;
  }
  template <int N, int M>
  __device__ __forceinline__ bool ld16vn(const float* base, int st, const int (&idx)[N], float (&v)[N][16],
                                         const int (&idx1)[M], float (&v1)[M]) {
    Poll16<N, M> P;
    poll_issue<N, M>(base, idx, idx1, P);
    return poll_finish<N, M>(base, st, idx, idx1, P, v, v1);
  }
  template <int N>
  __device__ __forceinline__ bool ld16v(const float* base, int st, const int (&idx)[N], float (&v)[N][16], int idx1,
                                        float& v1) {
    const int i1[1] = {idx1};
    float o1[1];
    const bool ok = ld16vn<N, 1>(base, st, idx, v, i1, o1);
    v1 = o1[0];
    return ok;
  }
  // The last vector this workgroup copied to LDS (stage_finish), if it is (base, st).
  const float* last_base = nullptr;
  int last_st = -1;
  const float* last_lds = nullptr;
  __device__ __forceinline__ const float* cached(const float* base, int st) const {
    return (base == last_base && st == last_st) ? last_lds : nullptr;
  }
  // First poll of a workgroup copy, issued before the stage's weight loads so
  // that its result does not queue behind them (loads return in order).
  static constexpr int kL = 4096 / (2 * kPersistThreads);   // b128 loads per thread
  struct VecPoll {
    u32x4 u[kL];
  };
  // K = 0 issues no memory access (empty descriptor).
  __device__ __forceinline__ void stage_issue(const float* base, int K, VecPoll& vp) {
    const __amdgpu_buffer_rsrc_t rs = rsrc_n(base, 8 * K);
    const int t = threadIdx.x;
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < kL; ++i) {
      const int p = min(2 * t + 2 * kPersistThreads * i, max(K - 2, 0));
      vp.u[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, p * 8, 0, kSc1);
    }
    asm volatile("" ::: "memory");   // nothing issued later may move ahead of these loads
  }
  __device__ __forceinline__ bool stage_vec(const float* base, int st, int K, float* lds) {
    VecPoll vp;
    stage_issue(base, K, vp);
    return stage_finish(base, st, K, lds, vp);
  }
  // The whole workgroup (kPersistThreads threads) copies elements [0, K) of a
  // tagged vector into lds as fp32, K <= kTagSlot and even: each thread checks the
  // tags of its pairs (first loads issued by stage_issue); after a miss every
  // wave polls 64 samples spread over the vector before loading its pairs
  // again.  Ends with a barrier.
  __device__ __forceinline__ static bool vec_tags(const VecPoll& vp, int K, uint32_t tg) {
    // t < kPersistThreads (the persistent kernel's workgroup size): with the
    // range stated, the bounds tests fold for K a multiple of 512 instead of
    // becoming lane masks that the compiler holds across the stage loop
    const int t = threadIdx.x & (kPersistThreads - 1);
    bool ok = true;
#pragma unroll
    for (int i = 0; i < kL; ++i) {
      const bool in = 2 * t + 2 * kPersistThreads * i < K;   // clamped duplicates are checked too: harmless
      ok = ok & (!in | ((vp.u[i][1] == tg) & (vp.u[i][3] == tg)));
    }
    return wave_all(ok);
  }
  __device__ __forceinline__ bool stage_finish(const float* base, int st, int K, float* lds, VecPoll& vp) {
    const uint32_t tg = tag(st);
    const int t = threadIdx.x, lane = t & 63;
    const bool hit = vec_tags(vp, K, tg);
    desc_put();
    mark(3);   // trace: first poll returned
    if (!hit) {
      const __amdgpu_buffer_rsrc_t rs = coh_rsrc(base);
      // 16 sampled lines per wave (lanes in groups of 4 share one), rotated per
      // workgroup so that the waiting workgroups spread their polls over the
      // whole vector instead of hammering the same few lines.
      const unsigned k2 = (unsigned)K >> 1;   // 16-byte units
      const unsigned sidx = (((unsigned)(lane >> 2) * k2) / 16u + 7u * (unsigned)blockIdx.x) % k2;
      unsigned polls = 0;
      do {
        if (!again(polls) || !sample(rs, (int)(2 * sidx + 1), tg, polls)) break;   // gave up: stale values
        stage_issue(base, K, vp);
      } while (!vec_tags(vp, K, tg));
      mark(4);   // trace: vector complete after a repoll
    }
    const int tt = t & (kPersistThreads - 1);   // the same range statement as in vec_tags
#pragma unroll
    for (int i = 0; i < kL; ++i) {
      const int p = 2 * tt + 2 * kPersistThreads * i;
      if (p < K) *reinterpret_cast<float2*>(lds + p) = make_float2(__uint_as_float(vp.u[i][0]), __uint_as_float(vp.u[i][2]));
    }
    __syncthreads();
    last_base = base;
    last_st = st;
    last_lds = lds;
    return true;
  }
  // base[idx .. idx + 3], idx even: two (value, tag) pairs per 16-byte store
  __device__ __forceinline__ void st4(float* base, int st, int idx, const float* v) {
    const uint32_t tg = tag(st);
    const __amdgpu_buffer_rsrc_t rs = coh_rsrc(base);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      u32x4 u;
      u[0] = __float_as_uint(v[2 * k]);
      u[1] = tg;
      u[2] = __float_as_uint(v[2 * k + 1]);
      u[3] = tg;
      __builtin_amdgcn_raw_buffer_store_b128(u, rs, (idx + 2 * k) * 8, 0, kSc1);
    }
  }
  __device__ __forceinline__ void st16(float* base, int st, int idx, const float* v) {
    const uint32_t tg = tag(st);
    const __amdgpu_buffer_rsrc_t rs = coh_rsrc(base);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      u32x4 u;
      u[0] = __float_as_uint(v[2 * k]);
      u[1] = tg;
      u[2] = __float_as_uint(v[2 * k + 1]);
      u[3] = tg;
      __builtin_amdgcn_raw_buffer_store_b128(u, rs, (idx + 2 * k) * 8, 0, kSc1);
    }
  }
};

// ===========================================================================
// GEMV: y = W x over up to four row segments sharing one activation vector.
// A wave owns batches of R rows (R = 1, 2, 4 or 8); lane l holds the
// 16-element chunks c = l + 64j of x in registers and streams the same chunks
// of each row with one 16-byte load per chunk (a row of 1024 int8 is one
// coalesced 1 KiB read across the wave).  After the lane partials, the R rows
// are folded by a transposed xor butterfly: at offsets 32, 16, 8 each lane
// keeps half of its rows and receives its partner's other half, then the
// remaining offsets finish the tree.  Lane l ends with row (l >> (6 - log2 R))
// & (R - 1).  Per row this is exactly the 64-lane xor tree of the C16 order,
// whatever R is (IEEE addition is commutative).
// ===========================================================================
template <typename T>
__device__ __forceinline__ T reduce8(T v[8], int lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = swap_add<32>(v[i], v[i + 4]);   // lanes with bit 32 keep v[i + 4]
#pragma unroll
  for (int i = 0; i < 2; ++i) v[i] = swap_add<16>(v[i], v[i + 2]);   // lanes with bit 16 keep v[i + 2]
  {
    const bool up = (lane & 8) != 0;
    const T send = up ? v[0] : v[1];
    const T keep = up ? v[1] : v[0];
    v[0] = keep + xperm<8>(send);
  }
  T r = v[0];
  r = r + xperm<4>(r);
  r = r + xperm<2>(r);
  r = r + xperm<1>(r);
  return r;
}

template <typename T>
__device__ __forceinline__ T reduce4(T v[4], int) {
#pragma unroll
  for (int i = 0; i < 2; ++i) v[i] = swap_add<32>(v[i], v[i + 2]);
  v[0] = swap_add<16>(v[0], v[1]);
  T r = v[0];
  r = r + xperm<8>(r);
  r = r + xperm<4>(r);
  r = r + xperm<2>(r);
  r = r + xperm<1>(r);
  return r;
}

template <typename T>
__device__ __forceinline__ T reduce1(T v[1], int) {
  T r = swap_add<32>(v[0], v[0]);
  r = swap_add<16>(r, r);
  r = r + xperm<8>(r);
  r = r + xperm<4>(r);
  r = r + xperm<2>(r);
  r = r + xperm<1>(r);
  return r;
}

template <int R, typename T>
__device__ __forceinline__ T reduce_rows(T v[R], int lane) {
  if constexpr (R == 8)
    return reduce8(v, lane);
  else if constexpr (R == 4)
    return reduce4(v, lane);
  else {
    // (two rows go through reduce4 with two zero rows: a two-row tree built on
    // the permlane swaps gave wrong sums for its second row)
    static_assert(R == 1, "rows per wave: 1, 4 or 8");
    return reduce1(v, lane);
  }
}
template <int R>
__device__ __forceinline__ int row_of_lane(int lane) {
  static_assert(R == 1 || R == 4 || R == 8, "rows per wave: 1, 4 or 8");
  return R == 1 ? 0 : (lane >> (R == 8 ? 3 : 4)) & (R - 1);
}

// 16 floats from global memory (load16g) or LDS (load16l), 16-byte aligned
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void load16g(const float* p, float* v) {
  const __attribute__((address_space(1))) f32x4* q = as_global(reinterpret_cast<const f32x4*>(p));
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const f32x4 t = q[k];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[4 * k + e] = t[e];
  }
}
__device__ __forceinline__ void load16l(const float* p, float* v) {
  const __attribute__((address_space(3))) f32x4* q = as_lds(reinterpret_cast<const f32x4*>(p));
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const f32x4 t = q[k];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[4 * k + e] = t[e];
  }
}
// Lane l's 16-element chunk of a 1024-element fp32 row stored lane-interleaved
// (element e at (e / 4) * 256 + 4 l + e % 4): each of the four loads of a wave
// reads 1 KiB of consecutive memory.
__device__ __forceinline__ void load16c(const float* row, int l, float* v) {
  const __attribute__((address_space(1))) f32x4* q = as_global(reinterpret_cast<const f32x4*>(row));
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const f32x4 t = q[64 * k + l];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[4 * k + e] = t[e];
  }
}
// load16c through a buffer descriptor (an empty one reads zeros); row_f: float offset of the row
__device__ __forceinline__ void load16c_rs(const __amdgpu_buffer_rsrc_t& rs, int row_f, int l, float* v) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(rs, (row_f + 256 * k + 4 * l) * 4, 0, 0);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[4 * k + e] = __uint_as_float(t[e]);
  }
}
// 16 int8 from global memory
__device__ __forceinline__ void load16b(const int8_t* p, uint32_t* w) {
  const u32x4 t = *as_global(reinterpret_cast<const u32x4*>(p));
#pragma unroll
  for (int e = 0; e < 4; ++e) w[e] = t[e];
}
__device__ __forceinline__ float i8_at(const uint32_t* w, int e) {
  return (float)(int)(int8_t)(w[e >> 2] >> (8 * (e & 3)));
}

// Whether epilogue / segment-kind bit `bit` is possible in a GEMV compiled for mask EM.
template <int EM>
__device__ __forceinline__ constexpr bool em_has(int bit) {
  return EM == 0 || (EM & bit) != 0;
}

// Per-row epilogue inputs, loaded by every lane for its row at batch start.
struct EpiAux {
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;   // residual | conv state cols 1..3 | A_log
  float w0 = 0.0f, w1 = 0.0f, w2 = 0.0f, w3 = 0.0f;   // conv taps | dt_bias
  float sc = 1.0f;                                     // the row's weight scale (int8 segments)
  Raw res;                                             // E_RESID: residual, resolved before use
};
// every input epi_prefetch loaded, read or not by the segment's epilogue
__device__ __forceinline__ void settle_aux(const EpiAux& x) {
  settle(x.a0), settle(x.a1), settle(x.a2), settle(x.a3);
  settle(x.w0), settle(x.w1), settle(x.w2), settle(x.w3);
  settle(x.sc), settle(x.res.v), settle(x.res.t);
}
// Every input an epilogue may need, loaded without a branch: inputs the
// segment's epilogue does not use come from zero-size descriptors (no memory
// access), so the load block stays straight-line and the compiler can count
// outstanding loads exactly.
template <int EM, class IO>
__device__ __forceinline__ void epi_prefetch(const Seg& g, int myrow, EpiAux& x, IO& io) {
  constexpr int kBig = 0x7ffffff0;
  const int r = min(myrow, g.rows - 1);   // always a valid address; unused rows are never stored
  const bool pair = em_has<EM>(kEmPair) && g.kind == SEG_PAIR;
  const bool f32 = em_has<EM>(kEmF32) && g.kind == SEG_F32;
  // the row's scale: lanes of a pair segment take even rows (gate) from sw and
  // odd rows (up) from sw2, so both are loaded through uniform descriptors
  const int i8n = (f32 || g.sw == nullptr) ? 0 : kBig;   // no scales: E_ACCI
  const int si = (pair ? (r >> 1) : r) * 4;
  const float sa = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsrc_n(g.sw, i8n), si, 0, 0));
  float sb = 0.0f;
  if constexpr (em_has<EM>(kEmPair))
    sb = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsrc_n(g.sw2, pair ? kBig : 0), si, 0, 0));
  x.sc = f32 ? 1.0f : ((pair && (r & 1)) ? sb : sa);
  if constexpr (em_has<EM>(1 << E_RESID))
    x.res = io.issue1(g.res, r, g.epi == E_RESID);   // residual: written by another workgroup
  if constexpr (em_has<EM>(1 << E_GATE_A)) {
    const bool ga = g.epi == E_GATE_A;
    x.a0 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsrc_n(g.c0, ga ? kBig : 0), r * 4, 0, 0));
    x.w0 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsrc_n(g.c1, ga ? kBig : 0), r * 4, 0, 0));
  }
  if constexpr (em_has<EM>(1 << E_CONV)) {
    const bool cv = g.epi == E_CONV;
    const u32x4 st = __builtin_amdgcn_raw_buffer_load_b128(rsrc_n(g.c2, cv ? kBig : 0), r * 16, 0, 0);
    const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rsrc_n(g.c0, cv ? kBig : 0), r * 16, 0, 0);
    if (cv) x.w0 = __uint_as_float(w[0]);   // (E_GATE_A keeps dt_bias in w0)
    x.a1 = __uint_as_float(st[1]);
    x.a2 = __uint_as_float(st[2]);
    x.a3 = __uint_as_float(st[3]);
    x.w1 = __uint_as_float(w[1]);
    x.w2 = __uint_as_float(w[2]);
    x.w3 = __uint_as_float(w[3]);
  }
}

// Row-batch epilogue: the writer lane of each row stores its result y.
template <int R, int EM, class IO>
__device__ __forceinline__ void gemv_epilogue(const Seg& g, int ost, int lane, int myrow, float y, int acci,
                                              const EpiAux& x, IO& io) {
  constexpr int LPR = 64 / R;   // lanes holding one row
  if constexpr (R >= 2 && em_has<EM>(1 << E_SWIGLU)) {
    if (g.epi == E_SWIGLU) {      // pair rows: even = gate i, odd = up i (mlp.hpp:17)
      const float yo = xperm<LPR>(y);
      if ((lane & (2 * LPR - 1)) == 0 && myrow < g.rows) io.st1(g.out, ost, myrow >> 1, dev_silu(y) * yo);
      return;
    }
  }
  if ((lane & (LPR - 1)) != 0 || myrow >= g.rows) return;
  if constexpr (EM == kEmResid) {   // the only epilogue of the 2x1 / 4x1 kinds
    io.st1(g.out, ost, myrow, x.a0 + y);
    return;
  }
  if constexpr (EM == kEmStore) {
    io.st1(g.out, ost, myrow, y);
    return;
  }
  const int epi = g.epi;
  if (em_has<EM>(1 << E_STORE) && epi == E_STORE) {
    io.st1(g.out, ost, myrow, y);
  } else if (em_has<EM>(1 << E_SILU) && epi == E_SILU) {   // silu(z) for the gated norm (norm.hpp:32)
    io.st1(g.out, ost, myrow, dev_silu(y));
  } else if (em_has<EM>(1 << E_RESID) && epi == E_RESID) {
    io.st1(g.out, ost, myrow, x.a0 + y);
  } else if (em_has<EM>(1 << E_ACC) && epi == E_ACC) {
    io.st1(g.out, ost, myrow, y);
    as_global_w(g.acc_out)[myrow] = acci;
  } else if (em_has<EM>(1 << E_ACCI) && epi == E_ACCI) {
    as_global_w(g.acc_out)[myrow] = acci;
  } else if (em_has<EM>(1 << E_GATE_B) && epi == E_GATE_B) {
    io.st1(g.out, ost, myrow, dev_sigmoid(y));
  } else if (em_has<EM>(1 << E_GATE_A) && epi == E_GATE_A) {
    io.st1(g.out, ost, myrow, -dev_expf(x.a0) * dev_softplus(y + x.w0));
  } else if (em_has<EM>(1 << E_CONV) && epi == E_CONV) {   // conv1d.hpp:22-36: window = state cols 1..3 + new
    float acc = 0.0f;
    acc = acc + x.a1 * x.w0;
    acc = acc + x.a2 * x.w1;
    acc = acc + x.a3 * x.w2;
    acc = acc + y * x.w3;
    *as_global_w(reinterpret_cast<f32x4*>(g.c2 + (size_t)myrow * 4)) = f32x4{x.a1, x.a2, x.a3, y};
    io.st1(g.out, ost, myrow, dev_silu(acc));
  }
}

// A segment descriptor with every field made wave-uniform (scalar registers):
// the loads, clamps and selects built from it are then scalar instructions, not
// per-lane address arithmetic on the stage's critical path.
__device__ __forceinline__ Seg seg_uniform(const Seg& s) {
  Seg g;
  g.kind = __builtin_amdgcn_readfirstlane(s.kind);
  g.epi = __builtin_amdgcn_readfirstlane(s.epi);
  g.batch0 = __builtin_amdgcn_readfirstlane(s.batch0);
  g.nbatch = __builtin_amdgcn_readfirstlane(s.nbatch);
  g.rows = __builtin_amdgcn_readfirstlane(s.rows);
  g.res_st = __builtin_amdgcn_readfirstlane(s.res_st);
  g.w = static_cast<const int8_t*>(wave_uniform(s.w));
  g.sw = static_cast<const float*>(wave_uniform(s.sw));
  g.wf = static_cast<const float*>(wave_uniform(s.wf));
  g.w2 = static_cast<const int8_t*>(wave_uniform(s.w2));
  g.sw2 = static_cast<const float*>(wave_uniform(s.sw2));
  g.out = static_cast<float*>(wave_uniform(s.out));
  g.acc_out = static_cast<int32_t*>(wave_uniform(s.acc_out));
  g.res = static_cast<const float*>(wave_uniform(s.res));
  g.c0 = static_cast<const float*>(wave_uniform(s.c0));
  g.c1 = static_cast<const float*>(wave_uniform(s.c1));
  g.c2 = static_cast<float*>(wave_uniform(s.c2));
  return g;
}

// Loads of one batch: every address is clamped into the segment (rows) and the
// vector (chunks), so the loads are unconditional and issue back to back.  A
// clamped chunk meets x = 0 (the prologue zeroes chunks beyond K) and a clamped
// row is never stored, so neither changes a result.  An fp32 segment has no
// int8 rows: its descriptors are empty and the loads read nothing.  g and row0
// are wave-uniform: a row's byte offset goes in the scalar offset of the
// buffer load, and only the lane's chunk offset is per lane.
// Cache policy of a GEMV stage's weight loads (EM: the stage kind's epilogue
// set).  The gate/up weights (176 MB over the 24 layers) and the attention
// q, k, v weights (31 MB) load with the default policy, so they stay in the
// 256 MB Infinity Cache from one token to the next.  Every other weight byte
// (in_proj, the 1024-row projections and, in the persistent kernel, the LM
// head: 545 MB, each read once per token) loads non-temporally so that it does
// not evict them.  More than that does not fit: adding in_proj (327 MB cached)
// or half the head (334 MB) made the decode slower than caching less.
template <int EM>
constexpr int weight_policy() {
  return (EM == kEmSwiglu || EM == kEmStore) ? 0 : kNt;
}

template <int NCH, int R, int EM>
__device__ __forceinline__ void load_batch(const Seg& g, int row0, int K, int nchunk, int lane,
                                           uint32_t (&w)[NCH][R][4]) {
  const bool pair = em_has<EM>(kEmPair) && g.kind == SEG_PAIR;
  const int n = (em_has<EM>(kEmF32) && g.kind == SEG_F32) ? 0 : 0x7ffffff0;
  const int last = g.rows - 1;
  const __amdgpu_buffer_rsrc_t rw = rsrc_n(g.w, n);
  const __amdgpu_buffer_rsrc_t rw2 = rsrc_n(pair ? g.w2 : g.w, n);
  int voff[NCH];
#pragma unroll
  for (int j = 0; j < NCH; ++j) voff[j] = 16 * min(lane + 64 * j, nchunk - 1);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = __builtin_amdgcn_readfirstlane(min(row0 + r, last));   // wave-uniform
    const bool second = pair && (row & 1);
    const int roff = __builtin_amdgcn_readfirstlane((pair ? (row >> 1) : row) * K);
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(second ? rw2 : rw, voff[j], roff, weight_policy<EM>());
      w[j][r][0] = t[0];
      w[j][r][1] = t[1];
      w[j][r][2] = t[2];
      w[j][r][3] = t[3];
    }
  }
}

// The quantised activation of a W8A8 GEMV workgroup: [NCH][64 lanes][4 dwords].
__device__ __forceinline__ uint32_t* gemv_qlds() {
  __shared__ __attribute__((aligned(16))) uint32_t q[4 * 64 * 4];
  return q;
}

// KC: the vector length when the caller knows it at compile time (the
// persistent kernel's stage kinds), 0 to take it from the descriptor.
template <int NCH, int MODE, int PRO, int R, int KC = 0, int EM = 0, class IO>
__device__ __forceinline__ bool gemv_body(const GemvArgs& a, int blk, int nblk, IO& io, int tokv) {
  const int lane = threadIdx.x & 63, nwv = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // The descriptor (a workgroup copy in LDS) is read into registers once, in one
  // batch of independent reads.  Read through the reference where it is used,
  // every field after a memory clobber (each poll has one) would be another LDS
  // read, and chains of them (the segment search, a weight row's matrix) are
  // dependent round trips on the stage's critical path.
  const int K = KC != 0 ? KC : __builtin_amdgcn_readfirstlane(a.K);
  const int nseg = a.nseg;
  const float* const ax = a.x;
  const float* const anw = a.nw;
  const int nw_lanes = a.nw_lanes;
  const float* const az = a.z;
  const int8_t* const axq = a.xq;
  const float* const asx = a.sx;
  const float eps = a.eps;
  const int8_t* const aemb = a.emb;
  const float* const aemb_s = a.emb_s;
  const int* const atok = a.tok;
  float* const ah_out = a.h_out;
  const int x_st = a.x_st, z_st = a.z_st, out_st = a.out_st;
  const float* const agw = a.gw;
  const int grows = a.grows;
  const int gblk0 = a.gblk;
  const float* const ag_alog = a.g_alog;
  const float* const ag_dtb = a.g_dtb;
  float* const agout = a.gout;
  int sb0[4], snb[4], skind[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    sb0[i] = a.seg[i].batch0;
    snb[i] = a.seg[i].nbatch;
    skind[i] = a.seg[i].kind;
  }
  const int nchunk = K >> 4;
  int total = 0;
  bool has_f32 = false;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (i < nseg) {
      total = sb0[i] + snb[i];   // segments are in batch order: the last one ends the range
      has_f32 = has_f32 || (em_has<EM>(kEmF32) && skind[i] == SEG_F32);
    }
  total = __builtin_amdgcn_readfirstlane(total);
  has_f32 = __builtin_amdgcn_readfirstlane((int)has_f32) != 0;
  // the segment holding batch bb (segments start at increasing batches)
  auto seg_index = [&](int bb) {
    int si = 0;
#pragma unroll
    for (int i = 1; i < 4; ++i)
      if (i < nseg && bb >= sb0[i]) si = i;
    return __builtin_amdgcn_readfirstlane(si);
  };
  const int stride = nblk * nwv;
  int b = blk * nwv + wave;

  io.arrive();
  io.mark(0);   // trace: stage entry
  if (blk * nwv >= total) return true;   // no rows for this workgroup (workgroup-uniform)
  // ---------------- 1. the first poll of x, then weights and epilogue inputs of the first batch
  // One straight-line block issues every load of the first batch: the first
  // poll of x, the norm gains, the gate row, the weights and the epilogue
  // inputs.  Waves without rows load the workgroup's last batch and drop it
  // (settled before they leave).
  const bool stage_x = PRO != P_LOADQ && !(PRO == P_NORM && aemb != nullptr);
  typename IO::VecPoll vx;
  if constexpr (PRO != P_LOADQ) io.stage_issue(ax, stage_x ? K : 0, vx);
  const int bq = min(b, total - 1);
  int si = seg_index(bq);
  Seg g = seg_uniform(a.seg[si]);   // this wave's segment, in scalar registers
  uint32_t w[NCH][R][4];
  EpiAux aux;
  float nwv16[NCH][16];   // norm gains: constants, loaded before the hand-over wait
  if constexpr (PRO == P_NORM || PRO == P_GATED) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = min(lane + 64 * j, nchunk - 1);
      if (PRO == P_NORM && nw_lanes)
        load16c(anw, c, nwv16[j]);   // K = 1024: c = lane
      else
        load16g(anw + (PRO == P_GATED ? ((16 * c) & 127) : 16 * c), nwv16[j]);
    }
  }
  // a DeltaNet gate row (GemvArgs::gw), wave 0 of workgroups gblk - r
  const int grow = (gblk0 >= 0 ? gblk0 : nblk - 1) - blk;
  const bool gate_wave = PRO == P_NORM && NCH == 1 && wave == 0 && grow >= 0 && grow < grows;
  float gwv[16];
  float g_alog = 0.0f, g_dtb = 0.0f;   // the head's A_log and dt_bias (g rows only)
  if constexpr (PRO == P_NORM && NCH == 1) {
    const __amdgpu_buffer_rsrc_t rg = rsrc_n(agw, gate_wave ? 0x7ffffff0 : 0);
    load16c_rs(rg, gate_wave ? grow * 1024 : 0, lane, gwv);
    // constants: loaded with the gate row, ahead of the hand-over wait (empty
    // descriptors read 0 on waves that compute no g)
    const bool g_row = gate_wave && grow >= 16;
    g_alog = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc_n(ag_alog, g_row ? 64 : 0),
                                                                           4 * (grow & 15), 0, 0));
    g_dtb = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc_n(ag_dtb, g_row ? 64 : 0),
                                                                          4 * (grow & 15), 0, 0));
  }
  // The weights and epilogue inputs come last: a wave's loads return in issue
  // order, so whatever the prologue reads (x, the norm gains, the gate row)
  // is issued before them and its wait does not include the weights.
  {
    const int row0 = __builtin_amdgcn_readfirstlane((bq - g.batch0) * R);
    load_batch<NCH, R, EM>(g, row0, K, nchunk, lane, w);   // SEG_F32: never read
    epi_prefetch<EM>(g, row0 + row_of_lane<R>(lane), aux, io);
  }
  if (!io.wait()) return false;
  // the workgroup's copy of x (and z): every wave takes part, rows or not
  const float* xl = nullptr;
  const float* zl = nullptr;
  if (stage_x) {
    float* buf = io.slot();
    if (!io.stage_finish(ax, x_st, K, buf, vx)) return false;
    xl = buf;
  }
  if constexpr (PRO == P_GATED) {
    float* buf = io.slot();
    if (!io.stage_vec(az, z_st, K, buf)) return false;
    zl = buf;
  }
  io.mark(1);   // trace: input vector in LDS

  // ---------------- 2. prologue: this lane's chunks c = lane + 64 j of x
  float xv[NCH][16];     // fp32 activation (W8A16) / dequantized q*s (W8A8)
  uint32_t xq[NCH][4];   // int8 activation (W8A8)
  float xs = 1.0f;       // activation scale (W8A8)
  if constexpr (PRO == P_LOADQ) {
    xs = asx != nullptr ? *as_global(asx) : 1.0f;   // E_ACCI needs no scale
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = lane + 64 * j;
      load16b(axq + 16 * min(c, nchunk - 1), xq[j]);
      if (c >= nchunk) xq[j][0] = xq[j][1] = xq[j][2] = xq[j][3] = 0u;
#pragma unroll
      for (int e = 0; e < 16; ++e) xv[j][e] = i8_at(xq[j], e) * xs;
    }
  } else {
    if (PRO == P_NORM && aemb != nullptr) {   // embed_row (gemv.hpp:76-84)
      // wave-uniform at once: the wait for the token load then sits here, on
      // this path only (consumed under the lane condition below, the load stayed
      // pending where the paths join and the compiler drained every load there,
      // the weights included)
      const int tok = __builtin_amdgcn_readfirstlane(atok != nullptr ? ldc_i(atok) : tokv);
      const int8_t* er = aemb + (size_t)tok * K;
      const float es = as_global(aemb_s)[tok];
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        const int c = lane + 64 * j;
        if (c < nchunk) {
          uint32_t t[4];
          load16b(er + 16 * c, t);
#pragma unroll
          for (int e = 0; e < 16; ++e) xv[j][e] = i8_at(t, e) * es;
          if (ah_out != nullptr && blk == 0 && threadIdx.x < 64) io.st16(ah_out, out_st, 16 * c, xv[j]);
        } else {
#pragma unroll
          for (int e = 0; e < 16; ++e) xv[j][e] = 0.0f;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        load16l(xl + 16 * min(lane + 64 * j, nchunk - 1), xv[j]);
        if (lane + 64 * j >= nchunk)
#pragma unroll
          for (int e = 0; e < 16; ++e) xv[j][e] = 0.0f;
      }
    }
    // W8A8: the norms apply the gains first and 1/rms last, y = (x g) * inv.
    // Then the activation maximum needs no second pass over y: rounding is
    // monotone, so max |fl(u inv)| = fl(max |u| inv) for u = x g, and max |u|
    // is reduced across the wave together with the sum of squares instead of
    // after it (golden/model.py:37-45 takes the maximum of y).  W8A16 keeps
    // norm.hpp's order, (x inv) g.
    float amax = 0.0f;   // W8A8: max |y| over the vector, once known
    if constexpr (PRO == P_NORM) {   // norm.hpp:13-20, sum of squares in C16 order
      float ss = 0.0f, mu = 0.0f;
#pragma unroll
      for (int j = 0; j < NCH; ++j)
        if (lane + 64 * j < nchunk) ss = dot16_f32(xv[j], xv[j], ss);
      if constexpr (MODE == M_W8A8) {
#pragma unroll
        for (int j = 0; j < NCH; ++j)
          if (lane + 64 * j < nchunk)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              xv[j][e] = xv[j][e] * (1.0f + nwv16[j][e]);
              mu = fmaxf(mu, fabsf(xv[j][e]));
            }
      }
      ss = xor_sum<64>(ss);
      if constexpr (MODE == M_W8A8) mu = xor_max<64>(mu);
      const float inv = 1.0f / sqrtf(ss / (float)K + eps);
#pragma unroll
      for (int j = 0; j < NCH; ++j)
        if (lane + 64 * j < nchunk)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            if constexpr (MODE == M_W8A8)
              xv[j][e] = xv[j][e] * inv;
            else
              xv[j][e] = (xv[j][e] * inv) * (1.0f + nwv16[j][e]);
          }
      amax = mu * inv;
    } else if constexpr (PRO == P_GATED) {   // heads of 128 = groups of 8 lanes; z holds silu(z)
      float zs[NCH][16];
#pragma unroll
      for (int j = 0; j < NCH; ++j) load16l(zl + 16 * (lane + 64 * j), zs[j]);
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        float ss = dot16_f32(xv[j], xv[j], 0.0f), mu = 0.0f;
        if constexpr (MODE == M_W8A8) {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            xv[j][e] = (xv[j][e] * nwv16[j][e]) * zs[j][e];
            mu = fmaxf(mu, fabsf(xv[j][e]));
          }
        }
        ss = xor_sum<8>(ss);
        if constexpr (MODE == M_W8A8) mu = xor_max<8>(mu);   // this head's max |u|
        const float inv = 1.0f / sqrtf(ss / 128.0f + eps);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          if constexpr (MODE == M_W8A8)
            xv[j][e] = xv[j][e] * inv;
          else
            xv[j][e] = ((xv[j][e] * inv) * nwv16[j][e]) * zs[j][e];   // norm.hpp:32
        }
        amax = fmaxf(amax, mu * inv);
      }
    }
    if constexpr (MODE == M_W8A8) {   // _qa (golden/model.py:37-45)
      float am = amax;   // P_NORM: already the vector's maximum
      if constexpr (PRO == P_GATED) am = xor_max<64>(am);   // the maximum over the heads
      if constexpr (PRO != P_NORM && PRO != P_GATED) {
#pragma unroll
        for (int j = 0; j < NCH; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) am = fmaxf(am, fabsf(xv[j][e]));
        am = xor_max<64>(am);
      }
      xs = quant_scale(am);
      const float rs = 1.0f / xs;
      if constexpr (NCH >= 2) {
        // Every wave needs the lane's 4 NCH packed dwords; the waves quantise
        // them round robin and the packed bytes meet in LDS.
        uint32_t* ql = gemv_qlds();
#pragma unroll
        for (int j = 0; j < NCH; ++j)
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            if (((4 * j + d) & (nwv - 1)) == wave) {   // nwv is 1, 2 or 4
              int q[4];
#pragma unroll
              for (int k = 0; k < 4; ++k) q[k] = quant_one_r(xv[j][4 * d + k], xs, rs);
              ql[(j * 64 + lane) * 4 + d] = pack4(q[0], q[1], q[2], q[3]);
            }
          }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
          const u32x4 t = *as_lds(reinterpret_cast<const u32x4*>(ql + (j * 64 + lane) * 4));
#pragma unroll
          for (int d = 0; d < 4; ++d) xq[j][d] = t[d];
        }
        if (has_f32) {   // fp32-weight segments take the dequantised activation
#pragma unroll
          for (int j = 0; j < NCH; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) xv[j][e] = i8_at(xq[j], e) * xs;
        }
      } else {   // one chunk per lane: every wave quantises it
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
          int q[16];
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            q[e] = quant_one_r(xv[j][e], xs, rs);
            xv[j][e] = (float)q[e] * xs;
          }
#pragma unroll
          for (int d = 0; d < 4; ++d) xq[j][d] = pack4(q[4 * d], q[4 * d + 1], q[4 * d + 2], q[4 * d + 3]);
        }
      }
    }
  }

  io.mark(2);   // trace: prologue done
  if constexpr (PRO == P_NORM && NCH == 1) {
    if (gate_wave) {   // deltanet.hpp:164-165 on the prologue's (normalised, quantised) activation
      const int hh = grow & 15;
      const float y = xor_sum<64>(dot16_f32(gwv, xv[0], 0.0f));
      float val;
      if (grow < 16)
        val = dev_sigmoid(y);   // beta
      else
        val = -dev_expf(g_alog) * dev_softplus(y + g_dtb);   // g
      if (lane == 0) io.st1(agout, out_st, 16 * hh + (grow < 16 ? 1 : 0), val);
    }
  }
  if (b >= total) {   // no rows for this wave (it took part in the barriers above)
#pragma unroll
    for (int j = 0; j < NCH; ++j)
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int d = 0; d < 4; ++d) settle(w[j][r][d]);
    settle_aux(aux);
    if constexpr (PRO == P_NORM && NCH == 1) {
#pragma unroll
      for (int e = 0; e < 16; ++e) settle(gwv[e]);
      settle(g_alog), settle(g_dtb);
    }
    return true;
  }
  const int b0 = b;
  // ---------------- 3. row batches (the next batch's loads overlap this batch's reduction)
  for (; b < total; b += stride) {
    const int row0 = __builtin_amdgcn_readfirstlane((b - g.batch0) * R);
    const int myrow = row0 + row_of_lane<R>(lane);
    float y = 0.0f;
    int acci = 0;
    float pf[R];
    int pi[R];
    const bool f32 = em_has<EM>(kEmF32) && g.kind == SEG_F32;
    if (f32) {   // fp32 weights (gemv.hpp:46-59)
#pragma unroll
      for (int r = 0; r < R; ++r) pf[r] = 0.0f;
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        const int c = lane + 64 * j;
        if (c < nchunk) {
#pragma unroll
          for (int r = 0; r < R; ++r) {
            if (row0 + r < g.rows) {
              float wf[16];
              load16g(g.wf + (size_t)(row0 + r) * K + 16 * c, wf);
              pf[r] = dot16_f32(wf, xv[j], pf[r]);
            }
          }
        }
      }
    } else if constexpr (MODE == M_W8A16) {   // int8 x fp32 (gemv.hpp:28-42)
#pragma unroll
      for (int r = 0; r < R; ++r) pf[r] = 0.0f;
#pragma unroll
      for (int j = 0; j < NCH; ++j)
        if (lane + 64 * j < nchunk)
#pragma unroll
          for (int r = 0; r < R; ++r) pf[r] = dot16_i8f(w[j][r], xv[j], pf[r]);
    } else {   // int8 x int8 -> int32 (export_gemv_tv.py:298)
#pragma unroll
      for (int r = 0; r < R; ++r) pi[r] = 0;
#pragma unroll
      for (int j = 0; j < NCH; ++j)
#pragma unroll
        for (int r = 0; r < R; ++r) pi[r] = dot16_i8i8(w[j][r], xq[j], pi[r]);
    }
    if (b == b0) {   // trace: dot products of the first batch done (its weights arrived)
      if constexpr (MODE == M_W8A8) {
        if (!f32) asm volatile("" ::"v"(pi[0]));
        else asm volatile("" ::"v"(pf[0]));
      } else {
        asm volatile("" ::"v"(pf[0]));
      }
      io.mark(5);
      if constexpr (PRO == P_NORM && NCH == 1) {   // the gate loads (issued before the weights) of other waves
#pragma unroll
        for (int e = 0; e < 16; ++e) settle(gwv[e]);
        settle(g_alog), settle(g_dtb);
      }
    }
    // issue the next batch's loads before reducing this one
    const int bn = b + stride;
    int sin = si;
    Seg gn = g;
    EpiAux auxn;
    if (bn < total) {
      sin = seg_index(bn);
      if (sin != si) gn = seg_uniform(a.seg[sin]);
      const int rn = __builtin_amdgcn_readfirstlane((bn - gn.batch0) * R);
      if (!(em_has<EM>(kEmF32) && gn.kind == SEG_F32)) load_batch<NCH, R, EM>(gn, rn, K, nchunk, lane, w);
      epi_prefetch<EM>(gn, rn + row_of_lane<R>(lane), auxn, io);
    }
    if (f32 || MODE == M_W8A16) {
      y = reduce_rows<R>(pf, lane);
      if (!f32) y = y * aux.sc;
    } else {
      acci = reduce_rows<R>(pi, lane);
      y = ((float)acci * xs) * aux.sc;   // float(acc)*sx*sw
    }
    if (em_has<EM>(1 << E_RESID) && g.epi == E_RESID &&
        !io.resolve1(aux.res, g.res, g.res_st, min(myrow, g.rows - 1), aux.a0))
      return false;
    gemv_epilogue<R, EM>(g, out_st, lane, myrow, y, acci, aux, io);
    settle_aux(aux);   // inputs this segment's epilogue did not read
    if (b == b0) io.mark(6);   // trace: first batch stored
    si = sin;
    g = gn;
    aux = auxn;
  }
  return true;
}

// ===========================================================================
// W8A8 GEMV with one output row per wave and the vector split over the
// workgroup's four waves (the 1024-row projections with K = 2048 or 3584:
// DeltaNet out_proj, attention o_proj, MLP down).  The workgroup owns rows
// rb .. rb + 3; wave w takes chunk jw = w % NCH of every lane (elements
// 16 (lane + 64 jw) .. +15) for the NCH rows of group w / NCH, so it stages,
// normalises and quantises a quarter (NCH = 4) or half (NCH = 2) of the vector
// instead of all of it.  The maxima of the chunks meet in LDS (max is exact in
// any order), every wave quantises its chunk with the vector's scale, forms the
// int32 lane partials of its rows, reduces them over the lanes and leaves them
// in LDS; wave w then adds the NCH partials of row rb + w (int32: exact in any
// order) and runs the row's epilogue.  Every value equals gemv_body's.
// Preconditions (gemv_splitk_ok): four waves, every workgroup's four rows in
// the one segment, one batch per wave.
// ===========================================================================
__device__ __forceinline__ int* splitk_lds() {
  __shared__ int v[4 + 4 * 4];   // chunk maxima (float bits) [wave], row partials [wave][row]
  return v;
}
__device__ __forceinline__ bool gemv_splitk_ok(const GemvArgs& a, int nblk, int nwv) {
  return nwv == 4 && a.nseg == 1 && a.seg[0].batch0 == 0 && (a.seg[0].nbatch & 3) == 0 &&
         a.seg[0].nbatch <= nblk * 4 && a.seg[0].kind == SEG_I8;
}
template <int NCH, int PRO, int KC, class IO>
__device__ __forceinline__ bool gemv_splitk(const GemvArgs& a, int blk, IO& io) {
  static_assert(NCH == 2 || NCH == 4, "two or four chunks per lane");
  static_assert(PRO == P_LOAD || PRO == P_GATED, "prologue");
  constexpr int EM = kEmResid;
  constexpr int K = KC, nchunk = K / 16, RW = NCH;   // rows per wave
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int jw = wave % NCH, grp = wave / NCH;
  const float* const ax = a.x;
  const float* const anw = a.nw;
  const float* const az = a.z;
  const float eps = a.eps;
  const int x_st = a.x_st, z_st = a.z_st, out_st = a.out_st;
  const int total = __builtin_amdgcn_readfirstlane(a.seg[0].nbatch);
  io.arrive();
  io.mark(0);   // trace: stage entry
  if (blk * 4 >= total) return true;   // no rows for this workgroup (workgroup-uniform)
  typename IO::VecPoll vx;
  io.stage_issue(ax, K, vx);
  const Seg g = seg_uniform(a.seg[0]);
  const int rb = __builtin_amdgcn_readfirstlane(blk * 4);
  const int c = lane + 64 * jw;           // this lane's chunk
  const int cc = min(c, nchunk - 1);
  float nw16[16];
  if constexpr (PRO == P_GATED) load16g(anw + ((16 * cc) & 127), nw16);   // the head's gains
  // weights: rows rb + grp * RW + r, chunk c (clamped; a chunk past K meets x = 0)
  uint32_t w[RW][4];
  {
    const __amdgpu_buffer_rsrc_t rw = rsrc_n(g.w, 0x7ffffff0);
    const int last = g.rows - 1;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int row = __builtin_amdgcn_readfirstlane(min(rb + grp * RW + r, last));
      const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(rw, 16 * cc, row * K, kNt);
      w[r][0] = t[0];
      w[r][1] = t[1];
      w[r][2] = t[2];
      w[r][3] = t[3];
    }
  }
  EpiAux aux;   // the output row of this wave, rb + wave
  epi_prefetch<EM>(g, rb + wave, aux, io);
  if (!io.wait()) return false;
  float* xl = io.slot();
  if (!io.stage_finish(ax, x_st, K, xl, vx)) return false;
  const float* zl = nullptr;
  if constexpr (PRO == P_GATED) {
    float* buf = io.slot();
    if (!io.stage_vec(az, z_st, K, buf)) return false;
    zl = buf;
  }
  io.mark(1);   // trace: input vector in LDS
  float xv[16];
  load16l(xl + 16 * cc, xv);
  if (c >= nchunk)
#pragma unroll
    for (int e = 0; e < 16; ++e) xv[e] = 0.0f;
  float amax = 0.0f;   // this lane's maximum |y| over its chunk
  if constexpr (PRO == P_GATED) {   // heads of 128 = groups of 8 lanes; z holds silu(z); W8A8 order (x g) inv
    float zs[16];
    load16l(zl + 16 * cc, zs);
    float ss = dot16_f32(xv, xv, 0.0f), mu = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      xv[e] = (xv[e] * nw16[e]) * zs[e];
      mu = fmaxf(mu, fabsf(xv[e]));
    }
    ss = xor_sum<8>(ss);
    mu = xor_max<8>(mu);   // this head's max |u|
    const float inv = 1.0f / sqrtf(ss / 128.0f + eps);
#pragma unroll
    for (int e = 0; e < 16; ++e) xv[e] = xv[e] * inv;
    amax = mu * inv;
  } else {
#pragma unroll
    for (int e = 0; e < 16; ++e) amax = fmaxf(amax, fabsf(xv[e]));
  }
  int* sk = splitk_lds();
  {
    const float cm = xor_max<64>(amax);   // the chunk's maximum
    if (lane == 0) as_lds_w(sk)[wave] = __float_as_int(cm);
  }
  __syncthreads();
  float am = 0.0f;   // _qa (golden/model.py:37-45): the vector's maximum
#pragma unroll
  for (int v = 0; v < 4; ++v) am = fmaxf(am, __int_as_float(as_lds(sk)[v]));
  const float xs = quant_scale(am);
  const float rs = 1.0f / xs;
  uint32_t xq[4];
  {
    int q[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) q[e] = quant_one_r(xv[e], xs, rs);
#pragma unroll
    for (int d = 0; d < 4; ++d) xq[d] = pack4(q[4 * d], q[4 * d + 1], q[4 * d + 2], q[4 * d + 3]);
  }
  io.mark(2);   // trace: prologue done
  int pi[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) pi[r] = dot16_i8i8(w[r], xq, 0);
  asm volatile("" ::"v"(pi[0]));
  io.mark(5);   // trace: dot products done (the weights arrived)
  {
    // the four-row transposed butterfly (rows past RW are zero): lane l ends with
    // row (l >> 4) & 3, and lanes 0, 16, 32, 48 write their rows' partials
    int p4[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) p4[r] = r < RW ? pi[r] : 0;
    const int part = reduce4(p4, lane);
    const int prow = row_of_lane<4>(lane);
    if ((lane & 15) == 0 && prow < RW) as_lds_w(sk)[4 + 4 * wave + prow] = part;
  }
  __syncthreads();
  // row rb + wave: the partials of the NCH waves of its group, at its position in the group
  int acci = 0;
#pragma unroll
  for (int jj = 0; jj < NCH; ++jj) acci += as_lds(sk)[4 + 4 * ((wave / NCH) * NCH + jj) + wave % NCH];
  const int myrow = rb + wave;
  const float y = ((float)acci * xs) * aux.sc;   // float(acc)*sx*sw
  if (!io.resolve1(aux.res, g.res, g.res_st, min(myrow, g.rows - 1), aux.a0)) return false;
  gemv_epilogue<1, EM>(g, out_st, lane, myrow, y, acci, aux, io);
  settle_aux(aux);   // inputs this segment's epilogue did not read
  io.mark(6);   // trace: row stored
  return true;
}

// ===========================================================================
// Tied LM head: final rmsnorm prologue, logits = (E row . h) * s in C16
// order, running argmax with the reference's rule (strict >, so the first
// index wins a tie; qwen_synth.hpp:81-88) folded per workgroup.  Two batches
// of 8 rows (16 KiB per wave) are in flight while a third is reduced.
// KEEP: every other batch loads with the default cache policy, so half the
// head stays in the Infinity Cache from one token to the next (the layer
// kernels' decode, whose weights all load non-temporally).  The persistent
// kernel loads the whole head non-temporally: its Infinity Cache holds the
// gate/up and q, k, v weights instead (weight_policy).
// ===========================================================================
__device__ __forceinline__ void better(float& bv, int& bi, float v, int i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

// Loads of one batch (8 rows and this lane's row scale).  Every load is issued
// unconditionally: a batch beyond the last one goes through empty descriptors
// (no memory access, reads 0), so the loop keeps no conditionally loaded
// registers and the compiler waits for exactly the batch it consumes.
// hw / hsw: the weight and scale bases, wave-uniform values the caller read
// from the descriptor once (read through the descriptor here, they would be
// read from LDS again at every batch: the logits stores may alias it).
template <int POL>
__device__ __forceinline__ void head_load(const int8_t* hw, const float* hsw, int b, int total, int lane, int rl,
                                          uint32_t (&w)[8][4], float& sc) {
  b = __builtin_amdgcn_readfirstlane(b);   // wave-uniform: scalar descriptors
  const bool in = b < total;
  const __amdgpu_buffer_rsrc_t rw = rsrc_n(hw, in ? 0x7ffffff0 : 0);
  const __amdgpu_buffer_rsrc_t rs = rsrc_n(hsw, in ? 0x7ffffff0 : 0);
  const int bb = in ? b : 0;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(rw, (bb * 8 + r) * 1024 + 16 * lane, 0, POL);
    w[r][0] = t[0];
    w[r][1] = t[1];
    w[r][2] = t[2];
    w[r][3] = t[3];
  }
  sc = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, (bb * 8 + rl) * 4, 0, 0));
}

template <bool KEEP, class IO>
__device__ __forceinline__ bool head_body(const HeadArgs& a, int blk, int nblk, IO& io, float* logits) {
  const int lane = threadIdx.x & 63, nwv = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int total = __builtin_amdgcn_readfirstlane(a.rows / kRowsPerBatch);
  const int8_t* const hw = static_cast<const int8_t*>(wave_uniform(a.w));
  const float* const hsw = static_cast<const float*>(wave_uniform(a.sw));
  const int stride = nblk * nwv;
  int b = blk * nwv + wave;
  const int rl = (lane >> 3) & 7;
  io.arrive();
  typename IO::VecPoll vh;
  io.stage_issue(a.h, 1024, vh);
  uint32_t w0[8][4], w1[8][4];
  float sc0 = 0.0f, sc1 = 0.0f;
  head_load<kNt>(hw, hsw, b, total, lane, rl, w0, sc0);   // two batches in flight before the norm prologue
  head_load<KEEP ? 0 : kNt>(hw, hsw, b + stride, total, lane, rl, w1, sc1);
  float xv[16], nw[16];
  if (a.nw_lanes)
    load16c(a.nw, lane, nw);
  else
    load16g(a.nw + 16 * lane, nw);
  if (!io.wait()) return false;
  {
    float* hl = io.slot();
    if (!io.stage_finish(a.h, a.h_st, 1024, hl, vh)) return false;
    load16l(hl + 16 * lane, xv);
  }
  float ss = dot16_f32(xv, xv, 0.0f);
  ss = xor_sum<64>(ss);
  const float inv = 1.0f / sqrtf(ss / 1024.0f + a.eps);
#pragma unroll
  for (int e = 0; e < 16; ++e) xv[e] = (xv[e] * inv) * (1.0f + nw[e]);
  float bv = -1e30f;
  int bi = 0;
  // batch bb from buffer (w, sc); the buffer is refilled with batch bb + 2 stride
  // before the reduction.  Both halves of the loop body run unconditionally (a
  // wave with an odd number of batches finishes in the tail), so the buffers
  // keep fixed registers and each wait covers exactly the batch consumed.
  auto batch = [&](auto pol, int bb, uint32_t (&w)[8][4], float& sc) {
    float p[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) p[r] = dot16_i8f(w[r], xv, 0.0f);
    float scur;   // an explicit copy frees sc's register for the next load (no copy at the loop latch)
    asm volatile("v_mov_b32 %0, %1" : "=v"(scur) : "v"(sc));
    head_load<decltype(pol)::value>(hw, hsw, bb + 2 * stride, total, lane, rl, w, sc);
    const float y = reduce8(p, lane) * scur;
    const int row = bb * 8 + rl;
    if ((lane & 7) == 0) {
      if (logits != nullptr) logits[row] = y;
      better(bv, bi, y, row);
    }
  };
  using Nt = std::integral_constant<int, kNt>;
  using Keep = std::integral_constant<int, KEEP ? 0 : kNt>;
  for (; b + stride < total; b += 2 * stride) {
    batch(Nt{}, b, w0, sc0);
    batch(Keep{}, b + stride, w1, sc1);
  }
  if (b < total) batch(Nt{}, b, w0, sc0);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    better(bv, bi, ov, oi);
  }
  __shared__ float sv[4];
  __shared__ int sx[4];
  if (lane == 0) {
    sv[wave] = bv;
    sx[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w2 = 1; w2 < nwv; ++w2) better(bv, bi, sv[w2], sx[w2]);
    // Every earlier store of this workgroup (cache rows, state) completes before
    // the partial that the next token waits for is published.
    if constexpr (IO::kTagged) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    io.st1(a.part_val, a.part_st, blk, bv);
    io.st1i(a.part_idx, a.part_st, blk, bi);
  }
  __syncthreads();
  return true;
}

// ===========================================================================
// Gated DeltaNet recurrent step (deltanet.hpp:58-127 and the l2norm / q-scale
// of deltanet.hpp:166-169).  Unit (head h, quarter vq) owns S[h][:, 32 vq ..
// 32 vq + 31]; wave w takes columns v = 32 vq + 8 w + (lane >> 3) and lane
// group kg = lane & 7 the 16 rows k = 16 kg .. 16 kg + 15 of its column, so
// the eight k-groups of a column sit in one lane octet and meet by the xor
// tree of offsets 4, 2, 1 (the pairwise tree of the device order).  Each lane
// holds the q and k chunks of its k-group and normalises them itself (the
// octet holds whole vectors).  Sweep A decays S and forms the k-group partial
// of k^T S; delta = (v - kv) * beta; sweep B applies the rank-1 update and
// forms q^T S_new.  No workgroup barrier, no LDS.  S is read and written once
// per step, always by the same unit.
// ===========================================================================
// Head h's gate projections from the layer input (see DnArgs), computed by a
// whole wave; every lane returns (g, beta).  Same operations as the in_proj
// prologue and its fp32 segments, so the values are bit-identical to
// computing them there.
template <class IO>
__device__ __forceinline__ bool deltanet_gates(const DnArgs& a, int h, int tokv, float& g, float& beta, IO& io) {
  const int lane = threadIdx.x & 63;
  float xv[16];
  if (a.emb != nullptr) {   // embed_row (gemv.hpp:76-84)
    const int tok = a.tok != nullptr ? ldc_i(a.tok) : tokv;
    uint32_t t4[4];
    load16b(a.emb + (size_t)tok * 1024 + 16 * lane, t4);
    const float es = as_global(a.emb_s)[tok];
#pragma unroll
    for (int e = 0; e < 16; ++e) xv[e] = i8_at(t4, e) * es;
  } else if (const float* xl = io.cached(a.gx, a.gx_st)) {   // the in_proj stage's copy
    load16l(xl + 16 * lane, xv);
  } else {
    int idx[1] = {16 * lane};
    float t1[1][16];
    if (!io.template ld16<1>(a.gx, a.gx_st, idx, t1)) return false;
#pragma unroll
    for (int e = 0; e < 16; ++e) xv[e] = t1[0][e];
  }
  if (a.gx_norm != nullptr) {   // norm.hpp:13-20, in the GEMV prologue's order for the mode
    float nw[16];
    if (a.lanes)
      load16c(a.gx_norm, lane, nw);
    else
      load16g(a.gx_norm + 16 * lane, nw);
    float ss = dot16_f32(xv, xv, 0.0f);
    ss = xor_sum<64>(ss);
    const float inv = 1.0f / sqrtf(ss / 1024.0f + a.eps);
    if (a.mode == M_W8A8) {
#pragma unroll
      for (int e = 0; e < 16; ++e) xv[e] = (xv[e] * (1.0f + nw[e])) * inv;
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) xv[e] = (xv[e] * inv) * (1.0f + nw[e]);
    }
  }
  if (a.mode == M_W8A8) {   // _qa (golden/model.py:37-45), dequantised
    float am = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) am = fmaxf(am, fabsf(xv[e]));
    am = xor_max<64>(am);
    const float xs = quant_scale(am);
    const float rs = 1.0f / xs;
#pragma unroll
    for (int e = 0; e < 16; ++e) xv[e] = (float)quant_one_r(xv[e], xs, rs) * xs;
  }
  float w[16], w2[16];
  if (a.lanes) {
    load16c(a.wb + (size_t)h * 1024, lane, w);
    load16c(a.wa + (size_t)h * 1024, lane, w2);
  } else {
    load16g(a.wb + (size_t)h * 1024 + 16 * lane, w);
    load16g(a.wa + (size_t)h * 1024 + 16 * lane, w2);
  }
  const float yb = xor_sum<64>(dot16_f32(w, xv, 0.0f));
  const float ya = xor_sum<64>(dot16_f32(w2, xv, 0.0f));
  beta = dev_sigmoid(yb);
  g = -dev_expf(as_global(a.A_log)[h]) * dev_softplus(ya + as_global(a.dt_bias)[h]);
  return true;
}

// GATES: g and beta are pairs 6144 + 16 h and 6144 + 16 h + 1 of the tagged
// convd vector (written by the in_proj stage, see GemvArgs::gw) and arrive
// with q, k and v; otherwise every wave computes them.
// LDS-resident state (persistent kernel): a unit's 128 x 32 slice of S lives in
// one LDS tile of its workgroup for the whole launch -- thread t's 16 values
// (rows 16 kg .. 16 kg + 15 of its column) as four quads at (q * 256 + t) * 4,
// so each of the four 16-byte reads and writes of a wave is one conflict-free
// 1 KiB span.  The launch loads the tiles from the state buffer at its start
// and writes them back at its end (persist_kernel); a token reads and writes
// only LDS.  Unit u of the stage with DnArgs::unit_base b runs on workgroup
// (b + u) % nblk and keeps its tile in slot (b + u) / nblk: the 18 layers' 1152
// units spread over all workgroups, kDnSlots tiles at most each.
constexpr int kDnTile = 128 * 32;   // floats
__device__ __forceinline__ float* dn_tiles() {
  __shared__ __attribute__((aligned(16))) float t[kDnSlots * kDnTile];
  return t;
}
__device__ __forceinline__ void dn_tile_read(const float* tile, float* s) {
  const __attribute__((address_space(3))) f32x4* q = as_lds(reinterpret_cast<const f32x4*>(tile));
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const f32x4 t = q[k * kPersistThreads + threadIdx.x];
#pragma unroll
    for (int e = 0; e < 4; ++e) s[4 * k + e] = t[e];
  }
}
__device__ __forceinline__ void dn_tile_write(float* tile, const float* s) {
  __attribute__((address_space(3))) f32x4* q = (__attribute__((address_space(3))) f32x4*)tile;
#pragma unroll
  for (int k = 0; k < 4; ++k) q[k * kPersistThreads + threadIdx.x] = f32x4{s[4 * k], s[4 * k + 1], s[4 * k + 2], s[4 * k + 3]};
}
// This thread's column and rows of unit u (see deltanet_body).
__device__ __forceinline__ int dn_col(int unit) {
  return (unit % kDnVQuarters) * 32 + 8 * (int)(threadIdx.x >> 6) + (int)((threadIdx.x & 63) >> 3);
}

template <bool GATES, bool LDSS, class IO>
__device__ __forceinline__ bool deltanet_body(const DnArgs& a, int unit, bool valid, IO& io, int tokv,
                                              float* tile = nullptr) {
  const int h = unit / kDnVQuarters, vq = unit % kDnVQuarters;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kg = lane & 7, v = vq * 32 + 8 * wave + (lane >> 3);
  float* Sh = a.S + (size_t)h * 128 * 128;
  io.arrive();
  io.mark(0);   // trace: stage entry
  // convd = q (2048) | k (2048) | v (2048), post-conv: the head's q and k (one 128-element region
  // each) and the v element of this lane's column
  constexpr int M = GATES ? 3 : 1;
  const int reg[2] = {h * 128, 2048 + h * 128};
  int iv[M];
  if constexpr (GATES) {
    iv[0] = 6144 + 16 * h;       // g
    iv[1] = 6144 + 16 * h + 1;   // beta
  }
  iv[M - 1] = 4096 + h * 128 + v;   // (the poll samples the last one)
  typename IO::template PollR<2, M> P;
  float s[16];
  float g = 0.0f, beta = 0.0f;
  if (valid) {
    io.template pollr_issue<2, M>(a.convd, reg, iv, P);
    if constexpr (LDSS) {
      dn_tile_read(tile, s);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) s[i] = as_global(Sh)[(kg * 16 + i) * 128 + v];
    }
    // inputs final before in_proj: computed while the hand-over is in flight
    if (!GATES && a.wa != nullptr && !deltanet_gates(a, h, tokv, g, beta, io)) return false;
  }
  if (!io.wait()) return false;
  if (!valid) return true;
  if constexpr (!IO::kTagged) {   // gates given by the op-level caller
    if (a.wa == nullptr) {
      g = ldcb(a.gb, h);
      beta = ldcb(a.gb, 16 + h);
    }
  }
  float qk[2][16], vv[M];
  float* wa = wave_area();
  if (!io.template pollr_finish<2, M>(a.convd, a.convd_st, reg, iv, P, wa, vv)) return false;
  load16l(wa + 16 * kg, qk[0]);         // q rows 16 kg .. 16 kg + 15
  load16l(wa + 128 + 16 * kg, qk[1]);   // k rows 16 kg .. 16 kg + 15
  if constexpr (GATES) {
    g = vv[0];
    beta = vv[1];
  }
  io.mark(1);   // trace: q, k, v of the head received
  if (a.normalize) {   // l2norm (deltanet.hpp:134); q also scaled by 1/sqrt(128) (deltanet.hpp:168-169)
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      float ss = dot16_f32(qk[w], qk[w], 0.0f);
      ss = xor_sum<8>(ss);
      const float inv = 1.0f / sqrtf(ss + 1e-6f);
#pragma unroll
      for (int e = 0; e < 16; ++e) qk[w][e] = qk[w][e] * inv;
    }
    const float sc = 1.0f / sqrtf(128.0f);
#pragma unroll
    for (int e = 0; e < 16; ++e) qk[0][e] = qk[0][e] * sc;
  }
  const float gexp = dev_expf(g);
  float p = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {   // sweep A
    s[i] = s[i] * gexp;
    p = p + s[i] * qk[1][i];
  }
  p = xor_sum<8>(p);
  const float d = (vv[M - 1] - p) * beta;
  io.mark(2);   // trace: delta computed (sweep A done)
  p = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {   // sweep B: reads the updated S
    s[i] = s[i] + qk[1][i] * d;
    p = p + s[i] * qk[0][i];
    if constexpr (!LDSS) as_global_w(Sh)[(kg * 16 + i) * 128 + v] = s[i];
  }
  p = xor_sum<8>(p);
  if (kg == 0) io.st1(a.o, a.o_st, h * 128 + v, p);
  if constexpr (LDSS) dn_tile_write(tile, s);
  return true;
}

// All heads * kDnVQuarters units; the first one of each workgroup prefetches.
// All heads * kDnVQuarters units; the first one of each workgroup prefetches.
template <class IO>
__device__ __forceinline__ bool deltanet_all(const DnArgs& a, int blk, int nblk, IO& io, int tokv) {
  const int units = a.heads * kDnVQuarters;
  if constexpr (IO::kTagged) {
    const int ub = __builtin_amdgcn_readfirstlane(a.unit_base);
    if (ub >= 0) {   // LDS-resident state: one unit per workgroup (nblk >= units, host-checked)
      const int u = ((blk - ub) % nblk + nblk) % nblk;
      const bool valid = u < units;
      float* tile = dn_tiles() + kDnTile * ((ub + (valid ? u : 0)) / nblk);
      return deltanet_body<true, true>(a, valid ? u : 0, valid, io, tokv, tile);
    }
  }
  if (IO::kTagged && a.gates_in_convd) {
    if (!deltanet_body<true, false>(a, blk, blk < units, io, tokv)) return false;
    for (int u = blk + nblk; u < units; u += nblk)
      if (!deltanet_body<true, false>(a, u, true, io, tokv)) return false;
  } else {
    if (!deltanet_body<false, false>(a, blk, blk < units, io, tokv)) return false;
    for (int u = blk + nblk; u < units; u += nblk)
      if (!deltanet_body<false, false>(a, u, true, io, tokv)) return false;
  }
  return true;
}

// The LDS tiles of workgroup blk: every DeltaNet stage of the program with a
// unit on this workgroup copies its slice of S between the state buffer and
// LDS (to_lds: at the launch start; otherwise back, at its end).
__device__ __forceinline__ void dn_tiles_copy(const Stage* prog, int nstage, int blk, int nblk, bool to_lds) {
  const int t = threadIdx.x, kg = (t & 63) & 7;
  for (int i = 0; i < nstage; ++i) {
    if (prog[i].kind != ST_DELTANET) continue;
    const int ub = prog[i].d.unit_base;
    if (ub < 0) continue;
    const int units = prog[i].d.heads * kDnVQuarters;
    const int u = ((blk - ub) % nblk + nblk) % nblk;
    if (u >= units) continue;
    float* tile = dn_tiles() + kDnTile * ((ub + u) / nblk);
    float* Sh = prog[i].d.S + (size_t)(u / kDnVQuarters) * 128 * 128;
    const int v = dn_col(u);
    float s[16];
    if (to_lds) {
#pragma unroll
      for (int k = 0; k < 16; ++k) s[k] = Sh[(kg * 16 + k) * 128 + v];
      dn_tile_write(tile, s);
    } else {
      dn_tile_read(tile, s);
#pragma unroll
      for (int k = 0; k < 16; ++k) Sh[(kg * 16 + k) * 128 + v] = s[k];
    }
  }
}

// ===========================================================================
// Gated GQA attention, split-K flash decoding (attention.hpp:25-95).
// Unit u = 2 s + j covers positions [16 s, 16 s + 16) of kv head j; wave i of
// the unit handles query head 4 j + i (GQA kv = h/4) on its own, so a unit
// needs no workgroup barrier and no LDS.  Before its inputs are ready a wave
// loads the split's cached K rows in the C16 layout (16 lanes x 16 dims, the
// four lane groups hold four positions, four rows each), the cached V rows
// with four dimensions per lane, the norm gains and this position's RoPE
// row.  The cache rows of a split are written (by the unit whose split holds
// the new slot) and read only by the same unit -- the same workgroup in the
// persistent kernel, for every token -- so they are read with ordinary loads.
// After the hand-over the wave normalises and rotates its query (QK-norm with
// (1+w), RoPE on dims 0..63); in the unit whose split holds slot T every wave
// also normalises and rotates the new K row and takes the new V elements, and
// wave 0 writes both to the cache.  Scores are C16 dots scaled by 1/16; per
// head the split max m, p = exp(s - m), the position-tree sum l of p and the
// position-ordered fma sum acc = sum p v are written for the combine step.
// ===========================================================================
struct AttnPre {
  float k[4][16];            // K row of position t0 + 4 it + pg, dims 16 g16 .. +15
  float v[kAttnSplit][4];    // V row of position t0 + u, dims 4 lane .. +3
  float qn[16], kn[16];      // q_norm / k_norm gains of dims 16 g16 .. +15
  float cs[16], sn[16];      // RoPE cos / sin[(16 g16 + e) & 31] (rope.hpp:30-41)
};

__device__ __forceinline__ void load16_rs(const __amdgpu_buffer_rsrc_t& rs, int byte_off, float* v) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(rs, byte_off + 16 * k, 0, 0);
    v[4 * k + 0] = __uint_as_float(t[0]);
    v[4 * k + 1] = __uint_as_float(t[1]);
    v[4 * k + 2] = __uint_as_float(t[2]);
    v[4 * k + 3] = __uint_as_float(t[3]);
  }
}

// Cache rows are read with ordinary loads.  A row is written once per launch,
// with sc1 (write-through) stores, by the new position's unit (or, above
// kAttnShortMax positions, by the owner of the split holding it), possibly on
// another XCD,
// and complete before the token's head partial is published.  Before that
// token no unit reads the row (rows are clamped to T - 1), so no other XCD's
// L2 holds a stale copy; the owner of a long split loads the row of slot T,
// replaces it in registers and writes it through its own L2.  Across launches
// the kernel boundary orders it.
// Straight-line loads, no branch: rows at or past slot T are clamped to row
// T - 1 (T = 0: an empty descriptor, reads 0).  Such a K row only meets a
// score that is masked to -inf, and such a V row lies past the positions the
// P.V loop visits, or is replaced by the new row.
__device__ __forceinline__ void attn_prefetch(const AttnArgs& a, int s, int j, int T, int rrow, AttnPre& pf) {
  const int lane = threadIdx.x & 63, g16 = lane & 15, pg = lane >> 4;
  const int t0 = s * kAttnSplit;
  constexpr int kBig = 0x7ffffff0;
  const __amdgpu_buffer_rsrc_t rk = rsrc_n(a.kc, T > 0 ? kBig : 0);
  const __amdgpu_buffer_rsrc_t rv = rsrc_n(a.vc, T > 0 ? kBig : 0);
  const int last = T > 0 ? T - 1 : 0;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int tp = min(t0 + 4 * it + pg, last);
    load16_rs(rk, (tp * 512 + j * 256 + 16 * g16) * 4, pf.k[it]);
  }
#pragma unroll
  for (int u = 0; u < kAttnSplit; ++u) {
    const int tp = min(t0 + u, last);
    const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(rv, (tp * 512 + j * 256 + 4 * lane) * 4, 0, 0);
#pragma unroll
    for (int e = 0; e < 4; ++e) pf.v[u][e] = __uint_as_float(t[e]);
  }
  load16_rs(rsrc_n(a.qn, kBig), 64 * g16, pf.qn);
  load16_rs(rsrc_n(a.kn, kBig), 64 * g16, pf.kn);
  const __amdgpu_buffer_rsrc_t rr = rsrc_n(a.rope, kBig);
  load16_rs(rr, (rrow * 64 + 16 * (g16 & 1)) * 4, pf.cs);
  load16_rs(rr, (rrow * 64 + 32 + 16 * (g16 & 1)) * 4, pf.sn);
}

// nw16: this lane's 16 gains; cs16 / sn16: cos / sin[(16 g16 + e) & 31] (lanes g16 < 4 use them)
__device__ __forceinline__ void qk_norm_rope(float* x, const float* nw16, float eps, int g16, const float* cs16,
                                             const float* sn16) {
  float ss = dot16_f32(x, x, 0.0f);
  ss = xor_sum<16>(ss);
  const float inv = 1.0f / sqrtf(ss / 256.0f + eps);
#pragma unroll
  for (int e = 0; e < 16; ++e) x[e] = (x[e] * inv) * (1.0f + nw16[e]);
  // rope.hpp:30-41 on dims 0..63 (lanes g16 = 0..3); partner dims +-32 live in lane g16 ^ 2
  float part[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) part[e] = xor_perm<2>(x[e]);
  if (g16 < 4) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float half = (g16 < 2) ? -part[e] : part[e];   // dims 0..31 take -x[i+32]
      x[e] = x[e] * cs16[e] + half * sn16[e];
    }
  }
}

// Contexts up to kAttnShortMax: unit (split s, kv head j) over the cached
// positions t0 .. min(t0 + 16, T) - 1; position T itself (the new K and V rows,
// attention.hpp:45-54) is a split of its own (attn_new_pos).  The poll of the
// query is issued first and the prefetch after it, so the poll does not queue
// behind the cache rows.
template <class IO>
__device__ __forceinline__ bool attn_unit(const AttnArgs& a, int s, int j, int T, int rrow, IO& io) {
  const int Tn = T;   // positions of this unit's split: < T
  const int lane = threadIdx.x & 63, g16 = lane & 15, pg = lane >> 4;
  const int i = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = 4 * j + i;                  // query head of this wave
  const int t0 = s * kAttnSplit;
  // qkv = q||gate (4096, interleaved per head) | k (512) | v (512): the query
  // (attention.hpp:40) as two 128-element regions
  constexpr int NR = 2;
  int reg[NR];
  reg[0] = h * 512;
  reg[1] = h * 512 + 128;
  const int iv[1] = {h * 512 + lane};   // (sampled while waiting: a query element)
  typename IO::template PollR<NR, 1> P;
  io.template pollr_issue<NR, 1>(a.qkv, reg, iv, P);
  AttnPre pf;
  attn_prefetch(a, s, j, T, rrow, pf);
  if (!io.wait()) return false;
  float* wa = wave_area();
  float unused[1];
  if (!io.template pollr_finish<NR, 1>(a.qkv, a.qkv_st, reg, iv, P, wa, unused)) return false;
  float t2[1][16];
  load16l(wa + 16 * g16, t2[0]);   // query dims 16 g16 .. + 15
  io.mark(1);   // trace: q received
  float* q = t2[0];
  qk_norm_rope(q, pf.qn, a.eps, g16, pf.cs, pf.sn);
  // scores of positions t0 + 4 it + pg (the same value in the 16 lanes of group pg)
  float sc[4], p[4];
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    float d = dot16_f32(q, pf.k[it], 0.0f);
    d = xor_sum<16>(d);
    sc[it] = t0 + 4 * it + pg < Tn ? d * 0.0625f : -__builtin_inff();
  }
  float m = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
  m = fmaxf(m, xor_perm<16>(m));
  m = fmaxf(m, xor_perm<32>(m));
#pragma unroll
  for (int it = 0; it < 4; ++it) p[it] = t0 + 4 * it + pg < Tn ? dev_expf(sc[it] - m) : 0.0f;
  // l: the 64-lane tree of p by position index (zeros past the split); pairs at
  // distance 8 and 4 are the registers it, it + 2 and it, it + 1 of one lane,
  // at distance 2 and 1 the lane groups pg ^ 2 (lane ^ 32) and pg ^ 1 (lane ^ 16)
  float l = (p[0] + p[2]) + (p[1] + p[3]);
  l = l + xor_perm<32>(l);
  l = l + xor_perm<16>(l);
  if (lane == 0) {
    io.st1(a.pm, a.part_st, h * a.nsplit_max + s, m);
    io.st1(a.pl, a.part_st, h * a.nsplit_max + s, l);
  }
  io.mark(2);   // trace: softmax of the split done
  // P.V in position order (attention.hpp:80-86); p of position u sits in lane 16 (u & 3), register u >> 2
  const int cnt = __builtin_amdgcn_readfirstlane(min(kAttnSplit, Tn - t0));
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int u = 0; u < kAttnSplit; ++u) {
    if (u < cnt) {
      const float pu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p[u >> 2]), 16 * (u & 3)));
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(pu, pf.v[u][e], acc[e]);
    }
  }
  io.st4(a.pacc, a.part_st, (h * a.nsplit_max + s) * 256 + 4 * lane, acc);
  return true;
}

// The new position T of kv head j, contexts up to kAttnShortMax: the last
// split (index sidx of the partials) with m = its score, l = 1 and acc = its V
// row.  Wave i takes query head 4 j + i: it fetches the query and the new K and
// V rows (six regions), normalises and rotates q and K (attention.hpp:39-50)
// and forms the score; wave 0 writes the new cache rows (attention.hpp:46-54).
template <class IO>
__device__ __forceinline__ bool attn_new_pos(const AttnArgs& a, int sidx, int j, int T, int rrow, IO& io) {
  constexpr int kBig = 0x7ffffff0;
  const int lane = threadIdx.x & 63, g16 = lane & 15, pg = lane >> 4;
  const int i = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = 4 * j + i;
  const int reg[6] = {h * 512, h * 512 + 128, 4096 + j * 256, 4096 + j * 256 + 128, 4608 + j * 256, 4608 + j * 256 + 128};
  const int iv[1] = {h * 512 + lane};
  typename IO::template PollR<6, 1> P;
  io.template pollr_issue<6, 1>(a.qkv, reg, iv, P);
  float qn16[16], kn16[16], cs16[16], sn16[16];
  load16_rs(rsrc_n(a.qn, kBig), 64 * g16, qn16);
  load16_rs(rsrc_n(a.kn, kBig), 64 * g16, kn16);
  {
    const __amdgpu_buffer_rsrc_t rr = rsrc_n(a.rope, kBig);
    load16_rs(rr, (rrow * 64 + 16 * (g16 & 1)) * 4, cs16);
    load16_rs(rr, (rrow * 64 + 32 + 16 * (g16 & 1)) * 4, sn16);
  }
  if (!io.wait()) return false;
  float* wa = wave_area();
  float unused[1];
  if (!io.template pollr_finish<6, 1>(a.qkv, a.qkv_st, reg, iv, P, wa, unused)) return false;
  float qv[16], kv[16], v4[4];
  load16l(wa + 16 * g16, qv);         // query dims 16 g16 .. + 15
  load16l(wa + 256 + 16 * g16, kv);   // new K row, same dims
  {
    const f32x4 t = *as_lds(reinterpret_cast<const f32x4*>(wa + 512 + 4 * lane));   // new V row, dims 4 lane ..
#pragma unroll
    for (int e = 0; e < 4; ++e) v4[e] = t[e];
  }
  io.mark(1);   // trace: q and the new k, v received
  qk_norm_rope(qv, qn16, a.eps, g16, cs16, sn16);
  qk_norm_rope(kv, kn16, a.eps, g16, cs16, sn16);
  if (i == 0) {
    if (pg == 0) stc16(a.kc, T * 512 + j * 256 + 16 * g16, kv);
    stc4(a.vc, T * 512 + j * 256 + 4 * lane, v4);
  }
  const float sc = xor_sum<16>(dot16_f32(qv, kv, 0.0f)) * 0.0625f;
  if (lane == 0) {
    io.st1(a.pm, a.part_st, h * a.nsplit_max + sidx, sc);
    io.st1(a.pl, a.part_st, h * a.nsplit_max + sidx, 1.0f);
  }
  io.mark(2);   // trace: score formed
  io.st4(a.pacc, a.part_st, (h * a.nsplit_max + sidx) * 256 + 4 * lane, v4);
  return true;
}

// ===========================================================================
// Long contexts (Tn = T + 1 > kAttnShortMax): splits of P = attn_split_len(Tn)
// positions.  Unit (split s, kv head j): wave w of the workgroup takes the
// iterations it = w, w + 4, ... of four positions t0 + 4 it + pg and computes
// all four query heads of kv head j on them, so a K or V row is read once per
// workgroup (and 2 / P of the cache bytes go to split partials).
//   pass 1  the K rows: the scores of (head, position) into LDS, and the
//           wave's maximum m_w per head;
//   pass 2  the V rows in the wave's position order (k ascending, then pg):
//           p = exp(s - m_w), l_w = l_w + p, acc_w = fma(p, v, acc_w);
//   merge   M = max m_w, e_w = exp(m_w - M) (0 for a wave without positions),
//           l = (l0 e0 + l1 e1) + (l2 e2 + l3 e3), acc the same; wave w stores
//           the partial of query head 4 j + w.
// Every wave runs kw iterations (the split's iterations per wave, rounded up to
// a multiple of kAttnLongD, the same for all four waves).  A position at or past
// the split's end has the score -inf and p = 0; its K / V loads re-read the
// split's last row, and fma(0, v, acc) and l + 0 leave acc and l unchanged.
// The loads stay straight-line: each unrolled step uses the rows loaded
// kAttnLongD steps earlier and issues the loads of kAttnLongD steps later.
// ===========================================================================
// Iterations of K rows in flight per wave (V: 4 rows per iteration).  Two:
// the C3 layer at T = 32768 took 47.6 us with 2, 48.4 with 3, 50.1 with 4 and
// 56.2 with 8 (each wave's iterations are padded to a multiple of this, and
// the padded steps still read rows), 50.8 with 1.
constexpr int kAttnLongD = 2;

template <bool OWNER, class IO>
__device__ __forceinline__ bool attn_unit_long(const AttnArgs& a, int s, int j, int T, int rrow, IO& io) {
  constexpr int D = kAttnLongD;
  constexpr int kBig = 0x7ffffff0;
  const int Tn = T + 1;
  const int P = attn_split_len(Tn);
  const int lane = threadIdx.x & 63, g16 = lane & 15, pg = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = 4 * j + w;   // the query head this wave normalises, and stores after the merge
  const int t0 = s * P, t1 = min(t0 + P, Tn), tlast = t1 - 1;
  const int nit = (t1 - t0 + 3) >> 2;                     // iterations of the split
  const int kw = ((nit + 3) / 4 + D - 1) / D * D;         // per wave, padded
  // inputs: the query of head h (two 128-element regions); the owner also takes
  // the new K and V rows of kv head j (two regions each), as the short unit
  constexpr int NR = OWNER ? 6 : 2;
  int reg[NR];
  reg[0] = h * 512;
  reg[1] = h * 512 + 128;
  if constexpr (OWNER) {
    reg[2] = 4096 + j * 256;
    reg[3] = 4096 + j * 256 + 128;
    reg[4] = 4608 + j * 256;
    reg[5] = 4608 + j * 256 + 128;
  }
  const int iv[1] = {h * 512 + lane};
  typename IO::template PollR<NR, 1> Pq;
  io.template pollr_issue<NR, 1>(a.qkv, reg, iv, Pq);
  const __amdgpu_buffer_rsrc_t rk = rsrc_n(a.kc, kBig);
  const __amdgpu_buffer_rsrc_t rv = rsrc_n(a.vc, kBig);
  auto row = [&](int k, int u) { return min(t0 + 4 * (w + 4 * k) + u, tlast); };   // position, clamped
  float kb[D][16];   // K: 16 dims (16 g16 ..) of position t0 + 4 (w + 4 k) + pg
#pragma unroll
  for (int d = 0; d < D; ++d) load16_rs(rk, (row(d, pg) * 512 + j * 256 + 16 * g16) * 4, kb[d]);
  float qn16[16], kn16[16], cs16[16], sn16[16];
  load16_rs(rsrc_n(a.qn, kBig), 64 * g16, qn16);
  load16_rs(rsrc_n(a.kn, kBig), 64 * g16, kn16);
  {
    const __amdgpu_buffer_rsrc_t rr = rsrc_n(a.rope, kBig);
    load16_rs(rr, (rrow * 64 + 16 * (g16 & 1)) * 4, cs16);
    load16_rs(rr, (rrow * 64 + 32 + 16 * (g16 & 1)) * 4, sn16);
  }
  if (!io.wait()) return false;
  float* wa = wave_area();
  float unused[1];
  if (!io.template pollr_finish<NR, 1>(a.qkv, a.qkv_st, reg, iv, Pq, wa, unused)) return false;
  float qh[16], knew[16], vnew[4];
  load16l(wa + 16 * g16, qh);
  if constexpr (OWNER) {
    load16l(wa + 256 + 16 * g16, knew);
    const f32x4 t = *as_lds(reinterpret_cast<const f32x4*>(wa + 512 + 4 * lane));
#pragma unroll
    for (int e = 0; e < 4; ++e) vnew[e] = t[e];
    qk_norm_rope(knew, kn16, a.eps, g16, cs16, sn16);
    if (w == 0) {   // wave 0 writes the new cache rows
      if (pg == 0) stc16(a.kc, T * 512 + j * 256 + 16 * g16, knew);
      stc4(a.vc, T * 512 + j * 256 + 4 * lane, vnew);
    }
  }
  io.mark(1);   // trace: q (and the new k, v) received
  qk_norm_rope(qh, qn16, a.eps, g16, cs16, sn16);
  // the four normalised queries meet in LDS
  float* ql = io.slot();   // [4 heads][256]
  float* sc = io.slot();   // [4 waves][4 heads][4 kw]: scores, then p
  if (pg == 0) {
#pragma unroll
    for (int e = 0; e < 16; e += 4)
      *as_lds_w(reinterpret_cast<f32x4*>(ql + w * 256 + 16 * g16 + e)) = f32x4{qh[e], qh[e + 1], qh[e + 2], qh[e + 3]};
  }
  lds_barrier();
  float q[4][16];
#pragma unroll
  for (int hh = 0; hh < 4; ++hh) load16l(ql + hh * 256 + 16 * g16, q[hh]);
  // ---- pass 1: scores and the wave's maxima
  float m[4] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
  float* scw = sc + w * 16 * kw;
  for (int k0 = 0; k0 < kw; k0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int k = k0 + d;
      const int t = t0 + 4 * (w + 4 * k) + pg;
      float kv[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) kv[e] = kb[d][e];
      if constexpr (OWNER) {
        const bool sel = t == T;
#pragma unroll
        for (int e = 0; e < 16; ++e) kv[e] = sel ? knew[e] : kv[e];
      }
      load16_rs(rk, (row(k + D, pg) * 512 + j * 256 + 16 * g16) * 4, kb[d]);   // k + D (clamped)
#pragma unroll
      for (int hh = 0; hh < 4; ++hh) {
        float dd = dot16_f32(q[hh], kv, 0.0f);
        dd = xor_sum<16>(dd);
        const float sv = t < t1 ? dd * 0.0625f : -__builtin_inff();
        m[hh] = fmaxf(m[hh], sv);
        if (g16 == hh) as_lds_w(scw)[(hh * kw + k) * 4 + pg] = sv;
      }
    }
  }
#pragma unroll
  for (int hh = 0; hh < 4; ++hh) {
    m[hh] = fmaxf(m[hh], xor_perm<16>(m[hh]));
    m[hh] = fmaxf(m[hh], xor_perm<32>(m[hh]));
  }
  // ---- V rows of the first D iterations, then p of this wave's positions (lane-parallel)
  float vb[D][4][4];
#pragma unroll
  for (int d = 0; d < D; ++d)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(rv, (row(d, u) * 512 + j * 256 + 4 * lane) * 4, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) vb[d][u][e] = __uint_as_float(t[e]);
    }
#pragma unroll
  for (int hh = 0; hh < 4; ++hh)
    for (int i = lane; i < 4 * kw; i += 64) {
      auto* c = as_lds_w(scw) + hh * 4 * kw + i;
      const float sv = *c;
      *c = sv == -__builtin_inff() ? 0.0f : dev_expf(sv - m[hh]);   // past the split's end: 0 (m may be -inf)
    }
  // ---- pass 2: p . V in the wave's position order
  float acc[4][4], l[4];
#pragma unroll
  for (int hh = 0; hh < 4; ++hh) {
    l[hh] = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[hh][e] = 0.0f;
  }
  for (int k0 = 0; k0 < kw; k0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int k = k0 + d;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int t = t0 + 4 * (w + 4 * k) + u;
        float vv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) vv[e] = vb[d][u][e];
        if constexpr (OWNER) {
          const bool sel = t == T;
#pragma unroll
          for (int e = 0; e < 4; ++e) vv[e] = sel ? vnew[e] : vv[e];
        }
        const u32x4 nv =
            __builtin_amdgcn_raw_buffer_load_b128(rv, (row(k + D, u) * 512 + j * 256 + 4 * lane) * 4, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) vb[d][u][e] = __uint_as_float(nv[e]);
#pragma unroll
        for (int hh = 0; hh < 4; ++hh) {
          const float pu = as_lds(scw)[(hh * kw + k) * 4 + u];
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[hh][e] = __builtin_fmaf(pu, vv[e], acc[hh][e]);
          l[hh] = l[hh] + pu;
        }
      }
    }
  }
  // the last refills re-read the split's last row: read (they returned with the rows used above)
#pragma unroll
  for (int d = 0; d < D; ++d) {
#pragma unroll
    for (int e = 0; e < 16; ++e) settle(kb[d][e]);
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) settle(vb[d][u][e]);
  }
  // ---- merge of the four waves: heads 0, 1 in one slot, heads 2, 3 in the next
  float* mg[2];
  mg[0] = io.slot();
  mg[1] = io.slot();
#pragma unroll
  for (int hh = 0; hh < 4; ++hh) {
    float* r = mg[hh >> 1];
    const int hl = hh & 1;
    *as_lds_w(reinterpret_cast<f32x4*>(r + 16 + (w * 2 + hl) * 256 + 4 * lane)) =
        f32x4{acc[hh][0], acc[hh][1], acc[hh][2], acc[hh][3]};
    if (lane == 0) {
      as_lds_w(r)[(w * 2 + hl) * 2] = m[hh];
      as_lds_w(r)[(w * 2 + hl) * 2 + 1] = l[hh];
    }
  }
  lds_barrier();
  {
    const float* r = mg[w >> 1];
    const int hl = w & 1;
    float mw[4], lw[4], ew[4];
    float M = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      mw[i] = as_lds(r)[(i * 2 + hl) * 2];
      lw[i] = as_lds(r)[(i * 2 + hl) * 2 + 1];
      M = fmaxf(M, mw[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) ew[i] = mw[i] == -__builtin_inff() ? 0.0f : dev_expf(mw[i] - M);
    const float L = (lw[0] * ew[0] + lw[1] * ew[1]) + (lw[2] * ew[2] + lw[3] * ew[3]);
    float A[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 t = *as_lds(reinterpret_cast<const f32x4*>(r + 16 + (i * 2 + hl) * 256 + 4 * lane));
#pragma unroll
      for (int e = 0; e < 4; ++e) A[i][e] = t[e];
    }
    float out[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = (A[0][e] * ew[0] + A[1][e] * ew[1]) + (A[2][e] * ew[2] + A[3][e] * ew[3]);
    if (lane == 0) {
      io.st1(a.pm, a.part_st, h * a.nsplit_max + s, M);
      io.st1(a.pl, a.part_st, h * a.nsplit_max + s, L);
    }
    io.mark(2);   // trace: the split's partials merged
    io.st4(a.pacc, a.part_st, (h * a.nsplit_max + s) * 256 + 4 * lane, out);
  }
  return true;
}

// Units u = blk, blk + nblk, ... of the 2 * ceil((T+1)/16) splits; T is the slot
// of this token (past tokens = T).
// LONG = false leaves the long-context unit out of a kernel whose cache never holds more than
// kAttnShortMax positions (its registers would otherwise weigh on the whole kernel); such a kernel
// refuses a longer context (false: the launch's failure path).
template <class IO, bool LONG = true>
__device__ __forceinline__ bool attn_body(const AttnArgs& a, int T, int blk, int nblk, IO& io) {
  const bool ok = T >= 0 && T < a.max_ctx;
  const bool lng = T + 1 > kAttnShortMax;
  const int ns = ok ? attn_nsplit(T + 1) : 0;   // short contexts: the last split is position T alone
  const int units = 2 * ns;
  io.arrive();
  if (!LONG && T + 1 > kAttnShortMax) return false;
  // units from the last workgroup down: in the persistent kernel the q, k, v
  // rows of the stage before run on the first workgroups, so the units'
  // workgroups enter this stage (and issue their cache loads) early
  const int r = nblk - 1 - blk;
  if (r >= units) return true;
  io.mark(0);   // trace: stage entry
  const int rrow = a.rope_row != nullptr ? ldc_i(a.rope_row) : T;
  for (int u = r; u < units; u += nblk) {
    bool done = false;
    if (LONG && lng) {
      if constexpr (LONG) {
        const int s = u >> 1, j = u & 1;
        const bool own = s == ns - 1;   // slot T lies in the last split
        done = own ? attn_unit_long<true>(a, s, j, T, rrow, io) : attn_unit_long<false>(a, s, j, T, rrow, io);
      }
    } else if (u < 2) {   // the new position's split (units 0, 1: the most idle workgroups)
      done = attn_new_pos(a, ns - 1, u, T, rrow, io);
    } else {
      done = attn_unit(a, (u - 2) >> 1, u & 1, T, rrow, io);
    }
    if (!done) return false;
  }
  return true;
}

// Merge the splits of head h in split order; output gate (attention.hpp:89-92).
// Workgroup (h, q) = blk / 4, blk % 4 owns dimensions 64 q .. 64 q + 63: its
// four waves fetch the partial sums of interleaved splits into LDS (a wave
// fetches few lines of freshly written partials, which is what the wait
// costs), then wave 0 folds them in split order, one dimension per lane.
constexpr int kCombineWGs = 32;
constexpr int kCombineChunk = 32;   // splits per LDS round (8 per wave)
// Long contexts (at most kAttnMaxSplits splits up to 65536 positions): the
// same workgroups, but wave w folds the contiguous quarter of the splits
// [w c, (w + 1) c), c = ceil(ns / 4), in split order (L_w = L_w + l_s e_s,
// ctx_w = ctx_w + acc_s e_s, e_s = exp(m_s - M), M the maximum over all
// splits), and the quarters meet in LDS as (q0 + q1) + (q2 + q3).
constexpr int kCombineLongPer = 32;   // splits per wave per round
template <class IO>
__device__ __forceinline__ bool combine_long(const AttnArgs& a, int T, int blk, IO& io) {
  const int h = blk >> 2, q = blk & 3;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int d = 64 * q + lane;
  const int ns = attn_nsplit(T + 1);
  const int base = h * a.nsplit_max;
  const int c = (ns + 3) / 4;
  const int s0 = min(wave * c, ns), s1 = min(s0 + c, ns);
  const Raw graw = io.issue1(a.qkv, h * 512 + 256 + d, wave == 0);   // the output gate of dimension d
  float M = -__builtin_inff();   // over every split (each wave: the same value)
  for (int b0 = 0; b0 < ns; b0 += 64) {
    float mv;
    if (!io.ld1(a.pm, a.part_st, base + min(b0 + lane, ns - 1), mv)) return false;
    M = fmaxf(M, xor_max<64>(mv));
  }
  float L = 0.0f, ctx = 0.0f;
  for (int r0 = s0; r0 < s1; r0 += kCombineLongPer) {
    const int n = min(kCombineLongPer, s1 - r0);
    int ia[kCombineLongPer];
    float pa[kCombineLongPer];
#pragma unroll
    for (int k = 0; k < kCombineLongPer; ++k) ia[k] = (base + r0 + min(k, n - 1)) * 256 + d;
    if (!io.template ldn<kCombineLongPer>(a.pacc, a.part_st, ia, pa)) return false;
    float mv, lv;
    const int sl = base + r0 + min(lane, n - 1);
    if (!io.ld1(a.pm, a.part_st, sl, mv) || !io.ld1(a.pl, a.part_st, sl, lv)) return false;
    const float e = dev_expf(mv - M);   // split r0 + lane
#pragma unroll
    for (int k = 0; k < kCombineLongPer; ++k) {
      if (k < n) {
        const float ek = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), k));
        const float lk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lv), k));
        L = L + lk * ek;
        ctx = ctx + pa[k] * ek;
      }
    }
  }
  float* buf = io.slot();   // [4 waves]: L at 0, ctx at 4 + 64 w
  as_lds_w(buf)[4 + 64 * wave + lane] = ctx;
  if (lane == 0) as_lds_w(buf)[wave] = L;
  lds_barrier();
  if (wave != 0) {
    settle(graw.v), settle(graw.t);
    return true;
  }
  const float Ls = (as_lds(buf)[0] + as_lds(buf)[1]) + (as_lds(buf)[2] + as_lds(buf)[3]);
  const float cs = (as_lds(buf)[4 + lane] + as_lds(buf)[68 + lane]) + (as_lds(buf)[132 + lane] + as_lds(buf)[196 + lane]);
  io.mark(1);   // trace: all split partials folded
  const float invL = 1.0f / Ls;
  float gate;
  if (!io.resolve1(graw, a.qkv, a.qkv_st, h * 512 + 256 + d, gate)) return false;
  io.st1(a.og, a.og_st, h * 256 + d, (cs * invL) * dev_sigmoid(gate));
  return true;
}

template <class IO, bool LONG = true>
__device__ __forceinline__ bool combine_body(const AttnArgs& a, int T, int blk, IO& io) {
  io.arrive();
  io.mark(0);   // trace: stage entry
  if (!io.wait()) return false;
  if (!LONG && T + 1 > kAttnShortMax) return false;
  if (blk >= kCombineWGs || T < 0 || T >= a.max_ctx) return true;
  if constexpr (LONG)
    if (T + 1 > kAttnShortMax) return combine_long(a, T, blk, io);
  const int h = blk >> 2, q = blk & 3;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int d = 64 * q + lane;
  const int ns = attn_nsplit(T + 1);   // the last split is position T alone
  const int base = h * a.nsplit_max;
  const Raw graw = io.issue1(a.qkv, h * 512 + 256 + d, wave == 0);   // the output gate of dimension d
  float* buf = io.slot();   // [kCombineChunk splits][64 dimensions]
  float M = -__builtin_inff();
  if (wave == 0) {
    for (int s0 = 0; s0 < ns; s0 += 64) {
      float mv;
      if (!io.ld1(a.pm, a.part_st, base + min(s0 + lane, ns - 1), mv)) return false;
      M = fmaxf(M, xor_max<64>(mv));
    }
  }
  float L = 0.0f, ctx = 0.0f;
  constexpr int kPer = kCombineChunk / 4;
  for (int s0 = 0; s0 < ns; s0 += kCombineChunk) {
    const int n = min(kCombineChunk, ns - s0);
    {   // splits s0 + wave + 4 k of this chunk
      int ia[kPer];
      float pa[kPer];
#pragma unroll
      for (int k = 0; k < kPer; ++k) ia[k] = (base + s0 + min(wave + 4 * k, n - 1)) * 256 + d;
      if (!io.template ldn<kPer>(a.pacc, a.part_st, ia, pa)) return false;
#pragma unroll
      for (int k = 0; k < kPer; ++k)
        if (wave + 4 * k < n) buf[(wave + 4 * k) * 64 + lane] = pa[k];
    }
    __syncthreads();
    if (wave == 0) {
      float mv, lv;
      const int sl = base + s0 + min(lane, n - 1);
      if (!io.ld1(a.pm, a.part_st, sl, mv) || !io.ld1(a.pl, a.part_st, sl, lv)) return false;
      const float e = dev_expf(mv - M);   // split s0 + lane
      for (int c = 0; c < n; ++c) {
        const float ec = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), c));
        const float lc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lv), c));
        L = L + lc * ec;
        ctx = ctx + buf[c * 64 + lane] * ec;
      }
    }
    __syncthreads();
  }
  if (wave != 0) return true;
  io.mark(1);   // trace: all split partials folded
  const float invL = 1.0f / L;
  float gate;
  if (!io.resolve1(graw, a.qkv, a.qkv_st, h * 512 + 256 + d, gate)) return false;
  io.st1(a.og, a.og_st, h * 256 + d, (ctx * invL) * dev_sigmoid(gate));
  return true;
}

}  // namespace qh
