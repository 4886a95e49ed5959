// Persistent decode kernel: one cooperative launch runs whole tokens -- every
// stage of every layer, the LM head, the argmax and the run_hls generation
// bookkeeping (run_hls.cpp:56-66) -- with a grid barrier between dependent
// stages instead of a kernel boundary.
//
// A workgroup arrives at the barrier as soon as its stores of stage k have
// completed, then issues stage k+1's first weight (and own-state) loads, then
// waits: HBM streaming and descriptor reads overlap the barrier latency.
// Consumers read handed-over activations with device-coherent loads
// (qh_device.hpp ldc*).
#include "qh_stages.hpp"

namespace qh {

namespace {

constexpr unsigned kSpinLimit = 1u << 21;   // ~1 s of polling: a barrier that never fills aborts

struct GridBar {
  unsigned* cnt;
  int* abort_flag;
  int blk, nblk;
  unsigned gen;
  int* s_stop;   // LDS: this workgroup saw an abort
  uint64_t* trace;
  unsigned trace_bars;

  // All waves' stores have completed (each wave waits for its own), then one
  // arrival per workgroup on counter blk % kBarCounters.
  __device__ __forceinline__ void arrive() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    ++gen;
    if (threadIdx.x == 0) {
      if (trace != nullptr && gen <= trace_bars)
        trace[((size_t)(gen - 1) * nblk + blk) * 2] = __builtin_amdgcn_s_memrealtime();
      __hip_atomic_fetch_add(cnt + (blk % kBarCounters) * kBarStride, 1u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  // Every counter has its workgroups of this generation; false after an abort.
  __device__ __forceinline__ bool wait() {
    const int t = threadIdx.x;
    if (t < kBarCounters) {
      const unsigned target = gen * (unsigned)(nblk / kBarCounters);
      const unsigned* c = cnt + t * kBarStride;
      unsigned spins = 0;
      while (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
        if ((++spins & 255u) == 0) {
          if (spins > kSpinLimit) {
            stc_i(abort_flag, 1);
            *s_stop = 1;
            break;
          }
          if (ldc_i(abort_flag) != 0) {
            *s_stop = 1;
            break;
          }
        }
      }
    }
    __syncthreads();
    if (trace != nullptr && t == 0 && gen <= trace_bars)
      trace[((size_t)(gen - 1) * nblk + blk) * 2 + 1] = __builtin_amdgcn_s_memrealtime();
    return *s_stop == 0;
  }
};

}  // namespace

template <int MODE>
__global__ __launch_bounds__(kPersistThreads) void persist_kernel(const PersistArgs P) {
  __shared__ int s_stop;
  __shared__ float s_bv[kPersistThreads / 64];
  __shared__ int s_bi[kPersistThreads / 64];
  const int blk = blockIdx.x, nblk = gridDim.x;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  if (t == 0) s_stop = 0;
  __syncthreads();
  GridBar bar{P.bar, P.abort_flag, blk, nblk, 0u, &s_stop, P.trace, (unsigned)P.trace_bars};

  // block-local copy of the generation state; every workgroup makes the same decisions
  int tok = P.ctl->tok, pos = P.ctl->pos, step = P.ctl->step, n_out = P.ctl->n_out;
  const int n_prompt = P.ctl->n_prompt, n_new = P.ctl->n_new, eos = P.ctl->eos, max_ctx = P.ctl->max_ctx;
  int argmax = P.ctl->argmax, done = 0, err = 0;

  while (true) {
    for (int i = 0; i < P.nstage; ++i) {
      const Stage& st = P.prog[i];
      switch (st.kind) {
        case ST_GEMV_NORM_1x8: gemv_body<1, MODE, P_NORM, 8>(st.g, blk, nblk, bar, tok); break;
        case ST_GEMV_GATED_2x4: gemv_body<2, MODE, P_GATED, 4>(st.g, blk, nblk, bar, tok); break;
        case ST_GEMV_LOAD_2x4: gemv_body<2, MODE, P_LOAD, 4>(st.g, blk, nblk, bar, tok); break;
        case ST_GEMV_LOAD_4x4: gemv_body<4, MODE, P_LOAD, 4>(st.g, blk, nblk, bar, tok); break;
        case ST_DELTANET: deltanet_all(st.d, blk, nblk, bar, tok); break;
        case ST_ATTN: attn_body(st.at, pos, blk, nblk, bar); break;
        case ST_COMBINE: combine_body(st.at, pos, blk, bar); break;
        default: head_body(st.hd, blk, nblk, bar, P.logits); break;
      }
      if (s_stop) break;
    }
    if (s_stop) break;
    // argmax over the LM-head partials (qwen_synth.hpp:81-88), then ++pos (:90)
    bar.arrive();
    if (!bar.wait()) break;
    float bv = -1e30f;
    int bi = 0;
    for (int b = t; b < nblk; b += kPersistThreads) better(bv, bi, ldc(P.part_val + b), ldc_i(P.part_idx + b));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const int oi = __shfl_xor(bi, off, 64);
      better(bv, bi, ov, oi);
    }
    if (lane == 0) {
      s_bv[wave] = bv;
      s_bi[wave] = bi;
    }
    __syncthreads();
    bv = s_bv[0];
    bi = s_bi[0];
    for (int w2 = 1; w2 < kPersistThreads / 64; ++w2) better(bv, bi, s_bv[w2], s_bi[w2]);
    __syncthreads();
    argmax = bi;
    pos += 1;
    // run_hls.cpp:56-66: feed the prompt, then each greedy argmax until n_new or eos
    const int next = step + 1;
    if (next < n_prompt) {
      tok = P.prompt[next];
      step = next;
    } else if (n_out >= n_new || argmax == eos) {
      done = 1;
    } else {
      if (blk == 0 && t == 0) P.out_ids[n_out] = argmax;
      n_out += 1;
      tok = argmax;
      step = next;
      if (pos >= max_ctx) {
        done = 1;
        err = 2;
      }
    }
    if (done) break;
  }
  if (blk == 0 && t == 0) {
    StepCtl* c = P.ctl;
    c->tok = tok;
    c->pos = pos;
    c->argmax = argmax;
    c->step = step;
    c->n_out = n_out;
    c->done = done;
    c->err = s_stop ? 3 : err;
  }
}

int persist_max_grid(int* grid) {
  int dev = 0, ncu = 0, coop = 0, occ = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess || !coop) return -1;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, persist_kernel<M_W8A16>, kPersistThreads, 0) !=
      hipSuccess)
    return -1;
  int occ2 = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ2, persist_kernel<M_W8A8>, kPersistThreads, 0) !=
      hipSuccess)
    return -1;
  occ = occ < occ2 ? occ : occ2;
  if (occ < 1) return -1;
  int g = ncu < 256 ? ncu : 256;   // one workgroup per CU
  g -= g % kBarCounters;
  if (g < kBarCounters) return -1;
  *grid = g;
  return 0;
}

hipError_t launch_persist(const PersistArgs& a, int grid, hipStream_t s) {
  if (grid < kBarCounters || grid % kBarCounters != 0) return hipErrorInvalidValue;
  void* args[] = {const_cast<PersistArgs*>(&a)};
  const void* fn = a.mode == M_W8A8 ? reinterpret_cast<const void*>(persist_kernel<M_W8A8>)
                                    : reinterpret_cast<const void*>(persist_kernel<M_W8A16>);
  return hipLaunchCooperativeKernel(fn, dim3(grid), dim3(kPersistThreads), args, 0, s);
}

}  // namespace qh
