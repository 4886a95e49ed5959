// Persistent decode kernel: one cooperative launch runs whole tokens -- every
// stage of every layer, the LM head, the argmax and the run_hls generation
// bookkeeping (run_hls.cpp:56-66).  There is no grid barrier: workgroups hand
// vectors to one another through tagged buffers (TagIO in qh_stages.hpp), so
// each one waits only for the inputs of its own next work item.  A workgroup
// that finishes a stage at once issues the next stage's first input poll and,
// right behind it, that stage's weight (and own-state) loads: the weights
// stream while the hand-over is awaited, and since a wave's loads return in
// issue order, the poll is never queued behind them.
//
// Every stage writes its own buffers (the engine gives each stage of the
// token program distinct output vectors), so within a token no buffer is
// written twice.  Across tokens, a stage rewrites its buffers only after the
// argmax of the previous token, which every workgroup computes from the head
// partials of all workgroups -- by then every workgroup has finished every
// stage of the previous token, including its reads.
#include "qh_decode.h"
#include "qh_stages.hpp"

namespace qh {

// The stage bodies read their descriptors from a workgroup copy in LDS: read
// from the program in global memory, every descriptor field would be a vector
// load whose wait also waits for every load and store issued before it.  The
// copy of stage i + 1 is loaded (one word per thread) at the start of stage i,
// ahead of that stage's own loads, and written to the other of two LDS slots
// at stage i's first tag check (TagIO::desc_put), or at the start of stage
// i + 1 by a thread that checked no tag in stage i; then one LDS-only
// workgroup barrier.  A slot is rewritten one stage after it was read: every
// wave has passed the barrier at the start of the stage in between, so no
// wave still reads it.  No global memory is exchanged through the barrier:
// the stage stores stay in flight into the next stage (their consumers poll
// tags), and the head stage orders the token's stores before its partials.
constexpr int kStageWords = (int)(sizeof(Stage) / 4);
static_assert(sizeof(Stage) % 4 == 0 && kStageWords <= kPersistThreads, "one descriptor word per thread");

// A wave that gave up a hand-over wait (TagIO::failed) finishes its stage with
// stale values; at the next stage boundary it raises the workgroup's failure
// flag in LDS, and after the boundary barrier every wave reads it and the
// workgroup leaves the launch as one -- no wave dispatches a stage whose
// descriptor an exited wave did not copy.  The flag is double-buffered like
// the descriptors: slot p is written before the barrier of a boundary and read
// after it, and written again only two boundaries later.
template <int MODE, bool LONG>
__global__ __launch_bounds__(kPersistThreads) void persist_kernel(const PersistArgs P) {
  __shared__ float s_bv[kPersistThreads / 64];
  __shared__ int s_bi[kPersistThreads / 64];
  __shared__ __attribute__((aligned(16))) uint32_t s_stage[2][kStageWords];
  __shared__ int s_fail[2];
  const int blk = blockIdx.x, nblk = gridDim.x;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  TagIO io;
  io.abort_flag = P.abort_flag;
  io.poll_limit = P.poll_limit;
  if (t < 2) s_fail[t] = 0;   // first read after the first stage barrier

  // block-local copy of the generation state; every workgroup makes the same decisions
  int tok = P.ctl->tok, pos = P.ctl->pos, step = P.ctl->step, n_out = P.ctl->n_out;
  const int n_prompt = P.ctl->n_prompt, n_new = P.ctl->n_new, eos = P.ctl->eos, max_ctx = P.ctl->max_ctx;
  int argmax = P.ctl->argmax, done = 0, err = 0, aborted = 0;
  const HeadArgs& hd = P.prog[P.nstage - 1].hd;
  if (P.dn_lds) dn_tiles_copy(P.prog, P.nstage, blk, nblk, true);   // this workgroup's DeltaNet state tiles

  const uint32_t* progw = reinterpret_cast<const uint32_t*>(P.prog);
  io.desc_next(progw, s_stage[0], kStageWords);   // descriptor of stage 0
  int slot = 0;
  for (int k = 0;; ++k) {
    io.tag0 = P.tag_base + (uint32_t)k * (uint32_t)kTagsPerToken;
    for (int i = 0; i < P.nstage; ++i) {
      io.desc_put();   // (a thread that checked no tag in the previous stage)
      if (io.failed) s_fail[slot] = 1;
      lds_barrier();
      if (s_fail[slot] != 0) {   // workgroup-uniform: read after the barrier
        aborted = 1;
        break;
      }
      const Stage& st = *reinterpret_cast<const Stage*>(s_stage[slot]);
      slot ^= 1;
      const int ni = i + 1 < P.nstage ? i + 1 : 0;   // the next stage (stage 0 after the head)
      io.desc_next(progw + (size_t)ni * kStageWords, s_stage[slot], kStageWords);
      asm volatile("" ::: "memory");   // issued before any load of this stage
      uint64_t* tr = (P.trace != nullptr && k < P.trace_tokens) ? P.trace + (((size_t)k * P.nstage + i) * nblk + blk) * kTraceSlots : nullptr;
      io.tr = tr;
      bool ok;
      switch (st.kind) {
        // the vector length and epilogues of each GEMV stage kind are fixed (the engine checks its program)
        case ST_GEMV_NORM_1x8: ok = gemv_body<1, MODE, P_NORM, 8, QH_HIDDEN, kEmInProj>(st.g, blk, nblk, io, tok); break;
        case ST_GEMV_QKV_1x8: ok = gemv_body<1, MODE, P_NORM, 8, QH_HIDDEN, kEmStore>(st.g, blk, nblk, io, tok); break;
        case ST_GEMV_GATEUP_1x8:
          ok = gemv_body<1, MODE, P_NORM, 8, QH_HIDDEN, kEmSwiglu>(st.g, blk, nblk, io, tok);
          break;
        // W8A8 1024-row projections: the vector split over the four waves (same values)
        case ST_GEMV_GATED_2x1:
          if (MODE == M_W8A8 && gemv_splitk_ok(st.g, nblk, kPersistThreads / 64))
            ok = gemv_splitk<2, P_GATED, QH_LH * QH_LV>(st.g, blk, io);
          else
            ok = gemv_body<2, MODE, P_GATED, 1, QH_LH * QH_LV, kEmResid>(st.g, blk, nblk, io, tok);
          break;
        case ST_GEMV_LOAD_2x1:
          if (MODE == M_W8A8 && gemv_splitk_ok(st.g, nblk, kPersistThreads / 64))
            ok = gemv_splitk<2, P_LOAD, QH_NH * QH_HD>(st.g, blk, io);
          else
            ok = gemv_body<2, MODE, P_LOAD, 1, QH_NH * QH_HD, kEmResid>(st.g, blk, nblk, io, tok);
          break;
        case ST_GEMV_LOAD_4x1:
          if (MODE == M_W8A8 && gemv_splitk_ok(st.g, nblk, kPersistThreads / 64))
            ok = gemv_splitk<4, P_LOAD, QH_INTER>(st.g, blk, io);
          else
            ok = gemv_body<4, MODE, P_LOAD, 1, QH_INTER, kEmResid>(st.g, blk, nblk, io, tok);
          break;
        case ST_DELTANET: ok = deltanet_all(st.d, blk, nblk, io, tok); break;
        case ST_ATTN: ok = attn_body<TagIO, LONG>(st.at, pos, blk, nblk, io); break;
        case ST_COMBINE: ok = combine_body<TagIO, LONG>(st.at, pos, blk, io); break;
        default: ok = head_body<false>(st.hd, blk, nblk, io, P.logits); break;
      }
      if (tr != nullptr && t == 0) tr[kTraceSlots - 1] = __builtin_amdgcn_s_memrealtime();
      if (!ok) io.failed = true;   // the stage body refused its arguments: same exit
    }
    if (aborted) break;
    // argmax over the LM-head partials of all workgroups (qwen_synth.hpp:81-88), then ++pos (:90)
    float bv = -1e30f;
    int bi = 0;
    {
      float* pv = io.slot();
      float* pi = io.slot();
      // (a failed wait here is noticed at the next stage boundary, or by the host)
      io.stage_vec(hd.part_val, hd.part_st, nblk, pv);
      io.stage_vec(reinterpret_cast<const float*>(hd.part_idx), hd.part_st, nblk, pi);
      for (int b = t; b < nblk; b += kPersistThreads) better(bv, bi, pv[b], __float_as_int(pi[b]));
    }
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
    argmax = min(max(bi, 0), hd.rows - 1);   // a stale partial (after a failed wait) stays an index
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
  if (P.dn_lds) dn_tiles_copy(P.prog, P.nstage, blk, nblk, false);   // the state back to its buffer
  if (blk == 0 && t == 0) {
    StepCtl* c = P.ctl;
    c->tok = tok;
    c->pos = pos;
    c->argmax = argmax;
    c->step = step;
    c->n_out = n_out;
    c->done = done;
    c->err = aborted ? 3 : err;
  }
}

int persist_max_grid(int* grid) {
  int dev = 0, ncu = 0, coop = 0, occ = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess || !coop) return -1;
  const void* fns[] = {reinterpret_cast<const void*>(persist_kernel<M_W8A16, false>),
                       reinterpret_cast<const void*>(persist_kernel<M_W8A8, false>),
                       reinterpret_cast<const void*>(persist_kernel<M_W8A16, true>),
                       reinterpret_cast<const void*>(persist_kernel<M_W8A8, true>)};
  occ = 1 << 30;
  for (const void* fn : fns) {
    int o = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, fn, kPersistThreads, 0) != hipSuccess) return -1;
    occ = o < occ ? o : occ;
  }
  if (occ < 1) return -1;
  int g = ncu < 256 ? ncu : 256;   // one workgroup per CU
  g -= g & 1;                      // the head partials are copied as pairs
  if (g < 2) return -1;
  *grid = g;
  return 0;
}

hipError_t launch_persist(const PersistArgs& a, int grid, hipStream_t s) {
  if (grid < 1 || grid > 256) return hipErrorInvalidValue;
  void* args[] = {const_cast<PersistArgs*>(&a)};
  const void* fn = a.long_ctx ? (a.mode == M_W8A8 ? reinterpret_cast<const void*>(persist_kernel<M_W8A8, true>)
                                                   : reinterpret_cast<const void*>(persist_kernel<M_W8A16, true>))
                             : (a.mode == M_W8A8 ? reinterpret_cast<const void*>(persist_kernel<M_W8A8, false>)
                                                 : reinterpret_cast<const void*>(persist_kernel<M_W8A16, false>));
  return hipLaunchCooperativeKernel(fn, dim3(grid), dim3(kPersistThreads), args, 0, s);
}

}  // namespace qh
