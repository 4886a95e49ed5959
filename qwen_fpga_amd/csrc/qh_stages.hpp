// Device bodies of the decode stages, shared by the per-stage kernels
// (qh_kernels.hip: op-level C ABI and the graph engine) and the persistent
// decode kernel (qh_persist.hip).  Each body runs as
//
//   sync.arrive()   this workgroup's earlier stores have completed; it
//                   announces that to the others
//   prefetch        weights / own state of the first work item in flight
//   sync.wait()     every workgroup has arrived: inputs are visible
//   compute         activations read with device-coherent loads (ldc*),
//                   results stored with device-coherent stores (stc*)
//
// The per-stage kernels pass a Sync whose wait() only checks the engine's stop
// flag; the persistent kernel passes its grid barrier.  Work items (row
// batches, heads, attention splits) are assigned to (workgroup, wave) by the
// same formulas in both, and every value is produced by the same code, so the
// two paths are bit-identical.
#pragma once
#include "qh_device.hpp"
#include "qh_kernels.hpp"

namespace qh {

struct NoSync {
  const int* done = nullptr;
  __device__ __forceinline__ void arrive() {}
  __device__ __forceinline__ bool wait() { return done == nullptr || ldc_i(done) == 0; }
};

// ===========================================================================
// GEMV: y = W x over up to four row segments sharing one activation vector.
// A wave owns batches of 8 rows; lane l holds the 16-element chunks
// c = l + 64j of x in registers and streams the same chunks of each row with
// one 16-byte load per chunk (a row of 1024 int8 is one coalesced 1 KiB read
// across the wave).  After the lane partials, reduce8 folds the 8 rows with a
// transposed xor butterfly: at offsets 32, 16, 8 each lane keeps half of its
// rows and receives its partner's other half, then offsets 4, 2, 1 finish the
// tree.  Lane l ends with row (l >> 3) & 7.  Per row this is exactly the
// 64-lane xor tree of the C16 order.
// ===========================================================================
template <typename T>
__device__ __forceinline__ T reduce8(T v[8], int lane) {
  {
    const bool up = (lane & 32) != 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const T send = up ? v[i] : v[i + 4];
      const T keep = up ? v[i + 4] : v[i];
      v[i] = keep + __shfl_xor(send, 32, 64);
    }
  }
  {
    const bool up = (lane & 16) != 0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const T send = up ? v[i] : v[i + 2];
      const T keep = up ? v[i + 2] : v[i];
      v[i] = keep + __shfl_xor(send, 16, 64);
    }
  }
  {
    const bool up = (lane & 8) != 0;
    const T send = up ? v[0] : v[1];
    const T keep = up ? v[1] : v[0];
    v[0] = keep + __shfl_xor(send, 8, 64);
  }
  T r = v[0];
  r = r + __shfl_xor(r, 4, 64);
  r = r + __shfl_xor(r, 2, 64);
  r = r + __shfl_xor(r, 1, 64);
  return r;
}

__device__ __forceinline__ void load16f(const float* p, float* v) {
  const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float4 t = q[k];
    v[4 * k + 0] = t.x;
    v[4 * k + 1] = t.y;
    v[4 * k + 2] = t.z;
    v[4 * k + 3] = t.w;
  }
}
__device__ __forceinline__ void store16f(float* p, const float* v) {
  float4* q = reinterpret_cast<float4*>(p);
#pragma unroll
  for (int k = 0; k < 4; ++k) q[k] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
}
__device__ __forceinline__ void load16b(const int8_t* p, uint32_t* w) {
  const uint4 t = *reinterpret_cast<const uint4*>(p);
  w[0] = t.x;
  w[1] = t.y;
  w[2] = t.z;
  w[3] = t.w;
}
__device__ __forceinline__ float i8_at(const uint32_t* w, int e) {
  return (float)(int)(int8_t)(w[e >> 2] >> (8 * (e & 3)));
}

__device__ __forceinline__ const int8_t* seg_row(const Seg& g, int row, int K) {
  if (g.kind == SEG_PAIR) return ((row & 1) ? g.w2 : g.w) + (size_t)(row >> 1) * K;
  return g.w + (size_t)row * K;
}
__device__ __forceinline__ float seg_scale(const Seg& g, int row) {
  if (g.kind == SEG_PAIR) return (row & 1) ? g.sw2[row >> 1] : g.sw[row >> 1];
  return g.sw[row];
}

// Transposed xor-butterfly over R rows (R = 4 or 8): at offsets 32, 16 (, 8)
// each lane keeps half of its rows and receives its partner's other half; the
// remaining offsets finish the tree.  Lane l ends with row (l >> (6 - log2 R))
// & (R - 1).  Per row this is the 64-lane xor tree of the C16 order.  Written
// out per R so every index is static (no private array can end up in memory).
template <typename T>
__device__ __forceinline__ T reduce4(T v[4], int lane) {
  {
    const bool up = (lane & 32) != 0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const T send = up ? v[i] : v[i + 2];
      const T keep = up ? v[i + 2] : v[i];
      v[i] = keep + __shfl_xor(send, 32, 64);
    }
  }
  {
    const bool up = (lane & 16) != 0;
    const T send = up ? v[0] : v[1];
    const T keep = up ? v[1] : v[0];
    v[0] = keep + __shfl_xor(send, 16, 64);
  }
  T r = v[0];
  r = r + __shfl_xor(r, 8, 64);
  r = r + __shfl_xor(r, 4, 64);
  r = r + __shfl_xor(r, 2, 64);
  r = r + __shfl_xor(r, 1, 64);
  return r;
}
template <int R, typename T>
__device__ __forceinline__ T reduce_rows(T v[R], int lane) {
  if constexpr (R == 8)
    return reduce8(v, lane);
  else
    return reduce4(v, lane);
}
template <int R>
__device__ __forceinline__ int row_of_lane(int lane) {
  return R == 1 ? 0 : (lane >> (R == 8 ? 3 : R == 4 ? 4 : 5)) & (R - 1);
}

// Per-row epilogue inputs, loaded by the writer lanes at kernel start.
struct EpiAux {
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;   // conv state cols 1..3 | residual | A_log
  float w0 = 0.0f, w1 = 0.0f, w2 = 0.0f, w3 = 0.0f;   // conv taps | dt_bias
  float sc = 1.0f;                                     // the row's weight scale (int8 segments)
};
__device__ __forceinline__ void epi_prefetch(const Seg& g, int myrow, EpiAux& x) {
  const int r = min(myrow, g.rows - 1);   // always a valid address; unused rows are never stored
  if (g.kind != SEG_F32) x.sc = seg_scale(g, r);
  switch (g.epi) {
    case E_RESID:
      x.a0 = ldcb(g.out, r);   // residual: written by another workgroup
      break;
    case E_GATE_A:
      x.a0 = g.c0[r];
      x.w0 = g.c1[r];
      break;
    case E_CONV: {
      const float4 st = *reinterpret_cast<const float4*>(g.c2 + (size_t)r * 4);
      const float4 w = *reinterpret_cast<const float4*>(g.c0 + (size_t)r * 4);
      x.a1 = st.y;
      x.a2 = st.z;
      x.a3 = st.w;
      x.w0 = w.x;
      x.w1 = w.y;
      x.w2 = w.z;
      x.w3 = w.w;
      break;
    }
    default:
      break;
  }
}

// Row-batch epilogue: the writer lane of each row stores its result y.
template <int R>
__device__ __forceinline__ void gemv_epilogue(const Seg& g, int lane, int myrow, float y, int acci,
                                              const EpiAux& x) {
  constexpr int LPR = 64 / R;   // lanes holding one row
  if (g.epi == E_SWIGLU) {      // pair rows: even = gate i, odd = up i (mlp.hpp:17)
    const float yo = __shfl_xor(y, LPR, 64);
    if ((lane & (2 * LPR - 1)) == 0 && myrow < g.rows) stcb(g.out, myrow >> 1, dev_silu(y) * yo);
    return;
  }
  if ((lane & (LPR - 1)) != 0 || myrow >= g.rows) return;
  switch (g.epi) {
    case E_STORE:
      stcb(g.out, myrow, y);
      break;
    case E_SILU:   // silu(z) for the gated norm (norm.hpp:32)
      stcb(g.out, myrow, dev_silu(y));
      break;
    case E_RESID:
      stcb(g.out, myrow, x.a0 + y);
      break;
    case E_ACC:
      stcb(g.out, myrow, y);
      g.acc_out[myrow] = acci;
      break;
    case E_GATE_B:
      stcb(g.out, myrow, dev_sigmoid(y));
      break;
    case E_GATE_A:
      stcb(g.out, myrow, -dev_expf(x.a0) * dev_softplus(y + x.w0));
      break;
    case E_CONV: {   // conv1d.hpp:22-36: window = state cols 1..3 + new sample
      float acc = 0.0f;
      acc = acc + x.a1 * x.w0;
      acc = acc + x.a2 * x.w1;
      acc = acc + x.a3 * x.w2;
      acc = acc + y * x.w3;
      *reinterpret_cast<float4*>(g.c2 + (size_t)myrow * 4) = make_float4(x.a1, x.a2, x.a3, y);
      stcb(g.out, myrow, dev_silu(acc));
      break;
    }
    default:
      break;
  }
}

// Loads of one batch: every address is clamped into the segment (rows) and the
// vector (chunks), so the loads are unconditional and issue back to back.  A
// clamped chunk meets x = 0 (the prologue zeroes chunks beyond K) and a clamped
// row is never stored, so neither changes a result.
template <int NCH, int R>
__device__ __forceinline__ void load_batch(const Seg& g, int row0, int K, int nchunk, int lane,
                                           uint32_t (&w)[NCH][R][4]) {
  const bool pair = g.kind == SEG_PAIR;
  const int8_t* w0 = g.w;
  const int8_t* w1 = pair ? g.w2 : g.w;
  const int last = g.rows - 1;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = min(row0 + r, last);
    const int8_t* base = pair ? (((row & 1) ? w1 : w0) + (size_t)(row >> 1) * K) : (w0 + (size_t)row * K);
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = min(lane + 64 * j, nchunk - 1);
      load16b(base + 16 * c, w[j][r]);
    }
  }
}

// Segment of batch b; b is wave-uniform, and readfirstlane makes that visible
// to the compiler so the descriptor is read with scalar loads.
__device__ __forceinline__ int seg_of(const GemvArgs& a, int b) {
  int si = 0;
  while (si + 1 < a.nseg && b >= a.seg[si + 1].batch0) ++si;
  return __builtin_amdgcn_readfirstlane(si);
}

template <int NCH, int MODE, int PRO, int R, class Sync>
__device__ __forceinline__ void gemv_body(const GemvArgs& a, int blk, int nblk, Sync& sync, int tokv) {
  const int lane = threadIdx.x & 63, nwv = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int K = a.K, nchunk = K >> 4;
  const int total = a.seg[a.nseg - 1].batch0 + a.seg[a.nseg - 1].nbatch;
  const int stride = nblk * nwv;
  int b = blk * nwv + wave;

  sync.arrive();
  // ---------------- 1. weights and epilogue inputs of the first batch in flight first
  uint32_t w[NCH][R][4];
  EpiAux aux;
  int si = 0;
  if (b < total) {
    si = seg_of(a, b);
    const Seg& g = a.seg[si];
    const int row0 = (b - g.batch0) * R;
    if (g.kind != SEG_F32) load_batch<NCH, R>(g, row0, K, nchunk, lane, w);
    epi_prefetch(g, row0 + row_of_lane<R>(lane), aux);
  }
  if (!sync.wait()) return;

  // ---------------- 2. prologue: this lane's chunks c = lane + 64 j of x
  float xv[NCH][16];     // fp32 activation (W8A16) / dequantized q*s (W8A8)
  uint32_t xq[NCH][4];   // int8 activation (W8A8)
  float xs = 1.0f;       // activation scale (W8A8)
  if constexpr (PRO == P_LOADQ) {
    xs = *a.sx;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = lane + 64 * j;
      load16b(a.xq + 16 * min(c, nchunk - 1), xq[j]);
      if (c >= nchunk) xq[j][0] = xq[j][1] = xq[j][2] = xq[j][3] = 0u;
#pragma unroll
      for (int e = 0; e < 16; ++e) xv[j][e] = i8_at(xq[j], e) * xs;
    }
  } else {
    float nwv16[NCH][16];
    if constexpr (PRO == P_NORM || PRO == P_GATED) {
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        const int c = min(lane + 64 * j, nchunk - 1);
        load16f(a.nw + (PRO == P_GATED ? ((16 * c) & 127) : 16 * c), nwv16[j]);
      }
    }
    if (PRO == P_NORM && a.emb != nullptr) {   // embed_row (gemv.hpp:76-84)
      const int tok = a.tok != nullptr ? ldc_i(a.tok) : tokv;
      const int8_t* er = a.emb + (size_t)tok * K;
      const float es = a.emb_s[tok];
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        const int c = lane + 64 * j;
        if (c < nchunk) {
          uint32_t t[4];
          load16b(er + 16 * c, t);
#pragma unroll
          for (int e = 0; e < 16; ++e) xv[j][e] = i8_at(t, e) * es;
          if (a.h_out != nullptr && blk == 0 && threadIdx.x < 64) stc16(a.h_out, 16 * c, xv[j]);
        } else {
#pragma unroll
          for (int e = 0; e < 16; ++e) xv[j][e] = 0.0f;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        const int c = lane + 64 * j;
        ldc16(a.x, 16 * min(c, nchunk - 1), xv[j]);
        if (c >= nchunk)
#pragma unroll
          for (int e = 0; e < 16; ++e) xv[j][e] = 0.0f;
      }
    }
    if constexpr (PRO == P_NORM) {   // norm.hpp:13-20, sum of squares in C16 order
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < NCH; ++j)
        if (lane + 64 * j < nchunk) ss = dot16_f32(xv[j], xv[j], ss);
      ss = xor_sum<64>(ss);
      const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
#pragma unroll
      for (int j = 0; j < NCH; ++j)
        if (lane + 64 * j < nchunk)
#pragma unroll
          for (int e = 0; e < 16; ++e) xv[j][e] = (xv[j][e] * inv) * (1.0f + nwv16[j][e]);
    } else if constexpr (PRO == P_GATED) {   // heads of 128 = groups of 8 lanes; z holds silu(z)
      float zs[NCH][16];
#pragma unroll
      for (int j = 0; j < NCH; ++j) ldc16(a.z, 16 * (lane + 64 * j), zs[j]);
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        float ss = dot16_f32(xv[j], xv[j], 0.0f);
        ss = xor_sum<8>(ss);
        const float inv = 1.0f / sqrtf(ss / 128.0f + a.eps);
#pragma unroll
        for (int e = 0; e < 16; ++e) xv[j][e] = ((xv[j][e] * inv) * nwv16[j][e]) * zs[j][e];
      }
    }
    if constexpr (MODE == M_W8A8) {   // _qa (golden/model.py:37-45)
      float am = 0.0f;
#pragma unroll
      for (int j = 0; j < NCH; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) am = fmaxf(am, fabsf(xv[j][e]));
      am = xor_max<64>(am);
      xs = quant_scale(am);
      const float rs = 1.0f / xs;
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

  // ---------------- 3. row batches (the next batch's loads overlap this batch's reduction)
  for (; b < total; b += stride) {
    const Seg& g = a.seg[si];
    const int row0 = (b - g.batch0) * R;
    const int myrow = row0 + row_of_lane<R>(lane);
    float y = 0.0f;
    int acci = 0;
    float pf[R];
    int pi[R];
    if (g.kind == SEG_F32) {   // fp32 weights (gemv.hpp:46-59)
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
              load16f(g.wf + (size_t)(row0 + r) * K + 16 * c, wf);
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
    // issue the next batch's loads before reducing this one
    const int bn = b + stride;
    int sin = si;
    EpiAux auxn;
    if (bn < total) {
      sin = seg_of(a, bn);
      const Seg& gn = a.seg[sin];
      const int rn = (bn - gn.batch0) * R;
      if (gn.kind != SEG_F32) load_batch<NCH, R>(gn, rn, K, nchunk, lane, w);
      epi_prefetch(gn, rn + row_of_lane<R>(lane), auxn);
    }
    if (g.kind == SEG_F32 || MODE == M_W8A16) {
      y = reduce_rows<R>(pf, lane);
      if (g.kind != SEG_F32) y = y * aux.sc;
    } else {
      acci = reduce_rows<R>(pi, lane);
      y = ((float)acci * xs) * aux.sc;   // float(acc)*sx*sw
    }
    gemv_epilogue<R>(g, lane, myrow, y, acci, aux);
    si = sin;
    aux = auxn;
  }
}

// ===========================================================================
// Tied LM head: final rmsnorm prologue, logits = (E row . h) * s in C16
// order, running argmax with the reference's rule (strict >, so the first
// index wins a tie; qwen_synth.hpp:81-88) folded per workgroup.
// ===========================================================================
__device__ __forceinline__ void better(float& bv, int& bi, float v, int i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

template <class Sync>
__device__ __forceinline__ void head_body(const HeadArgs& a, int blk, int nblk, Sync& sync, float* logits) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwv = blockDim.x >> 6;
  const int total = a.rows / kRowsPerBatch;
  const int stride = nblk * nwv;
  int b = blk * nwv + wave;
  const int rl = (lane >> 3) & 7;
  sync.arrive();
  uint32_t w[8][4];
  float sc = 0.0f;
  if (b < total) {   // first batch in flight before the norm prologue
#pragma unroll
    for (int r = 0; r < 8; ++r) load16b(a.w + (size_t)(b * 8 + r) * 1024 + 16 * lane, w[r]);
    sc = a.sw[b * 8 + rl];
  }
  if (!sync.wait()) return;
  float xv[16], nw[16];
  ldc16(a.h, 16 * lane, xv);
  load16f(a.nw + 16 * lane, nw);
  float ss = dot16_f32(xv, xv, 0.0f);
  ss = xor_sum<64>(ss);
  const float inv = 1.0f / sqrtf(ss / 1024.0f + a.eps);
#pragma unroll
  for (int e = 0; e < 16; ++e) xv[e] = (xv[e] * inv) * (1.0f + nw[e]);
  float bv = -1e30f;
  int bi = 0;
  for (; b < total; b += stride) {
    float p[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) p[r] = dot16_i8f(w[r], xv, 0.0f);
    const float scur = sc;
    const int bn = b + stride;
    if (bn < total) {   // next batch in flight during the reduction
#pragma unroll
      for (int r = 0; r < 8; ++r) load16b(a.w + (size_t)(bn * 8 + r) * 1024 + 16 * lane, w[r]);
      sc = a.sw[bn * 8 + rl];
    }
    const float y = reduce8(p, lane) * scur;
    const int row = b * 8 + rl;
    if ((lane & 7) == 0) {
      if (logits != nullptr) logits[row] = y;
      better(bv, bi, y, row);
    }
  }
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
    stc(a.part_val + blk, bv);
    stc_i(a.part_idx + blk, bi);
  }
  __syncthreads();
}

// ===========================================================================
// Gated DeltaNet recurrent step (deltanet.hpp:58-127 and the l2norm / q-scale
// of deltanet.hpp:166-169).  Unit (head h, quarter vq) owns S[h][:, 32 vq ..
// 32 vq + 31]: thread (kg, vl) holds the 16 rows k = 16 kg .. 16 kg + 15 of
// column v = 32 vq + vl.  Sweep A decays S and forms the k-group partial of
// k^T S; the 8 group partials meet in LDS and are added by the pairwise tree
// (offsets 4, 2, 1); delta = (v - kv) * beta; sweep B applies the rank-1
// update and forms q^T S_new the same way.  S is read and written once per
// step, always by the same unit.
// ===========================================================================
// Head h's gate projections from the layer input (see DnArgs), on one wave;
// lane 0 returns (g, beta).  Same operations as the in_proj prologue and its
// fp32 segments, so the values are bit-identical to computing them there.
__device__ __forceinline__ void deltanet_gates(const DnArgs& a, int h, int tokv, float& g, float& beta) {
  const int lane = threadIdx.x & 63;
  float xv[16];
  if (a.emb != nullptr) {   // embed_row (gemv.hpp:76-84)
    const int tok = a.tok != nullptr ? ldc_i(a.tok) : tokv;
    uint32_t t4[4];
    load16b(a.emb + (size_t)tok * 1024 + 16 * lane, t4);
    const float es = a.emb_s[tok];
#pragma unroll
    for (int e = 0; e < 16; ++e) xv[e] = i8_at(t4, e) * es;
  } else {
    ldc16(a.gx, 16 * lane, xv);
  }
  if (a.gx_norm != nullptr) {   // norm.hpp:13-20
    float nw[16];
    load16f(a.gx_norm + 16 * lane, nw);
    float ss = dot16_f32(xv, xv, 0.0f);
    ss = xor_sum<64>(ss);
    const float inv = 1.0f / sqrtf(ss / 1024.0f + a.eps);
#pragma unroll
    for (int e = 0; e < 16; ++e) xv[e] = (xv[e] * inv) * (1.0f + nw[e]);
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
  float w[16];
  load16f(a.wb + (size_t)h * 1024 + 16 * lane, w);
  const float yb = xor_sum<64>(dot16_f32(w, xv, 0.0f));
  load16f(a.wa + (size_t)h * 1024 + 16 * lane, w);
  const float ya = xor_sum<64>(dot16_f32(w, xv, 0.0f));
  beta = dev_sigmoid(yb);
  g = -dev_expf(a.A_log[h]) * dev_softplus(ya + a.dt_bias[h]);
}

template <class Sync>
__device__ __forceinline__ void deltanet_body(const DnArgs& a, int unit, bool valid, Sync& sync, int tokv) {
  const int h = unit / kDnVQuarters, vq = unit % kDnVQuarters;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int vl = t & 31, kg = t >> 5, v = vq * 32 + vl;
  float* Sh = a.S + (size_t)h * 128 * 128;
  __shared__ float gbs[2];
  sync.arrive();
  float s[16];
  if (valid) {
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = Sh[(kg * 16 + i) * 128 + v];   // state tile in flight first
    if (a.wa != nullptr && wave == 0) {   // inputs final before in_proj: off the critical path
      float g0, b0;
      deltanet_gates(a, h, tokv, g0, b0);
      if (lane == 0) {
        gbs[0] = g0;
        gbs[1] = b0;
      }
    }
  }
  if (!sync.wait() || !valid) return;
  __shared__ float qs[128], ks[128];
  __shared__ float part[8][32];
  __shared__ float dl[32];
  float g = 0.0f, beta = 0.0f;
  if (a.wa == nullptr) {
    g = ldcb(a.gb, h);
    beta = ldcb(a.gb, 16 + h);
  }
  const float vv = ldcb(a.convd, 4096 + h * 128 + v);
  if (wave < 2) {   // wave 0: q, wave 1: k; lanes 0..7 hold 16 elements each
    const int src = (wave == 0 ? 0 : 2048) + h * 128;
    float x[16];
    float ss = 0.0f;
    if (lane < 8) {
      ldc16(a.convd, src + 16 * lane, x);
      ss = dot16_f32(x, x, 0.0f);
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) x[e] = 0.0f;
    }
    if (a.normalize) {
      ss = xor_sum<8>(ss);
      const float inv = 1.0f / sqrtf(ss + 1e-6f);   // deltanet.hpp:134
#pragma unroll
      for (int e = 0; e < 16; ++e) x[e] = x[e] * inv;
      if (wave == 0) {
        const float sc = 1.0f / sqrtf(128.0f);   // deltanet.hpp:168-169
#pragma unroll
        for (int e = 0; e < 16; ++e) x[e] = x[e] * sc;
      }
    }
    if (lane < 8) store16f((wave == 0 ? qs : ks) + 16 * lane, x);
  }
  __syncthreads();
  if (a.wa != nullptr) {
    g = gbs[0];
    beta = gbs[1];
  }
  const float gexp = dev_expf(g);
  float p = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {   // sweep A
    const int k = kg * 16 + i;
    s[i] = s[i] * gexp;
    p = p + s[i] * ks[k];
  }
  part[kg][vl] = p;
  __syncthreads();
  if (kg == 0) {
    float pp[8];
#pragma unroll
    for (int gi = 0; gi < 8; ++gi) pp[gi] = part[gi][vl];
#pragma unroll
    for (int off = 4; off >= 1; off >>= 1)
#pragma unroll
      for (int gi = 0; gi < off; ++gi) pp[gi] = pp[gi] + pp[gi + off];
    dl[vl] = (vv - pp[0]) * beta;
  }
  __syncthreads();
  const float d = dl[vl];
  p = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {   // sweep B: reads the updated S
    const int k = kg * 16 + i;
    s[i] = s[i] + ks[k] * d;
    p = p + s[i] * qs[k];
    Sh[k * 128 + v] = s[i];
  }
  part[kg][vl] = p;
  __syncthreads();
  if (kg == 0) {
    float pp[8];
#pragma unroll
    for (int gi = 0; gi < 8; ++gi) pp[gi] = part[gi][vl];
#pragma unroll
    for (int off = 4; off >= 1; off >>= 1)
#pragma unroll
      for (int gi = 0; gi < off; ++gi) pp[gi] = pp[gi] + pp[gi + off];
    stcb(a.o, h * 128 + v, pp[0]);
  }
  __syncthreads();
}

// All heads * kDnVQuarters units; the first one of each workgroup prefetches.
template <class Sync>
__device__ __forceinline__ void deltanet_all(const DnArgs& a, int blk, int nblk, Sync& sync, int tokv) {
  const int units = a.heads * kDnVQuarters;
  deltanet_body(a, blk, blk < units, sync, tokv);
  NoSync none;
  for (int u = blk + nblk; u < units; u += nblk) deltanet_body(a, u, true, none, tokv);
}

// ===========================================================================
// Gated GQA attention, split-K flash decoding (attention.hpp:25-95).
// Unit u = 2 s + j covers positions [64 s, 64 s + 64) of kv head j for the
// four query heads 4j..4j+3 (GQA kv = h/4).  Each wave normalises and rotates
// the four queries (QK-norm with (1+w), RoPE on dims 0..63) in the C16 layout:
// 16 lanes x 16 dims, four positions per wave iteration.  The unit owning
// slot T first writes the new K (normed, rotated) and V rows.  Scores are C16
// dots scaled by 1/16; per head the split max m, p = exp(s - m), the 64-lane
// tree sum l and the position-ordered fma sum acc = sum p v are written for
// the combine step.  A given (s, j) always runs on the same workgroup, so the
// cache rows it reads are the ones it wrote.
// ===========================================================================
__device__ __forceinline__ void qk_norm_rope(float* x, const float* nw16, float eps, int g16,
                                             const float* cs, const float* sn) {
  float ss = dot16_f32(x, x, 0.0f);
  ss = xor_sum<16>(ss);
  const float inv = 1.0f / sqrtf(ss / 256.0f + eps);
#pragma unroll
  for (int e = 0; e < 16; ++e) x[e] = (x[e] * inv) * (1.0f + nw16[e]);
  // rope.hpp:30-41 on dims 0..63 (lanes g16 = 0..3); partner dims +-32 live in lane g16 ^ 2
  float part[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) part[e] = __shfl_xor(x[e], 2, 64);
  if (g16 < 4) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int i = 16 * g16 + e;
      const float half = (i < 32) ? -part[e] : part[e];
      x[e] = x[e] * cs[i & 31] + half * sn[i & 31];
    }
  }
}

// cached K rows (positions < T) of this wave's 16 positions of split s
__device__ __forceinline__ void attn_load_k(const AttnArgs& a, int s, int j, int T, float (&kreg)[4][16]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g16 = lane & 15, pg = lane >> 4;
  const int t0 = s * kAttnSplit;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int tp = t0 + 16 * wave + 4 * it + pg;
    if (tp < T) {
      load16f(a.kc + (size_t)tp * 512 + j * 256 + 16 * g16, kreg[it]);
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) kreg[it][e] = 0.0f;
    }
  }
}

__device__ __forceinline__ void attn_unit(const AttnArgs& a, int s, int j, int T, float (&kreg)[4][16]) {
  const int Tn = T + 1;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int g16 = lane & 15, pg = lane >> 4;
  const int rrow = a.rope_row != nullptr ? ldc_i(a.rope_row) : T;
  const float* cs = a.rope + (size_t)rrow * 64;
  const float* sn = cs + 32;
  __shared__ float sc[4][64];
  __shared__ float pp[4][64];
  const int t0 = s * kAttnSplit;
  float q[4][16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int h = 4 * j + i;
    ldc16(a.qg, h * 512 + 16 * g16, q[i]);   // query half of head h (attention.hpp:40)
    float w[16];
    load16f(a.qn + 16 * g16, w);
    qk_norm_rope(q[i], w, a.eps, g16, cs, sn);
  }
  if (T / kAttnSplit == s) {   // owner of slot T (attention.hpp:46-54)
    if (wave == 0) {
      float k[16], w[16], v[16];
      ldc16(a.kraw, j * 256 + 16 * g16, k);
      load16f(a.kn + 16 * g16, w);
      qk_norm_rope(k, w, a.eps, g16, cs, sn);
      ldc16(a.vraw, j * 256 + 16 * g16, v);
      if (pg == 0) {
        store16f(a.kc + (size_t)T * 512 + j * 256 + 16 * g16, k);
        store16f(a.vc + (size_t)T * 512 + j * 256 + 16 * g16, v);
      }
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 4; ++it)
      if (t0 + 16 * wave + 4 * it + pg == T) load16f(a.kc + (size_t)T * 512 + j * 256 + 16 * g16, kreg[it]);
  }
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int tl = 16 * wave + 4 * it + pg;   // position within the split
    const bool valid = t0 + tl < Tn;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float d = dot16_f32(q[i], kreg[it], 0.0f);
      d = xor_sum<16>(d);
      if (g16 == 0) sc[i][tl] = valid ? d * 0.0625f : -__builtin_inff();
    }
  }
  __syncthreads();
  {
    const int i = wave;
    const bool valid = t0 + lane < Tn;
    const float sv = sc[i][lane];
    const float m = xor_max<64>(valid ? sv : -__builtin_inff());
    const float p = valid ? dev_expf(sv - m) : 0.0f;
    const float l = xor_sum<64>(p);
    pp[i][lane] = p;
    if (lane == 0) {
      stcb(a.pm, (4 * j + i) * a.nsplit_max + s, m);
      stcb(a.pl, (4 * j + i) * a.nsplit_max + s, l);
    }
  }
  __syncthreads();
  {
    const int i = wave;
    const int cnt = min(kAttnSplit, Tn - t0);
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const float* vbase = a.vc + (size_t)t0 * 512 + j * 256 + 4 * lane;
    // 16 rows in flight per group; rows past cnt are clamped loads with p = 0 never added
    for (int tg = 0; tg < cnt; tg += 16) {
      float4 vv[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) vv[u] = *reinterpret_cast<const float4*>(vbase + (size_t)min(tg + u, cnt - 1) * 512);
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        if (tg + u < cnt) {   // position order (attention.hpp:80-86)
          const float pv = pp[i][tg + u];
          acc[0] = __builtin_fmaf(pv, vv[u].x, acc[0]);
          acc[1] = __builtin_fmaf(pv, vv[u].y, acc[1]);
          acc[2] = __builtin_fmaf(pv, vv[u].z, acc[2]);
          acc[3] = __builtin_fmaf(pv, vv[u].w, acc[3]);
        }
      }
    }
    stc4(a.pacc, ((4 * j + i) * a.nsplit_max + s) * 256 + 4 * lane, acc);
  }
  __syncthreads();
}

// Units u = blk, blk + nblk, ... of the 2 * ceil((T+1)/64) splits; T is the slot
// of this token (past tokens = T).
template <class Sync>
__device__ __forceinline__ void attn_body(const AttnArgs& a, int T, int blk, int nblk, Sync& sync) {
  const bool ok = T >= 0 && T < a.max_ctx;
  const int units = ok ? 2 * ((T + 1 + kAttnSplit - 1) / kAttnSplit) : 0;
  sync.arrive();
  float kreg[4][16];
  if (blk < units) attn_load_k(a, blk >> 1, blk & 1, T, kreg);
  if (!sync.wait()) return;
  for (int u = blk; u < units; u += nblk) {
    if (u != blk) attn_load_k(a, u >> 1, u & 1, T, kreg);
    attn_unit(a, u >> 1, u & 1, T, kreg);
  }
}

// Merge the splits of head h in split order; output gate (attention.hpp:89-92).
template <class Sync>
__device__ __forceinline__ void combine_body(const AttnArgs& a, int T, int blk, Sync& sync) {
  sync.arrive();
  if (!sync.wait()) return;
  const int h = blk, d = threadIdx.x;
  if (h >= 8 || T < 0 || T >= a.max_ctx) return;
  const int Tn = T + 1;
  const int ns = (Tn + kAttnSplit - 1) / kAttnSplit;
  const float* pm = a.pm + h * a.nsplit_max;
  const float* pl = a.pl + h * a.nsplit_max;
  float M = -__builtin_inff();
  for (int s = 0; s < ns; ++s) M = fmaxf(M, ldcb(pm, s));
  float L = 0.0f, ctx = 0.0f;
  for (int s = 0; s < ns; ++s) {
    const float e = dev_expf(ldcb(pm, s) - M);
    L = L + ldcb(pl, s) * e;
    ctx = ctx + ldcb(a.pacc, (h * a.nsplit_max + s) * 256 + d) * e;
  }
  const float invL = 1.0f / L;
  const float gate = ldcb(a.qg, h * 512 + 256 + d);
  stcb(a.og, h * 256 + d, (ctx * invL) * dev_sigmoid(gate));
}

}  // namespace qh
