// gfx950 kernels of the decode datapath: the per-stage kernels used by the
// op-level C ABI and the graph engine, over the bodies in qh_stages.hpp, plus
// the small op kernels.  Every reduction follows the fixed orders documented
// in qh_device.hpp, so results do not depend on grid size or timing.
#include <hip/hip_ext.h>

#include "qh_decode.h"
#include "qh_stages.hpp"

namespace qh {

template <int NCH, int MODE, int PRO, int R>
__global__ __launch_bounds__(256) void gemv_kernel(const GemvArgs a) {
  PlainIO io{a.done};
  gemv_body<NCH, MODE, PRO, R>(a, blockIdx.x, gridDim.x, io, a.tokv);
}

template <int NCH, int MODE, int R>
static void launch_gemv_pro(const GemvArgs& a, int grid, dim3 blk, hipStream_t s) {
  switch (a.prologue) {
    case P_NORM: gemv_kernel<NCH, MODE, P_NORM, R><<<grid, blk, 0, s>>>(a); break;
    case P_GATED: gemv_kernel<NCH, MODE, P_GATED, R><<<grid, blk, 0, s>>>(a); break;
    case P_LOADQ:
      if constexpr (MODE == M_W8A8) gemv_kernel<NCH, MODE, P_LOADQ, R><<<grid, blk, 0, s>>>(a);
      break;
    default: gemv_kernel<NCH, MODE, P_LOAD, R><<<grid, blk, 0, s>>>(a); break;
  }
}
template <int NCH, int R>
static void launch_gemv_mode(const GemvArgs& a, int grid, dim3 blk, hipStream_t s) {
  if (a.mode == M_W8A8)
    launch_gemv_pro<NCH, M_W8A8, R>(a, grid, blk, s);
  else
    launch_gemv_pro<NCH, M_W8A16, R>(a, grid, blk, s);
}
template <int R>
static hipError_t launch_gemv_r(const GemvArgs& a, int grid, dim3 blk, hipStream_t s) {
  switch ((a.K + 1023) / 1024) {
    case 1: launch_gemv_mode<1, R>(a, grid, blk, s); break;
    case 2: launch_gemv_mode<2, R>(a, grid, blk, s); break;
    case 3: launch_gemv_mode<3, R>(a, grid, blk, s); break;
    case 4: launch_gemv_mode<4, R>(a, grid, blk, s); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Rows per batch (a.rows_per_batch) must match how the segment batches were counted.
hipError_t launch_gemv(const GemvArgs& a, int waves_per_block, hipStream_t s) {
  if (a.nseg < 1 || a.nseg > 4 || (waves_per_block != 1 && waves_per_block != 2 && waves_per_block != 4))
    return hipErrorInvalidValue;
  if (a.prologue == P_LOADQ && a.mode != M_W8A8) return hipErrorInvalidValue;
  if (a.prologue == P_GATED && a.K != 2048) return hipErrorInvalidValue;
  const int total = a.seg[a.nseg - 1].batch0 + a.seg[a.nseg - 1].nbatch;
  const int grid = (total + waves_per_block - 1) / waves_per_block;
  const dim3 blk(64 * waves_per_block);
  if (a.rows_per_batch < 4)
    for (int i = 0; i < a.nseg; ++i)
      if (a.seg[i].epi == E_SWIGLU) return hipErrorInvalidValue;   // pair rows need R >= 4
  switch (a.rows_per_batch) {
    case 1: return launch_gemv_r<1>(a, grid, blk, s);
    case 4: return launch_gemv_r<4>(a, grid, blk, s);
    case 8: return launch_gemv_r<8>(a, grid, blk, s);
    default: return hipErrorInvalidValue;
  }
}

__global__ __launch_bounds__(256) void head_kernel(const HeadArgs a) {
  PlainIO io{a.done};
  head_body<true>(a, blockIdx.x, gridDim.x, io, a.logits);
}

hipError_t launch_head(const HeadArgs& a, int grid, hipStream_t s, hipEvent_t t0, hipEvent_t t1) {
  if (t0 == nullptr && t1 == nullptr) {
    head_kernel<<<grid, 256, 0, s>>>(a);
    return hipGetLastError();
  }
  // events stamped at the kernel's own start and end (no dispatch gap)
  void* args[] = {const_cast<HeadArgs*>(&a)};
  return hipExtLaunchKernel(reinterpret_cast<const void*>(head_kernel), dim3(grid), dim3(256), args, 0, s, t0, t1, 0);
}

__global__ __launch_bounds__(256) void argmax_kernel(const float* pv, const int* pi, int n, StepCtl* ctl,
                                                     int* out_idx) {
  if (ctl != nullptr && ctl->done != 0) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float bv = -1e30f;
  int bi = 0;
  for (int i = threadIdx.x; i < n; i += blockDim.x) better(bv, bi, pv[i], pi[i]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    better(bv, bi, ov, oi);
  }
  __shared__ float sv[4];
  __shared__ int si[4];
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w2 = 1; w2 < (int)(blockDim.x >> 6); ++w2) better(bv, bi, sv[w2], si[w2]);
    if (out_idx != nullptr) *out_idx = bi;
    if (ctl != nullptr) {
      ctl->argmax = bi;
      ctl->pos = ctl->pos + 1;   // qwen_synth.hpp:90 ++st.pos
    }
  }
}

hipError_t launch_argmax(const float* pv, const int* pi, int n, StepCtl* ctl, int* out_idx, hipStream_t s) {
  argmax_kernel<<<1, 256, 0, s>>>(pv, pi, n, ctl, out_idx);
  return hipGetLastError();
}

// Greedy-generation bookkeeping between steps (run_hls.cpp:56-66 on device).
__global__ void advance_kernel(StepCtl* c, const int* prompt, int* out_ids) {
  if (c->done != 0) return;
  const int am = c->argmax;
  const int next = c->step + 1;
  if (next < c->n_prompt) {
    c->tok = prompt[next];
    c->step = next;
    return;
  }
  if (c->n_out >= c->n_new || am == c->eos) {
    c->done = 1;
    return;
  }
  out_ids[c->n_out] = am;
  c->n_out = c->n_out + 1;
  c->tok = am;
  c->step = next;
  if (c->pos >= c->max_ctx) {
    c->done = 1;
    c->err = 2;
  }
}

hipError_t launch_advance(StepCtl* ctl, const int* prompt, int* out_ids, hipStream_t s) {
  advance_kernel<<<1, 1, 0, s>>>(ctl, prompt, out_ids);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void deltanet_kernel(const DnArgs a) {
  PlainIO io{a.done};
  deltanet_all(a, blockIdx.x, gridDim.x, io, 0);
}

hipError_t launch_deltanet(const DnArgs& a, hipStream_t s) {
  if (a.heads < 1 || a.heads > 16) return hipErrorInvalidValue;
  deltanet_kernel<<<a.heads * kDnVQuarters, 256, 0, s>>>(a);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void attn_kernel(const AttnArgs a) {
  PlainIO io{a.done};
  attn_body(a, ldc_i(a.T), blockIdx.x, gridDim.x, io);
}

__global__ __launch_bounds__(256) void attn_combine_kernel(const AttnArgs a) {
  PlainIO io{a.done};
  combine_body(a, ldc_i(a.T), blockIdx.x, io);
}

hipError_t launch_attn(const AttnArgs& a, hipStream_t s) {
  attn_kernel<<<2 * a.nsplit_max, 256, 0, s>>>(a);
  return hipGetLastError();
}
hipError_t launch_attn_combine(const AttnArgs& a, hipStream_t s) {
  attn_combine_kernel<<<kCombineWGs, 256, 0, s>>>(a);
  return hipGetLastError();
}

// ===========================================================================
// Small op-level kernels.
// ===========================================================================
__global__ void embed_kernel(float* h, const int8_t* w, const float* sc, int tok, int in) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < in) h[i] = (float)w[(size_t)tok * in + i] * sc[tok];
}
hipError_t launch_embed(float* h, const int8_t* w, const float* sc, int tok, int in, hipStream_t s) {
  embed_kernel<<<(in + 255) / 256, 256, 0, s>>>(h, w, sc, tok, in);
  return hipGetLastError();
}

// one wave: C16 sum of squares over n, then the (1+w) or gated scaling.
// One vector of n per workgroup: workgroup b normalises x[b n .. b n + n) (w shared).
__global__ void rmsnorm_kernel(float* y, const float* x, const float* w, const float* z, int n, float eps,
                               int gated) {
  const int lane = threadIdx.x;
  y += (size_t)blockIdx.x * n;
  x += (size_t)blockIdx.x * n;
  if (z != nullptr) z += (size_t)blockIdx.x * n;
  const int nchunk = (n + 15) / 16;
  float ss = 0.0f;
  for (int c = lane; c < nchunk; c += 64)
    for (int e = 0; e < 16 && 16 * c + e < n; ++e) ss = __builtin_fmaf(x[16 * c + e], x[16 * c + e], ss);
  ss = xor_sum<64>(ss);
  const float inv = 1.0f / sqrtf(ss / (float)n + eps);
  for (int i = lane; i < n; i += 64)   // elementwise: any lane order
    y[i] = gated ? ((x[i] * inv) * w[i]) * dev_silu(z[i]) : (x[i] * inv) * (1.0f + w[i]);
}
hipError_t launch_rmsnorm(float* y, const float* x, const float* w, const float* z, int n, float eps,
                          int gated, hipStream_t s, int groups) {
  rmsnorm_kernel<<<groups, 64, 0, s>>>(y, x, w, z, n, eps, gated);
  return hipGetLastError();
}

__global__ void l2norm_kernel(float* v, int n) {
  const int lane = threadIdx.x;
  const int nchunk = (n + 15) / 16;
  float ss = 0.0f;
  for (int c = lane; c < nchunk; c += 64)
    for (int e = 0; e < 16 && 16 * c + e < n; ++e) ss = __builtin_fmaf(v[16 * c + e], v[16 * c + e], ss);
  ss = xor_sum<64>(ss);
  const float inv = 1.0f / sqrtf(ss + 1e-6f);
  for (int c = lane; c < nchunk; c += 64)
    for (int e = 0; e < 16 && 16 * c + e < n; ++e) v[16 * c + e] = v[16 * c + e] * inv;
}
hipError_t launch_l2norm(float* v, int n, hipStream_t s) {
  l2norm_kernel<<<1, 64, 0, s>>>(v, n);
  return hipGetLastError();
}

// conv1d_step + SiLU of channel c (conv1d.hpp): state [C][4], weight [C][4]
__device__ __forceinline__ void conv1d_channel(float* out, const float* in, float* state, const float* w, int c) {
  float* st = state + (size_t)c * 4;
  const float* wc = w + (size_t)c * 4;
  const float w0 = st[1], w1 = st[2], w2 = st[3], w3 = in[c];
  float acc = 0.0f;
  acc = acc + w0 * wc[0];
  acc = acc + w1 * wc[1];
  acc = acc + w2 * wc[2];
  acc = acc + w3 * wc[3];
  st[0] = w0;
  st[1] = w1;
  st[2] = w2;
  st[3] = w3;
  out[c] = dev_silu(acc);
}
__global__ void conv1d_kernel(float* out, const float* in, float* state, const float* w, int C) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c < C) conv1d_channel(out, in, state, w, c);
}
// The DeltaNet step's inputs of the delta rule (deltanet.hpp:155-165): the short conv + SiLU of
// the 6144 qkv channels, and per head beta = sigmoid(b), g = -exp(A_log) softplus(a + dt_bias)
// into gb = g[16] | beta[16] (threads 6144 .. 6159).
__global__ void dn_step_pre_kernel(float* convd, float* gb, const float* qkv, float* state, const float* cw,
                                   const float* b, const float* a, const float* A_log, const float* dt_bias) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c < QH_CONV_DIM) {
    conv1d_channel(convd, qkv, state, cw, c);
  } else if (c < QH_CONV_DIM + QH_LH) {
    const int h = c - QH_CONV_DIM;
    gb[QH_LH + h] = dev_sigmoid(b[h]);
    gb[h] = -dev_expf(A_log[h]) * dev_softplus(a[h] + dt_bias[h]);
  }
}
hipError_t launch_dn_step_pre(float* convd, float* gb, const float* qkv, float* state, const float* cw,
                              const float* b, const float* a, const float* A_log, const float* dt_bias,
                              hipStream_t s) {
  dn_step_pre_kernel<<<(QH_CONV_DIM + QH_LH + 255) / 256, 256, 0, s>>>(convd, gb, qkv, state, cw, b, a, A_log, dt_bias);
  return hipGetLastError();
}
hipError_t launch_conv1d(float* out, const float* in, float* state, const float* w, int C, hipStream_t s) {
  conv1d_kernel<<<(C + 255) / 256, 256, 0, s>>>(out, in, state, w, C);
  return hipGetLastError();
}

__global__ void apply_rope_kernel(float* x, const float* cs, const float* sn) {
  const int i = threadIdx.x;   // 64 lanes: dims 0..63
  const float r = x[i];
  const float partner = __shfl_xor(r, 32, 64);
  const float half = (i < 32) ? -partner : partner;
  x[i] = r * cs[i] + half * sn[i];
}
hipError_t launch_apply_rope(float* x, const float* cs, const float* sn, hipStream_t s) {
  apply_rope_kernel<<<1, 64, 0, s>>>(x, cs, sn);
  return hipGetLastError();
}

__global__ void quant_kernel(int8_t* q, float* sx, const float* x, int n) {
  __shared__ float sm[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float am = 0.0f;
  for (int i = threadIdx.x; i < n; i += blockDim.x) am = fmaxf(am, fabsf(x[i]));
  am = xor_max<64>(am);
  if (lane == 0) sm[wave] = am;
  __syncthreads();
  am = fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3]));
  const float s = quant_scale(am);
  for (int i = threadIdx.x; i < n; i += blockDim.x) q[i] = (int8_t)quant_one(x[i], s);
  if (threadIdx.x == 0) *sx = s;
}
hipError_t launch_quant(int8_t* q, float* sx, const float* x, int n, hipStream_t s) {
  quant_kernel<<<1, 256, 0, s>>>(q, sx, x, n);
  return hipGetLastError();
}

// Offline per-row weight quantisation (quant.py:43-49 quant_rows, used by
// pack_weights.py:79-86): one wave per row.  A row of up to kQRowRegs * 256
// elements with cols % 4 == 0 and aligned pointers is read once into
// registers (fp32: 16-byte loads; bf16 bits: 8-byte loads widened exactly by a
// 16-bit shift), its amax taken with the xor tree (max is exact in any order),
// and written as one dword of four int8 per lane and chunk; other rows take
// two passes over memory.  s = amax/127 (1 if amax == 0) and the quotient
// RN(w/s) is Markstein's correction from rs = RN(1/s), exact on |w| <= amax.
// A row holding a NaN or an infinity gets scale NaN and q = 0.
constexpr int kQRowRegs = 16;
__device__ __forceinline__ float qr_widen(float v) { return v; }
__device__ __forceinline__ float qr_widen(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }
__device__ __forceinline__ void qr_load4(const float* p, float (&v)[4]) {
  const f32x4 t = *as_global(reinterpret_cast<const f32x4*>(p));
  v[0] = t[0];
  v[1] = t[1];
  v[2] = t[2];
  v[3] = t[3];
}
__device__ __forceinline__ void qr_load4(const uint16_t* p, float (&v)[4]) {
  const u32x2 t = *as_global(reinterpret_cast<const u32x2*>(p));
  v[0] = __uint_as_float(t[0] << 16);
  v[1] = __uint_as_float(t[0] & 0xffff0000u);
  v[2] = __uint_as_float(t[1] << 16);
  v[3] = __uint_as_float(t[1] & 0xffff0000u);
}
template <typename T>
__global__ __launch_bounds__(256) void quant_rows_kernel(int8_t* q, float* scale, const T* w, int rows, int cols,
                                                         int vec) {
  const int lane = threadIdx.x & 63;
  const int row = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (row >= rows) return;   // whole waves: no barrier follows
  const T* wr = w + (size_t)row * cols;
  int8_t* qr = q + (size_t)row * cols;
  float am = 0.0f;
  bool bad = false;
  if (vec) {   // cols % 4 == 0, cols <= kQRowRegs * 256, aligned
    float v[kQRowRegs][4];
#pragma unroll
    for (int c = 0; c < kQRowRegs; ++c) {
      const int i = 4 * (lane + 64 * c);
      if (i < cols) {
        qr_load4(wr + i, v[c]);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float a = fabsf(v[c][k]);
          bad = bad || !(a <= 3.402823466e38f);
          am = fmaxf(am, a);
        }
      }
    }
    am = xor_max<64>(am);
    bad = !wave_all(!bad);
    const float s = bad ? __builtin_nanf("") : quant_scale(am);
    const float rs = 1.0f / s;
#pragma unroll
    for (int c = 0; c < kQRowRegs; ++c) {
      const int i = 4 * (lane + 64 * c);
      if (i < cols) {
        int t[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) t[k] = bad ? 0 : quant_one_r(v[c][k], s, rs);
        *as_global_w(reinterpret_cast<uint32_t*>(qr + i)) = pack4(t[0], t[1], t[2], t[3]);
      }
    }
    if (lane == 0) scale[row] = s;
    return;
  }
  for (int i = lane; i < cols; i += 64) {
    const float a = fabsf(qr_widen(wr[i]));
    bad = bad || !(a <= 3.402823466e38f);
    am = fmaxf(am, a);
  }
  am = xor_max<64>(am);
  bad = !wave_all(!bad);
  const float s = bad ? __builtin_nanf("") : quant_scale(am);
  const float rs = 1.0f / s;
  for (int i = lane; i < cols; i += 64) qr[i] = bad ? (int8_t)0 : (int8_t)quant_one_r(qr_widen(wr[i]), s, rs);
  if (lane == 0) scale[row] = s;
}
template <typename T>
hipError_t launch_quant_rows_t(int8_t* q, float* scale, const T* w, int rows, int cols, hipStream_t s) {
  if (rows <= 0 || cols <= 0) return hipErrorInvalidValue;
  const size_t in_align = sizeof(T) == 4 ? 16 : 8;
  const int vec = cols % 4 == 0 && cols <= kQRowRegs * 256 && reinterpret_cast<uintptr_t>(w) % in_align == 0 &&
                  reinterpret_cast<uintptr_t>(q) % 4 == 0;
  quant_rows_kernel<T><<<(rows + 3) / 4, 256, 0, s>>>(q, scale, w, rows, cols, vec);
  return hipGetLastError();
}
hipError_t launch_quant_rows(int8_t* q, float* scale, const float* w, int rows, int cols, hipStream_t s) {
  return launch_quant_rows_t(q, scale, w, rows, cols, s);
}
hipError_t launch_quant_rows_bf16(int8_t* q, float* scale, const uint16_t* w, int rows, int cols, hipStream_t s) {
  return launch_quant_rows_t(q, scale, w, rows, cols, s);
}

// The RTL's fixed-point dequant (rtl/dequant.sv:23-27): p = acc * mult + 2^(shift-1)
// in 64 bits, y_q = p >>> shift (arithmetic), kept to its low outw bits as the
// OUTW-bit output register keeps them, sign-extended into int32.
__global__ void fixed_dequant_kernel(int32_t* yq, const int32_t* acc, const int32_t* mult, int n, int shift,
                                     int outw) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= n) return;
  const int64_t p = (int64_t)acc[i] * (int64_t)mult[i] + ((int64_t)1 << (shift - 1));
  const int64_t y = p >> shift;
  yq[i] = (int32_t)((int64_t)((uint64_t)y << (64 - outw)) >> (64 - outw));
}
hipError_t launch_fixed_dequant(int32_t* yq, const int32_t* acc, const int32_t* mult, int n, int shift, int outw,
                                hipStream_t s) {
  if (n <= 0 || shift < 1 || shift > 62 || outw < 1 || outw > 32) return hipErrorInvalidValue;
  fixed_dequant_kernel<<<(n + 255) / 256, 256, 0, s>>>(yq, acc, mult, n, shift, outw);
  return hipGetLastError();
}

__global__ void set_ints_kernel(int* dst, int a, int b) {
  dst[0] = a;
  dst[1] = b;
}
hipError_t launch_set_ints(int* dst, int a, int b, hipStream_t s) {
  set_ints_kernel<<<1, 1, 0, s>>>(dst, a, b);
  return hipGetLastError();
}

__global__ void set_int_kernel(int* dst, int v) { *dst = v; }
hipError_t launch_set_int(int* dst, int v, hipStream_t s) {
  set_int_kernel<<<1, 1, 0, s>>>(dst, v);
  return hipGetLastError();
}

__global__ void set_floats_kernel(float* dst, const Floats64 v, int n) {
  if ((int)threadIdx.x < n) dst[threadIdx.x] = v.v[threadIdx.x];
}
hipError_t launch_set_floats(float* dst, const Floats64& v, int n, hipStream_t s) {
  if (n < 0 || n > 64) return hipErrorInvalidValue;
  set_floats_kernel<<<1, 64, 0, s>>>(dst, v, n);
  return hipGetLastError();
}

// pos += 1 for a layer-range step (no head / argmax); honours the stop flag.
__global__ void bump_pos_kernel(StepCtl* c) {
  if (c->done == 0) c->pos = c->pos + 1;
}
hipError_t launch_bump_pos(StepCtl* ctl, hipStream_t s) {
  bump_pos_kernel<<<1, 1, 0, s>>>(ctl);
  return hipGetLastError();
}

__global__ void init_gen_kernel(StepCtl* c, int tok0, int n_prompt, int n_new, int eos) {
  c->tok = tok0;
  c->step = 0;
  c->n_prompt = n_prompt;
  c->n_new = n_new;
  c->n_out = 0;
  c->eos = eos;
  c->done = 0;
  c->err = 0;
}
hipError_t launch_init_gen(StepCtl* ctl, int tok0, int n_prompt, int n_new, int eos, hipStream_t s) {
  init_gen_kernel<<<1, 1, 0, s>>>(ctl, tok0, n_prompt, n_new, eos);
  return hipGetLastError();
}


// The delta-rule ops' inputs in the layout deltanet_body reads (convd = q | k | v
// at 0 / 2048 / 4096, gb = g[16] | beta[16]), gathered in one launch: nq
// elements of q and k, nv of v, nh gates (from g / beta, or the scalars gs /
// bs when those pointers are null).
__global__ void dn_gather_kernel(float* convd, float* gb, const float* q, const float* k, const float* v,
                                 const float* g, const float* beta, float gs, float bs, int nq, int nv, int nh) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < nq) {
    convd[i] = q[i];
    convd[2048 + i] = k[i];
  }
  if (i < nv) convd[4096 + i] = v[i];
  if (i < nh) {
    gb[i] = g != nullptr ? g[i] : gs;
    gb[16 + i] = beta != nullptr ? beta[i] : bs;
  }
}
hipError_t launch_dn_gather(float* convd, float* gb, const float* q, const float* k, const float* v, const float* g,
                            const float* beta, float gs, float bs, int nq, int nv, int nh, hipStream_t s) {
  const int n = nq > nv ? nq : nv;
  dn_gather_kernel<<<(n + 255) / 256, 256, 0, s>>>(convd, gb, q, k, v, g, beta, gs, bs, nq, nv, nh);
  return hipGetLastError();
}

}  // namespace qh
