/*
 * oracle.c -- CPU restatement of the reference decode datapath (see oracle.h).
 * TEST INFRASTRUCTURE: the checker for tests/, smoke() and bench's cpu_baseline.
 *
 * Build: gcc -O3 -ffp-contract=off (oracle/Makefile).  With contraction off and
 * SSE arithmetic, every OR_ORDER_REF expression rounds exactly as the reference
 * hls/src headers do under hls/Makefile:14-15.
 */
#include "oracle.h"

#include <math.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define HIDDEN 1024
#define N_LAYERS 24
#define INTER 3584
#define VOCAB 248320
#define EPS 1e-6f
#define LH 16
#define LK 128
#define LV 128
#define CONV_DIM 6144
#define CONV_K 4
#define Z_DIM 2048
#define VALUE_DIM 2048
#define NH 8
#define NKV 2
#define HD 256
#define Q_PROJ 4096
#define KV_PROJ 512
#define ATTN_O_IN 2048
#define ROPE_DIM 64
#define ROPE_THETA 10000000.0f
#define N_LINEAR 18
#define N_FULL 6
/* device-order constants: attention positions per split, DeltaNet k-groups */
#define DEV_ATTN_SPLIT 16
/* longer contexts (Tn > DEV_ATTN_SHORT_MAX): splits of dev_attn_split_len(Tn) positions */
#define DEV_ATTN_SHORT_MAX 2048
#define DEV_ATTN_MAX_SPLITS 128
#define DEV_ATTN_MAX_SPLIT_LEN 512
#define DEV_ATTN_LONG_D 2
#define DEV_DN_KGROUPS 8

static int is_linear(int layer) { return (layer % 4) != 3; }   /* types.hpp:47 */

/* Row loops (independent outputs) may run on several threads; every output is
 * still computed by one thread in the order stated, so results do not depend on
 * the thread count.  Default 1 (the reference csim is single-threaded). */
static int g_threads = 1;
void or_set_threads(int n) { g_threads = n < 1 ? 1 : n; }

/* ====================================================================
 * Device-order transcendentals.  exp: Cody-Waite reduction by ln2 (two-part
 * constant) and the degree-7 Taylor polynomial of e^r on |r| <= ln2/2, Horner
 * with fma, then exact scaling by 2^n.  log1p: in double, m*2^e with m in
 * [sqrt(1/2), sqrt(2)), log m = 2 atanh((m-1)/(m+1)) by its odd series to s^21,
 * rounded once to float.  Only IEEE +,-,*,/,fma and bit operations, so the HIP
 * kernels reproduce them bit for bit.
 * ================================================================== */
static inline float f_from_bits(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static inline uint32_t bits_of(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

float or_dev_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return INFINITY;
  if (x < -103.972084045410156f) return 0.0f;
  const float n = rintf(x * 1.44269502162933349609375f);
  float r = fmaf(n, -0.693145751953125f, x);
  r = fmaf(n, -1.428606765330187045e-06f, r);
  float p = 1.984126984126984e-4f;
  p = fmaf(p, r, 1.388888888888889e-3f);
  p = fmaf(p, r, 8.333333333333333e-3f);
  p = fmaf(p, r, 4.166666666666667e-2f);
  p = fmaf(p, r, 1.666666666666667e-1f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int ni = (int)n;
  if (ni > 127) { p = p * 2.0f; ni -= 1; }
  if (ni < -126) { p = p * 5.42101086242752217e-20f; ni += 64; }
  return p * f_from_bits((uint32_t)(ni + 127) << 23);
}

/* log(u) for u >= 1 in double: u = m * 2^e with m in [sqrt(1/2), sqrt(2)),
 * log m = 2 atanh(s), s = (m-1)/(m+1), odd series to s^21 (|s| <= 0.1716),
 * plus e*ln2 with ln2 split so that e*ln2_hi is exact. */
static double dev_log_d(double u) {
  uint64_t b;
  memcpy(&b, &u, 8);
  int e = (int)((b >> 52) & 0x7ffu) - 1023;
  const uint64_t mb = (b & 0x000fffffffffffffull) | 0x3ff0000000000000ull;
  double m;
  memcpy(&m, &mb, 8);
  if (m > 1.4142135623730951) { m = m * 0.5; e += 1; }
  const double s = (m - 1.0) / (m + 1.0);
  const double s2 = s * s;
  double t = 1.0 / 21.0;
  t = fma(t, s2, 1.0 / 19.0);
  t = fma(t, s2, 1.0 / 17.0);
  t = fma(t, s2, 1.0 / 15.0);
  t = fma(t, s2, 1.0 / 13.0);
  t = fma(t, s2, 1.0 / 11.0);
  t = fma(t, s2, 1.0 / 9.0);
  t = fma(t, s2, 1.0 / 7.0);
  t = fma(t, s2, 1.0 / 5.0);
  t = fma(t, s2, 1.0 / 3.0);
  t = fma(t, s2, 1.0);
  const double lm = (2.0 * s) * t;
  const double fe = (double)e;
  return fma(fe, 6.93147180369123816490e-01, fma(fe, 1.90821492927058770002e-10, lm));
}

/* log1p for y >= 0: y itself below 2^-28 (where y is the rounded log1p), else
 * the double log of 1 + y (exact in double there), rounded once to float. */
float or_dev_log1pf(float y) {
  if (y != y) return y;
  if (y == INFINITY) return y;
  if (y < 3.7252902984619140625e-09f) return y;
  return (float)dev_log_d(1.0 + (double)y);
}

/* ---- activations.hpp:7-14 ---- */
float or_expf(float x, int order) { return order == OR_ORDER_DEV ? or_dev_expf(x) : expf(x); }
float or_silu(float x, int order) { return x / (1.0f + or_expf(-x, order)); }
float or_sigmoid(float x, int order) { return 1.0f / (1.0f + or_expf(-x, order)); }
float or_softplus(float x, int order) {
  if (order == OR_ORDER_DEV) return x > 20.0f ? x : or_dev_log1pf(or_dev_expf(x));
  return x > 20.0f ? x : log1pf(expf(x));
}

/* ====================================================================
 * Device-order reduction: "C16".  Element i belongs to chunk i/16 (the last
 * chunk may be short) and chunk c to lane c mod 64;
 * each lane accumulates its elements in increasing i with fmaf from 0; the
 * L = min(64, pow2ceil(ceil(n/16))) lane partials are combined by the tree
 * p[l] += p[l+off] for off = L/2 .. 1 (the wavefront xor butterfly).
 * ================================================================== */
static int lanes_for(int n) {
  int c = (n + 15) / 16, L = 1;
  while (L < c && L < 64) L <<= 1;
  return L;
}
static float tree_sum(float* p, int L) {
  for (int off = L / 2; off >= 1; off >>= 1)
    for (int l = 0; l < off; ++l) p[l] = p[l] + p[l + off];
  return p[0];
}
static float c16_dot_f32(const float* a, const float* b, int n) {
  float p[64] = {0};
  const int L = lanes_for(n);
  for (int c = 0; c < (n + 15) / 16; ++c) {
    float acc = p[c % 64];
    for (int e = 0; e < 16 && 16 * c + e < n; ++e) acc = fmaf(a[16 * c + e], b[16 * c + e], acc);
    p[c % 64] = acc;
  }
  return tree_sum(p, L);
}
static float c16_dot_i8(const int8_t* a, const float* b, int n) {
  float p[64] = {0};
  const int L = lanes_for(n);
  for (int c = 0; c < (n + 15) / 16; ++c) {
    float acc = p[c % 64];
    for (int e = 0; e < 16 && 16 * c + e < n; ++e) acc = fmaf((float)a[16 * c + e], b[16 * c + e], acc);
    p[c % 64] = acc;
  }
  return tree_sum(p, L);
}
static float sumsq(const float* x, int n, int order) {
  if (order == OR_ORDER_DEV) return c16_dot_f32(x, x, n);
  float ss = 0.0f;
  for (int i = 0; i < n; ++i) ss += x[i] * x[i];
  return ss;
}

/* ====================================================================
 * Primitive kernels, reference loop order (gemv.hpp, norm.hpp, conv1d.hpp,
 * rope.hpp, deltanet.hpp).
 * ================================================================== */
void or_gemv_i8(float* y, const int8_t* w, const float* scale, const float* x, int out, int in) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int o = 0; o < out; ++o) {   /* gemv.hpp:31-41 */
    const int8_t* row = w + (long)o * in;
    float acc = 0.0f;
    for (int i = 0; i < in; ++i) acc += (float)row[i] * x[i];
    y[o] = acc * scale[o];
  }
}

void or_gemv_f32(float* y, const float* w, const float* x, int out, int in) {
  for (int o = 0; o < out; ++o) {   /* gemv.hpp:48-58 */
    const float* row = w + (long)o * in;
    float acc = 0.0f;
    for (int i = 0; i < in; ++i) acc += row[i] * x[i];
    y[o] = acc;
  }
}

float or_row_dot_i8(const int8_t* w, const float* scale, const float* h, int row, int in) {
  const int8_t* r = w + (long)row * in;   /* gemv.hpp:65-72 */
  float acc = 0.0f;
  for (int i = 0; i < in; ++i) acc += (float)r[i] * h[i];
  return acc * scale[row];
}

void or_embed_row(float* h, const int8_t* w, const float* scale, int tok, int in) {
  const int8_t* r = w + (long)tok * in;   /* gemv.hpp:77-83 */
  const float s = scale[tok];
  for (int i = 0; i < in; ++i) h[i] = (float)r[i] * s;
}

void or_rmsnorm(float* y, const float* x, const float* w, int n, float eps) {
  float ss = 0.0f;   /* norm.hpp:13-20 */
  for (int i = 0; i < n; ++i) ss += x[i] * x[i];
  const float inv = 1.0f / sqrtf(ss / (float)n + eps);
  for (int i = 0; i < n; ++i) y[i] = x[i] * inv * (1.0f + w[i]);
}

static void rmsnorm_o(float* y, const float* x, const float* w, int n, float eps, int order) {
  const float ss = sumsq(x, n, order);
  const float inv = 1.0f / sqrtf(ss / (float)n + eps);
  for (int i = 0; i < n; ++i) y[i] = x[i] * inv * (1.0f + w[i]);
}

void or_rmsnorm_gated(float* y, const float* x, const float* w, const float* z, int n, float eps) {
  float ss = 0.0f;   /* norm.hpp:25-33 */
  for (int i = 0; i < n; ++i) ss += x[i] * x[i];
  const float inv = 1.0f / sqrtf(ss / (float)n + eps);
  for (int i = 0; i < n; ++i) y[i] = x[i] * inv * w[i] * or_silu(z[i], OR_ORDER_REF);
}

static void rmsnorm_gated_o(float* y, const float* x, const float* w, const float* z, int n, float eps,
                            int order) {
  const float ss = sumsq(x, n, order);
  const float inv = 1.0f / sqrtf(ss / (float)n + eps);
  for (int i = 0; i < n; ++i) y[i] = x[i] * inv * w[i] * or_silu(z[i], order);
}

/* In W8A8 the norms the device fuses into a GEMV prologue (the layer-input
 * norms and the gated norm before out_proj) apply the gains first and 1/rms
 * last, y = (x g) * inv, so that the activation maximum of the quantization is
 * reduced together with the sum of squares.  W8A16 and the reference order
 * (ORDER_REF) keep norm.hpp's (x inv) g. */
static void gemv_rmsnorm_o(float* y, const float* x, const float* w, int n, float eps, int mode, int order) {
  if (order != OR_ORDER_DEV || mode != OR_W8A8) {
    rmsnorm_o(y, x, w, n, eps, order);
    return;
  }
  const float ss = sumsq(x, n, order);
  const float inv = 1.0f / sqrtf(ss / (float)n + eps);
  for (int i = 0; i < n; ++i) y[i] = (x[i] * (1.0f + w[i])) * inv;
}
static void gemv_rmsnorm_gated_o(float* y, const float* x, const float* w, const float* z, int n, float eps,
                                 int mode, int order) {
  if (order != OR_ORDER_DEV || mode != OR_W8A8) {
    rmsnorm_gated_o(y, x, w, z, n, eps, order);
    return;
  }
  const float ss = sumsq(x, n, order);
  const float inv = 1.0f / sqrtf(ss / (float)n + eps);
  for (int i = 0; i < n; ++i) y[i] = ((x[i] * w[i]) * or_silu(z[i], order)) * inv;
}

static void conv1d_step_o(float* out, const float* in_ch, float* state, const float* weight, int order) {
  for (int c = 0; c < CONV_DIM; ++c) {   /* conv1d.hpp:19-37 */
    float win[CONV_K];
    float* st = state + c * CONV_K;
    win[0] = st[1];
    win[1] = st[2];
    win[2] = st[3];
    win[3] = in_ch[c];
    float acc = 0.0f;
    const float* w = weight + c * CONV_K;
    for (int k = 0; k < CONV_K; ++k) {
      acc += win[k] * w[k];
      st[k] = win[k];
    }
    out[c] = or_silu(acc, order);
  }
}
void or_conv1d_step(float* out, const float* in_ch, float* state, const float* weight) {
  conv1d_step_o(out, in_ch, state, weight, OR_ORDER_REF);
}

void or_rope_cos_sin(int pos, float* cos_o, float* sin_o) {
  const int HALF = ROPE_DIM / 2;   /* rope.hpp:17-27 */
  for (int j = 0; j < HALF; ++j) {
    const float inv = 1.0f / powf(ROPE_THETA, (float)(2 * j) / (float)ROPE_DIM);
    const float f = (float)pos * inv;
    const float c = cosf(f), s = sinf(f);
    cos_o[j] = c;
    cos_o[j + HALF] = c;
    sin_o[j] = s;
    sin_o[j + HALF] = s;
  }
}

void or_apply_rope(float* x, const float* cos_, const float* sin_) {
  const int HALF = ROPE_DIM / 2;   /* rope.hpp:30-41 */
  float rot[ROPE_DIM];
  for (int i = 0; i < ROPE_DIM; ++i) rot[i] = x[i];
  for (int i = 0; i < ROPE_DIM; ++i) {
    const float half = (i < HALF) ? -rot[i + HALF] : rot[i - HALF];
    x[i] = rot[i] * cos_[i] + half * sin_[i];
  }
}

void or_l2norm(float* v, int n) {
  float ss = 0.0f;   /* deltanet.hpp:131-136 */
  for (int i = 0; i < n; ++i) ss += v[i] * v[i];
  const float inv = 1.0f / sqrtf(ss + 1e-6f);
  for (int i = 0; i < n; ++i) v[i] *= inv;
}
static void l2norm_o(float* v, int n, int order) {
  const float ss = sumsq(v, n, order);
  const float inv = 1.0f / sqrtf(ss + 1e-6f);
  for (int i = 0; i < n; ++i) v[i] *= inv;
}

void or_delta_rule_head(const float* q, const float* k, const float* v, float g, float beta, float* S,
                        float* out) {
  /* deltanet.hpp:58-115: decay + k^T S (sweep A), delta, rank-1 update + q^T S_new (sweep B) */
  const float gexp = expf(g);
  float kv[LV], delta[LV];
  for (int j = 0; j < LV; ++j) kv[j] = 0.0f;
  for (int a = 0; a < LK; ++a) {
    const float kk = k[a];
    for (int j = 0; j < LV; ++j) {
      const float s = S[a * LV + j] * gexp;
      S[a * LV + j] = s;
      kv[j] += s * kk;
    }
  }
  for (int j = 0; j < LV; ++j) {
    delta[j] = (v[j] - kv[j]) * beta;
    out[j] = 0.0f;
  }
  for (int a = 0; a < LK; ++a) {
    const float kk = k[a], qq = q[a];
    for (int j = 0; j < LV; ++j) {
      const float s = S[a * LV + j] + kk * delta[j];
      S[a * LV + j] = s;
      out[j] += s * qq;
    }
  }
}

/* device order: k split into DEV_DN_KGROUPS groups of 16, each summed in k order
 * (unfused), group partials combined by the pairwise tree (offsets 4,2,1). */
static void delta_rule_head_dev(const float* q, const float* k, const float* v, float g, float beta,
                                float* S, float* out) {
  const float gexp = or_dev_expf(g);
  const int G = DEV_DN_KGROUPS, KPG = LK / DEV_DN_KGROUPS;
  float delta[LV];
  for (int j = 0; j < LV; ++j) {
    float p[DEV_DN_KGROUPS];
    for (int gi = 0; gi < G; ++gi) {
      float acc = 0.0f;
      for (int a = gi * KPG; a < (gi + 1) * KPG; ++a) {
        const float s = S[a * LV + j] * gexp;
        S[a * LV + j] = s;
        acc = acc + s * k[a];
      }
      p[gi] = acc;
    }
    delta[j] = (v[j] - tree_sum(p, G)) * beta;
  }
  for (int j = 0; j < LV; ++j) {
    float p[DEV_DN_KGROUPS];
    for (int gi = 0; gi < G; ++gi) {
      float acc = 0.0f;
      for (int a = gi * KPG; a < (gi + 1) * KPG; ++a) {
        const float s = S[a * LV + j] + k[a] * delta[j];
        S[a * LV + j] = s;
        acc = acc + s * q[a];
      }
      p[gi] = acc;
    }
    out[j] = tree_sum(p, G);
  }
}

void or_delta_rule_layer(const float* q, const float* k, const float* v, const float* g,
                         const float* beta, float* S, float* out) {
  for (int h = 0; h < LH; ++h)   /* deltanet.hpp:118-127 */
    or_delta_rule_head(q + h * LK, k + h * LK, v + h * LV, g[h], beta[h], S + (long)h * LK * LV,
                       out + h * LV);
}

/* ---- device-order primitives (the twin of each gfx950 op kernel) ---- */
void or_dev_gemv_i8(float* y, const int8_t* w, const float* scale, const float* x, int out, int in) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int o = 0; o < out; ++o) y[o] = c16_dot_i8(w + (long)o * in, x, in) * scale[o];
}
void or_dev_gemv_f32(float* y, const float* w, const float* x, int out, int in) {
  for (int o = 0; o < out; ++o) y[o] = c16_dot_f32(w + (long)o * in, x, in);
}
void or_dev_rmsnorm(float* y, const float* x, const float* w, int n, float eps) {
  rmsnorm_o(y, x, w, n, eps, OR_ORDER_DEV);
}
void or_dev_rmsnorm_gated(float* y, const float* x, const float* w, const float* z, int n, float eps) {
  rmsnorm_gated_o(y, x, w, z, n, eps, OR_ORDER_DEV);
}
void or_dev_l2norm(float* v, int n) { l2norm_o(v, n, OR_ORDER_DEV); }
void or_dev_conv1d_step(float* out, const float* in_ch, float* state, const float* weight) {
  conv1d_step_o(out, in_ch, state, weight, OR_ORDER_DEV);
}
void or_dev_delta_rule_head(const float* q, const float* k, const float* v, float g, float beta, float* S,
                            float* out) {
  delta_rule_head_dev(q, k, v, g, beta, S, out);
}
void or_dev_delta_rule_layer(const float* q, const float* k, const float* v, const float* g,
                             const float* beta, float* S, float* out) {
  for (int h = 0; h < LH; ++h)
    delta_rule_head_dev(q + h * LK, k + h * LK, v + h * LV, g[h], beta[h], S + (long)h * LK * LV, out + h * LV);
}

/* ---- W8A8 ---- */
/* The gfx950 quantizer forms x/s as Markstein's correction from rs = RN(1/s)
 * (q0 = x*rs, r = fma(-s, q0, x), q = fma(r, rs, q0)); restated here so a test
 * can compare it with the true division of or_quant_act. */
void or_quant_act_markstein(int8_t* q, float* s, const float* x, int n) {
  float amax = 0.0f;
  for (int i = 0; i < n; ++i) {
    const float a = fabsf(x[i]);
    if (a > amax) amax = a;
  }
  const float sc = amax > 0.0f ? amax / 127.0f : 1.0f;
  const float rs = 1.0f / sc;
  for (int i = 0; i < n; ++i) {
    const float q0 = x[i] * rs;
    const float r = fmaf(-sc, q0, x[i]);
    float t = rintf(fmaf(r, rs, q0));
    t = fminf(fmaxf(t, -127.0f), 127.0f);
    q[i] = (int8_t)t;
  }
  *s = sc;
}

void or_quant_act(int8_t* q, float* s, const float* x, int n) {
  float amax = 0.0f;   /* model.py:41-45; export_gemv_tv.py:25-30 */
  for (int i = 0; i < n; ++i) {
    const float a = fabsf(x[i]);
    if (a > amax) amax = a;
  }
  const float sc = amax > 0.0f ? amax / 127.0f : 1.0f;
  for (int i = 0; i < n; ++i) {
    float r = rintf(x[i] / sc);
    r = fminf(fmaxf(r, -127.0f), 127.0f);   /* clip(-127, 127); NaN maps to -127 */
    q[i] = (int8_t)r;
  }
  *s = sc;
}

/* quant.py:43-49 quant_rows, the offline weight quantizer of pack_weights.py:
 * per output row amax = max|w|, s = amax/127 (1 if amax == 0), q = rint(w/s)
 * clipped to +-127, all in fp32 (numpy float32 division, round half to even):
 * per row exactly or_quant_act.  A row holding a NaN or an infinity has no
 * defined result in the reference (numpy casts NaN to int8); here, as on the
 * device, its scale is NaN and its q are 0, so a packer can reject it. */
void or_quant_rows(int8_t* q, float* s, const float* w, int rows, int cols) {
  for (int r = 0; r < rows; ++r) {
    const float* wr = w + (long)r * cols;
    int8_t* qr = q + (long)r * cols;
    int finite = 1;
    for (int i = 0; i < cols; ++i) finite &= isfinite(wr[i]) ? 1 : 0;
    if (!finite) {
      memset(qr, 0, (size_t)cols);
      s[r] = NAN;
      continue;
    }
    or_quant_act(qr, &s[r], wr, cols);
  }
}

/* rtl/matvec_i8.sv = gemv_i8.sv (acc: 32-bit signed sum of int8 products, row by
 * row) then dequant.sv:23-27: p = acc*mult + (1 << (SHIFT-1)) in 64 bits, y_q =
 * p >>> SHIFT assigned to an OUTW-bit register (low OUTW bits, two's complement). */
void or_matvec_fixed(int32_t* yq, int32_t* acc, const int8_t* w, const int32_t* mult, const int8_t* xq, int out,
                     int in, int shift, int outw) {
  for (int o = 0; o < out; ++o) {
    uint32_t a = 0u;   /* 32-bit register: wraps like the RTL accumulator */
    for (int i = 0; i < in; ++i) a += (uint32_t)((int32_t)w[(long)o * in + i] * (int32_t)xq[i]);
    acc[o] = (int32_t)a;
    const int64_t p = (int64_t)acc[o] * (int64_t)mult[o] + ((int64_t)1 << (shift - 1));
    const int64_t y = p >> shift;   /* arithmetic: gcc shifts signed values arithmetically */
    const uint64_t m = outw == 64 ? ~0ull : ((1ull << outw) - 1ull);
    uint64_t u = (uint64_t)y & m;
    if (outw < 64 && (u >> (outw - 1)) & 1ull) u |= ~m;   /* sign-extend the OUTW-bit value */
    yq[o] = (int32_t)(int64_t)u;
  }
}

void or_gemv_w8a8(float* y, int32_t* acc, const int8_t* w, const float* sw, const int8_t* xq, float sx,
                  int out, int in) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int o = 0; o < out; ++o) {
    const int8_t* row = w + (long)o * in;
    int32_t a = 0;
    for (int i = 0; i < in; ++i) a += (int32_t)row[i] * (int32_t)xq[i];
    if (acc) acc[o] = a;
    y[o] = (float)a * sx * sw[o];
  }
}

void or_gemv_acc_i64(int64_t* acc, const int8_t* w, const int8_t* xq, int out, int in) {
  for (int o = 0; o < out; ++o) {
    int64_t a = 0;
    for (int i = in - 1; i >= 0; --i) a += (int64_t)w[(long)o * in + i] * (int64_t)xq[i];
    acc[o] = a;
  }
}

/* projection of x through an int8 tensor in the given mode/order.
 * W8A8: xq/sx are the quantized activation (already computed by the caller). */
typedef struct act_t {
  const float* x;    /* fp32 activation (W8A16) */
  int8_t* q;         /* int8 activation (W8A8) */
  float s;
  float* xf;         /* dequantized q*s (fp32-weight projections in W8A8) */
} act_t;

static void act_prepare(act_t* a, const float* x, int n, int mode, int8_t* qbuf, float* xfbuf) {
  a->x = x;
  a->q = NULL;
  a->xf = NULL;
  a->s = 1.0f;
  if (mode == OR_W8A8) {
    or_quant_act(qbuf, &a->s, x, n);
    a->q = qbuf;
    /* model.py:45 returns rint(x/s).clip * s; with amax == 0 it returns x itself (zeros) */
    for (int i = 0; i < n; ++i) xfbuf[i] = (float)qbuf[i] * a->s;
    a->xf = xfbuf;
  }
}

static void proj_i8(float* y, const or_tensor* t, const act_t* a, int mode, int order) {
  if (mode == OR_W8A8) {
    or_gemv_w8a8(y, NULL, t->w_i8, t->scale, a->q, a->s, t->out, t->in);
    return;
  }
  if (order == OR_ORDER_DEV) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int o = 0; o < t->out; ++o)
      y[o] = c16_dot_i8(t->w_i8 + (long)o * t->in, a->x, t->in) * t->scale[o];
  } else {
    or_gemv_i8(y, t->w_i8, t->scale, a->x, t->out, t->in);
  }
}

static void proj_f32(float* y, const or_tensor* t, const act_t* a, int mode, int order) {
  const float* x = mode == OR_W8A8 ? a->xf : a->x;
  if (order == OR_ORDER_DEV) {
    for (int o = 0; o < t->out; ++o) y[o] = c16_dot_f32(t->w_f32 + (long)o * t->in, x, t->in);
  } else {
    or_gemv_f32(y, t->w_f32, x, t->out, t->in);
  }
}

/* ====================================================================
 * Layer ops (deltanet.hpp:141-182, attention.hpp:25-95, mlp.hpp:11-19) with
 * the W8A8 quantization points of golden/model.py.
 * ================================================================== */
/* The recurrent step between the projections (deltanet.hpp:154-179): short conv + SiLU over the
 * qkv stream, gates, l2norm, delta rule, per-head gated RMSNorm into og[VALUE_DIM]. */
static void deltanet_core(float* og, const float* qkv, const float* z, const float* b, const float* a,
                          const float* conv_w, const float* A_log, const float* dt_bias,
                          const float* gate_norm_w, float* rec, float* conv_state, int mode, int order) {
  float convd[CONV_DIM];
  float q[LH * LK], k[LH * LK], v[LH * LV], g[LH], beta[LH], o[LH * LV];
  conv1d_step_o(convd, qkv, conv_state, conv_w, order);
  for (int h = 0; h < LH; ++h) {   /* deltanet.hpp:160-170 */
    for (int i = 0; i < LK; ++i) q[h * LK + i] = convd[h * LK + i];
    for (int i = 0; i < LK; ++i) k[h * LK + i] = convd[VALUE_DIM + h * LK + i];
    for (int i = 0; i < LV; ++i) v[h * LV + i] = convd[2 * VALUE_DIM + h * LV + i];
    beta[h] = or_sigmoid(b[h], order);
    g[h] = -or_expf(A_log[h], order) * or_softplus(a[h] + dt_bias[h], order);
    l2norm_o(q + h * LK, LK, order);
    l2norm_o(k + h * LK, LK, order);
    const float scale = 1.0f / sqrtf((float)LK);
    for (int i = 0; i < LK; ++i) q[h * LK + i] *= scale;
  }
  for (int h = 0; h < LH; ++h) {
    if (order == OR_ORDER_DEV)
      delta_rule_head_dev(q + h * LK, k + h * LK, v + h * LV, g[h], beta[h], rec + (long)h * LK * LV,
                          o + h * LV);
    else
      or_delta_rule_head(q + h * LK, k + h * LK, v + h * LV, g[h], beta[h], rec + (long)h * LK * LV,
                         o + h * LV);
  }
  for (int h = 0; h < LH; ++h)   /* deltanet.hpp:177-179 */
    gemv_rmsnorm_gated_o(og + h * LV, o + h * LV, gate_norm_w, z + h * LV, LV, EPS, mode, order);
}

void or_deltanet_step(float* og, const float* qkv, const float* z, const float* b, const float* a,
                      const float* conv_w, const float* A_log, const float* dt_bias, const float* gate_norm_w,
                      float* rec, float* conv_state, int order) {
  deltanet_core(og, qkv, z, b, a, conv_w, A_log, dt_bias, gate_norm_w, rec, conv_state, OR_W8A16, order);
}

void or_deltanet_layer(float* out, const float* x, const or_tensor* qkv_w, const or_tensor* z_w,
                       const or_tensor* b_w, const or_tensor* a_w, const float* conv_w,
                       const float* A_log, const float* dt_bias, const float* gate_norm_w,
                       const or_tensor* out_w, float* rec, float* conv_state, int mode, int order) {
  float qkv[CONV_DIM], z[Z_DIM], b[LH], a[LH], og[VALUE_DIM];
  int8_t qbuf[VALUE_DIM];
  float xfbuf[VALUE_DIM];
  act_t act;
  act_prepare(&act, x, HIDDEN, mode, qbuf, xfbuf);   /* model.py:143 xq = _qa(x) */
  proj_i8(qkv, qkv_w, &act, mode, order);
  proj_i8(z, z_w, &act, mode, order);
  proj_f32(b, b_w, &act, mode, order);
  proj_f32(a, a_w, &act, mode, order);
  deltanet_core(og, qkv, z, b, a, conv_w, A_log, dt_bias, gate_norm_w, rec, conv_state, mode, order);
  act_t act2;
  act_prepare(&act2, og, VALUE_DIM, mode, qbuf, xfbuf);   /* model.py:191 _qa(o) */
  proj_i8(out, out_w, &act2, mode, order);
}

/* attention core for one layer, given q (normed+roped, [NH][HD]), the cache
 * holding Tn = T+1 tokens, and the gate; writes og[2048]. */
static void attn_core_ref(float* og, const float* q, const float* gate, const float* kcache,
                          const float* vcache, int Tn) {
  const int rep = NH / NKV;   /* attention.hpp:56-92 */
  const float scale = 1.0f / sqrtf((float)HD);
  float* sc = (float*)malloc(sizeof(float) * (size_t)Tn);
  float ctx[HD];
  for (int h = 0; h < NH; ++h) {
    const int kv = h / rep;
    float m = -1e30f;
    for (int t = 0; t < Tn; ++t) {
      const float* kt = kcache + (long)t * KV_PROJ + kv * HD;
      float d = 0.0f;
      for (int i = 0; i < HD; ++i) d += q[h * HD + i] * kt[i];
      d *= scale;
      sc[t] = d;
      if (d > m) m = d;
    }
    float denom = 0.0f;
    for (int t = 0; t < Tn; ++t) {
      sc[t] = expf(sc[t] - m);
      denom += sc[t];
    }
    const float invd = 1.0f / denom;
    for (int d = 0; d < HD; ++d) ctx[d] = 0.0f;
    for (int t = 0; t < Tn; ++t) {
      const float w = sc[t] * invd;
      const float* vt = vcache + (long)t * KV_PROJ + kv * HD;
      for (int d = 0; d < HD; ++d) ctx[d] += w * vt[d];
    }
    for (int d = 0; d < HD; ++d) og[h * HD + d] = ctx[d] * or_sigmoid(gate[h * HD + d], OR_ORDER_REF);
  }
  free(sc);
}

/* device order (qh_stages.hpp attn_unit / combine_body): the cached positions
 * 0 .. Tn - 2 in splits of DEV_ATTN_SPLIT; per split the score is a C16 dot, m the
 * split max, p = exp(s - m), l the 64-lane tree sum of p, acc the k-ordered fma sum
 * of p*v.  The new position Tn - 1 is a split of its own after them, with m its
 * score, l = 1 and acc its V row.  The splits are merged sequentially with
 * e_s = exp(m_s - M): L += l_s*e_s, acc += acc_s*e_s; ctx = acc * (1/L). */
static void attn_core_dev(float* og, const float* q, const float* gate, const float* kcache,
                          const float* vcache, int Tn) {
  const int rep = NH / NKV, P = DEV_ATTN_SPLIT;
  const int Tc = Tn - 1;                  /* cached positions */
  const int ns = (Tc + P - 1) / P + 1;    /* + the new position's split */
  float* ms = (float*)malloc(sizeof(float) * (size_t)ns);
  float* ls = (float*)malloc(sizeof(float) * (size_t)ns);
  float* accs = (float*)malloc(sizeof(float) * (size_t)ns * HD);
  for (int h = 0; h < NH; ++h) {
    const int kv = h / rep;
    for (int s = 0; s < ns; ++s) {
      float sc[DEV_ATTN_SPLIT], p[64];
      if (s == ns - 1) {   /* the new position: m = its score, l = 1, acc = its V row */
        const float* vrow = vcache + (long)Tc * KV_PROJ + kv * HD;
        ms[s] = c16_dot_f32(q + h * HD, kcache + (long)Tc * KV_PROJ + kv * HD, HD) * 0.0625f;
        ls[s] = 1.0f;
        for (int d = 0; d < HD; ++d) accs[(size_t)s * HD + d] = vrow[d];
        continue;
      }
      const int t0 = s * P, t1 = t0 + P < Tc ? t0 + P : Tc;
      float m = -INFINITY;
      for (int t = t0; t < t1; ++t) {
        const float d = c16_dot_f32(q + h * HD, kcache + (long)t * KV_PROJ + kv * HD, HD) * 0.0625f;
        sc[t - t0] = d;
        if (d > m) m = d;
      }
      for (int i = 0; i < 64; ++i) p[i] = 0.0f;
      for (int t = t0; t < t1; ++t) p[t - t0] = or_dev_expf(sc[t - t0] - m);
      float* acc = accs + (size_t)s * HD;
      for (int d = 0; d < HD; ++d) {
        float a = 0.0f;
        for (int t = t0; t < t1; ++t) a = fmaf(p[t - t0], vcache[(long)t * KV_PROJ + kv * HD + d], a);
        acc[d] = a;
      }
      ms[s] = m;
      ls[s] = tree_sum(p, 64);
    }
    float M = -INFINITY;
    for (int s = 0; s < ns; ++s)
      if (ms[s] > M) M = ms[s];
    float L = 0.0f;
    float ctx[HD];
    for (int d = 0; d < HD; ++d) ctx[d] = 0.0f;
    for (int s = 0; s < ns; ++s) {
      const float e = or_dev_expf(ms[s] - M);
      L = L + ls[s] * e;
      for (int d = 0; d < HD; ++d) ctx[d] = ctx[d] + accs[(size_t)s * HD + d] * e;
    }
    const float invL = 1.0f / L;
    for (int d = 0; d < HD; ++d)
      og[h * HD + d] = (ctx[d] * invL) * or_sigmoid(gate[h * HD + d], OR_ORDER_DEV);
  }
  free(ms);
  free(ls);
  free(accs);
}

/* device order for Tn > DEV_ATTN_SHORT_MAX (qh_stages.hpp attn_unit_long / combine_long).
 * P = 4*ceil(Tn/512) positions per split (at most 512).  Per split and head the four
 * waves w take the iterations it = w, w+4, ... of four positions t0+4it+u, kw per wave
 * (rounded up to a multiple of 4); wave w: m_w the maximum score of its positions,
 * then in its order (k ascending, then u) p = exp(s - m_w) (0 past the split's end,
 * where v is the split's last row), l_w = l_w + p, acc_w = fma(p, v, acc_w).  Merge:
 * M = max m_w, e_w = exp(m_w - M) (0 for m_w = -inf), l = (l0 e0 + l1 e1) + (l2 e2 +
 * l3 e3), acc likewise.  Combine: M = max m_s, e_s = exp(m_s - M); quarter w of the
 * splits [w c, (w+1) c), c = ceil(ns/4), folded in order (L = L + l e, ctx = ctx +
 * acc e); L = (L0 + L1) + (L2 + L3), ctx the same; ctx * (1/L) * sigmoid(gate). */
static int dev_attn_split_len(int Tn) {
  if (Tn <= DEV_ATTN_SHORT_MAX) return DEV_ATTN_SPLIT;
  const int P = 4 * ((Tn + 4 * DEV_ATTN_MAX_SPLITS - 1) / (4 * DEV_ATTN_MAX_SPLITS));
  return P < DEV_ATTN_MAX_SPLIT_LEN ? P : DEV_ATTN_MAX_SPLIT_LEN;
}
static void attn_core_dev_long(float* og, const float* q, const float* gate, const float* kcache,
                               const float* vcache, int Tn) {
  const int rep = NH / NKV, P = dev_attn_split_len(Tn), D = DEV_ATTN_LONG_D;
  const int ns = (Tn + P - 1) / P;
  float* ms = (float*)malloc(sizeof(float) * (size_t)ns);
  float* ls = (float*)malloc(sizeof(float) * (size_t)ns);
  float* accs = (float*)malloc(sizeof(float) * (size_t)ns * HD);
  float* sc = (float*)malloc(sizeof(float) * (size_t)P);
  for (int h = 0; h < NH; ++h) {
    const int kv = h / rep;
    for (int s = 0; s < ns; ++s) {
      const int t0 = s * P, t1 = t0 + P < Tn ? t0 + P : Tn;
      const int nit = (t1 - t0 + 3) / 4, kw = ((nit + 3) / 4 + D - 1) / D * D;
      for (int t = t0; t < t1; ++t)
        sc[t - t0] = c16_dot_f32(q + h * HD, kcache + (long)t * KV_PROJ + kv * HD, HD) * 0.0625f;
      float mw[4], lw[4], aw[4][HD];
      for (int w = 0; w < 4; ++w) {
        float m = -INFINITY;
        for (int k = 0; k < kw; ++k)
          for (int u = 0; u < 4; ++u) {
            const int t = t0 + 4 * (w + 4 * k) + u;
            if (t < t1 && sc[t - t0] > m) m = sc[t - t0];
          }
        float l = 0.0f;
        for (int d = 0; d < HD; ++d) aw[w][d] = 0.0f;
        for (int k = 0; k < kw; ++k)
          for (int u = 0; u < 4; ++u) {
            const int t = t0 + 4 * (w + 4 * k) + u;
            const float p = t < t1 ? or_dev_expf(sc[t - t0] - m) : 0.0f;
            const float* vt = vcache + (long)(t < t1 ? t : t1 - 1) * KV_PROJ + kv * HD;
            for (int d = 0; d < HD; ++d) aw[w][d] = fmaf(p, vt[d], aw[w][d]);
            l = l + p;
          }
        mw[w] = m;
        lw[w] = l;
      }
      float M = -INFINITY, e[4];
      for (int w = 0; w < 4; ++w)
        if (mw[w] > M) M = mw[w];
      for (int w = 0; w < 4; ++w) e[w] = mw[w] == -INFINITY ? 0.0f : or_dev_expf(mw[w] - M);
      ms[s] = M;
      ls[s] = (lw[0] * e[0] + lw[1] * e[1]) + (lw[2] * e[2] + lw[3] * e[3]);
      for (int d = 0; d < HD; ++d)
        accs[(size_t)s * HD + d] = (aw[0][d] * e[0] + aw[1][d] * e[1]) + (aw[2][d] * e[2] + aw[3][d] * e[3]);
    }
    float M = -INFINITY;
    for (int s = 0; s < ns; ++s)
      if (ms[s] > M) M = ms[s];
    const int c = (ns + 3) / 4;
    float Lq[4], cq[4][HD];
    for (int w = 0; w < 4; ++w) {
      const int s0 = w * c < ns ? w * c : ns, s1 = s0 + c < ns ? s0 + c : ns;
      Lq[w] = 0.0f;
      for (int d = 0; d < HD; ++d) cq[w][d] = 0.0f;
      for (int s = s0; s < s1; ++s) {
        const float es = or_dev_expf(ms[s] - M);
        Lq[w] = Lq[w] + ls[s] * es;
        for (int d = 0; d < HD; ++d) cq[w][d] = cq[w][d] + accs[(size_t)s * HD + d] * es;
      }
    }
    const float invL = 1.0f / ((Lq[0] + Lq[1]) + (Lq[2] + Lq[3]));
    for (int d = 0; d < HD; ++d) {
      const float ctx = (cq[0][d] + cq[1][d]) + (cq[2][d] + cq[3][d]);
      og[h * HD + d] = (ctx * invL) * or_sigmoid(gate[h * HD + d], OR_ORDER_DEV);
    }
  }
  free(ms);
  free(ls);
  free(accs);
  free(sc);
}

void or_attention_layer(float* out, const float* x, const or_tensor* q_w, const or_tensor* k_w,
                        const or_tensor* v_w, const or_tensor* o_w, const float* q_norm,
                        const float* k_norm, int pos, float* kcache, float* vcache, int T, int mode,
                        int order) {
  float qg[Q_PROJ], kflat[KV_PROJ], vflat[KV_PROJ], q[NH * HD], gate[ATTN_O_IN], og[ATTN_O_IN];
  float cosb[ROPE_DIM], sinb[ROPE_DIM];
  int8_t qbuf[ATTN_O_IN];
  float xfbuf[ATTN_O_IN];
  act_t act;
  act_prepare(&act, x, HIDDEN, mode, qbuf, xfbuf);   /* model.py:200 */
  proj_i8(qg, q_w, &act, mode, order);               /* attention.hpp:31-33 */
  proj_i8(kflat, k_w, &act, mode, order);
  proj_i8(vflat, v_w, &act, mode, order);
  or_rope_cos_sin(pos, cosb, sinb);
  for (int h = 0; h < NH; ++h) {   /* attention.hpp:39-43 */
    rmsnorm_o(q + h * HD, qg + h * HD * 2, q_norm, HD, EPS, order);
    or_apply_rope(q + h * HD, cosb, sinb);
    for (int d = 0; d < HD; ++d) gate[h * HD + d] = qg[h * HD * 2 + HD + d];
  }
  float* kslot = kcache + (long)T * KV_PROJ;   /* attention.hpp:46-54 */
  float* vslot = vcache + (long)T * KV_PROJ;
  for (int kv = 0; kv < NKV; ++kv) {
    float ktmp[HD];
    rmsnorm_o(ktmp, kflat + kv * HD, k_norm, HD, EPS, order);
    or_apply_rope(ktmp, cosb, sinb);
    for (int d = 0; d < HD; ++d) kslot[kv * HD + d] = ktmp[d];
    for (int d = 0; d < HD; ++d) vslot[kv * HD + d] = vflat[kv * HD + d];
  }
  if (order == OR_ORDER_DEV && T + 1 > DEV_ATTN_SHORT_MAX)
    attn_core_dev_long(og, q, gate, kcache, vcache, T + 1);
  else if (order == OR_ORDER_DEV)
    attn_core_dev(og, q, gate, kcache, vcache, T + 1);
  else
    attn_core_ref(og, q, gate, kcache, vcache, T + 1);
  act_t act2;
  act_prepare(&act2, og, ATTN_O_IN, mode, qbuf, xfbuf);   /* model.py:230 _qa(o) */
  proj_i8(out, o_w, &act2, mode, order);
}

void or_mlp_layer(float* out, const float* x, const or_tensor* gate_w, const or_tensor* up_w,
                  const or_tensor* down_w, int mode, int order) {
  static __thread float g[INTER], u[INTER], xfbuf[INTER];
  static __thread int8_t qbuf[INTER];
  act_t act;
  act_prepare(&act, x, HIDDEN, mode, qbuf, xfbuf);   /* model.py:234 */
  proj_i8(g, gate_w, &act, mode, order);             /* mlp.hpp:14-18 */
  proj_i8(u, up_w, &act, mode, order);
  for (int i = 0; i < INTER; ++i) g[i] = or_silu(g[i], order) * u[i];
  act_t act2;
  act_prepare(&act2, g, INTER, mode, qbuf, xfbuf);   /* model.py:237 _qa(g*u) */
  proj_i8(out, down_w, &act2, mode, order);
}

/* ====================================================================
 * Whole model (qwen_synth.hpp:39-92 / decoder.hpp:62-120).
 * ================================================================== */
typedef struct or_entry {
  char name[96];
  unsigned long long off, soff;
  int dtype, out, in;
} or_entry;

struct or_model {
  const uint8_t* blob;
  or_entry ent[400];
  int n_ent;
  int max_ctx;
  float* rec;    /* [18][16][128][128] */
  float* conv;   /* [18][6144][4] */
  float* kc;     /* [6][max_ctx][512] */
  float* vc;
  int pos;
};

static const or_entry* find(const or_model* m, const char* name) {
  for (int i = 0; i < m->n_ent; ++i)
    if (strcmp(m->ent[i].name, name) == 0) return &m->ent[i];
  fprintf(stderr, "oracle: tensor %s not in index\n", name);
  abort();
}

static or_tensor tensor_of(const or_model* m, const char* name) {
  const or_entry* e = find(m, name);   /* decoder.hpp:41-53 */
  or_tensor t;
  memset(&t, 0, sizeof t);
  t.out = e->out;
  t.in = e->in;
  if (e->dtype == 1) {
    t.w_i8 = (const int8_t*)(m->blob + e->off);
    t.scale = (const float*)(m->blob + e->soff);
  } else {
    t.w_f32 = (const float*)(m->blob + e->off);
  }
  return t;
}

static const float* f32_of(const or_model* m, const char* name) {
  return (const float*)(m->blob + find(m, name)->off);
}

or_model* or_model_new(const uint8_t* blob, const char* idx_text, int max_ctx) {
  or_model* m = (or_model*)calloc(1, sizeof(or_model));
  if (!m || max_ctx < 1) { free(m); return NULL; }
  m->blob = blob;
  m->max_ctx = max_ctx;
  const char* p = idx_text;
  while (*p) {   /* tb_decode.cpp:52-62 line format */
    or_entry e;
    unsigned long long nb, sn;
    int consumed = 0;
    if (m->n_ent >= 400) break;
    if (sscanf(p, "%95s %llu %llu %d %llu %llu %d %d%n", e.name, &e.off, &nb, &e.dtype, &e.soff, &sn,
               &e.out, &e.in, &consumed) != 8)
      break;
    m->ent[m->n_ent++] = e;
    p += consumed;
    while (*p == '\n' || *p == '\r' || *p == ' ') ++p;
  }
  m->rec = (float*)calloc((size_t)N_LINEAR * LH * LK * LV, sizeof(float));
  m->conv = (float*)calloc((size_t)N_LINEAR * CONV_DIM * CONV_K, sizeof(float));
  m->kc = (float*)calloc((size_t)N_FULL * max_ctx * KV_PROJ, sizeof(float));
  m->vc = (float*)calloc((size_t)N_FULL * max_ctx * KV_PROJ, sizeof(float));
  if (!m->rec || !m->conv || !m->kc || !m->vc) { or_model_free(m); return NULL; }
  return m;
}

void or_model_free(or_model* m) {
  if (!m) return;
  free(m->rec);
  free(m->conv);
  free(m->kc);
  free(m->vc);
  free(m);
}

void or_model_reset(or_model* m) {   /* state.hpp:24-34 */
  memset(m->rec, 0, sizeof(float) * (size_t)N_LINEAR * LH * LK * LV);
  memset(m->conv, 0, sizeof(float) * (size_t)N_LINEAR * CONV_DIM * CONV_K);
  memset(m->kc, 0, sizeof(float) * (size_t)N_FULL * m->max_ctx * KV_PROJ);
  memset(m->vc, 0, sizeof(float) * (size_t)N_FULL * m->max_ctx * KV_PROJ);
  m->pos = 0;
}

static void layers(or_model* m, int l0, int l1, float* h, int mode, int order) {
  float hn[HIDDEN], mix[HIDDEN], r[HIDDEN];
  char a[128], nm[160];
  int li = 0, fi = 0;
  for (int l = 0; l < l0; ++l) {
    if (is_linear(l)) ++li; else ++fi;
  }
  for (int layer = l0; layer < l1; ++layer) {   /* qwen_synth.hpp:47-77 */
    for (int i = 0; i < HIDDEN; ++i) r[i] = h[i];
    snprintf(nm, sizeof nm, "layers.%d.input_layernorm.weight", layer);
    gemv_rmsnorm_o(hn, h, f32_of(m, nm), HIDDEN, EPS, mode, order);
    if (is_linear(layer)) {
      snprintf(a, sizeof a, "layers.%d.linear_attn", layer);
#define T_(s) (snprintf(nm, sizeof nm, "%s." s, a), tensor_of(m, nm))
#define F_(s) (snprintf(nm, sizeof nm, "%s." s, a), f32_of(m, nm))
      or_tensor qkv = T_("in_proj_qkv.weight"), z = T_("in_proj_z.weight"), b = T_("in_proj_b.weight"),
                av = T_("in_proj_a.weight"), outp = T_("out_proj.weight");
      const float* cw = F_("conv1d.weight");
      const float* al = F_("A_log");
      const float* dtb = F_("dt_bias");
      const float* nw = F_("norm.weight");
      or_deltanet_layer(mix, hn, &qkv, &z, &b, &av, cw, al, dtb, nw, &outp,
                        m->rec + (size_t)li * LH * LK * LV, m->conv + (size_t)li * CONV_DIM * CONV_K,
                        mode, order);
      ++li;
    } else {
      snprintf(a, sizeof a, "layers.%d.self_attn", layer);
      or_tensor qp = T_("q_proj.weight"), kp = T_("k_proj.weight"), vp = T_("v_proj.weight"),
                op = T_("o_proj.weight");
      const float* qn = F_("q_norm.weight");
      const float* kn = F_("k_norm.weight");
      or_attention_layer(mix, hn, &qp, &kp, &vp, &op, qn, kn, m->pos,
                         m->kc + (size_t)fi * m->max_ctx * KV_PROJ,
                         m->vc + (size_t)fi * m->max_ctx * KV_PROJ, m->pos, mode, order);
      ++fi;
    }
    for (int i = 0; i < HIDDEN; ++i) h[i] = r[i] + mix[i];
    for (int i = 0; i < HIDDEN; ++i) r[i] = h[i];
    snprintf(nm, sizeof nm, "layers.%d.post_attention_layernorm.weight", layer);
    gemv_rmsnorm_o(hn, h, f32_of(m, nm), HIDDEN, EPS, mode, order);
    snprintf(a, sizeof a, "layers.%d.mlp", layer);
    or_tensor gp = T_("gate_proj.weight"), up = T_("up_proj.weight"), dp = T_("down_proj.weight");
    or_mlp_layer(mix, hn, &gp, &up, &dp, mode, order);
    for (int i = 0; i < HIDDEN; ++i) h[i] = r[i] + mix[i];
#undef T_
#undef F_
  }
}

void or_forward_layers(or_model* m, int l0, int l1, float* h, int mode, int order) {
  layers(m, l0, l1, h, mode, order);
  ++m->pos;
}

int or_decode_token(or_model* m, int tok, float* logits, int mode, int order) {
  float h[HIDDEN];
  const or_tensor emb = tensor_of(m, "embed_tokens.weight");
  or_embed_row(h, emb.w_i8, emb.scale, tok, HIDDEN);   /* qwen_synth.hpp:42-43 */
  layers(m, 0, N_LAYERS, h, mode, order);
  rmsnorm_o(h, h, f32_of(m, "norm.weight"), HIDDEN, EPS, order);   /* qwen_synth.hpp:79 */
  float* lg = logits ? logits : (float*)malloc(sizeof(float) * VOCAB);
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int vt = 0; vt < VOCAB; ++vt)
    lg[vt] = order == OR_ORDER_DEV ? c16_dot_i8(emb.w_i8 + (long)vt * HIDDEN, h, HIDDEN) * emb.scale[vt]
                                   : or_row_dot_i8(emb.w_i8, emb.scale, h, vt, HIDDEN);
  int best = 0;   /* qwen_synth.hpp:81-88: strict >, first index wins */
  float bestv = -1e30f;
  for (int vt = 0; vt < VOCAB; ++vt) {
    if (lg[vt] > bestv) {
      bestv = lg[vt];
      best = vt;
    }
  }
  if (!logits) free(lg);
  ++m->pos;
  return best;
}

int or_model_pos(const or_model* m) { return m->pos; }
float* or_model_rec(or_model* m) { return m->rec; }
float* or_model_conv(or_model* m) { return m->conv; }
float* or_model_kcache(or_model* m) { return m->kc; }
float* or_model_vcache(or_model* m) { return m->vc; }
