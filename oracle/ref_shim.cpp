// extern "C" wrappers over the reference's HLS C++ kernels.  TEST
// INFRASTRUCTURE: compiled by oracle/Makefile directly from the headers where
// they lie (/root/reference/hls/src, passed with -I) into oracle/_ref/libqref.so,
// with the reference's csim flags (hls/Makefile:14-15: -O2 -ffp-contract=off).
// Used only to pin the C restatement in oracle.c and as the CPU baseline.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <sstream>
#include <string>

#include "decoder.hpp"
#include "qwen_synth.hpp"

using namespace qwen;

namespace {
struct RefTensor {   // same field order as or_tensor / qh_tensor
  const int8_t* w_i8;
  const float* scale;
  const float* w_f32;
  int out, in;
};
Tensor T(const RefTensor* r) {
  Tensor t;
  t.w_i8 = r->w_i8;
  t.scale = r->scale;
  t.w_f32 = r->w_f32;
  t.out = r->out;
  t.in = r->in;
  return t;
}
}  // namespace

extern "C" {

void ref_gemv_i8(float* y, const int8_t* w, const float* s, const float* x, int out, int in) {
  gemv_i8(y, w, s, x, out, in);
}
void ref_gemv_f32(float* y, const float* w, const float* x, int out, int in) { gemv_f32(y, w, x, out, in); }
float ref_row_dot_i8(const int8_t* w, const float* s, const float* h, int row, int in) {
  return row_dot_i8(w, s, h, row, in);
}
void ref_embed_row(float* h, const int8_t* w, const float* s, int tok, int in) { embed_row(h, w, s, tok, in); }
void ref_rmsnorm(float* y, const float* x, const float* w, int n, float eps) { rmsnorm(y, x, w, n, eps); }
void ref_rmsnorm_gated(float* y, const float* x, const float* w, const float* z, int n, float eps) {
  rmsnorm_gated(y, x, w, z, n, eps);
}
float ref_silu(float x) { return silu(x); }
float ref_sigmoid(float x) { return sigmoidf(x); }
float ref_softplus(float x) { return softplusf(x); }
void ref_conv1d_step(float* out, const float* in, float* state, const float* w) {
  conv1d_step(out, in, reinterpret_cast<float(*)[CONV_K]>(state), w);
}
void ref_rope_cos_sin(int pos, float* c, float* s) { rope_cos_sin(pos, c, s); }
// The recurrent step between deltanet_layer's projections, from the
// reference's own functions in deltanet_layer's order (deltanet.hpp:154-179): conv1d_step,
// the gates, l2norm and q scaling, delta_rule_layer, per-head rmsnorm_gated.
void ref_deltanet_step(float* og, const float* qkv, const float* z, const float* b, const float* a,
                       const float* conv_w, const float* A_log, const float* dt_bias, const float* gate_norm_w,
                       float* rec, float* conv_state) {
  static float convd[CONV_DIM], q[H][K], k[H][K], v[H][V], g[H], beta[H], o[H][V];
  conv1d_step(convd, qkv, reinterpret_cast<float(*)[CONV_K]>(conv_state), conv_w);
  for (int h = 0; h < H; ++h) {
    for (int i = 0; i < K; ++i) q[h][i] = convd[h * K + i];
    for (int i = 0; i < K; ++i) k[h][i] = convd[VALUE_DIM + h * K + i];
    for (int i = 0; i < V; ++i) v[h][i] = convd[2 * VALUE_DIM + h * V + i];
    beta[h] = sigmoidf(b[h]);
    g[h] = -std::exp(A_log[h]) * softplusf(a[h] + dt_bias[h]);
    l2norm(q[h], K);
    l2norm(k[h], K);
    const float scale = 1.0f / std::sqrt(float(K));
    for (int i = 0; i < K; ++i) q[h][i] *= scale;
  }
  delta_rule_layer(q, k, v, g, beta, reinterpret_cast<float(*)[K][V]>(rec), o);
  for (int h = 0; h < H; ++h) rmsnorm_gated(&og[h * V], o[h], gate_norm_w, &z[h * V], V, EPS);
}
void ref_apply_rope(float* x, const float* c, const float* s) { apply_rope(x, c, s); }
void ref_l2norm(float* v, int n) { l2norm(v, n); }
void ref_delta_rule_head(const float* q, const float* k, const float* v, float g, float beta, float* S,
                         float* out) {
  delta_rule_head(q, k, v, g, beta, reinterpret_cast<float(*)[V]>(S), out);
}
void ref_delta_rule_layer(const float* q, const float* k, const float* v, const float* g, const float* beta,
                          float* S, float* out) {
  delta_rule_layer(reinterpret_cast<const float(*)[K]>(q), reinterpret_cast<const float(*)[K]>(k),
                   reinterpret_cast<const float(*)[V]>(v), g, beta, reinterpret_cast<float(*)[K][V]>(S),
                   reinterpret_cast<float(*)[V]>(out));
}
void ref_deltanet_layer(float* out, const float* x, const RefTensor* qkv, const RefTensor* z,
                        const RefTensor* b, const RefTensor* a, const float* conv_w, const float* A_log,
                        const float* dt_bias, const float* nw, const RefTensor* outw, float* rec,
                        float* conv) {
  deltanet_layer(out, x, T(qkv), T(z), T(b), T(a), conv_w, A_log, dt_bias, nw, T(outw),
                 reinterpret_cast<float(*)[K][V]>(rec), reinterpret_cast<float(*)[CONV_K]>(conv));
}
void ref_attention_layer(float* out, const float* x, const RefTensor* q, const RefTensor* k,
                         const RefTensor* v, const RefTensor* o, const float* qn, const float* kn, int pos,
                         float* kc, float* vc, int T_) {
  attention_layer(out, x, T(q), T(k), T(v), T(o), qn, kn, pos, kc, vc, T_);
}
void ref_mlp_layer(float* out, const float* x, const RefTensor* g, const RefTensor* u, const RefTensor* d) {
  mlp_layer(out, x, T(g), T(u), T(d));
}

// ---- whole-model decode (qwen_synth.hpp qwen_top / decoder.hpp decode_token)
void* ref_state_new() {
  DecodeState* st = new DecodeState();
  st->reset();
  return st;
}
void ref_state_free(void* st) { delete static_cast<DecodeState*>(st); }
void ref_state_reset(void* st) { static_cast<DecodeState*>(st)->reset(); }
int ref_state_pos(void* st) { return static_cast<DecodeState*>(st)->pos; }
float* ref_state_rec(void* st) { return &static_cast<DecodeState*>(st)->rec[0][0][0][0]; }
float* ref_state_conv(void* st) { return &static_cast<DecodeState*>(st)->conv[0][0][0]; }
float* ref_state_kc(void* st, int fi) { return static_cast<DecodeState*>(st)->kc[fi].data(); }
float* ref_state_vc(void* st, int fi) { return static_cast<DecodeState*>(st)->vc[fi].data(); }
int ref_qwen_top(const uint8_t* blob, void* st, int tok, float* logits) {
  return qwen_top(blob, *static_cast<DecodeState*>(st), tok, logits);
}
// decoder.hpp path, addressed through a weights.idx text (tb_decode.cpp:47-65)
int ref_decode_token(const uint8_t* blob, const char* idx_text, void* st, int tok, float* logits) {
  WeightBlob W;
  W.base = blob;
  std::istringstream g(idx_text);
  std::string name;
  uint64_t off, nbytes, so, sn;
  int dtype, out, in;
  while (g >> name >> off >> nbytes >> dtype >> so >> sn >> out >> in) {
    Entry e;
    e.off = off;
    e.scale_off = so;
    e.dtype = dtype;
    e.out = out;
    e.in = in;
    W.idx[name] = e;
  }
  return decode_token(W, *static_cast<DecodeState*>(st), tok, logits);
}
}
