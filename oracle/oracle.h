/*
 * oracle.h -- CPU restatement of the reference decode datapath.  TEST
 * INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg as the checker; never linked into the product.
 *
 * Two evaluation orders of the same algorithm:
 *   OR_ORDER_REF  -- the reference's own loop order: sequential fp32 sums,
 *                    unfused multiply-add, glibc expf/log1pf/powf/cosf/sinf
 *                    (the hls/src headers compiled with -ffp-contract=off,
 *                    hls/Makefile:14-15).  Pinned bit-exactly against the
 *                    reference headers compiled in oracle/_ref.
 *   OR_ORDER_DEV  -- the device-order twin: the identical algorithm with the
 *                    fixed reduction trees and the exp/log routines the gfx950
 *                    kernels use, so the HIP path can be compared bit for bit.
 *                    Pinned against OR_ORDER_REF at tolerance.
 *
 * Activation modes: OR_W8A16 (hls/src semantics: int8 weights x fp32 x) and
 * OR_W8A8 (golden/model.py with ACT_INT8: per-vector int8 activations where
 * model.py applies _qa, int32 accumulation, dequant float(acc)*sx*sw as in
 * scripts/export_gemv_tv.py:298-299).
 */
#ifndef QH_ORACLE_H
#define QH_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_ORDER_REF 0
#define OR_ORDER_DEV 1
#define OR_W8A16 0
#define OR_W8A8 1

typedef struct or_tensor {   /* hls/src/types.hpp:51-56 */
  const int8_t* w_i8;
  const float* scale;
  const float* w_f32;
  int out, in;
} or_tensor;

/* threads for independent row loops (results are thread-count independent) */
void or_set_threads(int n);

/* ---- scalar nonlinearities (activations.hpp:7-14) ---- */
float or_silu(float x, int order);
float or_sigmoid(float x, int order);
float or_softplus(float x, int order);
float or_expf(float x, int order);
/* device-order exp / log1p (own polynomial routines), exposed for tests */
float or_dev_expf(float x);
float or_dev_log1pf(float x);

/* ---- primitive kernels (reference loop order) ---- */
void or_gemv_i8(float* y, const int8_t* w, const float* scale, const float* x, int out, int in);
void or_gemv_f32(float* y, const float* w, const float* x, int out, int in);
float or_row_dot_i8(const int8_t* w, const float* scale, const float* h, int row, int in);
void or_embed_row(float* h, const int8_t* w, const float* scale, int tok, int in);
void or_rmsnorm(float* y, const float* x, const float* w, int n, float eps);
void or_rmsnorm_gated(float* y, const float* x, const float* w, const float* z, int n, float eps);
void or_conv1d_step(float* out, const float* in_ch, float* state, const float* weight);
void or_rope_cos_sin(int pos, float* cos_o, float* sin_o);
void or_apply_rope(float* x, const float* cos_, const float* sin_);
void or_l2norm(float* v, int n);
void or_delta_rule_head(const float* q, const float* k, const float* v, float g, float beta, float* S,
                        float* out);
void or_delta_rule_layer(const float* q, const float* k, const float* v, const float* g,
                         const float* beta, float* S, float* out);

/* ---- device-order primitives: the bit-exact twins of the gfx950 op kernels ---- */
void or_dev_gemv_i8(float* y, const int8_t* w, const float* scale, const float* x, int out, int in);
void or_dev_gemv_f32(float* y, const float* w, const float* x, int out, int in);
void or_dev_rmsnorm(float* y, const float* x, const float* w, int n, float eps);
void or_dev_rmsnorm_gated(float* y, const float* x, const float* w, const float* z, int n, float eps);
void or_dev_l2norm(float* v, int n);
void or_dev_conv1d_step(float* out, const float* in_ch, float* state, const float* weight);
void or_dev_delta_rule_head(const float* q, const float* k, const float* v, float g, float beta, float* S,
                            float* out);
void or_dev_delta_rule_layer(const float* q, const float* k, const float* v, const float* g,
                             const float* beta, float* S, float* out);
/* act-quant with the device's reciprocal-corrected quotient (must equal or_quant_act) */
void or_quant_act_markstein(int8_t* q, float* s, const float* x, int n);

/* ---- W8A8 primitives ---- */
/* model.py:37-45 _qa / export_gemv_tv.py:25-30 q_i8_vec */
void or_quant_act(int8_t* q, float* s, const float* x, int n);
/* quant.py:43-49 quant_rows: per row or_quant_act; a row with a non-finite
 * value gets scale NaN and q = 0 (undefined in the reference) */
void or_quant_rows(int8_t* q, float* s, const float* w, int rows, int cols);
/* rtl/matvec_i8.sv: int32 acc, then dequant.sv's (acc*mult + 2^(shift-1)) >>> shift in outw bits */
void or_matvec_fixed(int32_t* yq, int32_t* acc, const int8_t* w, const int32_t* mult, const int8_t* xq, int out,
                     int in, int shift, int outw);
/* export_gemv_tv.py:298-299: exact int32 acc, y = float(acc) * sx * sw */
void or_gemv_w8a8(float* y, int32_t* acc, const int8_t* w, const float* sw, const int8_t* xq, float sx,
                  int out, int in);
/* int64 brute force of the same accumulator (independent of the int32 loop) */
void or_gemv_acc_i64(int64_t* acc, const int8_t* w, const int8_t* xq, int out, int in);

/* ---- layer ops (mode OR_W8A16 / OR_W8A8, order REF / DEV) ---- */
/* BASELINE config C2: the recurrent step between the projections (deltanet.hpp:154-179) on the
 * projected qkv [6144], z [2048], b [16], a [16]; og = the gated-normed heads [2048] (fp32 order). */
void or_deltanet_step(float* og, const float* qkv, const float* z, const float* b, const float* a,
                      const float* conv_w, const float* A_log, const float* dt_bias, const float* gate_norm_w,
                      float* rec, float* conv_state, int order);
void or_deltanet_layer(float* out, const float* x, const or_tensor* qkv_w, const or_tensor* z_w,
                       const or_tensor* b_w, const or_tensor* a_w, const float* conv_w,
                       const float* A_log, const float* dt_bias, const float* gate_norm_w,
                       const or_tensor* out_w, float* rec, float* conv_state, int mode, int order);
void or_attention_layer(float* out, const float* x, const or_tensor* q_w, const or_tensor* k_w,
                        const or_tensor* v_w, const or_tensor* o_w, const float* q_norm,
                        const float* k_norm, int pos, float* kcache, float* vcache, int T, int mode,
                        int order);
void or_mlp_layer(float* out, const float* x, const or_tensor* gate_w, const or_tensor* up_w,
                  const or_tensor* down_w, int mode, int order);

/* ---- whole-model decode (qwen_synth.hpp:39-92 qwen_top) ---- */
typedef struct or_model or_model;
/* blob: packed weights; idx_text: weights.idx contents (tb_decode.cpp:47-65) */
or_model* or_model_new(const uint8_t* blob, const char* idx_text, int max_ctx);
void or_model_free(or_model* m);
void or_model_reset(or_model* m);
/* returns argmax (strict >, first index on ties) and fills logits[VOCAB] if not NULL */
int or_decode_token(or_model* m, int tok, float* logits, int mode, int order);
/* layers [l0,l1) on h in place (no embed / head), advances pos */
void or_forward_layers(or_model* m, int l0, int l1, float* h, int mode, int order);
int or_model_pos(const or_model* m);
float* or_model_rec(or_model* m);     /* [18][16][128][128] */
float* or_model_conv(or_model* m);    /* [18][6144][4] */
float* or_model_kcache(or_model* m);  /* [6][max_ctx][512] */
float* or_model_vcache(or_model* m);

#ifdef __cplusplus
}
#endif
#endif
