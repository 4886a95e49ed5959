/*
 * qh_decode.h -- C ABI of the MI355X (gfx950) batch-1 decode datapath for the
 * Qwen3.5-0.8B-shaped hybrid model (24 layers = [Gated DeltaNet x3, gated GQA
 * attention x1] x6, hidden 1024, tied 248320x1024 int8 head).
 *
 * Every entry point is extern "C", takes plain pointers and sizes, and returns
 * an int status: 0 on success, a negative QH_E* code for an argument / format
 * error detected on the host, or a positive hipError_t value for a HIP runtime
 * failure.  Op-level functions keep the names and argument order of the
 * reference's HLS kernels (namespace qwen in the hls/src headers) with a qh_ prefix;
 * fixed-size arrays become flat row-major device pointers and every function
 * takes a trailing stream (a hipStream_t, or NULL for the null stream).  Op
 * pointers are DEVICE pointers owned by the caller.  The ops keep no static
 * state and are reentrant; calls on one stream run in order.
 *
 * Layouts (all row-major, fp32 unless noted):
 *   int8 GEMV weight   w[out][in] int8, per-output-row scale[out]
 *   DeltaNet state     S[16][128][128]   (k-major: S[h][k][v])
 *   conv history       state[6144][4]    (column 0 kept, unused, as in the reference)
 *   KV cache           kcache/vcache [T_max][2][256] (token-major, kv head, dim)
 *
 * The engine keeps the packed int8 blob written by scripts/pack_weights.py
 * (tensors in kernel read order, 4 KiB aligned, int8 [out,in] followed by fp32
 * [out] scales) resident in HBM, owns all decode state, and replays one decode
 * step as a hipGraph.
 */
#ifndef QH_DECODE_H
#define QH_DECODE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------- */
#define QH_OK 0
#define QH_EINVAL (-1)   /* bad argument (null pointer, bad size)          */
#define QH_ERANGE (-2)   /* token id / position / context out of range      */
#define QH_EIO (-3)      /* file open / read / mmap failure                 */
#define QH_EFORMAT (-4)  /* weight index or blob does not match the layout  */
#define QH_ENOMEM (-5)   /* host or device allocation failed                */
#define QH_ESTATE (-6)   /* engine not in a state that allows the call      */
#define QH_EDEVICE (-7)  /* a hand-over wait of the persistent kernel gave up:
                            every workgroup left the launch; the engine refuses to
                            decode (QH_ESTATE) until qh_engine_reset.  The environment
                            variable QH_POLL_LIMIT, read at engine creation, sets the
                            failed polls a wait allows (default 2^20, about a second):
                            a test hook that forces this path.  A second hook,
                            QH_TAG_START, starts the persistent kernel's hand-over tags
                            at that value instead of 1, so that a test reaches the
                            launch that would run past 2^32 - 1 (the engine then
                            clears the tagged buffers and restarts the tags at 1). */

/* ---- model dimensions (hls/src/types.hpp:20-44) ----------------------- */
#define QH_HIDDEN 1024
#define QH_N_LAYERS 24
#define QH_INTER 3584
#define QH_VOCAB 248320
#define QH_LH 16         /* DeltaNet heads            */
#define QH_LK 128        /* DeltaNet key head dim     */
#define QH_LV 128        /* DeltaNet value head dim   */
#define QH_CONV_DIM 6144
#define QH_CONV_K 4
#define QH_Z_DIM 2048
#define QH_NH 8          /* attention query heads     */
#define QH_NKV 2         /* attention kv heads        */
#define QH_HD 256        /* attention head dim        */
#define QH_Q_PROJ 4096   /* query + output gate, interleaved per head */
#define QH_KV_PROJ 512
#define QH_ROPE_DIM 64
#define QH_N_TENSORS 320 /* entries in weights.idx    */
/* Largest KV context (engine max_ctx, attention T + 1): one layer's cache,
 * 2 KiB per token, is addressed with 32-bit byte offsets. */
#define QH_MAX_CTX 1048575

/* activation precision of the engine's / layer ops' projections */
#define QH_MODE_W8A16 0  /* int8 weights x fp32 activations (hls/src csim semantics) */
#define QH_MODE_W8A8 1   /* int8 weights x per-vector int8 activations, int32 accumulate
                            (golden/model.py with ACT_INT8 = True) */

/* Tensor view into a weight blob (hls/src/types.hpp:51-56 Tensor).  int8
 * tensors set w_i8 + scale, fp32 tensors set w_f32.  Device pointers. */
typedef struct qh_tensor {
  const int8_t* w_i8;
  const float* scale;
  const float* w_f32;
  int out;
  int in;
} qh_tensor;

const char* qh_strerror(int status);

/* ======================================================================
 * Op level.  Each replaces the HLS C++ function cited beside it.
 * ==================================================================== */

/* y[o] = (sum_i float(w[o,i]) * x[i]) * scale[o]            gemv.hpp:28-42 gemv_i8 */
int qh_gemv_i8(float* y, const int8_t* w, const float* scale, const float* x, int out, int in,
               void* stream);
/* y = W x with fp32 W                                       gemv.hpp:46-59 gemv_f32 */
int qh_gemv_f32(float* y, const float* w, const float* x, int out, int in, void* stream);
/* *result = (sum_i float(w[row,i]) * h[i]) * scale[row]     gemv.hpp:63-73 row_dot_i8
 * (the reference returns the float; here it is written to a device scalar) */
int qh_row_dot_i8(float* result, const int8_t* w, const float* scale, const float* h, int row,
                  int in, void* stream);
/* h[i] = float(w[tok,i]) * scale[tok]                        gemv.hpp:76-84 embed_row
 * (tok < 0 -> QH_ERANGE; like the reference, the upper bound is the caller's) */
int qh_embed_row(float* h, const int8_t* w, const float* scale, int tok, int in, void* stream);
/* y = x * (1/sqrt(mean(x^2) + eps)) * (1 + w)                norm.hpp:13-20 rmsnorm */
int qh_rmsnorm(float* y, const float* x, const float* w, int n, float eps, void* stream);
/* y = x * (1/sqrt(mean(x^2) + eps)) * w * silu(z)           norm.hpp:25-33 rmsnorm_gated */
int qh_rmsnorm_gated(float* y, const float* x, const float* w, const float* z, int n, float eps,
                     void* stream);
/* depthwise causal conv, width 4, then SiLU; state[6144][4]  conv1d.hpp:17-38 conv1d_step */
int qh_conv1d_step(float* out, const float* in_ch, float* state, const float* weight, void* stream);
/* cos/sin[64] for a position (theta 1e7, halves mirrored)    rope.hpp:17-27 rope_cos_sin */
int qh_rope_cos_sin(int pos, float* cos_o, float* sin_o, void* stream);
/* rotate dims 0..63 of one 256-dim head in place             rope.hpp:30-41 apply_rope */
int qh_apply_rope(float* x, const float* cos_, const float* sin_, void* stream);
/* v *= 1/sqrt(sum(v^2) + 1e-6)                               deltanet.hpp:131-136 l2norm */
int qh_l2norm(float* v, int n, void* stream);
/* one head of the gated delta rule; S[128][128] updated      deltanet.hpp:58-115 delta_rule_head */
int qh_delta_rule_head(const float* q, const float* k, const float* v, float g, float beta, float* S,
                       float* out, void* stream);
/* all 16 heads; q,k,v,out [16][128]; g,beta [16]; S[16][128][128]
 *                                                            deltanet.hpp:118-127 delta_rule_layer */
int qh_delta_rule_layer(const float* q, const float* k, const float* v, const float* g,
                        const float* beta, float* S, float* out, void* stream);
/* the DeltaNet recurrent step between the projections       deltanet.hpp:154-179 (inside deltanet_layer)
 * short conv + SiLU over the projected qkv [6144] (conv_state [6144][4] and
 * rec [16][128][128] updated in place), beta = sigmoid(b), g = -exp(A_log) softplus(a + dt_bias),
 * l2norm of q and k, q / sqrt(128), the delta rule, per-head gated RMSNorm with silu(z [2048]):
 * out [2048] (the input of out_proj).  The reference has no separate entry for this step; it is
 * the body of deltanet_layer.  Scratch comes from the caller: workspace, 256-byte aligned, at least
 * qh_deltanet_step_workspace() bytes (nothing is allocated). */
size_t qh_deltanet_step_workspace(void);
int qh_deltanet_step(float* out, const float* qkv, const float* z, const float* b, const float* a,
                     const float* conv_w, const float* A_log, const float* dt_bias, const float* gate_norm_w,
                     float* rec, float* conv_state, void* workspace, size_t workspace_bytes, void* stream);
/* full Gated DeltaNet decode step, x already input-normed    deltanet.hpp:141-182 deltanet_layer
 * rec[16][128][128] and conv_state[6144][4] are updated in place. */
int qh_deltanet_layer(float* out, const float* x, const qh_tensor* qkv_w, const qh_tensor* z_w,
                      const qh_tensor* b_w, const qh_tensor* a_w, const float* conv_w,
                      const float* A_log, const float* dt_bias, const float* gate_norm_w,
                      const qh_tensor* out_w, float* rec, float* conv_state, void* stream);
/* gated GQA attention decode step                            attention.hpp:25-95 attention_layer
 * kcache/vcache hold T past tokens as [T][512]; slot T is written; attends over T+1.
 * Unlike the reference (sc[8192]) any T < QH_MAX_CTX within the caller's buffer is
 * accepted (QH_ERANGE beyond). */
int qh_attention_layer(float* out, const float* x, const qh_tensor* q_w, const qh_tensor* k_w,
                       const qh_tensor* v_w, const qh_tensor* o_w, const float* q_norm,
                       const float* k_norm, int pos, float* kcache, float* vcache, int T,
                       void* stream);
/* SwiGLU MLP: down(silu(gate x) * up x)                      mlp.hpp:11-19 mlp_layer */
int qh_mlp_layer(float* out, const float* x, const qh_tensor* gate_w, const qh_tensor* up_w,
                 const qh_tensor* down_w, void* stream);
/* qh_attention_layer (mode QH_MODE_W8A16) or qh_attention_layer_w8a8 (QH_MODE_W8A8) without any
 * allocation: no counterpart in the reference; for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, kernels and results; the intermediate vectors live in one file-scope device array
 * of the library (1.1 MB on every GPU the library runs on, held until the process ends), so
 * T + 1 <= 65536 (above the reference's own sc[8192] bound, attention.hpp:66), else QH_ERANGE.
 * Every call on one GPU uses that GPU's array: calls that overlap on one GPU (other streams,
 * other host threads) race and must be serialised by the caller. */
int qh_attention_layer_noalloc(float* out, const float* x, const qh_tensor* q_w, const qh_tensor* k_w,
                               const qh_tensor* v_w, const qh_tensor* o_w, const float* q_norm,
                               const float* k_norm, int pos, float* kcache, float* vcache, int T, int mode,
                               void* stream);

/* ---- W8A8 (int8 activation) entry points; no C++ counterpart in hls/src ----
 * per-vector symmetric int8: s = amax/127 (1 if amax == 0), q = rint(x/s) clipped to +-127.
 *                          golden/model.py:37-45 _qa; scripts/export_gemv_tv.py:25-30 q_i8_vec */
int qh_quant_act(int8_t* xq, float* sx, const float* x, int n, void* stream);
/* ---- offline weight quantisation (the packer of scripts/pack_weights.py:79-86) ----
 * per output row of w[rows][cols]: s = amax/127 (1 if amax == 0), q = rint(w/s) clipped to
 * +-127, fp32 arithmetic, round half to even.        golden/quant.py:43-49 quant_rows
 * A row holding a NaN or an infinity gets scale NaN and q = 0 (the reference leaves it
 * undefined).  _bf16 takes the raw bfloat16 bits of a safetensors tensor and widens them
 * exactly (golden/loader.py:34-38 _bf16_to_f32). */
int qh_quant_rows(int8_t* q, float* scale, const float* w, int rows, int cols, void* stream);
int qh_quant_rows_bf16(int8_t* q, float* scale, const uint16_t* w, int rows, int cols, void* stream);
/* acc[o] = sum_i w[o,i]*xq[i] in int32; y[o] = float(acc[o]) * sx * scale[o]
 * (acc may be NULL)              rtl/gemv_i8.sv:52-72; scripts/export_gemv_tv.py:49-50 */
int qh_gemv_i8_w8a8(float* y, int32_t* acc, const int8_t* w, const float* scale, const int8_t* xq,
                    const float* sx, int out, int in, void* stream);
/* The RTL's int8 matvec primitive (rtl/matvec_i8.sv: gemv_i8.sv then dequant.sv), for RTL-level
 * parity: acc[o] = sum_i w[o,i]*xq[i] in int32 (exact); then per row
 *   y_q[o] = (acc[o]*mult[o] + 2^(shift-1)) >>> shift   (64-bit product, arithmetic shift)
 * kept to its low outw bits and sign-extended into int32, as the OUTW-bit y_q register keeps it
 * (the reference instantiates SHIFT = 16, OUTQ = 14, OUTW = 16).  1 <= shift <= 62, 1 <= outw <= 32.
 *                                  rtl/dequant.sv:12-29; rtl/gemv_i8.sv:52-72; rtl/matvec_i8.sv */
int qh_matvec_i8(int32_t* y_q, int32_t* acc, const int8_t* w, const int32_t* mult, const int8_t* xq, int out,
                 int in, int shift, int outw, void* stream);
/* Host side (no device memory): mult[o] = llround(sx*sw[o]*2^(outq+shift)) in double, ties away
 * from zero; QH_ERANGE when a multiplier does not fit the 32-bit mult port (the reference's cast
 * would wrap it).                                               rtl/tb/sim_matvec.cpp:36-41 */
int qh_dequant_mult(int32_t* mult, float sx, const float* sw, int out, int outq, int shift);
/* The three layer ops with the projections' inputs quantized where golden/model.py
 * applies _qa (model.py:143,191 / 200,230 / 234,237). Same arguments as above. */
int qh_deltanet_layer_w8a8(float* out, const float* x, const qh_tensor* qkv_w, const qh_tensor* z_w,
                           const qh_tensor* b_w, const qh_tensor* a_w, const float* conv_w,
                           const float* A_log, const float* dt_bias, const float* gate_norm_w,
                           const qh_tensor* out_w, float* rec, float* conv_state, void* stream);
int qh_attention_layer_w8a8(float* out, const float* x, const qh_tensor* q_w, const qh_tensor* k_w,
                            const qh_tensor* v_w, const qh_tensor* o_w, const float* q_norm,
                            const float* k_norm, int pos, float* kcache, float* vcache, int T,
                            void* stream);
int qh_mlp_layer_w8a8(float* out, const float* x, const qh_tensor* gate_w, const qh_tensor* up_w,
                      const qh_tensor* down_w, void* stream);

/* ======================================================================
 * Weight blob layout (scripts/pack_weights.py:25-101, emit_weight_index.py:13-22)
 * ==================================================================== */

/* Total bytes of the packed blob (758,618,112 for the 0.8B shape). */
size_t qh_blob_size(void);
/* Writes the weights.idx text of the canonical layout ("name off nbytes dtype
 * scale_off scale_nbytes out in" per line).  Returns the number of bytes needed
 * (excluding the NUL); writes at most cap bytes when buf is not NULL. */
size_t qh_layout_idx_text(char* buf, size_t cap);
/* Fills a host buffer of qh_blob_size() bytes with seeded synthetic weights in
 * the packed layout (int8 U{-127..127}, scales U[1e-3,1e-2], fp32 tensors per
 * tensor role).  Deterministic in (seed); padding bytes are zero. */
int qh_synth_blob(void* blob, size_t len, uint64_t seed);
/* Seeded fills used by benchmarks and tests (SplitMix64 stream `key`). */
int qh_synth_fill_i8(int8_t* dst, size_t n, uint64_t key);                   /* U{-127..127} */
int qh_synth_fill_uniform(float* dst, size_t n, uint64_t key, float lo, float hi);
int qh_synth_fill_normal(float* dst, size_t n, uint64_t key, float mean, float stddev);

/* ======================================================================
 * Engine: the decode top (hls/src/qwen_synth.hpp:39-92 qwen_top,
 * hls/src/decoder.hpp:62-120 decode_token) with device-resident state.
 * ==================================================================== */
typedef struct qh_engine qh_engine;

/* mmap `blob_path` (run_hls.cpp:27-35) and upload it; `idx_path` (may be NULL)
 * is a weights.idx whose every line must equal the canonical layout
 * (tb_decode.cpp:47-65).  max_ctx bounds the KV cache (tokens, 1 .. QH_MAX_CTX;
 * outside that range QH_ERANGE). */
int qh_engine_create(const char* blob_path, const char* idx_path, int max_ctx, qh_engine** out);
/* Same from a host buffer (copied to the device; the caller may free it). */
int qh_engine_create_from_memory(const void* blob, size_t blob_len, const char* idx_text,
                                 int max_ctx, qh_engine** out);
int qh_engine_destroy(qh_engine* e);
/* QH_MODE_W8A16 (default) or QH_MODE_W8A8. */
int qh_engine_set_mode(qh_engine* e, int mode);
/* How decode_token / generate run a token; both are bit-identical.
 * QH_EXEC_PERSISTENT: one cooperative launch per call runs every token; the
 * workgroups hand each stage's outputs to the next stage's consumers through
 * tagged buffers (no grid barrier).  QH_EXEC_GRAPH (default): one
 * replayed hipGraph of per-stage kernels per token.  No counterpart in the reference (its top is one HLS
 * function); returns QH_ESTATE if the device cannot run the persistent kernel.
 * If a cooperative launch is refused at run time (another process can hold the
 * device's cooperative-launch resources), the engine switches itself to
 * QH_EXEC_GRAPH and completes the call there: qh_engine_get_exec then reports
 * QH_EXEC_GRAPH, qh_engine_exec_fallbacks counts the refused launches, and with
 * QH_VERBOSE=1 in the environment each one is named on stderr. */
#define QH_EXEC_PERSISTENT 0
#define QH_EXEC_GRAPH 1
int qh_engine_set_exec(qh_engine* e, int exec);
int qh_engine_get_exec(const qh_engine* e);
/* Cooperative launches refused so far (each switched the engine to QH_EXEC_GRAPH). */
int qh_engine_exec_fallbacks(const qh_engine* e);
/* workgroups the LM head runs on under executor `exec` (its batches of 8 rows go to wave w of
 * workgroup b as batch 4 b + w, + 4 * grid, ...); QH_ESTATE for the persistent executor when the
 * device has no cooperative launch.  No counterpart in the reference (its head is one loop). */
int qh_engine_head_grid(const qh_engine* e, int exec);
/* Zero recurrent/conv state, empty KV cache, pos = 0 (state.hpp:24-34). */
int qh_engine_reset(qh_engine* e);
/* Decode one token (qwen_top): returns the argmax (ties -> lowest id) in
 * *argmax_out and, if logits is not NULL, all QH_VOCAB logits into the HOST
 * buffer `logits`.  Advances pos by one. */
int qh_decode_token(qh_engine* e, int tok, float* logits, int* argmax_out);
/* The run_hls loop (run_hls.cpp:56-66) on the device: feed n_prompt ids, then
 * greedily generate up to n_new ids, stopping before emitting `eos` (eos < 0:
 * never).  out_ids receives the generated ids, *n_out their count.  The token
 * feedback stays on the device: one persistent launch (or one graph replay per
 * token) and no host round trip between tokens. */
int qh_generate(qh_engine* e, const int* prompt, int n_prompt, int n_new, int eos, int* out_ids,
                int* n_out);
/* Tokens processed so far (DecodeState::pos). */
int qh_engine_pos(const qh_engine* e);
/* Argmax of the most recent completed step (the next greedy token). */
int qh_engine_last_argmax(const qh_engine* e);
/* Duration (ms) of the last persistent-kernel launch, from HIP events recorded
 * on the engine stream right before and after the cooperative launch (0 before
 * the first persistent launch).  Measurement hook; no counterpart in the
 * reference. */
float qh_engine_last_launch_ms(const qh_engine* e);
/* Run layers [l0, l1) of one decode step on a device hidden vector h (in place,
 * [1024]) without embed / final norm / head; state and pos advance as in a
 * full step.  Used for the 4-layer block configuration. */
int qh_engine_forward_layers(qh_engine* e, int l0, int l1, float* h);
/* Measurement hook: runs n_steps decode steps as plain stream launches (the
 * kernels of the step graph, each fed the current token) and returns the mean
 * step time and the mean duration of the LM-head kernel, both from HIP events
 * on the engine stream; the head's events are stamped at the kernel's own start
 * and end (hipExtLaunchKernel), so its duration excludes the dispatch gap.
 * Advances pos like n_steps decode_token calls. */
int qh_engine_profile(qh_engine* e, int n_steps, float* step_ms, float* head_ms);
/* The engine's HIP stream (a hipStream_t). */
void* qh_engine_stream(qh_engine* e);
/* Device pointers of engine-owned buffers (for parity checks):
 * which = 0 blob, 1 rec state [18][16][128][128], 2 conv state [18][6144][4],
 * 3 K cache [6][max_ctx][512], 4 V cache [6][max_ctx][512], 5 hidden h [1024]. */
void* qh_engine_device_ptr(qh_engine* e, int which);

#ifdef __cplusplus
}
#endif
#endif /* QH_DECODE_H */
