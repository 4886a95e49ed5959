// Op-level C ABI: the reference's per-kernel contracts (hls/src/*.hpp) on the
// device.  Every function validates its arguments on the host, enqueues on the
// caller's stream and returns without synchronising.  Layer ops that need
// intermediate buffers take them from the stream-ordered allocator
// (hipMallocAsync / hipFreeAsync on the same stream), so they stay reentrant.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "qh_common.hpp"
#include "qh_kernels.hpp"
#include "qh_layout.hpp"

using namespace qh;

namespace qh {

void rope_row(int pos, float* out64) {
  for (int j = 0; j < kRopeDim / 2; ++j) {
    const float inv = 1.0f / std::pow(kRopeTheta, float(2 * j) / float(kRopeDim));
    const float f = (float)pos * inv;
    out64[j] = std::cos(f);
    out64[32 + j] = std::sin(f);
  }
}

bool verbose() {
  static const bool v = [] {
    const char* s = std::getenv("QH_VERBOSE");
    return s != nullptr && s[0] != '\0' && s[0] != '0';
  }();
  return v;
}

int hip_report(hipError_t e, const char* what, const char* file, int line) {
  if (e == hipSuccess) return QH_OK;
  if (verbose()) std::fprintf(stderr, "[qh] %s:%d: %s -> %s (%d)\n", file, line, what, hipGetErrorString(e), (int)e);
  return (int)e;
}

}  // namespace qh

namespace {

hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Scratch carved into 256-byte aligned pieces: one stream-ordered allocation
// (hipMallocAsync / hipFreeAsync on the caller's stream), or -- for the
// entry point that allocates nothing -- a caller-provided device buffer.
struct Scratch {
  hipStream_t s;
  char* base = nullptr;
  size_t size = 0, used = 0;
  bool owned = false;
  explicit Scratch(hipStream_t st, char* given = nullptr, size_t given_size = 0)
      : s(st), base(given), size(given_size) {}
  int alloc(size_t total) {
    if (base != nullptr) return total <= size ? QH_OK : QH_ERANGE;   // given buffer: just check the fit
    size = total;
    owned = true;
    return hip_status(hipMallocAsync(reinterpret_cast<void**>(&base), total, s));
  }
  template <class T>
  T* take(size_t n) {
    const size_t bytes = (n * sizeof(T) + 255) & ~(size_t)255;
    T* p = reinterpret_cast<T*>(base + used);
    used += bytes;
    return p;
  }
  ~Scratch() {
    if (owned && base) (void)hipFreeAsync(base, s);
  }
};
constexpr size_t rnd(size_t bytes) { return (bytes + 255) & ~(size_t)255; }

// Scratch of one attention_layer call with ns splits: q||gate|k|v, the RoPE row, T and
// the RoPE row index, split maxima / sums / partial contexts, the gated context.
constexpr size_t attention_scratch_bytes(int ns) {
  return rnd(4 * (kQProj + 2 * kKVProj)) + rnd(4 * 64) + rnd(8) + 2 * rnd(4 * 8 * (size_t)ns) +
         rnd(4 * 8 * 256 * (size_t)ns) + rnd(4 * kNH * kHD);
}

// ---- the scratch of qh_attention_layer_noalloc: one file-scope device array ----
// Contexts up to 65536 positions (T + 1 <= 65536; above the reference's own bound,
// sc[8192], attention.hpp:66): at most kAttnMaxSplits splits, 1.1 MB held on every GPU
// the library runs on until the process ends.  In host code `scratch` names a host-side stand-in, not the device
// array: its device address is taken once per device (hipGetSymbolAddress, with that
// device current) and only that address reaches kernels.
constexpr int kNoallocMaxCtx = 65536;
constexpr size_t kNoallocBytes = attention_scratch_bytes(attn_nsplit_max(kNoallocMaxCtx));
static_assert(attn_nsplit_max(kNoallocMaxCtx) == kAttnMaxSplits + 1 && kNoallocBytes < (size_t)2 << 20,
              "a modest, fixed maximum");
__device__ __align__(256) char scratch[kNoallocBytes];
constexpr int kMaxDevices = 64;
char* g_scratch_dev[kMaxDevices] = {};
std::mutex g_scratch_mu;

// The device address of `scratch` on the current device, looked up on the first call there.
int noalloc_scratch(char** out) {
  int dev = 0;
  QH_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return QH_EINVAL;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* ptr = nullptr;
    QH_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (ptr == nullptr) return QH_ENOMEM;
    g_scratch_dev[dev] = static_cast<char*>(ptr);
  }
  *out = g_scratch_dev[dev];
  return QH_OK;
}

bool tensor_i8(const qh_tensor* t, int out, int in) {
  return t && t->w_i8 && t->scale && t->out == out && t->in == in && aligned16(t->w_i8);
}
bool tensor_f32(const qh_tensor* t, int out, int in) {
  return t && t->w_f32 && t->out == out && t->in == in && aligned16(t->w_f32);
}

Seg seg_i8(const int8_t* w, const float* sw, int rows, int batch0, float* out, int epi,
           int rpb = kRowsPerBatch) {
  Seg g;
  g.kind = SEG_I8;
  g.epi = epi;
  g.batch0 = batch0;
  g.rows = rows;
  g.nbatch = (rows + rpb - 1) / rpb;
  g.w = w;
  g.sw = sw;
  g.out = out;
  return g;
}

int check_gemv_shape(int out, int in) {
  if (out <= 0 || in <= 0 || in % 16 != 0 || in > 4096) return QH_EINVAL;
  return QH_OK;
}

// ---- layer compositions (shared by the W8A16 and W8A8 entry points) ----
int deltanet_layer(float* out, const float* x, const qh_tensor* qkv_w, const qh_tensor* z_w,
                   const qh_tensor* b_w, const qh_tensor* a_w, const float* conv_w, const float* A_log,
                   const float* dt_bias, const float* gate_norm_w, const qh_tensor* out_w, float* rec,
                   float* conv_state, int mode, hipStream_t s) {
  if (!out || !x || !conv_w || !A_log || !dt_bias || !gate_norm_w || !rec || !conv_state) return QH_EINVAL;
  if (!tensor_i8(qkv_w, kConvDim, kHidden) || !tensor_i8(z_w, kZDim, kHidden) ||
      !tensor_f32(b_w, kLH, kHidden) || !tensor_f32(a_w, kLH, kHidden) ||
      !tensor_i8(out_w, kHidden, kLH * kLV))
    return QH_EINVAL;
  if (!aligned16(x) || !aligned16(gate_norm_w)) return QH_EINVAL;
  Scratch sc(s);
  QH_TRY(sc.alloc(rnd(4 * kConvDim) + rnd(4 * kZDim) + rnd(4 * kLH * kLV)));
  float* convd = sc.take<float>(kConvDim);
  float* zb = sc.take<float>(kZDim);
  float* o = sc.take<float>(kLH * kLV);
  // in_proj_qkv / z / b / a over the shared activation (deltanet.hpp:149-152, model.py:143-147)
  GemvArgs a;
  a.K = kHidden;
  a.mode = mode;
  a.prologue = P_LOAD;
  a.x = x;
  a.nseg = 2;   // the fp32 gate projections b, a run in the DeltaNet stage
  int b0 = 0;
  a.seg[0] = seg_i8(qkv_w->w_i8, qkv_w->scale, kConvDim, b0, convd, E_CONV);
  a.seg[0].c0 = conv_w;
  a.seg[0].c2 = conv_state;
  b0 += a.seg[0].nbatch;
  a.seg[1] = seg_i8(z_w->w_i8, z_w->scale, kZDim, b0, zb, E_SILU);   // silu(z) for the gated norm
  QH_HIP(launch_gemv(a, 4, s));
  DnArgs d;   // gates (deltanet.hpp:164-165) on x itself, l2norm, delta rule
  d.convd = convd;
  d.gx = x;
  d.wb = b_w->w_f32;
  d.wa = a_w->w_f32;
  d.A_log = A_log;
  d.dt_bias = dt_bias;
  d.mode = mode;
  d.S = rec;
  d.o = o;
  QH_HIP(launch_deltanet(d, s));
  GemvArgs c;   // gated norm -> out_proj (deltanet.hpp:177-181, model.py:191)
  c.K = kLH * kLV;
  c.mode = mode;
  c.prologue = P_GATED;
  c.x = o;
  c.nw = gate_norm_w;
  c.z = zb;
  c.nseg = 1;
  c.rows_per_batch = 4;
  c.seg[0] = seg_i8(out_w->w_i8, out_w->scale, kHidden, 0, out, E_STORE, 4);
  QH_HIP(launch_gemv(c, 1, s));
  return QH_OK;
}

// given: a device buffer of given_size bytes to carve the scratch from (no allocation), or null
int attention_layer(float* out, const float* x, const qh_tensor* q_w, const qh_tensor* k_w,
                    const qh_tensor* v_w, const qh_tensor* o_w, const float* q_norm, const float* k_norm,
                    int pos, float* kcache, float* vcache, int T, int mode, hipStream_t s,
                    char* given = nullptr, size_t given_size = 0) {
  if (!out || !x || !q_norm || !k_norm || !kcache || !vcache) return QH_EINVAL;
  if (T < 0 || pos < 0 || T >= QH_MAX_CTX) return QH_ERANGE;
  if (!tensor_i8(q_w, kQProj, kHidden) || !tensor_i8(k_w, kKVProj, kHidden) ||
      !tensor_i8(v_w, kKVProj, kHidden) || !tensor_i8(o_w, kHidden, kNH * kHD))
    return QH_EINVAL;
  if (!aligned16(x) || !aligned16(q_norm) || !aligned16(k_norm) || !aligned16(kcache) || !aligned16(vcache))
    return QH_EINVAL;
  const int Tn = T + 1;
  const int ns = attn_nsplit(Tn);
  Scratch sc(s, given, given_size);
  QH_TRY(sc.alloc(attention_scratch_bytes(ns)));
  float* qkv = sc.take<float>(kQProj + 2 * kKVProj);   // q||gate | k | v
  float* qg = qkv;
  float* kraw = qkv + kQProj;
  float* vraw = qkv + kQProj + kKVProj;
  float* rope = sc.take<float>(64);
  int* ints = sc.take<int>(2);
  float* pm = sc.take<float>(8 * (size_t)ns);
  float* pl = sc.take<float>(8 * (size_t)ns);
  float* pacc = sc.take<float>(8 * 256 * (size_t)ns);
  float* og = sc.take<float>(kNH * kHD);
  GemvArgs a;   // q / k / v projections (attention.hpp:31-33, model.py:200-207)
  a.K = kHidden;
  a.mode = mode;
  a.prologue = P_LOAD;
  a.x = x;
  a.nseg = 3;
  a.seg[0] = seg_i8(q_w->w_i8, q_w->scale, kQProj, 0, qg, E_STORE);
  a.seg[1] = seg_i8(k_w->w_i8, k_w->scale, kKVProj, a.seg[0].nbatch, kraw, E_STORE);
  a.seg[2] = seg_i8(v_w->w_i8, v_w->scale, kKVProj, a.seg[0].nbatch + a.seg[1].nbatch, vraw, E_STORE);
  QH_HIP(launch_gemv(a, 4, s));
  Floats64 r;
  rope_row(pos, r.v);
  QH_HIP(launch_set_floats(rope, r, 64, s));
  QH_HIP(launch_set_ints(ints, T, 0, s));
  AttnArgs at;
  at.qkv = qkv;
  at.qn = q_norm;
  at.kn = k_norm;
  at.rope = rope;
  at.kc = kcache;
  at.vc = vcache;
  at.T = ints;
  at.rope_row = ints + 1;
  at.pm = pm;
  at.pl = pl;
  at.pacc = pacc;
  at.nsplit_max = ns;
  at.max_ctx = Tn;
  at.og = og;
  QH_HIP(launch_attn(at, s));
  QH_HIP(launch_attn_combine(at, s));
  GemvArgs c;   // o_proj (attention.hpp:94, model.py:230)
  c.K = kNH * kHD;
  c.mode = mode;
  c.prologue = P_LOAD;
  c.x = og;
  c.nseg = 1;
  c.rows_per_batch = 4;
  c.seg[0] = seg_i8(o_w->w_i8, o_w->scale, kHidden, 0, out, E_STORE, 4);
  QH_HIP(launch_gemv(c, 1, s));
  return QH_OK;
}

int mlp_layer(float* out, const float* x, const qh_tensor* gate_w, const qh_tensor* up_w,
              const qh_tensor* down_w, int mode, hipStream_t s) {
  if (!out || !x || !aligned16(x)) return QH_EINVAL;
  if (!tensor_i8(gate_w, kInter, kHidden) || !tensor_i8(up_w, kInter, kHidden) ||
      !tensor_i8(down_w, kHidden, kInter))
    return QH_EINVAL;
  Scratch sc(s);
  QH_TRY(sc.alloc(rnd(4 * kInter)));
  float* act = sc.take<float>(kInter);
  GemvArgs a;   // gate || up as row pairs, SwiGLU in the epilogue (mlp.hpp:14-17)
  a.K = kHidden;
  a.mode = mode;
  a.prologue = P_LOAD;
  a.x = x;
  a.nseg = 1;
  Seg g;
  g.kind = SEG_PAIR;
  g.epi = E_SWIGLU;
  g.rows = 2 * kInter;
  g.nbatch = 2 * kInter / kRowsPerBatch;
  g.w = gate_w->w_i8;
  g.sw = gate_w->scale;
  g.w2 = up_w->w_i8;
  g.sw2 = up_w->scale;
  g.out = act;
  a.seg[0] = g;
  QH_HIP(launch_gemv(a, 4, s));
  GemvArgs c;   // down (mlp.hpp:18, model.py:237)
  c.K = kInter;
  c.mode = mode;
  c.prologue = P_LOAD;
  c.x = act;
  c.nseg = 1;
  c.rows_per_batch = 4;
  c.seg[0] = seg_i8(down_w->w_i8, down_w->scale, kHidden, 0, out, E_STORE, 4);
  QH_HIP(launch_gemv(c, 1, s));
  return QH_OK;
}

}  // namespace

extern "C" {

const char* qh_strerror(int st) {
  switch (st) {
    case QH_OK: return "ok";
    case QH_EINVAL: return "invalid argument";
    case QH_ERANGE: return "token id, position or context out of range";
    case QH_EIO: return "file open/read/map failed";
    case QH_EFORMAT: return "weight index or blob does not match the packed layout";
    case QH_ENOMEM: return "allocation failed";
    case QH_ESTATE: return "engine state does not allow the call";
    case QH_EDEVICE: return "device-side wait timed out";
    default: return st > 0 ? hipGetErrorString((hipError_t)st) : "unknown status";
  }
}

int qh_gemv_i8(float* y, const int8_t* w, const float* scale, const float* x, int out, int in, void* stream) {
  if (!y || !w || !scale || !x || !aligned16(w) || !aligned16(x)) return QH_EINVAL;
  QH_TRY(check_gemv_shape(out, in));
  GemvArgs a;
  a.K = in;
  a.mode = M_W8A16;
  a.prologue = P_LOAD;
  a.x = x;
  a.nseg = 1;
  a.seg[0] = seg_i8(w, scale, out, 0, y, E_STORE);
  return hip_status(launch_gemv(a, 4, S(stream)));
}

int qh_gemv_f32(float* y, const float* w, const float* x, int out, int in, void* stream) {
  if (!y || !w || !x || !aligned16(w) || !aligned16(x)) return QH_EINVAL;
  QH_TRY(check_gemv_shape(out, in));
  GemvArgs a;
  a.K = in;
  a.mode = M_W8A16;
  a.prologue = P_LOAD;
  a.x = x;
  a.nseg = 1;
  Seg g;
  g.kind = SEG_F32;
  g.epi = E_STORE;
  g.rows = out;
  g.nbatch = (out + kRowsPerBatch - 1) / kRowsPerBatch;
  g.wf = w;
  g.out = y;
  a.seg[0] = g;
  return hip_status(launch_gemv(a, 4, S(stream)));
}

int qh_row_dot_i8(float* result, const int8_t* w, const float* scale, const float* h, int row, int in,
                  void* stream) {
  if (!result || !w || !scale || !h || row < 0) return QH_EINVAL;
  const int8_t* r = w + (size_t)row * in;
  if (!aligned16(r) || !aligned16(h)) return QH_EINVAL;
  QH_TRY(check_gemv_shape(1, in));
  GemvArgs a;
  a.K = in;
  a.mode = M_W8A16;
  a.prologue = P_LOAD;
  a.x = h;
  a.nseg = 1;
  a.seg[0] = seg_i8(r, scale + row, 1, 0, result, E_STORE);
  return hip_status(launch_gemv(a, 1, S(stream)));
}

int qh_embed_row(float* h, const int8_t* w, const float* scale, int tok, int in, void* stream) {
  if (!h || !w || !scale || in <= 0) return QH_EINVAL;
  if (tok < 0) return QH_ERANGE;
  return hip_status(launch_embed(h, w, scale, tok, in, S(stream)));
}

int qh_rmsnorm(float* y, const float* x, const float* w, int n, float eps, void* stream) {
  if (!y || !x || !w || n <= 0) return QH_EINVAL;
  return hip_status(launch_rmsnorm(y, x, w, nullptr, n, eps, 0, S(stream)));
}

int qh_rmsnorm_gated(float* y, const float* x, const float* w, const float* z, int n, float eps,
                     void* stream) {
  if (!y || !x || !w || !z || n <= 0) return QH_EINVAL;
  return hip_status(launch_rmsnorm(y, x, w, z, n, eps, 1, S(stream)));
}

int qh_conv1d_step(float* out, const float* in_ch, float* state, const float* weight, void* stream) {
  if (!out || !in_ch || !state || !weight) return QH_EINVAL;
  return hip_status(launch_conv1d(out, in_ch, state, weight, kConvDim, S(stream)));
}

int qh_rope_cos_sin(int pos, float* cos_o, float* sin_o, void* stream) {
  if (!cos_o || !sin_o) return QH_EINVAL;
  if (pos < 0) return QH_ERANGE;
  float r[64];
  rope_row(pos, r);
  Floats64 c, sn;   // rope.hpp:24-25: halves mirrored
  for (int j = 0; j < 32; ++j) {
    c.v[j] = c.v[j + 32] = r[j];
    sn.v[j] = sn.v[j + 32] = r[32 + j];
  }
  QH_HIP(launch_set_floats(cos_o, c, 64, S(stream)));
  return hip_status(launch_set_floats(sin_o, sn, 64, S(stream)));
}

int qh_apply_rope(float* x, const float* cos_, const float* sin_, void* stream) {
  if (!x || !cos_ || !sin_) return QH_EINVAL;
  return hip_status(launch_apply_rope(x, cos_, sin_, S(stream)));
}

int qh_l2norm(float* v, int n, void* stream) {
  if (!v || n <= 0) return QH_EINVAL;
  return hip_status(launch_l2norm(v, n, S(stream)));
}

int qh_delta_rule_head(const float* q, const float* k, const float* v, float g, float beta, float* S_,
                       float* out, void* stream) {
  if (!q || !k || !v || !S_ || !out) return QH_EINVAL;
  hipStream_t s = S(stream);
  Scratch sc(s);
  QH_TRY(sc.alloc(rnd(4 * kConvDim) + rnd(4 * 32)));
  float* convd = sc.take<float>(kConvDim);
  float* gb = sc.take<float>(32);
  QH_HIP(launch_dn_gather(convd, gb, q, k, v, nullptr, nullptr, g, beta, kLK, kLV, 1, s));
  DnArgs d;
  d.convd = convd;
  d.gb = gb;
  d.S = S_;
  d.o = out;
  d.normalize = 0;
  d.heads = 1;
  return hip_status(launch_deltanet(d, s));
}

int qh_delta_rule_layer(const float* q, const float* k, const float* v, const float* g, const float* beta,
                        float* S_, float* out, void* stream) {
  if (!q || !k || !v || !g || !beta || !S_ || !out) return QH_EINVAL;
  hipStream_t s = S(stream);
  Scratch sc(s);
  QH_TRY(sc.alloc(rnd(4 * kConvDim) + rnd(4 * 32)));
  float* convd = sc.take<float>(kConvDim);
  float* gb = sc.take<float>(32);
  QH_HIP(launch_dn_gather(convd, gb, q, k, v, g, beta, 0.0f, 0.0f, 2048, 2048, 16, s));
  DnArgs d;
  d.convd = convd;
  d.gb = gb;
  d.S = S_;
  d.o = out;
  d.normalize = 0;
  d.heads = 16;
  return hip_status(launch_deltanet(d, s));
}

// The scratch of qh_deltanet_step: post-conv qkv, g | beta, the delta-rule output.
constexpr size_t kDnStepWorkspace = rnd(4 * kConvDim) + rnd(4 * 2 * kLH) + rnd(4 * kLH * kLV);
size_t qh_deltanet_step_workspace(void) { return kDnStepWorkspace; }

int qh_deltanet_step(float* out, const float* qkv, const float* z, const float* b, const float* a,
                     const float* conv_w, const float* A_log, const float* dt_bias, const float* gate_norm_w,
                     float* rec, float* conv_state, void* workspace, size_t workspace_bytes, void* stream) {
  if (!out || !qkv || !z || !b || !a || !conv_w || !A_log || !dt_bias || !gate_norm_w || !rec || !conv_state ||
      !workspace)
    return QH_EINVAL;
  if (workspace_bytes < kDnStepWorkspace || (reinterpret_cast<uintptr_t>(workspace) & 255)) return QH_EINVAL;
  hipStream_t s = S(stream);
  Scratch sc(s, static_cast<char*>(workspace), workspace_bytes);
  float* convd = sc.take<float>(kConvDim);
  float* gb = sc.take<float>(2 * kLH);
  float* o = sc.take<float>(kLH * kLV);
  QH_HIP(launch_dn_step_pre(convd, gb, qkv, conv_state, conv_w, b, a, A_log, dt_bias, s));
  DnArgs d;   // l2norm, q scale, delta rule (deltanet.hpp:166-175)
  d.convd = convd;
  d.gb = gb;
  d.S = rec;
  d.o = o;
  d.heads = kLH;
  QH_HIP(launch_deltanet(d, s));
  // per-head gated RMSNorm with silu(z) (deltanet.hpp:177-179)
  return hip_status(launch_rmsnorm(out, o, gate_norm_w, z, kLV, kEps, 1, s, kLH));
}

int qh_deltanet_layer(float* out, const float* x, const qh_tensor* qkv_w, const qh_tensor* z_w,
                      const qh_tensor* b_w, const qh_tensor* a_w, const float* conv_w, const float* A_log,
                      const float* dt_bias, const float* gate_norm_w, const qh_tensor* out_w, float* rec,
                      float* conv_state, void* stream) {
  return deltanet_layer(out, x, qkv_w, z_w, b_w, a_w, conv_w, A_log, dt_bias, gate_norm_w, out_w, rec,
                        conv_state, M_W8A16, S(stream));
}
int qh_deltanet_layer_w8a8(float* out, const float* x, const qh_tensor* qkv_w, const qh_tensor* z_w,
                           const qh_tensor* b_w, const qh_tensor* a_w, const float* conv_w,
                           const float* A_log, const float* dt_bias, const float* gate_norm_w,
                           const qh_tensor* out_w, float* rec, float* conv_state, void* stream) {
  return deltanet_layer(out, x, qkv_w, z_w, b_w, a_w, conv_w, A_log, dt_bias, gate_norm_w, out_w, rec,
                        conv_state, M_W8A8, S(stream));
}

int qh_attention_layer(float* out, const float* x, const qh_tensor* q_w, const qh_tensor* k_w,
                       const qh_tensor* v_w, const qh_tensor* o_w, const float* q_norm, const float* k_norm,
                       int pos, float* kcache, float* vcache, int T, void* stream) {
  return attention_layer(out, x, q_w, k_w, v_w, o_w, q_norm, k_norm, pos, kcache, vcache, T, M_W8A16,
                         S(stream));
}
int qh_attention_layer_w8a8(float* out, const float* x, const qh_tensor* q_w, const qh_tensor* k_w,
                            const qh_tensor* v_w, const qh_tensor* o_w, const float* q_norm,
                            const float* k_norm, int pos, float* kcache, float* vcache, int T, void* stream) {
  return attention_layer(out, x, q_w, k_w, v_w, o_w, q_norm, k_norm, pos, kcache, vcache, T, M_W8A8,
                         S(stream));
}

int qh_attention_layer_noalloc(float* out, const float* x, const qh_tensor* q_w, const qh_tensor* k_w,
                               const qh_tensor* v_w, const qh_tensor* o_w, const float* q_norm,
                               const float* k_norm, int pos, float* kcache, float* vcache, int T, int mode,
                               void* stream) {
  if (mode != QH_MODE_W8A16 && mode != QH_MODE_W8A8) return QH_EINVAL;
  if (T < 0 || T + 1 > kNoallocMaxCtx) return QH_ERANGE;
  char* base = nullptr;
  QH_TRY(noalloc_scratch(&base));
  if (attention_scratch_bytes(attn_nsplit(T + 1)) > kNoallocBytes) return QH_ERANGE;
  return attention_layer(out, x, q_w, k_w, v_w, o_w, q_norm, k_norm, pos, kcache, vcache, T,
                         mode == QH_MODE_W8A8 ? M_W8A8 : M_W8A16, S(stream), base, kNoallocBytes);
}

int qh_mlp_layer(float* out, const float* x, const qh_tensor* gate_w, const qh_tensor* up_w,
                 const qh_tensor* down_w, void* stream) {
  return mlp_layer(out, x, gate_w, up_w, down_w, M_W8A16, S(stream));
}
int qh_mlp_layer_w8a8(float* out, const float* x, const qh_tensor* gate_w, const qh_tensor* up_w,
                      const qh_tensor* down_w, void* stream) {
  return mlp_layer(out, x, gate_w, up_w, down_w, M_W8A8, S(stream));
}

int qh_quant_act(int8_t* xq, float* sx, const float* x, int n, void* stream) {
  if (!xq || !sx || !x || n <= 0) return QH_EINVAL;
  return hip_status(launch_quant(xq, sx, x, n, S(stream)));
}

int qh_quant_rows(int8_t* q, float* scale, const float* w, int rows, int cols, void* stream) {
  if (!q || !scale || !w || rows <= 0 || cols <= 0) return QH_EINVAL;
  return hip_status(launch_quant_rows(q, scale, w, rows, cols, S(stream)));
}

int qh_quant_rows_bf16(int8_t* q, float* scale, const uint16_t* w, int rows, int cols, void* stream) {
  if (!q || !scale || !w || rows <= 0 || cols <= 0) return QH_EINVAL;
  return hip_status(launch_quant_rows_bf16(q, scale, w, rows, cols, S(stream)));
}

int qh_gemv_i8_w8a8(float* y, int32_t* acc, const int8_t* w, const float* scale, const int8_t* xq,
                    const float* sx, int out, int in, void* stream) {
  if (!y || !w || !scale || !xq || !sx || !aligned16(w) || !aligned16(xq)) return QH_EINVAL;
  QH_TRY(check_gemv_shape(out, in));
  GemvArgs a;
  a.K = in;
  a.mode = M_W8A8;
  a.prologue = P_LOADQ;
  a.xq = xq;
  a.sx = sx;
  a.nseg = 1;
  a.seg[0] = seg_i8(w, scale, out, 0, y, acc ? E_ACC : E_STORE);
  a.seg[0].acc_out = acc;
  return hip_status(launch_gemv(a, 4, S(stream)));
}

int qh_matvec_i8(int32_t* y_q, int32_t* acc, const int8_t* w, const int32_t* mult, const int8_t* xq, int out,
                 int in, int shift, int outw, void* stream) {
  if (!y_q || !acc || !w || !mult || !xq || !aligned16(w) || !aligned16(xq)) return QH_EINVAL;
  if (shift < 1 || shift > 62 || outw < 1 || outw > 32) return QH_EINVAL;
  QH_TRY(check_gemv_shape(out, in));
  GemvArgs a;   // gemv_i8.sv: exact int32 accumulators, no scales
  a.K = in;
  a.mode = M_W8A8;
  a.prologue = P_LOADQ;
  a.xq = xq;
  a.nseg = 1;
  a.seg[0] = seg_i8(w, nullptr, out, 0, nullptr, E_ACCI);
  a.seg[0].acc_out = acc;
  hipStream_t s = S(stream);
  QH_HIP(launch_gemv(a, 4, s));
  return hip_status(launch_fixed_dequant(y_q, acc, mult, out, shift, outw, s));   // dequant.sv
}

int qh_dequant_mult(int32_t* mult, float sx, const float* sw, int out, int outq, int shift) {
  if (!mult || !sw || out <= 0 || shift < 1 || shift > 62 || outq < 0 || outq + shift > 62) return QH_EINVAL;
  const double f = std::ldexp(1.0, outq + shift);
  for (int o = 0; o < out; ++o) {   // sim_matvec.cpp:37-40, in double, half away from zero
    const double c = (double)sx * (double)sw[o] * f;
    if (!(std::fabs(c) < 2147483647.5)) return QH_ERANGE;   // would not fit the 32-bit mult port
    mult[o] = (int32_t)std::llround(c);
  }
  return QH_OK;
}

// ---- layout / synthetic weights ----
size_t qh_blob_size(void) { return (size_t)canonical_layout().total; }

size_t qh_layout_idx_text(char* buf, size_t cap) {
  const std::string t = idx_text(canonical_layout());
  if (buf && cap > 0) {
    const size_t n = t.size() < cap - 1 ? t.size() : cap - 1;
    std::memcpy(buf, t.data(), n);
    buf[n] = '\0';
  }
  return t.size();
}

int qh_synth_blob(void* blob, size_t len, uint64_t seed) {
  const Layout& L = canonical_layout();
  if (!blob || len < L.total) return QH_EINVAL;
  synth_blob(static_cast<uint8_t*>(blob), L, seed);
  return QH_OK;
}

int qh_synth_fill_i8(int8_t* dst, size_t n, uint64_t key) {
  if (!dst) return QH_EINVAL;
  fill_i8(dst, n, key);
  return QH_OK;
}
int qh_synth_fill_uniform(float* dst, size_t n, uint64_t key, float lo, float hi) {
  if (!dst) return QH_EINVAL;
  fill_uniform(dst, n, key, lo, hi);
  return QH_OK;
}
int qh_synth_fill_normal(float* dst, size_t n, uint64_t key, float mean, float stddev) {
  if (!dst) return QH_EINVAL;
  fill_normal(dst, n, key, mean, stddev);
  return QH_OK;
}

}  // extern "C"
