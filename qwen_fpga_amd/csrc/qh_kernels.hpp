// Kernel argument structs and launch wrappers shared by the op-level C ABI
// (qh_ops.hip) and the engine (qh_engine.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qh {

constexpr int kRowsPerBatch = 8;     // rows one wave reduces together (LM head, large GEMVs)
constexpr int kAttnSplit = 16;       // positions per attention split, contexts up to kAttnShortMax
// Longer contexts: splits of attn_split_len(Tn) positions, a multiple of 4 and
// at most kAttnMaxSplitLen, so that there are at most kAttnMaxSplits splits per
// kv head up to 65536 positions (the units fill the GPU once; the split
// partials are 2 / P of the cache bytes).
constexpr int kAttnShortMax = 2048;
constexpr int kAttnMaxSplits = 128;
constexpr int kAttnMaxSplitLen = 512;
// positions per split for a context of Tn positions (the slot of this token included)
__host__ __device__ constexpr int attn_split_len(int Tn) {
  return Tn <= kAttnShortMax ? kAttnSplit
                             : (4 * ((Tn + 4 * kAttnMaxSplits - 1) / (4 * kAttnMaxSplits)) < kAttnMaxSplitLen
                                    ? 4 * ((Tn + 4 * kAttnMaxSplits - 1) / (4 * kAttnMaxSplits))
                                    : kAttnMaxSplitLen);
}
// Splits of a context of Tn positions: up to kAttnShortMax the Tn - 1 cached
// positions in splits of kAttnSplit, then the new position as a split of its
// own (at most 129); above, splits of attn_split_len(Tn) (at most kAttnMaxSplits).
__host__ __device__ constexpr int attn_nsplit(int Tn) {
  return Tn <= kAttnShortMax ? (Tn - 1 + kAttnSplit - 1) / kAttnSplit + 1
                             : (Tn + attn_split_len(Tn) - 1) / attn_split_len(Tn);
}
// the most splits any context up to max_ctx positions takes (buffer sizes)
__host__ __device__ constexpr int attn_nsplit_max(int max_ctx) {
  return max_ctx <= kAttnShortMax ? attn_nsplit(max_ctx)
                                  : (attn_nsplit(kAttnShortMax) > kAttnMaxSplits ? attn_nsplit(kAttnShortMax)
                                                                                 : kAttnMaxSplits);
}
static_assert(attn_nsplit(kAttnShortMax) == kAttnMaxSplits + 1 && attn_nsplit(kAttnShortMax + 1) <= kAttnMaxSplits,
              "split counts at the short / long boundary");
constexpr int kDnVQuarters = 4;      // DeltaNet workgroups per head (32 v columns each)
constexpr int kDnSlots = 5;          // persistent kernel: DeltaNet state tiles per workgroup (LDS)

enum SegKind : int { SEG_I8 = 0, SEG_F32 = 1, SEG_PAIR = 2 };
enum Epi : int {
  E_STORE = 0,   // out[row] = y
  E_RESID = 1,   // out[row] = out[row] + y                    (h = r + mix)
  E_CONV = 2,    // depthwise conv + SiLU into out, state c2 updated (conv1d.hpp:17-38)
  E_GATE_B = 3,  // out[row] = sigmoid(y)                     (beta, deltanet.hpp:164)
  E_GATE_A = 4,  // out[row] = -exp(A_log)*softplus(y+dt_bias) (g, deltanet.hpp:165)
  E_SWIGLU = 5,  // pair rows (gate i, up i): out[i] = silu(g)*u (mlp.hpp:17)
  E_ACC = 6,     // out[row] = y and acc_out[row] = int32 accumulator (W8A8 op)
  E_SILU = 7,    // out[row] = silu(y)  (the gated norm's silu(z), norm.hpp:32)
  E_ACCI = 8,    // acc_out[row] = int32 accumulator only (the RTL's gemv_i8; sw may be null)
};
enum Prologue : int {
  P_LOAD = 0,    // x[K] fp32 as given
  P_NORM = 1,    // rmsnorm(x, nw) with (1+w) (norm.hpp:13-20); optional embed row first
  P_GATED = 2,   // per-head rmsnorm_gated(o, nw, z) over 16 x 128 (deltanet.hpp:177-179);
                 // z holds silu(z) already (E_SILU of the producing GEMV)
  P_LOADQ = 3,   // int8 xq[K] + scale sx given (W8A8 op)
};
enum Mode : int { M_W8A16 = 0, M_W8A8 = 1 };

struct Seg {
  int kind = SEG_I8, epi = E_STORE;
  int batch0 = 0, nbatch = 0, rows = 0;   // batch range in the launch; valid rows
  const int8_t* w = nullptr;              // int8 [rows][K]
  const float* sw = nullptr;              // fp32 [rows] per-row scales
  const float* wf = nullptr;              // fp32 [rows][K] (SEG_F32)
  const int8_t* w2 = nullptr;             // SEG_PAIR second matrix (up)
  const float* sw2 = nullptr;
  float* out = nullptr;
  int32_t* acc_out = nullptr;
  const float* res = nullptr;             // E_RESID: residual input (== out for in-place plain I/O)
  int res_st = 0;                         // stage that produced res (tagged I/O)
  const float* c0 = nullptr;              // E_CONV: taps [C][4]   E_GATE_A: A_log
  const float* c1 = nullptr;              // E_GATE_A: dt_bias
  float* c2 = nullptr;                    // E_CONV: state [C][4]
};

struct GemvArgs {
  int K = 0, mode = M_W8A16, prologue = P_LOAD;
  int rows_per_batch = 8;       // 1, 4 or 8 rows reduced together per wave
  const float* x = nullptr;     // P_LOAD / P_NORM input, P_GATED o
  const float* nw = nullptr;    // P_NORM [K] gain, P_GATED [128] gain
  int nw_lanes = 0;             // P_NORM, K = 1024: nw in the lane-interleaved order (load16c)
  const float* z = nullptr;     // P_GATED gate input [2048]
  const int8_t* xq = nullptr;   // P_LOADQ
  const float* sx = nullptr;
  float eps = 1e-6f;
  const int8_t* emb = nullptr;  // P_NORM: if set, x = emb[tok]*emb_s[tok] (gemv.hpp:76-84)
  const float* emb_s = nullptr;
  const int* tok = nullptr;     // token id in device memory, or
  int tokv = 0;                 // the token id itself when tok is null
  float* h_out = nullptr;       // receives the embedded row (block 0)
  const int* done = nullptr;    // engine stop flag (skip when *done != 0)
  int x_st = 0, z_st = 0;       // producer stages of x / z (tagged I/O)
  int out_st = 0;               // this stage: tag of every output (segments and h_out)
  // DeltaNet gate rows (P_NORM, K = 1024; tagged in_proj): fp32 rows in the lane-interleaved
  // order, wb (beta, rows 0..15) then wa (g, rows 16..31); row r on wave 0 of workgroup
  // gblk - r (gblk < 0: nblk - 1), from the prologue's activation.  Head h's g goes to pair
  // 16 h of gout, beta to pair 16 h + 1 (deltanet.hpp:164-165).
  const float* gw = nullptr;
  int grows = 0;
  int gblk = -1;
  const float* g_alog = nullptr;
  const float* g_dtb = nullptr;
  float* gout = nullptr;
  int nseg = 0;
  Seg seg[4];
};

// LM head (tied embedding): logits = (E h_norm) * s, running argmax per block.
struct HeadArgs {
  const float* h = nullptr;     // [1024] final hidden (pre-norm)
  const float* nw = nullptr;    // final norm gain
  int nw_lanes = 0;             // nw in the lane-interleaved order (load16c)
  float eps = 1e-6f;
  const int8_t* w = nullptr;    // [rows][1024]
  const float* sw = nullptr;
  int rows = 0;
  float* logits = nullptr;      // optional [rows]
  float* part_val = nullptr;    // [grid] block maxima
  int* part_idx = nullptr;
  const int* done = nullptr;
  int h_st = 0, part_st = 0;    // producer of h / this stage (tagged I/O)
};

// Decode-step control block, device resident.
struct StepCtl {
  int tok;        // token fed this step
  int pos;        // tokens already processed (RoPE position and KV slot)
  int argmax;     // result of the last step
  int step;       // index of the fed token in prompt order (generation driver)
  int n_prompt;
  int n_new;
  int n_out;
  int eos;
  int done;
  int err;        // 1: token id out of range; 2: context full
  int max_ctx;
  int pad;
};

struct AttnArgs {
  const float* qkv = nullptr;    // [5120]: q || gate interleaved per head [4096], k [512], v [512]
  const float* qn = nullptr;     // q_norm [256]
  const float* kn = nullptr;     // k_norm [256]
  const float* rope = nullptr;   // [rows][64]: cos[32] then sin[32] per row
  float* kc = nullptr;           // [max_ctx][512]
  float* vc = nullptr;
  const int* T = nullptr;        // slot of this token (past tokens = T)
  const int* rope_row = nullptr; // row of `rope` to use
  float* pm = nullptr;           // [8][nsplit] split maxima
  float* pl = nullptr;           // [8][nsplit] split sums
  float* pacc = nullptr;         // [8][nsplit][256]
  int nsplit_max = 0;
  int max_ctx = 0;               // rows of kc / vc; a slot T >= max_ctx is never touched
  float* og = nullptr;           // combine output [2048]
  float eps = 1e-6f;
  const int* done = nullptr;
  int qkv_st = 0;                // producer of qkv (tagged I/O)
  int part_st = 0;               // attention stage: pm / pl / pacc
  int og_st = 0;                 // combine stage: og
};

struct DnArgs {
  const float* convd = nullptr;  // [6144] post-conv q | k | v
  const float* gb = nullptr;     // g[16] then beta[16] (used when wa is null)
  // Gate projections computed by each unit for its head (deltanet.hpp:164-165):
  // beta = sigmoid(wb[h] . x), g = -exp(A_log[h]) * softplus(wa[h] . x + dt_bias[h]),
  // x = the layer input (gx, rmsnorm'd with gx_norm when that is set; the
  // embedded token when emb is set), int8-quantised and dequantised in W8A8 as
  // the in_proj prologue does.  Reads only inputs that are final before in_proj.
  const float* gx = nullptr;
  const float* gx_norm = nullptr;
  float eps = 1e-6f;
  int lanes = 0;                 // gx_norm, wb and wa rows in the lane-interleaved order (load16c)
  const float* wb = nullptr;     // fp32 [16][1024]
  const float* wa = nullptr;     // fp32 [16][1024]
  const float* A_log = nullptr;
  const float* dt_bias = nullptr;
  const int8_t* emb = nullptr;
  const float* emb_s = nullptr;
  const int* tok = nullptr;      // token id in device memory (null: passed by the caller)
  int mode = M_W8A16;
  float* S = nullptr;            // [16][128][128]
  float* o = nullptr;            // [16][128]
  int gates_in_convd = 0;        // tagged I/O: g and beta of head h are pairs 6144 + 16 h and
                                 // 6144 + 16 h + 1 of convd (computed by the in_proj stage)
  int normalize = 1;             // l2norm q,k and scale q (0: given already normalized)
  int heads = 16;                // heads to process (1 for the single-head op)
  const int* done = nullptr;
  int convd_st = 0, gx_st = 0;   // producers of convd / gx (tagged I/O)
  int o_st = 0;                  // this stage
  int unit_base = -1;            // persistent kernel: >= 0 keeps S in LDS for the launch
                                 // (the layer's global unit index base; see dn_tiles)
};

struct Floats64 { float v[64]; };

// One stage of a decode step: the arguments a per-stage kernel would get, and
// which body runs them.  The three K > 1024 GEMVs use one row per wave batch
// (1024 rows = 1024 batches), so every wave of a 256-workgroup grid streams.
enum StageKind : int {
  ST_GEMV_NORM_1x8 = 0,    // gemv_body<1, mode, P_NORM, 8>   DeltaNet in_proj (conv + SiLU, SiLU(z), gate rows)
  ST_GEMV_GATED_2x1 = 1,   // gemv_body<2, mode, P_GATED, 1>  DeltaNet out_proj
  ST_GEMV_LOAD_2x1 = 2,    // gemv_body<2, mode, P_LOAD, 1>   attention o_proj
  ST_GEMV_LOAD_4x1 = 3,    // gemv_body<4, mode, P_LOAD, 1>   MLP down
  ST_DELTANET = 4,
  ST_ATTN = 5,
  ST_COMBINE = 6,
  ST_HEAD = 7,
  ST_GEMV_QKV_1x8 = 8,     // gemv_body<1, mode, P_NORM, 8>   attention q||gate, k, v (E_STORE only)
  ST_GEMV_GATEUP_1x8 = 9,  // gemv_body<1, mode, P_NORM, 8>   MLP gate||up pairs (E_SWIGLU only)
};
// The epilogues (and segment kinds) a GEMV stage kind may hold, as a mask of
// (1 << Epi) bits plus kEmPair / kEmF32; 0 allows everything.  The persistent
// kernel compiles each stage kind for its own set, so loads and branches for
// the others do not exist there; the engine checks its program against them.
constexpr int kEmPair = 1 << 14;   // SEG_PAIR segments
constexpr int kEmF32 = 1 << 13;    // SEG_F32 segments
constexpr int kEmInProj = (1 << E_CONV) | (1 << E_SILU);   // ST_GEMV_NORM_1x8 (DeltaNet in_proj)
constexpr int kEmStore = 1 << E_STORE;                     // ST_GEMV_QKV_1x8
constexpr int kEmSwiglu = (1 << E_SWIGLU) | kEmPair;       // ST_GEMV_GATEUP_1x8
constexpr int kEmResid = 1 << E_RESID;                     // the 2x1 / 4x1 kinds
constexpr int stage_em(int kind) {
  return kind == ST_GEMV_NORM_1x8     ? kEmInProj
         : kind == ST_GEMV_QKV_1x8    ? kEmStore
         : kind == ST_GEMV_GATEUP_1x8 ? kEmSwiglu
         : (kind == ST_GEMV_GATED_2x1 || kind == ST_GEMV_LOAD_2x1 || kind == ST_GEMV_LOAD_4x1) ? kEmResid
                                      : 0;
}
struct Stage {
  int kind = ST_GEMV_NORM_1x8;
  union {   // the arguments of `kind` (all members are trivially copyable)
    GemvArgs g;
    DnArgs d;
    AttnArgs at;
    HeadArgs hd;
  };
  Stage() : g() {}
};

// Persistent decode: prog[0..nstage) is one token (embed .. LM head).  The
// kernel runs tokens until the run_hls loop of StepCtl stops it.  Workgroups
// hand vectors to one another through tagged buffers (see TagIO): stage i of
// the k-th token of the launch tags its outputs tag_base + k * kTagsPerToken + i.
constexpr int kTagsPerToken = 256;
struct PersistArgs {
  const Stage* prog = nullptr;
  int nstage = 0;
  int mode = M_W8A16;
  uint32_t tag_base = 1;
  StepCtl* ctl = nullptr;       // in: tok, pos, step, n_prompt, n_new, n_out, eos, max_ctx; out: all
  const int* prompt = nullptr;  // [n_prompt]
  int* out_ids = nullptr;       // [n_new]
  float* logits = nullptr;      // optional: logits of every step (the last one remains)
  int* abort_flag = nullptr;    // set when a hand-over wait exceeds its poll limit
  unsigned poll_limit = 1u << 20;   // failed polls before a wait gives up (about a second)
  uint64_t* trace = nullptr;    // optional [trace_tokens][nstage][grid][kTraceSlots]: stage marks and end
  int trace_tokens = 0;
  int dn_lds = 0;               // DeltaNet stages keep S in LDS (their unit_base >= 0)
  int long_ctx = 0;             // the cache holds more than kAttnShortMax positions: the kernel
                                // instantiation with the long-context attention (else without it)
};
constexpr int kPersistThreads = 256;
constexpr int kTraceSlots = 8;  // marks 0..6 of a stage body, then its completion time

hipError_t launch_persist(const PersistArgs& a, int grid, hipStream_t s);
int persist_max_grid(int* grid);   // workgroups the cooperative launch can hold (a multiple of 16)

// ---- launch wrappers (return hipError_t) ----
hipError_t launch_gemv(const GemvArgs& a, int waves_per_block, hipStream_t s);
// t0 / t1 (optional): events stamped at the kernel's own start and end
hipError_t launch_head(const HeadArgs& a, int grid, hipStream_t s, hipEvent_t t0 = nullptr, hipEvent_t t1 = nullptr);
hipError_t launch_argmax(const float* pv, const int* pi, int n, StepCtl* ctl, int* out_idx,
                         hipStream_t s);
hipError_t launch_deltanet(const DnArgs& a, hipStream_t s);
hipError_t launch_attn(const AttnArgs& a, hipStream_t s);
hipError_t launch_attn_combine(const AttnArgs& a, hipStream_t s);
hipError_t launch_advance(StepCtl* ctl, const int* prompt, int* out_ids, hipStream_t s);

// small op kernels
hipError_t launch_embed(float* h, const int8_t* w, const float* sc, int tok, int in, hipStream_t s);
hipError_t launch_rmsnorm(float* y, const float* x, const float* w, const float* z, int n, float eps,
                          int gated, hipStream_t s,
                          int groups = 1);
hipError_t launch_l2norm(float* v, int n, hipStream_t s);
hipError_t launch_dn_step_pre(float* convd, float* gb, const float* qkv, float* state, const float* cw,
                              const float* b, const float* a, const float* A_log, const float* dt_bias,
                              hipStream_t s);
hipError_t launch_conv1d(float* out, const float* in, float* state, const float* w, int C,
                         hipStream_t s);
hipError_t launch_apply_rope(float* x, const float* cs, const float* sn, hipStream_t s);
hipError_t launch_quant(int8_t* q, float* sx, const float* x, int n, hipStream_t s);
hipError_t launch_fixed_dequant(int32_t* yq, const int32_t* acc, const int32_t* mult, int n, int shift, int outw,
                                hipStream_t s);
hipError_t launch_quant_rows(int8_t* q, float* scale, const float* w, int rows, int cols, hipStream_t s);
hipError_t launch_quant_rows_bf16(int8_t* q, float* scale, const uint16_t* w, int rows, int cols, hipStream_t s);
hipError_t launch_set_ints(int* dst, int a, int b, hipStream_t s);
hipError_t launch_set_int(int* dst, int v, hipStream_t s);
hipError_t launch_dn_gather(float* convd, float* gb, const float* q, const float* k, const float* v, const float* g,
                            const float* beta, float gs, float bs, int nq, int nv, int nh, hipStream_t s);
hipError_t launch_set_floats(float* dst, const Floats64& v, int n, hipStream_t s);
hipError_t launch_bump_pos(StepCtl* ctl, hipStream_t s);
hipError_t launch_init_gen(StepCtl* ctl, int tok0, int n_prompt, int n_new, int eos, hipStream_t s);

}  // namespace qh
