// The decode engine: replaces the HLS decode top (hls/src/qwen_synth.hpp:39-92
// qwen_top, hls/src/decoder.hpp:62-120 decode_token) and the DecodeState
// (hls/src/state.hpp:18-35) with device-resident buffers.  One decode step is
// recorded once as a hipGraph and replayed; the token, position and stop flag
// live in a device StepCtl, so greedy generation runs without host round trips.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include "qh_common.hpp"
#include "qh_kernels.hpp"
#include "qh_layout.hpp"

using namespace qh;

struct qh_engine {
  hipStream_t stream = nullptr;
  const Layout* L = nullptr;
  uint8_t* blob = nullptr;   // device copy of the packed weights
  int max_ctx = 0;
  int mode = M_W8A16;
  // DecodeState (state.hpp:18-35)
  float* rec = nullptr;    // [18][16][128][128]
  float* conv = nullptr;   // [18][6144][4]
  float* kc = nullptr;     // [6][max_ctx][512]
  float* vc = nullptr;
  // activations
  float* h = nullptr;      // residual stream [1024]
  float* convd = nullptr;  // [6144]
  float* zb = nullptr;     // [2048]
  float* gb = nullptr;     // g[16] beta[16]
  float* o = nullptr;      // [2048]
  float* act = nullptr;    // [3584]
  float* og = nullptr;     // [2048]
  float* qkv = nullptr;    // [5120] q||gate | k | v
  float* pm = nullptr;
  float* pl = nullptr;
  float* pacc = nullptr;
  int nsplit_max = 0;
  float* rope = nullptr;   // [max_ctx][64]
  float* logits = nullptr; // [VOCAB]
  float* part_val = nullptr;
  int* part_idx = nullptr;
  int head_grid = 0;
  StepCtl* ctl = nullptr;
  int* prompt_dev = nullptr;
  int* out_dev = nullptr;
  int io_cap = 0;
  int host_pos = 0;
  int last_argmax = -1;
  // graphs[mode][logits][advance]
  hipGraphExec_t graphs[2][2][2] = {};
  // persistent path: the per-token stage program per mode over the tagged
  // hand-over arena (every stage output its own region of 8-byte pairs)
  int exec = QH_EXEC_GRAPH;
  int persist_grid = 0;          // 0: cooperative launch not available (graph path only)
  Stage* prog[2] = {};
  int prog_n = 0;
  uint64_t* arena = nullptr;     // tagged vectors of the persistent program
  size_t arena_pairs = 0;
  uint32_t tag_next = 1;         // first unused tag (the arena holds only smaller tags)
  uint32_t tag_start = 1;        // tag_next once the arena is (re)allocated (test hook QH_TAG_START)
  int* abort_dev = nullptr;      // set by a hand-over wait that gave up
  // Lane-interleaved copies of the fp32 vectors a wave reads 16 elements per
  // lane (norm gains, the DeltaNet gate rows): element e of lane l's chunk of
  // each 1024-element row at (e / 4) * 256 + 4 l + e % 4, so one 16-byte load
  // instruction of a wave covers 1 KiB of consecutive memory.
  float* lanes = nullptr;
  int64_t lane_off[kLayers + 1][R_COUNT];   // float offset in lanes, or -1
  hipEvent_t launch_ev[2] = {};  // around the last persistent launch (engine stream)
  float last_launch_ms = 0.0f;
  unsigned poll_limit = 1u << 20;  // failed polls before a hand-over wait gives up (QH_POLL_LIMIT)
  bool broken = false;             // a launch returned QH_EDEVICE: decode refused until reset
  int fallbacks = 0;               // cooperative launches refused (each switched the engine to the graph path)
  bool dn_lds = false;             // the persistent kernel keeps the DeltaNet state in LDS (enough workgroups)
};

namespace {

const float* f32p(const qh_engine* e, int layer, Role r) {
  const Entry* en = e->L->get(layer, r);
  return reinterpret_cast<const float*>(e->blob + en->off);
}
const float* lanep(const qh_engine* e, int layer, Role r) {
  const int64_t o = e->lane_off[layer][r];
  return o < 0 ? nullptr : e->lanes + o;
}
const int8_t* i8p(const qh_engine* e, int layer, Role r) {
  return reinterpret_cast<const int8_t*>(e->blob + e->L->get(layer, r)->off);
}
const float* scp(const qh_engine* e, int layer, Role r) {
  return reinterpret_cast<const float*>(e->blob + e->L->get(layer, r)->soff);
}

Seg mkseg(int kind, int epi, int rows, int batch0, float* out, int rpb = kRowsPerBatch) {
  Seg g;
  g.kind = kind;
  g.epi = epi;
  g.rows = rows;
  g.batch0 = batch0;
  g.nbatch = (rows + rpb - 1) / rpb;
  g.out = out;
  g.res = out;
  return g;
}

template <class T>
int dalloc(T** p, size_t n) {
  return hip_status(hipMalloc(reinterpret_cast<void**>(p), n * sizeof(T)));
}

Stage gemv_stage(int kind, const GemvArgs& a) {
  Stage st;
  st.kind = kind;
  st.g = a;
  return st;
}

// Output vectors of the stages.  Plain (graph engine): the engine's fixed
// activation buffers, the residual stream updated in place.  Tagged
// (persistent kernel): a fresh region of the arena for every stage output, so
// no vector is written twice within a token.  With arena == nullptr the tagged
// form only counts pairs.
struct Bufs {
  bool tagged = false;
  uint64_t* arena = nullptr;
  size_t used = 0;   // pairs
  float* take(size_t n, float* plain) {
    if (!tagged) return plain;
    const size_t off = used;
    used += (n + 31) & ~(size_t)31;   // 256-byte aligned regions
    return arena != nullptr ? reinterpret_cast<float*>(arena + off) : nullptr;
  }
  // element n of a vector from take()
  float* at(float* v, size_t n) const {
    if (v == nullptr) return nullptr;
    return tagged ? reinterpret_cast<float*>(reinterpret_cast<uint64_t*>(v) + n) : v + n;
  }
};

// A hand-over vector and the stage that produces it.
struct Vec {
  float* p = nullptr;
  int st = 0;
};

// DeltaNet layer li's in_proj rows: q, k, v (which the DeltaNet units wait
// for), then z (only out_proj reads it), and the gate rows -- the longest work
// of a workgroup -- on wave 0 of the last 2 kLH workgroups.  When the persistent
// kernel keeps this layer's DeltaNet units (unit u on workgroup
// (kLH kDnVQuarters li + u) mod grid) on the z workgroups, z goes first instead,
// with the gate rows on its last workgroups, so that the units' workgroups
// compute only q, k, v rows before the DeltaNet stage.  (One batch per wave:
// batch b on workgroup b / 4.)
bool dn_z_first(const qh_engine* e, int li) {
  const int grid = e->persist_grid, units = kLH * kDnVQuarters;
  const int qb = kConvDim / kRowsPerBatch, zb = kZDim / kRowsPerBatch;
  if (grid * 4 != qb + zb || zb / 4 < 2 * kLH) return false;
  const int first = (units * li) % grid;
  return first + units > qb / 4;
}

// The stages of layers [l0, l1) of one decode step on the residual stream h
// (updated to the last stage's output).  The tagged program leaves the device
// StepCtl pointers out: the persistent kernel passes the token and position
// itself.
void build_layers(const qh_engine* e, int l0, int l1, bool embed, Bufs& B, std::vector<Stage>& out, Vec& h) {
  const bool tag = B.tagged;
  const int* done = tag ? nullptr : &e->ctl->done;
  int li = 0, fi = 0;
  for (int l = 0; l < l0; ++l) (is_linear(l) ? li : fi)++;
  for (int l = l0; l < l1; ++l) {
    if (is_linear(l)) {
      // in_ln rmsnorm (+ act-quant) -> qkv(conv+SiLU) | z   (deltanet.hpp:149-165)
      const int sA = (int)out.size();
      GemvArgs a;
      a.K = kHidden;
      a.mode = e->mode;
      a.prologue = P_NORM;
      a.x = h.p;
      a.x_st = h.st;
      a.out_st = sA;
      a.nw = lanep(e, l, R_IN_LN);
      a.nw_lanes = 1;
      a.eps = kEps;
      a.done = done;
      float* convd = B.take(tag ? kConvDim + 16 * kLH : kConvDim, e->convd);   // tagged: + the gates
      float* zb = B.take(kZDim, e->zb);
      if (embed && l == l0) {   // embed_row (qwen_synth.hpp:42-43), written to the residual
        a.emb = i8p(e, kLayers, R_EMBED);
        a.emb_s = scp(e, kLayers, R_EMBED);
        a.tok = tag ? nullptr : &e->ctl->tok;
        a.h_out = B.take(kHidden, e->h);
        h = Vec{a.h_out, sA};
      }
      a.nseg = 2;   // the fp32 gate projections b, a run in the DeltaNet stage
      const bool zfirst = tag && dn_z_first(e, li);
      Seg& sq = a.seg[zfirst ? 1 : 0];
      Seg& sz = a.seg[zfirst ? 0 : 1];
      const int nzb = (kZDim + kRowsPerBatch - 1) / kRowsPerBatch, nqb = (kConvDim + kRowsPerBatch - 1) / kRowsPerBatch;
      sq = mkseg(SEG_I8, E_CONV, kConvDim, zfirst ? nzb : 0, convd);
      sq.w = i8p(e, l, R_QKV);
      sq.sw = scp(e, l, R_QKV);
      sq.c0 = f32p(e, l, R_CONV);
      sq.c2 = e->conv + (size_t)li * kConvDim * kConvK;
      sz = mkseg(SEG_I8, E_SILU, kZDim, zfirst ? 0 : nqb, zb);   // silu(z) for the gated norm
      sz.w = i8p(e, l, R_Z);
      sz.sw = scp(e, l, R_Z);
      if (tag) {   // the gates b, a of the 16 heads, from this prologue's activation
        a.gw = lanep(e, l, R_B);   // wb rows, then the wa rows (consecutive in lanes)
        a.grows = 2 * kLH;
        a.gblk = zfirst ? nzb / 4 - 1 : -1;
        a.g_alog = f32p(e, l, R_ALOG);
        a.g_dtb = f32p(e, l, R_DTB);
        a.gout = B.at(convd, kConvDim);
      }
      out.push_back(gemv_stage(ST_GEMV_NORM_1x8, a));
      const int sB = (int)out.size();
      DnArgs d;   // gates b, a (deltanet.hpp:164-165), l2norm, delta rule (deltanet.hpp:166-173)
      d.convd = convd;
      d.convd_st = sA;
      d.gb = e->gb;
      d.gx = h.p;
      d.gx_st = h.st;
      d.gx_norm = lanep(e, l, R_IN_LN);
      d.eps = kEps;
      d.wb = lanep(e, l, R_B);
      d.wa = lanep(e, l, R_A);
      d.lanes = 1;
      d.A_log = f32p(e, l, R_ALOG);
      d.dt_bias = f32p(e, l, R_DTB);
      d.mode = e->mode;
      if (embed && l == l0) {   // layer 0 reads the embedded token, not the residual
        d.emb = i8p(e, kLayers, R_EMBED);
        d.emb_s = scp(e, kLayers, R_EMBED);
        d.tok = tag ? nullptr : &e->ctl->tok;
      }
      d.S = e->rec + (size_t)li * kLH * kLK * kLV;
      d.o = B.take(kLH * kLV, e->o);
      d.o_st = sB;
      d.gates_in_convd = tag ? 1 : 0;
      // persistent kernel: this layer's 64 units keep their state in LDS, on workgroups
      // (64 li + u) % grid, slot (64 li + u) / grid (dn_tiles)
      d.unit_base = tag && e->dn_lds ? li * kLH * kDnVQuarters : -1;
      d.done = done;
      Stage sd;
      sd.kind = ST_DELTANET;
      sd.d = d;
      out.push_back(sd);
      const int sC = (int)out.size();
      GemvArgs c;   // gated rmsnorm (+ quant) -> out_proj, residual add (deltanet.hpp:177-181)
      c.K = kLH * kLV;
      c.mode = e->mode;
      c.prologue = P_GATED;
      c.x = d.o;
      c.x_st = sB;
      c.nw = f32p(e, l, R_LNORM);
      c.z = zb;
      c.z_st = sA;
      c.out_st = sC;
      c.eps = kEps;
      c.done = done;
      c.nseg = 1;
      c.rows_per_batch = 1;
      c.seg[0] = mkseg(SEG_I8, E_RESID, kHidden, 0, B.take(kHidden, e->h), 1);
      c.seg[0].res = h.p;
      c.seg[0].res_st = h.st;
      c.seg[0].w = i8p(e, l, R_OUTP);
      c.seg[0].sw = scp(e, l, R_OUTP);
      out.push_back(gemv_stage(ST_GEMV_GATED_2x1, c));
      h = Vec{c.seg[0].out, sC};
      ++li;
    } else {
      const int sA = (int)out.size();
      GemvArgs a;   // in_ln rmsnorm (+ quant) -> q||gate, k, v (attention.hpp:31-33)
      a.K = kHidden;
      a.mode = e->mode;
      a.prologue = P_NORM;
      a.x = h.p;
      a.x_st = h.st;
      a.out_st = sA;
      a.nw = lanep(e, l, R_IN_LN);
      a.nw_lanes = 1;
      a.eps = kEps;
      a.done = done;
      a.nseg = 3;
      float* qkv = B.take(kQProj + 2 * kKVProj, e->qkv);   // q||gate | k | v
      a.seg[0] = mkseg(SEG_I8, E_STORE, kQProj, 0, qkv);
      a.seg[0].w = i8p(e, l, R_QP);
      a.seg[0].sw = scp(e, l, R_QP);
      a.seg[1] = mkseg(SEG_I8, E_STORE, kKVProj, a.seg[0].nbatch, B.at(qkv, kQProj));
      a.seg[1].w = i8p(e, l, R_KP);
      a.seg[1].sw = scp(e, l, R_KP);
      a.seg[2] = mkseg(SEG_I8, E_STORE, kKVProj, a.seg[1].batch0 + a.seg[1].nbatch, B.at(qkv, kQProj + kKVProj));
      a.seg[2].w = i8p(e, l, R_VP);
      a.seg[2].sw = scp(e, l, R_VP);
      out.push_back(gemv_stage(ST_GEMV_QKV_1x8, a));
      const int sB = (int)out.size();
      AttnArgs at;
      at.qkv = qkv;
      at.qkv_st = sA;
      at.qn = f32p(e, l, R_QN);
      at.kn = f32p(e, l, R_KN);
      at.rope = e->rope;
      at.kc = e->kc + (size_t)fi * e->max_ctx * kKVProj;
      at.vc = e->vc + (size_t)fi * e->max_ctx * kKVProj;
      at.T = tag ? nullptr : &e->ctl->pos;
      at.rope_row = tag ? nullptr : &e->ctl->pos;
      at.pm = B.take((size_t)8 * e->nsplit_max, e->pm);
      at.pl = B.take((size_t)8 * e->nsplit_max, e->pl);
      at.pacc = B.take((size_t)8 * e->nsplit_max * 256, e->pacc);
      at.part_st = sB;
      at.nsplit_max = e->nsplit_max;
      at.max_ctx = e->max_ctx;
      at.og = B.take(kNH * kHD, e->og);
      at.og_st = sB + 1;
      at.eps = kEps;
      at.done = done;
      Stage sa;
      sa.kind = ST_ATTN;
      sa.at = at;
      out.push_back(sa);
      sa.kind = ST_COMBINE;
      out.push_back(sa);
      const int sC = (int)out.size();
      GemvArgs c;   // (+ quant) o_proj, residual add (attention.hpp:94)
      c.K = kNH * kHD;
      c.mode = e->mode;
      c.prologue = P_LOAD;
      c.x = at.og;
      c.x_st = at.og_st;
      c.out_st = sC;
      c.done = done;
      c.nseg = 1;
      c.rows_per_batch = 1;
      c.seg[0] = mkseg(SEG_I8, E_RESID, kHidden, 0, B.take(kHidden, e->h), 1);
      c.seg[0].res = h.p;
      c.seg[0].res_st = h.st;
      c.seg[0].w = i8p(e, l, R_OP);
      c.seg[0].sw = scp(e, l, R_OP);
      out.push_back(gemv_stage(ST_GEMV_LOAD_2x1, c));
      h = Vec{c.seg[0].out, sC};
      ++fi;
    }
    // post_ln rmsnorm (+ quant) -> gate||up pairs with SwiGLU -> down, residual (mlp.hpp:11-19)
    const int sD = (int)out.size();
    GemvArgs m;
    m.K = kHidden;
    m.mode = e->mode;
    m.prologue = P_NORM;
    m.x = h.p;
    m.x_st = h.st;
    m.out_st = sD;
    m.nw = lanep(e, l, R_POST_LN);
    m.nw_lanes = 1;
    m.eps = kEps;
    m.done = done;
    m.nseg = 1;
    m.seg[0] = mkseg(SEG_PAIR, E_SWIGLU, 2 * kInter, 0, B.take(kInter, e->act));
    m.seg[0].w = i8p(e, l, R_GATE);
    m.seg[0].sw = scp(e, l, R_GATE);
    m.seg[0].w2 = i8p(e, l, R_UP);
    m.seg[0].sw2 = scp(e, l, R_UP);
    out.push_back(gemv_stage(ST_GEMV_GATEUP_1x8, m));
    const int sE = (int)out.size();
    GemvArgs dn;
    dn.K = kInter;
    dn.mode = e->mode;
    dn.prologue = P_LOAD;
    dn.x = m.seg[0].out;
    dn.x_st = sD;
    dn.out_st = sE;
    dn.done = done;
    dn.nseg = 1;
    dn.rows_per_batch = 1;
    dn.seg[0] = mkseg(SEG_I8, E_RESID, kHidden, 0, B.take(kHidden, e->h), 1);
    dn.seg[0].res = h.p;
    dn.seg[0].res_st = h.st;
    dn.seg[0].w = i8p(e, l, R_DOWN);
    dn.seg[0].sw = scp(e, l, R_DOWN);
    out.push_back(gemv_stage(ST_GEMV_LOAD_4x1, dn));
    h = Vec{dn.seg[0].out, sE};
  }
}

// Final norm + tied LM head (qwen_synth.hpp:74-88).
Stage head_stage(const qh_engine* e, Bufs& B, const Vec& h, bool with_logits, int st_self, int nparts) {
  Stage st;
  st.kind = ST_HEAD;
  HeadArgs& hd = st.hd;
  hd.h = h.p;
  hd.h_st = h.st;
  hd.nw = lanep(e, kLayers, R_FINAL);
  hd.nw_lanes = 1;
  hd.eps = kEps;
  hd.w = i8p(e, kLayers, R_EMBED);
  hd.sw = scp(e, kLayers, R_EMBED);
  hd.rows = kVocab;
  hd.logits = with_logits ? e->logits : nullptr;
  hd.part_val = B.take(nparts, e->part_val);
  hd.part_idx = reinterpret_cast<int*>(B.take(nparts, reinterpret_cast<float*>(e->part_idx)));
  hd.part_st = st_self;
  hd.done = B.tagged ? nullptr : &e->ctl->done;
  return st;
}

// Stream launches of a stage list (the per-stage kernels); the head is followed
// by the cross-block argmax, which also advances pos.
int launch_stages(qh_engine* e, const std::vector<Stage>& v, hipStream_t s, hipEvent_t head_t0 = nullptr,
                  hipEvent_t head_t1 = nullptr) {
  for (const Stage& st : v) {
    switch (st.kind) {
      case ST_GEMV_NORM_1x8:
      case ST_GEMV_QKV_1x8:
      case ST_GEMV_GATEUP_1x8:
      case ST_GEMV_GATED_2x1:
      case ST_GEMV_LOAD_2x1:
      case ST_GEMV_LOAD_4x1: QH_HIP(launch_gemv(st.g, 4, s)); break;
      case ST_DELTANET: QH_HIP(launch_deltanet(st.d, s)); break;
      case ST_ATTN: QH_HIP(launch_attn(st.at, s)); break;
      case ST_COMBINE: QH_HIP(launch_attn_combine(st.at, s)); break;
      default:
        QH_HIP(launch_head(st.hd, e->head_grid, s, head_t0, head_t1));
        QH_HIP(launch_argmax(e->part_val, e->part_idx, e->head_grid, e->ctl, nullptr, s));
        break;
    }
  }
  return QH_OK;
}

int enqueue_layers(qh_engine* e, int l0, int l1, bool embed, hipStream_t s) {
  std::vector<Stage> v;
  Bufs B;
  Vec h{e->h, 0};
  build_layers(e, l0, l1, embed, B, v, h);
  return launch_stages(e, v, s);
}

// The persistent kernel's per-token program for the current mode, over the
// tagged arena (allocated and zeroed on first use; both modes share it).
int ensure_prog(qh_engine* e) {
  if (e->prog[e->mode]) return QH_OK;
  std::vector<Stage> v;
  Vec h;
  if (e->arena == nullptr) {
    Bufs cnt;
    cnt.tagged = true;
    build_layers(e, 0, kLayers, true, cnt, v, h);
    (void)head_stage(e, cnt, h, false, (int)v.size(), e->persist_grid);
    QH_TRY(dalloc(&e->arena, cnt.used));
    QH_HIP(hipMemset(e->arena, 0, sizeof(uint64_t) * cnt.used));
    e->arena_pairs = cnt.used;
    e->tag_next = e->tag_start;
    v.clear();
    h = Vec{};
  }
  Bufs B;
  B.tagged = true;
  B.arena = e->arena;
  build_layers(e, 0, kLayers, true, B, v, h);
  v.push_back(head_stage(e, B, h, false, (int)v.size(), e->persist_grid));
  if ((int)v.size() >= kTagsPerToken || B.used != e->arena_pairs) return QH_ESTATE;
  // the persistent kernel compiles each GEMV stage kind for one vector length and one set of
  // epilogues and segment kinds
  for (const Stage& st : v) {
    const int want = (st.kind == ST_GEMV_NORM_1x8 || st.kind == ST_GEMV_QKV_1x8 || st.kind == ST_GEMV_GATEUP_1x8)
                         ? kHidden
                     : st.kind == ST_GEMV_GATED_2x1 ? kLH * kLV
                     : st.kind == ST_GEMV_LOAD_2x1  ? kNH * kHD
                     : st.kind == ST_GEMV_LOAD_4x1  ? kInter
                                                    : -1;
    if (want < 0) continue;
    if (st.g.K != want) return QH_ESTATE;
    const int em = stage_em(st.kind);
    for (int i = 0; i < st.g.nseg; ++i) {
      const Seg& g = st.g.seg[i];
      if (!(em & (1 << g.epi))) return QH_ESTATE;
      if (g.kind == SEG_PAIR && !(em & kEmPair)) return QH_ESTATE;
      if (g.kind == SEG_F32 && !(em & kEmF32)) return QH_ESTATE;
    }
  }
  QH_TRY(dalloc(&e->prog[e->mode], v.size()));
  QH_HIP(hipMemcpy(e->prog[e->mode], v.data(), sizeof(Stage) * v.size(), hipMemcpyHostToDevice));
  e->prog_n = (int)v.size();
  return QH_OK;
}

// run_persist's answer when the cooperative launch itself is refused (the
// device's cooperative resources can be held by another process): the engine
// switches to the graph path, which runs the same kernels bit for bit.
constexpr int kUseGraph = 1000;

// One persistent launch: the prompt (already in prompt_dev) through the
// run_hls loop, n_new greedy tokens at most, token feedback on the device.
int run_persist(qh_engine* e, int tok0, int n_prompt, int n_new, int eos, bool with_logits, StepCtl* out) {
  QH_TRY(ensure_prog(e));
  hipStream_t s = e->stream;
  // tags of this launch: tag_base + k * kTagsPerToken + stage, k < n_prompt + n_new
  const uint64_t need = ((uint64_t)n_prompt + (uint64_t)n_new + 1) * kTagsPerToken;
  if ((uint64_t)e->tag_next + need > 0xFFFFFFFFull) {   // tags would wrap: clear the arena
    QH_HIP(hipMemsetAsync(e->arena, 0, sizeof(uint64_t) * e->arena_pairs, s));
    e->tag_next = 1;
  }
  StepCtl c;
  std::memset(&c, 0, sizeof c);
  c.tok = tok0;
  c.pos = e->host_pos;
  c.argmax = e->last_argmax;
  c.n_prompt = n_prompt;
  c.n_new = n_new;
  c.eos = eos;
  c.max_ctx = e->max_ctx;
  QH_HIP(hipMemcpyAsync(e->ctl, &c, sizeof c, hipMemcpyHostToDevice, s));
  QH_HIP(hipMemsetAsync(e->abort_dev, 0, sizeof(int), s));
  PersistArgs a;
  // QH_TRACE_FILE=path: completion time of every stage on every workgroup for
  // the first two tokens of this launch, written as text (s_memrealtime ticks).
  const char* trace_path = std::getenv("QH_TRACE_FILE");
  uint64_t* trace = nullptr;
  const int trace_tokens = 2;
  const size_t trace_n = (size_t)trace_tokens * e->prog_n * e->persist_grid * kTraceSlots;
  if (trace_path != nullptr && trace_path[0] != '\0') {
    QH_TRY(dalloc(&trace, trace_n));
    QH_HIP(hipMemsetAsync(trace, 0, sizeof(uint64_t) * trace_n, s));
    a.trace = trace;
    a.trace_tokens = trace_tokens;
  }
  a.prog = e->prog[e->mode];
  a.nstage = e->prog_n;
  a.mode = e->mode;
  a.tag_base = e->tag_next;
  a.ctl = e->ctl;
  a.prompt = e->prompt_dev;
  a.out_ids = e->out_dev;
  a.logits = with_logits ? e->logits : nullptr;
  a.abort_flag = e->abort_dev;
  a.poll_limit = e->poll_limit;
  a.dn_lds = e->dn_lds ? 1 : 0;
  a.long_ctx = e->max_ctx > kAttnShortMax ? 1 : 0;
  QH_HIP(hipEventRecord(e->launch_ev[0], s));
  if (const hipError_t le = launch_persist(a, e->persist_grid, s); le != hipSuccess) {
    (void)hipGetLastError();
    if (trace != nullptr) (void)hipFree(trace);
    e->persist_grid = 0;
    e->exec = QH_EXEC_GRAPH;
    e->fallbacks += 1;
    if (verbose())
      std::fprintf(stderr, "[qh] cooperative launch of the persistent kernel refused (%s): engine switched to the graph executor\n",
                   hipGetErrorString(le));
    return kUseGraph;
  }
  QH_HIP(hipEventRecord(e->launch_ev[1], s));
  e->tag_next += (uint32_t)need;
  int aborted = 0;
  QH_HIP(hipMemcpyAsync(out, e->ctl, sizeof *out, hipMemcpyDeviceToHost, s));
  QH_HIP(hipMemcpyAsync(&aborted, e->abort_dev, sizeof(int), hipMemcpyDeviceToHost, s));
  QH_HIP(hipStreamSynchronize(s));
  if (trace != nullptr) {
    std::vector<uint64_t> hbuf(trace_n);
    const hipError_t ce = hipMemcpy(hbuf.data(), trace, trace_n * sizeof(uint64_t), hipMemcpyDeviceToHost);
    (void)hipFree(trace);
    QH_HIP(ce);
    if (FILE* f = std::fopen(trace_path, "w")) {
      std::fprintf(f, "# token stage block m0..m%d done (s_memrealtime ticks; 0 = not reached); %d stages per token, kinds:",
                   kTraceSlots - 2, e->prog_n);
      std::vector<Stage> kinds(e->prog_n);
      if (hipMemcpy(kinds.data(), e->prog[e->mode], sizeof(Stage) * e->prog_n, hipMemcpyDeviceToHost) == hipSuccess)
        for (const Stage& k : kinds) std::fprintf(f, " %d", k.kind);
      std::fprintf(f, "\n");
      for (int k = 0; k < trace_tokens; ++k)
        for (int i = 0; i < e->prog_n; ++i)
          for (int b = 0; b < e->persist_grid; ++b) {
            const uint64_t* q = &hbuf[(((size_t)k * e->prog_n + i) * e->persist_grid + b) * kTraceSlots];
            std::fprintf(f, "%d %d %d", k, i, b);
            for (int m = 0; m < kTraceSlots; ++m) std::fprintf(f, " %llu", (unsigned long long)q[m]);
            std::fprintf(f, "\n");
          }
      std::fclose(f);
    }
  }
  QH_HIP(hipEventElapsedTime(&e->last_launch_ms, e->launch_ev[0], e->launch_ev[1]));
  if (out->err == 3 || aborted != 0) {   // state and position are undefined until a reset
    e->broken = true;
    return QH_EDEVICE;
  }
  e->host_pos = out->pos;
  e->last_argmax = out->argmax;
  return QH_OK;
}

// One full decode step (qwen_top): embed, 24 layers, final norm, tied head,
// argmax (+ pos), optionally the generation bookkeeping.
int enqueue_step(qh_engine* e, bool with_logits, bool advance, hipStream_t s,
                 hipEvent_t head_t0 = nullptr, hipEvent_t head_t1 = nullptr) {
  std::vector<Stage> v;
  Bufs B;
  Vec h{e->h, 0};
  build_layers(e, 0, kLayers, true, B, v, h);
  v.push_back(head_stage(e, B, h, with_logits, (int)v.size(), e->head_grid));
  QH_TRY(launch_stages(e, v, s, head_t0, head_t1));
  if (advance) QH_HIP(launch_advance(e->ctl, e->prompt_dev, e->out_dev, s));
  return QH_OK;
}

int get_graph(qh_engine* e, bool with_logits, bool advance, hipGraphExec_t* out) {
  hipGraphExec_t& ge = e->graphs[e->mode][with_logits][advance];
  if (ge == nullptr) {
    hipGraph_t g = nullptr;
    QH_HIP(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
    const int st = enqueue_step(e, with_logits, advance, e->stream);
    const hipError_t ec = hipStreamEndCapture(e->stream, &g);
    if (st != QH_OK) {
      if (g) (void)hipGraphDestroy(g);
      return st;
    }
    QH_HIP(ec);
    const hipError_t ei = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    QH_HIP(ei);
  }
  *out = ge;
  return QH_OK;
}

void release(qh_engine* e) {
  if (!e) return;
  if (e->stream) (void)hipStreamSynchronize(e->stream);
  for (auto& a : e->graphs)
    for (auto& b : a)
      for (auto& g : b)
        if (g) (void)hipGraphExecDestroy(g);
  void* bufs[] = {e->blob, e->rec, e->conv, e->kc, e->vc, e->h, e->convd, e->zb, e->gb, e->o, e->act,
                  e->og, e->qkv, e->pm, e->pl, e->pacc, e->rope, e->logits, e->part_val,
                  e->part_idx, e->ctl, e->prompt_dev, e->out_dev, e->prog[0], e->prog[1], e->arena,
                  e->abort_dev, e->lanes};
  for (void* p : bufs)
    if (p) (void)hipFree(p);
  for (hipEvent_t ev : e->launch_ev)
    if (ev) (void)hipEventDestroy(ev);
  if (e->stream) (void)hipStreamDestroy(e->stream);
  delete e;
}

int ensure_io(qh_engine* e, int n) {
  if (n <= e->io_cap) return QH_OK;
  if (e->prompt_dev) (void)hipFree(e->prompt_dev);
  if (e->out_dev) (void)hipFree(e->out_dev);
  e->prompt_dev = e->out_dev = nullptr;
  // the generation graphs bake these pointers in
  for (auto& a : e->graphs)
    for (auto& b : a)
      if (b[1]) {
        (void)hipGraphExecDestroy(b[1]);
        b[1] = nullptr;
      }
  int cap = 1024;
  while (cap < n) cap *= 2;
  QH_TRY(dalloc(&e->prompt_dev, (size_t)cap));
  QH_TRY(dalloc(&e->out_dev, (size_t)cap));
  e->io_cap = cap;
  return QH_OK;
}

// Rows of 1024 fp32 from the blob into the lane-interleaved order (see qh_engine::lanes).
int build_lanes(qh_engine* e, const uint8_t* blob) {
  const Role roles[] = {R_IN_LN, R_POST_LN, R_B, R_A, R_FINAL};
  std::vector<float> host;
  for (int l = 0; l <= kLayers; ++l)
    for (int r = 0; r < R_COUNT; ++r) e->lane_off[l][r] = -1;
  for (int l = 0; l <= kLayers; ++l)
    for (Role r : roles) {
      const Entry* en = e->L->get(l, r);
      if (en == nullptr || en->dtype != 0 || en->numel() % 1024 != 0) continue;
      const float* src = reinterpret_cast<const float*>(blob + en->off);
      e->lane_off[l][r] = (int64_t)host.size();
      const size_t rows = (size_t)(en->numel() / 1024);
      for (size_t row = 0; row < rows; ++row) {
        const size_t base = host.size();
        host.resize(base + 1024);
        for (int ln = 0; ln < 64; ++ln)
          for (int el = 0; el < 16; ++el) host[base + (el / 4) * 256 + 4 * ln + el % 4] = src[row * 1024 + 16 * ln + el];
      }
    }
  QH_TRY(dalloc(&e->lanes, host.size()));
  QH_HIP(hipMemcpy(e->lanes, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice));
  return QH_OK;
}

// The KV cache of one attention layer ([max_ctx][512] fp32, 2 KiB per token) is
// addressed with 32-bit byte offsets through one buffer descriptor.
static_assert((long long)QH_MAX_CTX * kKVProj * 4 <= 0x7ffffff0LL, "cache slice beyond one descriptor");

int create(const void* blob, size_t blob_len, const char* idx_text, int max_ctx, qh_engine** out) {
  if (!out) return QH_EINVAL;
  *out = nullptr;
  if (!blob) return QH_EINVAL;
  if (max_ctx < 1 || max_ctx > QH_MAX_CTX) return QH_ERANGE;
  const Layout& L = canonical_layout();
  if (blob_len != L.total) return QH_EFORMAT;
  if (idx_text && !check_idx_text(idx_text, L).empty()) return QH_EFORMAT;
  qh_engine* e = new (std::nothrow) qh_engine();
  if (!e) return QH_ENOMEM;
  e->L = &L;
  e->max_ctx = max_ctx;
  if (const char* pl = std::getenv("QH_POLL_LIMIT")) {   // test hook: force a hand-over wait to give up
    const long v = std::strtol(pl, nullptr, 10);
    if (v >= 0 && v <= (1L << 20)) e->poll_limit = (unsigned)v;
  }
  if (const char* ts = std::getenv("QH_TAG_START")) {   // test hook: start the tags near the wrap
    const unsigned long long v = std::strtoull(ts, nullptr, 10);
    if (v >= 1 && v <= 0xFFFFFFFFull) e->tag_start = (uint32_t)v;
  }
  e->nsplit_max = attn_nsplit_max(max_ctx);
  e->head_grid = kVocab / (kRowsPerBatch * 4 * 4);   // 4 waves x 4 batches per block
  int st = QH_OK;
#define QH_C(expr)             \
  do {                         \
    st = (expr);               \
    if (st != QH_OK) goto fail; \
  } while (0)
  QH_C(hip_status(hipStreamCreate(&e->stream)));
  QH_C(dalloc(&e->blob, blob_len));
  QH_C(hip_status(hipMemcpy(e->blob, blob, blob_len, hipMemcpyHostToDevice)));
  QH_C(build_lanes(e, static_cast<const uint8_t*>(blob)));
  QH_C(dalloc(&e->rec, (size_t)kNLinear * kLH * kLK * kLV));
  QH_C(dalloc(&e->conv, (size_t)kNLinear * kConvDim * kConvK));
  QH_C(dalloc(&e->kc, (size_t)kNFull * max_ctx * kKVProj));
  QH_C(dalloc(&e->vc, (size_t)kNFull * max_ctx * kKVProj));
  QH_C(dalloc(&e->h, kHidden));
  QH_C(dalloc(&e->convd, kConvDim));
  QH_C(dalloc(&e->zb, kZDim));
  QH_C(dalloc(&e->gb, 32));
  QH_C(dalloc(&e->o, kLH * kLV));
  QH_C(dalloc(&e->act, kInter));
  QH_C(dalloc(&e->og, kNH * kHD));
  QH_C(dalloc(&e->qkv, kQProj + 2 * kKVProj));
  QH_C(dalloc(&e->pm, (size_t)8 * e->nsplit_max));
  QH_C(dalloc(&e->pl, (size_t)8 * e->nsplit_max));
  QH_C(dalloc(&e->pacc, (size_t)8 * e->nsplit_max * 256));
  QH_C(dalloc(&e->rope, (size_t)max_ctx * 64));
  QH_C(dalloc(&e->logits, kVocab));
  QH_C(dalloc(&e->part_val, e->head_grid > 256 ? e->head_grid : 256));
  QH_C(dalloc(&e->part_idx, e->head_grid > 256 ? e->head_grid : 256));
  QH_C(dalloc(&e->abort_dev, 1));
  if (persist_max_grid(&e->persist_grid) != 0) e->persist_grid = 0;
  // every workgroup holds at most kDnSlots DeltaNet state tiles, one unit per stage
  e->dn_lds = e->persist_grid >= kLH * kDnVQuarters &&
              e->persist_grid * kDnSlots >= kNLinear * kLH * kDnVQuarters;
  if (e->persist_grid == 0) e->exec = QH_EXEC_GRAPH;
  QH_C(hip_status(hipEventCreate(&e->launch_ev[0])));
  QH_C(hip_status(hipEventCreate(&e->launch_ev[1])));
  QH_C(dalloc(&e->ctl, 1));
  {
    std::vector<float> rope((size_t)max_ctx * 64);
    for (int p = 0; p < max_ctx; ++p) rope_row(p, &rope[(size_t)p * 64]);
    QH_C(hip_status(hipMemcpy(e->rope, rope.data(), rope.size() * 4, hipMemcpyHostToDevice)));
  }
  QH_C(ensure_io(e, 1024));
  QH_C(qh_engine_reset(e));
#undef QH_C
  *out = e;
  return QH_OK;
fail:
  release(e);
  return st;
}

}  // namespace

extern "C" {

int qh_engine_create_from_memory(const void* blob, size_t blob_len, const char* idx_text, int max_ctx,
                                 qh_engine** out) {
  return create(blob, blob_len, idx_text, max_ctx, out);
}

int qh_engine_create(const char* blob_path, const char* idx_path, int max_ctx, qh_engine** out) {
  if (!blob_path || !out) return QH_EINVAL;
  std::string idx;
  if (idx_path) {   // tb_decode.cpp:47-51
    std::ifstream f(idx_path);
    if (!f) return QH_EIO;
    std::stringstream ss;
    ss << f.rdbuf();
    idx = ss.str();
  }
  const int fd = ::open(blob_path, O_RDONLY);   // run_hls.cpp:27-35
  if (fd < 0) return QH_EIO;
  struct stat sb;
  if (::fstat(fd, &sb) != 0) {
    ::close(fd);
    return QH_EIO;
  }
  const size_t len = (size_t)sb.st_size;
  if (len != canonical_layout().total) {
    ::close(fd);
    return QH_EFORMAT;
  }
  void* p = ::mmap(nullptr, len, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (p == MAP_FAILED) return QH_EIO;
  const int st = create(p, len, idx_path ? idx.c_str() : nullptr, max_ctx, out);
  ::munmap(p, len);
  return st;
}

int qh_engine_destroy(qh_engine* e) {
  if (!e) return QH_EINVAL;
  release(e);
  return QH_OK;
}

int qh_engine_set_mode(qh_engine* e, int mode) {
  if (!e || (mode != QH_MODE_W8A16 && mode != QH_MODE_W8A8)) return QH_EINVAL;
  e->mode = mode == QH_MODE_W8A8 ? M_W8A8 : M_W8A16;
  return QH_OK;
}

int qh_engine_set_exec(qh_engine* e, int exec) {
  if (!e || (exec != QH_EXEC_PERSISTENT && exec != QH_EXEC_GRAPH)) return QH_EINVAL;
  if (exec == QH_EXEC_PERSISTENT && e->persist_grid == 0) return QH_ESTATE;
  e->exec = exec;
  return QH_OK;
}

int qh_engine_get_exec(const qh_engine* e) { return e ? e->exec : QH_EINVAL; }
int qh_engine_head_grid(const qh_engine* e, int exec) {
  if (!e || (exec != QH_EXEC_PERSISTENT && exec != QH_EXEC_GRAPH)) return QH_EINVAL;
  if (exec == QH_EXEC_PERSISTENT) return e->persist_grid > 0 ? e->persist_grid : QH_ESTATE;
  return e->head_grid;
}

int qh_engine_exec_fallbacks(const qh_engine* e) { return e ? e->fallbacks : QH_EINVAL; }

int qh_engine_reset(qh_engine* e) {
  if (!e) return QH_EINVAL;
  hipStream_t s = e->stream;
  QH_HIP(hipMemsetAsync(e->rec, 0, sizeof(float) * (size_t)kNLinear * kLH * kLK * kLV, s));
  QH_HIP(hipMemsetAsync(e->conv, 0, sizeof(float) * (size_t)kNLinear * kConvDim * kConvK, s));
  QH_HIP(hipMemsetAsync(e->kc, 0, sizeof(float) * (size_t)kNFull * e->max_ctx * kKVProj, s));
  QH_HIP(hipMemsetAsync(e->vc, 0, sizeof(float) * (size_t)kNFull * e->max_ctx * kKVProj, s));
  StepCtl c;
  std::memset(&c, 0, sizeof c);
  c.max_ctx = e->max_ctx;
  c.eos = -1;
  QH_HIP(hipMemcpyAsync(e->ctl, &c, sizeof c, hipMemcpyHostToDevice, s));
  QH_HIP(hipStreamSynchronize(s));
  e->host_pos = 0;
  e->last_argmax = -1;
  e->broken = false;
  return QH_OK;
}

int qh_decode_token(qh_engine* e, int tok, float* logits, int* argmax_out) {
  if (!e || !argmax_out) return QH_EINVAL;
  if (e->broken) return QH_ESTATE;
  if (tok < 0 || tok >= kVocab) return QH_ERANGE;
  if (e->host_pos >= e->max_ctx) return QH_ERANGE;
  if (e->exec == QH_EXEC_PERSISTENT) {   // one token = a prompt of one, no new tokens
    QH_HIP(hipMemcpyAsync(e->prompt_dev, &tok, sizeof(int), hipMemcpyHostToDevice, e->stream));
    StepCtl c;
    const int st = run_persist(e, tok, 1, 0, -1, logits != nullptr, &c);
    if (st != kUseGraph) {
      QH_TRY(st);
      if (logits) QH_HIP(hipMemcpy(logits, e->logits, sizeof(float) * kVocab, hipMemcpyDeviceToHost));
      *argmax_out = c.argmax;
      return QH_OK;
    }
  }
  hipGraphExec_t g;
  QH_TRY(get_graph(e, logits != nullptr, false, &g));
  hipStream_t s = e->stream;
  QH_HIP(launch_set_int(&e->ctl->tok, tok, s));
  QH_HIP(launch_set_int(&e->ctl->done, 0, s));
  QH_HIP(hipGraphLaunch(g, s));
  StepCtl c;
  QH_HIP(hipMemcpyAsync(&c, e->ctl, sizeof c, hipMemcpyDeviceToHost, s));
  if (logits) QH_HIP(hipMemcpyAsync(logits, e->logits, sizeof(float) * kVocab, hipMemcpyDeviceToHost, s));
  QH_HIP(hipStreamSynchronize(s));
  e->host_pos = c.pos;
  e->last_argmax = c.argmax;
  *argmax_out = c.argmax;
  return QH_OK;
}

int qh_generate(qh_engine* e, const int* prompt, int n_prompt, int n_new, int eos, int* out_ids, int* n_out) {
  if (!e || !prompt || n_prompt < 1 || n_new < 0 || (n_new > 0 && !out_ids) || !n_out) return QH_EINVAL;
  if (e->broken) return QH_ESTATE;
  for (int i = 0; i < n_prompt; ++i)
    if (prompt[i] < 0 || prompt[i] >= kVocab) return QH_ERANGE;
  if ((long)e->host_pos + n_prompt + n_new > e->max_ctx) return QH_ERANGE;
  QH_TRY(ensure_io(e, n_prompt > n_new ? n_prompt : n_new));
  hipStream_t s = e->stream;
  QH_HIP(hipMemcpyAsync(e->prompt_dev, prompt, sizeof(int) * (size_t)n_prompt, hipMemcpyHostToDevice, s));
  QH_HIP(hipStreamSynchronize(s));
  if (e->exec == QH_EXEC_PERSISTENT) {
    StepCtl c;
    const int st = run_persist(e, prompt[0], n_prompt, n_new, eos, false, &c);
    if (st != kUseGraph) {
      QH_TRY(st);
      if (c.n_out > 0)
        QH_HIP(hipMemcpy(out_ids, e->out_dev, sizeof(int) * (size_t)c.n_out, hipMemcpyDeviceToHost));
      *n_out = c.n_out;
      return c.err == 2 ? QH_ERANGE : QH_OK;
    }
  }
  hipGraphExec_t g;
  QH_TRY(get_graph(e, false, true, &g));
  QH_HIP(launch_init_gen(e->ctl, prompt[0], n_prompt, n_new, eos, s));
  for (int i = 0; i < n_prompt + n_new; ++i) QH_HIP(hipGraphLaunch(g, s));
  StepCtl c;
  QH_HIP(hipMemcpyAsync(&c, e->ctl, sizeof c, hipMemcpyDeviceToHost, s));
  QH_HIP(hipStreamSynchronize(s));
  if (c.n_out > 0) QH_HIP(hipMemcpy(out_ids, e->out_dev, sizeof(int) * (size_t)c.n_out, hipMemcpyDeviceToHost));
  *n_out = c.n_out;
  e->host_pos = c.pos;
  e->last_argmax = c.argmax;
  QH_HIP(launch_set_int(&e->ctl->done, 0, s));
  QH_HIP(hipStreamSynchronize(s));
  return c.err == 2 ? QH_ERANGE : QH_OK;
}

int qh_engine_pos(const qh_engine* e) { return e ? e->host_pos : -1; }
int qh_engine_last_argmax(const qh_engine* e) { return e ? e->last_argmax : -1; }
float qh_engine_last_launch_ms(const qh_engine* e) { return e ? e->last_launch_ms : 0.0f; }

int qh_engine_forward_layers(qh_engine* e, int l0, int l1, float* h) {
  if (!e || !h || l0 < 0 || l1 > kLayers || l0 >= l1) return QH_EINVAL;
  if (e->broken) return QH_ESTATE;
  if (e->host_pos >= e->max_ctx) return QH_ERANGE;
  hipStream_t s = e->stream;
  QH_HIP(launch_set_int(&e->ctl->done, 0, s));
  QH_HIP(hipMemcpyAsync(e->h, h, sizeof(float) * kHidden, hipMemcpyDeviceToDevice, s));
  QH_TRY(enqueue_layers(e, l0, l1, false, s));
  QH_HIP(launch_bump_pos(e->ctl, s));
  QH_HIP(hipMemcpyAsync(h, e->h, sizeof(float) * kHidden, hipMemcpyDeviceToDevice, s));
  QH_HIP(hipStreamSynchronize(s));
  e->host_pos += 1;
  return QH_OK;
}

int qh_engine_profile(qh_engine* e, int n_steps, float* step_ms, float* head_ms) {
  if (!e || n_steps < 1 || !step_ms || !head_ms) return QH_EINVAL;
  if (e->broken) return QH_ESTATE;
  if ((long)e->host_pos + n_steps > e->max_ctx) return QH_ERANGE;
  hipStream_t s = e->stream;
  hipEvent_t a = nullptr, b = nullptr, h0 = nullptr, h1 = nullptr;
  int st = QH_OK;
  float tot_head = 0.0f, tot = 0.0f;
  if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess || hipEventCreate(&h0) != hipSuccess ||
      hipEventCreate(&h1) != hipSuccess) {
    st = QH_ENOMEM;
  }
  for (int i = 0; st == QH_OK && i < n_steps; ++i) {
    st = hip_status(launch_set_int(&e->ctl->done, 0, s));
    if (st == QH_OK) st = hip_status(hipEventRecord(a, s));
    if (st == QH_OK) st = enqueue_step(e, false, false, s, h0, h1);   // head events: kernel start / end
    if (st == QH_OK) st = hip_status(hipEventRecord(b, s));
    if (st == QH_OK) st = hip_status(hipEventSynchronize(b));
    float t = 0.0f, th = 0.0f;
    if (st == QH_OK) st = hip_status(hipEventElapsedTime(&t, a, b));
    if (st == QH_OK) st = hip_status(hipEventElapsedTime(&th, h0, h1));
    tot += t;
    tot_head += th;
  }
  if (a) (void)hipEventDestroy(a);
  if (b) (void)hipEventDestroy(b);
  if (h0) (void)hipEventDestroy(h0);
  if (h1) (void)hipEventDestroy(h1);
  if (st != QH_OK) return st;
  StepCtl c;
  QH_HIP(hipMemcpy(&c, e->ctl, sizeof c, hipMemcpyDeviceToHost));
  e->host_pos = c.pos;
  e->last_argmax = c.argmax;
  *step_ms = tot / n_steps;
  *head_ms = tot_head / n_steps;
  return QH_OK;
}

void* qh_engine_stream(qh_engine* e) { return e ? (void*)e->stream : nullptr; }

void* qh_engine_device_ptr(qh_engine* e, int which) {
  if (!e) return nullptr;
  switch (which) {
    case 0: return e->blob;
    case 1: return e->rec;
    case 2: return e->conv;
    case 3: return e->kc;
    case 4: return e->vc;
    case 5: return e->h;
    default: return nullptr;
  }
}

}  // extern "C"
