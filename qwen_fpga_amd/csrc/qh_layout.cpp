// Layout builder, weights.idx text, and the seeded synthetic model.
#include "qh_layout.hpp"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <sstream>
#include <thread>

namespace qh {

namespace {

struct Spec {
  const char* suffix;
  Role role;
  std::vector<int> shape;
  bool quant;   // int8 + per-row scales (golden/quant.py:13-25 QUANT_SUFFIXES, 2-D only)
};

Layout build() {
  Layout L;
  for (auto& row : L.index)
    for (int& v : row) v = -1;
  // pack_weights.py:28-47 read_order: per layer in_ln, mixer tensors, post_ln, mlp; then norm, embed.
  const std::vector<Spec> lin = {
      {"linear_attn.in_proj_qkv.weight", R_QKV, {kConvDim, kHidden}, true},
      {"linear_attn.in_proj_z.weight", R_Z, {kZDim, kHidden}, true},
      {"linear_attn.in_proj_b.weight", R_B, {kLH, kHidden}, false},
      {"linear_attn.in_proj_a.weight", R_A, {kLH, kHidden}, false},
      {"linear_attn.conv1d.weight", R_CONV, {kConvDim, 1, kConvK}, false},
      {"linear_attn.A_log", R_ALOG, {kLH}, false},
      {"linear_attn.dt_bias", R_DTB, {kLH}, false},
      {"linear_attn.norm.weight", R_LNORM, {kLV}, false},
      {"linear_attn.out_proj.weight", R_OUTP, {kHidden, kLH * kLV}, true},
  };
  const std::vector<Spec> full = {
      {"self_attn.q_proj.weight", R_QP, {kQProj, kHidden}, true},
      {"self_attn.k_proj.weight", R_KP, {kKVProj, kHidden}, true},
      {"self_attn.v_proj.weight", R_VP, {kKVProj, kHidden}, true},
      {"self_attn.q_norm.weight", R_QN, {kHD}, false},
      {"self_attn.k_norm.weight", R_KN, {kHD}, false},
      {"self_attn.o_proj.weight", R_OP, {kHidden, kNH * kHD}, true},
  };
  const std::vector<Spec> mlp = {
      {"mlp.gate_proj.weight", R_GATE, {kInter, kHidden}, true},
      {"mlp.up_proj.weight", R_UP, {kInter, kHidden}, true},
      {"mlp.down_proj.weight", R_DOWN, {kHidden, kInter}, true},
  };
  uint64_t off = 0;
  auto add = [&](const std::string& name, int layer, const Spec& s) {
    off += (kAlign - off % kAlign) % kAlign;   // pack_weights.py:71-74
    Entry e;
    e.name = name;
    e.layer = layer;
    e.role = s.role;
    e.shape = s.shape;
    e.off = off;
    e.out = s.shape.size() >= 1 ? s.shape[0] : 0;   // emit_weight_index.py:16-17
    e.in = s.shape.size() >= 2 ? s.shape[1] : 0;
    if (s.quant) {   // pack_weights.py:76-84
      e.dtype = 1;
      e.nbytes = e.numel();
      e.soff = off + e.nbytes;
      e.snbytes = 4ull * (uint64_t)e.out;
      off += e.nbytes + e.snbytes;
    } else {         // pack_weights.py:85-89
      e.dtype = 0;
      e.nbytes = 4ull * e.numel();
      off += e.nbytes;
    }
    L.index[layer][s.role] = (int)L.entries.size();
    L.entries.push_back(e);
  };
  for (int l = 0; l < kLayers; ++l) {
    const std::string p = "layers." + std::to_string(l) + ".";
    add(p + "input_layernorm.weight", l, {"", R_IN_LN, {kHidden}, false});
    for (const Spec& s : is_linear(l) ? lin : full) add(p + s.suffix, l, s);
    add(p + "post_attention_layernorm.weight", l, {"", R_POST_LN, {kHidden}, false});
    for (const Spec& s : mlp) add(p + s.suffix, l, s);
  }
  add("norm.weight", kLayers, {"", R_FINAL, {kHidden}, false});
  add("embed_tokens.weight", kLayers, {"", R_EMBED, {kVocab, kHidden}, true});
  L.total = off;
  return L;
}

}  // namespace

const Layout& canonical_layout() {
  static const Layout L = build();
  return L;
}

std::string idx_text(const Layout& L) {
  std::string s;
  char line[256];
  for (const Entry& e : L.entries) {
    std::snprintf(line, sizeof line, "%s %llu %llu %d %llu %llu %d %d\n", e.name.c_str(),
                  (unsigned long long)e.off, (unsigned long long)e.nbytes, e.dtype,
                  (unsigned long long)e.soff, (unsigned long long)e.snbytes, e.out, e.in);
    s += line;
  }
  return s;
}

std::string check_idx_text(const std::string& text, const Layout& L) {
  std::istringstream in(text);
  std::string name;
  unsigned long long off, nb, so, sn;
  int dt, out, inn;
  size_t k = 0;
  // tb_decode.cpp:52-62: whitespace-separated fields, one tensor per line.
  while (in >> name >> off >> nb >> dt >> so >> sn >> out >> inn) {
    if (k >= L.entries.size()) return "idx has more than " + std::to_string(L.entries.size()) + " entries";
    const Entry& e = L.entries[k];
    if (name != e.name || off != e.off || nb != e.nbytes || dt != e.dtype || so != e.soff ||
        sn != e.snbytes || out != e.out || inn != e.in)
      return "idx line " + std::to_string(k + 1) + " (" + name + ") differs from the layout (" + e.name + ")";
    ++k;
  }
  if (!in.eof()) return "idx line " + std::to_string(k + 1) + " is malformed";
  if (k != L.entries.size())
    return "idx has " + std::to_string(k) + " entries, layout has " + std::to_string(L.entries.size());
  return "";
}

namespace {
template <class F>
void parallel_for(size_t n, F f) {
  unsigned nt = std::thread::hardware_concurrency();
  if (nt == 0) nt = 1;
  if (nt > 16) nt = 16;
  if (n < (1u << 16) || nt == 1) {
    f(0, n);
    return;
  }
  std::vector<std::thread> ts;
  const size_t chunk = (n + nt - 1) / nt;
  for (unsigned t = 0; t < nt; ++t) {
    const size_t a = t * chunk, b = std::min(n, a + chunk);
    if (a < b) ts.emplace_back([=] { f(a, b); });
  }
  for (auto& t : ts) t.join();
}
}  // namespace

void fill_i8(int8_t* dst, size_t n, uint64_t key) {
  parallel_for(n, [&](size_t a, size_t b) {
    for (size_t i = a; i < b; ++i) dst[i] = (int8_t)((int)(rng_u64(key, i) % 255u) - 127);
  });
}

void fill_uniform(float* dst, size_t n, uint64_t key, float lo, float hi) {
  parallel_for(n, [&](size_t a, size_t b) {
    for (size_t i = a; i < b; ++i) {
      const double u = (double)(rng_u64(key, i) >> 40) * (1.0 / 16777216.0);   // [0,1), 24 bits
      dst[i] = (float)((double)lo + ((double)hi - (double)lo) * u);
    }
  });
}

void fill_normal(float* dst, size_t n, uint64_t key, float mean, float stddev) {
  parallel_for(n, [&](size_t a, size_t b) {
    for (size_t i = a; i < b; ++i) {   // Box-Muller, one variate per element
      const double u1 = ((double)(rng_u64(key, 2 * i) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
      const double u2 = (double)(rng_u64(key, 2 * i + 1) >> 11) * (1.0 / 9007199254740992.0);
      const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
      dst[i] = (float)((double)mean + (double)stddev * z);
    }
  });
}

void synth_blob(uint8_t* blob, const Layout& L, uint64_t seed) {
  std::memset(blob, 0, L.total);
  for (size_t k = 0; k < L.entries.size(); ++k) {
    const Entry& e = L.entries[k];
    const uint64_t key = rng_u64(seed, 4 * k);
    const uint64_t key2 = rng_u64(seed, 4 * k + 1);
    if (e.dtype == 1) {
      fill_i8(reinterpret_cast<int8_t*>(blob + e.off), e.nbytes, key);
      fill_uniform(reinterpret_cast<float*>(blob + e.soff), (size_t)e.out, key2, 1e-3f, 1e-2f);
      continue;
    }
    float* f = reinterpret_cast<float*>(blob + e.off);
    const size_t n = (size_t)e.numel();
    switch (e.role) {
      case R_IN_LN: case R_POST_LN: case R_FINAL: case R_QN: case R_KN:
        fill_normal(f, n, key, 0.0f, 0.1f);   // zero-centred gains, used as (1 + w)
        break;
      case R_B: case R_A:
        fill_normal(f, n, key, 0.0f, 1.0f / 32.0f);   // unit-variance b, a for unit-rms x
        break;
      case R_CONV:
        fill_normal(f, n, key, 0.0f, 0.5f);
        break;
      case R_ALOG: {   // A = exp(A_log) ~ U[1, 16]
        fill_uniform(f, n, key, 1.0f, 16.0f);
        for (size_t i = 0; i < n; ++i) f[i] = std::log(f[i]);
        break;
      }
      case R_DTB:
        for (size_t i = 0; i < n; ++i) f[i] = 0.0f;
        break;
      case R_LNORM:   // gated-norm weight is ones-initialised (model.py:183-188)
        for (size_t i = 0; i < n; ++i) f[i] = 1.0f;
        break;
      default:
        fill_normal(f, n, key, 0.0f, 0.1f);
        break;
    }
  }
}

}  // namespace qh
