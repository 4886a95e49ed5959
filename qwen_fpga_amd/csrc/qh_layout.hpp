// Packed weight-blob layout of the 0.8B hybrid model and the seeded synthetic
// weight generator.
//
// The layout restates scripts/pack_weights.py:25-101 (reference): tensors in the
// order the decode kernel reads them (pack_weights.py:28-47 read_order), each
// start padded to 4 KiB, an int8 tensor stored as [out,in] int8 followed by its
// [out] fp32 per-row scales, an fp32 tensor stored as-is.  The per-tensor text
// line is scripts/emit_weight_index.py:13-22 ("name off nbytes dtype scale_off
// scale_nbytes out in").
#pragma once
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace qh {

constexpr int kHidden = 1024, kLayers = 24, kInter = 3584, kVocab = 248320;
constexpr int kLH = 16, kLK = 128, kLV = 128, kConvDim = 6144, kConvK = 4, kZDim = 2048;
constexpr int kNH = 8, kNKV = 2, kHD = 256, kQProj = 4096, kKVProj = 512, kRopeDim = 64;
constexpr int kNLinear = 18, kNFull = 6;
constexpr uint64_t kAlign = 4096;
constexpr float kEps = 1e-6f;
constexpr float kRopeTheta = 10000000.0f;

// hls/src/types.hpp:47
inline bool is_linear(int layer) { return (layer % 4) != 3; }

// One tensor role per (layer, slot); FINAL and EMBED live at layer index kLayers.
enum Role : int {
  R_IN_LN = 0, R_QKV, R_Z, R_B, R_A, R_CONV, R_ALOG, R_DTB, R_LNORM, R_OUTP,
  R_QP, R_KP, R_VP, R_QN, R_KN, R_OP,
  R_POST_LN, R_GATE, R_UP, R_DOWN,
  R_FINAL, R_EMBED, R_COUNT
};

struct Entry {
  std::string name;
  uint64_t off = 0, nbytes = 0, soff = 0, snbytes = 0;
  int dtype = 0;         // 0 fp32, 1 int8
  int out = 0, in = 0;   // 2-D GEMV dims as in weights.idx (0 for non-matrix)
  int layer = 0;
  Role role = R_IN_LN;
  std::vector<int> shape;
  uint64_t numel() const {
    uint64_t n = 1;
    for (int s : shape) n *= (uint64_t)s;
    return n;
  }
};

struct Layout {
  std::vector<Entry> entries;          // read order
  uint64_t total = 0;                  // blob bytes (pack_weights.py:92)
  int index[kLayers + 1][R_COUNT];     // entry index or -1
  const Entry* get(int layer, Role r) const {
    const int i = index[layer][r];
    return i < 0 ? nullptr : &entries[(size_t)i];
  }
};

const Layout& canonical_layout();
std::string idx_text(const Layout& L);
// Parses a weights.idx text and checks every line against the canonical layout.
// Returns "" when it matches, else a description of the first difference.
std::string check_idx_text(const std::string& text, const Layout& L);

// SplitMix64 stream with state `key`: element i is the (i+1)-th output.
inline uint64_t rng_u64(uint64_t key, uint64_t i) {
  uint64_t z = key + (i + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
void fill_i8(int8_t* dst, size_t n, uint64_t key);
void fill_uniform(float* dst, size_t n, uint64_t key, float lo, float hi);
void fill_normal(float* dst, size_t n, uint64_t key, float mean, float stddev);
// Writes the synthetic model into blob (len must be >= L.total).
void synth_blob(uint8_t* blob, const Layout& L, uint64_t seed);

}  // namespace qh
