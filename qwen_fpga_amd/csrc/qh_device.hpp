// Device helpers for the gfx950 decode kernels: deterministic transcendentals
// and the fixed-order wavefront reductions every kernel uses.
//
// Determinism contract.  Every floating-point value the kernels produce is a
// fixed sequence of IEEE-754 operations (round-to-nearest +, -, *, /, sqrt,
// fma), independent of launch geometry and timing: no float atomics, fixed
// reduction trees, and exp / log1p built here from those operations only.  The
// code is compiled with -ffp-contract=off, so an fma appears exactly where
// fmaf() is written.
//
// "C16" order for a length-n dot product or sum of squares: element i is in
// chunk i/16, chunk c is owned by lane c mod 64, each lane accumulates its
// elements in increasing i with fma starting from 0, and the L lane partials
// (L = min(64, pow2ceil(ceil(n/16)))) are combined by the xor butterfly with
// offsets L/2, ..., 1.  Since IEEE addition is commutative, every lane of a
// butterfly group ends with the same, fully determined value.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qh {

// exp: n = rint(x*log2 e); r = x - n*ln2 with a two-part ln2 (Cody-Waite);
// e^r by its degree-7 Taylor polynomial (Horner, fma) on |r| <= ln2/2; exact
// scaling by 2^n in at most two steps (overflow -> inf, deep underflow -> 0).
__device__ __forceinline__ float dev_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return __builtin_inff();
  if (x < -103.972084045410156f) return 0.0f;
  const float n = __builtin_rintf(x * 1.44269502162933349609375f);
  float r = __builtin_fmaf(n, -0.693145751953125f, x);
  r = __builtin_fmaf(n, -1.428606765330187045e-06f, r);
  float p = 1.984126984126984e-4f;
  p = __builtin_fmaf(p, r, 1.388888888888889e-3f);
  p = __builtin_fmaf(p, r, 8.333333333333333e-3f);
  p = __builtin_fmaf(p, r, 4.166666666666667e-2f);
  p = __builtin_fmaf(p, r, 1.666666666666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int ni = (int)n;
  if (ni > 127) { p = p * 2.0f; ni -= 1; }
  if (ni < -126) { p = p * 5.42101086242752217e-20f; ni += 64; }
  return p * __uint_as_float((uint32_t)(ni + 127) << 23);
}

// log(u) for u >= 1 in double: u = m*2^e, m in [sqrt(1/2), sqrt(2)); log m =
// 2*atanh(s), s = (m-1)/(m+1), odd series to s^21; e*ln2 with ln2 split so that
// e*ln2_hi is exact.
__device__ __forceinline__ double dev_log_d(double u) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(u);
  int e = (int)((b >> 52) & 0x7ffu) - 1023;
  double m = __longlong_as_double((long long)((b & 0x000fffffffffffffull) | 0x3ff0000000000000ull));
  if (m > 1.4142135623730951) { m = m * 0.5; e += 1; }
  const double s = (m - 1.0) / (m + 1.0);
  const double s2 = s * s;
  double t = 1.0 / 21.0;
  t = __builtin_fma(t, s2, 1.0 / 19.0);
  t = __builtin_fma(t, s2, 1.0 / 17.0);
  t = __builtin_fma(t, s2, 1.0 / 15.0);
  t = __builtin_fma(t, s2, 1.0 / 13.0);
  t = __builtin_fma(t, s2, 1.0 / 11.0);
  t = __builtin_fma(t, s2, 1.0 / 9.0);
  t = __builtin_fma(t, s2, 1.0 / 7.0);
  t = __builtin_fma(t, s2, 1.0 / 5.0);
  t = __builtin_fma(t, s2, 1.0 / 3.0);
  t = __builtin_fma(t, s2, 1.0);
  const double lm = (2.0 * s) * t;
  const double fe = (double)e;
  return __builtin_fma(fe, 6.93147180369123816490e-01, __builtin_fma(fe, 1.90821492927058770002e-10, lm));
}

// log1p for y >= 0: y itself below 2^-28 (the rounded log1p there), else the
// double log of 1 + y (exact in double), rounded once to float.
__device__ __forceinline__ float dev_log1pf(float y) {
  if (y != y) return y;
  if (y == __builtin_inff()) return y;
  if (y < 3.7252902984619140625e-09f) return y;
  return (float)dev_log_d(1.0 + (double)y);
}

// hls/src/activations.hpp:7-14 with the device exp / log1p.
__device__ __forceinline__ float dev_silu(float x) { return x / (1.0f + dev_expf(-x)); }
__device__ __forceinline__ float dev_sigmoid(float x) { return 1.0f / (1.0f + dev_expf(-x)); }
__device__ __forceinline__ float dev_softplus(float x) {
  return x > 20.0f ? x : dev_log1pf(dev_expf(x));
}

// Marks a loaded value as read without using it.  A load whose result is
// never read keeps its registers pending; the next write to one of them -- at
// the stage boundary, where the compiler cannot count the loads in flight --
// then waits for every load and store of the wave.  Placed after a wait that
// already covers the load (a later load's), it costs nothing.
template <typename T>
__device__ __forceinline__ void settle(const T& v) {
  asm volatile("" ::"v"(v));
}

// Workgroup barrier for LDS hand-offs: the fences cover LDS only, so this
// wave's global loads and stores stay in flight across it (__syncthreads()
// orders global memory too).  Used where waves exchange only LDS data; vectors
// produced by other workgroups arrive through tagged polls, which need no
// ordering.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// gfx950's permlane swaps, written as inline assembly with both registers as
// in/out operands: v_permlane32_swap a, b exchanges the upper 32 lanes of a with
// the lower 32 lanes of b (afterwards a = [a.lo, b.lo], b = [a.hi, b.hi]);
// v_permlane16_swap does the same for the odd 16-lane rows of a and the even
// rows of b (a = [a.r0, b.r0, a.r2, b.r2], b = [a.r1, b.r1, a.r3, b.r3]).  The
// s_nop pairs cover the VALU-write / permlane-read wait states, which the
// compiler does not insert around inline assembly.  (The two-result builtin
// is not used: this compiler folds its second result into the first when both
// feed arithmetic.)
__device__ __forceinline__ void permlane32_swap(unsigned& a, unsigned& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void permlane16_swap(unsigned& a, unsigned& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

// threadIdx.x, opaque to the optimiser.  A lane mask formed from it (a 64-bit
// scalar register pair) is then formed where it is used: from threadIdx.x
// itself the compiler hoists such masks out of the persistent kernel's stage
// loop and holds them across every stage, which spills scalar registers.
__device__ __forceinline__ int tid_here() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// Lane l receives the value of lane l ^ OFF, with VALU instructions only (no
// LDS round trip): quad permutations (DPP) for 1 and 2; row_half_mirror
// (l ^ 7) then quad_perm [3,2,1,0] (l ^ 3) for 4; rotation of a 16-lane row by
// 8 (DPP row_ror) for 8; a permlane swap for 16 and 32.  Each is an exact
// permutation, so a butterfly built from them is bit-identical to one built
// from __shfl_xor.
template <int OFF>
__device__ __forceinline__ int xor_perm_i(int v) {
  static_assert(OFF == 1 || OFF == 2 || OFF == 4 || OFF == 8 || OFF == 16 || OFF == 32, "xor offset");
  if constexpr (OFF == 1) return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  if constexpr (OFF == 2) return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  if constexpr (OFF == 4) {
    const int t = __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);                 // row_half_mirror
    return __builtin_amdgcn_update_dpp(0, t, 0x1B, 0xF, 0xF, false);                         // quad_perm [3,2,1,0]
  }
  if constexpr (OFF == 8) return __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false);  // row_ror:8
  unsigned a = (unsigned)v, b = (unsigned)v;
  if constexpr (OFF == 16) {
    permlane16_swap(a, b);   // a = v of the even row of each pair, b = v of the odd row
    return (int)((tid_here() & 16) ? a : b);
  }
  permlane32_swap(a, b);     // a = lower half of v (both halves), b = upper half
  return (int)((tid_here() & 32) ? a : b);
}
template <int OFF>
__device__ __forceinline__ float xor_perm(float v) {
  return __int_as_float(xor_perm_i<OFF>(__float_as_int(v)));
}

// One level of a transposed butterfly at offset 16 or 32: every lane keeps
// `lo` if its bit OFF is clear and `hi` if it is set, and adds the value its
// partner (lane ^ OFF) does not keep.  One permlane swap of (lo, hi) places
// both addends of every lane in its two registers, so the level costs one
// swap and one add; the sum equals keep + partner's send (commuted on the
// upper lanes, which IEEE addition does not notice).
template <int OFF, typename T>
__device__ __forceinline__ T swap_add(T lo, T hi) {
  static_assert(OFF == 16 || OFF == 32, "swap level");
  unsigned a = __builtin_bit_cast(unsigned, lo), b = __builtin_bit_cast(unsigned, hi);
  if constexpr (OFF == 16)
    permlane16_swap(a, b);
  else
    permlane32_swap(a, b);
  return __builtin_bit_cast(T, a) + __builtin_bit_cast(T, b);
}

// xor butterfly over groups of WIDTH lanes (offsets WIDTH/2 .. 1); every lane
// of a group ends with the same, fully determined value.
template <int WIDTH>
__device__ __forceinline__ float xor_sum(float v) {
  if constexpr (WIDTH >= 64) v = swap_add<32>(v, v);
  if constexpr (WIDTH >= 32) v = swap_add<16>(v, v);
  if constexpr (WIDTH >= 16) v = v + xor_perm<8>(v);
  if constexpr (WIDTH >= 8) v = v + xor_perm<4>(v);
  if constexpr (WIDTH >= 4) v = v + xor_perm<2>(v);
  if constexpr (WIDTH >= 2) v = v + xor_perm<1>(v);
  return v;
}
template <int WIDTH>
__device__ __forceinline__ int xor_sum_i(int v) {
  if constexpr (WIDTH >= 64) v = swap_add<32>(v, v);
  if constexpr (WIDTH >= 32) v = swap_add<16>(v, v);
  if constexpr (WIDTH >= 16) v = v + xor_perm_i<8>(v);
  if constexpr (WIDTH >= 8) v = v + xor_perm_i<4>(v);
  if constexpr (WIDTH >= 4) v = v + xor_perm_i<2>(v);
  if constexpr (WIDTH >= 2) v = v + xor_perm_i<1>(v);
  return v;
}
template <int WIDTH>
__device__ __forceinline__ float xor_max(float v) {
  if constexpr (WIDTH >= 64) v = fmaxf(v, xor_perm<32>(v));
  if constexpr (WIDTH >= 32) v = fmaxf(v, xor_perm<16>(v));
  if constexpr (WIDTH >= 16) v = fmaxf(v, xor_perm<8>(v));
  if constexpr (WIDTH >= 8) v = fmaxf(v, xor_perm<4>(v));
  if constexpr (WIDTH >= 4) v = fmaxf(v, xor_perm<2>(v));
  if constexpr (WIDTH >= 2) v = fmaxf(v, xor_perm<1>(v));
  return v;
}

// Lane partial of a C16 dot over one 16-element chunk (fma, increasing index).
__device__ __forceinline__ float dot16_f32(const float* a, const float* b, float acc) {
#pragma unroll
  for (int e = 0; e < 16; ++e) acc = __builtin_fmaf(a[e], b[e], acc);
  return acc;
}

// int8 weights packed in 4 dwords (byte b of dword d = element 4d+b) times fp32.
__device__ __forceinline__ float dot16_i8f(const uint32_t w[4], const float* x, float acc) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float wf = (float)(int)(int8_t)(w[d] >> (8 * b));
      acc = __builtin_fmaf(wf, x[4 * d + b], acc);
    }
  }
  return acc;
}

// int8 x int8 -> int32 over 16 elements (v_dot4 on gfx950).
__device__ __forceinline__ int dot16_i8i8(const uint32_t w[4], const uint32_t x[4], int acc) {
  acc = __builtin_amdgcn_sdot4((int)w[0], (int)x[0], acc, false);
  acc = __builtin_amdgcn_sdot4((int)w[1], (int)x[1], acc, false);
  acc = __builtin_amdgcn_sdot4((int)w[2], (int)x[2], acc, false);
  acc = __builtin_amdgcn_sdot4((int)w[3], (int)x[3], acc, false);
  return acc;
}

// Per-vector symmetric int8 (golden/model.py:37-45 _qa): s = amax/127 (1 if
// amax == 0), q = rint(x/s) clipped to +-127.
__device__ __forceinline__ float quant_scale(float amax) { return amax > 0.0f ? amax / 127.0f : 1.0f; }
__device__ __forceinline__ int quant_one(float x, float s) {
  float r = __builtin_rintf(x / s);
  r = fminf(fmaxf(r, -127.0f), 127.0f);
  return (int)r;
}
// Same q with the quotient formed by Markstein's correction from rs = RN(1/s):
// q0 = x*rs, r = fma(-s, q0, x), q = fma(r, rs, q0) equals RN(x/s) on this
// domain (|x| <= amax) except for the sign of a zero quotient, which rint and
// the int conversion erase.
__device__ __forceinline__ int quant_one_r(float x, float s, float rs) {
  const float q0 = x * rs;
  const float r = __builtin_fmaf(-s, q0, x);
  float t = __builtin_rintf(__builtin_fmaf(r, rs, q0));
  t = fminf(fmaxf(t, -127.0f), 127.0f);
  return (int)t;
}
__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
  return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
         ((uint32_t)(d & 0xff) << 24);
}

// Device-coherent access to the activation vectors that workgroups hand to one
// another: loads and stores with the sc1 cache-policy bit (device scope), which
// bypass the per-XCD L2 state.  Within one kernel launch a workgroup on
// another XCD sees such a store once it has completed; an ordinary load could
// hit a stale line in its own XCD's L2.  The vector forms are plain buffer
// loads/stores (not atomics), so a lane's loads issue back to back; their base
// pointer must be the same on every lane of the wave.  Weights and state that
// one workgroup owns use ordinary accesses.
constexpr int kSc1 = 16;   // cache-policy operand: sc1
constexpr int kNt = 2;     // cache-policy operand: nt (non-temporal)

// A buffer descriptor sits in scalar registers.  Every base address that
// builds one here is the same on all lanes of the wave (a kernel argument or a
// stage-descriptor field that every lane reads from the same LDS word), but a
// value read from LDS lands in a vector register and the compiler cannot see
// that it is uniform: it would wrap each access in a loop over the distinct
// values.  readfirstlane states the uniformity, so an access is one
// instruction.  Callers must pass wave-uniform values.
__device__ __forceinline__ void* wave_uniform(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coh_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(wave_uniform(base), (short)0, 0x7ffffff0, 0x00020000);
}
// Global / LDS views of generic pointers.  An access through a generic
// pointer is a flat_* instruction, which the hardware counts against both the
// vector-memory and the LDS counters: every wait for an LDS read would then
// also wait for the flat accesses in flight (weight prefetches, state
// stores).  Through these views the compiler emits global_* (vector-memory
// counter only) or ds_* instructions.  The pointer must address that memory.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* as_global(const T* p) {
  return (const __attribute__((address_space(1))) T*)p;
}
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* as_global_w(T* p) {
  return (__attribute__((address_space(1))) T*)p;
}
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(3))) T* as_lds(const T* p) {
  return (const __attribute__((address_space(3))) T*)p;
}
template <typename T>
__device__ __forceinline__ __attribute__((address_space(3))) T* as_lds_w(T* p) {
  return (__attribute__((address_space(3))) T*)p;
}

__device__ __forceinline__ float ldc(const float* p) {
  return __uint_as_float(__hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ int ldc_i(const int* p) {
  return __hip_atomic_load(as_global(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stc(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stc_i(int* p, int v) {
  __hip_atomic_store(as_global_w(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// base[idx] (uniform base, per-lane idx)
__device__ __forceinline__ float ldcb(const float* base, int idx) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(coh_rsrc(base), idx * 4, 0, kSc1));
}
__device__ __forceinline__ void stcb(float* base, int idx, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), coh_rsrc(base), idx * 4, 0, kSc1);
}
// base[idx .. idx+3], idx a multiple of 4
__device__ __forceinline__ void ldc4(const float* base, int idx, float* v) {
  const auto u = __builtin_amdgcn_raw_buffer_load_b128(coh_rsrc(base), idx * 4, 0, kSc1);
  v[0] = __uint_as_float(u[0]);
  v[1] = __uint_as_float(u[1]);
  v[2] = __uint_as_float(u[2]);
  v[3] = __uint_as_float(u[3]);
}
__device__ __forceinline__ void stc4(float* base, int idx, const float* v) {
  __attribute__((ext_vector_type(4))) uint32_t u;
  u[0] = __float_as_uint(v[0]);
  u[1] = __float_as_uint(v[1]);
  u[2] = __float_as_uint(v[2]);
  u[3] = __float_as_uint(v[3]);
  __builtin_amdgcn_raw_buffer_store_b128(u, coh_rsrc(base), idx * 4, 0, kSc1);
}
// base[idx .. idx+15], idx a multiple of 4
__device__ __forceinline__ void ldc16(const float* base, int idx, float* v) {
#pragma unroll
  for (int k = 0; k < 4; ++k) ldc4(base, idx + 4 * k, v + 4 * k);
}
__device__ __forceinline__ void stc16(float* base, int idx, const float* v) {
#pragma unroll
  for (int k = 0; k < 4; ++k) stc4(base, idx + 4 * k, v + 4 * k);
}

}  // namespace qh
