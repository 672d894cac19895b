// Device helpers for gfx950: fp16 pair arithmetic, exact integer->fp16 code
// expansion, DPP lane reductions and the argmax comparator.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "aexq_internal.hpp"

namespace aexq {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f16x2 as_h2(uint32_t u) { return __builtin_bit_cast(f16x2, u); }
__device__ __forceinline__ uint32_t as_u(f16x2 h) { return __builtin_bit_cast(uint32_t, h); }

// v_dot2_f32_f16: c + a.x*b.x + a.y*b.y with fp32 accumulation.
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
}

// Four int8 codes of one word -> two fp16 pairs holding the exact integers.
// Biasing by 0x80 gives u = q + 128 in [0, 255]; the fp16 with bits 0x6400|u is
// 1024 + u exactly, so subtracting 1152 yields q with no rounding.
// lo = (q0, q1), hi = (q2, q3) in element order.
__device__ __forceinline__ void q8_pairs(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const uint32_t u = w ^ 0x80808080u;
  const f16x2 bias = {(f16)1152.0f, (f16)1152.0f};
  lo = as_u(as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias);
  hi = as_u(as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias);
}

// Eight offset-8 nibbles of one word (n0 in bits 0-3) -> four fp16 pairs of the
// exact codes q = n - 8.  Pair p holds elements (p, p + 4): bits 0x6400|n give
// 1024 + n, and subtracting 1032 is exact.
__device__ __forceinline__ void q4_pairs(uint32_t w, uint32_t q[4]) {
  const uint32_t M = 0x000F000Fu, E = 0x64006400u;
  const f16x2 bias = {(f16)1032.0f, (f16)1032.0f};
  q[0] = as_u(as_h2((w & M) | E) - bias);
  q[1] = as_u(as_h2(((w >> 4) & M) | E) - bias);
  q[2] = as_u(as_h2(((w >> 8) & M) | E) - bias);
  q[3] = as_u(as_h2(((w >> 12) & M) | E) - bias);
}

// Reorders 8 consecutive fp16 activations (a=(x0,x1) b=(x2,x3) c=(x4,x5)
// d=(x6,x7)) into the (p, p+4) pairs that q4_pairs produces.
__device__ __forceinline__ void q4_xpairs(uint32_t a, uint32_t b, uint32_t c, uint32_t d,
                                          uint32_t* out) {
  out[0] = __builtin_amdgcn_perm(c, a, 0x05040100u);  // (x0, x4)
  out[1] = __builtin_amdgcn_perm(c, a, 0x07060302u);  // (x1, x5)
  out[2] = __builtin_amdgcn_perm(d, b, 0x05040100u);  // (x2, x6)
  out[3] = __builtin_amdgcn_perm(d, b, 0x07060302u);  // (x3, x7)
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of LPR lanes (16, 32 or 64); every lane of a group
// receives the group total.  Within a 16-lane DPP row: rotate by 8 and 4, then
// quad swaps; across rows: lane shuffles.
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp<0x128>(v);  // row_ror:8
  v += dpp<0x124>(v);  // row_ror:4
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  if constexpr (LPR >= 32) v += __shfl_xor(v, 16, 64);
  if constexpr (LPR >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

// Argmax order of the reference scan (MM:645-686: element 0 first, then any
// later value > best): a NaN at index 0 is never replaced, a NaN elsewhere never
// wins, ties go to the lower index.  Returns true when (av, ai) beats (bv, bi).
__device__ __forceinline__ bool argmax_beats(float av, int ai, float bv, int bi) {
  const bool an = __builtin_isnan(av), bn = __builtin_isnan(bv);
  if (an && ai == 0) return true;
  if (bn && bi == 0) return false;
  if (an) return false;
  if (bn) return true;
  if (av != bv) return av > bv;
  return ai < bi;
}

// Merge (ov, oi, os) into (bv, bi, bs): best value, its index, and the best
// value among the other candidates (NaN ignored).
__device__ __forceinline__ void argmax_merge(float& bv, int& bi, float& bs, float ov, int oi,
                                             float os) {
  if (argmax_beats(ov, oi, bv, bi)) {
    bs = fmaxf(os, fmaxf(bv, bs));
    bv = ov;
    bi = oi;
  } else {
    bs = fmaxf(bs, fmaxf(ov, os));
  }
}

__device__ __forceinline__ void argmax_wave_reduce(float& bv, int& bi, float& bs) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    const float os = __shfl_xor(bs, off, 64);
    argmax_merge(bv, bi, bs, ov, oi, os);
  }
}

__device__ __forceinline__ float load_scale(const void* s, long long i, bool f16_scale) {
  return f16_scale ? (float)((const f16*)s)[i] : ((const float*)s)[i];
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

}  // namespace aexq
