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
// fp32 from raw bits.  Vector elements go through this by-value parameter:
// ROCm 7.2 clang lowers __builtin_bit_cast(float, v[i]) on an ext_vector
// element to element 0 for every i.
__device__ __forceinline__ float as_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
// ...and raw bits of an fp32 value (same by-value detour).
__device__ __forceinline__ uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
__device__ __forceinline__ uint32_t as_u(f16x2 h) { return __builtin_bit_cast(uint32_t, h); }

// v_dot2_f32_f16: c + a.x*b.x + a.y*b.y with fp32 accumulation.
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
}

// Four Q8 codes of one device word -> two fp16 pairs holding the exact integers.
// The device copy stores every int8 code biased by 128 (u = q + 128 in [1, 255],
// applied once at upload), so the fp16 with bits 0x6400|u is 1024 + u exactly
// and subtracting 1152 yields q with no rounding.
// lo = (q0, q1), hi = (q2, q3) in element order.
__device__ __forceinline__ void q8_pairs(uint32_t u, uint32_t& lo, uint32_t& hi) {
  const f16x2 bias = {(f16)1152.0f, (f16)1152.0f};
  lo = as_u(as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias);
  hi = as_u(as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias);
}

// Eight offset-8 nibbles of one device word (n0 in bits 0-3; the device copy
// always holds offset-8 codes n = q + 8) -> four fp16 pairs of the exact codes,
// pair p holding elements (p, p + 4).  One shift, four v_and_or_b32 and four
// packed fp16 operations, all exact:
//   even nibbles: bits 0x6400|n       = 1024 + n    ; + (-1032)         -> n - 8
//   odd nibbles:  bits 0x6400|(n<<4)  = 1024 + 16n  ; * 1/16 + (-72)    -> n - 8
// gfx950's VOP3 encoding takes no literal operand, so with the masks and the
// exponent pattern as literals (w & m) | E compiles to a v_and_b32 and a
// v_or_b32; held in registers (the empty asm statements hide the values from
// constant folding) it is a single v_and_or_b32.
__device__ __forceinline__ void q4_pairs(uint32_t w, uint32_t q[4]) {
  uint32_t E = 0x64006400u, lo = 0x000F000Fu, hi = 0x00F000F0u;
  __asm__("" : "+v"(E));
  __asm__("" : "+s"(lo));
  __asm__("" : "+s"(hi));
  const f16x2 b_even = {(f16)-1032.0f, (f16)-1032.0f};
  const f16x2 s_odd = {(f16)0.0625f, (f16)0.0625f};
  const f16x2 b_odd = {(f16)-72.0f, (f16)-72.0f};
  const uint32_t w8 = w >> 8;
  const f16x2 a = as_h2((w & lo) | E);   // (n0, n4)
  const f16x2 b = as_h2((w & hi) | E);   // (n1, n5) * 16
  const f16x2 c = as_h2((w8 & lo) | E);  // (n2, n6)
  const f16x2 d = as_h2((w8 & hi) | E);  // (n3, n7) * 16
  q[0] = as_u(a + b_even);
  q[1] = as_u(__builtin_elementwise_fma(b, s_odd, b_odd));
  q[2] = as_u(c + b_even);
  q[3] = as_u(__builtin_elementwise_fma(d, s_odd, b_odd));
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

// Maximum over the 64 lanes, by the same DPP steps as group_sum.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0x128>(v));  // row_ror:8
  v = fmaxf(v, dpp<0x124>(v));  // row_ror:4
  v = fmaxf(v, dpp<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  return fmaxf(v, __shfl_xor(v, 32, 64));
}

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

// One (best, index, second) argmax partial of a workgroup; with the in-kernel
// merge the stores are agent-coherent (written through to the level every
// XCD reads), since the merging workgroup may run on another XCD.
__device__ __forceinline__ void argmax_partial_store(const QmvParams& p, long long o, float v, int i,
                                                     float s) {
  if (p.am_count) {
    __hip_atomic_store(p.part_best + o, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(p.part_index + o, i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(p.part_second + o, s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    p.part_best[o] = v;
    p.part_index[o] = i;
    p.part_second[o] = s;
  }
}

// In-kernel merge of the argmax partials (p.am_count non-null), called by every
// thread of every workgroup after its partial stores.  Each workgroup counts
// in on its group's counter (workgroup b in group b % groups); the last of a
// group counts in on the top counter, and the last of those merges all
// partials of every row with the argmax comparator (the first-maximum rule of
// MM:645-686; the merge order is free) and writes the index and top-2 gap.
// The last arrivals reset the counters, so the launch replays without
// clearing.  The merge result equals argmax_finalize_kernel's.
__device__ __forceinline__ void argmax_tail(const QmvParams& p) {
  if (!p.am_count) return;
  __shared__ int s_last;
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
  __syncthreads();
  const int parts = p.parts;
  if (threadIdx.x == 0) {
    const int groups = parts < kArgGroups ? parts : kArgGroups;
    const int g = blockIdx.x % groups;
    const int members = (parts - 1 - g) / groups + 1;
    int* gc = p.am_count + g * kArgCounterStride;
    int* top = p.am_count + kArgGroups * kArgCounterStride;
    int last = 0;
    if (atomicAdd(gc, 1) == members - 1) {
      atomicExch(gc, 0);
      if (atomicAdd(top, 1) == groups - 1) {
        atomicExch(top, 0);
        last = 1;
      }
    }
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;
  __shared__ float mv[kWaves], ms[kWaves];
  __shared__ int mi[kWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int kBatch = 8;
  for (int m = 0; m < p.m; ++m) {
    const long long base = (long long)(p.m_base + m) * parts;
    float bv = __builtin_nanf("");
    int bi = 0x7fffffff;
    float bs = -INFINITY;
    for (int i0 = threadIdx.x; i0 < parts; i0 += kThreads * kBatch) {
      float v[kBatch], sv[kBatch];
      int ix[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int i = i0 + j * kThreads;
        const bool in = i < parts;
        v[j] = in ? __hip_atomic_load(p.part_best + base + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                  : __builtin_nanf("");
        ix[j] = in ? __hip_atomic_load(p.part_index + base + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                   : 0x7fffffff;
        sv[j] = in ? __hip_atomic_load(p.part_second + base + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                   : -INFINITY;
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) argmax_merge(bv, bi, bs, v[j], ix[j], sv[j]);
    }
    argmax_wave_reduce(bv, bi, bs);
    if (lane == 0) {
      mv[wave] = bv;
      mi[wave] = bi;
      ms[wave] = bs;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int w = 1; w < kWaves; ++w) argmax_merge(bv, bi, bs, mv[w], mi[w], ms[w]);
      p.am_out[p.m_base + m] = bi == 0x7fffffff ? 0 : bi;
      if (p.am_gap) p.am_gap[p.m_base + m] = bs == -INFINITY ? INFINITY : bv - bs;
    }
    __syncthreads();
  }
}

// Rank of workgroup bid among the grid's workgroups such that the ranks of
// one XCD (bid % 8: workgroups are dispatched to the XCDs in turn) are one
// contiguous run: persistent kernels that give workgroup rank r the r-th
// contiguous range of work then keep neighbouring work -- the tiles of one
// copy of a batched launch, and that copy's activation rows -- in one L2.
__device__ __forceinline__ int xcd_rank(int bid, int grid) {
  const int x = bid & 7, j = bid >> 3, q = grid >> 3, r = grid & 7;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + j;
}

// The (tile, item) of a tiled-GEMM workgroup.  Workgroup b is dispatched to
// XCD b % 8; XCD x takes the contiguous tile range [x T / 8, (x + 1) T / 8)
// of the launch's `tiles` tiles, `per` consecutive workgroups per tile (its
// row tiles and K chunks).  Consecutive tiles are the weight tiles of one
// copy of a batched launch (or of one matrix), so a copy's activation tile is
// fetched into one XCD's L2 and re-read there by every weight tile of the
// copy, and a weight tile by every row tile; spreading a copy over the eight
// XCDs would fetch its activations once per XCD through the shared fabric,
// where they compete with the weight stream.  tile < 0: no work (the grid is
// ceil(T / 8) * 8 * per workgroups).
__device__ __forceinline__ void gemm_block_tile(int bid, int tiles, int per, int& tile, int& item) {
  const int x = bid & 7, j = bid >> 3;
  const int t0 = (x * tiles) >> 3, t1 = ((x + 1) * tiles) >> 3;
  const int tl = j / per;
  tile = t0 + tl < t1 ? t0 + tl : -1;
  item = j - tl * per;
}

__device__ __forceinline__ float load_scale(const void* s, long long i, bool f16_scale) {
  return f16_scale ? (float)((const f16*)s)[i] : ((const float*)s)[i];
}

// Fourth dword of a raw buffer resource on gfx9-family parts (32-bit data
// format, no swizzle); loads past num_records return zero.
constexpr int kBufferRsrcWord3 = 0x00020000;
// Cache policy of the streamed weight loads: non-temporal.
constexpr int kStreamAux = 2;

// fp16 or fp32 scale from the aligned dword `dw` loaded at byte offset
// (off & ~3): an fp16 scale is the half selected by bit 1 of the offset.
__device__ __forceinline__ float scale_at(uint32_t dw, int off, bool f16_scale) {
  if (f16_scale) {
    const uint16_t h = (uint16_t)(dw >> ((off & 2) * 8));
    return (float)__builtin_bit_cast(f16, h);
  }
  return __builtin_bit_cast(float, dw);
}

// Raw bits of scale i (fp16 in the low half, or fp32); scale_of() widens them
// exactly (fp16 subnormals included) once the load has landed.
__device__ __forceinline__ uint32_t load_scale_bits(const void* s, long long i, bool f16_scale) {
  return f16_scale ? (uint32_t)((const uint16_t*)s)[i] : ((const uint32_t*)s)[i];
}
__device__ __forceinline__ float scale_of(uint32_t bits, bool f16_scale) {
  return f16_scale ? (float)__builtin_bit_cast(f16, (uint16_t)bits) : __builtin_bit_cast(float, bits);
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

// Element index of output (row, n) of matrix mt: row-major, or the attention
// head-packed layout of MM:1192-1318 -- slice head / 4 of rows x head_dim
// texels, lane head % 4 -- whose row index counts from the tensor's first row
// (the host leaves such an output's pointer at row 0 for every row block).
__device__ __forceinline__ long long out_index(const QmvParams& p, const QmvMat& mt, int row,
                                               int n) {
  if (mt.y_hd == 0) return (long long)row * mt.y_rstride + n;
  const int head = n / mt.y_hd, d = n - head * mt.y_hd;
  return (((long long)(head >> 2) * p.y_rows + p.m_base + row) * mt.y_hd + d) * 4 + (head & 3);
}

// The LM head's epilogue: gemm_epilogue without a C term (the argmax
// launches take none), the same arithmetic.
// The logit an argmax compares: fp16-rounded when the reference's logits
// texture is ARGBHalf (GL:383-396; its argmax reads those values, MM:645-686).
__device__ __forceinline__ float argmax_logit(const QmvParams& p, float v) {
  return (p.flags & kFlagArgF16) ? (float)(f16)v : v;
}

__device__ __forceinline__ float argmax_epilogue(const QmvParams& p, float v) {
  return (p.flags & kFlagAlphaIn) ? p.alpha * (0.0f + v) : 0.0f + p.alpha * v;
}

// The operands of gemm_epilogue, for loops that finish many outputs: taken
// out of the kernel arguments once (epi_args) and held in scalar registers.
struct EpiArgs {
  const __attribute__((address_space(1))) float* c;  // global (not flat) loads
  float alpha, beta;
  int bcast, c_rstride, flags;
};

// Bias, alpha and beta as the reference Gemm resolves them (MM:688-705, 812-820):
// Pack4-linear output is alpha*(beta*C + sum), tiled output beta*C + alpha*sum.
__device__ __forceinline__ float gemm_epilogue(const EpiArgs& e, int m, int r, float v) {
  float bias = 0.0f;
  if (e.c) {
    switch (e.bcast) {
      case 0: bias = e.c[0]; break;
      case 1: bias = e.c[m]; break;
      case 3: bias = e.c[(long long)m * e.c_rstride + r]; break;
      case 4: bias = e.c[r]; break;
      default: bias = 0.0f; break;
    }
    bias *= e.beta;
  }
  return (e.flags & kFlagAlphaIn) ? e.alpha * (bias + v) : bias + e.alpha * v;
}
__device__ __forceinline__ float gemm_epilogue(const QmvParams& p, int m, int r, float v) {
  return gemm_epilogue(EpiArgs{(const __attribute__((address_space(1))) float*)p.c, p.alpha,
                               p.beta, p.bcast, p.c_rstride, p.flags},
                       m, r, v);
}

// A wave-uniform value computed once: the readfirstlane makes it an
// instruction result, so the compiler keeps it in a scalar register instead
// of loading it from the kernel arguments again inside a loop.
__device__ __forceinline__ int sreg(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ float sreg(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}
template <typename T>
__device__ __forceinline__ T* sreg(T* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (T*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ EpiArgs epi_args(const QmvParams& p) {
  return EpiArgs{(const __attribute__((address_space(1))) float*)sreg(p.c), sreg(p.alpha),
                 sreg(p.beta), sreg(p.bcast), sreg(p.c_rstride), sreg(p.flags)};
}

}  // namespace aexq
