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

// DPP broadcast across rows into the rows enabled in ROWS (the others read
// `old`): row_bcast:15 (0x142) gives rows 1 and 3 lane 15 of rows 0 and 2,
// row_bcast:31 (0x143) gives rows 2 and 3 lane 31.
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_rows(float old, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                               __builtin_bit_cast(int, v), CTRL,
                                                               ROWS, 0xF, false));
}
__device__ __forceinline__ float lane_value(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over aligned groups of LPR lanes (16, 32 or 64); every lane of a group
// receives the group total.  Within a 16-lane DPP row: rotate by 8 and 4, then
// quad swaps.  Across rows (no LDS round trip): rows 1 and 3 add lane 15 of
// rows 0 and 2 by row_bcast:15, rows 2 and 3 then add lane 31 by row_bcast:31,
// and the totals are read from lanes 31 and 63.  Lane 63 holds
// (S3 + S2) + (S1 + S0) for row sums S0..S3, the same value (addition
// commutes) as the pairwise (S0 + S1) + (S2 + S3) of a butterfly.  Needs every
// lane active, like the row steps.
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp<0x128>(v);  // row_ror:8
  v += dpp<0x124>(v);  // row_ror:4
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  if constexpr (LPR >= 32) {
    v += dpp_rows<0x142, 0xA>(0.0f, v);  // rows 1, 3: S1 + S0, S3 + S2
    if constexpr (LPR == 32) {
      const float lo = lane_value(v, 31), hi = lane_value(v, 63);
      return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)) < 32 ? lo : hi;
    } else {
      v += dpp_rows<0x143, 0xC>(0.0f, v);  // row 3: (S3 + S2) + (S1 + S0)
      return lane_value(v, 63);
    }
  }
  return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

// Maximum over the 64 lanes, by the same DPP steps as group_sum.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0x128>(v));  // row_ror:8
  v = fmaxf(v, dpp<0x124>(v));  // row_ror:4
  v = fmaxf(v, dpp<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_rows<0x142, 0xA>(v, v));
  v = fmaxf(v, dpp_rows<0x143, 0xC>(v, v));
  return lane_value(v, 63);
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

// The tag of this launch's argmax partials (in-kernel merge): the epoch the
// previous merging launch left, plus one, never 0 (the words of a scratch
// buffer start at tag 0).  Every workgroup reads it before its partial store;
// the merging workgroup stores it back only after every partial of the launch
// carries it, so the whole grid reads the same value.  An agent-coherent
// load: the previous launch's last workgroup, on any XCD, stored the word, and
// another XCD's L2 may still hold the line from an earlier read.
__device__ __forceinline__ uint32_t argmax_tag(const QmvParams& p) {
  if (!p.am_tagged) return 0;
  const uint32_t e = __hip_atomic_load(p.am_epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return e == 0xffffffffu ? 1u : e + 1u;
}

// One (best, index, second) argmax partial of a workgroup: three tagged
// 64-bit words, each stored whole and agent-coherent (written through to the
// level every XCD reads, since the merging workgroup may run on another XCD);
// no fence and no arrival count.
__device__ __forceinline__ void argmax_partial_store(const QmvParams& p, long long o, float v, int i,
                                                     float s, uint32_t tag) {
  const unsigned long long t = (unsigned long long)tag << 32;
  __hip_atomic_store(p.am_tagged + o, t | __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(p.am_tagged + p.am_plane + o, t | (uint32_t)i, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(p.am_tagged + 2 * p.am_plane + o, t | __float_as_uint(s), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// Order-preserving map of a non-NaN float to an unsigned integer (-0 taken as
// +0, which the argmax compares equal), and its inverse; the inverse of
// 0xffffffff is a NaN.
__device__ __forceinline__ uint32_t argmax_ord(float f) {
  const uint32_t u = __float_as_uint(f == 0.0f ? 0.0f : f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float argmax_unord(uint32_t u) {
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}

// Top-2 of packed argmax keys: insert a key into (k1 >= k2), and combine two
// such pairs.  Every key but the largest reaches k2 (inserted directly, or
// pushed down by a larger one), and k2 never exceeds the second-largest.
__device__ __forceinline__ void argmax_top2_insert(unsigned long long& k1, unsigned long long& k2,
                                                   unsigned long long key) {
  const unsigned long long lo = k1 < key ? k1 : key;
  k1 = k1 < key ? key : k1;
  k2 = k2 < lo ? lo : k2;
}
__device__ __forceinline__ void argmax_top2_combine(unsigned long long& k1, unsigned long long& k2,
                                                    uint32_t& ks, unsigned long long o1,
                                                    unsigned long long o2, uint32_t os) {
  argmax_top2_insert(k1, k2, o1);
  k2 = k2 < o2 ? o2 : k2;
  ks = ks < os ? os : ks;
}

// Polls n tagged partials from entry e0 of the first plane at `base` (the
// other two planes `plane` words on), thread gl of a row's gsz threads taking
// entries gl, gl + gsz, ...; folds each into (k1, k2, ks).  False: a wait ran
// out.  Addresses are a uniform base plus 32-bit byte offsets (every plane
// holds fewer than 2^29 words), one register per load rather than a pointer
// pair, which keeps the poll within the kernel's register budget.
template <int kB>
__device__ __forceinline__ bool argmax_poll(const unsigned long long* base, long long plane,
                                            long long e0, int n, int gl, int gsz, uint32_t tag,
                                            unsigned long long& k1, unsigned long long& k2,
                                            uint32_t& ks) {
  const char* b0 = (const char*)base;
  const uint32_t o0 = (uint32_t)(e0 * 8), pb = (uint32_t)(plane * 8);
  auto word = [&](int e, int q) {
    return __hip_atomic_load((const unsigned long long*)(b0 + (o0 + (uint32_t)e * 8u + q * pb)),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  for (int i0 = gl; i0 < n; i0 += gsz * kB) {
    unsigned long long a[kB], b[kB], c[kB];
    bool ok[kB];
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      const int e = i0 + j * gsz;
      ok[j] = e >= n;
      if (!ok[j]) {
        a[j] = word(e, 0);
        b[j] = word(e, 1);
        c[j] = word(e, 2);
      }
    }
    for (int spin = 0;; ++spin) {
      bool all = true;
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        if (!ok[j]) {
          ok[j] = (uint32_t)(a[j] >> 32) == tag && (uint32_t)(b[j] >> 32) == tag &&
                  (uint32_t)(c[j] >> 32) == tag;
          all = all && ok[j];
        }
      }
      if (all) break;
      if (spin >= kArgSpinLimit) return false;
      __builtin_amdgcn_s_sleep(2);
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        const int e = i0 + j * gsz;
        if (!ok[j]) {
          a[j] = word(e, 0);
          b[j] = word(e, 1);
          c[j] = word(e, 2);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      if (i0 + j * gsz < n) {
        const float v = __uint_as_float((uint32_t)a[j]);
        const float sv = __uint_as_float((uint32_t)c[j]);
        const uint32_t ix = (uint32_t)b[j];
        if (!__builtin_isnan(sv)) {
          const uint32_t o = argmax_ord(sv);
          ks = ks < o ? o : ks;
        }
        if (!__builtin_isnan(v))
          argmax_top2_insert(k1, k2, ((unsigned long long)argmax_ord(v) << 32) | (uint32_t)~ix);
        else if (ix == 0)
          argmax_top2_insert(k1, k2, ~0ull);
      }
    }
  }
  return true;
}

// In-kernel merge of the argmax partials (p.am_tagged non-null), called by
// every thread of every workgroup after its partial stores; only the grid's
// last workgroup works, and with p.am_group = g > 0 the last workgroup of each
// full run of G = 2^g as well.  A merging workgroup waits only on partials of
// workgroups with lower indices, dispatched before it; those finish or wait
// in turn only on lower indices, so every wait ends.  (Should dispatch order
// differ across XCDs, a waiting run merger holds one slot, and the host keeps
// the run mergers fewer than one XCD's resident slots.)  Two levels keep the
// merge at one poll round per level when the grid queues thousands of
// workgroups: a run merger folds its G partials into a group partial of the
// same three-word form while the rest of the grid still streams.
//
// Its threads split into one group per row (a power of two, 256 / rows or
// less); a thread polls its share of the row's partials (agent-coherent loads,
// kB partials in flight -- 8 in the register-tight streaming kernel, 16 in
// the MFMA one --, a pause between polls, at most kArgSpinLimit
// polls) and folds each partial whose three words carry the tag into its own
//   k1, k2 = the two largest keys, key = ord(best) << 32 | ~index (a larger
//            value wins, then the lower index; a NaN at index 0 takes the
//            largest key, any other NaN none): k1 is the first-maximum rule of
//            MM:645-686 whatever the order the partials arrive in;
//   ks     = the largest second value.
// The group combines them by lane shuffles (then through LDS across waves).
// The top-2 gap is best - max(ks, value of k2): the best of all candidates but
// the winner, as the sequential scan forms it.  A wait that runs out writes
// index -1 and a NaN gap for every row.  Then the tag becomes the next
// launch's epoch.  A run merger whose wait runs out stores no group partial,
// so the grid's last workgroup runs out too and reports the failure.
template <int kB>
__device__ __forceinline__ void argmax_tail(const QmvParams& p, uint32_t tag) {
  if (!p.am_tagged) return;
  const int parts = p.parts, gs = p.am_group, G = gs > 0 ? 1 << gs : 0;
  const bool last = blockIdx.x == gridDim.x - 1;
  if (!last && (gs <= 0 || ((int)blockIdx.x & (G - 1)) != G - 1)) return;
  __shared__ unsigned long long s_k1[kArgMergeRows], s_k2[kArgMergeRows];
  __shared__ uint32_t s_ks[kArgMergeRows];
  __shared__ int s_fail;
  const int rows = p.m;  // <= kArgMergeRows (host-checked)
  // full runs before the last workgroup's; their group partials follow the
  // grid's partials in each row (parts = grid + groups words a row), so the
  // last workgroup's run and the group partials are one range
  const int groups = gs > 0 ? ((int)gridDim.x - 1) >> gs : 0;
  int gsz = kThreads;  // threads per row
  while (gsz > 8 && gsz * rows > kThreads) gsz >>= 1;
  const int r = (int)threadIdx.x / gsz, gl = (int)threadIdx.x % gsz;
  if (threadIdx.x == 0) s_fail = 0;
  __syncthreads();
  unsigned long long k1 = 0ull, k2 = 0ull;
  uint32_t ks = argmax_ord(-INFINITY);
  bool fail = false;
  if (r < rows) {
    const long long row = p.m_base + r;
    // this workgroup's run: every partial, the last run with the group
    // partials, or a full run (run merging needs partial i to be workgroup i's)
    const int first = last ? groups * (G > 0 ? G : 0) : (int)blockIdx.x - (G - 1);
    fail = !argmax_poll<kB>(p.am_tagged, p.am_plane, row * parts + first,
                            last ? parts - first : G, gl, gsz, tag, k1, k2, ks);
  }
  // combine within each group (aligned lanes of one wave), then per wave
  const int span = gsz < 64 ? gsz : 64;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    if (off < span) {
      const unsigned long long o1 = __shfl_xor(k1, off, 64), o2 = __shfl_xor(k2, off, 64);
      const uint32_t os = __shfl_xor(ks, off, 64);
      argmax_top2_combine(k1, k2, ks, o1, o2, os);
    }
  }
  if (fail) s_fail = 1;  // benign race: every writer stores 1
  // the leader of each group, or of each wave of a group wider than a wave
  const int slot = (int)threadIdx.x / span;
  if ((int)threadIdx.x % span == 0 && r < rows) {
    s_k1[slot] = k1;
    s_k2[slot] = k2;
    s_ks[slot] = ks;
  }
  __syncthreads();
  if ((int)threadIdx.x < rows) {
    const int per = gsz / span;  // slots of one row
    const int q0 = (int)threadIdx.x * per;
    unsigned long long b1 = s_k1[q0], b2 = s_k2[q0];
    uint32_t bks = s_ks[q0];
    for (int q = 1; q < per; ++q)
      argmax_top2_combine(b1, b2, bks, s_k1[q0 + q], s_k2[q0 + q], s_ks[q0 + q]);
    const float bv = b1 ? argmax_unord((uint32_t)(b1 >> 32)) : __builtin_nanf("");
    const int bi = b1 ? (int)~(uint32_t)b1 : 0;
    float bs = argmax_unord(bks);
    if (b2) bs = fmaxf(bs, argmax_unord((uint32_t)(b2 >> 32)));
    const bool bad = s_fail != 0;
    if (!last) {
      // the run's group partial (an empty run: NaN at index 0x7fffffff, which
      // never wins; a NaN at index 0 keeps index 0)
      if (!bad)
        argmax_partial_store(p, (long long)(p.m_base + threadIdx.x) * parts + (int)gridDim.x +
                                    ((int)blockIdx.x >> gs),
                             bv, b1 ? bi : 0x7fffffff, bs, tag);
    } else {
      p.am_out[p.m_base + threadIdx.x] = bad ? -1 : bi;
      if (p.am_gap)
        p.am_gap[p.m_base + threadIdx.x] =
            bad ? __builtin_nanf("") : (bs == -INFINITY ? INFINITY : bv - bs);
    }
  }
  if (last && threadIdx.x == 0)
    __hip_atomic_store(p.am_epoch, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
