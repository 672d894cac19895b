// The decoder layers of one decode step as one persistent launch (gfx950).
//
// Reference: Qwen35DecoderSession.DecodeCore (DEC:463-585) runs every layer as
// a chain of separate dispatches (RMSNorm, Gemm, RoPE, SDPA, Gemm + residual,
// RMSNorm, Gemm pair + SwiGLU, Gemm + residual; per-layer loop LF:996-1136).
// At M = 1 each of those moves 0.3-4 MB, so a chain of kernel launches is
// bound by launch and round-trip latency, not by HBM.  Here a grid of G
// co-resident workgroups walks all layers in one launch.  Each layer is six
// phases:
//
//   P1  q/k/v                        rows of [Wq; Wk; Wv] split over the grid
//   P2a attention splits             workgroup (kv head g, split s) of `sp`
//                                    positions: scores, softmax statistics,
//                                    P.V partials
//   P2b split merge                  (q head, slice of dims) per workgroup, on
//                                    the two poll waves (half of the dims each),
//                                    which also store the merged slice
//   P3  o_proj + residual            rows of Wo
//   P4  gate/up + SwiGLU             rows of the gate/up pair
//   P5  down + residual              rows of Wdown
//
// Phases hand their outputs over in device memory as tagged 32-bit words: a
// vector element is (16-bit tag << 16 | fp16 bits), an attention partial is
// an fp32 whose low 8 mantissa bits hold an 8-bit tag.  The tag is the
// phase's epoch (a device counter advanced by 6 x layers per launch), so a
// consumer polls the data itself with agent-coherent loads until every word
// it needs carries the current epoch: one store-to-load round trip per
// phase, with no separate barrier.  Every word of every exchange buffer is
// rewritten in every layer, so a stale word is at most a few epochs old and
// never carries the current tag.  Each phase reads all of its predecessor's
// outputs, or (P2a, P2b) those of its kv head, so a buffer is never
// rewritten while a slower workgroup still reads it.  The vectors that every
// workgroup polls (q/k/v, the merged attention, x after attention, the SwiGLU
// output, the layer output) are written in kStepReplicas copies on separate
// 4 KB pages and workgroup b polls copy b % kStepReplicas: a grid polling one
// 4-14 KB vector otherwise meets on the few memory channels holding it, and
// its polls delay the producers' stores there.  Spins are bounded: a
// wait that exceeds kSpinLimit sets the error word and gives up (the launch
// still ends; the host reports the error).
//
// A workgroup is 9 compute waves, one store wave and two poll waves.  While
// the compute waves run phase p, the poll waves wait for phase p's outputs of
// the whole grid (the inputs of phase p + 1) and leave them in LDS, ready at
// the next workgroup barrier; they also do the work between a poll and the
// next linear: the RMSNorm-in (for layer 0's input, in the prologue, bit-exact
// with the streaming kernel's staged path; for every later one, gamma x in
// fp16 before the barrier and 1 / rms after it, which the compute waves apply
// to each row's sum), RoPE of q and the new k row, the split merge and the
// RMSNorm gammas.  The compute waves load
// each phase's weights (and the split's cached K/V rows) one to three phases
// ahead into registers, issuing them at the start of a phase so that the
// grid-wide burst drains while they compute, before the phase's outputs are
// handed over, and leave their outputs in LDS; the store wave writes
// them (and the K/V append) to device memory.  On this part loads and stores
// share one vector-memory counter, which counts in issue order and, once both
// kinds are in flight, makes any wait a wait for everything: so the compute
// waves issue only loads (a use of a register loaded two phases ago waits for
// exactly that load) and the store wave only stores.  The poll waves load,
// and the merging one also stores its merged slice: its next wait is for its
// next poll, which waits for everything before it in any case.
//
// The layer weights are Q4 with one scale per 32 codes (the benchmark's
// format), Q4 with one per 16 (the reference's shipping archives, Q8A:116-139)
// or Q8 with one scale per row (Q8A:94-114), scales fp16 or fp32; the format
// is a template parameter of the kernel.  Arithmetic of the linears follows
// the streaming kernel (aexq_qmv.hpp) for the same format: the same RMSNorm-in
// (sums of squares over 8-element slices, DPP wave sums, four partials in
// order; fp16(x * inv * gamma)), the same per-chunk dot-product order and
// group-scale fmaf, the same DPP row reduction and epilogue.  q/k/v, gate/up
// and down use the streaming kernel's lanes per row and chunks per lane, so
// layer 0's q/k/v outputs are bit-identical to those of aexq_linear at M = 1;
// o_proj takes 64 lanes per row (one row per wave, eight waves busy instead of
// four at half the chunks per lane), so its sums are grouped differently; and
// after layer 0 the RMSNorm-in's 1 / rms multiplies each row's sum of
// W (fp16(gamma x)) rather than each element before its fp16 rounding, the
// same product rounded differently, so the barrier before a linear does not
// wait for the vector's sum of squares.  Attention
// follows MM:420-544 (scale, max-subtracted softmax, sum floored at 1e-20)
// with positions split over workgroups and waves.
#include <math.h>

#include "aexq_device.hpp"
#include "aexq_step.hpp"

namespace aexq {

// Phase timing (built only with -DAEXQ_STEP_STAMPS, the instrumented library
// bench.py --decode-phases loads): the store wave of every workgroup records
// s_memrealtime (100 MHz) when its compute waves have finished a phase and
// again after the phase's workgroup barrier, 10 stamps per layer, into
// g_step_stamps[(layer * 10 + k) * grid + workgroup] (layers < 64, grid <= 256);
// aexq_step_stamps copies them out.  The store wave only stores, so the stamps
// add no wait to any role.
#ifdef AEXQ_STEP_STAMPS
__device__ unsigned long long g_step_stamps[64 * 10 * 256];
#define AEXQ_STAMP(l, k, lane, b)                                                          \
  if ((lane) == 0 && (l) < 64)                                                             \
  g_step_stamps[((l) * 10 + (k)) * gridDim.x + (b)] = __builtin_amdgcn_s_memrealtime()
#else
#define AEXQ_STAMP(l, k, lane, b) ((void)0)
#endif

namespace {

constexpr int kSt = kStepThreads;
constexpr int kStW = kSt / 64;
constexpr int kCW = kStepComputeWaves;  // compute waves 0 .. kCW - 1
constexpr int kSW = kCW;                // the store wave
constexpr int kPW = kStW - kCW - 1;     // poll waves kCW + 1 ..
static_assert(kPW == 2, "two poll waves");
constexpr int kHd = kStepHeadDim;
constexpr int kHalf = kHd / 2;
constexpr int kAP = kStepMaxSplitPos;   // positions of an attention workgroup
constexpr int kAW = kAP / 8;            // attention waves: 8 positions each
static_assert(kAW <= kCW, "attention waves are compute waves");
constexpr int kSpinLimit = 1 << 15;
constexpr int kCoh = 16;  // buffer-load cache policy sc1: read at agent coherence
constexpr int kNoOff = 0x7ffffff0;

__device__ __forceinline__ void st_word(uint32_t* p, uint32_t w) {
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16 bytes of tagged words at byte offset `off` of the buffer `rs`, written
// with the same agent coherence as st_word; every word carries its own tag, so
// a reader never needs the four words to land together.
__device__ __forceinline__ void st_quad(__amdgpu_buffer_rsrc_t rs, int off, const u32x4& v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, rs, off, 0, kCoh);
}
__device__ __forceinline__ uint32_t ld_word(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t h_bits(f16 v) { return (uint32_t)__builtin_bit_cast(uint16_t, v); }
__device__ __forceinline__ uint32_t tag_f16(f16 v, uint32_t tag) {
  return ((tag & 0xffffu) << 16) | h_bits(v);
}
// fp32 carrying an 8-bit tag in its low mantissa bits; trunc_f32 is the value
// a reader recovers (the writer uses the same value where it matters)
__device__ __forceinline__ float trunc_f32(float v) { return as_f32(f32_bits(v) & ~0xffu); }
__device__ __forceinline__ uint32_t tag_f32(float v, uint32_t tag) {
  return (f32_bits(v) & ~0xffu) | (tag & 0xffu);
}
// a finite stand-in for -inf: an exp() against any live maximum gives 0, and
// it survives the tag bits
constexpr float kNegBig = -3.0e38f;

template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// The thread index, hidden from the optimizer: per-lane offsets derived from it
// are recomputed in each phase instead of being hoisted out of the layer loop
// and held in registers across all of it.
__device__ __forceinline__ int opaque_tid() {
  int t = threadIdx.x;
  __asm__ volatile("" : "+v"(t));
  return t;
}
// The compute waves' thread index.  Q4: the plain index, so the per-lane
// offsets of every prefetch are computed once and held across the layer loop
// (the kernels then take 157-165 VGPRs): each phase's loads issue without
// their address arithmetic, which is what delays a wave's start on its dot
// products.  Q8: hidden, since its twice-wider weight registers leave no room
// for the offsets (they would spill).
template <int FMT>
__device__ __forceinline__ int cw_tid() {
  return FMT == kQ8 ? opaque_tid() : (int)threadIdx.x;
}

// A pointer of the layer table staged in LDS, made wave-uniform (SGPRs): the
// buffer resources built from it need no waterfall loop, and reading it
// waits on LDS, never behind the vector-memory loads and stores in flight.
template <typename T>
__device__ __forceinline__ T* lds_ptr(T* const* slot) {
  const unsigned long long v = *(const unsigned long long*)slot;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (T*)(((unsigned long long)hi << 32) | lo);
}

// Poll wave: waits until the NV 16-byte groups at word offsets off[i] of src
// (off[i] < 0: none) carry `tag` in every word (tag bits: (w >> shift) & mask).
template <int NV>
__device__ __forceinline__ void pw_wait(const uint32_t* src, int words, const int (&off)[NV],
                                        uint32_t tag, int shift, uint32_t mask, u32x4 (&v)[NV],
                                        int* err, bool& broken) {
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, words * 4, kBufferRsrcWord3);
  tag &= mask;
  for (int spin = 0;; ++spin) {
#pragma unroll
    for (int i = 0; i < NV; ++i)
      v[i] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off[i] >= 0 ? off[i] * 4 : kNoOff, 0, kCoh));
    bool ok = true;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) ok = ok && (off[i] < 0 || ((v[i][e] >> shift) & mask) == tag);
    if (ok || broken) break;
    if (spin >= kSpinLimit) {
      atomicOr(err, 1);
      broken = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// fp16 halves of four tagged words, as two dwords (x0, x1), (x2, x3).
__device__ __forceinline__ void halves(const u32x4& v, uint32_t& a, uint32_t& b) {
  a = __builtin_amdgcn_perm(v[1], v[0], 0x05040100u);
  b = __builtin_amdgcn_perm(v[3], v[2], 0x05040100u);
}

// Poll wave pw of kPW: its share of a tagged fp16 vector of `count` words
// (count % 8 == 0, count <= 256 * NV * kPW) into dst in the order row_dot
// consumes: the nibble-pair order of q4_xpairs per 8 elements for Q4 weights
// (PAIRS), plain for Q8.
template <int NV, bool PAIRS>
__device__ __forceinline__ void pw_vec_pairs(const uint32_t* src, int count, uint32_t tag, f16* dst,
                                             int lane, int pw, int* err, bool& broken) {
  static_assert(NV % 2 == 0, "two groups per 8 elements");
  int off[NV];
#pragma unroll
  for (int i = 0; i < NV / 2; ++i) {
    const int w0 = (lane + 64 * (pw + kPW * i)) * 8;
    off[2 * i] = w0 < count ? w0 : -1;
    off[2 * i + 1] = w0 < count ? w0 + 4 : -1;
  }
  u32x4 v[NV];
  pw_wait<NV>(src, count, off, tag, 16, 0xffffu, v, err, broken);
#pragma unroll
  for (int i = 0; i < NV / 2; ++i)
    if (off[2 * i] >= 0) {
      uint32_t a, b, c, d, xp[4];
      halves(v[2 * i], a, b);
      halves(v[2 * i + 1], c, d);
      if constexpr (PAIRS) {
        q4_xpairs(a, b, c, d, xp);
      } else {
        xp[0] = a;
        xp[1] = b;
        xp[2] = c;
        xp[3] = d;
      }
      *(u32x4*)(dst + off[2 * i]) = u32x4{xp[0], xp[1], xp[2], xp[3]};
    }
}

// Poll wave: RMSNorm-in of the fp16 row x (LDS, plain, k <= 2048) into out
// (LDS, nibble-pair order for Q4 weights, plain for Q8), bit-exact with the
// streaming kernel's staged path
// (Qmv::stage_finish): that path's 256 threads each own the 8-element slice
// vt * 8 and their sums of squares meet as four wave sums added in order;
// lane l here stands in for threads l, l + 64, l + 128, l + 192.  Each element
// is rounded once as fp16(x * inv * gamma[i]).
template <bool PAIRS>
__device__ __forceinline__ void pw_rms(const f16* x, const float* gamma, f16* out, int k, float eps,
                                       int lane) {
  u32x4 xv[4];
  float part[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int e0 = (lane + 64 * v) * 8;
    xv[v] = e0 < k ? *(const u32x4*)(x + e0) : u32x4{0u, 0u, 0u, 0u};
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const f16x2 h = as_h2(xv[v][e]);
      const float a = (float)h[0], b = (float)h[1];
      ss = fmaf(a, a, ss);
      ss = fmaf(b, b, ss);
    }
    part[v] = wave_sum(ss);
  }
  float tot = 0.0f;
#pragma unroll
  for (int v = 0; v < 4; ++v) tot += part[v];
  const float inv = rsqrtf(fmaxf(tot / (float)k + eps, 1e-20f));
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int e0 = (lane + 64 * v) * 8;
    if (e0 < k) {
      const f32x4 g0 = *(const f32x4*)(gamma + e0);
      const f32x4 g1 = *(const f32x4*)(gamma + e0 + 4);
      const float g[8] = {g0[0], g0[1], g0[2], g0[3], g1[0], g1[1], g1[2], g1[3]};
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f16x2 h = as_h2(xv[v][e]);
        const float a = (float)h[0] * inv, b = (float)h[1] * inv;
        const f16x2 r = {(f16)(a * g[2 * e]), (f16)(b * g[2 * e + 1])};
        o[e] = as_u(r);
      }
      uint32_t xp[4];
      if constexpr (PAIRS) {
        q4_xpairs(o[0], o[1], o[2], o[3], xp);
      } else {
        xp[0] = o[0];
        xp[1] = o[1];
        xp[2] = o[2];
        xp[3] = o[3];
      }
      *(u32x4*)(out + e0) = u32x4{xp[0], xp[1], xp[2], xp[3]};
    }
  }
}

// Both poll waves: the tagged fp16 vector x of k <= 1024 words at src into
// plain (LDS, plain order) and fp16(x * gamma) into out (LDS, nibble-pair
// order for Q4 weights): the RMSNorm-in without its 1 / rms factor, which the
// compute waves apply to each row's sum (y = W (gamma x) / rms(x)) once
// pw_inv_publish has formed it, so the workgroup barrier does not wait for
// the sum of squares.  Wave pw takes the 8-element slices (lane + 64 v) of
// v = pw and pw + 2 and keeps them in xv for pw_inv_publish.
template <bool PAIRS>
__device__ __forceinline__ void pw_vec_gx(const uint32_t* src, int k, uint32_t tag, f16* plain,
                                          const float* gamma, f16* out, int lane, int pw,
                                          u32x4 (&xv)[2], int* err, bool& broken) {
  int off[4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int e0 = (lane + 64 * (pw + 2 * j)) * 8;
    off[2 * j] = e0 < k ? e0 : -1;
    off[2 * j + 1] = e0 < k ? e0 + 4 : -1;
  }
  u32x4 t[4];
  pw_wait<4>(src, k, off, tag, 16, 0xffffu, t, err, broken);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    xv[j] = u32x4{0u, 0u, 0u, 0u};
    const int e0 = off[2 * j];
    if (e0 >= 0) {
      uint32_t a, b, c, d;
      halves(t[2 * j], a, b);
      halves(t[2 * j + 1], c, d);
      xv[j] = u32x4{a, b, c, d};
      *(u32x4*)(plain + e0) = xv[j];
      const f32x4 g0 = *(const f32x4*)(gamma + e0);
      const f32x4 g1 = *(const f32x4*)(gamma + e0 + 4);
      const float g[8] = {g0[0], g0[1], g0[2], g0[3], g1[0], g1[1], g1[2], g1[3]};
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f16x2 h = as_h2(xv[j][e]);
        const f16x2 r = {(f16)((float)h[0] * g[2 * e]), (f16)((float)h[1] * g[2 * e + 1])};
        o[e] = as_u(r);
      }
      uint32_t xp[4];
      if constexpr (PAIRS) {
        q4_xpairs(o[0], o[1], o[2], o[3], xp);
      } else {
        xp[0] = o[0];
        xp[1] = o[1];
        xp[2] = o[2];
        xp[3] = o[3];
      }
      *(u32x4*)(out + e0) = u32x4{xp[0], xp[1], xp[2], xp[3]};
    }
  }
}

// Both poll waves, after the workgroup barrier that released the compute
// waves: 1 / rms of the vector pw_vec_gx left in xv, with pw_rms's arithmetic
// (sums of squares over 8-element slices, four wave sums meeting in s_part and
// added in order), into *inv; *done advances by one once it is there.
// `count` is the LDS counter the two waves meet on (target advances by 2).
__device__ __forceinline__ void pw_inv_publish(const u32x4 (&xv)[2], int k, float eps, int lane,
                                               int pw, float* s_part, int* count, int& target,
                                               float* inv, int* done, int* err, bool& broken) {
  float part[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const f16x2 h = as_h2(xv[j][e]);
      const float a = (float)h[0], b = (float)h[1];
      ss = fmaf(a, a, ss);
      ss = fmaf(b, b, ss);
    }
    part[j] = wave_sum(ss);
  }
  if (lane == 0) {
    s_part[pw] = part[0];
    s_part[pw + 2] = part[1];
  }
  target += 2;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  if (lane == 0) __hip_atomic_fetch_add(count, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  for (int spin = 0;; ++spin) {
    if (__hip_atomic_load(count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target || broken)
      break;
    if (spin >= kSpinLimit) {
      atomicOr(err, 1);
      broken = true;
      break;
    }
    __builtin_amdgcn_s_sleep(0);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  if (pw == 0) {
    float tot = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) tot += s_part[v];
    if (lane == 0) *inv = rsqrtf(fmaxf(tot / (float)k + eps, 1e-20f));
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (lane == 0) __hip_atomic_fetch_add(done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
}

// Poll wave: fp32 gamma[k] (k <= 1024) into registers, 16 values per lane
// (a null gamma loads zeros).
__device__ __forceinline__ void pw_gamma_issue(const float* gamma, int k, f32x4 (&g)[4], int lane) {
  const __amdgpu_buffer_rsrc_t gr =
      __builtin_amdgcn_make_buffer_rsrc((void*)gamma, (short)0, gamma ? k * 4 : 0, kBufferRsrcWord3);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    g[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(gr, (lane * 16 + 4 * i) * 4, 0, 0));
}
__device__ __forceinline__ void pw_gamma_store(const f32x4 (&g)[4], float* dst, int k, int lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (lane * 16 + 4 * i < k) *(f32x4*)(dst + lane * 16 + 4 * i) = g[i];
}

// Barrier of the compute waves only (the poll wave may be polling): an LDS
// counter every compute wave adds to and waits on; bounded like the polls.
__device__ __forceinline__ void cbar(int* ctr, int& target, int lane, int* err, bool& broken) {
  target += kCW;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  if (lane == 0) __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  for (int spin = 0;; ++spin) {
    if (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target || broken)
      break;
    if (spin >= kSpinLimit) {
      atomicOr(err, 1);
      broken = true;
      break;
    }
    __builtin_amdgcn_s_sleep(0);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Compute waves: the 1 / rms pw_inv_publish forms for this phase's input,
// once *done has reached target (bounded like the other waits).
__device__ __forceinline__ float cw_inv(const float* inv, int* done, int target, int* err,
                                        bool& broken) {
  for (int spin = 0;; ++spin) {
    if (__hip_atomic_load(done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target || broken)
      break;
    if (spin >= kSpinLimit) {
      atomicOr(err, 1);
      broken = true;
      break;
    }
    __builtin_amdgcn_s_sleep(0);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  return *inv;
}

// Compute waves: this wave's writes to s_out are done.
__device__ __forceinline__ void cw_signal(int* ctr, int lane) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  if (lane == 0) __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Store wave: waits until every compute wave has signalled this phase.
__device__ __forceinline__ void sw_wait(int* ctr, int& target, int* err, bool& broken) {
  target += kCW;
  for (int spin = 0;; ++spin) {
    if (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target || broken)
      break;
    if (spin >= kSpinLimit) {
      atomicOr(err, 1);
      broken = true;
      break;
    }
    __builtin_amdgcn_s_sleep(0);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}
// The store wave's lanes over (copy, word) pairs of a replicated vector for a
// workgroup's n <= 64 words of one phase: a store instruction covers 64 / n
// copies.  Computed once per launch (it divides).
struct RepLanes {
  int copy;  // the lane's first copy
  int word;  // the lane's word (64: none)
  int step;  // copies per store instruction
};
__device__ __forceinline__ RepLanes rep_lanes(int n, int lane) {
  RepLanes m;
  m.step = 64 / n;
  m.copy = lane / n;
  m.word = m.copy < m.step ? lane - m.copy * n : 64;
  return m;
}
// Store wave: n tagged words from LDS into every copy of a replicated vector
// (`copies` copies, `stride` words apart).
__device__ __forceinline__ void sw_copy_rep(uint32_t* dst, int stride, const uint32_t* src, int n,
                                            const RepLanes& m, int copies = kStepReplicas) {
  if (m.word < n) {
    const uint32_t v = src[m.word];
    for (int r = m.copy; r < copies; r += m.step) st_word(dst + r * stride + m.word, v);
  }
}

// Scale words a lane holds per row slot: one per row (Q8), one per 32-code
// chunk (Q4, groups of 32) or two (Q4, groups of 16).
template <int FMT, int GM, int CPL>
constexpr int slot_scales() {
  return FMT == kQ8 ? 1 : (GM == kG16 ? 2 * CPL : CPL);
}
// Scales per row of a matrix with `chunks` code chunks per row.
template <int FMT, int GM>
__device__ __forceinline__ int row_scales(int chunks) {
  return FMT == kQ8 ? 1 : (GM == kG16 ? 2 * chunks : chunks);
}

// Prefetched codes and scale words of one row slot (NW = 2: a gate/up pair).
template <int FMT, int GM, int CPL, int NW>
struct Slot {
  u32x4 w[NW][CPL];
  uint32_t s[NW][slot_scales<FMT, GM, CPL>()];
};

// Issues one wave's slot loads: rows r0 + slot of a matrix of n rows and
// `chunks` 16-byte code chunks per row (32 Q4 or 16 Q8 codes each).  Rows
// past n, chunks past K and a dead wave (live false) read zeros without
// traffic.
template <int LPR, int CPL, int NW, int FMT, int GM>
__device__ __forceinline__ void issue_slot(Slot<FMT, GM, CPL, NW>& sl, const uint32_t* w0,
                                           const void* s0, const uint32_t* w1, const void* s1,
                                           int n, int r0, int chunks, bool sf16, bool live,
                                           int t) {
  const int lane = t & 63, sub = lane % LPR, slot = lane / LPR;
  const int row_bytes = chunks * 16;
  const int rows = live && n > r0 ? n - r0 : 0;
  const int sb = sf16 ? 2 : 4;
  const int spr = row_scales<FMT, GM>(chunks);
  const int sbytes = live ? (n * spr * sb + 3) & ~3 : 0;
#pragma unroll
  for (int h = 0; h < NW; ++h) {
    const char* wb = (const char*)(h ? w1 : w0) + (long long)(live ? r0 : 0) * row_bytes;
    const __amdgpu_buffer_rsrc_t wr =
        __builtin_amdgcn_make_buffer_rsrc((void*)wb, (short)0, rows * row_bytes, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t sr =
        __builtin_amdgcn_make_buffer_rsrc((void*)(h ? s1 : s0), (short)0, sbytes, kBufferRsrcWord3);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ci = sub + c * LPR;
      const int off = ci < chunks ? slot * row_bytes + ci * 16 : kNoOff;
      sl.w[h][c] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, kStreamAux));
    }
    if constexpr (FMT == kQ8) {
      sl.s[h][0] = __builtin_amdgcn_raw_buffer_load_b32(sr, ((r0 + slot) * sb) & ~3, 0, 0);
    } else {
      constexpr int SPC = GM == kG16 ? 2 : 1;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int ci = sub + c * LPR;
#pragma unroll
        for (int g = 0; g < SPC; ++g) {
          const int soff = ci < chunks ? ((r0 + slot) * spr + SPC * ci + g) * sb : kNoOff;
          sl.s[h][SPC * c + g] = __builtin_amdgcn_raw_buffer_load_b32(sr, soff & ~3, 0, 0);
        }
      }
    }
  }
}

// Dot product of one row slot with the fp16 activation row in LDS (stored in
// the nibble-pair order of q4_xpairs per 8 elements for Q4, plain for Q8), in
// the streaming kernel's order for the format (Qmv::compute: Q4 group partial
// sums scaled into the accumulator, one or two groups per 32-code chunk; Q8
// the whole row, scaled once after the reduction), reduced over the slot's
// LPR lanes.  Every lane of the slot returns the row's sum.
template <int LPR, int CPL, int FMT, int GM>
__device__ __forceinline__ float row_dot(const u32x4 (&w)[CPL],
                                         const uint32_t (&s)[slot_scales<FMT, GM, CPL>()],
                                         const f16* xl, int chunks, int row, bool sf16, int t) {
  const int sub = (t & 63) % LPR;
  const int sb = sf16 ? 2 : 4;
  constexpr int XW = FMT == kQ8 ? 8 : 16;  // activation dwords per chunk
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ci = sub + c * LPR;
    uint32_t xr[XW];
    if (ci < chunks) {
      const u32x4* src = (const u32x4*)(xl + ci * (2 * XW));
#pragma unroll
      for (int v = 0; v < XW / 4; ++v) {
        const u32x4 t4 = src[v];
        xr[4 * v + 0] = t4[0];
        xr[4 * v + 1] = t4[1];
        xr[4 * v + 2] = t4[2];
        xr[4 * v + 3] = t4[3];
      }
    } else {
#pragma unroll
      for (int d = 0; d < XW; ++d) xr[d] = 0u;
    }
    if constexpr (FMT == kQ8) {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        uint32_t lo, hi;
        q8_pairs(w[c][d], lo, hi);
        acc = dot2(hi, xr[2 * d + 1], dot2(lo, xr[2 * d], acc));
      }
    } else {
      constexpr int SPC = GM == kG16 ? 2 : 1;
      float part[SPC];
#pragma unroll
      for (int g = 0; g < SPC; ++g) part[g] = 0.0f;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        uint32_t q[4];
        q4_pairs(w[c][d], q);
        const int g = GM == kG16 ? (d >> 1) : 0;
        float tt = part[g];
        tt = dot2(q[0], xr[4 * d + 0], tt);
        tt = dot2(q[1], xr[4 * d + 1], tt);
        tt = dot2(q[2], xr[4 * d + 2], tt);
        tt = dot2(q[3], xr[4 * d + 3], tt);
        part[g] = tt;
      }
#pragma unroll
      for (int g = 0; g < SPC; ++g)
        acc = fmaf(part[g], scale_at(s[SPC * c + g], (row * SPC * chunks + SPC * ci + g) * sb, sf16),
                   acc);
    }
  }
  float v = group_sum<LPR>(acc);
  if constexpr (FMT == kQ8) v *= scale_at(s[0], row * sb, sf16);
  return v;
}

// row_dot of a gate/up pair of row slots against one read of the activation
// chunks: each row's sums in row_dot's order (bit-identical to two row_dots).
template <int LPR, int CPL, int FMT, int GM>
__device__ __forceinline__ void row_dot2(const u32x4 (&w)[2][CPL],
                                         const uint32_t (&s)[2][slot_scales<FMT, GM, CPL>()],
                                         const f16* xl, int chunks, int row, bool sf16, int t,
                                         float& out0, float& out1) {
  const int sub = (t & 63) % LPR;
  const int sb = sf16 ? 2 : 4;
  constexpr int XW = FMT == kQ8 ? 8 : 16;  // activation dwords per chunk
  float acc[2] = {0.0f, 0.0f};
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ci = sub + c * LPR;
    uint32_t xr[XW];
    if (ci < chunks) {
      const u32x4* src = (const u32x4*)(xl + ci * (2 * XW));
#pragma unroll
      for (int v = 0; v < XW / 4; ++v) {
        const u32x4 t4 = src[v];
        xr[4 * v + 0] = t4[0];
        xr[4 * v + 1] = t4[1];
        xr[4 * v + 2] = t4[2];
        xr[4 * v + 3] = t4[3];
      }
    } else {
#pragma unroll
      for (int d = 0; d < XW; ++d) xr[d] = 0u;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if constexpr (FMT == kQ8) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          uint32_t lo, hi;
          q8_pairs(w[h][c][d], lo, hi);
          acc[h] = dot2(hi, xr[2 * d + 1], dot2(lo, xr[2 * d], acc[h]));
        }
      } else {
        constexpr int SPC = GM == kG16 ? 2 : 1;
        float part[SPC];
#pragma unroll
        for (int g = 0; g < SPC; ++g) part[g] = 0.0f;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          uint32_t q[4];
          q4_pairs(w[h][c][d], q);
          const int g = GM == kG16 ? (d >> 1) : 0;
          float tt = part[g];
          tt = dot2(q[0], xr[4 * d + 0], tt);
          tt = dot2(q[1], xr[4 * d + 1], tt);
          tt = dot2(q[2], xr[4 * d + 2], tt);
          tt = dot2(q[3], xr[4 * d + 3], tt);
          part[g] = tt;
        }
#pragma unroll
        for (int g = 0; g < SPC; ++g)
          acc[h] = fmaf(part[g],
                        scale_at(s[h][SPC * c + g], (row * SPC * chunks + SPC * ci + g) * sb, sf16),
                        acc[h]);
      }
    }
  }
  float v0 = group_sum<LPR>(acc[0]), v1 = group_sum<LPR>(acc[1]);
  if constexpr (FMT == kQ8) {
    v0 *= scale_at(s[0][0], row * sb, sf16);
    v1 *= scale_at(s[1][0], row * sb, sf16);
  }
  out0 = v0;
  out1 = v1;
}

// Rows of one phase for this workgroup and compute wave: [row0 + wave * slots, +slots).
struct WaveRows {
  int r0;     // first row of the wave (in the phase's row space)
  bool live;  // the wave has rows
};
__device__ __forceinline__ WaveRows wave_rows(int per_wg, int slots, int total) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  WaveRows w;
  w.r0 = blockIdx.x * per_wg + wave * slots;
  w.live = wave < kCW && wave * slots < per_wg && w.r0 < total;
  return w;
}

}  // namespace

template <int FMT, int GM, int GQ, int L1, int C1, int L2, int C2, int L3, int C3>
__global__ __launch_bounds__(kSt) void decode_layers_kernel(const StepParams p) {
  constexpr int S1 = 64 / L1, S2 = 64 / L2, S3 = 64 / L3;  // row slots per wave
  constexpr int kCE = FMT == kQ8 ? 16 : 32;                  // codes per 16-byte chunk
  constexpr bool kPairs = FMT == kQ4;                        // activations in q4_xpairs order
  // Q4 weights are prefetched one to three phases ahead; Q8 rows are twice the
  // bytes, so each matrix is issued two phases before its use (at most three
  // matrices in flight), which keeps the wave within the register budget of
  // three waves per SIMD
  // inputs of the phases (written by the poll wave one phase earlier)
  __shared__ __align__(16) f16 s_xa[kStepMaxHidden];   // layer input, plain (P3 residual)
  __shared__ __align__(16) f16 s_xb[kStepMaxHidden];   // after attention, plain (P5 residual)
  __shared__ __align__(16) f16 s_xn[kStepMaxHidden];   // RMSNorm-in output, pair order (P1, P4)
  __shared__ __align__(16) float s_ga[kStepMaxHidden]; // gamma before q/k/v
  __shared__ __align__(16) float s_gm[kStepMaxHidden]; // gamma before gate/up
  __shared__ __align__(16) f16 s_q[GQ * kHd];          // rotated q of the kv head's q heads
  __shared__ __align__(16) f16 s_kn[kHd];              // the new K row (rotated)
  __shared__ __align__(16) f16 s_vn[kHd];              // the new V row
  __shared__ __align__(16) f16 s_at[kStepMaxQ];        // attention output, pair order (P3)
  __shared__ __align__(16) f16 s_h[kStepMaxInter];     // SwiGLU output, pair order (P5)
  // attention scratch of the compute waves
  __shared__ __align__(16) f16 s_v[kAP * kHd];         // V rows (wave w: rows 8w .. 8w + 7)
  __shared__ __align__(16) float s_e[kAW][GQ][8];      // the wave's scores per head
  __shared__ __align__(16) float s_x[kAW][GQ][8];      // exp(score - wave max)
  __shared__ float s_wm[kAW][GQ], s_wl[kAW][GQ];       // wave max, wave sum
  __shared__ __align__(16) float s_wacc[kAW][GQ][kHd]; // wave P.V sums
  __shared__ StepLayer s_layers[kStepMaxLayers];        // the layer table
  __shared__ __align__(16) uint32_t s_out[kStepOutWords];  // this phase's tagged outputs
  __shared__ int s_done;                               // compute waves done with s_out
  __shared__ int s_cbar;
  __shared__ float s_rpart[4];                         // the RMSNorm's four wave sums
  __shared__ int s_rms;                                // RMSNorm halves done (both poll waves)
  __shared__ float s_inv;                              // 1 / rms of the phase's RMSNorm-in input
  __shared__ int s_invc;                               // 1 / rms values published
  __shared__ uint32_t s_e0;

  const int b = blockIdx.x;
  const int wave_u = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool store = wave_u == kSW;
  const bool compute = wave_u < kCW;
  const int pw = wave_u - kSW - 1;  // poll wave index (when poll)
  const bool sf16 = p.sf16 != 0;
  const int hid = p.hidden, qw = p.qw, kvw = p.kvw, inter = p.inter;
  const int ch1 = hid / kCE, ch2 = qw / kCE, ch3 = inter / kCE;  // code chunks per row
  const int nqkv = qw + 2 * kvw;
  int* err = p.err;
  bool broken = false;
  int cbar_target = 0;
  int done_target = 0;

  int pos = *p.pos;
  pos = pos < 0 ? 0 : (pos >= p.cap ? p.cap - 1 : pos);
  const int len = pos + 1;

  // row partitions (host-checked: multiples of the slot counts, within the compute waves)
  const WaveRows w1 = wave_rows(p.rows_qkv, S1, nqkv);
  const WaveRows w3 = wave_rows(p.rows_hid, S2, hid);
  const WaveRows w4 = wave_rows(p.rows_inter, S1, inter);
  const WaveRows w5 = wave_rows(p.rows_hid, S3, hid);
  // attention split of this workgroup
  const int S = p.splits, sp = p.split_pos;
  const bool attn_wg = b < p.hkv * S;
  const int ag = attn_wg ? b / S : 0, as = attn_wg ? b % S : 0;
  const int ap0 = as * sp;  // first position of the split
  const bool live_split = attn_wg && ap0 < len;
  const int sl_len = live_split ? (len - ap0 < sp ? len - ap0 : sp) : 0;
  const bool has_new = live_split && pos < ap0 + sp;
  // merge slice of this workgroup: q head mh, dims md0 .. md0 + per
  const int per = p.merge_dims;
  const int mh = (b * per) / kHd, md0 = (b * per) % kHd;
  const bool mwg = mh < p.hq;

  // matrix of a q/k/v wave (wave-uniform)
  auto qkv_mat = [&](const StepLayer& L, int r0, const uint32_t*& w, const void*& s, int& n,
                     int& lr) {
    const int j = r0 < qw ? 0 : (r0 < qw + kvw ? 1 : 2);
    w = lds_ptr(&L.w[j]);
    s = lds_ptr(&L.s[j]);
    n = j == 0 ? qw : kvw;
    lr = r0 - (j == 0 ? 0 : (j == 1 ? qw : qw + kvw));
  };

  // compute-wave registers: prefetched weights and the split's K/V rows
  Slot<FMT, GM, C1, 1> wqkv;
  Slot<FMT, GM, C2, 1> wo;
  Slot<FMT, GM, C1, 2> wgu;
  Slot<FMT, GM, C3, 1> wd;
  u32x4 kreg[2], vreg[2];  // thread t < 8 kAP: position ap0 + t / 8, dims 16 (t % 8) .. + 16

  auto issue_qkv = [&](int l, int t) {
    const uint32_t* w; const void* s; int n, lr;
    qkv_mat(s_layers[l], w1.live ? w1.r0 : 0, w, s, n, lr);
    issue_slot<L1, C1, 1>(wqkv, w, s, nullptr, nullptr, n, lr, ch1, sf16, w1.live, t);
  };
  auto issue_kv = [&](int l, int t, bool want_k, bool want_v) {
    const long long head_off = (long long)ag * p.cap * kHd;
    const int lim = live_split ? ap0 + sl_len : 0;
    const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const f16*)lds_ptr(&s_layers[l].kc) + head_off), (short)0, lim * kHd * 2,
        kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const f16*)lds_ptr(&s_layers[l].vc) + head_off), (short)0, lim * kHd * 2,
        kBufferRsrcWord3);
    const int pl = t >> 3, j = t & 7;
    const int off = pl < sp ? ((ap0 + pl) * kHd + j * 16) * 2 : kNoOff;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (want_k)
        kreg[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, off + 16 * i, 0, kStreamAux));
      if (want_v)
        vreg[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, off + 16 * i, 0, kStreamAux));
    }
  };
  auto issue_o = [&](int l, int t) {
    const StepLayer& L = s_layers[l];
    issue_slot<L2, C2, 1>(wo, lds_ptr(&L.w[3]), lds_ptr(&L.s[3]), nullptr, nullptr, hid,
                          w3.live ? w3.r0 : 0, ch2, sf16, w3.live, t);
  };
  auto issue_gu = [&](int l, int t) {
    const StepLayer& L = s_layers[l];
    issue_slot<L1, C1, 2>(wgu, lds_ptr(&L.w[4]), lds_ptr(&L.s[4]), lds_ptr(&L.w[5]),
                          lds_ptr(&L.s[5]), inter, w4.live ? w4.r0 : 0, ch1, sf16, w4.live, t);
  };
  auto issue_d = [&](int l, int t) {
    const StepLayer& L = s_layers[l];
    issue_slot<L3, C3, 1>(wd, lds_ptr(&L.w[6]), lds_ptr(&L.s[6]), nullptr, nullptr, hid,
                          w5.live ? w5.r0 : 0, ch3, sf16, w5.live, t);
  };

  // ---------------- prologue: the layer table into LDS; layer 0's input and normalised row
  {
    const int words = p.nlayers * (int)(sizeof(StepLayer) / 4);
    for (int i = threadIdx.x; i < words; i += kSt)
      ((uint32_t*)s_layers)[i] = ((const uint32_t*)p.layers)[i];
    if (threadIdx.x == 0) {
      s_cbar = 0;
      s_rms = 0;
      s_invc = 0;
      s_done = 0;
      s_e0 = ld_word(p.epoch);
    }
  }
  __syncthreads();
  const uint32_t e0 = s_e0;
  const int nl = p.nlayers;

  // Each role runs its own loop over the layers, with the same five workgroup
  // barriers per layer (one per phase); keeping the roles' code apart keeps
  // the compiler's vector-memory wait counts of each role exact.
  if (compute) {
    {
      const int t = cw_tid<FMT>();
      issue_qkv(0, t);
      issue_kv(0, t, true, true);
    }
    __syncthreads();
    for (int l = 0; l < nl; ++l) {
      const StepLayer& L = s_layers[l];
      const uint32_t tg = e0 + 1 + 6u * (uint32_t)l;  // tags of P1..P5 are tg .. tg + 5
      // ---------------- P1: q/k/v
      {
        const int t = cw_tid<FMT>(), lane = t & 63;
        issue_o(l, t);
        if constexpr (FMT != kQ8) issue_d(l, t);
        if (w1.live) {
          const uint32_t* w; const void* s; int n, lr;
          qkv_mat(L, w1.r0, w, s, n, lr);
          const int row = lr + lane / L1;
          float v = row_dot<L1, C1, FMT, GM>(wqkv.w[0], wqkv.s[0], s_xn, ch1, row, sf16, t);
          // layer 0's input is normalised whole (the prologue); later layers'
          // rows take 1 / rms here
          if (l > 0) v *= cw_inv(&s_inv, &s_invc, 2 * l, err, broken);
          v += 0.0f;
          if (lane % L1 == 0 && row < n)
            s_out[w1.r0 + lane / L1 - b * p.rows_qkv] = tag_f16((f16)v, tg);
        }
        cw_signal(&s_done, lane);
      }
      __syncthreads();
      // ---------------- P2: attention splits
      {
        const int t = cw_tid<FMT>(), lane = t & 63, wave = t >> 6;
        issue_gu(l, t);
        if (attn_wg) {
          const int pl = t >> 3, j = t & 7;  // position pl of the split, dims 16 j .. 16 j + 15
          if (live_split && wave < kAW) {
            if (has_new && ap0 + pl == pos) {
              kreg[0] = *(const u32x4*)&s_kn[j * 16];
              kreg[1] = *(const u32x4*)&s_kn[j * 16 + 8];
              vreg[0] = *(const u32x4*)&s_vn[j * 16];
              vreg[1] = *(const u32x4*)&s_vn[j * 16 + 8];
            }
            *(u32x4*)&s_v[pl * kHd + j * 16] = vreg[0];
            *(u32x4*)&s_v[pl * kHd + j * 16 + 8] = vreg[1];
            const bool live = pl < sl_len;
            // scores of all heads first (independent chains the compiler interleaves)
            float sc[GQ];
#pragma unroll
            for (int h = 0; h < GQ; ++h) {
              const u32x4 q0 = *(const u32x4*)&s_q[h * kHd + j * 16];
              const u32x4 q1 = *(const u32x4*)&s_q[h * kHd + j * 16 + 8];
              float a = 0.0f;
#pragma unroll
              for (int e = 0; e < 4; ++e) a = dot2(kreg[0][e], q0[e], a);
#pragma unroll
              for (int e = 0; e < 4; ++e) a = dot2(kreg[1][e], q1[e], a);
              a += dppf<0xB1>(a);   // quad_perm [1,0,3,2]
              a += dppf<0x4E>(a);   // quad_perm [2,3,0,1]
              a += dppf<0x141>(a);  // row_half_mirror: the other quad of the 8 lanes
              sc[h] = live ? a * p.scale : -INFINITY;
            }
            // softmax statistics through LDS (a wave's LDS accesses complete in
            // order): the 8 scores per head give every lane the wave maximum,
            // each position's lanes form its exp once, and the 8 exps per head
            // come back for the sums and P.V
            if (j == 0) {
#pragma unroll
              for (int h = 0; h < GQ; ++h) s_e[wave][h][pl & 7] = sc[h];
            }
            __asm__ volatile("" ::: "memory");
            float mh[GQ];
#pragma unroll
            for (int h = 0; h < GQ; ++h) {
              const f32x4 e0 = *(const f32x4*)&s_e[wave][h][0];
              const f32x4 e1 = *(const f32x4*)&s_e[wave][h][4];
              mh[h] = fmaxf(fmaxf(fmaxf(e0[0], e0[1]), fmaxf(e0[2], e0[3])),
                            fmaxf(fmaxf(e1[0], e1[1]), fmaxf(e1[2], e1[3])));
            }
            // this lane's dims 2l, 2l + 1 of the wave's 8 V rows, for every head
            f16x2 vv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i)
              vv[i] = as_h2(*(const uint32_t*)&s_v[(wave * 8 + i) * kHd + 2 * lane]);
            __asm__ volatile("" ::: "memory");
            if (j == 0) {
#pragma unroll
              for (int h = 0; h < GQ; ++h) s_x[wave][h][pl & 7] = live ? __expf(sc[h] - mh[h]) : 0.0f;
            }
            __asm__ volatile("" ::: "memory");
            // P.V over the wave's 8 positions: lane l owns dims 2l, 2l + 1 of every head
#pragma unroll
            for (int h = 0; h < GQ; ++h) {
              const f32x4 x0 = *(const f32x4*)&s_x[wave][h][0];
              const f32x4 x1 = *(const f32x4*)&s_x[wave][h][4];
              const float e8[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
              float l = 0.0f, a0 = 0.0f, a1 = 0.0f;
#pragma unroll
              for (int i = 0; i < 8; ++i) {
                l += e8[i];
                a0 = fmaf(e8[i], (float)vv[i][0], a0);
                a1 = fmaf(e8[i], (float)vv[i][1], a1);
              }
              *(float2*)&s_wacc[wave][h][2 * lane] = make_float2(a0, a1);
              if (lane == 0) {
                s_wm[wave][h] = mh[h] == -INFINITY ? kNegBig : mh[h];
                s_wl[wave][h] = l;
              }
            }
          }
          cbar(&s_cbar, cbar_target, lane, err, broken);
          // the split's partial per head: the waves combined (a split past the
          // live length stores the neutral partial, so every word is rewritten)
          if (t < GQ * kHd) {
            const int h = t / kHd, d = t % kHd;
            float m = kNegBig, sum = 0.0f, a = 0.0f;
            if (live_split) {
              for (int w = 0; w < kAW; ++w) m = fmaxf(m, s_wm[w][h]);
              m = trunc_f32(m);  // the value the merge reads back
              for (int w = 0; w < kAW; ++w) {
                const float f = __expf(s_wm[w][h] - m);
                sum = fmaf(s_wl[w][h], f, sum);
                a = fmaf(s_wacc[w][h][d], f, a);
              }
            }
            uint32_t* row = s_out + h * kStepPartStride;
            row[4 + d] = tag_f32(a, tg + 1);
            if (d == 0) {
              // the pad words carry the tag too, so the header polls as one group
              row[0] = tag_f32(m, tg + 1);
              row[1] = tag_f32(sum, tg + 1);
              row[2] = tag_f32(0.0f, tg + 1);
              row[3] = tag_f32(0.0f, tg + 1);
            }
          }
        }
        cw_signal(&s_done, lane);
      }
      __syncthreads();
      // ---------------- P3: o_proj + residual
      {
        const int t = cw_tid<FMT>(), lane = t & 63;
        if constexpr (FMT == kQ8) {
          issue_d(l, t);
        } else {
          if (l + 1 < nl) issue_qkv(l + 1, t);
        }
        if (w3.live) {
          const int row = w3.r0 + lane / L2;
          float v = 0.0f + row_dot<L2, C2, FMT, GM>(wo.w[0], wo.s[0], s_at, ch2, row, sf16, t);
          if (row < hid) v += (float)s_xa[row];
          if (lane % L2 == 0 && row < hid) s_out[row - b * p.rows_hid] = tag_f16((f16)v, tg + 3);
        }
        cw_signal(&s_done, lane);
      }
      __syncthreads();
      // ---------------- P4: gate/up + SwiGLU-out
      {
        const int t = cw_tid<FMT>(), lane = t & 63;
        if constexpr (FMT == kQ8) {
          if (l + 1 < nl) issue_qkv(l + 1, t);
        }
        if (l + 1 < nl) issue_kv(l + 1, t, true, false);
        if (w4.live) {
          const int row = w4.r0 + lane / L1;
          float g, u;
          row_dot2<L1, C1, FMT, GM>(wgu.w, wgu.s, s_xn, ch1, row, sf16, t, g, u);
          const float inv = cw_inv(&s_inv, &s_invc, 2 * l + 1, err, broken);
          g = g * inv + 0.0f;
          u = u * inv + 0.0f;
          const float v = silu(g) * u;
          if (lane % L1 == 0 && row < inter)
            s_out[row - b * p.rows_inter] = tag_f16((f16)v, tg + 4);
        }
        cw_signal(&s_done, lane);
      }
      __syncthreads();
      // ---------------- P5: down + residual
      {
        const int t = cw_tid<FMT>(), lane = t & 63;
        if (l + 1 < nl) issue_kv(l + 1, t, false, true);
        if (w5.live) {
          const int row = w5.r0 + lane / L3;
          float v = 0.0f + row_dot<L3, C3, FMT, GM>(wd.w[0], wd.s[0], s_h, ch3, row, sf16, t);
          if (row < hid) v += (float)s_xb[row];
          if (lane % L3 == 0 && row < hid) s_out[row - b * p.rows_hid] = tag_f16((f16)v, tg + 5);
        }
        cw_signal(&s_done, lane);
      }
      __syncthreads();
    }
  } else if (store) {
    __syncthreads();
    const int lane = opaque_tid() & 63;
    const RepLanes rl_qkv = rep_lanes(p.rows_qkv, lane), rl_hid = rep_lanes(p.rows_hid, lane),
                   rl_inter = rep_lanes(p.rows_inter, lane);
    for (int l = 0; l < nl; ++l) {
      const StepLayer& L = s_layers[l];
      // P1: q/k/v rows
      {
        sw_wait(&s_done, done_target, err, broken);
        AEXQ_STAMP(l, 0, lane, b);
        const int r0 = b * p.rows_qkv;
        const int n = nqkv - r0 < p.rows_qkv ? nqkv - r0 : p.rows_qkv;
        if (n > 0) sw_copy_rep(p.qkv_t + r0, p.qkv_rs, s_out, n, rl_qkv);
      }
      __syncthreads();
      AEXQ_STAMP(l, 1, lane, b);
      // P2: the K/V append, the split partials, the merged attention slice
      {
        if (has_new) {
          // the rotated k row and the v row at `pos`
          uint32_t* kc = (uint32_t*)((f16*)lds_ptr(&L.kc) + ((long long)ag * p.cap + pos) * kHd);
          uint32_t* vc = (uint32_t*)((f16*)lds_ptr(&L.vc) + ((long long)ag * p.cap + pos) * kHd);
          kc[lane] = ((const uint32_t*)s_kn)[lane];
          vc[lane] = ((const uint32_t*)s_vn)[lane];
        }
        sw_wait(&s_done, done_target, err, broken);
        AEXQ_STAMP(l, 2, lane, b);
        if (attn_wg && lane < kStepPartStride / 4) {
          // the split's partial of each head, 16 bytes a lane: every LDS read
          // first, then the stores (one LDS round trip)
          u32x4 pv[GQ];
#pragma unroll
          for (int h = 0; h < GQ; ++h) pv[h] = *(const u32x4*)(s_out + h * kStepPartStride + 4 * lane);
          const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
              (void*)p.part_t, (short)0, p.hq * S * kStepPartStride * 4, kBufferRsrcWord3);
#pragma unroll
          for (int h = 0; h < GQ; ++h)
            st_quad(pr, (((ag * GQ + h) * S + as) * kStepPartStride + 4 * lane) * 4, pv[h]);
        }
      }
      __syncthreads();
      AEXQ_STAMP(l, 3, lane, b);
      // P3: rows after attention
      {
        sw_wait(&s_done, done_target, err, broken);
        AEXQ_STAMP(l, 4, lane, b);
        const int r0 = b * p.rows_hid;
        const int n = hid - r0 < p.rows_hid ? hid - r0 : p.rows_hid;
        if (n > 0) sw_copy_rep(p.xb_t + r0, p.xb_rs, s_out, n, rl_hid);
      }
      __syncthreads();
      AEXQ_STAMP(l, 5, lane, b);
      // P4: SwiGLU rows
      {
        sw_wait(&s_done, done_target, err, broken);
        AEXQ_STAMP(l, 6, lane, b);
        const int r0 = b * p.rows_inter;
        const int n = inter - r0 < p.rows_inter ? inter - r0 : p.rows_inter;
        if (n > 0) sw_copy_rep(p.h_t + r0, p.h_rs, s_out, n, rl_inter, kStepReplicasH);
      }
      __syncthreads();
      AEXQ_STAMP(l, 7, lane, b);
      // P5: the layer's output rows (and the step's output after the last layer)
      {
        sw_wait(&s_done, done_target, err, broken);
        AEXQ_STAMP(l, 8, lane, b);
        const int r0 = b * p.rows_hid;
        const int n = hid - r0 < p.rows_hid ? hid - r0 : p.rows_hid;
        if (n > 0) {
          sw_copy_rep(p.xa_t + r0, p.xa_rs, s_out, n, rl_hid);
          if (l + 1 == nl)
            for (int i = lane; i < n; i += 64) p.out[r0 + i] = (uint16_t)(s_out[i] & 0xffffu);
        }
      }
      __syncthreads();
      AEXQ_STAMP(l, 9, lane, b);
    }
    if (b == 0 && lane == 0) st_word(p.epoch, e0 + 6u * (uint32_t)nl);
  } else {
    const int lane = opaque_tid() & 63;
    const int rc = b % kStepReplicas;  // the copy of every polled vector this workgroup reads
    int rms_target = 0;
    u32x4 xa_g[2];  // the next layer's input slices (pw_vec_gx), for its 1 / rms
    if (pw == 0) {
      f32x4 g[4];
      pw_gamma_issue(lds_ptr(&s_layers[0].g_attn), hid, g, lane);
      // the token's row of the tied Q8 table (embed_q8_kernel's arithmetic:
      // fp16((code - 128) * scale))
      int tok = *p.token;
      tok = tok < 0 ? 0 : (tok >= p.vocab ? p.vocab - 1 : tok);
      const float sc = load_scale(p.emb_scales, tok, p.emb_sf16 != 0);
      const uint8_t* row = (const uint8_t*)p.emb_codes + (long long)tok * hid;
      for (int d = lane; d < hid; d += 64) s_xa[d] = (f16)((float)((int)row[d] - 128) * sc);
      pw_gamma_store(g, s_ga, hid, lane);
      __asm__ volatile("" ::: "memory");
      pw_rms<kPairs>(s_xa, s_ga, s_xn, hid, p.eps, lane);
    }
    __syncthreads();
    for (int l = 0; l < nl; ++l) {
      const StepLayer& L = s_layers[l];
      const uint32_t tg = e0 + 1 + 6u * (uint32_t)l;
      // during P1: 1 / rms of the layer's input (layers after the first); q/k/v
      // of the kv head, RoPE of q and the new k row
      if (l > 0)
        pw_inv_publish(xa_g, hid, p.eps, lane, pw, s_rpart, &s_rms, rms_target, &s_inv, &s_invc,
                       err, broken);
      if (attn_wg && pw == 0) {
        // this position's RoPE row (DEC:1660-1675 tables), entry `lane`
        const float cs = p.cos_t[(long long)pos * kHalf + lane];
        const float sn = p.sin_t[(long long)pos * kHalf + lane];
        constexpr int NQ = GQ * kHd / 256;  // 16-byte groups of q per lane
        int off[NQ + 1];
#pragma unroll
        for (int i = 0; i < NQ; ++i) off[i] = ag * GQ * kHd + (lane + 64 * i) * 4;
        off[NQ] = lane < 32 ? qw + ag * kHd + lane * 4 : qw + kvw + ag * kHd + (lane - 32) * 4;
        u32x4 v[NQ + 1];
        pw_wait<NQ + 1>(p.qkv_t + rc * p.qkv_rs, nqkv, off, tg, 16, 0xffffu, v, err, broken);
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
          uint32_t a, c;
          halves(v[i], a, c);
          uint32_t* d = (uint32_t*)(s_q + (lane + 64 * i) * 4);
          d[0] = a;
          d[1] = c;
        }
        {
          uint32_t a, c;
          halves(v[NQ], a, c);
          uint32_t* d = (uint32_t*)((lane < 32 ? s_kn + lane * 4 : s_vn + (lane - 32) * 4));
          d[0] = a;
          d[1] = c;
        }
        __asm__ volatile("" ::: "memory");
        // rotate-half pairs (j, j + 64) with j = lane, rounded to fp16 (the
        // attention kernel's arithmetic)
#pragma unroll
        for (int h = 0; h < GQ; ++h) {
          const float qa = (float)s_q[h * kHd + lane], qb = (float)s_q[h * kHd + lane + kHalf];
          s_q[h * kHd + lane] = (f16)(qa * cs - qb * sn);
          s_q[h * kHd + lane + kHalf] = (f16)(qa * sn + qb * cs);
        }
        const float x0 = (float)s_kn[lane], x1 = (float)s_kn[lane + kHalf];
        const f16 k0 = (f16)(x0 * cs - x1 * sn), k1 = (f16)(x0 * sn + x1 * cs);
        s_kn[lane] = k0;
        s_kn[lane + kHalf] = k1;
      }
      __syncthreads();
      // during P2: the gamma before gate/up; the split merge; the attention output
      if (pw == 1) {
        f32x4 gm[4];
        pw_gamma_issue(lds_ptr(&L.g_mlp), hid, gm, lane);
        pw_gamma_store(gm, s_gm, hid, lane);
      }
      if (mwg) {
        // the split merge of (q head mh, dims md0 .. md0 + per), MM:420-544's
        // softmax over all positions, on both poll waves: wave pw merges dims
        // md0 + hp pw .. + hp (hp = per / 2) in lq quads of 4 dims, each held by
        // sl = 64 / lq lanes, lane = quad q4 * sl + split s; every lane reads
        // its split's (max, sum) header.  A quad's lanes sum over the splits with
        // group_sum (no LDS round trip), and its first kStepReplicas lanes write
        // the merged 4 dims into the copies of the attention output themselves.
        static_assert(kStepReplicas <= 16, "a quad has at least 16 lanes");
        const int hp = per / 2, lq = hp / 4, sl = 64 / lq, q4 = lane / sl, s = lane % sl;
        const int d0 = md0 + hp * pw + 4 * q4;
        const bool in = s < S;
        const int rb = (mh * S + (in ? s : 0)) * kStepPartStride;
        int off[2] = {in ? rb + 4 + d0 : -1, in ? rb : -1};
        u32x4 v[2];
        pw_wait<2>(p.part_t, p.hq * S * kStepPartStride, off, tg + 1, 0, 0xffu, v, err, broken);
        // absent splits are neutral
        const float ms = in ? as_f32(v[1][0] & ~0xffu) : kNegBig;
        const float ls = in ? as_f32(v[1][1] & ~0xffu) : 0.0f;
        const float M = wave_max(ms);
        const float f = __expf(ms - M);
        const float lsum = wave_sum(q4 == 0 ? ls * f : 0.0f);
        float a[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) a[e] = in ? as_f32(v[0][e] & ~0xffu) * f : 0.0f;
        if (sl == 64) {
#pragma unroll
          for (int e = 0; e < 4; ++e) a[e] = group_sum<64>(a[e]);
        } else if (sl == 32) {
#pragma unroll
          for (int e = 0; e < 4; ++e) a[e] = group_sum<32>(a[e]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) a[e] = group_sum<16>(a[e]);
        }
        if (s < kStepReplicas) {
          const float inv_l = 1.0f / fmaxf(lsum, 1e-20f);
          u32x4 w0;
#pragma unroll
          for (int e = 0; e < 4; ++e) w0[e] = tag_f16((f16)(a[e] * inv_l), tg + 2);
          const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc(
              (void*)p.attn_t, (short)0, kStepReplicas * p.attn_rs * 4, kBufferRsrcWord3);
          st_quad(ar, (s * p.attn_rs + mh * kHd + d0) * 4, w0);
        }
      }
      // the attention output of the whole grid (the merges of every workgroup)
      pw_vec_pairs<kStepMaxQ / 256 / kPW, kPairs>(p.attn_t + rc * p.attn_rs, qw, tg + 2, s_at, lane,
                                                  pw, err, broken);
      __syncthreads();
      // during P3: x after attention, and gamma x for the next linear (both
      // poll waves); the next layer's gamma
      if (pw == 1 && l + 1 < nl) {
        f32x4 ga[4];
        pw_gamma_issue(lds_ptr(&s_layers[l + 1].g_attn), hid, ga, lane);
        pw_gamma_store(ga, s_ga, hid, lane);
      }
      u32x4 xb_g[2];
      pw_vec_gx<kPairs>(p.xb_t + rc * p.xb_rs, hid, tg + 3, s_xb, s_gm, s_xn, lane, pw, xb_g, err,
                        broken);
      __syncthreads();
      // during P4: 1 / rms of x after attention; the SwiGLU output
      pw_inv_publish(xb_g, hid, p.eps, lane, pw, s_rpart, &s_rms, rms_target, &s_inv, &s_invc,
                     err, broken);
      pw_vec_pairs<kStepMaxInter / 256 / kPW, kPairs>(p.h_t + (b % kStepReplicasH) * p.h_rs, inter, tg + 4, s_h, lane,
                                                      pw, err, broken);
      __syncthreads();
      // during P5: the next layer's input, and gamma x for its q/k/v (both
      // poll waves)
      if (l + 1 < nl)
        pw_vec_gx<kPairs>(p.xa_t + rc * p.xa_rs, hid, tg + 5, s_xa, s_ga, s_xn, lane, pw, xa_g, err,
                          broken);
      __syncthreads();
    }
  }
}

// The instantiations (lanes x chunks per row of the hidden-width, q-width and
// intermediate-width inputs): Q4 (groups of 32 or 16) for rows of 17..32 /
// 33..64 / 65..128 chunks, 16 x 2, 64 x 1, 64 x 2; Q8 for 33..64 / 65..128 /
// 129..256 chunks, 16 x 4, 64 x 2, 64 x 4; four q heads per kv head.
#define AEXQ_STEP_Q4(GM) decode_layers_kernel<kQ4, GM, 4, 16, 2, 64, 1, 64, 2>
#define AEXQ_STEP_Q8 decode_layers_kernel<kQ8, kGRow, 4, 16, 4, 64, 2, 64, 4>

bool decode_layers_supported(int fmt, int gmode, int gq, int ch1, int ch2, int ch3) {
  if (gq != 4) return false;
  if (fmt == kQ4 && (gmode == kG32 || gmode == kG16))
    return ch1 > 16 && ch1 <= 32 && ch2 > 32 && ch2 <= 64 && ch3 > 64 && ch3 <= 128;
  if (fmt == kQ8 && gmode == kGRow)
    return ch1 > 32 && ch1 <= 64 && ch2 > 64 && ch2 <= 128 && ch3 > 128 && ch3 <= 256;
  return false;
}

hipError_t decode_layers_occupancy(int fmt, int gmode, int* per_cu) {
  if (fmt == kQ8)
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, AEXQ_STEP_Q8, kSt, 0);
  if (gmode == kG16)
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, AEXQ_STEP_Q4(kG16), kSt, 0);
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, AEXQ_STEP_Q4(kG32), kSt, 0);
}

#ifdef AEXQ_STEP_STAMPS
// The phase stamps of the last launch (n words) into host memory.
extern "C" int aexq_step_stamps(void* host, long long n) {
  if (n > 64LL * 10 * 256) n = 64LL * 10 * 256;
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_step_stamps), (size_t)n * 8, 0,
                                  hipMemcpyDeviceToHost);
}
#endif

hipError_t decode_layers_launch(const StepParams& p, int grid, hipStream_t stream) {
  const int ce = p.fmt == kQ8 ? 16 : 32;
  if (!decode_layers_supported(p.fmt, p.gmode, p.hq / p.hkv, p.hidden / ce, p.qw / ce,
                               p.inter / ce))
    return hipErrorInvalidValue;
  if (p.fmt == kQ8)
    hipLaunchKernelGGL((AEXQ_STEP_Q8), dim3(grid), dim3(kSt), 0, stream, p);
  else if (p.gmode == kG16)
    hipLaunchKernelGGL((AEXQ_STEP_Q4(kG16)), dim3(grid), dim3(kSt), 0, stream, p);
  else
    hipLaunchKernelGGL((AEXQ_STEP_Q4(kG32)), dim3(grid), dim3(kSt), 0, stream, p);
  return hipGetLastError();
}

}  // namespace aexq
