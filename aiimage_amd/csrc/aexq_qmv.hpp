// Persistent streaming matvec / small-M matmul kernel for gfx950 (M <= 8).
//
// The weight is a row-major [N][K] stream of device codes (Q8: int8 biased by
// 128; Q4: offset-8 nibbles, low nibble first) -- the reference's packed words
// (MM:707-734) recoded once at upload.  A wave owns a contiguous range of
// "wave tiles" of RW rows over every (matrix, batch entry, row tile) of the
// launch and walks it with its next tile's loads in flight (two register
// buffers), so each wave keeps 2 x U x CPL 16-byte loads outstanding and no
// barrier ever stops the stream.  Inside a tile, LPR lanes share a row; lane
// `sub` owns 16-byte code chunks sub, sub+LPR, ... of it.  Codes become exact
// fp16 integers in registers (q8_pairs / q4_pairs) and meet the fp16
// activations, which stay in registers while the activation row is unchanged,
// in v_dot2_f32_f16 with fp32 accumulation.  Scales are applied in fp32: once
// per row for Q8, once per 16- or 32-code group for Q4.  Rows are reduced
// across their LPR lanes with DPP.  RMSNorm-in normalises the activation
// registers before the first tile; the epilogues (alpha/beta/C, SwiGLU-out,
// residual, argmax partials) run before the single store.
#pragma once

#include <math.h>

#include "aexq_device.hpp"

namespace aexq {

template <int FMT, int LPR, int CPL, int U, int MMAX, bool PAIR, bool ARGMAX, int GM>
struct Qmv {
  static constexpr int SLOTS = 64 / LPR;                 // rows sharing one wave at once
  static constexpr int RW = SLOTS * U;                   // rows per wave tile
  static constexpr int XW = FMT == kQ8 ? 8 : 16;         // activation dwords per code chunk
  static constexpr int NW = PAIR ? 2 : 1;                // gate (+ up) weights
  static constexpr int NS = FMT == kQ8 ? 1 : (GM == kG16 ? 2 * CPL : CPL);  // scales per row
  // vector memory reads of one tile: residual (M = 1), codes, scales
  static constexpr int kLoadsPerTile = (MMAX == 1 && !ARGMAX ? U : 0) + NW * U * (CPL + NS);
#ifndef QMV_VALU_PER_LOAD
#define QMV_VALU_PER_LOAD 8
#endif
  static constexpr int kValuPerLoad = QMV_VALU_PER_LOAD;

  // Wave-uniform: matrix, batch entry, row tile.  The LM head (ARGMAX) is one
  // matrix of one batch entry (host-checked) and its waves own row ranges,
  // not tile ranges: rt is then the tile's first row and rend the end of the
  // wave's range (rows from rend on belong to the next wave).
  struct Cursor {
    int j, b, rt, rend;
  };

  static __device__ __forceinline__ int row0(const Cursor& c) { return ARGMAX ? c.rt : c.rt * RW; }
  // rows of the tile's matrix this wave loads and computes: below n and, for
  // the LM head, below its range's end
  static __device__ __forceinline__ int row_limit(const QmvMat& mt, const Cursor& c) {
    return ARGMAX && c.rend < mt.n ? c.rend : mt.n;
  }

  struct Buf {
    u32x4 w[NW][U][CPL];
    uint32_t s[NW][U][NS];  // raw scale bits, widened when consumed (keeps loads in flight)
    uint32_t r[U];          // M = 1: the rows' fp16 residual bits, loaded with the tile
  };

  typedef uint32_t XRegs[MMAX][CPL][XW];

  // The LM head's cursor (rt the row, rend the range's end) keeps the tile
  // loop's bookkeeping in plain scalar arithmetic; its kernel forms the first
  // one itself.
  static __device__ __forceinline__ Cursor locate(const QmvParams& p, int t) {
    if constexpr (ARGMAX) return Cursor{0, 0, t, 0};
    int j = 0;
    for (int i = 1; i < p.nmat; ++i)
      if (t >= p.mat[i].tile_base) j = i;
    const int local = t - p.mat[j].tile_base;
    Cursor c;
    c.rend = 0;
    c.j = j;
    c.b = local / p.mat[j].tiles;
    c.rt = local - c.b * p.mat[j].tiles;
    return c;
  }

  static __device__ __forceinline__ Cursor advance(const QmvParams& p, Cursor c) {
    if constexpr (ARGMAX) return Cursor{0, 0, c.rt + RW, c.rend};
    if (++c.rt == p.mat[c.j].tiles) {
      c.rt = 0;
      if (++c.b == p.batch) {
        c.b = 0;
        ++c.j;
      }
    }
    return c;
  }

  // Lane-constant byte offsets of the code chunks and scales of a tile's
  // first row group (u = 0), relative to the tile's first row; row group u
  // adds the wave-uniform u_code_bytes(u) / u_scale_bytes(u).
  struct Offsets {
    int w[CPL];
    int s[NS];
  };
  // byte offset beyond any resource (weight copies are < 2 GiB)
  static constexpr int kNoChunk = 0x7ffffff0;

  static __device__ __forceinline__ Offsets offsets(const QmvParams& p, int sub, int slot) {
    Offsets o;
    const int row_bytes = p.chunks * 16;
    const int sb = (p.flags & kFlagScaleF16) ? 2 : 4;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      // a chunk past K points beyond every resource (also after adding a row
      // group's u_code_bytes): it reads 0 with no traffic
      const int ci = sub + c * LPR;
      o.w[c] = ci < p.chunks ? slot * row_bytes + ci * 16 : kNoChunk;
    }
    if constexpr (FMT == kQ8) {
      o.s[0] = slot * sb;
    } else {
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int ci = sub + c * LPR;
        const int g0 = slot * p.groups_per_row;
        if constexpr (GM == kG16) {
          o.s[2 * c] = (g0 + 2 * ci) * sb;
          o.s[2 * c + 1] = (g0 + 2 * ci + 1) * sb;
        } else {
          o.s[c] = (g0 + (ci * 32) / p.group) * sb;
        }
      }
    }
    return o;
  }

  static __device__ __forceinline__ int u_code_bytes(const QmvParams& p, int u) {
    return u * SLOTS * p.chunks * 16;
  }
  static __device__ __forceinline__ int u_scale_bytes(const QmvParams& p, int u) {
    const int sb = (p.flags & kFlagScaleF16) ? 2 : 4;
    const int sper = FMT == kQ8 ? 1 : p.groups_per_row;
    return u * SLOTS * sper * sb;
  }

  // Byte offset of a tile's first scale inside its weight copy's scale array.
  static __device__ __forceinline__ int scale_tile_offset(const QmvParams& p, const Cursor& cu) {
    const int sb = (p.flags & kFlagScaleF16) ? 2 : 4;
    const int sper = FMT == kQ8 ? 1 : p.groups_per_row;
    return row0(cu) * sper * sb;
  }

  // Issues the loads of one tile without a branch.  Codes: buffer loads
  // against a resource that starts at the tile's first row and ends at row N,
  // so rows past N, and chunks past K, read as zero without memory traffic
  // (and are never stored / meet zero activations).  Scales:
  // the aligned dword holding each scale, from a resource over the copy's
  // whole (256-byte aligned, dword-padded) scale array, widened when consumed.
  // `live` false issues the same loads against empty resources (the prefetch
  // after a wave's last tile): they read 0 without memory traffic.
  static __device__ __forceinline__ void load(const QmvParams& p, const Cursor& cu,
                                              const Offsets& o, Buf& buf, bool live,
                                              int slot) {
    const QmvMat& mt = p.mat[cu.j];
    const int sb = (p.flags & kFlagScaleF16) ? 2 : 4;
    const long long row_bytes = (long long)p.chunks * 16;
    const int r0 = row0(cu);
    // rows of the matrix at or after the tile's first row (and, for the LM
    // head, before the wave's range ends); a tile inside the Pack4 padding rows
    // (r0 >= n) gets an empty resource: every load reads 0
    const int rlim = row_limit(mt, cu);
    const int rows = live && rlim > r0 ? rlim - r0 : 0;
    const int sper = FMT == kQ8 ? 1 : p.groups_per_row;
    const int sbytes = live ? (mt.n * sper * sb + 3) & ~3 : 0;
    if constexpr (MMAX == 1 && !ARGMAX) {
      // fp16 residual rows of the tile, loaded with it (an empty resource
      // without one); fp32 outputs read theirs in the epilogue
      const bool res = mt.res && (p.flags & kFlagResidual) && !(p.flags & kFlagYf32);
      const char* rb =
          res ? (const char*)mt.res + (cu.b * mt.r_bstride + r0) * 2 : (const char*)mt.w;
      const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
          (void*)rb, (short)0, res ? rows * 2 : 0, kBufferRsrcWord3);
#pragma unroll
      for (int u = 0; u < U; ++u)
        buf.r[u] = __builtin_amdgcn_raw_buffer_load_b16(rr, (u * SLOTS + slot) * 2, 0, 0);
    }
    const int toff = scale_tile_offset(p, cu);
#pragma unroll
    for (int h = 0; h < NW; ++h) {
      const char* wb = (const char*)(h == 0 ? mt.w : mt.w2) + (cu.b * mt.w_bstride) * 4 +
                       (long long)r0 * row_bytes;
      const char* sbase = (const char*)(h == 0 ? mt.s : mt.s2) + cu.b * mt.s_bstride * sb;
      const __amdgpu_buffer_rsrc_t wr =
          __builtin_amdgcn_make_buffer_rsrc((void*)wb, (short)0, (int)(rows * row_bytes),
                                            kBufferRsrcWord3);
      const __amdgpu_buffer_rsrc_t sr =
          __builtin_amdgcn_make_buffer_rsrc((void*)sbase, (short)0, sbytes, kBufferRsrcWord3);
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int c = 0; c < CPL; ++c)
          buf.w[h][u][c] = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, o.w[c], u_code_bytes(p, u),
                                                           kStreamAux));
#pragma unroll
        for (int i = 0; i < NS; ++i)
          buf.s[h][u][i] = __builtin_amdgcn_raw_buffer_load_b32(
              sr, (toff + u_scale_bytes(p, u) + o.s[i]) & ~3, 0, 0);
      }
    }
  }

  // Activation rows of one batch entry into registers.  With the RMSNorm-in
  // epilogue the registers hold fp16(x * inv * gamma), inv = rsqrt(max(mean x^2
  // + eps, 1e-20)), rounded once as the reference's separate RMSNorm dispatch
  // rounds into its fp16 texture (CC:4548-4561): the raw row lands in the
  // registers first, sum(x^2) is reduced from them -- the LPR lanes of a slot
  // hold the whole row -- and only then is each element normalised, so the
  // fp16 value stays bounded by sqrt(K) * |gamma| whatever the row's scale.
  static __device__ __forceinline__ void load_x(const QmvParams& p, const f16* xb, int sub,
                                                XRegs& xr) {
    const bool rms = (p.flags & kFlagRms) != 0;
    const __amdgpu_buffer_rsrc_t grsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)p.gamma, (short)0, p.gamma ? p.k * 4 : 0, kBufferRsrcWord3);
#pragma unroll
    for (int m = 0; m < MMAX; ++m) {
      if (m < p.m) {
        const f16* row = xb + (long long)m * p.x_rstride;
        float ss = 0.0f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          const int ci = sub + c * LPR;
          if (ci < p.chunks) {
            const u32x4* src = (const u32x4*)(row + (long long)ci * (XW * 2));
#pragma unroll
            for (int v = 0; v < XW / 4; ++v) {
              const u32x4 t = src[v];
              xr[m][c][4 * v + 0] = t[0];
              xr[m][c][4 * v + 1] = t[1];
              xr[m][c][4 * v + 2] = t[2];
              xr[m][c][4 * v + 3] = t[3];
            }
          } else {
#pragma unroll
            for (int d = 0; d < XW; ++d) xr[m][c][d] = 0u;
          }
          if (rms) {
#pragma unroll
            for (int d = 0; d < XW; ++d) {
              const f16x2 h = as_h2(xr[m][c][d]);
              const float a = (float)h[0], b = (float)h[1];
              ss = fmaf(a, a, ss);
              ss = fmaf(b, b, ss);
            }
          }
        }
        if (rms) {
          const float inv = rsqrtf(fmaxf(group_sum<LPR>(ss) / (float)p.k + p.eps, 1e-20f));
          const bool use_gamma = p.gamma != nullptr;
          // the registers are re-read below: without this the compiler keeps
          // the sum's fp32 conversions of every element live across the
          // reduction instead of converting again (64 more registers)
#pragma unroll
          for (int c = 0; c < CPL; ++c)
#pragma unroll
            for (int d = 0; d < XW; ++d) __asm__("" : "+v"(xr[m][c][d]));
#pragma unroll
          for (int c = 0; c < CPL; ++c) {
            // gamma through a buffer resource: one offset register per chunk,
            // the rest are immediate offsets (the streaming kernels require
            // gamma to cover K; shorter affine vectors take the generic path).
            // A chunk past K reads gamma 0 against x 0, without a branch.
            const int goff = (sub + c * LPR) * XW * 2 * 4;
#pragma unroll
            for (int d = 0; d < XW; d += 2) {
              const f32x4 t = __builtin_bit_cast(
                  f32x4, __builtin_amdgcn_raw_buffer_load_b128(grsrc, goff + d * 8, 0, 0));
#pragma unroll
              for (int e = 0; e < 2; ++e) {
                const f16x2 h = as_h2(xr[m][c][d + e]);
                const float a = (float)h[0] * inv, b = (float)h[1] * inv;
                const float g0 = use_gamma ? t[2 * e] : 1.0f;
                const float g1 = use_gamma ? t[2 * e + 1] : 1.0f;
                const f16x2 o = {(f16)(a * g0), (f16)(b * g1)};
                xr[m][c][d + e] = as_u(o);
              }
              // one gamma vector in flight at a time: hoisting them all would
              // need 4 * XW * CPL more registers next to the tile buffers
              __builtin_amdgcn_sched_barrier(0);
            }
          }
        }
        if constexpr (FMT == kQ4) {
#pragma unroll
          for (int c = 0; c < CPL; ++c)
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              const uint32_t a = xr[m][c][4 * d], b = xr[m][c][4 * d + 1],
                             e = xr[m][c][4 * d + 2], f = xr[m][c][4 * d + 3];
              q4_xpairs(a, b, e, f, &xr[m][c][4 * d]);
            }
        }
      } else {
#pragma unroll
        for (int c = 0; c < CPL; ++c)
#pragma unroll
          for (int d = 0; d < XW; ++d) xr[m][c][d] = 0u;
      }
    }
  }

  // M = 1 RMSNorm-in with one activation row for the whole launch
  // (kFlagXShared): the workgroup's 256 threads stage fp16(x * inv * gamma)
  // into LDS, 8 elements each per pass -- one memory round trip and two
  // barriers for every wave of the workgroup, instead of each wave walking its
  // chunks' activations and gamma.  stage_issue() issues every pass's x and
  // gamma loads (before the tile's weight loads, so that waiting for them does
  // not wait for the weights); stage_finish() stores the raw row and reduces
  // sum(x^2) through LDS, then each thread normalises the elements it stored.
  // Every thread of the workgroup calls both.
  static constexpr int kStagePasses = 2;
  static_assert(kStagePasses * kThreads * 8 == kQmvStageMaxK, "staged row length");
  struct Stage {
    u32x4 x[kStagePasses];
    f32x4 g[kStagePasses][2];
  };

  static __device__ __forceinline__ void stage_issue(const QmvParams& p, Stage& st) {
    const bool use_gamma = p.gamma != nullptr;
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)p.mat[0].x, (short)0, p.k * 2, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t grs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)p.gamma, (short)0, use_gamma ? p.k * 4 : 0, kBufferRsrcWord3);
#pragma unroll
    for (int it = 0; it < kStagePasses; ++it) {
      const int e0 = (it * kThreads + (int)threadIdx.x) * 8;  // past K: reads 0
      st.x[it] =
          __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, e0 * 2, 0, 0));
    }
#pragma unroll
    for (int it = 0; it < kStagePasses; ++it) {
      const int e0 = (it * kThreads + (int)threadIdx.x) * 8;
      st.g[it][0] =
          __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(grs, e0 * 4, 0, 0));
      st.g[it][1] =
          __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(grs, e0 * 4 + 16, 0, 0));
    }
  }

  static __device__ __forceinline__ void stage_finish(const QmvParams& p, const Stage& st,
                                                      int lane, int wave) {
    extern __shared__ __align__(16) uint8_t qmv_stage[];
    f16* xs = (f16*)qmv_stage;
    float* red = (float*)(qmv_stage + (((size_t)p.k * 2 + 15) & ~(size_t)15));
    const bool use_gamma = p.gamma != nullptr;
    float ss = 0.0f;
#pragma unroll
    for (int it = 0; it < kStagePasses; ++it) {
      const int e0 = (it * kThreads + (int)threadIdx.x) * 8;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f16x2 h = as_h2(st.x[it][e]);
        const float a = (float)h[0], b = (float)h[1];
        ss = fmaf(a, a, ss);
        ss = fmaf(b, b, ss);
      }
      if (e0 < p.k) *(u32x4*)(xs + e0) = st.x[it];
    }
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) tot += red[w];
    const float inv = rsqrtf(fmaxf(tot / (float)p.k + p.eps, 1e-20f));
#pragma unroll
    for (int it = 0; it < kStagePasses; ++it) {
      const int e0 = (it * kThreads + (int)threadIdx.x) * 8;
      if (e0 < p.k) {
        // the thread's own elements: no barrier between its store and this load
        const u32x4 x = *(const u32x4*)(xs + e0);
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const f16x2 h = as_h2(x[e]);
          const float a = (float)h[0] * inv, b = (float)h[1] * inv;
          const float g0 = use_gamma ? st.g[it][e / 2][2 * (e % 2)] : 1.0f;
          const float g1 = use_gamma ? st.g[it][e / 2][2 * (e % 2) + 1] : 1.0f;
          const f16x2 r = {(f16)(a * g0), (f16)(b * g1)};
          o[e] = as_u(r);
        }
        *(u32x4*)(xs + e0) = o;
      }
    }
    __syncthreads();
  }

  // A wave's activation registers from the staged row.
  static __device__ __forceinline__ void load_x_staged(const QmvParams& p, int sub, XRegs& xr) {
    extern __shared__ __align__(16) uint8_t qmv_stage[];
    const f16* xs = (const f16*)qmv_stage;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ci = sub + c * LPR;
      uint32_t raw[XW];
      if (ci < p.chunks) {
        const u32x4* src = (const u32x4*)(xs + ci * (XW * 2));
#pragma unroll
        for (int v = 0; v < XW / 4; ++v) {
          const u32x4 t = src[v];
          raw[4 * v + 0] = t[0];
          raw[4 * v + 1] = t[1];
          raw[4 * v + 2] = t[2];
          raw[4 * v + 3] = t[3];
        }
      } else {
#pragma unroll
        for (int d = 0; d < XW; ++d) raw[d] = 0u;
      }
      if constexpr (FMT == kQ8) {
#pragma unroll
        for (int d = 0; d < XW; ++d) xr[0][c][d] = raw[d];
      } else {
#pragma unroll
        for (int d = 0; d < 4; ++d)
          q4_xpairs(raw[4 * d], raw[4 * d + 1], raw[4 * d + 2], raw[4 * d + 3], &xr[0][c][4 * d]);
      }
    }
  }

  // Dot products, row reduction, epilogue and store of one tile.
  static __device__ __forceinline__ void compute(const QmvParams& p, const Cursor& cu,
                                                 const Offsets& o, const Buf& buf,
                                                 const XRegs& xr, int sub, int slot, float (&bv)[MMAX],
                                                 int (&bi)[MMAX], float (&bs)[MMAX],
                                                 float* lg = nullptr, int lg_r0 = 0) {
    const QmvMat& mt = p.mat[cu.j];
    const bool scl16 = (p.flags & kFlagScaleF16) != 0;
    const int toff = scale_tile_offset(p, cu);
    float acc[NW][U][MMAX];
#pragma unroll
    for (int h = 0; h < NW; ++h)
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int m = 0; m < MMAX; ++m) acc[h][u][m] = 0.0f;

#pragma unroll
    for (int h = 0; h < NW; ++h)
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          if constexpr (FMT == kQ8) {
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              uint32_t lo, hi;
              q8_pairs(buf.w[h][u][c][d], lo, hi);
#pragma unroll
              for (int m = 0; m < MMAX; ++m)
                acc[h][u][m] =
                    dot2(hi, xr[m][c][2 * d + 1], dot2(lo, xr[m][c][2 * d], acc[h][u][m]));
            }
          } else {
            constexpr int SPC = GM == kG16 ? 2 : 1;
            float part[SPC][MMAX];
#pragma unroll
            for (int g = 0; g < SPC; ++g)
#pragma unroll
              for (int m = 0; m < MMAX; ++m) part[g][m] = 0.0f;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              uint32_t q[4];
              q4_pairs(buf.w[h][u][c][d], q);
              const int g = GM == kG16 ? (d >> 1) : 0;
#pragma unroll
              for (int m = 0; m < MMAX; ++m) {
                float t = part[g][m];
                t = dot2(q[0], xr[m][c][4 * d + 0], t);
                t = dot2(q[1], xr[m][c][4 * d + 1], t);
                t = dot2(q[2], xr[m][c][4 * d + 2], t);
                t = dot2(q[3], xr[m][c][4 * d + 3], t);
                part[g][m] = t;
              }
            }
#pragma unroll
            for (int g = 0; g < SPC; ++g)
#pragma unroll
              for (int m = 0; m < MMAX; ++m)
                acc[h][u][m] = fmaf(part[g][m],
                                    scale_at(buf.s[h][u][c * SPC + g],
                                             toff + u_scale_bytes(p, u) + o.s[c * SPC + g], scl16),
                                    acc[h][u][m]);
          }
        }

    // The next tile's loads, issued just before this call, go out one at a
    // time between groups of these dot products: a burst of them would hold
    // the wave at the memory-instruction queue while its VALU work waits.
#pragma unroll
    for (int i = 0; i < kLoadsPerTile; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one VMEM read
      __builtin_amdgcn_sched_group_barrier(0x002, kValuPerLoad, 0);
    }

#pragma unroll
    for (int h = 0; h < NW; ++h)
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int m = 0; m < MMAX; ++m) {
          float v = group_sum<LPR>(acc[h][u][m]);
          if constexpr (FMT == kQ8)
            v *= scale_at(buf.s[h][u][0], toff + u_scale_bytes(p, u) + o.s[0], scl16);
          acc[h][u][m] = v;
        }

    const bool yf32 = (p.flags & kFlagYf32) != 0;
    char* yb = (char*)mt.y + cu.b * mt.y_bstride * (yf32 ? 4 : 2);
    const char* rb =
        mt.res ? (const char*)mt.res + cu.b * mt.r_bstride * (yf32 ? 4 : 2) : nullptr;
    const int rlim = row_limit(mt, cu);
    // the LM head stores the wave's own rows, Pack4 padding included
    const int rstore = ARGMAX && cu.rend < mt.n_store ? cu.rend : mt.n_store;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = row0(cu) + u * SLOTS + slot;
#pragma unroll
      for (int m = 0; m < MMAX; ++m) {
        float v = 0.0f;
        const bool live = r < rlim && m < p.m;
        if constexpr (ARGMAX) {
          // no C and no residual (host-checked); the logits wait in LDS until
          // the tile loop ends, so the loop issues loads only
          if (live) v = argmax_epilogue(p, acc[0][u][m]);
          const int li = (r - lg_r0) * MMAX + m;
          if (sub == ((u * MMAX + m) & (LPR - 1)) && r < rstore && m < p.m &&
              li < kArgLogitsMax)
            lg[li] = v;
          if (sub == 0 && live) argmax_merge(bv[m], bi[m], bs[m], argmax_logit(p, v), r, -INFINITY);
          continue;
        }
        if (live) {
          v = gemm_epilogue(p, m, r, acc[0][u][m]);
          if constexpr (PAIR) v = silu(v) * gemm_epilogue(p, m, r, acc[1][u][m]);
          if (rb && (p.flags & kFlagResidual)) {
            if (MMAX == 1 && !yf32) {
              v += (float)as_h2(buf.r[u])[0];
            } else {
              const long long ri = (long long)m * p.r_rstride + r;
              v += yf32 ? ((const float*)rb)[ri] : (float)((const f16*)rb)[ri];
            }
          }
        }
        // one lane per row stores; the lanes of a slot hold identical values
        if (sub == ((u * MMAX + m) & (LPR - 1)) && r < mt.n_store && m < p.m && mt.y) {
          const long long yi = out_index(p, mt, m, r);
          if (yf32)
            ((float*)yb)[yi] = v;
          else
            ((f16*)yb)[yi] = (f16)v;
        }
      }
    }
  }
};

// Resident waves per SIMD the register budget is sized for: 4 (128 VGPRs)
// for the lean M = 1 shapes, fewer where the tile's registers need more.
template <int FMT, int CPL, int MMAX, bool PAIR, int GM>
constexpr int qmv_waves_per_eu() {
  if (MMAX > 1 || (FMT == kQ4 && CPL >= 4) || (PAIR && CPL >= 4)) return 2;
  return FMT == kQ4 && GM == kG16 ? 3 : 4;
}

template <int FMT, int LPR, int CPL, int U, int MMAX, bool PAIR, bool ARGMAX, int GM>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(qmv_waves_per_eu<FMT, CPL, MMAX, PAIR, GM>())))
void qmv_kernel(const QmvParams p) {
  using Q = Qmv<FMT, LPR, CPL, U, MMAX, PAIR, ARGMAX, GM>;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane & (LPR - 1), slot = lane / LPR;
  const int gw = blockIdx.x * kWaves + wave;
  const int nw = gridDim.x * kWaves;
  // The LM head splits its rows (Pack4 padding included) evenly over the
  // waves, so that no wave streams more than one row above the average; its
  // tiles start at the range's first row and the last one stops at its end.
  // Other launches split whole tiles.
  const int n_rows = ARGMAX ? p.mat[0].n_store : 0;
  const int wr0 = ARGMAX ? (int)((long long)gw * n_rows / nw) : 0;
  const int wr1 = ARGMAX ? (int)((long long)(gw + 1) * n_rows / nw) : 0;
  const int t0 = ARGMAX ? 0 : (int)((long long)gw * p.total_tiles / nw);
  const int t1 = ARGMAX ? (wr1 - wr0 + Q::RW - 1) / Q::RW
                        : (int)((long long)(gw + 1) * p.total_tiles / nw);

  float bv[MMAX], bs[MMAX];
  int bi[MMAX];
#pragma unroll
  for (int m = 0; m < MMAX; ++m) {
    bv[m] = __builtin_nanf("");
    bi[m] = 0x7fffffff;
    bs[m] = -INFINITY;
  }

  // a wave without tiles (t0 == t1) still takes part in the staging barrier
  const bool has_tiles = t0 < t1;
  // the LM head's logits of this workgroup's rows (its waves' row ranges are
  // contiguous), stored after the tile loop
  __shared__ float s_lg[ARGMAX ? kArgLogitsMax : 1];
  const int lg_r0 = ARGMAX ? (int)((long long)blockIdx.x * kWaves * n_rows / nw) : 0;
  float* const lg = ARGMAX ? s_lg : nullptr;
  const typename Q::Offsets o = Q::offsets(p, sub, slot);
  typename Q::Cursor cu = Q::locate(p, has_tiles ? t0 : 0);
  if constexpr (ARGMAX) cu = typename Q::Cursor{0, 0, wr0, wr1};
  typename Q::Buf A, B;
  typename Q::XRegs xr;
  const f16* xcur = (const f16*)p.mat[cu.j].x + cu.b * p.mat[cu.j].x_bstride;
  bool staged = false;
  if constexpr (MMAX == 1) {
    if (p.flags & kFlagXShared) {
      typename Q::Stage st;
      Q::stage_issue(p, st);
      __builtin_amdgcn_sched_barrier(0);  // the staging loads go out before the codes
      Q::load(p, cu, o, A, has_tiles, slot);
      Q::stage_finish(p, st, lane, wave);
      Q::load_x_staged(p, sub, xr);
      staged = true;
    }
  }
  if (!staged) {
    Q::load(p, cu, o, A, has_tiles, slot);
    if (has_tiles) Q::load_x(p, xcur, sub, xr);
  }

  if (has_tiles) {
    // Tiles alternate between two register sets: while one is consumed, the
    // next tile's loads are in flight in the other.  The loop takes tiles in
    // pairs and leaves only at its head, and an odd last tile is consumed
    // after it: with no exit between the halves, the wait counts the
    // compiler places at the loop head see just the loads of the tile in A
    // (an exit path joining the back edge would add B's loads, pending, and
    // turn the head's register reuse into a wait for the whole prefetch).
    // Activation rows change only between batch entries of a batched x (a
    // cold path).
    auto next_x = [&]() {
      if constexpr (!ARGMAX) {
        const f16* xp = (const f16*)p.mat[cu.j].x + cu.b * p.mat[cu.j].x_bstride;
        if (__builtin_expect(xp != xcur, 0)) {
          Q::load_x(p, xp, sub, xr);
          xcur = xp;
        }
      }
    };
    int t = t0;
    while (t + 1 < t1) {
      // tile t is in A; tile t+1's loads go into B
      typename Q::Cursor nx = Q::advance(p, cu);
      Q::load(p, nx, o, B, true, slot);
      Q::compute(p, cu, o, A, xr, sub, slot, bv, bi, bs, lg, lg_r0);
      cu = nx;
      next_x();
      // tile t+1 is in B; tile t+2's loads (against empty resources past the
      // last tile) go into A
      const bool more = t + 2 < t1;
      nx = more ? Q::advance(p, cu) : cu;
      Q::load(p, nx, o, A, more, slot);
      Q::compute(p, cu, o, B, xr, sub, slot, bv, bi, bs, lg, lg_r0);
      cu = nx;
      next_x();
      t += 2;
    }
    if (t < t1) Q::compute(p, cu, o, A, xr, sub, slot, bv, bi, bs, lg, lg_r0);
  }

  if constexpr (ARGMAX) {
    // every workgroup (also one whose waves had no tiles) writes one partial
    // per row m: its waves' partials merged through LDS
    __shared__ float lv[MMAX][kWaves], ls[MMAX][kWaves];
    __shared__ int li[MMAX][kWaves];
#pragma unroll
    for (int m = 0; m < MMAX; ++m) {
      float v = bv[m], s = bs[m];
      int i = bi[m];
      argmax_wave_reduce(v, i, s);
      if (lane == 0) {
        lv[m][wave] = v;
        li[m][wave] = i;
        ls[m][wave] = s;
      }
    }
    __syncthreads();
    {
      const QmvMat& mt = p.mat[0];
      const int lg_r1 = (int)((long long)(blockIdx.x + 1) * kWaves * n_rows / nw);
      const int rows_x_m = (lg_r1 - lg_r0) * MMAX;
      const int cnt = rows_x_m < kArgLogitsMax ? rows_x_m : kArgLogitsMax;
      if (mt.y) {
        const bool yf32 = (p.flags & kFlagYf32) != 0;
        for (int i = threadIdx.x; i < cnt; i += kThreads) {
          const int r = lg_r0 + i / MMAX, m = i % MMAX;
          if (r < mt.n_store && m < p.m) {
            const long long yi = out_index(p, mt, m, r);
            if (yf32)
              ((float*)mt.y)[yi] = s_lg[i];
            else
              ((f16*)mt.y)[yi] = (f16)s_lg[i];
          }
        }
      }
    }
    // the launch's tag, read only now: a load issued at the start would sit
    // ahead of the weight loads in the memory counter, and the first wait
    // for them would wait for this agent-coherent round trip too
    const uint32_t tag = argmax_tag(p);
    if (threadIdx.x < MMAX && (int)threadIdx.x < p.m) {
      const int m = threadIdx.x;
      float v = lv[m][0], s = ls[m][0];
      int i = li[m][0];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) argmax_merge(v, i, s, lv[m][w], li[m][w], ls[m][w]);
      argmax_partial_store(p, (long long)m * p.parts + blockIdx.x, v, i, s, tag);
    }
    argmax_tail<4>(p, tag);
  }
}

}  // namespace aexq
