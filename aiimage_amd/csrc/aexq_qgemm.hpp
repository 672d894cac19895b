// Tiled quantized GEMM for M > 32 activation rows on gfx950 MFMA:
// Y[M][N] = X[M][K] W[N][K]^T for Q8 with one scale per row and Q4 with one
// scale per multiple of 32 codes, K a multiple of 64.
//
// A workgroup owns one output tile: BM activation rows by 128 weight rows (a
// SwiGLU pair: 64 gate rows and the same 64 up rows).  Per 64-wide K step its
// 256 threads fetch the step's codes once -- each thread the 32 codes of one
// row that one 16-byte (Q4) or two (Q8) loads bring -- and store them in LDS
// as they are (in fragment order), beside the step's activation tile.  The four waves (2 x 2, each
// BM/2 rows by 64 weight rows) read their MFMA B fragments as raw codes (8
// bytes per lane for Q8, 4 for Q4: LDS carries a half or a quarter of what
// fp16 weights would), expand them to exact fp16 integers in registers and run
// v_mfma_f32_16x16x32_f16.  Q4 nibbles expand in (p, p + 4) pair order, so the
// Q4 activation tile is stored in that order too (the products pair up as in
// K order).  One Q4 scale group is one MFMA K extent: a group's product is
// scaled in fp32 into the accumulator, so the dequantised weight stays exactly
// float(q) * scale; Q8 accumulates the whole row in the MFMA and applies its
// row scale once.  With SPLIT (Q4, fp16 scales of magnitude <= 4096) the scale
// goes into B instead: s = s_hi + s_lo with s_hi the top 7 significand bits,
// and q * s_hi, q * s_lo are exact fp16 values (|q| <= 8 has at most 3
// significant bits), so two MFMAs accumulate x * (q * s) exactly in the fp32
// accumulator with no per-output scaling -- the B expansion is shared by the
// tile's BM / 32 A blocks, where the per-group FMAs were per output.  Global
// loads are issued two steps ahead of the MFMAs (two register sets); LDS is
// double-buffered with one barrier per step.  (In the conditional loop the
// compiler's wait before each LDS store also covers the loads issued just
// before it; the exact-wait form measured slower for these tiles.)
//
// G16 (Q4 with one scale per 16 codes, the reference's shipping format): an
// MFMA K extent holds two groups, lanes l / 16 = 0, 1 the first and 2, 3 the
// second; two MFMAs, each with the other group's lanes' codes zeroed, give
// the two groups' products, each scaled in fp32 into the accumulator -- the
// same exact float(q) * scale at twice the MFMA work.
//
// Workgroup b runs on XCD b % 8: the numbering puts the BM-row tiles of one
// weight tile on one XCD, whose L2 then fetches that weight tile once.
//
// MFMA 16x16x32 f16 lane layout (lane l): A[l % 16][8 (l / 16) + j],
// B[8 (l / 16) + j][l % 16], D[4 (l / 16) + r][l % 16], j < 8, r < 4.
#pragma once

#include "aexq_qmm.hpp"

namespace aexq {

template <int FMT, int BM, bool PAIR, bool SF16, bool SPLIT, bool G16>
struct QGemm {
  static_assert(!SPLIT || (FMT == kQ4 && SF16), "split scales are for Q4 with fp16 scales");
  static_assert(!G16 || (FMT == kQ4 && !SPLIT), "16-code groups are a Q4 per-group form");
  static constexpr int GS = G16 ? 4 : 2;             // Q4 scale groups per K step
  static constexpr int BN = 128;                     // weight rows of a tile
  static constexpr int BK = 64;                      // K per step
  static constexpr int NOUT = PAIR ? BN / 2 : BN;    // output columns of a tile
  static constexpr int WM = BM / 2;                  // activation rows per wave
  static constexpr int TM = WM / 16;                 // 16-row A blocks per wave
  static constexpr int TN = 4;                       // 16-row B blocks per wave
  static constexpr int LS = BK + 8;                  // activation LDS row stride in halves (144 B)
  // Code tile in LDS, fragment-major: piece (row, group kk, quarter lk) -- the
  // P bytes holding codes 32 kk + 8 lk .. + 7 of the row -- sits at
  //   kk * KB + (row / 16) * 64 P + lk * 16 P + (row % 16) * P,
  // so the 64 lanes of a fragment read take one contiguous run, and group 1
  // is skewed by 64 bytes so the two groups' stores fall on different banks.
  static constexpr int P = FMT == kQ8 ? 8 : 4;
  static constexpr int KB = (BN / 16) * 64 * P + 64;
  static constexpr int CB = 2 * KB;  // bytes of one code buffer
  static constexpr int XV = BM * BK / 8 / kThreads;  // 16-byte activation loads per thread
  static constexpr int CV = FMT == kQ8 ? 2 : 1;      // 16-byte code loads per thread

  struct Regs {
    u32x4 x[XV];
    u32x4 c[CV];
    uint32_t s[G16 ? 2 : 1];  // Q4: raw bits of the thread's group scale(s)
  };

  // Per-workgroup resources of one tile (wave-uniform).
  struct Src {
    __amdgpu_buffer_rsrc_t xr, wr, sr;
    int rs2;   // bytes between activation rows
    int rb;    // code bytes per weight row
    int brl;   // this thread's row inside its weight resource
    int sub;   // Q4: group of the step; Q8: half of the step's codes
  };

  // Weight rows of B block tn for wave column wn (rows of the tile's LDS block).
  static __device__ __forceinline__ int brow(int wn, int tn) {
    if constexpr (PAIR) return ((tn & 2) ? 64 : 0) + 32 * wn + 16 * (tn & 1);
    return 64 * wn + 16 * tn;
  }

  static __device__ __forceinline__ Src source(const QmvParams& p, const QmvMat& mt, int b,
                                               int n0, int m0, int tid, int wave) {
    Src s;
    const int row = tid >> 1;             // 0..127: the tile row this thread fetches
    const bool up = PAIR && wave >= 2;    // rows 64..127 of a pair tile: the up weight
    s.sub = tid & 1;
    s.brl = PAIR ? (row & 63) : row;
    s.rb = FMT == kQ8 ? p.k : p.k / 2;
    constexpr int sb = SF16 ? 2 : 4;
    const int rows = mt.n > n0 ? min(mt.n - n0, NOUT) : 0;
    const char* wb = (const char*)(up ? mt.w2 : mt.w) + (long long)b * mt.w_bstride * 4 +
                     (long long)n0 * s.rb;
    s.wr = __builtin_amdgcn_make_buffer_rsrc((void*)wb, (short)0, rows * s.rb, kBufferRsrcWord3);
    const char* sp = (const char*)(up ? mt.s2 : mt.s) +
                     ((long long)b * mt.s_bstride + (long long)n0 * p.groups_per_row) * sb;
    s.sr = __builtin_amdgcn_make_buffer_rsrc((void*)sp, (short)0,
                                             FMT == kQ8 ? 0 : rows * p.groups_per_row * sb,
                                             kBufferRsrcWord3);
    s.rs2 = (int)(p.x_rstride * 2);
    const char* xb = (const char*)mt.x + (long long)b * mt.x_bstride * 2 + (long long)m0 * s.rs2;
    const int mrows = p.m - m0 < BM ? p.m - m0 : BM;
    s.xr = __builtin_amdgcn_make_buffer_rsrc((void*)xb, (short)0, mrows * s.rs2,
                                             kBufferRsrcWord3);
    return s;
  }

  // Issues the global loads of step st (rows past M or N read 0).  A step
  // past the thread's range (live false) is still issued, at an offset past
  // every resource's end, so it reads zeros without a memory access: loads
  // issued on every path keep the compiler's wait counts exact, where a
  // skipped load makes the wait before a store also cover the loads issued
  // after it (the prefetch distance would drop to one step).
  static __device__ __forceinline__ void load(const QmvParams& p, const Src& s, int st, bool live,
                                              int tid, Regs& r) {
    const int oob = live ? 0 : (1 << 30);
#pragma unroll
    for (int v = 0; v < XV; ++v) {
      const int c = tid + kThreads * v;
      r.x[v] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     s.xr, oob + (c >> 3) * s.rs2 + (st * BK + (c & 7) * 8) * 2, 0, 0));
    }
    if constexpr (FMT == kQ8) {
#pragma unroll
      for (int i = 0; i < CV; ++i)
        r.c[i] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       s.wr, oob + s.brl * s.rb + st * BK + 32 * s.sub + 16 * i, 0, 0));
      r.s[0] = 0;
    } else {
      r.c[0] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     s.wr, oob + s.brl * s.rb + st * 32 + 16 * s.sub, 0, 0));
      const int g = (st * BK + 32 * s.sub) / p.group;
      const int si = oob / 4 + s.brl * p.groups_per_row + g;
      if constexpr (G16) {
        // the two 16-code groups of the thread's 32 codes (si even: aligned)
        if constexpr (SF16) {
          const uint32_t v = __builtin_amdgcn_raw_buffer_load_b32(s.sr, si * 2, 0, 0);
          r.s[0] = v & 0xFFFFu;
          r.s[1] = v >> 16;
        } else {
          typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
          const u32x2 v =
              __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(s.sr, si * 4, 0, 0));
          r.s[0] = v[0];
          r.s[1] = v[1];
        }
      } else if constexpr (SF16) {
        r.s[0] = __builtin_amdgcn_raw_buffer_load_b16(s.sr, si * 2, 0, 0);
      } else {
        r.s[0] = __builtin_amdgcn_raw_buffer_load_b32(s.sr, si * 4, 0, 0);
      }
    }
  }

  // Stores a step's registers into LDS buffer (xs, wc, ss): the activation
  // chunks (Q4: in the pair order of q4_pairs) and the codes as loaded.
  static __device__ __forceinline__ void store(int tid, const Regs& r, f16* xs, uint8_t* wc,
                                               float* ss) {
#pragma unroll
    for (int v = 0; v < XV; ++v) {
      const int c = tid + kThreads * v;
      u32x4 xv = r.x[v];
      if constexpr (FMT == kQ4) {
        uint32_t xp[4];
        q4_xpairs(xv[0], xv[1], xv[2], xv[3], xp);
        xv = u32x4{xp[0], xp[1], xp[2], xp[3]};
      }
      *(u32x4*)&xs[(c >> 3) * LS + (c & 7) * 8] = xv;
    }
    const int row = tid >> 1, sub = tid & 1;  // the thread holds group `sub` of the step
    uint8_t* dst = wc + sub * KB + (row >> 4) * 64 * P + (row & 15) * P;
#pragma unroll
    for (int lk = 0; lk < 4; ++lk) {
      if constexpr (FMT == kQ8) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x4& c = r.c[lk >> 1];
        *(u32x2*)&dst[lk * 16 * P] = u32x2{c[2 * (lk & 1)], c[2 * (lk & 1) + 1]};
      } else {
        *(uint32_t*)&dst[lk * 16 * P] = r.c[0][lk];
      }
    }
    if constexpr (SPLIT) {
      // (s_hi, s_lo): s_hi keeps the top 7 significand bits, s_lo = s - s_hi exactly
      const f16 sv = __builtin_bit_cast(f16, (uint16_t)r.s[0]);
      const f16 hi = __builtin_bit_cast(f16, (uint16_t)(r.s[0] & 0xFFF0u));
      const f16 lo = sv - hi;
      const f16x2 pr = {hi, lo};
      ((uint32_t*)ss)[row * 2 + sub] = as_u(pr);
    } else if constexpr (G16) {
      ss[row * 4 + 2 * sub] = scale_of(r.s[0], SF16);
      ss[row * 4 + 2 * sub + 1] = scale_of(r.s[1], SF16);
    } else if constexpr (FMT == kQ4) {
      ss[row * 2 + sub] = scale_of(r.s[0], SF16);
    }
  }

  // The MFMAs of one step from LDS buffer (xs, wc, ss).
  static __device__ __forceinline__ void compute(int lane, int wm, int wn, const f16* xs,
                                                 const uint8_t* wc, const float* ss,
                                                 f32x4 (&acc)[TM][TN]) {
    const int l16 = lane & 15, lk = lane >> 4;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      f16x8 a[TM], bq[TN];
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
        a[tm] = *(const f16x8*)&xs[(wm * WM + 16 * tm + l16) * LS + 32 * kk + 8 * lk];
      if constexpr (SPLIT) {
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
          const uint8_t* src =
              wc + kk * KB + (brow(wn, tn) >> 4) * 64 * P + lk * 16 * P + l16 * P;
          uint32_t e[4];
          q4_pairs(*(const uint32_t*)src, e);
          const f16x2 sp = as_h2(((const uint32_t*)ss)[(brow(wn, tn) + l16) * 2 + kk]);
          const f16x2 shi = {sp[0], sp[0]}, slo = {sp[1], sp[1]};
          const f16x8 bhi = pack8(as_u(as_h2(e[0]) * shi), as_u(as_h2(e[1]) * shi),
                                  as_u(as_h2(e[2]) * shi), as_u(as_h2(e[3]) * shi));
          const f16x8 blo = pack8(as_u(as_h2(e[0]) * slo), as_u(as_h2(e[1]) * slo),
                                  as_u(as_h2(e[2]) * slo), as_u(as_h2(e[3]) * slo));
#pragma unroll
          for (int tm = 0; tm < TM; ++tm) {
            acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[tm], bhi, acc[tm][tn], 0, 0, 0);
            acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[tm], blo, acc[tm][tn], 0, 0, 0);
          }
        }
        continue;
      }
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        // codes 32 kk + 8 lk .. + 7 of row brow + l16
        const uint8_t* src = wc + kk * KB + (brow(wn, tn) >> 4) * 64 * P + lk * 16 * P + l16 * P;
        if constexpr (FMT == kQ8) {
          typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
          const u32x2 raw = *(const u32x2*)src;
          uint32_t e0, e1, e2, e3;
          q8_pairs(raw[0], e0, e1);
          q8_pairs(raw[1], e2, e3);
          bq[tn] = pack8(e0, e1, e2, e3);
        } else {
          uint32_t e[4];
          q4_pairs(*(const uint32_t*)src, e);
          bq[tn] = pack8(e[0], e[1], e[2], e[3]);
        }
      }
      if constexpr (FMT == kQ8) {
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
          for (int tn = 0; tn < TN; ++tn)
            acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[tm], bq[tn], acc[tm][tn], 0, 0, 0);
      } else if constexpr (G16) {
        // group 2 kk in lanes lk < 2, group 2 kk + 1 in lanes lk >= 2
        // one B block's two operands at a time (register budget)
        const bool first = lk < 2;
        const f16x8 zero = {};
        const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
          const float s0 = ss[(brow(wn, tn) + l16) * 4 + 2 * kk];
          const float s1 = ss[(brow(wn, tn) + l16) * 4 + 2 * kk + 1];
          const f16x8 b0 = first ? bq[tn] : zero;
          const f16x8 b1 = first ? zero : bq[tn];
#pragma unroll
          for (int tm = 0; tm < TM; ++tm) {
            const f32x4 t0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[tm], b0, z, 0, 0, 0);
            const f32x4 t1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[tm], b1, z, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              acc[tm][tn][r] = fmaf(s0, t0[r], acc[tm][tn][r]);
              acc[tm][tn][r] = fmaf(s1, t1[r], acc[tm][tn][r]);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
        float sc[TN];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) sc[tn] = ss[(brow(wn, tn) + l16) * 2 + kk];
        const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
          for (int tn = 0; tn < TN; ++tn) {
            const f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[tm], bq[tn], z, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[tm][tn][r] = fmaf(sc[tn], t[r], acc[tm][tn][r]);
          }
        __builtin_amdgcn_sched_barrier(0);  // one group's products live at a time
      }
    }
  }

  // Row scale (Q8), epilogue and store of the finished tile.
  static __device__ __forceinline__ void finish(const QmvParams& p, const QmvMat& mt, int b,
                                                int n0, int m0, int lane, int wm, int wn,
                                                const f32x4 (&acc)[TM][TN]) {
    const int l16 = lane & 15, lk = lane >> 4;
    const bool yf32 = (p.flags & kFlagYf32) != 0;
    constexpr int sb = SF16 ? 2 : 4;
    char* yb = (char*)mt.y + (long long)b * mt.y_bstride * (yf32 ? 4 : 2);
    const char* rb =
        mt.res ? (const char*)mt.res + (long long)b * mt.r_bstride * (yf32 ? 4 : 2) : nullptr;
    constexpr int TO = PAIR ? TN / 2 : TN;  // output blocks per wave
#pragma unroll
    for (int to = 0; to < TO; ++to) {
      const int n = n0 + (PAIR ? 32 * wn + 16 * to : 64 * wn + 16 * to) + l16;
      float rs0 = 1.0f, rs1 = 1.0f;
      if constexpr (FMT == kQ8) {
        const char* s0 = (const char*)mt.s + (long long)b * mt.s_bstride * sb;
        rs0 = n < mt.n ? load_scale(s0, n, SF16) : 0.0f;
        if constexpr (PAIR) {
          const char* s1 = (const char*)mt.s2 + (long long)b * mt.s_bstride * sb;
          rs1 = n < mt.n ? load_scale(s1, n, SF16) : 0.0f;
        }
      }
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm * WM + 16 * tm + 4 * lk + r;
          if (m < p.m && n < mt.n_store && mt.y) {
            float v = 0.0f;
            if (n < mt.n) {
              v = gemm_epilogue(p, p.m_base + m, n, acc[tm][to][r] * rs0);
              if constexpr (PAIR)
                v = silu(v) * gemm_epilogue(p, p.m_base + m, n, acc[tm][to + 2][r] * rs1);
              if (rb && (p.flags & kFlagResidual)) {
                const long long ri = (long long)m * p.r_rstride + n;
                v += yf32 ? ((const float*)rb)[ri] : (float)((const f16*)rb)[ri];
              }
            }
            const long long yi = out_index(p, mt, m, n);
            if (yf32)
              ((float*)yb)[yi] = v;
            else
              ((f16*)yb)[yi] = (f16)v;
          }
        }
    }
  }

  // Split K: the thread's raw accumulators of K chunk c (no row scale, no
  // epilogue) into partial plane c.
  static __device__ __forceinline__ void spill(const QmvParams& p, const QmvMat& mt, int b,
                                               int n0, int m0, int lane, int wm, int wn, int c,
                                               const f32x4 (&acc)[TM][TN]) {
    const int l16 = lane & 15, lk = lane >> 4;
    constexpr int NW = PAIR ? 2 : 1;
    constexpr int TO = PAIR ? TN / 2 : TN;
    float* base = p.sk_part + (long long)c * p.sk_plane + mt.sk_off +
                  (long long)b * p.m * NW * mt.n_store;
#pragma unroll
    for (int to = 0; to < TO; ++to) {
      const int n = n0 + (PAIR ? 32 * wn + 16 * to : 64 * wn + 16 * to) + l16;
      if (n >= mt.n) continue;
#pragma unroll
      for (int h = 0; h < NW; ++h)
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = m0 + wm * WM + 16 * tm + 4 * lk + r;
            if (m < p.m) base[((long long)m * NW + h) * mt.n_store + n] = acc[tm][to + 2 * h][r];
          }
    }
  }
};

template <int FMT, int BM, bool PAIR, bool SF16, bool SPLIT, bool G16>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void qgemm_kernel(const QmvParams p, int mtiles) {
  using G = QGemm<FMT, BM, PAIR, SF16, SPLIT, G16>;
  __shared__ __align__(16) f16 xs[2][BM * G::LS];
  __shared__ __align__(16) uint8_t ws[2][G::CB];
  __shared__ float ss[2][FMT == kQ8 ? 1 : G::BN * G::GS];  // Q4 group scales of a step
  // weight tile tn, row tile tm and K chunk kc of this workgroup (see the
  // header; the chunks of a split K sit next to each other on one XCD)
  // (readfirstlane: the tile coordinates are workgroup-uniform, so the buffer
  // resources built from them stay in scalar registers)
  const int S = p.sk_chunks > 1 ? p.sk_chunks : 1;
  const int per = mtiles * S;
  const int bid = blockIdx.x, i = bid >> 3;
  const int tn = __builtin_amdgcn_readfirstlane((i / per) * 8 + (bid & 7));
  const int rem = i - (i / per) * per;
  const int tm = __builtin_amdgcn_readfirstlane(rem / S);
  const int kc = __builtin_amdgcn_readfirstlane(rem - (rem / S) * S);
  if (tn >= p.total_tiles) return;
  int j = 0;
  for (int q = 1; q < p.nmat; ++q)
    if (tn >= p.mat[q].tile_base) j = q;
  j = __builtin_amdgcn_readfirstlane(j);
  const QmvMat& mt = p.mat[j];
  const int local = tn - mt.tile_base;
  const int b = __builtin_amdgcn_readfirstlane(local / mt.tiles);
  const int n0 = __builtin_amdgcn_readfirstlane((local - b * mt.tiles) * G::NOUT);
  const int m0 = tm * BM;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const typename G::Src src = G::source(p, mt, b, n0, m0, tid, wave);
  const int steps = p.k / G::BK;
  const int cs = S > 1 ? p.sk_cs : steps;
  const int s0 = kc * cs, s1 = min(s0 + cs, steps);  // this workgroup's K steps
  if (s0 >= s1) return;

  f32x4 acc[G::TM][G::TN];
#pragma unroll
  for (int a = 0; a < G::TM; ++a)
#pragma unroll
    for (int c = 0; c < G::TN; ++c) acc[a][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  typename G::Regs ra, rb;
  if constexpr (!G16) {
    // Two register sets rotate: while LDS buffer (st & 1) is consumed, step
    // st + 1 waits in one set (stored after the MFMAs) and step st + 2 is being
    // fetched into the other, so a load has two steps of MFMAs to land.
    G::load(p, src, s0, true, tid, ra);
    if (s0 + 1 < s1) G::load(p, src, s0 + 1, true, tid, rb);
    G::store(tid, ra, xs[0], ws[0], ss[0]);
    __syncthreads();
    for (int st = s0;;) {
      if (st + 2 < s1) G::load(p, src, st + 2, true, tid, ra);
      __builtin_amdgcn_sched_barrier(0);  // the loads stay ahead of the MFMAs
      G::compute(lane, wm, wn, xs[0], ws[0], ss[0], acc);
      if (st + 1 < s1) G::store(tid, rb, xs[1], ws[1], ss[1]);
      __syncthreads();
      if (++st >= s1) break;
      if (st + 2 < s1) G::load(p, src, st + 2, true, tid, rb);
      __builtin_amdgcn_sched_barrier(0);
      G::compute(lane, wm, wn, xs[1], ws[1], ss[1], acc);
      if (st + 1 < s1) G::store(tid, ra, xs[0], ws[0], ss[0]);
      __syncthreads();
      if (++st >= s1) break;
    }
  } else {
    // Group 16: the same rotation in a counted loop, two steps per
    // iteration, with loads and stores on every path (past the range they
    // move zeros into the buffer that is no longer read): the compiler then
    // needs 128 registers here instead of 236 (four workgroups per CU
    // instead of two), and no wait before a store covers the loads issued
    // after it.  Buffer 0 holds step st and rb step st + 1 at the loop head.
    G::load(p, src, s0, true, tid, ra);
    G::load(p, src, s0 + 1, s0 + 1 < s1, tid, rb);
    G::store(tid, ra, xs[0], ws[0], ss[0]);
    __syncthreads();
    int st = s0;
    for (int it = (s1 - s0) >> 1; it > 0; --it) {
      G::load(p, src, st + 2, st + 2 < s1, tid, ra);
      __builtin_amdgcn_sched_barrier(0);
      G::compute(lane, wm, wn, xs[0], ws[0], ss[0], acc);
      G::store(tid, rb, xs[1], ws[1], ss[1]);
      __syncthreads();
      G::load(p, src, st + 3, st + 3 < s1, tid, rb);
      __builtin_amdgcn_sched_barrier(0);
      G::compute(lane, wm, wn, xs[1], ws[1], ss[1], acc);
      G::store(tid, ra, xs[0], ws[0], ss[0]);
      __syncthreads();
      st += 2;
    }
    if ((s1 - s0) & 1) G::compute(lane, wm, wn, xs[0], ws[0], ss[0], acc);
  }
  if (S == 1)
    G::finish(p, mt, b, n0, m0, lane, wm, wn, acc);
  else
    G::spill(p, mt, b, n0, m0, lane, wm, wn, kc, acc);
}

}  // namespace aexq
