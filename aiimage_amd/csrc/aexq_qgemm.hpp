// Tiled quantized GEMM for M > 32 activation rows on gfx950 MFMA:
// Y[M][N] = X[M][K] W[N][K]^T for Q8 with one scale per row and Q4 with one
// scale per multiple of 32 codes, K a multiple of 64.
//
// A workgroup owns one output tile: BM activation rows by 128 weight rows (a
// SwiGLU pair: 64 gate rows and the same 64 up rows).  Per 64-wide K step its
// 256 threads fetch the step's codes once -- each thread the 32 codes of one
// row that one 16-byte (Q4) or two (Q8) loads bring -- expand them to exact
// fp16 integers and store them in LDS beside the step's activation tile.  The
// four waves (2 x 2, each BM/2 rows by 64 weight rows) then run
// v_mfma_f32_16x16x32_f16 from LDS.  One Q4 scale group is one MFMA K extent,
// so a group's product is scaled in fp32 into the accumulator and the
// dequantised weight stays exactly float(q) * scale; Q8 accumulates the whole
// row in the MFMA and applies its row scale once.  The next step's global
// loads are in flight while the current step's MFMAs run; LDS is
// double-buffered with one barrier per step.
//
// Workgroup b runs on XCD b % 8: the numbering puts the BM-row tiles of one
// weight tile on one XCD, whose L2 then fetches that weight tile once.
//
// MFMA 16x16x32 f16 lane layout (lane l): A[l % 16][8 (l / 16) + j],
// B[8 (l / 16) + j][l % 16], D[4 (l / 16) + r][l % 16], j < 8, r < 4.
#pragma once

#include "aexq_qmm.hpp"

namespace aexq {

template <int FMT, int BM, bool PAIR, bool SF16>
struct QGemm {
  static constexpr int BN = 128;                     // weight rows of a tile
  static constexpr int BK = 64;                      // K per step
  static constexpr int NOUT = PAIR ? BN / 2 : BN;    // output columns of a tile
  static constexpr int WM = BM / 2;                  // activation rows per wave
  static constexpr int TM = WM / 16;                 // 16-row A blocks per wave
  static constexpr int TN = 4;                       // 16-row B blocks per wave
  static constexpr int LS = BK + 8;                  // LDS row stride in halves (144 bytes)
  static constexpr int XV = BM * BK / 8 / kThreads;  // 16-byte activation loads per thread
  static constexpr int CV = FMT == kQ8 ? 2 : 1;      // 16-byte code loads per thread

  struct Regs {
    u32x4 x[XV];
    u32x4 c[CV];
    uint32_t s;  // Q4: raw bits of the thread's group scale
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

  // Issues the global loads of step st (rows past M or N read 0).
  static __device__ __forceinline__ void load(const QmvParams& p, const Src& s, int st, int tid,
                                              Regs& r) {
#pragma unroll
    for (int v = 0; v < XV; ++v) {
      const int c = tid + kThreads * v;
      r.x[v] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     s.xr, (c >> 3) * s.rs2 + (st * BK + (c & 7) * 8) * 2, 0, 0));
    }
    if constexpr (FMT == kQ8) {
#pragma unroll
      for (int i = 0; i < CV; ++i)
        r.c[i] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       s.wr, s.brl * s.rb + st * BK + 32 * s.sub + 16 * i, 0, 0));
      r.s = 0;
    } else {
      r.c[0] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(s.wr, s.brl * s.rb + st * 32 + 16 * s.sub,
                                                       0, 0));
      const int g = (st * BK + 32 * s.sub) / p.group;
      const int si = s.brl * p.groups_per_row + g;
      if constexpr (SF16)
        r.s = __builtin_amdgcn_raw_buffer_load_b16(s.sr, si * 2, 0, 0);
      else
        r.s = __builtin_amdgcn_raw_buffer_load_b32(s.sr, si * 4, 0, 0);
    }
  }

  // Stores a step's registers into LDS buffer (xs, ws, ss): the activation
  // chunks as loaded, the codes as exact fp16 integers in K order.
  static __device__ __forceinline__ void store(int tid, const Regs& r, f16* xs, f16* ws,
                                               float* ss) {
#pragma unroll
    for (int v = 0; v < XV; ++v) {
      const int c = tid + kThreads * v;
      *(u32x4*)&xs[(c >> 3) * LS + (c & 7) * 8] = r.x[v];
    }
    const int row = tid >> 1, sub = tid & 1;
    f16* dst = ws + row * LS + 32 * sub;
    if constexpr (FMT == kQ8) {
#pragma unroll
      for (int i = 0; i < CV; ++i) {
        uint32_t e[8];
#pragma unroll
        for (int w = 0; w < 4; ++w) q8_pairs(r.c[i][w], e[2 * w], e[2 * w + 1]);
        *(u32x4*)&dst[16 * i] = u32x4{e[0], e[1], e[2], e[3]};
        *(u32x4*)&dst[16 * i + 8] = u32x4{e[4], e[5], e[6], e[7]};
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t q[4];
        q4_pairs(r.c[0][i], q);  // (n0, n4), (n1, n5), (n2, n6), (n3, n7)
        u32x4 o;
        o[0] = __builtin_amdgcn_perm(q[1], q[0], 0x05040100u);  // (n0, n1)
        o[1] = __builtin_amdgcn_perm(q[3], q[2], 0x05040100u);  // (n2, n3)
        o[2] = __builtin_amdgcn_perm(q[1], q[0], 0x07060302u);  // (n4, n5)
        o[3] = __builtin_amdgcn_perm(q[3], q[2], 0x07060302u);  // (n6, n7)
        *(u32x4*)&dst[8 * i] = o;
      }
      ss[row * 2 + sub] = scale_of(r.s, SF16);
    }
  }

  // The MFMAs of one step from LDS buffer (xs, ws, ss).
  static __device__ __forceinline__ void compute(int lane, int wm, int wn, const f16* xs,
                                                 const f16* ws, const float* ss,
                                                 f32x4 (&acc)[TM][TN]) {
    const int l16 = lane & 15, lk = lane >> 4;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      f16x8 a[TM], bq[TN];
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
        a[tm] = *(const f16x8*)&xs[(wm * WM + 16 * tm + l16) * LS + 32 * kk + 8 * lk];
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
        bq[tn] = *(const f16x8*)&ws[(brow(wn, tn) + l16) * LS + 32 * kk + 8 * lk];
      if constexpr (FMT == kQ8) {
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
          for (int tn = 0; tn < TN; ++tn)
            acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[tm], bq[tn], acc[tm][tn], 0, 0, 0);
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
        // one MFMA, then the four scale FMAs of an earlier one: short-lived products
#pragma unroll
        for (int i = 0; i < TM * TN; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
        }
        __builtin_amdgcn_sched_barrier(0);  // one group's fragments live at a time
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
            const long long yi = (long long)m * mt.y_rstride + n;
            if (yf32)
              ((float*)yb)[yi] = v;
            else
              ((f16*)yb)[yi] = (f16)v;
          }
        }
    }
  }
};

template <int FMT, int BM, bool PAIR, bool SF16>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void qgemm_kernel(const QmvParams p, int mtiles) {
  using G = QGemm<FMT, BM, PAIR, SF16>;
  __shared__ __align__(16) f16 xs[2][BM * G::LS];
  __shared__ __align__(16) f16 ws[2][G::BN * G::LS];
  __shared__ float ss[2][G::BN * 2];
  // weight tile tn and row tile tm of this workgroup (see the header)
  const int bid = blockIdx.x, i = bid >> 3;
  const int tn = (i / mtiles) * 8 + (bid & 7), tm = i - (i / mtiles) * mtiles;
  if (tn >= p.total_tiles) return;
  int j = 0;
  for (int q = 1; q < p.nmat; ++q)
    if (tn >= p.mat[q].tile_base) j = q;
  const QmvMat& mt = p.mat[j];
  const int local = tn - mt.tile_base;
  const int b = local / mt.tiles;
  const int n0 = (local - b * mt.tiles) * G::NOUT;
  const int m0 = tm * BM;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const typename G::Src src = G::source(p, mt, b, n0, m0, tid, wave);
  const int steps = p.k / G::BK;

  f32x4 acc[G::TM][G::TN];
#pragma unroll
  for (int a = 0; a < G::TM; ++a)
#pragma unroll
    for (int c = 0; c < G::TN; ++c) acc[a][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  typename G::Regs r;
  G::load(p, src, 0, tid, r);
  G::store(tid, r, xs[0], ws[0], ss[0]);
  __syncthreads();
  for (int st = 0; st < steps; ++st) {
    const int cur = st & 1;
    const bool more = st + 1 < steps;
    if (more) G::load(p, src, st + 1, tid, r);
    __builtin_amdgcn_sched_barrier(0);  // the next step's loads stay ahead of the MFMAs
    G::compute(lane, wm, wn, xs[cur], ws[cur], ss[cur], acc);
    if (more) G::store(tid, r, xs[cur ^ 1], ws[cur ^ 1], ss[cur ^ 1]);
    __syncthreads();
  }
  G::finish(p, mt, b, n0, m0, lane, wm, wn, acc);
}

}  // namespace aexq
