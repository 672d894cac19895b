// Tiled quantized GEMM for M > 32 activation rows, register-staged: Q4 with
// one scale per larger multiple of 32 codes (64, 96, ...; the LDS-direct
// kernel of aexq_qgemm_dl.hpp covers Q8 and groups of 16 or 32), K a
// multiple of 64.  Y[M][N] = X[M][K] W[N][K]^T.
//
// A workgroup owns one output tile: 64 activation rows by 128 weight rows (a
// SwiGLU pair: 64 gate rows and the same 64 up rows).  Per 64-wide K step its
// 256 threads fetch the step's codes once -- each thread the 32 codes of one
// row that one 16-byte load brings -- and store them in LDS as they are (in
// fragment order), beside the step's activation tile.  The four waves (2 x 2,
// each 32 rows by 64 weight rows) read their MFMA B fragments as raw codes (4
// bytes per lane), expand them to exact fp16 integers in registers and run
// v_mfma_f32_16x16x32_f16.  Nibbles expand in (p, p + 4) pair order, so the
// activation tile is stored in that order too (the products pair up as in K
// order).  One 32-code MFMA K extent lies inside one scale group: its product
// is scaled in fp32 into the accumulator, so the dequantised weight stays
// exactly float(q) * scale.  Global loads are issued two steps ahead of the
// MFMAs (two register sets); LDS is double-buffered with one barrier per step.
//
// Workgroup b runs on XCD b % 8, which takes a contiguous range of tiles
// (gemm_block_tile): the row tiles of one weight tile, and the weight tiles
// of one copy, share that XCD's L2.
//
// MFMA 16x16x32 f16 lane layout (lane l): A[l % 16][8 (l / 16) + j],
// B[8 (l / 16) + j][l % 16], D[4 (l / 16) + r][l % 16], j < 8, r < 4.
#pragma once

#include "aexq_qmm.hpp"

namespace aexq {

template <bool PAIR, bool SF16>
struct QGemm {
  static constexpr int BM = 64;                      // activation rows of a tile
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
  static constexpr int P = 4;
  static constexpr int KB = (BN / 16) * 64 * P + 64;
  static constexpr int CB = 2 * KB;  // bytes of one code buffer
  static constexpr int XV = BM * BK / 8 / kThreads;  // 16-byte activation loads per thread

  struct Regs {
    u32x4 x[XV];
    u32x4 c;
    uint32_t s;  // raw bits of the thread's group scale
  };

  // Per-workgroup resources of one tile (wave-uniform).
  struct Src {
    __amdgpu_buffer_rsrc_t xr, wr, sr;
    int rs2;   // bytes between activation rows
    int rb;    // code bytes per weight row
    int brl;   // this thread's row inside its weight resource
    int sub;   // the thread's 32-code half of the step
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
    s.rb = p.k / 2;
    constexpr int sb = SF16 ? 2 : 4;
    const int rows = mt.n > n0 ? min(mt.n - n0, NOUT) : 0;
    const char* wb = (const char*)(up ? mt.w2 : mt.w) + (long long)b * mt.w_bstride * 4 +
                     (long long)n0 * s.rb;
    s.wr = __builtin_amdgcn_make_buffer_rsrc((void*)wb, (short)0, rows * s.rb, kBufferRsrcWord3);
    const char* sp = (const char*)(up ? mt.s2 : mt.s) +
                     ((long long)b * mt.s_bstride + (long long)n0 * p.groups_per_row) * sb;
    s.sr = __builtin_amdgcn_make_buffer_rsrc((void*)sp, (short)0, rows * p.groups_per_row * sb,
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
    r.c = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                        s.wr, oob + s.brl * s.rb + st * 32 + 16 * s.sub, 0, 0));
    const int g = (st * BK + 32 * s.sub) / p.group;
    const int si = oob / 4 + s.brl * p.groups_per_row + g;
    if constexpr (SF16)
      r.s = __builtin_amdgcn_raw_buffer_load_b16(s.sr, si * 2, 0, 0);
    else
      r.s = __builtin_amdgcn_raw_buffer_load_b32(s.sr, si * 4, 0, 0);
  }

  // Stores a step's registers into LDS buffer (xs, wc, ss): the activation
  // chunks (Q4: in the pair order of q4_pairs) and the codes as loaded.
  static __device__ __forceinline__ void store(int tid, const Regs& r, f16* xs, uint8_t* wc,
                                               float* ss) {
#pragma unroll
    for (int v = 0; v < XV; ++v) {
      const int c = tid + kThreads * v;
      const u32x4 xv = r.x[v];
      uint32_t xp[4];
      q4_xpairs(xv[0], xv[1], xv[2], xv[3], xp);
      *(u32x4*)&xs[(c >> 3) * LS + (c & 7) * 8] = u32x4{xp[0], xp[1], xp[2], xp[3]};
    }
    const int row = tid >> 1, sub = tid & 1;  // the thread holds group `sub` of the step
    uint8_t* dst = wc + sub * KB + (row >> 4) * 64 * P + (row & 15) * P;
#pragma unroll
    for (int lk = 0; lk < 4; ++lk) *(uint32_t*)&dst[lk * 16 * P] = r.c[lk];
    ss[row * 2 + sub] = scale_of(r.s, SF16);
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
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        // codes 32 kk + 8 lk .. + 7 of row brow + l16
        const uint8_t* src = wc + kk * KB + (brow(wn, tn) >> 4) * 64 * P + lk * 16 * P + l16 * P;
        uint32_t e[4];
        q4_pairs(*(const uint32_t*)src, e);
        bq[tn] = pack8(e[0], e[1], e[2], e[3]);
      }
      {
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

  // Epilogue and store of the finished tile.
  static __device__ __forceinline__ void finish(const QmvParams& p, const QmvMat& mt, int b,
                                                int n0, int m0, int lane, int wm, int wn,
                                                const f32x4 (&acc)[TM][TN]) {
    const int l16 = lane & 15, lk = lane >> 4;
    const bool yf32 = (p.flags & kFlagYf32) != 0;
    char* yb = (char*)mt.y + (long long)b * mt.y_bstride * (yf32 ? 4 : 2);
    const char* rb =
        mt.res ? (const char*)mt.res + (long long)b * mt.r_bstride * (yf32 ? 4 : 2) : nullptr;
    constexpr int TO = PAIR ? TN / 2 : TN;  // output blocks per wave
#pragma unroll
    for (int to = 0; to < TO; ++to) {
      const int n = n0 + (PAIR ? 32 * wn + 16 * to : 64 * wn + 16 * to) + l16;
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm * WM + 16 * tm + 4 * lk + r;
          if (m < p.m && n < mt.n_store && mt.y) {
            float v = 0.0f;
            if (n < mt.n) {
              v = gemm_epilogue(p, p.m_base + m, n, acc[tm][to][r]);
              if constexpr (PAIR) v = silu(v) * gemm_epilogue(p, p.m_base + m, n, acc[tm][to + 2][r]);
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

template <bool PAIR, bool SF16>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void qgemm_kernel(const QmvParams p, int mtiles) {
  using G = QGemm<PAIR, SF16>;
  constexpr int BM = G::BM;
  __shared__ __align__(16) f16 xs[2][BM * G::LS];
  __shared__ __align__(16) uint8_t ws[2][G::CB];
  __shared__ float ss[2][G::BN * 2];  // the group scales of a step
  // weight tile tn, row tile tm and K chunk kc of this workgroup (see the
  // header; the chunks of a split K sit next to each other on one XCD)
  // (readfirstlane: the tile coordinates are workgroup-uniform, so the buffer
  // resources built from them stay in scalar registers)
  const int S = p.sk_chunks > 1 ? p.sk_chunks : 1;
  const int per = mtiles * S;
  int tile, rem;
  gemm_block_tile(blockIdx.x, p.total_tiles, per, tile, rem);
  const int tn = __builtin_amdgcn_readfirstlane(tile);
  const int tm = __builtin_amdgcn_readfirstlane(rem / S);
  const int kc = __builtin_amdgcn_readfirstlane(rem - (rem / S) * S);
  if (tn < 0) return;
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
  if (S == 1)
    G::finish(p, mt, b, n0, m0, lane, wm, wn, acc);
  else
    G::spill(p, mt, b, n0, m0, lane, wm, wn, kc, acc);
}

}  // namespace aexq
