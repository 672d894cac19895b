// Small-M (2..32 rows per launch) quantized matmul on gfx950 MFMA: Y[M][N] = X[M][K] W[N][K]^T.
//
// Persistent waves, like the matvec: each wave owns a contiguous range of
// "steps" -- (weight tile of TN = 16 x NT rows, 128-wide K slice) pairs over
// every matrix and batch entry of the launch -- and keeps the next step's
// loads in flight while the current one is consumed.  Per step and 16-row
// weight block the four 16-lane rows of a wave read 64 contiguous code bytes
// of each weight row (16 bytes per lane) straight from HBM.  For Q4 a lane's
// 16 bytes are one 32-code group; a 4x4 dword transpose across the four lane
// rows (v_permlane32_swap / v_permlane16_swap) turns them into four MFMA B
// fragments that each cover exactly one scale group.  Codes
// become exact fp16 integers (q4_pairs / q8_pairs) and meet fp16 activations
// in v_mfma_f32_16x16x32_f16.  Q4 scales are applied in fp32 to each group's
// MFMA result (one group = one MFMA K-extent, so the dequantised weight is
// exactly float(q) * scale as in the reference); Q8 accumulates the whole row
// in the MFMA and applies its per-row scale once.  The scale dtype (fp16 /
// fp32) is a compile-time parameter: one static path per kernel.  Activations are read from
// L2 with a buffer resource whose bound zero-fills rows past M.
//
// MFMA 16x16x32 f16 lane layout (lane l): A[l % 16][8 (l / 16) + j],
// B[8 (l / 16) + j][l % 16], D[4 (l / 16) + r][l % 16], j < 8, r < 4.
#pragma once

#include <math.h>

#include "aexq_device.hpp"

namespace aexq {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// 4x4 transpose of dwords across the four 16-lane rows of a wave: on return,
// register q of row R holds what register R of row q held.
__device__ __forceinline__ void rows_transpose4(uint32_t& c0, uint32_t& c1, uint32_t& c2,
                                                uint32_t& c3) {
  const auto s02 = __builtin_amdgcn_permlane32_swap(c0, c2, false, false);
  const auto s13 = __builtin_amdgcn_permlane32_swap(c1, c3, false, false);
  const auto t0 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
  const auto t1 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
  c0 = t0[0];
  c1 = t0[1];
  c2 = t1[0];
  c3 = t1[1];
}

__device__ __forceinline__ f16x8 pack8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  const u32x4v v = {a, b, c, d};
  return __builtin_bit_cast(f16x8, v);
}

template <int FMT, int GM, int MT, int NT, bool PAIR, bool SF16>
struct Qmm {
  static constexpr int TN = 16 * NT;            // weight rows per tile
  static constexpr int NW = PAIR ? 2 : 1;
  static constexpr int WV = FMT == kQ8 ? 2 : 1;  // 16-byte code loads per 16-row block
  static constexpr int SV = FMT == kQ8 ? 1 : (GM == kG16 ? 2 : 1);  // 16-byte scale loads

  struct Cursor {
    int j, b, rt, s;  // matrix, batch entry, row tile, 128-wide K slice (wave-uniform)
  };

  struct Buf {
    u32x4 w[NW][NT][WV];
    u32x4 s[NW][NT][SV];
    u32x4 x[MT][4];
  };

  struct Acc {
    f32x4 v[NW][MT][NT];
  };

  static __device__ __forceinline__ Cursor locate(const QmvParams& p, int t) {
    const int steps = p.k / 128;
    const int tile = t / steps;
    int j = 0;
    for (int i = 1; i < p.nmat; ++i)
      if (tile >= p.mat[i].tile_base) j = i;
    const int local = tile - p.mat[j].tile_base;
    Cursor c;
    c.j = j;
    c.b = local / p.mat[j].tiles;
    c.rt = local - c.b * p.mat[j].tiles;
    c.s = t - tile * steps;
    return c;
  }

  static __device__ __forceinline__ Cursor advance(const QmvParams& p, Cursor c) {
    if (++c.s == p.k / 128) {
      c.s = 0;
      if (++c.rt == p.mat[c.j].tiles) {
        c.rt = 0;
        if (++c.b == p.batch) {
          c.b = 0;
          ++c.j;
        }
      }
    }
    return c;
  }

  // Issues every load of one step without a branch (buffer resources whose
  // bounds zero-fill rows past N and activation rows past M).
  static __device__ __forceinline__ void load(const QmvParams& p, const Cursor& cu, int lane,
                                              Buf& buf) {
    const QmvMat& mt = p.mat[cu.j];
    const int n_l = lane & 15, kb = lane >> 4;
    constexpr int sb = SF16 ? 2 : 4;
    const int row_bytes = FMT == kQ8 ? p.k : p.k / 2;
    const int r0 = cu.rt * TN;
    const int rows = mt.n > r0 ? mt.n - r0 : 0;
    // codes: base advanced to this K slice, bound shrunk by the same amount
    const int wstep = FMT == kQ8 ? 128 : 64;  // code bytes per K slice
    const int wnum = rows > 0 ? rows * row_bytes - cu.s * wstep : 0;
    // scales of this slice (Q4: 4 groups of 32 or 8 of 16 per slice; Q8: per row)
    const int gstep = FMT == kQ8 ? 0 : (GM == kG16 ? 8 : 4);
    const int sper = FMT == kQ8 ? 1 : p.groups_per_row;
    // +16: a 16-byte scale load of the last row's last slice may run past the
    // array's end into the upload's zeroed tail padding (its lanes are unused)
    const int snum = rows > 0 ? (rows * sper - cu.s * gstep) * sb + 16 : 0;
#pragma unroll
    for (int h = 0; h < NW; ++h) {
      const char* wb = (const char*)(h == 0 ? mt.w : mt.w2) + (cu.b * mt.w_bstride) * 4 +
                       (long long)r0 * row_bytes + cu.s * wstep;
      const char* sbp = (const char*)(h == 0 ? mt.s : mt.s2) +
                        (cu.b * mt.s_bstride + (long long)r0 * sper + cu.s * gstep) * sb;
      const __amdgpu_buffer_rsrc_t wr =
          __builtin_amdgcn_make_buffer_rsrc((void*)wb, (short)0, wnum, kBufferRsrcWord3);
      const __amdgpu_buffer_rsrc_t sr =
          __builtin_amdgcn_make_buffer_rsrc((void*)sbp, (short)0, snum, kBufferRsrcWord3);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int rr = 16 * nt + n_l;
        if constexpr (FMT == kQ8) {
          // codes 16 kb .. 16 kb + 15 and 64 + 16 kb .. 64 + 16 kb + 15 of the slice
          buf.w[h][nt][0] = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, rr * row_bytes + 16 * kb, 0,
                                                           kStreamAux));
          buf.w[h][nt][1] = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, rr * row_bytes + 16 * kb + 64, 0,
                                                           kStreamAux));
          buf.s[h][nt][0] = u32x4{0u, 0u, 0u, 0u};
        } else {
          // group 4 s + kb: 32 codes
          buf.w[h][nt][0] = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, rr * row_bytes + 16 * kb, 0,
                                                           kStreamAux));
#pragma unroll
          for (int v = 0; v < SV; ++v)
            buf.s[h][nt][v] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(sr, rr * sper * sb + 16 * v, 0, 0));
        }
      }
    }
    // activations of this slice
    const long long rs2 = p.x_rstride * 2;
    const char* xb = (const char*)mt.x + cu.b * mt.x_bstride * 2 + cu.s * 256;
    const int xnum = (int)(p.m * rs2) - cu.s * 256;
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc((void*)xb, (short)0, xnum, kBufferRsrcWord3);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const int off = (16 * m + n_l) * (int)rs2;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        // Q4: group q of the slice, 8 codes at 8 kb; Q8: the lane's B codes of MFMA q,
        // 8 at 16 kb + 8 q (q < 2) or 64 + 16 kb + 8 (q - 2)
        const int ko = FMT == kQ8 ? ((q >> 1) * 64 + 16 * kb + 8 * (q & 1)) : (32 * q + 8 * kb);
        buf.x[m][q] =
            __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off + 2 * ko, 0, 0));
      }
    }
  }

  static __device__ __forceinline__ float scale16(const u32x4& v, int i) {
    const uint32_t d = v[i >> 1];
    return (float)__builtin_bit_cast(f16, (uint16_t)(d >> ((i & 1) * 16)));
  }

  // Consumes one step: four 32-wide K groups.
  static __device__ __forceinline__ void compute(const QmvParams& p, int lane, const Buf& buf,
                                                 Acc& acc) {
    const int kb = lane >> 4;
    // B codes per (h, nt, group q): one dword per lane
    uint32_t code[NW][NT][4][WV == 2 ? 2 : 1];
#pragma unroll
    for (int h = 0; h < NW; ++h)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        if constexpr (FMT == kQ8) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const u32x4& src = buf.w[h][nt][q >> 1];
            code[h][nt][q][0] = src[2 * (q & 1)];
            code[h][nt][q][1] = src[2 * (q & 1) + 1];
          }
        } else {
          uint32_t c0 = buf.w[h][nt][0][0], c1 = buf.w[h][nt][0][1], c2 = buf.w[h][nt][0][2],
                   c3 = buf.w[h][nt][0][3];
          rows_transpose4(c0, c1, c2, c3);
          code[h][nt][0][0] = c0;
          code[h][nt][1][0] = c1;
          code[h][nt][2][0] = c2;
          code[h][nt][3][0] = c3;
        }
      }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // B fragments of group q
      f16x8 bf[NW][NT];
#pragma unroll
      for (int h = 0; h < NW; ++h)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          if constexpr (FMT == kQ8) {
            uint32_t a0, a1, b0, b1;
            q8_pairs(code[h][nt][q][0], a0, a1);
            q8_pairs(code[h][nt][q][1], b0, b1);
            bf[h][nt] = pack8(a0, a1, b0, b1);
          } else {
            uint32_t e[4];
            q4_pairs(code[h][nt][q][0], e);
            bf[h][nt] = pack8(e[0], e[1], e[2], e[3]);
          }
        }
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const u32x4 xv = buf.x[m][q];
        f16x8 af;
        if constexpr (FMT == kQ8) {
          af = __builtin_bit_cast(f16x8, xv);
        } else {
          uint32_t xp[4];
          q4_xpairs(xv[0], xv[1], xv[2], xv[3], xp);
          af = pack8(xp[0], xp[1], xp[2], xp[3]);
        }
#pragma unroll
        for (int h = 0; h < NW; ++h)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            if constexpr (FMT == kQ8) {
              acc.v[h][m][nt] =
                  __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[h][nt], acc.v[h][m][nt], 0, 0, 0);
            } else if constexpr (GM == kG32) {
              const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
              const f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[h][nt], z, 0, 0, 0);
              float sc;
              if constexpr (SF16)
                sc = scale16(buf.s[h][nt][0], q);
              else
                sc = as_f32(buf.s[h][nt][0][q]);
#pragma unroll
              for (int r = 0; r < 4; ++r) acc.v[h][m][nt][r] = fmaf(sc, t[r], acc.v[h][m][nt][r]);
            } else {
              // group 16: slots 0-1 hold group 2q, slots 2-3 group 2q+1
              const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
              const f16x8 zero8 = {};
              const f16x8 blo = kb < 2 ? bf[h][nt] : zero8;
              const f16x8 bhi = kb < 2 ? zero8 : bf[h][nt];
              const f32x4 tl = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, blo, z, 0, 0, 0);
              const f32x4 th = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bhi, z, 0, 0, 0);
              float sl, shv;
              if constexpr (SF16) {
                sl = scale16(buf.s[h][nt][0], 2 * q);
                shv = scale16(buf.s[h][nt][0], 2 * q + 1);
              } else {
                const u32x4& sv = buf.s[h][nt][q >> 1];
                sl = as_f32(sv[2 * (q & 1)]);
                shv = as_f32(sv[2 * (q & 1) + 1]);
              }
#pragma unroll
              for (int r = 0; r < 4; ++r)
                acc.v[h][m][nt][r] = fmaf(shv, th[r], fmaf(sl, tl[r], acc.v[h][m][nt][r]));
            }
          }
      }
    }
  }

  // Scale (Q8), epilogue and store of a finished tile; zeroes the accumulators.
  // rs_pre: Q8 row scales the caller loaded ahead ([NW][NT], the lane's
  // output row of each block); null: loaded here
  static __device__ __forceinline__ void finish(const QmvParams& p, const Cursor& cu, int lane,
                                                Acc& acc, const float* rs_pre = nullptr) {
    const QmvMat& mt = p.mat[cu.j];
    const int n_l = lane & 15, mq = lane >> 4;
    const bool yf32 = (p.flags & kFlagYf32) != 0;
    constexpr int sb = SF16 ? 2 : 4;
    char* yb = (char*)mt.y + cu.b * mt.y_bstride * (yf32 ? 4 : 2);
    const char* rb =
        mt.res ? (const char*)mt.res + cu.b * mt.r_bstride * (yf32 ? 4 : 2) : nullptr;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int n = cu.rt * TN + 16 * nt + n_l;
      float rs[NW];
#pragma unroll
      for (int h = 0; h < NW; ++h) {
        rs[h] = 1.0f;
        if constexpr (FMT == kQ8) {
          if (rs_pre) {
            rs[h] = rs_pre[h * NT + nt];
          } else {
            const char* sp = (const char*)(h == 0 ? mt.s : mt.s2) + cu.b * mt.s_bstride * sb;
            rs[h] = n < mt.n ? load_scale(sp, n, SF16) : 0.0f;
          }
        }
      }
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 16 * m + 4 * mq + r;
          if (row < p.m && n < mt.n_store && mt.y) {
            float v = 0.0f;
            if (n < mt.n) {
              v = gemm_epilogue(p, p.m_base + row, n, acc.v[0][m][nt][r] * rs[0]);
              if constexpr (PAIR)
                v = silu(v) * gemm_epilogue(p, p.m_base + row, n, acc.v[1][m][nt][r] * rs[1]);
              if (rb && (p.flags & kFlagResidual)) {
                const long long ri = (long long)row * p.r_rstride + n;
                v += yf32 ? ((const float*)rb)[ri] : (float)((const f16*)rb)[ri];
              }
            }
            const long long yi = out_index(p, mt, row, n);
            if (yf32)
              ((float*)yb)[yi] = v;
            else
              ((f16*)yb)[yi] = (f16)v;
          }
        }
    }
#pragma unroll
    for (int h = 0; h < NW; ++h)
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc.v[h][m][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  // Split K: the wave's raw accumulators of K chunk c (no row scale, no
  // epilogue) into partial plane c, then zeroed for the next segment.
  static __device__ __forceinline__ void spill(const QmvParams& p, const Cursor& cu, int lane,
                                               int c, Acc& acc) {
    const QmvMat& mt = p.mat[cu.j];
    const int n_l = lane & 15, mq = lane >> 4;
    // the matrix's block of the plane through a buffer resource (scalar
    // registers) and 32-bit lane offsets
    const float* base = p.sk_part + (long long)c * p.sk_plane + mt.sk_off +
                        (long long)cu.b * p.m * NW * mt.n_store;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)base, (short)0, p.m * NW * mt.n_store * 4, kBufferRsrcWord3);
    const int rstride = NW * mt.n_store * 4;  // bytes between partial rows
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int n = cu.rt * TN + 16 * nt + n_l;
      if (n >= mt.n) continue;
#pragma unroll
      for (int h = 0; h < NW; ++h)
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = 16 * m + 4 * mq + r;
            if (row < p.m)
              __builtin_amdgcn_raw_buffer_store_b32(
                  f32_bits(acc.v[h][m][nt][r]), rs,
                  row * rstride + (h * mt.n_store + n) * 4, 0, 0);
          }
    }
#pragma unroll
    for (int h = 0; h < NW; ++h)
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc.v[h][m][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
};

template <int FMT, int GM, int MT, int NT, bool PAIR, bool SF16>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void qmm_kernel(const QmvParams p) {
  using Q = Qmm<FMT, GM, MT, NT, PAIR, SF16>;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gw = blockIdx.x * kWaves + wave;
  const int nw = gridDim.x * kWaves;
  // A wave's range is whole (tile, K chunk) items: a tile's K slices split
  // only at chunk boundaries (split K, sk_chunks > 1), whose partials the
  // fix-up launch sums.  Items are numbered tile-major, so a range is one
  // contiguous run of (tile, slice) units.
  const int steps = p.k / 128;
  const int S = p.sk_chunks > 1 ? p.sk_chunks : 1;
  const int cs = S > 1 ? p.sk_cs : steps;
  const long long items = (long long)p.total_tiles * S;
  const long long i0 = (long long)gw * items / nw, i1 = (long long)(gw + 1) * items / nw;
  const int t0 = (int)((i0 / S) * steps + (i0 % S) * cs);
  const int t1 = i1 > i0 ? (int)(((i1 - 1) / S) * steps + min((int)((i1 - 1) % S + 1) * cs, steps))
                         : t0;
  if (t0 >= t1) return;

  typename Q::Cursor cu = Q::locate(p, t0);
  typename Q::Buf A, B;
  typename Q::Acc acc;
#pragma unroll
  for (int h = 0; h < Q::NW; ++h)
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc.v[h][m][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  Q::load(p, cu, lane, A);
  int t = t0;
  // K slices left in the running chunk: a countdown (integer division would be
  // a VALU sequence in this loop); a tile's shorter last chunk ends with it
  int seg = cs;
  auto segment_end = [&](const typename Q::Cursor& c) {
    if (S == 1)
      Q::finish(p, c, lane, acc);
    else
      Q::spill(p, c, lane, c.s / cs, acc);
  };
  while (true) {
    bool more = t + 1 < t1;
    typename Q::Cursor nx = more ? Q::advance(p, cu) : cu;
    Q::load(p, nx, lane, B);
    // keep the prefetch issued ahead of the consumer (the scheduler otherwise
    // sinks it below the MFMAs and every slice waits for its own loads)
    __builtin_amdgcn_sched_barrier(0);
    Q::compute(p, lane, A, acc);
    if (--seg == 0 || cu.s == steps - 1) {
      segment_end(cu);
      seg = cs;
    }
    if (!more) break;
    ++t;
    cu = nx;
    more = t + 1 < t1;
    nx = more ? Q::advance(p, cu) : cu;
    Q::load(p, nx, lane, A);
    __builtin_amdgcn_sched_barrier(0);
    Q::compute(p, lane, B, acc);
    if (--seg == 0 || cu.s == steps - 1) {
      segment_end(cu);
      seg = cs;
    }
    if (!more) break;
    ++t;
    cu = nx;
  }
}

}  // namespace aexq
