// Small-M (2..32 rows per launch) quantized matmul on gfx950 MFMA, wide-step
// form: Y[M][N] = X[M][K] W[N][K]^T for Q4 with one scale per 32 codes and
// Q8 with one scale per row, K a multiple of 256.
//
// A workgroup owns a contiguous range of (weight tile of 4 waves x 16 NT
// rows, 256-wide K step) pairs and walks them with its four waves in step:
// each wave streams its NT 16-row blocks of the tile, the activation rows of
// the step (16 MT rows x 256 codes) are loaded once per workgroup into a
// double-buffered LDS slice that every wave reads its MFMA A fragments from,
// and one barrier per step publishes the next slice.  The slice's loads are
// issued before the next step's weight loads, so that barrier never waits on
// HBM.  Codes are fetched the way HBM serves them best: every load
// instruction covers 8 rows x 128 contiguous bytes (lane l: row l / 8, bytes
// 16 (l % 8)); a block then goes through a wave-private LDS buffer laid out
// so that MFMA lane (n, kb) reads its row's B units for all eight 32-code
// groups with two (Q4) or four (Q8) 16-byte reads (a wave's LDS operations
// complete in order, so this needs no barrier).  Codes become exact fp16
// integers in registers; Q4 scales are applied in fp32 to each group's MFMA
// result (one group = one MFMA K extent), Q8 row scales once at the end, as
// in aexq_qmm.hpp.
#pragma once

#include "aexq_qmm.hpp"

namespace aexq {

template <int FMT, int MT, int NT, bool PAIR, bool SF16, bool ARGMAX, bool RMSX = false,
          bool G16 = false>
struct QmmW {
  // G16: Q4 with one scale per 16 codes (the reference's shipping Q4): an MFMA
  // K extent holds two groups, lane quarters kb = 0, 1 the first and 2, 3 the
  // second, so two MFMAs with the other group's quarters zeroed give each
  // group's product, scaled in fp32 like a 32-code group's
  static_assert(!G16 || FMT == kQ4, "16-code groups are a Q4 form");
  static constexpr int GM = FMT == kQ8 ? kGRow : (G16 ? kG16 : kG32);
  static constexpr int GPS = G16 ? 16 : 8;  // scale groups per 256-wide step
  using Base = Qmm<FMT, GM, MT, NT, PAIR, SF16>;
  using Cursor = typename Base::Cursor;  // s = 256-wide K step
  using Acc = typename Base::Acc;
  static constexpr int TN = 16 * NT;          // rows of one wave's blocks
  static constexpr int TNG = kWaves * TN;     // rows of a workgroup tile
  // LDS activation row stride (256 fp16 + 32 bytes): MFMA lane (n, kb)'s
  // 16-byte A reads of rows n = 0..15 fall on distinct 16-byte slots of a
  // 512-byte bank line (gfx950 serves 32 lanes' 16-byte reads per pass), and
  // every 32-lane pass of store_x writes one whole row
  static constexpr int XRS = 512 + 32;
  static constexpr int XSL = 16 * MT * XRS;   // LDS bytes of one activation slice
  static constexpr int XV = 2 * MT;           // 16-byte activation loads per thread per step
  static constexpr int NW = PAIR ? 2 : 1;
  static constexpr int RB = FMT == kQ8 ? 256 : 128;  // code bytes of a row per step
  static constexpr int WI = RB / 64;                 // 16-byte loads per lane per 16-row block
  static constexpr int BLK = 16 * RB;                // LDS bytes of one 16-row block
  static constexpr int LDS_WAVE = NW * NT * BLK;
  static constexpr int SV = FMT == kQ8 ? 0 : (SF16 ? 1 : 2) * (G16 ? 2 : 1);  // 16-byte scale loads per block

  struct Buf {
    u32x4 w[NW][NT][WI];
    u32x4 s[NW][NT][SV > 0 ? SV : 1];
    // Q8: the row scale (raw bits) of the lane's output row of each block,
    // loaded with a tile's last step (the other steps load it from past the
    // resource: no traffic), so the tile's epilogue waits for no load of its
    // own -- a load there would also wait for the next step's codes, which
    // are issued before it (the vector-memory counter counts in order)
    uint32_t q8s[NW][NT];
  };

  static __device__ __forceinline__ Cursor locate(const QmvParams& p, int t) {
    const int steps = p.k / 256;
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
    if (++c.s == p.k / 256) {
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

  // The weight loads of one step for this wave's blocks (rows r0 + [0, TN) of
  // the workgroup tile), branch-free (buffer resources zero-fill rows past N).
  static __device__ __forceinline__ void load(const QmvParams& p, const Cursor& cu, int lane,
                                              int wave, Buf& buf) {
    const QmvMat& mt = p.mat[cu.j];
    const int n_l = lane & 15;
    const int lr = lane >> 3, lc = lane & 7;  // load pattern: row lr (+8), 16-byte column lc
    constexpr int sb = SF16 ? 2 : 4;
    const int row_bytes = FMT == kQ8 ? p.k : p.k / 2;
    const int r0 = cu.rt * TNG + wave * TN;
    const int rows = mt.n > r0 ? mt.n - r0 : 0;
    const int wnum = rows > 0 ? rows * row_bytes - cu.s * RB : 0;
    const int sper = FMT == kQ8 ? 1 : p.groups_per_row;
    const int snum = rows > 0 ? (rows * sper - cu.s * GPS) * sb + 16 : 0;
#pragma unroll
    for (int h = 0; h < NW; ++h) {
      const char* wb = (const char*)(h == 0 ? mt.w : mt.w2) + (cu.b * mt.w_bstride) * 4 +
                       (long long)r0 * row_bytes + cu.s * RB;
      const __amdgpu_buffer_rsrc_t wr =
          __builtin_amdgcn_make_buffer_rsrc((void*)wb, (short)0, wnum, kBufferRsrcWord3);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int i = 0; i < WI; ++i) {
          // Q4: i = row half; Q8: bit 0 = row half, bit 1 = 128-byte half of the step
          const int rr = 16 * nt + 8 * (i & 1) + lr;
          const int cb = 128 * (i >> 1) + 16 * lc;
          buf.w[h][nt][i] = __builtin_bit_cast(
              u32x4,
              __builtin_amdgcn_raw_buffer_load_b128(wr, rr * row_bytes + cb, 0, kStreamAux));
        }
      if constexpr (FMT == kQ8) {
        const char* sbp = (const char*)(h == 0 ? mt.s : mt.s2) + cu.b * mt.s_bstride * sb;
        // rows of the wave's blocks past N read zero (their outputs are never
        // stored or compared); not the tile's last step: past the resource
        const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)sbp, (short)0, (mt.n * sb + 3) & ~3, kBufferRsrcWord3);
        const bool last = cu.s == p.k / 256 - 1;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int off = last ? (r0 + 16 * nt + n_l) * sb : (1 << 30);
          buf.q8s[h][nt] = SF16 ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(sr, off, 0, 0)
                                : __builtin_amdgcn_raw_buffer_load_b32(sr, off, 0, 0);
        }
      }
      if constexpr (SV > 0) {
        const char* sbp = (const char*)(h == 0 ? mt.s : mt.s2) +
                          (cu.b * mt.s_bstride + (long long)r0 * sper + cu.s * GPS) * sb;
        const __amdgpu_buffer_rsrc_t sr =
            __builtin_amdgcn_make_buffer_rsrc((void*)sbp, (short)0, snum, kBufferRsrcWord3);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int v = 0; v < SV; ++v)
            buf.s[h][nt][v] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           sr, (16 * nt + n_l) * sper * sb + 16 * v, 0, 0));
      }
    }
  }

  // The workgroup's activation slice of one step (16 MT rows x 256 codes):
  // thread t loads 16-byte chunk t % 32 of rows t / 32 and t / 32 + 8 per
  // 16-row tile (rows past M read 0), so 32 lanes cover one row.
  static __device__ __forceinline__ void load_x(const QmvParams& p, const Cursor& cu,
                                                u32x4 (&xv)[XV]) {
    const QmvMat& mt = p.mat[cu.j];
    const long long rs2 = p.x_rstride * 2;
    const char* xb = (const char*)mt.x + cu.b * mt.x_bstride * 2 + cu.s * 512;
    const int xnum = (int)(p.m * rs2) - cu.s * 512;
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc((void*)xb, (short)0, xnum, kBufferRsrcWord3);
    const int row = threadIdx.x >> 5, col = (threadIdx.x & 31) * 16;
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int v = 0; v < 2; ++v)
        xv[2 * m + v] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       xr, (16 * m + row + 8 * v) * (int)rs2 + col, 0, 0));
  }

  // RMSNorm-in inside the kernel (RMSX: launches with one item per workgroup,
  // where the row pre-pass would be a launch of its own): gamma[0, K) staged in
  // LDS and 1 / rms of the workgroup's 16 MT activation rows over all of K,
  // as the pre-pass forms them (CC:4531-4557).
  static constexpr int kMaxRmsK = 4096;
  static __device__ __forceinline__ void rms_prologue(const QmvParams& p, const Cursor& cu,
                                                      int lane, int wave, float* gs, float* inv) {
    const int kg = p.k < kMaxRmsK ? p.k : kMaxRmsK;  // the plan keeps K <= kMaxRmsK
    for (int i = threadIdx.x; i < kg; i += kThreads)
      gs[i] = p.gamma ? p.gamma[i < p.gamma_size - 1 ? i : p.gamma_size - 1] : 1.0f;
    const QmvMat& mt = p.mat[cu.j];
    const int rs2 = (int)(p.x_rstride * 2);
    const char* xb = (const char*)mt.x + cu.b * mt.x_bstride * 2;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)xb, (short)0, p.m * rs2, kBufferRsrcWord3);  // rows past M read 0
    constexpr int RPW = 16 * MT / kWaves;  // rows per wave: wave + kWaves r
    float ss[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) ss[r] = 0.0f;
    for (int c8 = lane; c8 < p.k / 8; c8 += 64) {
      u32x4 v[RPW];
#pragma unroll
      for (int r = 0; r < RPW; ++r)
        v[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             xr, (wave + kWaves * r) * rs2 + c8 * 16, 0, 0));
#pragma unroll
      for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const f16x2 h = as_h2(v[r][e]);
          ss[r] = fmaf((float)h[0], (float)h[0], ss[r]);
          ss[r] = fmaf((float)h[1], (float)h[1], ss[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const float t = wave_sum(ss[r]);
      if (lane == 0) inv[wave + kWaves * r] = rsqrtf(fmaxf(t / (float)p.k + p.eps, 1e-20f));
    }
  }

  // Stores the slice; Q4 chunks of 8 activations go in the (p, p + 4) pair
  // order that q4_pairs gives the codes, once per workgroup rather than per
  // MFMA.  RMSX: each activation becomes fp16(x * inv[row] * gamma[k]) first.
  static __device__ __forceinline__ void store_x(uint8_t* xs, const u32x4 (&xv)[XV],
                                                 int step = 0, const float* gs = nullptr,
                                                 const float* inv = nullptr) {
    const int row = threadIdx.x >> 5, col = (threadIdx.x & 31) * 16;
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        u32x4 c = xv[2 * m + v];
        if constexpr (RMSX) {
          const float iv = inv[16 * m + row + 8 * v];
          const float* g = gs + step * 256 + (col >> 1);  // col counts bytes
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const f16x2 h = as_h2(c[e]);
            const f16x2 o = {(f16)((float)h[0] * iv * g[2 * e]),
                             (f16)((float)h[1] * iv * g[2 * e + 1])};
            c[e] = as_u(o);
          }
        }
        if constexpr (FMT == kQ4) {
          uint32_t xp[4];
          q4_xpairs(c[0], c[1], c[2], c[3], xp);
          c = u32x4{xp[0], xp[1], xp[2], xp[3]};
        }
        *(u32x4*)(xs + (16 * m + row + 8 * v) * XRS + col) = c;
      }
  }

  // Argmax partials (the LM head): each lane keeps the (best, index, second)
  // of its output column for every row it holds (rows 16 m + 4 (lane / 16) + r)
  // over the tiles the wave finishes; the epilogue value is the one finish()
  // stores as the logit.
  struct Best {
    float v[MT][4], s[MT][4];
    int i[MT][4];
  };

  static __device__ __forceinline__ void best_init(Best& b) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        b.v[m][r] = __builtin_nanf("");
        b.i[m][r] = 0x7fffffff;
        b.s[m][r] = -INFINITY;
      }
  }

  static __device__ __forceinline__ void best_update(const QmvParams& p, const Cursor& cu,
                                                     int lane, const Acc& acc, const Buf& buf,
                                                     Best& b) {
    const QmvMat& mt = p.mat[cu.j];
    const int n_l = lane & 15, mq = lane >> 4;
    constexpr int sb = SF16 ? 2 : 4;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int n = cu.rt * Base::TN + 16 * nt + n_l;
      if (n >= mt.n) continue;
      float rs = 1.0f;
      if constexpr (FMT == kQ8) rs = scale_of(buf.q8s[0][nt], SF16);
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 16 * m + 4 * mq + r;
          if (row < p.m) {
            const float v =
                argmax_logit(p, gemm_epilogue(p, p.m_base + row, n, acc.v[0][m][nt][r] * rs));
            argmax_merge(b.v[m][r], b.i[m][r], b.s[m][r], v, n, -INFINITY);
          }
        }
    }
  }

  // One partial per row and workgroup: the 16 lanes of a row group, then the
  // four waves through LDS.  Every wave of the workgroup calls it.
  static __device__ __forceinline__ void best_write(const QmvParams& p, int lane, int wave,
                                                    Best& b, uint32_t tag) {
    __shared__ float lv[16 * MT][kWaves], ls[16 * MT][kWaves];
    __shared__ int li[16 * MT][kWaves];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = b.v[m][r], sv = b.s[m][r];
        int ix = b.i[m][r];
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
          const float ov = __shfl_xor(v, off, 64);
          const int oi = __shfl_xor(ix, off, 64);
          const float os = __shfl_xor(sv, off, 64);
          argmax_merge(v, ix, sv, ov, oi, os);
        }
        if ((lane & 15) == 0) {
          const int row = 16 * m + 4 * (lane >> 4) + r;
          lv[row][wave] = v;
          li[row][wave] = ix;
          ls[row][wave] = sv;
        }
      }
    __syncthreads();
    const int row = threadIdx.x;
    if (row < 16 * MT && row < p.m) {
      float v = lv[row][0], sv = ls[row][0];
      int ix = li[row][0];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) argmax_merge(v, ix, sv, lv[row][w], li[row][w], ls[row][w]);
      argmax_partial_store(p, (long long)(p.m_base + row) * p.parts + blockIdx.x, v, ix, sv, tag);
    }
  }

  // Consumes one step: the codes pass through LDS into MFMA layout, then
  // eight 32-code groups.
  static __device__ __forceinline__ void compute(const QmvParams& p, int lane, uint8_t* lds,
                                                 const uint8_t* xs, const Buf& buf, Acc& acc) {
    const int n_l = lane & 15, kb = lane >> 4;
    const int lr = lane >> 3, lc = lane & 7;
    // LDS, per 16-row block: the 16-byte run v of MFMA lane (n, kb) -- its
    // 8-code unit kb of groups 4 v .. 4 v + 3 (Q4, 4 bytes a unit) or 2 v,
    // 2 v + 1 (Q8, 8 bytes) -- at v * 1024 + (16 kb + n') * 16, with the row
    // swizzled (Q4: n' = n ^ 4 v; Q8: n' = n ^ (2 (v & 1) + 4 (kb / 2))): a
    // lane's runs are 16-byte reads whose 32-lane passes cover 32 distinct
    // slots of a 512-byte bank line, and the transposing stores (Q4: 4 bytes,
    // 32 lanes a pass; Q8: 8 bytes, 16 lanes a pass) meet distinct banks
#pragma unroll
    for (int h = 0; h < NW; ++h)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        uint8_t* blk = lds + (h * NT + nt) * BLK;
#pragma unroll
        for (int i = 0; i < WI; ++i) {
          const int n = 8 * (i & 1) + lr;
          const u32x4 c = buf.w[h][nt][i];
          if constexpr (FMT == kQ8) {
            // bytes 128 (i >> 1) + 16 lc: group 4 (i >> 1) + lc / 2, units 2 (lc & 1) + {0, 1}
            const int g = 4 * (i >> 1) + (lc >> 1);
            const int u0 = 2 * (lc & 1);
            const int np = n ^ (2 * (lc >> 2) + 4 * (lc & 1));  // (g / 2) & 1 = lc / 4, kb / 2 = lc & 1
            uint8_t* d = blk + (g >> 1) * 1024 + (g & 1) * 8;
            typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
            *(u32x2v*)(d + (16 * u0 + np) * 16) = u32x2v{c[0], c[1]};
            *(u32x2v*)(d + (16 * (u0 + 1) + np) * 16) = u32x2v{c[2], c[3]};
          } else {
            // 16 bytes = group lc, units 0..3
            const int np = n ^ (4 * (lc >> 2));
            uint8_t* d = blk + (lc >> 2) * 1024 + (lc & 3) * 4;
#pragma unroll
            for (int u = 0; u < 4; ++u) *(uint32_t*)(d + (16 * u + np) * 16) = c[u];
          }
        }
      }
    __builtin_amdgcn_wave_barrier();
    // B units of lane (n_l, kb): Q4 one dword per group, Q8 two
    constexpr int UW = FMT == kQ8 ? 2 : 1;
    uint32_t unit[NW][NT][8][UW];
#pragma unroll
    for (int h = 0; h < NW; ++h)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const uint8_t* src = lds + (h * NT + nt) * BLK;
#pragma unroll
        for (int v = 0; v < 2 * UW; ++v) {
          const int np = FMT == kQ8 ? n_l ^ (2 * (v & 1) + 4 * (kb >> 1)) : n_l ^ (4 * v);
          const u32x4 t = *(const u32x4*)(src + v * 1024 + (16 * kb + np) * 16);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int d = 4 * v + e;  // dword index in the lane's contiguous run
            unit[h][nt][d / UW][d % UW] = t[e];
          }
        }
      }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      f16x8 bf[NW][NT];
#pragma unroll
      for (int h = 0; h < NW; ++h)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          if constexpr (FMT == kQ8) {
            uint32_t a0, a1, b0, b1;
            q8_pairs(unit[h][nt][g][0], a0, a1);
            q8_pairs(unit[h][nt][g][1], b0, b1);
            bf[h][nt] = pack8(a0, a1, b0, b1);
          } else {
            uint32_t e[4];
            q4_pairs(unit[h][nt][g][0], e);
            bf[h][nt] = pack8(e[0], e[1], e[2], e[3]);
          }
        }
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        // (Q4: already in pair order, see store_x)
        const f16x8 af =
            *(const f16x8*)(xs + (16 * m + n_l) * XRS + 2 * (32 * g + 8 * kb));
#pragma unroll
        for (int h = 0; h < NW; ++h)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            if constexpr (FMT == kQ8) {
              acc.v[h][m][nt] =
                  __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[h][nt], acc.v[h][m][nt], 0, 0, 0);
            } else if constexpr (G16) {
              const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
              const f16x8 zb = {};
              const bool first = kb < 2;
              const f32x4 t0 =
                  __builtin_amdgcn_mfma_f32_16x16x32_f16(af, first ? bf[h][nt] : zb, z, 0, 0, 0);
              const f32x4 t1 =
                  __builtin_amdgcn_mfma_f32_16x16x32_f16(af, first ? zb : bf[h][nt], z, 0, 0, 0);
              float s0, s1;
              if constexpr (SF16) {
                s0 = Base::scale16(buf.s[h][nt][g >> 2], (2 * g) & 7);
                s1 = Base::scale16(buf.s[h][nt][g >> 2], (2 * g + 1) & 7);
              } else {
                s0 = as_f32(buf.s[h][nt][g >> 1][(2 * g) & 3]);
                s1 = as_f32(buf.s[h][nt][g >> 1][(2 * g + 1) & 3]);
              }
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                acc.v[h][m][nt][r] = fmaf(s0, t0[r], acc.v[h][m][nt][r]);
                acc.v[h][m][nt][r] = fmaf(s1, t1[r], acc.v[h][m][nt][r]);
              }
            } else {
              const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
              const f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[h][nt], z, 0, 0, 0);
              float sc;
              if constexpr (SF16)
                sc = Base::scale16(buf.s[h][nt][0], g);
              else
                sc = as_f32(buf.s[h][nt][g >> 2][g & 3]);
#pragma unroll
              for (int r = 0; r < 4; ++r) acc.v[h][m][nt][r] = fmaf(sc, t[r], acc.v[h][m][nt][r]);
            }
          }
      }
    }
  }
};

template <int FMT, int MT, int NT, bool PAIR, bool SF16, bool ARGMAX, bool RMSX, bool G16>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void qmmw_kernel(const QmvParams p) {
  using Q = QmmW<FMT, MT, NT, PAIR, SF16, ARGMAX, RMSX, G16>;
  __shared__ float rms_g[RMSX ? Q::kMaxRmsK : 1];   // gamma (RMSX)
  __shared__ float rms_inv[RMSX ? 16 * MT : 1];      // 1 / rms per activation row (RMSX)
  __shared__ __align__(16) uint8_t lds_all[kWaves][Q::LDS_WAVE];
  __shared__ __align__(16) uint8_t xs_all[2][Q::XSL];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint8_t* lds = lds_all[wave];
  // A workgroup's range is whole (tile, K chunk) items: a tile's K steps split
  // only at chunk boundaries (split K, sk_chunks > 1), whose partials the
  // fix-up launch sums.  Items are numbered tile-major, so a range is one
  // contiguous run of (tile, step) units.
  const int steps = p.k / 256;
  const int S = !ARGMAX && p.sk_chunks > 1 ? p.sk_chunks : 1;
  const int cs = S > 1 ? p.sk_cs : steps;
  const long long items = (long long)p.total_tiles * S;
  const int rank = xcd_rank(blockIdx.x, gridDim.x);  // one XCD: one contiguous run of items
  const long long i0 = (long long)rank * items / gridDim.x;
  const long long i1 = (long long)(rank + 1) * items / gridDim.x;
  const int t0 = (int)((i0 / S) * steps + (i0 % S) * cs);
  const int t1 = i1 > i0 ? (int)(((i1 - 1) / S) * steps + min((int)((i1 - 1) % S + 1) * cs, steps))
                         : t0;
  if (t0 >= t1) {  // the whole workgroup: no barrier is left waiting
    if constexpr (ARGMAX) {
      const uint32_t tag = argmax_tag(p);
      // an empty partial for each row (it never wins the merge)
      const int row = threadIdx.x;
      if (row < 16 * MT && row < p.m)
        argmax_partial_store(p, (long long)(p.m_base + row) * p.parts + blockIdx.x,
                             __builtin_nanf(""), 0x7fffffff, -INFINITY, tag);
      argmax_tail<4>(p, tag);
    }
    return;
  }
  typename Q::Best best;
  if constexpr (ARGMAX) Q::best_init(best);

  typename Q::Cursor cu = Q::locate(p, t0);
  typename Q::Buf A, B;
  typename Q::Acc acc;
  u32x4 xv[Q::XV];
#pragma unroll
  for (int h = 0; h < Q::NW; ++h)
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc.v[h][m][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // the wave's own cursor for the weight rows and the epilogue
  auto mine = [&](typename Q::Cursor c) {
    c.rt = c.rt * kWaves + wave;
    return c;
  };
  // the last step of a K chunk: the whole tile's K finishes it here, a chunk
  // of a split tile leaves its partial (the host never splits an argmax launch)
  auto segment_end = [&](const typename Q::Cursor& c, const typename Q::Buf& bf) {
    float rsp[Q::NW][NT];  // Q8: the tile's row scales, loaded with its last step
#pragma unroll
    for (int h = 0; h < Q::NW; ++h)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) rsp[h][nt] = FMT == kQ8 ? scale_of(bf.q8s[h][nt], SF16) : 1.0f;
    if constexpr (ARGMAX) {
      Q::best_update(p, mine(c), lane, acc, bf, best);
      Q::Base::finish(p, mine(c), lane, acc, &rsp[0][0]);
    } else if (S == 1) {
      Q::Base::finish(p, mine(c), lane, acc, &rsp[0][0]);
    } else {
      Q::Base::spill(p, mine(c), lane, c.s / cs, acc);
    }
  };
  if constexpr (RMSX) Q::rms_prologue(p, cu, lane, wave, rms_g, rms_inv);
  Q::load_x(p, cu, xv);
  Q::load(p, cu, lane, wave, A);
  if constexpr (RMSX) __syncthreads();  // gamma and 1 / rms in LDS
  Q::store_x(xs_all[0], xv, cu.s, rms_g, rms_inv);
  __syncthreads();
  int t = t0;
  int sl = 0;
  // steps left in the running K chunk (ranges start at chunk boundaries; a
  // tile's shorter last chunk ends with the tile): a countdown, since integer
  // division would be a VALU sequence in this loop
  int seg = cs;
  while (true) {
    // step t: codes in A, activations in slice sl; step t + 1's activation
    // loads go out first, then its codes into B
    bool more = t + 1 < t1;
    typename Q::Cursor nx = more ? Q::advance(p, cu) : cu;
    Q::load_x(p, nx, xv);
    Q::load(p, nx, lane, wave, B);
    __builtin_amdgcn_sched_barrier(0);
    Q::compute(p, lane, lds, xs_all[sl], A, acc);
    if (--seg == 0 || cu.s == steps - 1) {
      segment_end(cu, A);
      seg = cs;
    }
    if (!more) break;
    Q::store_x(xs_all[sl ^ 1], xv, nx.s, rms_g, rms_inv);
    __syncthreads();
    ++t;
    cu = nx;
    sl ^= 1;
    more = t + 1 < t1;
    nx = more ? Q::advance(p, cu) : cu;
    Q::load_x(p, nx, xv);
    Q::load(p, nx, lane, wave, A);
    __builtin_amdgcn_sched_barrier(0);
    Q::compute(p, lane, lds, xs_all[sl], B, acc);
    if (--seg == 0 || cu.s == steps - 1) {
      segment_end(cu, B);
      seg = cs;
    }
    if (!more) break;
    Q::store_x(xs_all[sl ^ 1], xv, nx.s, rms_g, rms_inv);
    __syncthreads();
    ++t;
    cu = nx;
    sl ^= 1;
  }
  if constexpr (ARGMAX) {
    // the launch's tag, read only now: issued at the start, it would sit
    // ahead of the weight loads in the memory counter, and the first wait for
    // them would wait for this agent-coherent round trip too
    const uint32_t tag = argmax_tag(p);
    Q::best_write(p, lane, wave, best, tag);
    argmax_tail<4>(p, tag);
  }
}

}  // namespace aexq
