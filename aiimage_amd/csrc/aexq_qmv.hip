// Quantized matvec / small-M matmul kernels for gfx950 (M <= 8).
//
// The weight is a row-major [N][K] stream of int8 (Q8) or nibble (Q4) codes,
// exactly the reference's packed words (MM:707-734).  Each 16-byte chunk of a
// row is one 128-bit load; LPR lanes share a row, CPL chunks per lane cover K.
// Codes become exact fp16 integers in registers (q8_pairs / q4_pairs) and meet
// the fp16 activations in v_dot2_f32_f16 with fp32 accumulation.  Scales are
// applied in fp32: once per row for Q8 (per-output-row scale), once per
// 32-code chunk for Q4 (or per 16 codes for group 16).  Rows are reduced with
// DPP inside the wave.  Epilogues (bias/alpha/beta, RMSNorm-in, SwiGLU-out,
// residual, fused argmax) are applied before the single store.
#include <math.h>

#include "aexq_device.hpp"

namespace aexq {

// Row groups per wave: about four 16-byte loads in flight per lane at M = 1,
// fewer when eight activation rows occupy the registers.
template <int CPL, int MMAX>
struct UnrollFor {
  static constexpr int base = CPL >= 4 ? 1 : (CPL >= 2 ? 2 : 4);
  static constexpr int value = MMAX >= 8 ? (base > 1 ? base / 2 : 1) : base;
};

template <int FMT, int LPR, int CPL, int MMAX = 1>
struct Geometry {
  static constexpr int SLOTS = 64 / LPR;                // rows sharing a wave at once
  static constexpr int U = UnrollFor<CPL, MMAX>::value; // row groups per wave
  static constexpr int RW = SLOTS * U;                  // rows per wave
  static constexpr int RWG = RW * kWaves;               // rows per workgroup
  static constexpr int XW = FMT == kQ8 ? 8 : 16;        // activation dwords per chunk
};

// Loads the lane's activation chunks for row m (optionally RMS-normalised) as
// fp16 pairs in the order the code expansion consumes them.
template <int FMT, int LPR, int CPL>
__device__ __forceinline__ void load_x(const QmvParams& p, const f16* xrow, int sub, float inv,
                                       bool rms, uint32_t (&xr)[CPL][Geometry<FMT, LPR, CPL>::XW]) {
  constexpr int XW = Geometry<FMT, LPR, CPL>::XW;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ci = sub + c * LPR;
    uint32_t raw[XW];
    if (ci < p.chunks) {
      const u32x4* src = (const u32x4*)(xrow + (long long)ci * (XW * 2));
#pragma unroll
      for (int v = 0; v < XW / 4; ++v) {
        const u32x4 t = src[v];
        raw[4 * v + 0] = t[0];
        raw[4 * v + 1] = t[1];
        raw[4 * v + 2] = t[2];
        raw[4 * v + 3] = t[3];
      }
      if (rms) {
        const int k0 = ci * XW * 2;
#pragma unroll
        for (int d = 0; d < XW; ++d) {
          const f16x2 h = as_h2(raw[d]);
          float a = (float)h[0] * inv;
          float b = (float)h[1] * inv;
          if (p.gamma) {
            const int last = p.gamma_size - 1;
            const int ka = k0 + 2 * d, kb = ka + 1;
            a *= p.gamma[ka < last ? ka : last];
            b *= p.gamma[kb < last ? kb : last];
          }
          f16x2 o = {(f16)a, (f16)b};
          raw[d] = as_u(o);
        }
      }
    } else {
#pragma unroll
      for (int d = 0; d < XW; ++d) raw[d] = 0u;
    }
    if constexpr (FMT == kQ8) {
#pragma unroll
      for (int d = 0; d < XW; ++d) xr[c][d] = raw[d];
    } else {
#pragma unroll
      for (int d = 0; d < 4; ++d)
        q4_xpairs(raw[4 * d], raw[4 * d + 1], raw[4 * d + 2], raw[4 * d + 3], &xr[c][4 * d]);
    }
  }
}

// Bias, alpha and beta as the reference Gemm resolves them (MM:688-705, 812-820):
// Pack4-linear output is alpha*(beta*C + sum), tiled output beta*C + alpha*sum.
__device__ __forceinline__ float gemm_epilogue(const QmvParams& p, int m, int r, float v) {
  float bias = 0.0f;
  if (p.c) {
    switch (p.bcast) {
      case 0: bias = p.c[0]; break;
      case 1: bias = p.c[m]; break;
      case 3: bias = p.c[(long long)m * p.c_rstride + r]; break;
      case 4: bias = p.c[r]; break;
      default: bias = 0.0f; break;
    }
    bias *= p.beta;
  }
  return (p.flags & kFlagAlphaIn) ? p.alpha * (bias + v) : bias + p.alpha * v;
}

template <int FMT, int LPR, int CPL, int MMAX, bool PAIR, bool ARGMAX, bool G16>
__global__ __launch_bounds__(kThreads) void qmv_kernel(const QmvParams p) {
  using Geo = Geometry<FMT, LPR, CPL, MMAX>;
  constexpr int SLOTS = Geo::SLOTS, U = Geo::U, RW = Geo::RW, RWG = Geo::RWG, XW = Geo::XW;
  constexpr int NW = PAIR ? 2 : 1;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int sub = lane & (LPR - 1), slot = lane / LPR;

  // ---- which matrix / batch entry / row tile this workgroup owns
  const int b = blockIdx.x;
  int j = 0;
  for (int t = 1; t < p.nmat; ++t)
    if (b >= p.mat[t].tile_base) j = t;
  const QmvMat& mt = p.mat[j];
  const int local = b - mt.tile_base;
  const int bi = local / mt.tiles;
  const int tile = local - bi * mt.tiles;

  const bool scl16 = (p.flags & kFlagScaleF16) != 0;
  const int sbytes = scl16 ? 2 : 4;
  const long long row_words = (long long)p.chunks * 4;
  const uint32_t* wsrc[NW];
  const char* ssrc[NW];
  wsrc[0] = mt.w + bi * mt.w_bstride;
  ssrc[0] = (const char*)mt.s + bi * mt.s_bstride * sbytes;
  if constexpr (PAIR) {
    wsrc[1] = mt.w2 + bi * mt.w_bstride;
    ssrc[1] = (const char*)mt.s2 + bi * mt.s_bstride * sbytes;
  }
  const int rbase = tile * RWG + wave * RW;

  // ---- issue the weight stream first so it is in flight during the prologue
  u32x4 wv[NW][U][CPL];
#pragma unroll
  for (int h = 0; h < NW; ++h)
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = rbase + u * SLOTS + slot;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int ci = sub + c * LPR;
        if (r < mt.n && ci < p.chunks) {
          wv[h][u][c] = *(const u32x4*)(wsrc[h] + (long long)r * row_words + (long long)ci * 4);
        } else {
          wv[h][u][c] = u32x4{0u, 0u, 0u, 0u};
        }
      }
    }

  // scales: per row for Q8; per chunk (two per chunk for group 16) for Q4
  constexpr int SPC = G16 ? 2 : 1;
  float sc[NW][U][FMT == kQ8 ? 1 : CPL][FMT == kQ8 ? 1 : SPC];
#pragma unroll
  for (int h = 0; h < NW; ++h)
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = rbase + u * SLOTS + slot;
      if constexpr (FMT == kQ8) {
        sc[h][u][0][0] = r < mt.n ? load_scale(ssrc[h], r, scl16) : 0.0f;
      } else {
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          const int ci = sub + c * LPR;
          const bool ok = r < mt.n && ci < p.chunks;
          if constexpr (G16) {
            const long long g0 = (long long)r * p.groups_per_row + 2LL * ci;
            sc[h][u][c][0] = ok ? load_scale(ssrc[h], g0, scl16) : 0.0f;
            sc[h][u][c][1] = ok ? load_scale(ssrc[h], g0 + 1, scl16) : 0.0f;
          } else {
            const long long g = (long long)r * p.groups_per_row + (long long)(ci * 32) / p.group;
            sc[h][u][c][0] = ok ? load_scale(ssrc[h], g, scl16) : 0.0f;
          }
        }
      }
    }

  // ---- RMSNorm-in: every workgroup reduces sum(x^2) over the full row
  const f16* xb = (const f16*)mt.x + bi * mt.x_bstride;
  const bool rms = (p.flags & kFlagRms) != 0;
  float inv[MMAX];
#pragma unroll
  for (int m = 0; m < MMAX; ++m) inv[m] = 1.0f;
  if (rms) {
    __shared__ float red[MMAX][kWaves];
#pragma unroll
    for (int m = 0; m < MMAX; ++m) {
      float ss = 0.0f;
      if (m < p.m) {
        const f16* xr = xb + (long long)m * p.x_rstride;
        for (int kk = tid * 2; kk < p.k; kk += kThreads * 2) {
          const f16x2 h = *(const f16x2*)(xr + kk);
          const float a = (float)h[0], c = (float)h[1];
          ss = fmaf(a, a, ss);
          ss = fmaf(c, c, ss);
        }
      }
      ss = wave_sum(ss);
      if (lane == 0) red[m][wave] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MMAX; ++m) {
      const float ss = red[m][0] + red[m][1] + red[m][2] + red[m][3];
      inv[m] = rsqrtf(fmaxf(ss / (float)p.k + p.eps, 1e-20f));
    }
  }

  // ---- activations into registers
  uint32_t xr[MMAX][CPL][XW];
#pragma unroll
  for (int m = 0; m < MMAX; ++m) {
    if (m < p.m) {
      load_x<FMT, LPR, CPL>(p, xb + (long long)m * p.x_rstride, sub, inv[m], rms, xr[m]);
    } else {
#pragma unroll
      for (int c = 0; c < CPL; ++c)
#pragma unroll
        for (int d = 0; d < XW; ++d) xr[m][c][d] = 0u;
    }
  }

  // ---- dot products
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
            q8_pairs(wv[h][u][c][d], lo, hi);
#pragma unroll
            for (int m = 0; m < MMAX; ++m)
              acc[h][u][m] = dot2(hi, xr[m][c][2 * d + 1], dot2(lo, xr[m][c][2 * d], acc[h][u][m]));
          }
        } else {
          float part[SPC][MMAX];
#pragma unroll
          for (int g = 0; g < SPC; ++g)
#pragma unroll
            for (int m = 0; m < MMAX; ++m) part[g][m] = 0.0f;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            uint32_t q[4];
            q4_pairs(wv[h][u][c][d] ^ p.xor_mask, q);
            const int g = G16 ? (d >> 1) : 0;
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
              acc[h][u][m] = fmaf(part[g][m], sc[h][u][c][g], acc[h][u][m]);
        }
      }

  // ---- reduce each row over its LPR lanes
#pragma unroll
  for (int h = 0; h < NW; ++h)
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int m = 0; m < MMAX; ++m) {
        float v = group_sum<LPR>(acc[h][u][m]);
        if constexpr (FMT == kQ8) v *= sc[h][u][0][0];
        acc[h][u][m] = v;
      }

  // ---- epilogue and store
  const bool yf32 = (p.flags & kFlagYf32) != 0;
  char* yb = (char*)mt.y + bi * mt.y_bstride * (yf32 ? 4 : 2);
  const char* rb = mt.res ? (const char*)mt.res + bi * mt.r_bstride * (yf32 ? 4 : 2) : nullptr;
  float outv[U][MMAX];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int r = rbase + u * SLOTS + slot;
#pragma unroll
    for (int m = 0; m < MMAX; ++m) {
      float v = 0.0f;
      if (r < mt.n && m < p.m) {
        v = gemm_epilogue(p, m, r, acc[0][u][m]);
        if constexpr (PAIR) v = silu(v) * gemm_epilogue(p, m, r, acc[1][u][m]);
        if (rb && (p.flags & kFlagResidual)) {
          const long long ri = (long long)m * p.r_rstride + r;
          v += yf32 ? ((const float*)rb)[ri] : (float)((const f16*)rb)[ri];
        }
      }
      outv[u][m] = v;
      // one lane per row stores; lanes of a slot hold identical values
      if (sub == ((u * MMAX + m) & (LPR - 1)) && r < mt.n_store && m < p.m && mt.y) {
        const long long yi = (long long)m * mt.y_rstride + r;
        if (yf32)
          ((float*)yb)[yi] = v;
        else
          ((f16*)yb)[yi] = (f16)v;
      }
    }
  }

  if constexpr (ARGMAX) {
    // candidates of this workgroup -> LDS -> one wave reduces -> partial
    __shared__ float cand[MMAX][RWG];
    if (sub == 0) {
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int m = 0; m < MMAX; ++m) cand[m][wave * RW + u * SLOTS + slot] = outv[u][m];
    }
    __syncthreads();
    if (wave == 0) {
      for (int m = 0; m < p.m; ++m) {
        float bv = __builtin_nanf("");
        int bix = 0x7fffffff;
        float bs = -INFINITY;
        const int r = tile * RWG + lane;
        if (lane < RWG && r < mt.n) {
          bv = cand[m][lane];
          bix = r;
        }
        argmax_wave_reduce(bv, bix, bs);
        if (lane == 0) {
          const long long pi = (long long)m * p.parts + tile;
          p.part_best[pi] = bv;
          p.part_index[pi] = bix;
          p.part_second[pi] = bs;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Generic kernel: any K, any scale block, fp16 or fp32 activations; decodes
// element by element with the reference formula (MM:707-727).  One wave per
// output row, lanes stride over K, up to 16 activation rows per launch row.
// ---------------------------------------------------------------------------
constexpr int kGenericM = 16;

template <int FMT>
__global__ __launch_bounds__(kThreads) void generic_kernel(const QmvParams p) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = blockIdx.x;
  int j = 0;
  for (int t = 1; t < p.nmat; ++t)
    if (b >= p.mat[t].tile_base) j = t;
  const QmvMat& mt = p.mat[j];
  const int local = b - mt.tile_base;
  const int bi = local / mt.tiles;
  const int tile = local - bi * mt.tiles;
  const int r = tile * kWaves + wave;
  const int m0 = blockIdx.y * kGenericM;
  const int mcount = min(kGenericM, p.m - m0);

  const bool scl16 = (p.flags & kFlagScaleF16) != 0;
  const bool xf32 = (p.flags & kFlagXf32) != 0;
  const bool yf32 = (p.flags & kFlagYf32) != 0;
  const uint32_t* w = mt.w + bi * mt.w_bstride;
  const char* s = (const char*)mt.s + bi * mt.s_bstride * (scl16 ? 2 : 4);
  const char* xb = (const char*)mt.x + bi * mt.x_bstride * (xf32 ? 4 : 2);
  const bool rms = (p.flags & kFlagRms) != 0;

  float inv[kGenericM];
  for (int i = 0; i < kGenericM; ++i) inv[i] = 1.0f;
  if (rms) {
    for (int i = 0; i < mcount; ++i) {
      float ss = 0.0f;
      for (int kk = lane; kk < p.k; kk += 64) {
        const long long xi = (long long)(m0 + i) * p.x_rstride + kk;
        const float a = xf32 ? ((const float*)xb)[xi] : (float)((const f16*)xb)[xi];
        ss = fmaf(a, a, ss);
      }
      ss = wave_sum(ss);
      inv[i] = rsqrtf(fmaxf(ss / (float)p.k + p.eps, 1e-20f));
    }
  }

  float acc[kGenericM];
  for (int i = 0; i < kGenericM; ++i) acc[i] = 0.0f;
  if (r < mt.n) {
    for (int kk = lane; kk < p.k; kk += 64) {
      const long long idx = (long long)r * p.k + kk;
      int sv;
      if constexpr (FMT == kQ8) {
        const uint32_t raw = (w[idx >> 2] >> ((idx & 3) * 8)) & 0xffu;
        sv = raw >= 128u ? (int)raw - 256 : (int)raw;
      } else {
        const uint32_t raw = ((w[idx >> 3] >> ((idx & 7) * 4)) & 0xfu) ^ (p.xor_mask & 0xfu);
        sv = (int)raw - 8;
      }
      const long long si = FMT == kQ8 ? (long long)r : idx / p.group;
      const float wval = (float)sv * load_scale(s, si, scl16);
      for (int i = 0; i < mcount; ++i) {
        const long long xi = (long long)(m0 + i) * p.x_rstride + kk;
        float a = xf32 ? ((const float*)xb)[xi] : (float)((const f16*)xb)[xi];
        if (rms) {
          a *= inv[i];
          if (p.gamma) a *= p.gamma[min(kk, p.gamma_size - 1)];
          if (!xf32) a = (float)(f16)a;
        }
        acc[i] = fmaf(a, wval, acc[i]);
      }
    }
  }
  char* yb = (char*)mt.y + bi * mt.y_bstride * (yf32 ? 4 : 2);
  const char* rb = mt.res ? (const char*)mt.res + bi * mt.r_bstride * (yf32 ? 4 : 2) : nullptr;
  for (int i = 0; i < mcount; ++i) {
    float v = wave_sum(acc[i]);
    const int m = m0 + i;
    if (lane == (i & 63) && r < mt.n_store) {
      if (r < mt.n) {
        v = gemm_epilogue(p, m, r, v);
        if (rb && (p.flags & kFlagResidual)) {
          const long long ri = (long long)m * p.r_rstride + r;
          v += yf32 ? ((const float*)rb)[ri] : (float)((const f16*)rb)[ri];
        }
      } else {
        v = 0.0f;
      }
      const long long yi = (long long)m * mt.y_rstride + r;
      if (yf32)
        ((float*)yb)[yi] = v;
      else
        ((f16*)yb)[yi] = (f16)v;
    }
  }
}

// ---------------------------------------------------------------------------
// Argmax over existing fp32 logits rows, and the final merge of partials.
// ---------------------------------------------------------------------------
constexpr int kArgmaxCols = 4096;

__global__ __launch_bounds__(kThreads) void logits_argmax_kernel(const float* logits, int n,
                                                                 long long rstride, float* pv,
                                                                 int* pi, float* ps, int parts) {
  const int m = blockIdx.y, part = blockIdx.x;
  const int c0 = part * kArgmaxCols;
  const int c1 = min(n, c0 + kArgmaxCols);
  float bv = __builtin_nanf("");
  int bix = 0x7fffffff;
  float bs = -INFINITY;
  for (int c = c0 + (int)threadIdx.x; c < c1; c += kThreads) {
    argmax_merge(bv, bix, bs, logits[(long long)m * rstride + c], c, -INFINITY);
  }
  argmax_wave_reduce(bv, bix, bs);
  __shared__ float sv[kWaves], ss[kWaves];
  __shared__ int si[kWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bix;
    ss[wave] = bs;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kWaves; ++w) argmax_merge(bv, bix, bs, sv[w], si[w], ss[w]);
    const long long o = (long long)m * parts + part;
    pv[o] = bv;
    pi[o] = bix;
    ps[o] = bs;
  }
}

__global__ __launch_bounds__(kThreads) void argmax_finalize_kernel(const ArgmaxParams a) {
  const int m = blockIdx.x;
  float bv = __builtin_nanf("");
  int bix = 0x7fffffff;
  float bs = -INFINITY;
  for (int i = threadIdx.x; i < a.parts; i += kThreads) {
    const long long o = (long long)m * a.parts + i;
    argmax_merge(bv, bix, bs, a.pv[o], a.pi[o], a.ps[o]);
  }
  argmax_wave_reduce(bv, bix, bs);
  __shared__ float sv[kWaves], ss[kWaves];
  __shared__ int si[kWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bix;
    ss[wave] = bs;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kWaves; ++w) argmax_merge(bv, bix, bs, sv[w], si[w], ss[w]);
    a.out_index[m] = bix == 0x7fffffff ? 0 : bix;
    if (a.out_gap) a.out_gap[m] = bs == -INFINITY ? INFINITY : bv - bs;
  }
}

// ---------------------------------------------------------------------------
// Dequantization to fp32 [N][K].  Chunk-aligned rows use the same code
// expansion as the matvec kernels; other shapes decode element by element.
// ---------------------------------------------------------------------------
template <int FMT>
__global__ __launch_bounds__(kThreads) void dequant_chunk_kernel(const uint32_t* w, const void* s,
                                                                 int scl16, int n, int k, int group,
                                                                 uint32_t xor_mask, float* out) {
  const int chunks = FMT == kQ8 ? k / 16 : k / 32;
  const long long total = (long long)n * chunks;
  for (long long t = blockIdx.x * (long long)kThreads + threadIdx.x; t < total;
       t += (long long)gridDim.x * kThreads) {
    const int r = (int)(t / chunks);
    const int ci = (int)(t - (long long)r * chunks);
    const u32x4 v = *(const u32x4*)(w + t * 4);
    if constexpr (FMT == kQ8) {
      const float sc = load_scale(s, r, scl16);
      float* o = out + (long long)r * k + ci * 16;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        uint32_t lo, hi;
        q8_pairs(v[d], lo, hi);
        const f16x2 a = as_h2(lo), b = as_h2(hi);
        o[4 * d + 0] = (float)a[0] * sc;
        o[4 * d + 1] = (float)a[1] * sc;
        o[4 * d + 2] = (float)b[0] * sc;
        o[4 * d + 3] = (float)b[1] * sc;
      }
    } else {
      float* o = out + (long long)r * k + ci * 32;
      const long long flat0 = (long long)r * k + ci * 32;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        uint32_t q[4];
        q4_pairs(v[d] ^ xor_mask, q);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const f16x2 h = as_h2(q[e]);
          const long long i0 = flat0 + 8 * d + e, i1 = i0 + 4;
          o[8 * d + e] = (float)h[0] * load_scale(s, i0 / group, scl16);
          o[8 * d + e + 4] = (float)h[1] * load_scale(s, i1 / group, scl16);
        }
      }
    }
  }
}

template <int FMT>
__global__ __launch_bounds__(kThreads) void dequant_elem_kernel(const uint32_t* w, const void* s,
                                                                int scl16, int n, int k, int group,
                                                                uint32_t xor_mask, float* out) {
  const long long total = (long long)n * k;
  for (long long idx = blockIdx.x * (long long)kThreads + threadIdx.x; idx < total;
       idx += (long long)gridDim.x * kThreads) {
    int sv;
    long long si;
    if constexpr (FMT == kQ8) {
      const uint32_t raw = (w[idx >> 2] >> ((idx & 3) * 8)) & 0xffu;
      sv = raw >= 128u ? (int)raw - 256 : (int)raw;
      si = idx / k;
    } else {
      const uint32_t raw = ((w[idx >> 3] >> ((idx & 7) * 4)) & 0xfu) ^ (xor_mask & 0xfu);
      sv = (int)raw - 8;
      si = idx / group;
    }
    out[idx] = (float)sv * load_scale(s, si, scl16);
  }
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
using QmvFn = void (*)(const QmvParams);

template <int FMT, int LPR, int CPL, int MMAX, bool PAIR, bool ARGMAX, bool G16>
constexpr QmvFn qmv_fn() {
  return &qmv_kernel<FMT, LPR, CPL, MMAX, PAIR, ARGMAX, G16>;
}

struct QmvEntry {
  QmvConfig cfg;
  QmvFn fn;
  int rwg;
};

#define AEXQ_QMV(FMT, LPR, CPL, MMAX, PAIR, ARGMAX, G16)                                   \
  QmvEntry {                                                                              \
    QmvConfig{FMT, LPR, CPL, MMAX, PAIR, ARGMAX, G16},                                    \
        qmv_fn<FMT, LPR, CPL, MMAX, PAIR, ARGMAX, G16>(),                                 \
        Geometry<FMT, LPR, CPL, MMAX>::RWG                                                \
  }

#define AEXQ_QMV_SHAPES(FMT, MMAX, PAIR, ARGMAX, G16)                                      \
  AEXQ_QMV(FMT, 16, 1, MMAX, PAIR, ARGMAX, G16), AEXQ_QMV(FMT, 32, 1, MMAX, PAIR, ARGMAX, G16), \
      AEXQ_QMV(FMT, 64, 1, MMAX, PAIR, ARGMAX, G16),                                      \
      AEXQ_QMV(FMT, 64, 2, MMAX, PAIR, ARGMAX, G16),                                      \
      AEXQ_QMV(FMT, 64, 4, MMAX, PAIR, ARGMAX, G16)

#define AEXQ_QMV_SHAPES_M8(FMT, PAIR, ARGMAX, G16)                                        \
  AEXQ_QMV(FMT, 16, 1, 8, PAIR, ARGMAX, G16), AEXQ_QMV(FMT, 32, 1, 8, PAIR, ARGMAX, G16),      \
      AEXQ_QMV(FMT, 64, 1, 8, PAIR, ARGMAX, G16), AEXQ_QMV(FMT, 64, 2, 8, PAIR, ARGMAX, G16)

static const QmvEntry kQmvTable[] = {
    AEXQ_QMV_SHAPES(kQ8, 1, false, false, false), AEXQ_QMV_SHAPES_M8(kQ8, false, false, false),
    AEXQ_QMV_SHAPES(kQ8, 1, true, false, false),  AEXQ_QMV_SHAPES_M8(kQ8, true, false, false),
    AEXQ_QMV_SHAPES(kQ8, 1, false, true, false),  AEXQ_QMV_SHAPES_M8(kQ8, false, true, false),
    AEXQ_QMV_SHAPES(kQ4, 1, false, false, false), AEXQ_QMV_SHAPES_M8(kQ4, false, false, false),
    AEXQ_QMV_SHAPES(kQ4, 1, true, false, false),  AEXQ_QMV_SHAPES_M8(kQ4, true, false, false),
    AEXQ_QMV_SHAPES(kQ4, 1, false, false, true),  AEXQ_QMV_SHAPES_M8(kQ4, false, false, true),
    AEXQ_QMV_SHAPES(kQ4, 1, true, false, true),   AEXQ_QMV_SHAPES_M8(kQ4, true, false, true),
};

static const QmvEntry* find_qmv(const QmvConfig& c) {
  for (const QmvEntry& e : kQmvTable) {
    const QmvConfig& q = e.cfg;
    if (q.fmt == c.fmt && q.lpr == c.lpr && q.cpl == c.cpl && q.mmax == c.mmax &&
        q.pair == c.pair && q.argmax == c.argmax && q.g16 == c.g16)
      return &e;
  }
  return nullptr;
}

bool qmv_has_config(const QmvConfig& cfg) { return find_qmv(cfg) != nullptr; }

int qmv_rows_per_wg(const QmvConfig& cfg) {
  const QmvEntry* e = find_qmv(cfg);
  return e ? e->rwg : 0;
}

hipError_t qmv_launch(const QmvConfig& cfg, const QmvParams& p, int grid, hipStream_t stream) {
  const QmvEntry* e = find_qmv(cfg);
  if (!e) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(e->fn, dim3(grid), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

int generic_rows_per_wg() { return kWaves; }

hipError_t generic_launch(int fmt, const QmvParams& p, int grid, hipStream_t stream) {
  const dim3 g(grid, (p.m + kGenericM - 1) / kGenericM);
  if (fmt == kQ8)
    hipLaunchKernelGGL(generic_kernel<kQ8>, g, dim3(kThreads), 0, stream, p);
  else
    hipLaunchKernelGGL(generic_kernel<kQ4>, g, dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

int logits_argmax_cols_per_wg() { return kArgmaxCols; }

hipError_t logits_argmax_launch(const float* logits, int m, int n, long long rstride, float* pv,
                                int* pi, float* ps, int parts, hipStream_t stream) {
  hipLaunchKernelGGL(logits_argmax_kernel, dim3(parts, m), dim3(kThreads), 0, stream, logits, n,
                     rstride, pv, pi, ps, parts);
  return hipGetLastError();
}

hipError_t argmax_finalize_launch(const ArgmaxParams& a, hipStream_t stream) {
  hipLaunchKernelGGL(argmax_finalize_kernel, dim3(a.m), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

hipError_t dequant_launch(int fmt, const uint32_t* w, const void* s, int scale_f16, int n, int k,
                          int group, uint32_t xor_mask, float* out, hipStream_t stream) {
  const bool chunked = fmt == kQ8 ? (k % 16 == 0) : (k % 32 == 0);
  const long long work = chunked ? (long long)n * (fmt == kQ8 ? k / 16 : k / 32) : (long long)n * k;
  long long blocks = (work + kThreads - 1) / kThreads;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  if (chunked) {
    if (fmt == kQ8)
      hipLaunchKernelGGL(dequant_chunk_kernel<kQ8>, dim3(blocks), dim3(kThreads), 0, stream, w, s,
                         scale_f16, n, k, group, xor_mask, out);
    else
      hipLaunchKernelGGL(dequant_chunk_kernel<kQ4>, dim3(blocks), dim3(kThreads), 0, stream, w, s,
                         scale_f16, n, k, group, xor_mask, out);
  } else {
    if (fmt == kQ8)
      hipLaunchKernelGGL(dequant_elem_kernel<kQ8>, dim3(blocks), dim3(kThreads), 0, stream, w, s,
                         scale_f16, n, k, group, xor_mask, out);
    else
      hipLaunchKernelGGL(dequant_elem_kernel<kQ4>, dim3(blocks), dim3(kThreads), 0, stream, w, s,
                         scale_f16, n, k, group, xor_mask, out);
  }
  return hipGetLastError();
}

}  // namespace aexq
