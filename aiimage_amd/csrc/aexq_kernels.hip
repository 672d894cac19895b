// Support kernels of the aexq library for gfx950: the element-wise generic
// Gemm (any K, any scale block, fp32 activations, M > 8), argmax over logits
// and its partial merge, dequantization, and the streaming-kernel registry.
//
// Device code layouts (recoded once at upload from the reference's packed
// words, MM:707-734): Q8 bytes hold q + 128, Q4 nibbles hold q + 8.
#include <math.h>

#include "aexq_device.hpp"

namespace aexq {

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
        sv = (int)((w[idx >> 2] >> ((idx & 3) * 8)) & 0xffu) - 128;
      } else {
        sv = (int)((w[idx >> 3] >> ((idx & 7) * 4)) & 0xfu) - 8;
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
      const long long yi = out_index(p, mt, m, r);
      if (yf32)
        ((float*)yb)[yi] = v;
      else
        ((f16*)yb)[yi] = (f16)v;
    }
  }
}

// ---------------------------------------------------------------------------
// RMSNorm-in for M > 1 (CC:4531-4557): one workgroup per activation row
// writes the normalised row as fp16, the activation precision the matmul
// kernels consume.  out[b][m][k] (rows contiguous).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void rmsnorm_rows_kernel(const void* x, int x_f32,
                                                                long long x_rstride,
                                                                long long x_bstride, int m, int k,
                                                                const float* gamma, int gamma_size,
                                                                float eps, f16* out) {
  const int row = blockIdx.x, b = blockIdx.y;
  const long long base = (long long)b * x_bstride + (long long)row * x_rstride;
  float ss = 0.0f;
  for (int i = threadIdx.x; i < k; i += kThreads) {
    const float v = x_f32 ? ((const float*)x)[base + i] : (float)((const f16*)x)[base + i];
    ss = fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  __shared__ float red[kWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) tot += red[w];
  const float inv = rsqrtf(fmaxf(tot / (float)k + eps, 1e-20f));
  f16* o = out + ((long long)b * m + row) * k;
  for (int i = threadIdx.x; i < k; i += kThreads) {
    const float v = x_f32 ? ((const float*)x)[base + i] : (float)((const f16*)x)[base + i];
    float y = v * inv;
    if (gamma) y *= gamma[i < gamma_size - 1 ? i : gamma_size - 1];
    o[i] = (f16)y;
  }
}

hipError_t rmsnorm_rows_launch(const void* x, int x_f32, long long x_rstride, long long x_bstride,
                               int batch, int m, int k, const float* gamma, int gamma_size,
                               float eps, void* out, hipStream_t stream) {
  hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(m, batch), dim3(kThreads), 0, stream, x, x_f32,
                     x_rstride, x_bstride, m, k, gamma, gamma_size, eps, (f16*)out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Argmax over existing logits rows in one launch: workgroup b takes row
// b / parts and that row's column slice b % parts, forms the slice's (best,
// index, second) with the first-maximum rule (MM:645-686), stores it as a
// tagged partial, and the grid's last workgroup merges every row's partials
// (argmax_tail).  VEC logits per load (16 bytes when the rows and slices are
// 16-byte aligned, else 1), kArgmaxLoads loads per thread in flight.
// ---------------------------------------------------------------------------
constexpr int kArgmaxLoads = 8;

template <typename T, bool ROUND, int VEC>
__global__ __launch_bounds__(kThreads) void logits_argmax_kernel(const T* logits, int n,
                                                                 long long rstride, int cols,
                                                                 const QmvParams p) {
  const uint32_t tag = argmax_tag(p);
  const int m = blockIdx.x / p.parts, part = blockIdx.x % p.parts;
  const int c0 = part * cols;
  const int c1 = min(n, c0 + cols);
  const T* row = logits + (long long)m * rstride;
  float bv = __builtin_nanf("");
  int bix = 0x7fffffff;
  float bs = -INFINITY;
  auto take = [&](float v, int c) { argmax_merge(bv, bix, bs, ROUND ? (float)(f16)v : v, c, -INFINITY); };
  constexpr int kStep = kThreads * VEC;
  for (int c = c0 + (int)threadIdx.x * VEC; c < c1; c += kStep * kArgmaxLoads) {
    if constexpr (VEC == 1) {
      float v[kArgmaxLoads];
#pragma unroll
      for (int j = 0; j < kArgmaxLoads; ++j) {
        const int cj = c + j * kStep;
        v[j] = cj < c1 ? (float)row[cj] : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < kArgmaxLoads; ++j)
        if (c + j * kStep < c1) take(v[j], c + j * kStep);
    } else {
      // whole vectors inside the slice; the row's last partial vector
      // element by element
      u32x4 w[kArgmaxLoads];
#pragma unroll
      for (int j = 0; j < kArgmaxLoads; ++j) {
        const int cj = c + j * kStep;
        w[j] = cj + VEC <= c1 ? *(const u32x4*)(row + cj) : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int j = 0; j < kArgmaxLoads; ++j) {
        const int cj = c + j * kStep;
        if (cj + VEC <= c1) {
          const T* e = (const T*)&w[j];
#pragma unroll
          for (int i = 0; i < VEC; ++i) take((float)e[i], cj + i);
        } else {
          for (int i = 0; cj + i < c1; ++i) take((float)row[cj + i], cj + i);
        }
      }
    }
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
    argmax_partial_store(p, (long long)m * p.parts + part, bv, bix, bs, tag);
  }
  argmax_tail<8>(p, tag);
}

// ---------------------------------------------------------------------------
// AQSGET8 record payload -> device layout.  A Q8 (Q4) record's payload is,
// per block of `block` flat elements, an fp32 scale and then the block's int8
// codes (two's-complement nibbles, low nibble = even element; Q8A:94-139).
// Block b starts at byte b * (4 + codes bytes of a full block): every block
// but the last is full.  Thread per output word: the codes land as the packed
// words of ReadPackedArray / ReadQ4PackedArray (Q8A:341-431) already recoded
// to device form (Q8 q + 128, Q4 q + 8; elements past the count are code 0),
// and one thread per block copies its scale.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void record_repack_kernel(const uint8_t* payload,
                                                                 long long count, int block,
                                                                 int bits, uint32_t* codes,
                                                                 float* scales) {
  const long long words = bits == 8 ? (count + 3) / 4 : (count + 7) / 8;
  const long long nblocks = (count + block - 1) / block;
  const long long bstride = 4 + (bits == 8 ? block : (block + 1) / 2);
  const long long total = words > nblocks ? words : nblocks;
  for (long long t = blockIdx.x * (long long)kThreads + threadIdx.x; t < total;
       t += (long long)gridDim.x * kThreads) {
    if (t < words) {
      uint32_t word = 0u;
      if (bits == 8) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const long long idx = t * 4 + e;
          uint32_t b = 0x80u;  // code 0
          if (idx < count) {
            const long long bi = idx / block, i = idx - bi * block;
            b = (uint32_t)payload[bi * bstride + 4 + i] ^ 0x80u;
          }
          word |= b << (8 * e);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const long long idx = t * 8 + e;
          uint32_t nib = 0x8u;  // code 0
          if (idx < count) {
            const long long bi = idx / block, i = idx - bi * block;
            const uint32_t byte = payload[bi * bstride + 4 + (i >> 1)];
            nib = ((byte >> ((i & 1) * 4)) & 0xfu) ^ 0x8u;
          }
          word |= nib << (4 * e);
        }
      }
      codes[t] = word;
    }
    if (t < nblocks) {
      const uint8_t* sp = payload + t * bstride;
      const uint32_t u = (uint32_t)sp[0] | ((uint32_t)sp[1] << 8) | ((uint32_t)sp[2] << 16) |
                         ((uint32_t)sp[3] << 24);
      scales[t] = __builtin_bit_cast(float, u);
    }
  }
}

hipError_t record_repack_launch(const void* payload, long long count, int block, int bits,
                                uint32_t* codes, float* scales, hipStream_t stream) {
  const long long words = bits == 8 ? (count + 3) / 4 : (count + 7) / 8;
  const long long nblocks = (count + block - 1) / block;
  const long long total = words > nblocks ? words : nblocks;
  long long grid = (total + kThreads - 1) / kThreads;
  if (grid > 65536) grid = 65536;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL(record_repack_kernel, dim3((unsigned)grid), dim3(kThreads), 0, stream,
                     (const uint8_t*)payload, count, block, bits, codes, scales);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Dequantization to fp32 [N][K].  Chunk-aligned rows use the same code
// expansion as the matvec kernels; other shapes decode element by element.
// ---------------------------------------------------------------------------
template <int FMT>
__global__ __launch_bounds__(kThreads) void dequant_chunk_kernel(const uint32_t* w, const void* s,
                                                                 int scl16, int n, int k, int group,
                                                                 float* out) {
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
        q4_pairs(v[d], q);
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
                                                                float* out) {
  const long long total = (long long)n * k;
  for (long long idx = blockIdx.x * (long long)kThreads + threadIdx.x; idx < total;
       idx += (long long)gridDim.x * kThreads) {
    int sv;
    long long si;
    if constexpr (FMT == kQ8) {
      sv = (int)((w[idx >> 2] >> ((idx & 3) * 8)) & 0xffu) - 128;
      si = idx / k;
    } else {
      sv = (int)((w[idx >> 3] >> ((idx & 7) * 4)) & 0xfu) - 8;
      si = idx / group;
    }
    out[idx] = (float)sv * load_scale(s, si, scl16);
  }
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
const QmvEntry* qmv_find(const QmvConfig& c) {
  int n = 0;
  const QmvEntry* t = c.fmt == kQ8 ? qmv_table_q8(&n) : qmv_table_q4(&n);
  for (int i = 0; i < n; ++i) {
    const QmvConfig& q = t[i].cfg;
    if (q.lpr == c.lpr && q.cpl == c.cpl && q.u == c.u && q.mmax == c.mmax && q.pair == c.pair &&
        q.argmax == c.argmax && q.gmode == c.gmode)
      return &t[i];
  }
  return nullptr;
}

// Occupancy of each entry, queried once per entry (the device is the same for
// every context of a process that uses one GPU model).
int qmv_blocks_per_cu(const QmvEntry* e) {
  static int cache_q8[512], cache_q4[512];
  int n8 = 0, n4 = 0;
  const QmvEntry* t8 = qmv_table_q8(&n8);
  const QmvEntry* t4 = qmv_table_q4(&n4);
  int* slot = nullptr;
  if (e >= t8 && e < t8 + n8 && e - t8 < 512) slot = &cache_q8[e - t8];
  if (e >= t4 && e < t4 + n4 && e - t4 < 512) slot = &cache_q4[e - t4];
  if (slot && *slot > 0) return *slot;
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, e->fn, kThreads, 0) != hipSuccess ||
      blocks <= 0)
    blocks = 1;
  if (slot) *slot = blocks;
  return blocks;
}

hipError_t qmv_launch(const QmvEntry* e, const QmvParams& p, int grid, hipStream_t stream) {
  if (!e) return hipErrorInvalidConfiguration;
  // a shared activation row is staged once per workgroup in dynamic LDS
  const size_t lds = (p.flags & kFlagXShared) ? qmv_stage_bytes(p.k) : 0;
  hipLaunchKernelGGL(e->fn, dim3(grid), dim3(kThreads), lds, stream, p);
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

// ---------------------------------------------------------------------------
// Largest scale magnitude of a weight (load time): |s| as fp32 bits orders
// like the value, so one unsigned atomicMax per workgroup after a wave and
// workgroup reduction.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void scale_absmax_kernel(const void* s, long long count,
                                                                int f16s, unsigned* out) {
  unsigned m = 0;
  for (long long i = (long long)blockIdx.x * kThreads + threadIdx.x; i < count;
       i += (long long)gridDim.x * kThreads) {
    const float v = f16s ? (float)((const f16*)s)[i] : ((const float*)s)[i];
    const unsigned b = __builtin_bit_cast(unsigned, v) & 0x7fffffffu;
    m = b > m ? b : m;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned o = __shfl_xor(m, off, 64);
    m = o > m ? o : m;
  }
  __shared__ unsigned wm[kWaves];
  if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kWaves; ++w) m = wm[w] > m ? wm[w] : m;
    atomicMax(out, m);
  }
}

hipError_t scale_absmax_launch(const void* scales, long long count, int f16, unsigned* out,
                               hipStream_t stream) {
  if (count <= 0) return hipSuccess;
  long long blocks = (count + kThreads - 1) / kThreads;
  if (blocks > 1024) blocks = 1024;
  hipLaunchKernelGGL(scale_absmax_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, scales,
                     count, f16, out);
  return hipGetLastError();
}

hipError_t logits_argmax_launch(const void* logits, int mode, int n, long long rstride, int cols,
                                int vec, const QmvParams& p, hipStream_t stream) {
  const dim3 grid(p.parts * p.m);
#define AEXQ_ARGMAX_LAUNCH(T, ROUND, VEC)                                                       \
  hipLaunchKernelGGL((logits_argmax_kernel<T, ROUND, VEC>), grid, dim3(kThreads), 0, stream,  \
                     (const T*)logits, n, rstride, cols, p)
  if (mode == kLogitsF16) {
    if (vec > 1) AEXQ_ARGMAX_LAUNCH(f16, false, 8);
    else AEXQ_ARGMAX_LAUNCH(f16, false, 1);
  } else if (mode == kLogitsF32AsF16) {
    if (vec > 1) AEXQ_ARGMAX_LAUNCH(float, true, 4);
    else AEXQ_ARGMAX_LAUNCH(float, true, 1);
  } else {
    if (vec > 1) AEXQ_ARGMAX_LAUNCH(float, false, 4);
    else AEXQ_ARGMAX_LAUNCH(float, false, 1);
  }
#undef AEXQ_ARGMAX_LAUNCH
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Attention head-packed input (the SDPA context o_proj reads, MM:1320-1389:
// AexisReadPack4Channel(arr, dim, row, head)) into dense rows: one thread per
// element of [batch][rows][heads * head_dim].
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kThreads) void head_gather_kernel(const T* src, int rows, int heads,
                                                               int head_dim, long long sbs,
                                                               T* dst) {
  const int width = heads * head_dim;
  const long long per = (long long)rows * width;
  const long long i = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (i >= per) return;
  const int b = blockIdx.y;
  const int row = (int)(i / width), col = (int)(i - (long long)row * width);
  const int head = col / head_dim, d = col - head * head_dim;
  dst[b * per + i] =
      src[b * sbs + (((long long)(head >> 2) * rows + row) * head_dim + d) * 4 + (head & 3)];
}

hipError_t head_gather_launch(const void* src, int f32, int rows, int heads, int head_dim,
                              int batch, long long src_bstride, void* dst, hipStream_t stream) {
  const long long per = (long long)rows * heads * head_dim;
  const long long blocks = (per + kThreads - 1) / kThreads;
  if (blocks <= 0 || blocks > 0x7fffffffLL || batch <= 0 || batch > 65535)
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)blocks, (unsigned)batch);
  if (f32)
    hipLaunchKernelGGL(head_gather_kernel<float>, grid, dim3(kThreads), 0, stream,
                       (const float*)src, rows, heads, head_dim, src_bstride, (float*)dst);
  else
    hipLaunchKernelGGL(head_gather_kernel<f16>, grid, dim3(kThreads), 0, stream,
                       (const f16*)src, rows, heads, head_dim, src_bstride, (f16*)dst);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Split-K fix-up of the MFMA kernels: one thread per stored output element
// (matrix j = blockIdx.y, so its fields are workgroup-uniform scalar loads;
// batch entry b, row, column n < n_store).  The sk_chunks partials
// are summed in chunk order (the result depends on the plan's chunking only,
// never on which workgroup finished first), then the epilogue runs as the
// kernels' finish() runs it (MM:1101 / MM:2301 bias forms, SwiGLU-out,
// residual); columns in [n, n_store) are written as 0.
// ---------------------------------------------------------------------------
template <int NW>
__global__ __launch_bounds__(kThreads) void splitk_reduce_kernel(const QmvParams p, int q8_scale,
                                                                 int sf16) {
  const long long i = (long long)blockIdx.x * kThreads + threadIdx.x;
  const QmvMat& mt = p.mat[blockIdx.y];
  if (!mt.y || i >= (long long)p.batch * p.m * mt.n_store) return;
  const int n = (int)(i % mt.n_store);
  const long long t = i / mt.n_store;
  const int row = (int)(t % p.m), b = (int)(t / p.m);
  const bool yf32 = (p.flags & kFlagYf32) != 0;
  float v = 0.0f;
  if (n < mt.n) {
    const float* src = p.sk_part + mt.sk_off + ((long long)b * p.m + row) * NW * mt.n_store + n;
    // eight chunks' loads in flight at a time, then added in chunk order
    float g = 0.0f, u = 0.0f;
    for (int c0 = 0; c0 < p.sk_chunks; c0 += 8) {
      float gv[8], uv[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const long long o = (long long)(c0 + q) * p.sk_plane;
        gv[q] = c0 + q < p.sk_chunks ? src[o] : 0.0f;
        uv[q] = NW == 2 && c0 + q < p.sk_chunks ? src[o + mt.n_store] : 0.0f;
      }
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (c0 + q < p.sk_chunks) {
          g += gv[q];
          if (NW == 2) u += uv[q];
        }
    }
    float rs0 = 1.0f, rs1 = 1.0f;
    if (q8_scale) {
      const int sb = sf16 ? 2 : 4;
      rs0 = load_scale((const char*)mt.s + b * mt.s_bstride * sb, n, sf16);
      if (NW == 2) rs1 = load_scale((const char*)mt.s2 + b * mt.s_bstride * sb, n, sf16);
    }
    v = gemm_epilogue(p, p.m_base + row, n, g * rs0);
    if (NW == 2) v = silu(v) * gemm_epilogue(p, p.m_base + row, n, u * rs1);
    if (mt.res && (p.flags & kFlagResidual)) {
      const char* rb = (const char*)mt.res + b * mt.r_bstride * (yf32 ? 4 : 2);
      const long long ri = (long long)row * p.r_rstride + n;
      v += yf32 ? ((const float*)rb)[ri] : (float)((const f16*)rb)[ri];
    }
  }
  char* yb = (char*)mt.y + b * mt.y_bstride * (yf32 ? 4 : 2);
  const long long yi = out_index(p, mt, row, n);
  if (yf32)
    ((float*)yb)[yi] = v;
  else
    ((f16*)yb)[yi] = (f16)v;
}

hipError_t splitk_reduce_launch(const QmvParams& p, int nw, int q8_scale, int sf16,
                                hipStream_t stream) {
  long long most = 0;  // outputs of the largest matrix
  for (int j = 0; j < p.nmat; ++j) {
    const long long cnt = (long long)p.batch * p.m * p.mat[j].n_store;
    most = cnt > most ? cnt : most;
  }
  const long long blocks = (most + kThreads - 1) / kThreads;
  if (blocks <= 0 || blocks > 0x7fffffffLL || p.nmat < 1 || p.nmat > kMaxGroup ||
      p.sk_chunks < 2 || !p.sk_part)
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)blocks, (unsigned)p.nmat);
  if (nw == 2)
    hipLaunchKernelGGL(splitk_reduce_kernel<2>, grid, dim3(kThreads), 0, stream, p, q8_scale,
                       sf16);
  else
    hipLaunchKernelGGL(splitk_reduce_kernel<1>, grid, dim3(kThreads), 0, stream, p, q8_scale,
                       sf16);
  return hipGetLastError();
}

hipError_t dequant_launch(int fmt, const uint32_t* w, const void* s, int scale_f16, int n, int k,
                          int group, float* out, hipStream_t stream) {
  const bool chunked = fmt == kQ8 ? (k % 16 == 0) : (k % 32 == 0);
  const long long work = chunked ? (long long)n * (fmt == kQ8 ? k / 16 : k / 32) : (long long)n * k;
  long long blocks = (work + kThreads - 1) / kThreads;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  if (chunked) {
    if (fmt == kQ8)
      hipLaunchKernelGGL(dequant_chunk_kernel<kQ8>, dim3(blocks), dim3(kThreads), 0, stream, w, s,
                         scale_f16, n, k, group, out);
    else
      hipLaunchKernelGGL(dequant_chunk_kernel<kQ4>, dim3(blocks), dim3(kThreads), 0, stream, w, s,
                         scale_f16, n, k, group, out);
  } else {
    if (fmt == kQ8)
      hipLaunchKernelGGL(dequant_elem_kernel<kQ8>, dim3(blocks), dim3(kThreads), 0, stream, w, s,
                         scale_f16, n, k, group, out);
    else
      hipLaunchKernelGGL(dequant_elem_kernel<kQ4>, dim3(blocks), dim3(kThreads), 0, stream, w, s,
                         scale_f16, n, k, group, out);
  }
  return hipGetLastError();
}

}  // namespace aexq
