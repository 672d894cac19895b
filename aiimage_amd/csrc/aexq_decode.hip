// Decode-step kernels around the quantized linears (gfx950): the tied Q8 token
// embedding, RoPE with KV-cache append, GQA decode attention over an fp16 KV
// cache (split over positions, then combined), and a standalone RMSNorm.
//
// Reference semantics (paths relative to the reference root):
//   embedding gather   Qwen35SharedTokenEmbeddingWeights.cs:185-198, BT:13-26
//   RoPE (rotate-half) AexisKernels.Pack4PointwiseNorm.hlsl:414-473
//   SDPA               AexisKernels.Pack4Matmul.hlsl:420-544 (scale, max-subtracted
//                      softmax divided by max(sum, 1e-20), GQA key head = head / group)
#include <math.h>

#include "aexq_device.hpp"

namespace aexq {

// ---------------------------------------------------------------------------
// Embedding: out[m][d] = fp16(q[tok_m][d] * scale[tok_m]) from the device Q8
// copy (bytes hold q + 128).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void embed_q8_kernel(const uint32_t* codes,
                                                            const void* scales, int scale_f16,
                                                            int k, const int32_t* tokens,
                                                            int vocab, f16* out) {
  const int m = blockIdx.x;
  int tok = tokens[m];
  tok = tok < 0 ? 0 : (tok >= vocab ? vocab - 1 : tok);
  const float s = load_scale(scales, tok, scale_f16 != 0);
  const uint8_t* row = (const uint8_t*)codes + (long long)tok * k;
  for (int d = threadIdx.x; d < k; d += kThreads)
    out[(long long)m * k + d] = (f16)((float)((int)row[d] - 128) * s);
}

hipError_t embed_q8_launch(const uint32_t* codes, const void* scales, int scale_f16, int k,
                           const int32_t* tokens, int m, int vocab, void* out,
                           hipStream_t stream) {
  hipLaunchKernelGGL(embed_q8_kernel, dim3(m), dim3(kThreads), 0, stream, codes, scales,
                     scale_f16, k, tokens, vocab, (f16*)out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// RoPE + KV append for one decode position.  q [hq][d], k/v [hkv][d] (fp16,
// rows contiguous); caches [hkv][cap][d].  cos/sin hold the position's
// d/2 table entries (fp32).  One workgroup per head (q heads, then kv heads);
// q is rotated in place, k is rotated into the cache, v is copied.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void rope_kv_kernel(f16* q, const f16* k, const f16* v,
                                                           f16* kcache, f16* vcache, int hq,
                                                           int hkv, int d, int cap, int pos,
                                                           const float* cosv,
                                                           const float* sinv) {
  const int head = blockIdx.x;
  const int half = d / 2;
  for (int j = threadIdx.x; j < half; j += kThreads) {
    const float c = cosv[j], s = sinv[j];
    if (head < hq) {
      f16* row = q + (long long)head * d;
      const float x0 = (float)row[j], x1 = (float)row[j + half];
      row[j] = (f16)(x0 * c - x1 * s);
      row[j + half] = (f16)(x0 * s + x1 * c);
    } else {
      const int g = head - hq;
      const f16* kr = k + (long long)g * d;
      const float x0 = (float)kr[j], x1 = (float)kr[j + half];
      f16* kc = kcache + ((long long)g * cap + pos) * d;
      kc[j] = (f16)(x0 * c - x1 * s);
      kc[j + half] = (f16)(x0 * s + x1 * c);
      const f16* vr = v + (long long)g * d;
      f16* vc = vcache + ((long long)g * cap + pos) * d;
      vc[j] = vr[j];
      vc[j + half] = vr[j + half];
    }
  }
}

hipError_t rope_kv_launch(void* q, const void* k, const void* v, void* kcache, void* vcache,
                          int hq, int hkv, int d, int cap, int pos, const float* cosv,
                          const float* sinv, hipStream_t stream) {
  hipLaunchKernelGGL(rope_kv_kernel, dim3(hq + hkv), dim3(kThreads), 0, stream, (f16*)q,
                     (const f16*)k, (const f16*)v, (f16*)kcache, (f16*)vcache, hq, hkv, d, cap,
                     pos, cosv, sinv);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// GQA decode attention, split over positions.  Workgroup (kv head g, split c)
// covers positions [c * kAttnChunk, ...) of length `len` for the G = hq / hkv
// query heads of g: every cached K and V row is read once.  Thread t scores
// position t / G for head t % G (the G threads of a position read the same K
// row); then thread t accumulates output dimension t for every head.  The
// partial (max, sum, acc[d]) goes to part[h][split]; the combine kernel merges
// the splits.  d == kAttnDim, G * kAttnChunk == kAttnThreads.
// ---------------------------------------------------------------------------
constexpr int kAttnDim = 128;
constexpr int kAttnThreads = 128;
constexpr int kAttnChunk = 32;  // positions per split for G = 4

template <int G>
__global__ __launch_bounds__(kAttnThreads) void attn_split_kernel(
    const f16* q, const f16* kcache, const f16* vcache, int cap, int len, float scale, int splits,
    float* part, const f16* knew, const f16* vnew, f16* kcache_w, f16* vcache_w,
    const float* cosv, const float* sinv) {
  // knew != nullptr: fused RoPE + append.  q and the new k row are rotated here
  // (rounded to fp16 as a separate RoPE launch would store them); the split that
  // covers position len - 1 writes the new K/V rows to the cache and every
  // split uses the rotated q.
  constexpr int CH = kAttnThreads / G;  // positions per split
  const int g = blockIdx.x, c = blockIdx.y;
  const int t = threadIdx.x;
  __shared__ float qs[G][kAttnDim];
  __shared__ float ps[G][CH];
  __shared__ float stat[G][2];
  const bool rope = knew != nullptr;
  const int half = kAttnDim / 2;
  if (rope) {
    for (int i = t; i < G * half; i += kAttnThreads) {
      const int h = i / half, j = i % half;
      const f16* qr = q + ((long long)g * G + h) * kAttnDim;
      const float x0 = (float)qr[j], x1 = (float)qr[j + half];
      qs[h][j] = (float)(f16)(x0 * cosv[j] - x1 * sinv[j]);
      qs[h][j + half] = (float)(f16)(x0 * sinv[j] + x1 * cosv[j]);
    }
    const int pos = len - 1;
    if (pos / CH == c) {
      for (int j = t; j < half; j += kAttnThreads) {
        const f16* kr = knew + (long long)g * kAttnDim;
        const float x0 = (float)kr[j], x1 = (float)kr[j + half];
        f16* kc = kcache_w + ((long long)g * cap + pos) * kAttnDim;
        kc[j] = (f16)(x0 * cosv[j] - x1 * sinv[j]);
        kc[j + half] = (f16)(x0 * sinv[j] + x1 * cosv[j]);
        f16* vc = vcache_w + ((long long)g * cap + pos) * kAttnDim;
        vc[j] = vnew[(long long)g * kAttnDim + j];
        vc[j + half] = vnew[(long long)g * kAttnDim + j + half];
      }
    }
  } else {
    for (int i = t; i < G * kAttnDim; i += kAttnThreads)
      qs[i / kAttnDim][i % kAttnDim] =
          (float)q[((long long)g * G + i / kAttnDim) * kAttnDim + i % kAttnDim];
  }
  // the appended rows are read back below by other threads of this workgroup
  __syncthreads();

  const int p0 = c * CH;
  {
    const int pl = t / G, h = t % G;
    const int p = p0 + pl;
    float s = -INFINITY;
    if (p < len) {
      const u32x4* kr = (const u32x4*)(kcache + ((long long)g * cap + p) * kAttnDim);
      float acc = 0.0f;
#pragma unroll 4
      for (int v = 0; v < kAttnDim / 8; ++v) {
        const u32x4 w = kr[v];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const f16x2 kk = as_h2(w[e]);
          acc = fmaf(qs[h][8 * v + 2 * e], (float)kk[0], acc);
          acc = fmaf(qs[h][8 * v + 2 * e + 1], (float)kk[1], acc);
        }
      }
      s = acc * scale;
    }
    ps[h][pl] = s;
  }
  __syncthreads();
  if (t < G) {
    float mx = -INFINITY;
    for (int i = 0; i < CH; ++i) mx = fmaxf(mx, ps[t][i]);
    float sum = 0.0f;
    for (int i = 0; i < CH; ++i) {
      const float e = ps[t][i] == -INFINITY ? 0.0f : __expf(ps[t][i] - mx);
      ps[t][i] = e;
      sum += e;
    }
    stat[t][0] = mx;
    stat[t][1] = sum;
  }
  __syncthreads();
  // thread t: output dimension t of every head
  float acc[G];
#pragma unroll
  for (int h = 0; h < G; ++h) acc[h] = 0.0f;
  const int n = len - p0 < CH ? len - p0 : CH;
  for (int i = 0; i < n; ++i) {
    const float vv = (float)vcache[((long long)g * cap + p0 + i) * kAttnDim + t];
#pragma unroll
    for (int h = 0; h < G; ++h) acc[h] = fmaf(ps[h][i], vv, acc[h]);
  }
  const int stride = kAttnDim + 2;
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float* o = part + ((long long)(g * G + h) * splits + c) * stride;
    o[2 + t] = acc[h];
    if (t == 0) {
      o[0] = stat[h][0];
      o[1] = stat[h][1];
    }
  }
}

// Merges the splits of each query head: M = max m_s, L = sum l_s e^(m_s - M),
// out = sum acc_s e^(m_s - M) / max(L, 1e-20), stored fp16 [hq][d].  The split
// statistics are staged in LDS with one load per thread, so no thread walks a
// chain of dependent loads; thread t then sums dimension t over the splits.
constexpr int kMaxSplits = 1024;

__global__ __launch_bounds__(kAttnThreads) void attn_combine_kernel(const float* part, int splits,
                                                                    f16* out) {
  const int h = blockIdx.x, t = threadIdx.x;
  const int stride = kAttnDim + 2;
  const float* ph = part + (long long)h * splits * stride;
  __shared__ float wm[kMaxSplits];
  __shared__ float red[kAttnThreads / 64];
  float mx = -INFINITY;
  for (int s = t; s < splits; s += kAttnThreads) {
    wm[s] = ph[(long long)s * stride];
    mx = fmaxf(mx, wm[s]);
  }
  mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 4, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 8, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  if ((t & 63) == 0) red[t >> 6] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int w = 1; w < kAttnThreads / 64; ++w) mx = fmaxf(mx, red[w]);
  __syncthreads();
  float lsum = 0.0f;
  for (int s = t; s < splits; s += kAttnThreads) {
    const float w = wm[s] == -INFINITY ? 0.0f : __expf(wm[s] - mx);
    wm[s] = w;
    lsum = fmaf(ph[(long long)s * stride + 1], w, lsum);
  }
  lsum = wave_sum(lsum);
  __syncthreads();
  if ((t & 63) == 0) red[t >> 6] = lsum;
  __syncthreads();
  float l = 0.0f;
#pragma unroll
  for (int w = 0; w < kAttnThreads / 64; ++w) l += red[w];
  float acc = 0.0f;
#pragma unroll 8
  for (int s = 0; s < splits; ++s) acc = fmaf(ph[(long long)s * stride + 2 + t], wm[s], acc);
  out[(long long)h * kAttnDim + t] = (f16)(acc / fmaxf(l, 1e-20f));
}

int attn_splits(int len, int group) { return (len + kAttnThreads / group - 1) / (kAttnThreads / group); }

hipError_t attn_decode_launch(const void* q, const void* kcache, const void* vcache, int hq,
                              int hkv, int cap, int len, float scale, float* part, void* out,
                              const void* knew, const void* vnew, const float* cosv,
                              const float* sinv, hipStream_t stream) {
  const int group = hq / hkv;
  const int splits = attn_splits(len, group);
  if (splits > kMaxSplits) return hipErrorInvalidValue;
  const dim3 grid(hkv, splits);
#define AEXQ_ATTN(G)                                                                            \
  hipLaunchKernelGGL(attn_split_kernel<G>, grid, dim3(kAttnThreads), 0, stream, (const f16*)q,  \
                     (const f16*)kcache, (const f16*)vcache, cap, len, scale, splits, part,     \
                     (const f16*)knew, (const f16*)vnew, (f16*)kcache, (f16*)vcache, cosv, sinv)
  switch (group) {
    case 1: AEXQ_ATTN(1); break;
    case 2: AEXQ_ATTN(2); break;
    case 4: AEXQ_ATTN(4); break;
    case 8: AEXQ_ATTN(8); break;
    default: return hipErrorInvalidValue;
  }
#undef AEXQ_ATTN
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(hq), dim3(kAttnThreads), 0, stream, part, splits,
                     (f16*)out);
  return hipGetLastError();
}

}  // namespace aexq
