// Decode-step kernels around the quantized linears (gfx950): the tied Q8 token
// embedding, RoPE with KV-cache append, GQA decode attention over an fp16 KV
// cache (split over positions, the splits merged by the last one to finish),
// and a standalone RMSNorm.
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
// GQA decode attention in one launch.  Workgroup (kv head g, split c) covers
// positions [64 c, 64 c + 64) of the `len` cached ones for the G = hq / hkv
// query heads of g, so every cached K and V row is read once.  Every load of
// the workgroup -- q, the RoPE tables and new row, then its K and V rows --
// is issued before the first wait, and q (rotated here when RoPE is fused)
// meets K after one barrier:
//   scores   lanes 4i..4i+3 own position p0 + i, lane 4i + j the dims
//            32 r + 8 j + [0, 8) for r < 4 (so one load instruction covers 64
//            contiguous bytes of 16 rows), for all G heads (v_dot2 with fp32
//            accumulation, quad reduction);
//   softmax  max / sum per head over the split's positions (wave shuffles,
//            then LDS across the 4 waves);
//   P V      wave w owns positions p0 + 16 w + [0, 16), lane l dimensions
//            2l and 2l + 1; the four waves' sums meet in LDS.
// The split's (max, sum, acc[128]) per head goes to part[h][split].  The last
// workgroup of kv head g to finish (a device-scope counter that the same
// workgroup resets to 0, so the launch needs no clearing and replays inside a
// graph) merges the splits of its G heads:
//   M = max m_s, L = sum l_s e^(m_s - M), out = sum acc_s e^(m_s - M) / max(L, 1e-20).
// head_dim == 128.
// ---------------------------------------------------------------------------
constexpr int kAttnDim = 128;
constexpr int kAttnThreads = 256;

// Device-coherent (agent scope) fp32 store / load: written through to, and
// read from, the level all XCDs share.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
constexpr int kAttnPos = 64;         // positions per split
constexpr int kAttnStride = kAttnDim + 4;  // partial row: max, sum, 2 pad, acc[128] (16-byte aligned)
constexpr int kCoherentAux = 16;     // buffer-load cache policy sc1: read at agent coherence
// One counter per 256-byte line: atomics to one line are serialized where they
// are performed (about 15 ns each), so the kv heads' counters do not share one.
constexpr int kAttnCounterStride = 64;
constexpr int kAttnMaxSplits = 512;  // combine staging in LDS

template <int G>
__global__ __launch_bounds__(kAttnThreads) void attn_decode_kernel(
    const f16* q, const f16* kcache, const f16* vcache, int cap, int len, float scale,
    int splits, float* part, int* counters, f16* out, const f16* knew, const f16* vnew,
    f16* kcache_w, f16* vcache_w, const float* cosv, const float* sinv, const int* posp) {
  const int g = blockIdx.x, c = blockIdx.y;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  constexpr int half = kAttnDim / 2;
  if (posp) {
    // decode position in device memory (a captured graph advances it): the
    // grid covers the cache capacity, the tables hold [cap][half] rows
    const int pp = min(max(*posp, 0), cap - 1);
    len = pp + 1;
    cosv += (long long)pp * half;
    sinv += (long long)pp * half;
  }
  const int live_splits = (len + kAttnPos - 1) / kAttnPos;
  const int p0 = c * kAttnPos;
  const int pl = t >> 2, qq = t & 3;  // scores: position p0 + pl, dims 32 qq .. 32 qq + 31
  const bool rope = knew != nullptr;
  const int pos = len - 1;             // the appended position when RoPE is fused
  const bool has_new = rope && pos >= p0 && pos < p0 + kAttnPos;
  const long long head_off = (long long)g * cap * kAttnDim;
  // P V sums: the four waves of a split, then the merge's eight row groups
  __shared__ __align__(16) float pv[kAttnThreads / 32][G][kAttnDim];
  __shared__ int last;
  if (c >= live_splits) {
    // a split past the live length (the grid was sized for the capacity):
    // nothing to score, but it still counts in so the merge starts once
    if (t == 0) last = atomicAdd(&counters[g * kAttnCounterStride], 1) == splits - 1;
    __syncthreads();
    if (!last) return;
  } else {

    // 1. loads, all issued before the first wait; q and the new row first, so
    // that waiting for them leaves the K/V loads in flight.  Absent tables and
    // rows come through empty buffer resources (they read 0).
    constexpr int QI = (G * half + kAttnThreads - 1) / kAttnThreads;  // (head, j) pairs per thread
    float qa[QI], qb[QI], cs[QI], sn[QI];
    const __amdgpu_buffer_rsrc_t trs_c = __builtin_amdgcn_make_buffer_rsrc(
        (void*)cosv, (short)0, rope ? half * 4 : 0, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t trs_s = __builtin_amdgcn_make_buffer_rsrc(
        (void*)sinv, (short)0, rope ? half * 4 : 0, kBufferRsrcWord3);
#pragma unroll
    for (int r = 0; r < QI; ++r) {
      const int i = min(t + r * kAttnThreads, G * half - 1);
      const int h = i / half, j = i % half;
      const f16* qr = q + ((long long)g * G + h) * kAttnDim;
      qa[r] = (float)qr[j];
      qb[r] = (float)qr[j + half];
      cs[r] = as_f32(__builtin_amdgcn_raw_buffer_load_b32(trs_c, j * 4, 0, 0));
      sn[r] = as_f32(__builtin_amdgcn_raw_buffer_load_b32(trs_s, j * 4, 0, 0));
    }
    const int jn = t & (half - 1);
    const __amdgpu_buffer_rsrc_t nrs_k = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(rope ? knew + (long long)g * kAttnDim : q), (short)0, has_new ? kAttnDim * 2 : 0,
        kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t nrs_v = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(rope ? vnew + (long long)g * kAttnDim : q), (short)0, has_new ? kAttnDim * 2 : 0,
        kBufferRsrcWord3);
    const uint32_t kn0 = __builtin_amdgcn_raw_buffer_load_b16(nrs_k, jn * 2, 0, 0);
    const uint32_t kn1 = __builtin_amdgcn_raw_buffer_load_b16(nrs_k, (jn + half) * 2, 0, 0);
    const uint32_t vn0 = __builtin_amdgcn_raw_buffer_load_b16(nrs_v, jn * 2, 0, 0);
    const uint32_t vn1 = __builtin_amdgcn_raw_buffer_load_b16(nrs_v, (jn + half) * 2, 0, 0);
    const float tc = as_f32(__builtin_amdgcn_raw_buffer_load_b32(trs_c, jn * 4, 0, 0));
    const float ts = as_f32(__builtin_amdgcn_raw_buffer_load_b32(trs_s, jn * 4, 0, 0));
    __builtin_amdgcn_sched_barrier(0);  // keeps the q-side loads ahead of K and V
    // K rows of the split (rows >= len read 0): position p0 + pl, 64 bytes per lane
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(kcache + head_off), (short)0, len * kAttnDim * 2, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(vcache + head_off), (short)0, len * kAttnDim * 2, kBufferRsrcWord3);
    u32x4 kreg[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      kreg[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                              krs, (p0 + pl) * 256 + i * 64 + qq * 16, 0, 0));
    // V rows: wave w owns positions p0 + 16 w + [0, 16), lane l dimensions 2l, 2l + 1
    uint32_t vreg[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
      vreg[i] = __builtin_amdgcn_raw_buffer_load_b32(
          vrs, ((p0 + 16 * wave + i) * kAttnDim + 2 * lane) * 2, 0, 0);

    // 2. q of the G heads (rotated and rounded to fp16 when RoPE is fused) and,
    // in the split that holds it, the appended K/V row
    __shared__ __align__(16) f16 qs[G][kAttnDim];
    __shared__ __align__(16) f16 kn[kAttnDim];
    __shared__ __align__(16) f16 vn[kAttnDim];
#pragma unroll
    for (int r = 0; r < QI; ++r) {
      const int i = t + r * kAttnThreads;
      if (i < G * half) {
        const int h = i / half, j = i % half;
        qs[h][j] = rope ? (f16)(qa[r] * cs[r] - qb[r] * sn[r]) : (f16)qa[r];
        qs[h][j + half] = rope ? (f16)(qa[r] * sn[r] + qb[r] * cs[r]) : (f16)qb[r];
      }
    }
    if (has_new && t < half) {
      const float x0 = (float)__builtin_bit_cast(f16, (uint16_t)kn0);
      const float x1 = (float)__builtin_bit_cast(f16, (uint16_t)kn1);
      const f16 k0 = (f16)(x0 * tc - x1 * ts), k1 = (f16)(x0 * ts + x1 * tc);
      const f16 v0 = __builtin_bit_cast(f16, (uint16_t)vn0);
      const f16 v1 = __builtin_bit_cast(f16, (uint16_t)vn1);
      kn[t] = k0;
      kn[t + half] = k1;
      vn[t] = v0;
      vn[t + half] = v1;
      f16* kc = kcache_w + head_off + (long long)pos * kAttnDim;
      f16* vc = vcache_w + head_off + (long long)pos * kAttnDim;
      kc[t] = k0;
      kc[t + half] = k1;
      vc[t] = v0;
      vc[t + half] = v1;
    }
    __syncthreads();
    if (has_new) {
      // the cache row at `pos` was loaded before it was written: take the new one
      if (p0 + pl == pos) {
#pragma unroll
        for (int i = 0; i < 4; ++i) kreg[i] = *(const u32x4*)&kn[i * 32 + qq * 8];
      }
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (p0 + 16 * wave + i == pos) vreg[i] = *(const uint32_t*)&vn[2 * lane];
    }

    // 3. scores of position p0 + pl for every head (quad sums by DPP)
    const bool live = p0 + pl < len;
    float sc[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4 qw = *(const u32x4*)&qs[h][i * 32 + qq * 8];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = dot2(kreg[i][e], qw[e], acc);
      }
      sc[h] = acc;
    }
#pragma unroll
    for (int h = 0; h < G; ++h) sc[h] += dpp<0xB1>(sc[h]);  // quad_perm [1,0,3,2]
#pragma unroll
    for (int h = 0; h < G; ++h) {
      sc[h] += dpp<0x4E>(sc[h]);  // quad_perm [2,3,0,1]
      sc[h] = live ? sc[h] * scale : -INFINITY;
    }

    // 4. softmax statistics of the split per head: the 16 positions of a wave
    // reduce within DPP rows (row_ror 4, 8), then across rows with the lane
    // shuffles of all heads issued together; the 4 waves meet in LDS
    __shared__ float red[kAttnThreads / 64][G];
    __shared__ float es[G][kAttnPos];
    float mx[G], rr[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      rr[h] = fmaxf(sc[h], dpp<0x124>(sc[h]));
      rr[h] = fmaxf(rr[h], dpp<0x128>(rr[h]));
    }
#pragma unroll
    for (int h = 0; h < G; ++h) rr[h] = fmaxf(rr[h], __shfl_xor(rr[h], 16, 64));
#pragma unroll
    for (int h = 0; h < G; ++h) rr[h] = fmaxf(rr[h], __shfl_xor(rr[h], 32, 64));
    if (lane == 0) {
#pragma unroll
      for (int h = 0; h < G; ++h) red[wave][h] = rr[h];
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float m = red[0][h];
#pragma unroll
      for (int w = 1; w < kAttnThreads / 64; ++w) m = fmaxf(m, red[w][h]);
      mx[h] = m;  // finite: every split holds at least one live position
    }
    __syncthreads();
    float ex[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      ex[h] = live ? __expf(sc[h] - mx[h]) : 0.0f;
      rr[h] = ex[h] + dpp<0x124>(ex[h]);
      rr[h] += dpp<0x128>(rr[h]);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) rr[h] += __shfl_xor(rr[h], 16, 64);
#pragma unroll
    for (int h = 0; h < G; ++h) rr[h] += __shfl_xor(rr[h], 32, 64);
    if (qq == 0) {
#pragma unroll
      for (int h = 0; h < G; ++h) es[h][pl] = ex[h];
    }
    if (lane == 0) {
#pragma unroll
      for (int h = 0; h < G; ++h) red[wave][h] = rr[h];
    }
    __syncthreads();
    float sm[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float s = 0.0f;
#pragma unroll
      for (int w = 0; w < kAttnThreads / 64; ++w) s += red[w][h];
      sm[h] = s;
    }

    // 5. P V: wave w, dimensions 2 lane and 2 lane + 1 over its 16 positions;
    // the four waves' sums meet in LDS
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float e = es[h][16 * wave + i];
        const f16x2 vv = as_h2(vreg[i]);
        a0 = fmaf(e, (float)vv[0], a0);
        a1 = fmaf(e, (float)vv[1], a1);
      }
      pv[wave][h][2 * lane] = a0;
      pv[wave][h][2 * lane + 1] = a1;
    }
    __syncthreads();
    const int d = t & (kAttnDim - 1), vh = t >> 7;
    if (vh == 0) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float a = 0.0f;
#pragma unroll
        for (int w = 0; w < kAttnThreads / 64; ++w) a += pv[w][h][d];
        float* o = part + ((long long)(g * G + h) * splits + c) * kAttnStride;
        store_coherent(o + 4 + d, a);
        if (d == 0) {
          store_coherent(o, mx[h]);
          store_coherent(o + 1, sm[h]);
        }
      }
    }

    // 6. the last split of kv head g merges all of them.  Partials travel
    // through device-coherent stores and loads (they bypass the per-XCD L2
    // that plain accesses would leave stale), ordered by waiting for the
    // stores before the counter increment.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t == 0) last = atomicAdd(&counters[g * kAttnCounterStride], 1) == splits - 1;
    __syncthreads();
    if (!last) return;
  }
  // Loads of the merge: the split statistics (row t of the G * splits rows
  // (head, split) in registers), then the first chunk of accumulator rows, all
  // in flight together.  Thread (rg = t / 32, dq = t % 32) reads dims 4 dq ..
  // 4 dq + 3 of splits rg + 8 j of every head; splits past the last live one
  // are sent out of the buffer range, which reads 0.  Rows keep the grid's
  // pitch (`splits`); only the first live_splits of each head hold partials
  // of this launch.
  const int nsp = live_splits;
  __shared__ float cm[G * kAttnMaxSplits];  // split maxima, then weights
  __shared__ float cl[G * kAttnMaxSplits];  // split sums
  const int rows = G * splits;
  const float* pg = part + (long long)g * rows * kAttnStride;
  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)pg, (short)0, rows * kAttnStride * 4, kBufferRsrcWord3);
  constexpr int JJ = 16 / G;  // accumulator rows per head and thread in one chunk
  constexpr int kChunk = 8 * JJ;
  const int dq = t & 31, rg = t >> 5;
  const float m0 = as_f32(__builtin_amdgcn_raw_buffer_load_b32(prs, t * kAttnStride * 4, 0, kCoherentAux));
  const float l0 = as_f32(__builtin_amdgcn_raw_buffer_load_b32(prs, (t * kAttnStride + 1) * 4, 0, kCoherentAux));
  u32x4 av[G][JJ];
  auto issue = [&](int s0) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int j = 0; j < JJ; ++j) {
        const int s2 = s0 + rg + 8 * j;
        const int off = s2 < nsp ? ((h * splits + s2) * kAttnStride + 4 + 4 * dq) * 4 : 0x7FFFFFF0;
        av[h][j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, off, 0, kCoherentAux));
      }
  };
  issue(0);
  if (t < rows) {
    const bool ok = t % splits < nsp;
    cm[t] = ok ? m0 : -INFINITY;
    cl[t] = ok ? l0 : 0.0f;
  }
  for (int i = t + kAttnThreads; i < rows; i += kAttnThreads) {
    const bool ok = i % splits < nsp;
    cm[i] = ok ? as_f32(__builtin_amdgcn_raw_buffer_load_b32(prs, i * kAttnStride * 4, 0, kCoherentAux))
               : -INFINITY;
    cl[i] = ok ? as_f32(__builtin_amdgcn_raw_buffer_load_b32(prs, (i * kAttnStride + 1) * 4, 0, kCoherentAux))
               : 0.0f;
  }
  __syncthreads();
  // per head: M = max m_s (each wave reduces the heads h == wave mod 4)
  __shared__ float hm[G], hl[G];
  for (int h = wave; h < G; h += kAttnThreads / 64) {
    float m = -INFINITY;
    for (int s2 = lane; s2 < nsp; s2 += 64) m = fmaxf(m, cm[h * splits + s2]);
    m = wave_max(m);
    float l = 0.0f;
    for (int s2 = lane; s2 < nsp; s2 += 64) {
      const float w = __expf(cm[h * splits + s2] - m);
      cm[h * splits + s2] = w;
      l = fmaf(cl[h * splits + s2], w, l);
    }
    l = wave_sum(l);
    if (lane == 0) {
      hm[h] = m;
      hl[h] = l;
    }
  }
  __syncthreads();
  float ac[G][4];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 4; ++e) ac[h][e] = 0.0f;
  for (int s0 = 0;;) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int j = 0; j < JJ; ++j) {
        const int s2 = min(s0 + rg + 8 * j, nsp - 1);  // rows past the end loaded 0
        const float w = cm[h * splits + s2];
#pragma unroll
        for (int e = 0; e < 4; ++e) ac[h][e] = fmaf(as_f32(av[h][j][e]), w, ac[h][e]);
      }
    s0 += kChunk;
    if (s0 >= nsp) break;
    issue(s0);
  }
  // the eight row groups' sums meet in LDS
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const f32x4 v = {ac[h][0], ac[h][1], ac[h][2], ac[h][3]};
    *(f32x4*)&pv[rg][h][4 * dq] = v;
  }
  __syncthreads();
  for (int i = t; i < G * kAttnDim; i += kAttnThreads) {
    const int h = i / kAttnDim, dd = i % kAttnDim;
    float a = 0.0f;
#pragma unroll
    for (int w = 0; w < kAttnThreads / 32; ++w) a += pv[w][h][dd];
    out[((long long)g * G + h) * kAttnDim + dd] = (f16)(a / fmaxf(hl[h], 1e-20f));
  }
  if (t == 0) counters[g * kAttnCounterStride] = 0;  // ready for the next launch
}

// ---------------------------------------------------------------------------
// End of a decode step (Qwen35DecoderSession.Generate, DEC:1160-1237: the
// argmax becomes the next input token and the position advances), done on the
// device so that one captured step replays token after token.
// ---------------------------------------------------------------------------
__global__ void decode_advance_kernel(int* position, int* token, const int* argmax,
                                      int* tokens_out, int out_cap) {
  const int pos = *position;
  const int tok = *argmax;
  if (tokens_out && pos >= 0 && pos < out_cap) tokens_out[pos] = tok;
  *token = tok;
  *position = pos + 1;
}

hipError_t decode_advance_launch(int* position, int* token, const int* argmax, int* tokens_out,
                                 int out_cap, hipStream_t stream) {
  hipLaunchKernelGGL(decode_advance_kernel, dim3(1), dim3(1), 0, stream, position, token, argmax,
                     tokens_out, out_cap);
  return hipGetLastError();
}

int attn_splits(int len) { return (len + kAttnPos - 1) / kAttnPos; }
int attn_max_splits() { return kAttnMaxSplits; }
int attn_part_stride() { return kAttnStride; }
int attn_counter_stride() { return kAttnCounterStride; }

hipError_t attn_decode_launch(const void* q, const void* kcache, const void* vcache, int hq,
                              int hkv, int cap, int len, float scale, float* part, int* counters,
                              void* out, const void* knew, const void* vnew, const float* cosv,
                              const float* sinv, const int* posp, hipStream_t stream) {
  const int group = hq / hkv;
  // a device-side position: the grid covers the capacity, the kernel reads
  // the live length
  if (posp) len = cap;
  const int splits = attn_splits(len);
  if (splits > kAttnMaxSplits) return hipErrorInvalidValue;
  const dim3 grid(hkv, splits);
#define AEXQ_ATTN(G)                                                                             \
  hipLaunchKernelGGL(attn_decode_kernel<G>, grid, dim3(kAttnThreads), 0, stream, (const f16*)q, \
                     (const f16*)kcache, (const f16*)vcache, cap, len, scale, splits, part,      \
                     counters, (f16*)out, (const f16*)knew, (const f16*)vnew, (f16*)kcache,      \
                     (f16*)vcache, cosv, sinv, (const int*)posp)
  switch (group) {
    case 1: AEXQ_ATTN(1); break;
    case 2: AEXQ_ATTN(2); break;
    case 4: AEXQ_ATTN(4); break;
    case 8: AEXQ_ATTN(8); break;
    default: return hipErrorInvalidValue;
  }
#undef AEXQ_ATTN
  return hipGetLastError();
}

}  // namespace aexq
