// Instantiations of the tiled quantized GEMM and its table: the LDS-direct
// kernel (aexq_qgemm_dl.hpp) for Q8 with one scale per row and Q4 with one
// scale per 16 or 32 codes, the register-staged one (aexq_qgemm.hpp) for Q4
// with one scale per larger multiple of 32; fp16 or fp32 scales, single
// weights or SwiGLU pairs.
#include "aexq_qgemm.hpp"
#include "aexq_qgemm_dl.hpp"

namespace aexq {

// the register-staged kernel: Q4 with scale groups of 64 or more codes
#define QGE(PAIR, SF16)                                                              \
  QgemmEntry {                                                                       \
    QgemmConfig{kQ4, 64, PAIR, SF16, false, false, false}, &qgemm_kernel<PAIR, SF16> \
  }
// LDS-direct forms (aexq_qgemm_dl.hpp): Q8; Q4 in groups of 16 or 32, with
// fp16 dequantisation (FD) or exact per-group fp32 scaling; fp16 or fp32
// scales; 128-row tiles two workgroups per CU, 64-row tiles three
#define QGDL(FMT, BM, PAIR, SF16, G, FD)                                      \
  QgemmEntry {                                                                \
    QgemmConfig{FMT, BM, PAIR, SF16, G == 16, true, FD},                      \
        &qgemm_dl_kernel<FMT, BM, PAIR, SF16, G, FD, BM == 128 ? 2 : 3>       \
  }
#define QGDL_PS(FMT, BM, G, FD)                                                \
  QGDL(FMT, BM, false, true, G, FD), QGDL(FMT, BM, false, false, G, FD),      \
      QGDL(FMT, BM, true, true, G, FD), QGDL(FMT, BM, true, false, G, FD)
#define QGDL_BM(BM)                                                            \
  QGDL_PS(kQ8, BM, 0, false), QGDL_PS(kQ4, BM, 32, false), QGDL_PS(kQ4, BM, 16, false), \
      QGDL_PS(kQ4, BM, 32, true), QGDL_PS(kQ4, BM, 16, true)

// Q4 fp16 tiles at 64-row tiles with 128-wide K steps: two LDS stages (25-28
// KB each), three workgroups per CU where they fit
#define QGDL128(PAIR, SF16, G)                                                  \
  QgemmEntry {                                                                 \
    QgemmConfig{kQ4, 64, PAIR, SF16, G == 16, true, true, true},               \
        &qgemm_dl_kernel<kQ4, 64, PAIR, SF16, G, true, 3, 128, 2>              \
  }
#define QGDL128_G(G)                                                           \
  QGDL128(false, true, G), QGDL128(false, false, G), QGDL128(true, true, G),   \
      QGDL128(true, false, G)

static const QgemmEntry kTableG[] = {QGE(false, true), QGE(false, false), QGE(true, true),
                                     QGE(true, false), QGDL_BM(64), QGDL_BM(128),
                                     QGDL128_G(32), QGDL128_G(16)};

static constexpr int kCountG = (int)(sizeof(kTableG) / sizeof(kTableG[0]));

const QgemmEntry* qgemm_find(const QgemmConfig& c) {
  for (int i = 0; i < kCountG; ++i) {
    const QgemmConfig& q = kTableG[i].cfg;
    if (q.fmt == c.fmt && q.bm == c.bm && q.pair == c.pair && q.sf16 == c.sf16 &&
        q.g16 == c.g16 && q.direct == c.direct && q.fd == c.fd && q.k128 == c.k128)
      return &kTableG[i];
  }
  return nullptr;
}

int qgemm_rows_per_tile(bool pair) { return pair ? 64 : 128; }

int qgemm_blocks_per_cu(const QgemmEntry* e) {
  static int cache[kCountG] = {0};
  const int idx = (int)(e - kTableG);
  if (idx < 0 || idx >= kCountG) return 1;
  if (cache[idx] == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, e->fn, kThreads, 0) != hipSuccess || n < 1)
      n = 1;
    cache[idx] = n;
  }
  return cache[idx];
}

hipError_t qgemm_launch(const QgemmEntry* e, const QmvParams& p, hipStream_t stream) {
  if (!e) return hipErrorInvalidConfiguration;
  const int mtiles = (p.m + e->cfg.bm - 1) / e->cfg.bm;
  const long long groups = (p.total_tiles + 7) / 8;
  const long long grid = groups * 8 * mtiles * (p.sk_chunks > 1 ? p.sk_chunks : 1);
  if (grid <= 0 || grid > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(e->fn, dim3((unsigned)grid), dim3(kThreads), 0, stream, p, mtiles);
  return hipGetLastError();
}

}  // namespace aexq
