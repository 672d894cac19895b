// Instantiations of the tiled quantized GEMM (aexq_qgemm.hpp) and its table:
// Q8 with one scale per row and Q4 with one scale per multiple of 32 codes,
// fp16 or fp32 scales, single weights or SwiGLU pairs; 64-row activation
// tiles (Q4, Q8) and 128-row tiles (Q8; Q4 with split fp16 scales).
#include "aexq_qgemm.hpp"
#include "aexq_qgemm_dl.hpp"

namespace aexq {

#define QGEG(FMT, BM, PAIR, SF16, SPLIT, G16)                                 \
  QgemmEntry {                                                                \
    QgemmConfig{FMT, BM, PAIR, SF16, SPLIT, G16, false},                      \
        &qgemm_kernel<FMT, BM, PAIR, SF16, SPLIT, G16>                        \
  }
// LDS-direct forms: 128-row tiles two workgroups per CU, 64-row tiles three
#define QGDL(FMT, BM, PAIR, SF16, G)                                          \
  QgemmEntry {                                                                \
    QgemmConfig{FMT, BM, PAIR, SF16, FMT == kQ4, G == 16, true},              \
        &qgemm_dl_kernel<FMT, BM, PAIR, SF16, G, BM == 128 ? 2 : 3>           \
  }
#define QGDL_BM(BM)                                                            \
  QGDL(kQ8, BM, false, true, 0), QGDL(kQ8, BM, false, false, 0),              \
      QGDL(kQ8, BM, true, true, 0), QGDL(kQ8, BM, true, false, 0),            \
      QGDL(kQ4, BM, false, true, 32), QGDL(kQ4, BM, true, true, 32),          \
      QGDL(kQ4, BM, false, true, 16), QGDL(kQ4, BM, true, true, 16)
#define QGE(FMT, BM, PAIR, SF16, SPLIT) QGEG(FMT, BM, PAIR, SF16, SPLIT, false)

#define QG_BM(FMT, BM) \
  QGE(FMT, BM, false, true, false), QGE(FMT, BM, false, false, false), \
      QGE(FMT, BM, true, true, false), QGE(FMT, BM, true, false, false)

// Q4 with fp16 scales split into B (128-row tiles): single weights and pairs;
// Q4 with 16-code groups (64-row tiles)
static const QgemmEntry kTableG[] = {
    QG_BM(kQ4, 64), QG_BM(kQ8, 64), QG_BM(kQ8, 128), QGE(kQ4, 128, false, true, true),
    QGE(kQ4, 128, true, true, true), QGEG(kQ4, 64, false, true, false, true),
    QGEG(kQ4, 64, false, false, false, true), QGEG(kQ4, 64, true, true, false, true),
    QGEG(kQ4, 64, true, false, false, true), QGDL_BM(64), QGDL_BM(128)};

static constexpr int kCountG = (int)(sizeof(kTableG) / sizeof(kTableG[0]));

const QgemmEntry* qgemm_find(const QgemmConfig& c) {
  for (int i = 0; i < kCountG; ++i) {
    const QgemmConfig& q = kTableG[i].cfg;
    if (q.fmt == c.fmt && q.bm == c.bm && q.pair == c.pair && q.sf16 == c.sf16 &&
        q.split == c.split && q.g16 == c.g16 && q.direct == c.direct)
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
