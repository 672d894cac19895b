// Instantiations of the small-M MFMA kernel (aexq_qmm.hpp) and its table.
// MT 16-row activation tiles (M <= 16 MT, at most 32 rows per launch; the host
// walks larger M in 32-row blocks) by NT 16-row weight blocks per wave.
#include "aexq_qmm.hpp"

namespace aexq {

#define QMME(FMT, GM, MT, NT, PAIR, SF16)                                                        \
  QmmEntry {                                                                                    \
    QmmConfig{FMT, GM, MT, NT, PAIR, SF16, false, false},                                     \
        &qmm_kernel<FMT, GM, MT, NT, PAIR, SF16>,                                               \
        16 * NT                                                                                 \
  }

// single weights: 4 blocks at M <= 16, 2 at M <= 32; SwiGLU pairs stream two
// weights, so half as many blocks
#define QMM_SHAPES(FMT, GM, SF16)                                                               \
  QMME(FMT, GM, 1, 4, false, SF16), QMME(FMT, GM, 2, 2, false, SF16),                           \
      QMME(FMT, GM, 1, 2, true, SF16), QMME(FMT, GM, 2, 1, true, SF16)

static const QmmEntry kTable[] = {
    QMM_SHAPES(kQ8, kGRow, true), QMM_SHAPES(kQ8, kGRow, false),
    QMM_SHAPES(kQ4, kG32, true),  QMM_SHAPES(kQ4, kG32, false),
    QMM_SHAPES(kQ4, kG16, true),  QMM_SHAPES(kQ4, kG16, false),
};

static constexpr int kCount = (int)(sizeof(kTable) / sizeof(kTable[0]));

const QmmEntry* qmm_find(const QmmConfig& c) {
  int nw = 0;
  const QmmEntry* tw = qmmw_table(&nw);
  const QmmEntry* t = c.wide ? tw : kTable;
  const int n = c.wide ? nw : kCount;
  for (int i = 0; i < n; ++i) {
    const QmmConfig& q = t[i].cfg;
    if (q.fmt == c.fmt && q.gmode == c.gmode && q.mt == c.mt && q.nt == c.nt &&
        q.pair == c.pair && q.sf16 == c.sf16 && q.argmax == c.argmax && q.rmsx == c.rmsx)
      return &t[i];
  }
  return nullptr;
}

int qmm_blocks_per_cu(const QmmEntry* e) {
  static int cache[kCount], cache_w[64];
  int nw = 0;
  const QmmEntry* tw = qmmw_table(&nw);
  int* slot = nullptr;
  if (e >= kTable && e < kTable + kCount) slot = &cache[e - kTable];
  if (e >= tw && e < tw + nw && e - tw < 64) slot = &cache_w[e - tw];
  if (slot && *slot > 0) return *slot;
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, e->fn, kThreads, 0) != hipSuccess ||
      blocks <= 0)
    blocks = 1;
  if (slot) *slot = blocks;
  return blocks;
}

hipError_t qmm_launch(const QmmEntry* e, const QmvParams& p, int grid, hipStream_t stream) {
  if (!e) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(e->fn, dim3(grid), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace aexq
