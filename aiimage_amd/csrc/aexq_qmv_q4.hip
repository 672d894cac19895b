// Q4 instantiations of the streaming kernel (aexq_qmv.hpp) and their table:
// scale groups of 16 codes (the reference's shipping Q4) and of multiples of 32
// codes (the benchmark's group 32, and one scale per row).  Shapes cover
// K = 32..8192 in 16-byte (32-code) chunks.
#include "aexq_qmv.hpp"

namespace aexq {

#define Q4E(LPR, CPL, U, MMAX, PAIR, GM)                                                        \
  QmvEntry {                                                                                  \
    QmvConfig{kQ4, LPR, CPL, U, MMAX, PAIR, false, GM},                                       \
        &qmv_kernel<kQ4, LPR, CPL, U, MMAX, PAIR, false, GM>,                                 \
        Qmv<kQ4, LPR, CPL, U, MMAX, PAIR, false, GM>::RW                                      \
  }

#define Q4_M1(PAIR, GM)                                                                       \
  Q4E(16, 1, 4, 1, PAIR, GM), Q4E(16, 2, 2, 1, PAIR, GM), Q4E(16, 4, 1, 1, PAIR, GM),         \
      Q4E(32, 1, 4, 1, PAIR, GM), Q4E(32, 2, 2, 1, PAIR, GM), Q4E(32, 4, 1, 1, PAIR, GM),     \
      Q4E(64, 1, 4, 1, PAIR, GM), Q4E(64, 2, 2, 1, PAIR, GM), Q4E(64, 4, 1, 1, PAIR, GM)

// gate/up pairs stream two weights: half the rows per lane keeps the same
// bytes in flight in the same registers
#define Q4_M1_PAIR(GM)                                                                        \
  Q4E(16, 1, 2, 1, true, GM), Q4E(16, 2, 1, 1, true, GM), Q4E(16, 4, 1, 1, true, GM),         \
      Q4E(32, 1, 2, 1, true, GM), Q4E(32, 2, 1, 1, true, GM), Q4E(32, 4, 1, 1, true, GM),     \
      Q4E(64, 1, 2, 1, true, GM), Q4E(64, 2, 1, 1, true, GM), Q4E(64, 4, 1, 1, true, GM)

#define Q4_M8(PAIR, GM)                                                                       \
  Q4E(16, 1, 1, 8, PAIR, GM), Q4E(32, 1, 1, 8, PAIR, GM), Q4E(64, 1, 1, 8, PAIR, GM)

static const QmvEntry kTable[] = {
    Q4_M1(false, kG32), Q4_M1_PAIR(kG32), Q4_M1(false, kG16), Q4_M1_PAIR(kG16),
    Q4_M8(false, kG32), Q4_M8(true, kG32), Q4_M8(false, kG16), Q4_M8(true, kG16),
};

const QmvEntry* qmv_table_q4(int* count) {
  *count = (int)(sizeof(kTable) / sizeof(kTable[0]));
  return kTable;
}

}  // namespace aexq
