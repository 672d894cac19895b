// Q8 instantiations of the streaming kernel (aexq_qmv.hpp) and their table.
// Shapes (LPR lanes per row, CPL chunks per lane, U rows per lane) cover
// K = 16..4096 in 16-byte (16-code) chunks; MMAX = 8 shapes keep the eight
// activation rows within the register budget.
#include "aexq_qmv.hpp"

namespace aexq {

#define Q8E(LPR, CPL, U, MMAX, PAIR, ARGMAX)                                                    \
  QmvEntry {                                                                                  \
    QmvConfig{kQ8, LPR, CPL, U, MMAX, PAIR, ARGMAX, kGRow},                                   \
        &qmv_kernel<kQ8, LPR, CPL, U, MMAX, PAIR, ARGMAX, kGRow>,                             \
        Qmv<kQ8, LPR, CPL, U, MMAX, PAIR, ARGMAX, kGRow>::RW                                  \
  }

#define Q8_M1(PAIR, ARGMAX)                                                                   \
  Q8E(16, 1, 4, 1, PAIR, ARGMAX), Q8E(16, 2, 2, 1, PAIR, ARGMAX),                             \
      Q8E(16, 4, 1, 1, PAIR, ARGMAX), Q8E(32, 1, 4, 1, PAIR, ARGMAX),                         \
      Q8E(32, 2, 2, 1, PAIR, ARGMAX), Q8E(32, 4, 1, 1, PAIR, ARGMAX),                         \
      Q8E(64, 1, 4, 1, PAIR, ARGMAX), Q8E(64, 2, 2, 1, PAIR, ARGMAX),                         \
      Q8E(64, 4, 1, 1, PAIR, ARGMAX)

// gate/up pairs stream two weights: half the rows per lane keeps the same
// bytes in flight in the same registers
#define Q8_M1_PAIR()                                                                          \
  Q8E(16, 1, 2, 1, true, false), Q8E(16, 2, 1, 1, true, false),                               \
      Q8E(16, 4, 1, 1, true, false), Q8E(32, 1, 2, 1, true, false),                           \
      Q8E(32, 2, 1, 1, true, false), Q8E(32, 4, 1, 1, true, false),                           \
      Q8E(64, 1, 2, 1, true, false), Q8E(64, 2, 1, 1, true, false),                           \
      Q8E(64, 4, 1, 1, true, false)

#define Q8_M8(PAIR, ARGMAX)                                                                   \
  Q8E(16, 1, 1, 8, PAIR, ARGMAX), Q8E(32, 1, 1, 8, PAIR, ARGMAX),                             \
      Q8E(64, 1, 1, 8, PAIR, ARGMAX), Q8E(64, 2, 1, 8, PAIR, ARGMAX)

static const QmvEntry kTable[] = {
    Q8_M1(false, false), Q8_M1_PAIR(), Q8_M1(false, true),
    Q8_M8(false, false), Q8_M8(true, false), Q8_M8(false, true),
};

const QmvEntry* qmv_table_q8(int* count) {
  *count = (int)(sizeof(kTable) / sizeof(kTable[0]));
  return kTable;
}

}  // namespace aexq
