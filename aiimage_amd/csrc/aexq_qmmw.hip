// Instantiations of the wide-step small-M MFMA kernel (aexq_qmmw.hpp) and its
// table: Q4 with one scale per 32 codes and Q8 with one scale per row, fp16
// or fp32 scales; MT 16-row activation tiles by NT 16-row weight blocks.
#include "aexq_qmmw.hpp"

namespace aexq {

#define QMMWG(FMT, MT, NT, PAIR, SF16, AM, RX, G16)                                           \
  QmmEntry {                                                                                  \
    QmmConfig{FMT, FMT == kQ8 ? kGRow : (G16 ? kG16 : kG32), MT, NT, PAIR, SF16, true, AM, RX}, \
        &qmmw_kernel<FMT, MT, NT, PAIR, SF16, AM, RX, G16>, kWaves * 16 * NT                  \
  }
#define QMMWX(FMT, MT, NT, PAIR, SF16, AM, RX) QMMWG(FMT, MT, NT, PAIR, SF16, AM, RX, false)
#define QMMWA(FMT, MT, NT, PAIR, SF16, AM) QMMWX(FMT, MT, NT, PAIR, SF16, AM, false)
#define QMMWE(FMT, MT, NT, PAIR, SF16) QMMWA(FMT, MT, NT, PAIR, SF16, false)
#define QMMWR(FMT, MT, NT, PAIR, SF16) QMMWX(FMT, MT, NT, PAIR, SF16, false, true)

// Blocks per wave: 4 at M <= 16, 2 at M <= 32, halved for SwiGLU pairs; Q8
// at M <= 16 half of that (its steps carry twice the code bytes, and the
// shorter tile measured faster there)
#define QMMW_Q4(SF16)                                                                         \
  QMMWE(kQ4, 1, 4, false, SF16), QMMWE(kQ4, 2, 2, false, SF16), QMMWE(kQ4, 1, 2, true, SF16), \
      QMMWE(kQ4, 2, 1, true, SF16)
#define QMMW_Q8(SF16)                                                                         \
  QMMWE(kQ8, 1, 2, false, SF16), QMMWE(kQ8, 2, 2, false, SF16), QMMWE(kQ8, 1, 1, true, SF16), \
      QMMWE(kQ8, 2, 1, true, SF16)

// RMSNorm-in inside the kernel, for launches with one item per workgroup
#define QMMW_R(FMT, SF16)                                                                     \
  QMMWR(FMT, 1, FMT == kQ8 ? 2 : 4, false, SF16), QMMWR(FMT, 2, 2, false, SF16),              \
      QMMWR(FMT, 1, FMT == kQ8 ? 1 : 2, true, SF16), QMMWR(FMT, 2, 1, true, SF16)

// Q4 with one scale per 16 codes (the reference's shipping Q4), plain and with
// RMSNorm-in inside the kernel
// (half the blocks per wave of group 32: a block carries twice the scales)
#define QMMW_G16(SF16, RX)                                                                    \
  QMMWG(kQ4, 1, 2, false, SF16, false, RX, true), QMMWG(kQ4, 2, 1, false, SF16, false, RX, true), \
      QMMWG(kQ4, 1, 1, true, SF16, false, RX, true), QMMWG(kQ4, 2, 1, true, SF16, false, RX, true)

// LM heads at M = 2..32 with the fused argmax partials (single weights)
#define QMMW_AM(FMT, SF16) QMMWA(FMT, 1, 1, false, SF16, true), QMMWA(FMT, 2, 1, false, SF16, true)

static const QmmEntry kTableW[] = {
    QMMW_Q4(true),       QMMW_Q4(false),       QMMW_Q8(true),       QMMW_Q8(false),
    QMMW_AM(kQ4, true),  QMMW_AM(kQ4, false),  QMMW_AM(kQ8, true),  QMMW_AM(kQ8, false),
    QMMW_R(kQ4, true),   QMMW_R(kQ4, false),   QMMW_R(kQ8, true),   QMMW_R(kQ8, false),
    QMMW_G16(true, false), QMMW_G16(false, false), QMMW_G16(true, true), QMMW_G16(false, true)};

static constexpr int kCountW = (int)(sizeof(kTableW) / sizeof(kTableW[0]));

const QmmEntry* qmmw_table(int* count) {
  *count = kCountW;
  return kTableW;
}

}  // namespace aexq
