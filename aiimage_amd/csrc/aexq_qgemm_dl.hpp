// Tiled quantized GEMM for M > 32 activation rows with LDS-direct loads
// (gfx950 `buffer_load_dwordx4 ... lds`): Y[M][N] = X[M][K] W[N][K]^T for Q8
// with one scale per row and Q4 with one scale (fp16 or fp32) per 16 or 32
// codes, K a multiple of 64.
//
// A workgroup owns one output tile: BM activation rows by 128 weight rows (a
// SwiGLU pair: 64 gate rows and the same 64 up rows), 256 threads.  Each
// 64-wide K step's activation tile, code tile and (Q4) scales travel from
// global memory straight into LDS: every 16-byte load instruction of a wave
// writes 1 KB of LDS, lane i at byte 16 i, so the lanes' global addresses are
// chosen to give the layout the MFMA fragment reads want, and no register
// holds a step in transit.  Three LDS stages rotate with one barrier per
// step, so a step's loads have two steps of MFMAs to land.
//
// Q8 permutes the K order inside a step: the MFMA's lane group g (l / 16)
// carries codes 16 g .. 16 g + 15 of the step, the first eight in the step's
// first MFMA K extent and the rest in the second, so a lane's codes for both
// extents are one 16-byte read, and the activation fragments are read in the
// same order (the products of K order, summed in another order in fp32).
// Q4 with fp16 weight tiles permutes the same way (a lane's two 8-code chunks
// are one 8-byte read, and both lie in one scale group of 32, or one of 16):
// read in K order (lane group g taking chunk 4 kk + g of extent kk) the
// activation fragments meet LDS bank conflicts (1.3 stall cycles per read on
// gfx950), in this order none.  Exact Q4 keeps K order inside each 32-code
// extent, so that an extent holds one scale group of 32 or two of 16.
//
// Codes become exact fp16 integers in registers.  Q8 accumulates the row in
// the MFMA and applies its row scale once at the end.  Q4 has two forms:
//  * fp16 dequantisation (FD, the default): each lane's codes share one scale
//    (lane group g holds codes 16 g .. 16 g + 15 of the step: scale group
//    g / 2 of 32, or g of 16), and the B fragment is formed as
//    fp16(q * s) by one packed fp16 multiply (one rounding; fp32 scales are
//    rounded to fp16 first), the weight tile dequantised to fp16 as the
//    benchmark's batched case specifies; the MFMA then accumulates the whole
//    row in fp32 with no per-group work, for groups of 16 as for 32.  The host
//    takes this form only for weights whose scales keep 8 |s| within the fp16
//    range.
//  * exact (AEXQ_EPI_EXACT_DEQUANT): each group's product is scaled in fp32
//    into the accumulator, so the dequantised weight is exactly
//    float(q) * scale: one MFMA per 32-code extent, or for groups of 16 two,
//    each with the other group's lanes' codes zeroed.  (Folding fp16 scales
//    into B as two exact fp16 parts measured slower: twice the MFMAs.)
//
// Activation rows are 128 bytes per step in LDS with their 16-byte chunks
// XOR-swizzled by the row (chunk c of row r at slot c ^ ((r & 7) ^ ((r >> 3) & 1))),
// so the 16 rows of a fragment read spread over every bank.  The code tile is
// stored per 16-row block in read order (Q8: [16-byte quarter][row]; Q4:
// [half][row]), so a fragment read is one contiguous run.
//
// Waves: 1 x 4, each every activation row of the tile by 32 weight rows, so
// a code fragment is expanded to fp16 once per workgroup (a 2 x 2 layout
// expands every B block in two waves: Q4 at M = 512 measured 7% slower).
// Inside a step the barrier sits between the two K halves: the first half's
// MFMAs cover the second half's fragment reads and the barrier wait, the
// second half's MFMAs cover the next step's first fragment reads.
//
// Workgroup b runs on XCD b % 8, which takes a contiguous range of tiles
// (gemm_block_tile): the BM-row tiles of one weight tile, and the weight
// tiles of one copy, share that XCD's L2.
//
// MFMA 16x16x32 f16 lane layout (lane l): A[l % 16][8 (l / 16) + j],
// B[8 (l / 16) + j][l % 16], D[4 (l / 16) + r][l % 16], j < 8, r < 4.
#pragma once

#include "aexq_qmm.hpp"

namespace aexq {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(1))) char gchar;  // global memory
typedef __attribute__((address_space(1))) f32x4 gf32x4;
typedef __attribute__((address_space(1))) u32x4 gu32x4;

// LDS byte address of a generic pointer into LDS (the low half of the
// generic address), wave-uniform.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}

// One LDS-direct load: lane i's BYTES (16 or 4) at byte voff of resource r go
// to LDS byte lds + BYTES * i; offsets past the resource's end write zeros.
// Written as assembly so that the compiler does not see LDS stores in flight:
// it would otherwise wait for every outstanding load before each LDS read.
// The kernel orders them itself -- s_waitcnt vmcnt for its own loads, then a
// barrier for the other waves' -- and the memory clobber keeps the compiler
// from moving LDS accesses across a load.
template <int BYTES>
__device__ __forceinline__ void dma(__amdgpu_buffer_rsrc_t r, uint32_t lds, int voff) {
  static_assert(BYTES == 16 || BYTES == 4, "dword or dwordx4");
  if constexpr (BYTES == 16)
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds), "v"(voff), "s"(r)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                 :
                 : "s"(lds), "v"(voff), "s"(r)
                 : "memory", "m0");
}

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | 0x70 | 0xF00 | ((N >> 4) << 14));
}
// s_waitcnt lgkmcnt(0).
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }
// Workgroup barrier without the fence __syncthreads() adds (whose vmcnt(0)
// would also wait for the LDS-direct loads of the steps ahead); the empty asm
// statements keep the compiler from moving LDS accesses across it.
__device__ __forceinline__ void bar() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// silu(g) = g / (1 + e^-g) with the division as a reciprocal (v_rcp_f32, 1 ulp)
// times g: the SwiGLU epilogue of a tile forms it for every output, and the
// IEEE division's expansion made up most of the epilogue's VALU work.
__device__ __forceinline__ float silu_rcp(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

// Eight offset-8 nibbles (n0 in bits 0-3) -> four fp16 pairs of the exact
// codes n - 8 in element order: pair j = (n_2j, n_2j+1).  Byte j goes to both
// halves (v_perm), the mask keeps n_2j low in half 0 and n_2j+1 at bits 4-7
// of half 1; with the exponent pattern 0x6400 the halves are 1024 + n_2j and
// 1024 + 16 n_2j+1, and one fma with (1, 1/16), (-1032, -72) gives both codes.
__device__ __forceinline__ void q4_pairs_seq(uint32_t w, uint32_t q[4]) {
  uint32_t E = 0x64006400u, m = 0x00F0000Fu;
  __asm__("" : "+v"(E));
  __asm__("" : "+s"(m));
  const f16x2 mul = {(f16)1.0f, (f16)0.0625f};
  const f16x2 add = {(f16)-1032.0f, (f16)-72.0f};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t t = __builtin_amdgcn_perm(w, w, 0x0C000C00u | (j << 16) | j);
    q[j] = as_u(__builtin_elementwise_fma(as_h2((t & m) | E), mul, add));
  }
}

template <int FMT, int BM, bool PAIR, bool SF16, int G, bool FD, int KS = 64>
struct QGemmDL {
  static_assert(FMT == kQ8 ? G == 0 : (G == 16 || G == 32),
                "Q8 (row scales) or Q4 in groups of 16 or 32");
  static_assert(!FD || FMT == kQ4, "fp16 dequantisation is a Q4 form");
  static_assert(BM == 64 || BM == 128, "64- or 128-row activation tiles");
  static_assert(KS == 64 || (KS == 128 && FD), "128-wide K steps are a form of Q4 fp16 tiles");
  static constexpr int BN = 128;                  // weight rows of a tile
  static constexpr int BK = KS;                   // K per step
  static constexpr int NE = BK / 32;              // MFMA K extents per step
  static constexpr int RA = 2 * BK;               // activation bytes per row and step
  static constexpr int NOUT = PAIR ? BN / 2 : BN;  // output columns of a tile
  static constexpr int WR = BN / 4;               // weight rows per wave (32)
  static constexpr int TN = WR / 16;              // 16-row B blocks per wave (2)
  static constexpr int TM = BM / 16;              // 16-row A blocks per wave (every row)
  static constexpr int CP = FMT == kQ8 ? 64 : BK / 2;  // code bytes per row and step
  // codes read as Q8's: a lane's 16 bytes of a 64-byte row step (Q8, Q4 at KS 128)
  static constexpr bool C16 = CP == 64;
  static constexpr int A_BYTES = BM * RA;
  static constexpr int B_BYTES = BN * CP;
  static constexpr int SPR = FMT == kQ8 ? 0 : BK / G;    // Q4 scales per row and step
  static constexpr int SB = SF16 ? 2 : 4;                // bytes per scale
  static constexpr int S_BYTES = FMT == kQ8 ? 0 : BN * SPR * SB;
  static constexpr int S_AREA = FMT == kQ8 ? 0 : (S_BYTES < 1024 ? 1024 : S_BYTES);
  static constexpr int STAGE = A_BYTES + B_BYTES + S_AREA;
  static constexpr int A_INST = A_BYTES / 1024 / 4;  // direct loads per wave and step
  static constexpr int B_INST = B_BYTES / 1024 / 4;
  // dword loads of the step's scales per wave (256 bytes each; with 512
  // bytes of scales waves 2 and 3 load past the resource into spare LDS)
  static constexpr int S_INST = FMT == kQ8 ? 0 : (S_BYTES <= 1024 ? 1 : S_BYTES / 1024);
  static constexpr int S_RPI = FMT == kQ8 ? 1 : 256 / (SPR * SB);  // rows per scale load
  static constexpr int NL = A_INST + B_INST + S_INST;

  // Tile row (0..127 of the code tile) of B block tn of wave column wn.
  static __device__ __forceinline__ int brow(int wn, int tn) {
    if constexpr (PAIR)
      return (tn >= TN / 2 ? 64 : 0) + wn * (WR / 2) + 16 * (tn % (TN / 2));
    return wn * WR + 16 * tn;
  }

  // Chunk swizzle of activation row r (16-byte chunk c of the row at slot
  // c ^ aswz(r)): the fragment reads of 16 rows by four lane quarters then
  // fall on distinct 16-byte slots of each 512-byte bank line (gfx950 serves
  // 32 lanes' 16-byte LDS reads per pass).  8 chunks a row (64-wide steps):
  // (r & 7) ^ ((r >> 3) & 1); 16 chunks (128-wide): ((r >> 1) & 3) + 8 ((r >> 3) & 1).
  static __device__ __forceinline__ int aswz(int r) {
    if constexpr (RA == 128)
      return (r & 7) ^ ((r >> 3) & 1);
    else
      return ((r >> 1) & 3) + 8 * ((r >> 3) & 1);
  }

  struct Src {
    __amdgpu_buffer_rsrc_t xr, wr, sr;
    int oa[A_INST];  // per-lane byte offsets of step 0
    int ob[B_INST];
    int os[S_INST > 0 ? S_INST : 1];
  };

  static __device__ __forceinline__ Src source(const QmvParams& p, const QmvMat& mt, int b,
                                               int n0, int m0, int lane, int wave) {
    Src s;
    const int rb = FMT == kQ8 ? p.k : p.k / 2;  // code bytes per weight row
    const int rows = mt.n > n0 ? min(mt.n - n0, NOUT) : 0;
    // B rows of this wave's code loads: Q8 blocks 2w, 2w + 1 (rows 32 w ..), Q4
    // rows 32 w ..: the up weight for w >= 2 of a pair
    const bool up = PAIR && wave >= 2;
    const char* wb = (const char*)(up ? mt.w2 : mt.w) + (long long)b * mt.w_bstride * 4 +
                     (long long)n0 * rb;
    s.wr = __builtin_amdgcn_make_buffer_rsrc((void*)wb, (short)0, rows * rb, kBufferRsrcWord3);
    const int rs2 = (int)(p.x_rstride * 2);
    const char* xb = (const char*)mt.x + (long long)b * mt.x_bstride * 2 + (long long)m0 * rs2;
    const int mrows = p.m - m0 < BM ? p.m - m0 : BM;
    s.xr = __builtin_amdgcn_make_buffer_rsrc((void*)xb, (short)0, mrows * rs2, kBufferRsrcWord3);
#pragma unroll
    for (int t = 0; t < A_INST; ++t) {
      // an instruction covers 1024 / RA rows; chunk slot (lane % CH) of a row
      // holds chunk slot ^ aswz(row)
      constexpr int CH = RA / 16;  // 16-byte chunks per activation row and step
      const int row = (1024 / RA) * (wave * A_INST + t) + lane / CH;
      const int c = (lane % CH) ^ aswz(row);
      s.oa[t] = row * rs2 + c * 16;
    }
    if constexpr (C16) {
#pragma unroll
      for (int t = 0; t < B_INST; ++t) {
        const int r = 16 * (wave * B_INST + t) + (lane & 15);
        s.ob[t] = (PAIR ? (r & 63) : r) * rb + 16 * (lane >> 4);
      }
    } else {
      const int r = 32 * wave + 16 * (lane >> 5) + (lane & 15);
      s.ob[0] = (PAIR ? (r & 63) : r) * rb + 16 * ((lane >> 4) & 1);
    }
    if constexpr (FMT == kQ8) {
      // row scales: wave 0 rows 0-63 (the gate rows of a pair), wave 1 rows
      // 64-127 (the up rows); fp16: lane i fetches rows 2i, 2i + 1 (lanes 32..
      // fall past the rows), fp32: row i
      constexpr int sb = SF16 ? 2 : 4;
      const bool sup = PAIR && wave == 1;
      const int base_row = PAIR ? 0 : 64 * (wave & 1);
      const char* sp = (const char*)(sup ? mt.s2 : mt.s) + (long long)b * mt.s_bstride * sb +
                       (long long)(n0 + base_row) * sb;
      const int srows = __builtin_amdgcn_readfirstlane(min(max(rows - base_row, 0), 64));
      // (the range in whole dwords: a dword only partly inside reads zero, which
      // at an odd row count with fp16 scales would zero the last row's scale;
      // a weight's scale storage runs at least 16 bytes past its last scale)
      s.sr = __builtin_amdgcn_make_buffer_rsrc((void*)sreg(sp), (short)0, (srows * sb + 3) & ~3,
                                               kBufferRsrcWord3);
      s.os[0] = 4 * lane;
    } else {
      // scales: load i of wave w covers rows S_RPI (w S_INST + i) .. (every
      // row's SPR scales of the step); one weight per wave (the up weight of
      // a pair from row 64)
      const int row0 = S_RPI * wave * S_INST;
      const bool sup = PAIR && row0 >= 64;
      const char* sp = (const char*)(sup ? mt.s2 : mt.s) +
                       ((long long)b * mt.s_bstride + (long long)n0 * p.groups_per_row) * SB;
      s.sr = __builtin_amdgcn_make_buffer_rsrc((void*)sp, (short)0,
                                               rows * p.groups_per_row * SB, kBufferRsrcWord3);
#pragma unroll
      for (int i = 0; i < S_INST; ++i) {
        const int j = wave * S_INST + i;  // load index over the workgroup
        const int byte = 256 * j + 4 * lane;  // in the step's scale block [row][SPR]
        const int srow = byte / (SPR * SB), sin = byte % (SPR * SB);
        const int wrow = PAIR ? (srow & 63) : srow;
        s.os[i] = 256 * j >= S_BYTES ? (1 << 30) : wrow * p.groups_per_row * SB + sin;
      }
    }
    return s;
  }

  // The direct loads of step st into the LDS stage at byte `base`.
  static __device__ __forceinline__ void issue(const Src& s, uint32_t base, int wave, int st) {
#pragma unroll
    for (int t = 0; t < A_INST; ++t)
      dma<16>(s.xr, base + (wave * A_INST + t) * 1024, s.oa[t] + st * RA);
#pragma unroll
    for (int t = 0; t < B_INST; ++t)
      dma<16>(s.wr, base + A_BYTES + (wave * B_INST + t) * 1024, s.ob[t] + st * CP);
    if constexpr (FMT == kQ4) {
#pragma unroll
      for (int i = 0; i < S_INST; ++i)
        dma<4>(s.sr, base + A_BYTES + B_BYTES + (wave * S_INST + i) * 256,
               s.os[i] + st * SPR * SB);
    }
  }

  // Fragments of one step a wave reads from LDS: the activation blocks of one
  // K half and the raw codes (and Q4 scales) of both halves.
  // (Q4: the lane's 8 codes of each MFMA extent and the row's scales of the
  // step, one per extent or two for groups of 16; FD: the lane's own scale)
  // (FD: the scale groups of a lane's chunks of a step: one, or two for groups
  // of 16 at 128-wide steps)
  static constexpr int NS = FMT == kQ8 ? 1 : (FD ? (NE * 8 / G > 1 ? NE * 8 / G : 1) : SPR);
  // K order permuted as Q8's (lane group g: chunks NE g .. NE g + NE - 1 of the
  // step, one per MFMA extent)
  static constexpr bool PERM = FMT == kQ8 || FD;
  struct Frag {
    f16x8 a[TM];
    typename std::conditional<C16, u32x4, u32x2>::type c[TN];
    uint32_t s[TN][NS];
  };

  struct Lane {
    int a_off[NE];  // activation fragment offset of extent 0 .. NE - 1 (row l16 of block 0)
    int b_off;     // code fragment offset inside a 16-row block
    int s_off;     // scale offset (row l16, the lane group's scale group) inside block row 0
  };

  static __device__ __forceinline__ Lane lane_offsets(int lane) {
    Lane L;
    const int l16 = lane & 15, lk = lane >> 4;
    const int f = aswz(l16);
#pragma unroll
    for (int kk = 0; kk < NE; ++kk)
      L.a_off[kk] = l16 * RA + (((PERM ? NE * lk + kk : 4 * kk + lk) ^ f) << 4);
    // 16-byte code reads (C16): [quarter][row] per 16-row block, lane l at 16 l.
    // Q4 codes [half][row] per 16-row block: FD chunks 2 lk, 2 lk + 1 (half
    // lk / 2, bytes 8 (lk % 2) ..); exact: dword lk of each half (+ 256 kk)
    L.b_off = C16 ? 16 * lane
                  : (FD ? (lk >> 1) * 256 + l16 * 16 + (lk & 1) * 8 : l16 * 16 + 4 * lk);
    // FD: the scale group of chunk NE lk (lk / 2 for groups of 32 at 64-wide
    // steps, lk for 16 or for 32 at 128-wide, 2 lk for 16 at 128-wide)
    L.s_off = FMT == kQ8 ? 0 : l16 * (SPR * SB) + (FD ? (NE * lk * 8 / G) * SB : 0);
    return L;
  }

  static __device__ __forceinline__ void read_a(const char* base, const Lane& L, int kk,
                                                f16x8 (&a)[TM]) {
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
      a[tm] = *(const f16x8*)(base + 16 * tm * RA + L.a_off[kk]);
  }

  static __device__ __forceinline__ void read_b(const char* base, const Lane& L, int wn, Frag& f) {
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int blk = brow(wn, tn) >> 4;
      if constexpr (C16) {
        f.c[tn] = *(const u32x4*)(base + A_BYTES + blk * 1024 + L.b_off);
      } else {
        const char* bb = base + A_BYTES + blk * 512 + L.b_off;
        if constexpr (FD)
          f.c[tn] = *(const u32x2*)bb;  // chunk 2 lk, then 2 lk + 1
        else
          f.c[tn] = u32x2{*(const uint32_t*)bb, *(const uint32_t*)(bb + 256)};
      }
      if constexpr (FMT == kQ4) {
        const char* sb = base + A_BYTES + B_BYTES + blk * 16 * (SPR * SB) + L.s_off;
#pragma unroll
        for (int i = 0; i < NS; ++i)
          f.s[tn][i] = SF16 ? (uint32_t) * (const uint16_t*)(sb + SB * i)
                            : *(const uint32_t*)(sb + 4 * i);
      }
    }
  }

  // The MFMAs of K extent kk from the activation blocks a and the step's codes.
  static __device__ __forceinline__ void mfma_half(int kk, const f16x8 (&a)[TM], const Frag& f,
                                                   f32x4 (&acc)[TM][TN]) {
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      if constexpr (FMT == kQ8) {
        uint32_t e0, e1, e2, e3;
        q8_pairs(f.c[tn][2 * kk], e0, e1);
        q8_pairs(f.c[tn][2 * kk + 1], e2, e3);
        const f16x8 bq = pack8(e0, e1, e2, e3);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
          acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[tm], bq, acc[tm][tn], 0, 0, 0);
      } else if constexpr (FD) {
        // fp16(q * s): the exact codes times the lane's scale, one rounding;
        // the MFMA accumulates the row
        uint32_t e[4];
        q4_pairs_seq(f.c[tn][kk], e);
        const f16 s16 = (f16)scale_of(f.s[tn][kk * NS / NE], SF16);
        const f16x2 s2 = {s16, s16};
#pragma unroll
        for (int j = 0; j < 4; ++j) e[j] = as_u(as_h2(e[j]) * s2);
        const f16x8 bw = pack8(e[0], e[1], e[2], e[3]);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
          acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[tm], bw, acc[tm][tn], 0, 0, 0);
      } else {
        // one group per extent (32) or two (16: lane groups 0-1 and 2-3, each
        // MFMA with the other group's codes zeroed); each group's product is
        // scaled in fp32 into the accumulator: exactly float(q) * scale
        uint32_t e[4];
        q4_pairs_seq(f.c[tn][kk], e);
        const f16x8 bq = pack8(e[0], e[1], e[2], e[3]);
        const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (G == 32) {
          const float sc = scale_of(f.s[tn][kk], SF16);
#pragma unroll
          for (int tm = 0; tm < TM; ++tm) {
            const f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[tm], bq, z, 0, 0, 0);
            acc[tm][tn] = __builtin_elementwise_fma(f32x4{sc, sc, sc, sc}, t, acc[tm][tn]);
          }
        } else {
          const float s0 = scale_of(f.s[tn][2 * kk], SF16);
          const float s1 = scale_of(f.s[tn][2 * kk + 1], SF16);
          const bool first = (__lane_id() >> 4) < 2;
          const f16x8 zero = {};
          const f16x8 b0 = first ? bq : zero, b1 = first ? zero : bq;
#pragma unroll
          for (int tm = 0; tm < TM; ++tm) {
            const f32x4 t0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[tm], b0, z, 0, 0, 0);
            const f32x4 t1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[tm], b1, z, 0, 0, 0);
            const f32x4 a0 = __builtin_elementwise_fma(f32x4{s0, s0, s0, s0}, t0, acc[tm][tn]);
            acc[tm][tn] = __builtin_elementwise_fma(f32x4{s1, s1, s1, s1}, t1, a0);
          }
        }
        // the scaled sums are formed here, not deferred by the compiler (which
        // would keep every MFMA result of the step alive: spills)
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) asm volatile("" : "+v"(acc[tm][tn]));
      }
    }
  }

  // Output column (tile-relative) of output block `to` of wave column wn.
  static __device__ __forceinline__ int ocol(int wn, int to) {
    return PAIR ? wn * (WR / 2) + 16 * to : wn * WR + 16 * to;
  }

  // The finished tile, through LDS.  The waves of activation rows 64 h ..
  // 64 h + 63 write their raw accumulators into an fp32 tile C[64][CW] (the
  // pipeline's stages are free by then); then each thread finishes 8
  // consecutive outputs of a row per pass -- row scale (Q8), bias, alpha/beta,
  // SwiGLU, residual -- and stores them with one 16-byte (fp16) or two
  // (fp32) stores where the layout allows, element by element otherwise.
  // One short loop for every output keeps the code (and the instruction
  // cache) small, and the stores cover whole rows of the tile.
  static constexpr int CW = BN + 4;            // floats per LDS row of C
  static constexpr int TPR = NOUT / 8;         // threads per output row
  static constexpr int RPP = kThreads / TPR;   // rows per pass
  static constexpr int C_BYTES = 64 * CW * 4;

  // Rows 64 h .. 64 h + 63 of the tile's raw accumulators into C, then a
  // barrier (a barrier first for h > 0: every thread has read the last half).
  static __device__ __forceinline__ void stage_c(int h, int lane, int wn,
                                                 const f32x4 (&acc)[TM][TN], float* C) {
    const int l16 = lane & 15, lk = lane >> 4;
    if (h > 0) bar();
#pragma unroll
    for (int tq = 0; tq < 4; ++tq)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          C[(16 * tq + 4 * lk + r) * CW + brow(wn, tn) + l16] = acc[4 * h + tq][tn][r];
    wait_lgkm0();
    bar();
  }

  static __device__ __forceinline__ void finish(const QmvParams& p, const QmvMat& mt, int b,
                                                int n0, int m0, int tid, int lane, int wn, const f32x4 (&acc)[TM][TN], float* C,
                                                const char* qs) {
    const int l16 = lane & 15, lk = lane >> 4;
    // everything the loops below use, in registers (see sreg)
    const EpiArgs E = epi_args(p);
    const bool yf32 = (E.flags & kFlagYf32) != 0;
    const bool resid = mt.res && (E.flags & kFlagResidual);
    const int esz = yf32 ? 4 : 2;
    // (global pointers: the stores and residual loads are global, not flat)
    gchar* const yb = (gchar*)sreg((char*)mt.y + (long long)b * mt.y_bstride * esz);
    const gchar* const rb =
        resid ? (const gchar*)sreg((const char*)mt.res + (long long)b * mt.r_bstride * esz)
              : nullptr;
    const int mn = sreg(mt.n), nst = sreg(mt.n_store), pm = sreg(p.m), mbase = sreg(p.m_base);
    const long long yrs = ((long long)sreg((int)(mt.y_rstride >> 32)) << 32) |
                          (uint32_t)sreg((int)mt.y_rstride);
    const long long rrs = ((long long)sreg((int)(p.r_rstride >> 32)) << 32) |
                          (uint32_t)sreg((int)p.r_rstride);
    const int cg = tid % TPR, r0 = tid / TPR;
    const int nb = n0 + 8 * cg;  // first of the thread's 8 output columns
    // 8-wide rows: row-major output, every column stored, aligned rows
    const bool vec = mt.y_hd == 0 && nb + 8 <= nst && (yrs & 7) == 0 &&
                     ((uintptr_t)yb & 15) == 0 &&
                     (!resid || ((rrs & 7) == 0 && ((uintptr_t)rb & 15) == 0));
    // every column stored and real, no bias: the branch-free form below
    const bool fast = vec && nb + 8 <= mn && !E.c;
    const bool alpha_in = (E.flags & kFlagAlphaIn) != 0;
    const float a_in = alpha_in ? E.alpha : 1.0f, a_out = alpha_in ? 1.0f : E.alpha;
    float rs0[8], rs1[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      rs0[j] = 1.0f;
      rs1[j] = 1.0f;
      if constexpr (FMT == kQ8) {
        // row scales as the prologue placed them: tile row r at (r / 64) * 512
        // + (r % 64) * (2 or 4) bytes; the up half of a pair from row 64
        const int r = 8 * cg + j;
        rs0[j] = scale_of(SF16 ? *(const uint16_t*)(qs + (r >> 6) * 512 + (r & 63) * 2)
                               : *(const uint32_t*)(qs + (r >> 6) * 512 + (r & 63) * 4),
                          SF16);
        if constexpr (PAIR)
          rs1[j] = scale_of(SF16 ? *(const uint16_t*)(qs + 512 + r * 2)
                                 : *(const uint32_t*)(qs + 512 + r * 4),
                            SF16);
      }
    }
#pragma unroll
    for (int h = 0; h < BM / 64; ++h) {
      stage_c(h, lane, wn, acc, C);
#pragma unroll 1
      for (int row = r0; row < 64; row += RPP) {
        const int m = m0 + 64 * h + row;
        if (m >= pm || !yb) continue;
        float g[8], u[8];
        *(f32x4*)&g[0] = *(const f32x4*)&C[row * CW + 8 * cg];
        *(f32x4*)&g[4] = *(const f32x4*)&C[row * CW + 8 * cg + 4];
        if constexpr (PAIR) {
          *(f32x4*)&u[0] = *(const f32x4*)&C[row * CW + 64 + 8 * cg];
          *(f32x4*)&u[4] = *(const f32x4*)&C[row * CW + 64 + 8 * cg + 4];
        }
        float res[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) res[j] = 0.0f;
        if (resid) {
          const long long ri = (long long)m * rrs + nb;
          if (vec) {
            if (yf32) {
              *(f32x4*)&res[0] = *(const gf32x4*)(rb + ri * 4);
              *(f32x4*)&res[4] = *(const gf32x4*)(rb + ri * 4 + 16);
            } else {
              const u32x4 h8 = *(const gu32x4*)(rb + ri * 2);
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const f16x2 hv = as_h2(h8[q]);
                res[2 * q] = (float)hv[0];
                res[2 * q + 1] = (float)hv[1];
              }
            }
          } else {
#pragma unroll
            for (int j = 0; j < 8; ++j)
              if (nb + j < mn)
                res[j] = yf32 ? ((const __attribute__((address_space(1))) float*)rb)[ri + j]
                              : (float)((const __attribute__((address_space(1))) f16*)rb)[ri + j];
          }
        }
        float v[8];
        if (fast) {
          // no bias: alpha * (0 + x) or 0 + alpha * x as a_in * (0 + a_out * x),
          // the same roundings with no branch per output
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            v[j] = a_in * (0.0f + a_out * (g[j] * rs0[j]));
            if constexpr (PAIR) v[j] = silu_rcp(v[j]) * (a_in * (0.0f + a_out * (u[j] * rs1[j])));
            v[j] += res[j];
          }
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int n = nb + j;
            v[j] = 0.0f;
            if (n < mn) {
              v[j] = gemm_epilogue(E, mbase + m, n, g[j] * rs0[j]);
              if constexpr (PAIR)
                v[j] = silu_rcp(v[j]) * gemm_epilogue(E, mbase + m, n, u[j] * rs1[j]);
              v[j] += res[j];
            }
          }
        }
        if (vec) {
          const long long yi = (long long)m * yrs + nb;
          if (yf32) {
            *(gf32x4*)(yb + yi * 4) = f32x4{v[0], v[1], v[2], v[3]};
            *(gf32x4*)(yb + yi * 4 + 16) = f32x4{v[4], v[5], v[6], v[7]};
          } else {
            u32x4 o;
#pragma unroll
            for (int q = 0; q < 4; ++q) o[q] = as_u(f16x2{(f16)v[2 * q], (f16)v[2 * q + 1]});
            *(gu32x4*)(yb + yi * 2) = o;
          }
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int n = nb + j;
            if (n < nst) {
              const long long yi = out_index(p, mt, m, n);
              if (yf32)
                ((__attribute__((address_space(1))) float*)yb)[yi] = v[j];
              else
                ((__attribute__((address_space(1))) f16*)yb)[yi] = (f16)v[j];
            }
          }
        }
      }
    }
  }

  // Split K: the raw accumulators of K chunk c (no row scale, no epilogue)
  // into partial plane c, through C as in finish: 8 consecutive partials of
  // a row per thread, two 16-byte stores where the plane is aligned.
  static __device__ __forceinline__ void spill(const QmvParams& p, const QmvMat& mt, int b,
                                               int n0, int m0, int tid, int lane, int wn, int c,
                                               const f32x4 (&acc)[TM][TN], float* C) {
    constexpr int NW = PAIR ? 2 : 1;
    const int nst = sreg(mt.n_store), mn = sreg(mt.n), pm = sreg(p.m);
    float* const base = sreg(p.sk_part + (long long)c * p.sk_plane + mt.sk_off +
                             (long long)b * p.m * NW * mt.n_store);
    gchar* const gb = (gchar*)base;
    const int cg = tid % TPR, r0 = tid / TPR;
    const int nb = n0 + 8 * cg;
    const bool vec = nb + 8 <= mn && (nst & 3) == 0 && ((uintptr_t)base & 15) == 0;
#pragma unroll
    for (int h = 0; h < BM / 64; ++h) {
      stage_c(h, lane, wn, acc, C);
#pragma unroll 1
      for (int row = r0; row < 64; row += RPP) {
        const int m = m0 + 64 * h + row;
        if (m >= pm) continue;
#pragma unroll
        for (int hh = 0; hh < NW; ++hh) {
          const f32x4 v0 = *(const f32x4*)&C[row * CW + 64 * hh + 8 * cg];
          const f32x4 v1 = *(const f32x4*)&C[row * CW + 64 * hh + 8 * cg + 4];
          const long long o = ((long long)m * NW + hh) * nst + nb;
          if (vec) {
            *(gf32x4*)(gb + o * 4) = v0;
            *(gf32x4*)(gb + o * 4 + 16) = v1;
          } else {
#pragma unroll
            for (int j = 0; j < 8; ++j)
              if (nb + j < mn)
                ((__attribute__((address_space(1))) float*)gb)[o + j] = j < 4 ? v0[j] : v1[j - 4];
          }
        }
      }
    }
  }
};

// Waits until the loads of at most min(KMAX, ahead) steps (NL instructions
// each) are outstanding, the older ones landed; `ahead` is wave-uniform.
template <int NL, int KMAX>
__device__ __forceinline__ void wait_steps(int ahead) {
  if constexpr (KMAX > 0) {
    if (ahead >= KMAX)
      wait_vm<KMAX * NL>();
    else
      wait_steps<NL, KMAX - 1>(ahead);
  } else {
    wait_vm<0>();
  }
}

// One step of the pipeline on LDS stage `cur` of an NST-stage ring (the next
// step's stage `nxt`; the stage refilled with step st + NST is `cur` itself):
// on entry f holds the step's codes and first-extent activation blocks; on
// return, the next step's.  The barrier sits before the last extent's MFMAs,
// which cover the next step's first fragment reads; the MFMAs before it
// cover the reads of the extents after them and the barrier wait.
template <typename G, int NST>
__device__ __forceinline__ void qgemm_dl_step(const typename G::Src& src, const typename G::Lane& L,
                                              char* cur, char* nxt, int wave, int wn,
                                              int st, int s1, typename G::Frag& f,
                                              f32x4 (&acc)[G::TM][G::TN]) {
  f16x8 a1[G::TM];
  G::read_a(cur, L, 1, a1);
  __builtin_amdgcn_sched_barrier(0);  // the reads go out ahead of the MFMAs
  G::mfma_half(0, f.a, f, acc);
  if constexpr (G::NE == 4) {
    f16x8 a2[G::TM];
    G::read_a(cur, L, 2, a2);
    __builtin_amdgcn_sched_barrier(0);
    G::mfma_half(1, a1, f, acc);
    G::read_a(cur, L, 3, a1);
    __builtin_amdgcn_sched_barrier(0);
    G::mfma_half(2, a2, f, acc);
  }
  // this step's fragments are in registers before any wave refills `cur`;
  // step st + 1's loads (the oldest in flight) have landed
  wait_lgkm0();
  wait_steps<G::NL, NST - 2>(s1 - st - 2);
  bar();
  if (st + NST < s1) G::issue(src, lds_addr(cur), wave, st + NST);
  typename G::Frag g;
  if (st + 1 < s1) {
    G::read_a(nxt, L, 0, g.a);
    G::read_b(nxt, L, wn, g);
  }
  __builtin_amdgcn_sched_barrier(0);
  G::mfma_half(G::NE - 1, a1, f, acc);
  f = g;
}

template <int FMT, int BM, bool PAIR, bool SF16, int G, bool FD, int WPE, int KS = 64, int NST = 3>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(WPE)))
void qgemm_dl_kernel(const QmvParams p, int mtiles) {
  using Q = QGemmDL<FMT, BM, PAIR, SF16, G, FD, KS>;
  static_assert(NST == 2 || NST == 3, "a ring of two or three LDS stages");
  static_assert(Q::C_BYTES <= NST * Q::STAGE, "the accumulator tile reuses the stages");
  __shared__ __align__(1024) char lds[NST * Q::STAGE];
  __shared__ __align__(16) char qs[FMT == kQ8 ? 1024 : 16];  // Q8 row scales of the tile
  char* const sg[3] = {lds, lds + Q::STAGE, lds + (NST - 1) * Q::STAGE};
  // weight tile tn, row tile tm and K chunk kc of this workgroup (the chunks
  // of a split K sit next to each other on one XCD); readfirstlane keeps the
  // workgroup-uniform coordinates in scalar registers
  const int S = p.sk_chunks > 1 ? p.sk_chunks : 1;
  const int per = mtiles * S;
  int tile, rem;
  gemm_block_tile(blockIdx.x, p.total_tiles, per, tile, rem);
  const int tn = __builtin_amdgcn_readfirstlane(tile);
  const int tm = __builtin_amdgcn_readfirstlane(rem / S);
  const int kc = __builtin_amdgcn_readfirstlane(rem - (rem / S) * S);
  if (tn < 0) return;
  int j = 0;
  for (int q = 1; q < p.nmat; ++q)
    if (tn >= p.mat[q].tile_base) j = q;
  j = __builtin_amdgcn_readfirstlane(j);
  const QmvMat& mt = p.mat[j];
  const int local = tn - mt.tile_base;
  const int b = __builtin_amdgcn_readfirstlane(local / mt.tiles);
  const int n0 = __builtin_amdgcn_readfirstlane((local - b * mt.tiles) * Q::NOUT);
  const int m0 = tm * BM;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wn = wave;  // the wave's 32 weight rows
  const int steps = p.k / Q::BK;
  const int cs = S > 1 ? p.sk_cs : steps;
  const int s0 = kc * cs, s1 = min(s0 + cs, steps);  // this workgroup's K steps
  if (s0 >= s1) return;
  const typename Q::Src src = Q::source(p, mt, b, n0, m0, lane, wave);
  const typename Q::Lane L = Q::lane_offsets(lane);

  f32x4 acc[Q::TM][Q::TN];
#pragma unroll
  for (int a = 0; a < Q::TM; ++a)
#pragma unroll
    for (int c = 0; c < Q::TN; ++c) acc[a][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // prologue: steps s0 .. s0 + NST - 1 in flight, step s0 landed and its
  // first fragments read
  // Q8: the tile's row scales go to LDS with the first step (waves 0 and 1:
  // rows 0-63 and 64-127, or the gate and up rows of a pair)
  if constexpr (FMT == kQ8)
    if (S == 1 && wave < 2) dma<4>(src.sr, lds_addr(qs) + wave * 512, src.os[0]);
#pragma unroll
  for (int i = 0; i < NST; ++i)
    if (s0 + i < s1) Q::issue(src, lds_addr(sg[i]), wave, s0 + i);
  // (the row scales, issued first, have landed with step s0)
  wait_steps<Q::NL, NST - 1>(s1 - s0 - 1);
  bar();
  typename Q::Frag f;
  Q::read_a(sg[0], L, 0, f.a);
  Q::read_b(sg[0], L, wn, f);
  // NST steps per iteration: the stages rotate with compile-time names
  int st = s0;
  for (int it = (s1 - s0) / NST; it > 0; --it) {
#pragma unroll
    for (int i = 0; i < NST; ++i)
      qgemm_dl_step<Q, NST>(src, L, sg[i], sg[(i + 1) % NST], wave, wn, st + i, s1, f, acc);
    st += NST;
  }
  const int tail = s1 - st;
#pragma unroll
  for (int i = 0; i < NST - 1; ++i)
    if (tail > i) qgemm_dl_step<Q, NST>(src, L, sg[i], sg[i + 1], wave, wn, st + i, s1, f, acc);
  wait_lgkm0();  // the last fragments are read before the stages become C
  bar();
  if (S == 1)
    Q::finish(p, mt, b, n0, m0, threadIdx.x, lane, wn, acc, (float*)lds, qs);
  else
    Q::spill(p, mt, b, n0, m0, threadIdx.x, lane, wn, kc, acc, (float*)lds);
}

}  // namespace aexq
